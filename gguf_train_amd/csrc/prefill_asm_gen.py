"""Generator of the software-pipelined prefill kernel body: gfx950 assembly for fp16 attention
with head size 128, emitted as the text of one inline-assembly statement that
attn_prefill_asm.hip places in a HIP kernel (which supplies the kernel descriptor, the
arguments and the LDS allocation).  It replaces the reference's scalar loop
(csrc/gt_ops_nn.cpp:2468-2522) for fp16 q/k/v, D = Dv = 128, no mask, no dropout, keys in
whole 128-key pairs of tiles; everything else runs on the HIP kernels.

    python prefill_asm_gen.py OUT.inc      writes the macros GT_PREFILL_ASM_CAUSAL and
                                           GT_PREFILL_ASM_FULL (the two kernel bodies)

Work decomposition (the HIP kernel's, attn_prefill.hip): a workgroup of 2 wavefronts runs the
query tiles qa = nq-1-p and qb = p (128 rows) of one head one after the other; each wavefront
owns 64 query rows, as two 32-row blocks qb0/qb1, and holds their Q^T fragments (a[128:191])
and O^T accumulators (a[0:127]) in accumulation registers for the whole tile, so one wavefront
per SIMD (512 registers) and two workgroups per CU.  K and V stream through LDS in tiles of 64
keys, two stages each (K at 0 / 16 KB, V at 32 / 48 KB), written by global_load_lds_dwordx4
with the 16-byte chunk swizzle of the HIP kernel (chunk c of row r at c ^ ((r ^ 4r) & 15)).

Each 32-key block b of a query tile passes three stages:
    S_b   = K_b . Q^T         16 MFMAs (8 k-steps x 2 row blocks), K fragments ds_read_b128
    P_b   = 2^(S_b c - m)     VALU: fma, exp, fp16 pack, row sums by v_dot2 (no row max)
    O^T  += V_b^T . P_b^T     16 MFMAs, V^T fragments by ds_read_b64_tr_b16
and step u of the loop issues S_{u+1} and O += V_{u-1} P_{u-1} (32 MFMAs) with the VALU work of
P_u spread between them (3 VALU instructions per MFMA): the MFMA pipe never waits for the
softmax.  The K and V rings are one tile apart (K_{j+1} and V_j are loaded while S reads K_j
and P.V reads V_{j-1}), with one barrier per tile.

Reference point without a row max: P_b is formed against the row's current reference point m;
a lane whose 16 probabilities of a block sum above 2^8 (an overflow of the fp16 pack gives inf,
which also counts) makes the wavefront take the slow path once: row max of S_b, m moves to it
(with the huge-value margin of the HIP kernel), O and the running sum are rescaled and P_b is
formed again.  The first block of every tile always takes it (m = -inf until then).

Causal tiles: the last four blocks of a query tile straddle the diagonal; a 32-row block is
FULL (every key visible), DIAG (the block on the diagonal: the S accumulator starts from a
0/-inf triangle instead of 0) or INVISIBLE (skipped: no S, P or P.V work).  Those blocks run
in per-wavefront copies of the last pipeline steps.
"""

from __future__ import annotations

import sys
from pathlib import Path

# ---------------------------------------------------------------- registers
V_TID = 0
V_LANE, V_LROW, V_HALF = 1, 2, 3
V_KOFS = 8      # 8: LDS byte offset of K fragment t (row lrow, chunk (2t+half) ^ swz)
V_VOFS0 = 16    # 4: V^T fragment (db) first 4 keys; V_VOFS1: keys +8
V_VOFS1 = 20
V_DOFF = 24     # 8: global byte offset of this lane's chunk of tile load n (K and V rows)
V_TRI = 32      # 16: diagonal block initial S (0 visible, -inf above the diagonal)
V_M = 48        # 2: reference point (log2 domain) of this lane's row in qb0 / qb1
V_NM = 50       # 2: -m
V_LS = 52       # 2: this lane's share of the row sum
V_PART = 54     # 2: the current block's share
V_ONES = 56     # fp16 pair (1, 1)
V_NEGINF = 57
V_QOFF = 58     # 2: byte offset of this lane's q row (+ 16 half) in the head
V_OOFF = 60     # 2: byte offset of this lane's o row (+ 8 half)
V_T = 62        # 8: softmax temporaries
V_W = 70        # 10: slow path / set-up temporaries
V_S = (80, 112)     # S^T accumulators of the two block parities: qb0 +0, qb1 +16
V_P = (144, 160)    # packed P^T of the two parities: qb * 8 + hs * 4
V_KF = 176      # 8 x 4: K fragments of a block
V_VF = 208      # 8 x 4: V^T fragments of a block (4 hs + db)
V_E = 240       # 16: epilogue temporaries
A_O = 0         # O^T (qb, db): a[64 qb + 16 db : +15]
A_Q = 128       # Q^T (qb, t):  a[128 + 32 qb + 4 t : +3]
A_QN = 192      # the second query tile's Q^T

S_W = 40        # wavefront index in the workgroup
S_FIRST = 41    # 1 until the first block's slow path of a query tile
S_LIVE = 42     # slow path: bit qb set when row block qb is not INVISIBLE
S_RET = 44      # 2: slow-path return address
S_TGT = 46      # 2
S_TMP = 48      # 2
S_KT = 50       # 2: global address of the next K tile to load
S_VT = 52       # 2: next V tile
S_M0K = 54      # LDS byte address of this wavefront's part of K stage 0
S_M0V = 55      # same for V stage 0
S_THR = 56      # 256.0: a block share above it takes the slow path
S_LOOP = 57     # pipeline pairs left
S_NT = 58       # key tiles of the current query tile
S_PART = 59     # query tile index within the pair (0, 1)
S_QT = 60       # current query tile
S_P20 = 62      # 2^20
S_PM21 = 63     # 2^-21
S_LN2 = 64
S_TILEB = 65    # bytes per K/V tile (64 rows)
S_QBASE = 66    # 2: q of (b, h)
S_SAVE = 68     # 2: saved exec
S_KB = 70       # 2: k of (b, kv head)
S_VB = 72       # 2: v of (b, kv head)
S_OBASE = 74    # 2: o of (b, h)
S_LSEB = 76     # 2: lse of (b, h)
S_X = 78        # 2: temporaries
S_M0SAVE = 80
S_ROW0 = 81     # first query row of this wavefront in the current tile
S_LM1 = 82      # L - 1

NEG_INF = "0xff800000"
ONE_H2 = "0x3c003c00"


def vr(i: int, n: int = 1) -> str:
    return f"v{i}" if n == 1 else f"v[{i}:{i + n - 1}]"


def ar(i: int, n: int = 1) -> str:
    return f"a{i}" if n == 1 else f"a[{i}:{i + n - 1}]"


def sr(i: int, n: int = 1) -> str:
    return f"s{i}" if n == 1 else f"s[{i}:{i + n - 1}]"


# ---------------------------------------------------------------- block modes
F, DG, INV = "F", "D", "I"


def diag_modes(rel: int, w: int) -> tuple[str, str]:
    """Modes of row blocks qb0/qb1 of wavefront w for the block `rel` (0..3) of the four that
    cover the tile's own 128 keys: row block 2w + qb sits on the diagonal block rel = 2w + qb."""
    out = []
    for qb in (0, 1):
        d = 2 * w + qb
        out.append(F if rel < d else DG if rel == d else INV)
    return tuple(out)


class Ctx:
    def __init__(self, tag: str):
        self.tag = tag        # label prefix (unique per kernel body)
        self.n = 0

    def label(self, name: str) -> str:
        self.n += 1
        return f"{self.tag}_{name}_{self.n}_%="


# ---------------------------------------------------------------- pieces
def call_slow(ctx: Ctx, par: int) -> list[str]:
    lab = ctx.label("call")
    return [
        f"s_getpc_b64 {sr(S_TGT, 2)}",
        f"{lab}:",
        f"s_add_u32 {sr(S_TGT)}, {sr(S_TGT)}, {ctx.tag}_SLOW{par}_%= - {lab}",
        f"s_addc_u32 {sr(S_TGT + 1)}, {sr(S_TGT + 1)}, 0",
        f"s_swappc_b64 {sr(S_RET, 2)}, {sr(S_TGT, 2)}",
    ]


def softmax_valu(par: int, qb: int, trot: list[int]) -> list[str]:
    """P^T of row block qb from S^T of parity `par` against the reference point: 16 fma + 16
    exp + 8 fp16 packs + 8 pair sums (the block share in V_PART + qb).  The 8 pairs run
    software-pipelined by one (fma of pair k+1 between the exponentials of pair k and their
    pack): a VALU instruction reading a v_exp result needs one wait state after it."""
    s0 = V_S[par] + 16 * qb
    pairs = []
    for hs in (0, 1):
        for e2 in range(4):
            i0 = 8 * hs + 2 * e2
            ta, tb = trot[0], trot[1]
            trot[:] = trot[2:] + trot[:2]
            p = V_P[par] + 8 * qb + 4 * hs + e2
            first = hs == 0 and e2 == 0
            pairs.append((
                [f"v_fma_f32 {vr(ta)}, {vr(s0 + i0)}, %[c], {vr(V_NM + qb)}",
                 f"v_fma_f32 {vr(tb)}, {vr(s0 + i0 + 1)}, %[c], {vr(V_NM + qb)}"],
                [f"v_exp_f32 {vr(ta)}, {vr(ta)}", f"v_exp_f32 {vr(tb)}, {vr(tb)}"],
                [f"v_cvt_pk_f16_f32 {vr(p)}, {vr(ta)}, {vr(tb)}",
                 f"v_dot2_f32_f16 {vr(V_PART + qb)}, {vr(p)}, {vr(V_ONES)}, " + ("0" if first else vr(V_PART + qb))],
            ))
    out = pairs[0][0] + pairs[0][1]
    for k in range(1, 8):
        out += pairs[k][0] + pairs[k - 1][2] + pairs[k][1]
    out += ["s_nop 0"] + pairs[7][2]
    return out


def slow_path(ctx: Ctx, par: int) -> list[str]:
    """Subroutine: row max of the block, new reference points, O and row sums rescaled (not on
    a tile's first block), P^T and the block share formed again.  Row blocks whose bit in
    S_LIVE is clear are left alone."""
    out = [f"{ctx.tag}_SLOW{par}_%=:"] + ["s_nop 7"] * 4
    W = V_W
    for qb in (0, 1):
        skip = ctx.label("sk")
        norm = ctx.label("nr")
        s0 = V_S[par] + 16 * qb
        out += [f"s_bitcmp1_b32 {sr(S_LIVE)}, {qb}", f"s_cbranch_scc0 {skip}"]
        out.append(f"v_max3_f32 {vr(W)}, {vr(s0)}, {vr(s0 + 1)}, {vr(s0 + 2)}")
        for i in range(3, 15, 2):
            out.append(f"v_max3_f32 {vr(W)}, {vr(W)}, {vr(s0 + i)}, {vr(s0 + i + 1)}")
        out.append(f"v_max_f32 {vr(W)}, {vr(W)}, {vr(s0 + 15)}")
        out += [
            f"v_mov_b32 {vr(W + 1)}, {vr(W)}",
            f"v_mov_b32 {vr(W + 2)}, {vr(W)}",
            "s_nop 1",
            f"v_permlane32_swap_b32 {vr(W + 1)}, {vr(W + 2)}",
            f"v_max_f32 {vr(W)}, {vr(W + 1)}, {vr(W + 2)}",
            f"v_mul_f32 {vr(W)}, %[c], {vr(W)}",                       # tm (log2 units)
            f"v_and_b32 {vr(W + 1)}, 0x7fffffff, {vr(W)}",
            f"v_cmp_le_f32 vcc, {sr(S_P20)}, {vr(W + 1)}",             # |tm| >= 2^20
            f"v_mul_f32 {vr(W + 1)}, {sr(S_PM21)}, {vr(W + 1)}",
            "s_nop 1",
            f"v_cndmask_b32 {vr(W + 1)}, 0, {vr(W + 1)}, vcc",
            f"v_add_f32 {vr(W)}, {vr(W)}, {vr(W + 1)}",                # tm + margin
            f"v_max_f32 {vr(W)}, {vr(V_M + qb)}, {vr(W)}",             # new reference point
            f"v_sub_f32 {vr(W + 1)}, {vr(V_M + qb)}, {vr(W)}",
            f"v_exp_f32 {vr(W + 1)}, {vr(W + 1)}",                     # alpha
            f"v_cmp_eq_f32 vcc, {NEG_INF}, {vr(W)}",
            "s_nop 1",
            f"v_cndmask_b32_e64 {vr(W + 1)}, {vr(W + 1)}, 1.0, vcc",  # nothing visible yet: 1
            f"v_mul_f32 {vr(V_LS + qb)}, {vr(V_LS + qb)}, {vr(W + 1)}",
            f"v_mov_b32 {vr(V_M + qb)}, {vr(W)}",
            f"v_sub_f32 {vr(V_NM + qb)}, 0, {vr(W)}",
            f"s_cmp_eq_u32 {sr(S_FIRST)}, 0",
            f"s_cbranch_scc0 {norm}",
        ]
        # O^T of the row block times alpha (the MFMAs writing it have retired: s_nop above)
        for i in range(0, 64, 4):
            out += [f"v_accvgpr_read_b32 {vr(W + 2 + e)}, {ar(A_O + 64 * qb + i + e)}" for e in range(4)]
            out += [f"v_mul_f32 {vr(W + 2 + e)}, {vr(W + 1)}, {vr(W + 2 + e)}" for e in range(4)]
            out += [f"v_accvgpr_write_b32 {ar(A_O + 64 * qb + i + e)}, {vr(W + 2 + e)}" for e in range(4)]
        out.append(f"{norm}:")
        out += softmax_valu(par, qb, [V_T + i for i in range(8)])
        out.append(f"{skip}:")
    out += ["s_nop 4", f"s_setpc_b64 {sr(S_RET, 2)}"]
    return out


def dma_tile(kind: str, stage: int) -> list[list[str]]:
    """The 8 loads (1 KB each) of this wavefront's half of a 64-key K or V tile into `stage`,
    then the tile pointer's advance; each element is one issue group."""
    base = S_M0K if kind == "K" else S_M0V
    ptr = S_KT if kind == "K" else S_VT
    groups = []
    for n in range(8):
        groups.append([
            f"s_add_u32 m0, {sr(base)}, {stage * 16384 + n * 1024}",
            "s_nop 0",
            f"global_load_lds_dwordx4 {vr(V_DOFF + n)}, {sr(ptr, 2)}",
        ])
    groups[-1] += [
        f"s_add_u32 {sr(ptr)}, {sr(ptr)}, {sr(S_TILEB)}",
        f"s_addc_u32 {sr(ptr + 1)}, {sr(ptr + 1)}, 0",
    ]
    return groups


def emit_step(ctx: Ctx, u: int, nb: int, nt: int, modes_of, final_extra=None) -> list[str]:
    """Pipeline step u: [barrier + tile loads], S_{u+1}, P_u (with its check), O += V_{u-1} P_{u-1}."""
    out: list[str] = []
    dma_groups: list[list[str]] = []
    if u == -1 or u % 2 == 1:
        j = (u + 1) // 2
        out += ["s_waitcnt vmcnt(0)", "s_barrier"]
        if j + 1 < nt:
            dma_groups += dma_tile("K", (j + 1) % 2)
        if j < nt:
            dma_groups += dma_tile("V", j % 2)
        if j == nt and final_extra:
            out += final_extra(ctx)
    mf: list[tuple[str, list]] = []
    reads: list[tuple[tuple, str]] = []
    b = u + 1
    if 0 <= b < nb:
        modes = modes_of(b)
        tile, kb = b // 2, b % 2
        if any(m != INV for m in modes):
            off = (tile % 2) * 16384 + kb * 8192
            for t in range(8):
                reads.append((("K", t), f"ds_read_b128 {vr(V_KF + 4 * t, 4)}, {vr(V_KOFS + t)} offset:{off}"))
            for t in range(8):
                for qb in (0, 1):
                    if modes[qb] == INV:
                        continue
                    dst = V_S[b % 2] + 16 * qb
                    if t == 0:
                        c = "0" if modes[qb] == F else vr(V_TRI, 16)
                    else:
                        c = vr(dst, 16)
                    mf.append((f"v_mfma_f32_32x32x16_f16 {vr(dst, 16)}, {vr(V_KF + 4 * t, 4)}, "
                               f"{ar(A_Q + 32 * qb + 4 * t, 4)}, {c}", [("K", t)]))
    b = u - 1
    if 0 <= b < nb:
        modes = modes_of(b)
        tile, kb = b // 2, b % 2
        if any(m != INV for m in modes):
            for hs in (0, 1):
                for db in range(4):
                    f = 4 * hs + db
                    off = 32768 + (tile % 2) * 16384 + 4096 * (2 * kb + hs)
                    reads.append((("V", f, 0), f"ds_read_b64_tr_b16 {vr(V_VF + 4 * f, 2)}, {vr(V_VOFS0 + db)} offset:{off}"))
                    reads.append((("V", f, 1), f"ds_read_b64_tr_b16 {vr(V_VF + 4 * f + 2, 2)}, {vr(V_VOFS1 + db)} offset:{off}"))
            for hs in (0, 1):
                for db in range(4):
                    f = 4 * hs + db
                    for qb in (0, 1):
                        if modes[qb] == INV:
                            continue
                        o = A_O + 64 * qb + 16 * db
                        c = "0" if (b == 0 and hs == 0) else ar(o, 16)
                        mf.append((f"v_mfma_f32_32x32x16_f16 {ar(o, 16)}, {vr(V_VF + 4 * f, 4)}, "
                                   f"{vr(V_P[b % 2] + 8 * qb + 4 * hs, 4)}, {c}", [("V", f, 0), ("V", f, 1)]))
    valu: list[str] = []
    sm_live: list[int] = []
    if 0 <= u < nb:
        modes = modes_of(u)
        trot = [V_T + i for i in range(8)]
        for qb in (0, 1):
            if modes[qb] != INV:
                sm_live.append(qb)
                if u > 0:  # block 0 always takes the slow path, which forms its P
                    valu += softmax_valu(u % 2, qb, trot)
    if valu and not mf:
        out += ["s_nop 7"] * 4  # S of this block may have been the previous step's last MFMAs

    # ---- schedule: reads ahead of their MFMAs, VALU and tile loads between MFMAs
    order = {key: i for i, (key, _) in enumerate(reads)}
    issued = 0
    done_upto = 0          # reads known complete
    LIMIT = 10             # outstanding LDS reads
    PRE = 6

    def issue_reads(n):
        nonlocal issued
        k = 0
        while issued < len(reads) and k < n and issued - done_upto < LIMIT:
            out.append(reads[issued][1])
            issued += 1
            k += 1

    issue_reads(PRE)
    nm = len(mf)
    per = -(-len(valu) // nm) if nm else 0
    vi = 0
    di = 0
    dma_every = max(1, nm // max(1, len(dma_groups))) if dma_groups else 0
    for i, (txt, needs) in enumerate(mf):
        last = max(order[k] for k in needs)
        while issued <= last:
            issue_reads(1)
            if issued <= last and issued - done_upto >= LIMIT:
                # make room: wait for the oldest
                out.append(f"s_waitcnt lgkmcnt({LIMIT - 1})")
                done_upto = issued - (LIMIT - 1)
        if last >= done_upto:
            cnt = issued - (last + 1)
            out.append(f"s_waitcnt lgkmcnt({min(cnt, 15)})")
            done_upto = last + 1
        out.append(txt)
        out += valu[vi:vi + per]
        vi += per
        issue_reads(1)
        if dma_groups and di < len(dma_groups) and i % dma_every == 0:
            out += dma_groups[di]
            di += 1
    out += valu[vi:]
    while di < len(dma_groups):
        out += dma_groups[di]
        di += 1
    assert issued == len(reads), (u, issued, len(reads))

    # ---- the block's check: any lane share above 2^8 (or inf/the first block) -> slow path
    if sm_live:
        par = u % 2
        live_mask = sum(1 << qb for qb in sm_live)
        if u == 0:
            out += [f"s_mov_b32 {sr(S_LIVE)}, {live_mask}"] + call_slow(ctx, par) + [f"s_mov_b32 {sr(S_FIRST)}, 0"]
        else:
            noslow = ctx.label("ns")
            out.append(f"v_cmp_lt_f32 vcc, {sr(S_THR)}, {vr(V_PART + sm_live[0])}")
            if len(sm_live) == 2:
                out += [f"v_cmp_lt_f32_e64 {sr(S_TMP, 2)}, {sr(S_THR)}, {vr(V_PART + sm_live[1])}",
                        "s_nop 1", f"s_or_b64 vcc, vcc, {sr(S_TMP, 2)}"]
            out += ["s_nop 4", f"s_cbranch_vccz {noslow}", f"s_mov_b32 {sr(S_LIVE)}, {live_mask}"]
            out += call_slow(ctx, par)
            out.append(f"{noslow}:")
        for qb in sm_live:
            out.append(f"v_add_f32 {vr(V_LS + qb)}, {vr(V_LS + qb)}, {vr(V_PART + qb)}")
    return out


# ---------------------------------------------------------------- kernel sections
def setup() -> list[str]:
    W = V_W
    out = [
        f"s_mov_b32 {sr(S_M0SAVE)}, m0",
        f"v_and_b32 {vr(V_LANE)}, 63, {vr(V_TID)}",
        f"v_lshrrev_b32 {vr(W)}, 6, {vr(V_TID)}",
        f"v_readfirstlane_b32 {sr(S_W)}, {vr(W)}",
        f"v_and_b32 {vr(V_LROW)}, 31, {vr(V_LANE)}",
        f"v_lshrrev_b32 {vr(V_HALF)}, 5, {vr(V_LANE)}",
        f"s_mov_b64 {sr(S_QBASE, 2)}, %[q]",
        f"s_mov_b64 {sr(S_KB, 2)}, %[k]",
        f"s_mov_b64 {sr(S_VB, 2)}, %[v]",
        f"s_mov_b64 {sr(S_OBASE, 2)}, %[o]",
        f"s_mov_b64 {sr(S_LSEB, 2)}, %[lse]",
        f"s_mov_b32 {sr(S_THR)}, 0x43800000",
        f"s_mov_b32 {sr(S_P20)}, 0x49800000",
        f"s_mov_b32 {sr(S_PM21)}, 0x35000000",
        f"s_mov_b32 {sr(S_LN2)}, 0x3f317218",
        f"s_lshl_b32 {sr(S_TILEB)}, %[kvrow], 6",
        f"s_add_u32 {sr(S_LM1)}, %[L], -1",
        f"v_mov_b32 {vr(V_ONES)}, {ONE_H2}",
        f"v_mov_b32 {vr(V_NEGINF)}, {NEG_INF}",
        # swz(lrow) in W
        f"v_lshlrev_b32 {vr(W)}, 2, {vr(V_LROW)}",
        f"v_xor_b32 {vr(W)}, {vr(W)}, {vr(V_LROW)}",
        f"v_and_b32 {vr(W)}, 15, {vr(W)}",
        f"v_lshlrev_b32 {vr(W + 1)}, 8, {vr(V_LROW)}",
        f"v_add_u32 {vr(W + 1)}, %[lds], {vr(W + 1)}",
    ]
    for t in range(8):
        out += [
            f"v_or_b32 {vr(W + 2)}, {2 * t}, {vr(V_HALF)}",
            f"v_xor_b32 {vr(W + 2)}, {vr(W + 2)}, {vr(W)}",
            f"v_lshl_add_u32 {vr(V_KOFS + t)}, {vr(W + 2)}, 4, {vr(W + 1)}",
        ]
    # V^T fragments: row = 4 half + ((lane >> 2) & 3), chunk = 4 db + 2 ((lane >> 4) & 1) + ((lane >> 1) & 1),
    # + 8 (lane & 1) bytes; rows +8 flip bit 3 of the swizzle
    out += [
        f"v_bfe_u32 {vr(W)}, {vr(V_LANE)}, 2, 2",
        f"v_lshl_add_u32 {vr(W)}, {vr(V_HALF)}, 2, {vr(W)}",          # row
        f"v_lshlrev_b32 {vr(W + 1)}, 2, {vr(W)}",
        f"v_xor_b32 {vr(W + 1)}, {vr(W + 1)}, {vr(W)}",
        f"v_and_b32 {vr(W + 1)}, 15, {vr(W + 1)}",                    # swz(row)
        f"v_bfe_u32 {vr(W + 2)}, {vr(V_LANE)}, 4, 1",
        f"v_bfe_u32 {vr(W + 3)}, {vr(V_LANE)}, 1, 1",
        f"v_lshl_add_u32 {vr(W + 2)}, {vr(W + 2)}, 1, {vr(W + 3)}",   # chunk base
        f"v_and_b32 {vr(W + 3)}, 1, {vr(V_LANE)}",
        f"v_lshlrev_b32 {vr(W + 3)}, 3, {vr(W + 3)}",
        f"v_lshlrev_b32 {vr(W + 4)}, 8, {vr(W)}",
        f"v_add3_u32 {vr(W + 3)}, {vr(W + 3)}, {vr(W + 4)}, %[lds]",  # lds + row*256 + 8 (lane & 1)
        f"v_xor_b32 {vr(W + 5)}, 8, {vr(W + 1)}",                      # swz(row + 8)
    ]
    for db in range(4):
        out += [
            f"v_add_u32 {vr(W + 4)}, {4 * db}, {vr(W + 2)}",
            f"v_xor_b32 {vr(W + 6)}, {vr(W + 4)}, {vr(W + 1)}",
            f"v_lshl_add_u32 {vr(V_VOFS0 + db)}, {vr(W + 6)}, 4, {vr(W + 3)}",
            f"v_xor_b32 {vr(W + 6)}, {vr(W + 4)}, {vr(W + 5)}",
            f"v_lshl_add_u32 {vr(W + 6)}, {vr(W + 6)}, 4, {vr(W + 3)}",
            f"v_add_u32 {vr(V_VOFS1 + db)}, 0x800, {vr(W + 6)}",
        ]
    # tile loads: load n of wavefront w fills rows 4 (8 w + n) + (lane >> 4), LDS chunk lane & 15
    # with global chunk (lane & 15) ^ swz(row); byte offset row * kvrow + 16 chunk
    out += [
        f"v_lshrrev_b32 {vr(W)}, 4, {vr(V_LANE)}",                    # g16
        f"v_and_b32 {vr(W + 1)}, 15, {vr(V_LANE)}",
        f"s_lshl_b32 {sr(S_X)}, {sr(S_W)}, 5",
    ]
    for n in range(8):
        out += [
            f"v_add_u32 {vr(W + 2)}, {4 * n}, {vr(W)}",                # (4n + g16), row mod 16 source
            f"v_and_b32 {vr(W + 3)}, 15, {vr(W + 2)}",
            f"v_lshlrev_b32 {vr(W + 4)}, 2, {vr(W + 3)}",
            f"v_xor_b32 {vr(W + 4)}, {vr(W + 4)}, {vr(W + 3)}",
            f"v_and_b32 {vr(W + 4)}, 15, {vr(W + 4)}",
            f"v_xor_b32 {vr(W + 4)}, {vr(W + 4)}, {vr(W + 1)}",        # global chunk
            f"v_add_u32 {vr(W + 2)}, {sr(S_X)}, {vr(W + 2)}",          # row = 32 w + 4 n + g16
            f"v_mul_lo_u32 {vr(W + 2)}, {vr(W + 2)}, %[kvrow]",
            f"v_lshl_add_u32 {vr(V_DOFF + n)}, {vr(W + 4)}, 4, {vr(W + 2)}",
        ]
    out += [
        f"s_lshl_b32 {sr(S_X)}, {sr(S_W)}, 13",
        f"s_add_u32 {sr(S_M0K)}, %[lds], {sr(S_X)}",
        f"s_add_u32 {sr(S_M0V)}, {sr(S_M0K)}, 32768",
        f"v_lshlrev_b32 {vr(W)}, 2, {vr(V_HALF)}",
    ]
    # diagonal triangle: key 8 (i/4) + 4 half + i%4 visible to row lrow when <= lrow
    for i in range(16):
        out += [
            f"v_add_u32 {vr(W + 1)}, {8 * (i // 4) + i % 4}, {vr(W)}",
            f"v_cmp_gt_u32 vcc, {vr(W + 1)}, {vr(V_LROW)}",
            "s_nop 1",
            f"v_cndmask_b32 {vr(V_TRI + i)}, 0, {vr(V_NEGINF)}, vcc",
        ]
    return out


def load_q(aset: int, qt_sgpr: str) -> list[str]:
    """Q^T fragments of query tile `qt_sgpr` into a[aset:aset+63]: this lane's rows (clamped to
    L-1), 16 bytes at dims 16 t + 8 half."""
    W = V_W
    out = [
        f"s_lshl_b32 {sr(S_X)}, {qt_sgpr}, 7",
        f"s_lshl_b32 {sr(S_X + 1)}, {sr(S_W)}, 6",
        f"s_add_u32 {sr(S_X)}, {sr(S_X)}, {sr(S_X + 1)}",
    ]
    for qb in (0, 1):
        out += [
            f"v_add3_u32 {vr(W)}, {sr(S_X)}, {32 * qb}, {vr(V_LROW)}",
            f"v_min_u32 {vr(W)}, {sr(S_LM1)}, {vr(W)}",
            f"v_mul_lo_u32 {vr(W)}, {vr(W)}, %[qsl]",
            f"v_lshl_add_u32 {vr(W)}, {vr(V_HALF)}, 4, {vr(W)}",
        ]
        for t in range(8):
            out.append(f"global_load_dwordx4 {ar(aset + 32 * qb + 4 * t, 4)}, {vr(W)}, {sr(S_QBASE, 2)} offset:{32 * t}")
    return out


def part_start(ctx: Ctx, causal: bool) -> list[str]:
    """Query tile set-up: tile index, key tiles, rows, Q (first tile: both tiles' Q; second:
    copied from the second set), reference points, the first K tile's loads (the first tile
    only: the second tile's were issued at the end of the first)."""
    W = V_W
    second = ctx.label("p2")
    qdone = ctx.label("qd")
    out = [
        f"s_cmp_eq_u32 {sr(S_PART)}, 0",
        f"s_cselect_b32 {sr(S_QT)}, %[qa], %[qb]",
    ]
    if causal:
        out += [f"s_add_u32 {sr(S_NT)}, {sr(S_QT)}, 1", f"s_lshl_b32 {sr(S_NT)}, {sr(S_NT)}, 1"]
    else:
        out += [f"s_mov_b32 {sr(S_NT)}, %[ntk]"]
    out += [
        f"s_lshl_b32 {sr(S_ROW0)}, {sr(S_QT)}, 7",
        f"s_lshl_b32 {sr(S_X)}, {sr(S_W)}, 6",
        f"s_add_u32 {sr(S_ROW0)}, {sr(S_ROW0)}, {sr(S_X)}",
        f"s_mov_b64 {sr(S_VT, 2)}, {sr(S_VB, 2)}",
        f"s_mov_b32 {sr(S_FIRST)}, 1",
        f"v_mov_b32 {vr(V_M)}, {NEG_INF}",
        f"v_mov_b32 {vr(V_M + 1)}, {NEG_INF}",
        f"v_mov_b32 {vr(V_NM)}, 0x7f800000",
        f"v_mov_b32 {vr(V_NM + 1)}, 0x7f800000",
        f"v_mov_b32 {vr(V_LS)}, 0",
        f"v_mov_b32 {vr(V_LS + 1)}, 0",
    ]
    for qb in (0, 1):
        out += [
            f"v_add3_u32 {vr(W)}, {sr(S_ROW0)}, {32 * qb}, {vr(V_LROW)}",
            f"v_lshlrev_b32 {vr(V_OOFF + qb)}, 8, {vr(W)}",
            f"v_lshl_add_u32 {vr(V_OOFF + qb)}, {vr(V_HALF)}, 3, {vr(V_OOFF + qb)}",
        ]
    out += [f"s_cmp_eq_u32 {sr(S_PART)}, 0", f"s_cbranch_scc0 {second}"]
    # first tile: both tiles' Q, and its first K tile (the second tile's is loaded at the first
    # tile's last barrier, next_k0)
    out += load_q(A_Q, "%[qa]")
    out += [f"s_cmp_lt_u32 1, %[np]", f"s_cbranch_scc0 {qdone}"]
    out += load_q(A_QN, "%[qb]")
    out += [f"{qdone}:", f"s_mov_b64 {sr(S_KT, 2)}, {sr(S_KB, 2)}"]
    for g in dma_tile("K", 0):
        out += g
    out += [f"s_branch {qdone}_x", f"{second}:"]
    out += ["s_nop 7"] * 4
    out += [f"v_accvgpr_mov_b32 {ar(A_Q + i)}, {ar(A_QN + i)}" for i in range(64)]
    out += ["s_nop 2", f"{qdone}_x:"]
    return out


def next_k0(ctx: Ctx) -> list[str]:
    """At the last tile barrier of the first query tile: the second tile's first K tile (every
    wavefront has read its last K tile by then)."""
    lab = ctx.label("nk")
    out = [f"s_cmp_lt_u32 1, %[np]", f"s_cbranch_scc0 {lab}", f"s_cmp_eq_u32 {sr(S_PART)}, 0",
           f"s_cbranch_scc0 {lab}", f"s_mov_b64 {sr(S_KT, 2)}, {sr(S_KB, 2)}"]
    for g in dma_tile("K", 0):
        out += g
    out.append(f"{lab}:")
    return out


def epilogue(ctx: Ctx) -> list[str]:
    """O = O^T / l as fp16 rows, and the log-sum-exp (natural log), for rows < L."""
    E = V_E
    W = V_W
    out = ["s_nop 7"] * 4
    for qb in (0, 1):
        nolse = ctx.label("nl")
        out += [
            f"v_mov_b32 {vr(W + 1)}, {vr(V_LS + qb)}",
            f"v_mov_b32 {vr(W + 2)}, {vr(V_LS + qb)}",
            "s_nop 1",
            f"v_permlane32_swap_b32 {vr(W + 1)}, {vr(W + 2)}",
            f"v_add_f32 {vr(W)}, {vr(W + 1)}, {vr(W + 2)}",            # l
            f"v_rcp_f32 {vr(W + 1)}, {vr(W)}",
            f"v_cmp_lt_f32 vcc, 0, {vr(W)}",
            "s_nop 1",
            f"v_cndmask_b32 {vr(W + 1)}, 0, {vr(W + 1)}, vcc",         # 1/l (0 when l = 0)
            f"v_log_f32 {vr(W + 2)}, {vr(W)}",
            "s_nop 0",
            f"v_add_f32 {vr(W + 2)}, {vr(V_M + qb)}, {vr(W + 2)}",
            f"v_mul_f32 {vr(W + 2)}, {sr(S_LN2)}, {vr(W + 2)}",
            f"v_mov_b32 {vr(W + 3)}, 0x7f800000",
            f"v_cndmask_b32 {vr(W + 2)}, {vr(W + 3)}, {vr(W + 2)}, vcc",  # lse (+inf when l = 0)
            f"v_add3_u32 {vr(W + 3)}, {sr(S_ROW0)}, {32 * qb}, {vr(V_LROW)}",   # row
            f"v_cmp_gt_u32 vcc, %[L], {vr(W + 3)}",
            "s_nop 1",
            f"s_and_saveexec_b64 {sr(S_SAVE, 2)}, vcc",
        ]
        for db in range(4):
            for g in range(4):
                a0 = A_O + 64 * qb + 16 * db + 4 * g
                out += [f"v_accvgpr_read_b32 {vr(E + e)}, {ar(a0 + e)}" for e in range(4)]
                out += [f"v_mul_f32 {vr(E + e)}, {vr(W + 1)}, {vr(E + e)}" for e in range(4)]
                out += [
                    f"v_cvt_pk_f16_f32 {vr(E + 4)}, {vr(E)}, {vr(E + 1)}",
                    f"v_cvt_pk_f16_f32 {vr(E + 5)}, {vr(E + 2)}, {vr(E + 3)}",
                    f"global_store_dwordx2 {vr(V_OOFF + qb)}, {vr(E + 4, 2)}, {sr(S_OBASE, 2)} offset:{64 * db + 16 * g}",
                ]
        out += [
            f"s_cmp_eq_u64 {sr(S_LSEB, 2)}, 0",
            f"s_cbranch_scc1 {nolse}",
            f"v_cmp_eq_u32 vcc, 0, {vr(V_HALF)}",
            "s_nop 1",
            "s_and_b64 exec, exec, vcc",
            f"v_lshlrev_b32 {vr(W + 3)}, 2, {vr(W + 3)}",
            f"global_store_dword {vr(W + 3)}, {vr(W + 2)}, {sr(S_LSEB, 2)}",
            f"{nolse}:",
            f"s_mov_b64 exec, {sr(S_SAVE, 2)}",
        ]
    return out


def body(causal: bool) -> list[str]:
    tag = "PC" if causal else "PN"
    ctx = Ctx(tag)
    full = lambda b: (F, F)
    out = setup()
    out += [f"s_mov_b32 {sr(S_PART)}, 0", f"{tag}_PART_%=:"]
    out += part_start(ctx, causal)
    nxt = next_k0
    if causal:
        # query tile 0 (2 key tiles): every block is on the diagonal
        out += [f"s_cmp_eq_u32 {sr(S_NT)}, 2", f"s_cbranch_scc0 {tag}_GEN_%="]
        for w in (0, 1):
            out += [f"s_cmp_eq_u32 {sr(S_W)}, {w}", f"s_cbranch_scc0 {tag}_SM{w}_END_%="]
            mo = lambda b, w=w: diag_modes(b, w)
            for u in range(-1, 5):
                out += emit_step(ctx, u, 4, 2, mo, nxt)
            out += [f"s_branch {tag}_EPI_%=", f"{tag}_SM{w}_END_%=:"]
        out.append(f"{tag}_GEN_%=:")
    # prologue and the first pair (no diagonal blocks: at least 4 key tiles)
    for u in range(-1, 3):
        out += emit_step(ctx, u, 16, 8, full, nxt)
    # generic pairs j = 2 .. (nt-3 causal | nt-2 full): count nt-4 | nt-3
    out += [f"s_sub_u32 {sr(S_LOOP)}, {sr(S_NT)}, {4 if causal else 3}", f"{tag}_LOOP_%=:",
            f"s_cmp_eq_u32 {sr(S_LOOP)}, 0", f"s_cbranch_scc1 {tag}_TAIL_%="]
    for u in (3, 4):
        out += emit_step(ctx, u, 16, 8, full, nxt)
    out += [f"s_sub_u32 {sr(S_LOOP)}, {sr(S_LOOP)}, 1", f"s_cmp_eq_u32 {sr(S_LOOP)}, 0",
            f"s_cbranch_scc1 {tag}_TAIL_%="]
    for u in (5, 6):
        out += emit_step(ctx, u, 16, 8, full, nxt)
    out += [f"s_sub_u32 {sr(S_LOOP)}, {sr(S_LOOP)}, 1", f"s_branch {tag}_LOOP_%=", f"{tag}_TAIL_%=:"]
    if causal:
        # pairs nt-2, nt-1, nt (steps 2nt-5 .. 2nt), the last four blocks on the diagonal
        for w in (0, 1):
            out += [f"s_cmp_eq_u32 {sr(S_W)}, {w}", f"s_cbranch_scc0 {tag}_T{w}_END_%="]
            mo = lambda b, w=w: diag_modes(b - 12, w) if b >= 12 else (F, F)
            for u in range(11, 17):
                out += emit_step(ctx, u, 16, 8, mo, nxt)
            out += [f"s_branch {tag}_EPI_%=", f"{tag}_T{w}_END_%=:"]
    else:
        for u in range(13, 17):
            out += emit_step(ctx, u, 16, 8, full, nxt)
    out.append(f"{tag}_EPI_%=:")
    out += epilogue(ctx)
    out += [f"s_add_u32 {sr(S_PART)}, {sr(S_PART)}, 1", f"s_cmp_lt_u32 {sr(S_PART)}, %[np]",
            f"s_cbranch_scc1 {tag}_PART_%=", f"s_branch {tag}_END_%="]
    out += slow_path(ctx, 0) + slow_path(ctx, 1)
    out += [f"{tag}_END_%=:", "s_waitcnt vmcnt(0) lgkmcnt(0)", f"s_mov_b32 m0, {sr(S_M0SAVE)}"]
    return out


def as_macro(name: str, lines: list[str]) -> str:
    body = "".join(f'    "{l}\\n"\n' for l in lines)
    return f"#define {name} \\\n" + body.rstrip("\n").replace("\n", " \\\n") + "\n"


def clobbers() -> str:
    regs = [f'"v{i}"' for i in range(1, 256)] + [f'"a{i}"' for i in range(256)] + [f'"s{i}"' for i in range(40, 84)]
    return "#define GT_PREFILL_ASM_CLOBBERS " + ", ".join(regs + ['"vcc"', '"scc"', '"memory"']) + "\n"


def generate() -> str:
    return ("// generated by prefill_asm_gen.py: do not edit\n" + as_macro("GT_PREFILL_ASM_CAUSAL", body(True))
            + as_macro("GT_PREFILL_ASM_FULL", body(False)) + clobbers())


def main(argv: list[str]) -> int:
    out = Path(argv[1])
    text = generate()
    if not out.exists() or out.read_text() != text:
        out.write_text(text)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
