// Single-query (decode) attention over a GGUF Q8_0 K/V cache, fp16 query.
//
// The reference reads a Q8_0 tensor only after gt_dequantize (ggml to_float,
// csrc/gt_core.cpp:800-808: y = qs * d); passed straight to gt_flash_attention it would read
// zeros (csrc/gt_internal.h:243-259).  This kernel computes attention over exactly the
// dequantized values without materialising them: HBM traffic is the 34-byte blocks
// (1.0625 bytes per value), read once per kv head.
//
// Same streaming decomposition as the fp16 decode kernel: workgroup = (kv head of one
// sequence, split), steps of 128 keys with the next step's loads in flight, wave w owns keys
// [32w, 32w + 32) of a step with its own online softmax, one combine at the end, a merge
// kernel when there are several splits.
//
// Loads: a lane reads 12 bytes (3 dwords, 4-byte aligned) of one key row: the 8 quantized
// values it needs plus, for the first lane of a block, the block's fp16 scale.  qs starts at
// byte 34j + 2 of block j, 2 mod 4 for even j (the load starts 2 bytes early, on d) and 0 mod
// 4 for odd j (the load starts 4 bytes early; d is the high half of the first dword).  A row
// is 34 D/32 bytes, so every load stays inside its row.
//
// Exact int8 -> fp16 without a convert per value: for u = qs ^ 0x80 (= qs + 128) the fp16 bit
// pattern 0x6400 | u is exactly 1024 + u = qs + 1152; one v_perm_b32 places two bytes under a
// zero high byte and one xor sets the 0x64 exponent and flips the sign bit.
//   scores: S^T = K . Q^T on v_mfma_f32_16x16x32_f16, one MFMA per 32-value block (the block
//           is the MFMA's k = 32): acc_j = sum (qs + 1152) q = sum qs q + 1152 sum_block q,
//           so s = sum_j d_j (acc_j - 1152 cq_j) with cq_j the block sums of q.
//   P.V:    o += (p d) (qs + 1152) with v_fma_mix (exact fp16 operand, fp32 accumulation); the
//           offset 1152 sum (p d) is subtracted once at the end.

#include "attn_common.h"
#include "decode_merge.h"
#include "gt_internal.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>

namespace {

constexpr int kStep = 128;  // keys per step of a workgroup (32 per wave)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kMagic = 1152.0f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }
__device__ inline float hlo(uint32_t a) { return (float)__builtin_bit_cast(half2_t, a)[0]; }
__device__ inline float hhi(uint32_t a) { return (float)__builtin_bit_cast(half2_t, a)[1]; }
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Eight qs bytes of a loaded 12-byte group (`odd`: block index odd, see the header), and the
// raw fp16 scale bits (meaningful in the block's first lane).
__device__ inline void extract12(u32x3 w, bool odd, uint32_t &q0, uint32_t &q1, uint32_t &dbits) {
    if (odd) {
        q0 = w[1];
        q1 = w[2];
        dbits = w[0] >> 16;
    } else {
        q0 = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
        q1 = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
        dbits = w[0] & 0xffffu;
    }
}

// Four bytes u = qs + 128 (the sign bit flipped) -> two packed fp16 0x64uu = 1024 + u = qs + 1152:
// one v_perm_b32 puts two bytes under 0x64 exponent bytes taken from the constant.
constexpr uint32_t kExp64 = 0x64646464u;
constexpr uint32_t kSelLo = 0x04010400u;  // (u.b0, 0x64, u.b1, 0x64)
constexpr uint32_t kSelHi = 0x04030402u;  // (u.b2, 0x64, u.b3, 0x64)
__device__ inline u32x2 magic4(uint32_t u) {
    return u32x2{__builtin_amdgcn_perm(kExp64, u, kSelLo), __builtin_amdgcn_perm(kExp64, u, kSelHi)};
}
constexpr uint32_t kFlip = 0x80808080u;

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
__device__ inline u32x2 read_tr8(const uint8_t *p) {
    return __builtin_bit_cast(
        u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2 *)(__attribute__((address_space(3))) char *)p));
}

__device__ inline uint32_t pack_h2(float x, float y) {
    const half2_t v = {(_Float16)x, (_Float16)y};  // round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// MASK: 0 = none, 1 = bool bytes, 2 = additive float.
//
// Per wave and step of 32 keys (v_mfma_f32_16x16x32_f16 layouts, lane l: A[m = l%16][k = 8(l/16)
// + 0..7], B[k = 8(l/16) + 0..7][n = l%16], C[m = 4(l/16) + i][n = l%16]):
//   scores S^T = K . Q^T: A = key rows 16kb + l%16 straight from the loaded blocks, B = Q^T (the
//     G heads as columns), one MFMA per Q8_0 block; lane l ends with the scores of keys
//     16kb + 4(l/16) + i of head l%16, and the softmax runs on those in registers.
//   O^T += V^T . P'^T per Q8_0 block: A = V^T, 16 dims x 32 keys, read from the wave's LDS copy
//     of its 32 V rows with ds_read_b64_tr_b8 (lane i of a 16-lane group receives byte i of 8
//     consecutive rows); B = P'^T with P'[key][head] = p * d_v[key][block] rounded to fp16, the
//     block's scale folded into the probabilities.  The k order of both operands is fixed by
//     storing key r of the step in LDS row 8((r%16)/4) + 4(r/16) + r%4, so that k-slot e of lane
//     group g is key 16(e/4) + 4g + e%4: the probabilities a lane already holds.  The bytes are
//     stored as u = qs + 128, read as fp16 (qs + 1152), and the offset is removed by one more MFMA
//     per accumulator, -1152 x P'^T.
//   The rescale of the accumulators by exp2(m_old - m_new) is skipped when no lane's max moved.
template <int D, int G, int MASK>
__global__ __launch_bounds__(256, 2) void decode_q8_mfma_kernel(DecodeArgs a) {
    constexpr int NB = D / 32;     // Q8_0 blocks per row = k-steps of the score MFMA
    constexpr int RB = NB * 34;    // bytes per row
    constexpr int LPR = D / 8;     // lanes per V row (8 values each)
    constexpr int RPW = 64 / LPR;  // V rows per wave load
    constexpr int NV = 32 / RPW;   // V loads per lane and step
    constexpr int VP = D + 16;     // LDS pitch of a staged V row: 16 consecutive rows hit distinct banks
    __shared__ __attribute__((aligned(16))) uint8_t s_v[4][32 * VP];  // per-wave V bytes u = qs + 128
    __shared__ __attribute__((aligned(16))) float s_dv[4][NB][32];    // per-wave V block scales (k-slot rows)
    __shared__ __attribute__((aligned(16))) float s_d[4][32][NB];     // per-wave K block scales
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int sub = lane % LPR, vrow = lane / LPR;
    const int vblk = sub >> 2, vpart = sub & 3;  // V: block and 8-value part of this lane
    const int split = blockIdx.x;
    // blockIdx.y = (sequence, kv head, head group): the kv head's gtot query heads run in
    // groups of G (the last group may hold fewer, gv; its padding columns are blocked)
    const int gtot = (int)(f.H / f.Hkv), ngrp = (gtot + G - 1) / G;
    const int64_t bkg = blockIdx.y, bk = bkg / ngrp, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int hg = (int)(bkg % ngrp);
    const int h0 = (int)hk * gtot + hg * G, gv = min(G, gtot - hg * G);
    const int S = (int)f.S;
    const int span = ((S + kStep - 1) / kStep + a.nsplit - 1) / a.nsplit * kStep;
    const int kbeg = split * span, kend = min(attn_decode_end(f, b), kbeg + span);
    const int nsteps = kend > kbeg ? (kend - kbeg + kStep - 1) / kStep : 0;

    // B operand (Q^T, fp16): lane holds Q[head h0 + l16][32t + 8 q4 + 0..7]; columns l16 >= gv
    // repeat head h0 + gv - 1 and are discarded.  cq[t]: 1152 x the sum of block t of that query.
    half8_t qb[NB];
    float cq[NB];
    {
        const _Float16 *qr = (const _Float16 *)f.q + b * f.q_sb + (h0 + min(l16, gv - 1)) * f.q_sh + 8 * q4;
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const u32x4 x = *(const u32x4 *)(qr + 32 * t);
            qb[t] = __builtin_bit_cast(half8_t, x);
            float c = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t xe = x[e];  // through a scalar: bit-casting a vector element reads element 0
                c += hlo(xe) + hhi(xe);
            }
            c += __shfl_xor(c, 16, 64);
            c += __shfl_xor(c, 32, 64);
            cq[t] = kMagic * c;
        }
    }

    // Byte offsets from the (b, kv head) slices (dense Q8_0 rows of RB bytes) fit 32 bits
    // (checked by the launcher).  Keys past S read row S-1 (finite; masked / weight 0).
    const int64_t slice = (b * f.Hkv + hk) * (int64_t)S * RB;
    const uint8_t *kbase = (const uint8_t *)f.k + slice;
    const uint8_t *vbase = (const uint8_t *)f.v + slice;
    // lane offsets inside a row: K block t, part q4; V block vblk, part vpart
    auto in_row = [](int blk, int part) { return 34 * blk + 8 * part - ((blk & 1) ? 2 : 0); };
    struct Tile {
        u32x3 k[2][NB];  // key 16kb + l16 of the wave's 32, block t, part q4
        u32x3 v[NV];     // V row RPW*i + vrow of the wave's 32, block vblk, part vpart
    };
    auto load = [&](int step, Tile &tl) {
        // steps past the split re-read its last step (cache hits) instead of new lines
        const int k0 = kbeg + min(step, max(nsteps - 1, 0)) * kStep + 32 * w;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const uint32_t row = (uint32_t)min(k0 + 16 * kb + l16, S - 1) * RB;
#pragma unroll
            for (int t = 0; t < NB; ++t)
                tl.k[kb][t] = __builtin_nontemporal_load((const u32x3 *)(kbase + row + in_row(t, q4)));
        }
        const int voff = in_row(vblk, vpart);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t row = (uint32_t)min(k0 + RPW * i + vrow, S - 1) * RB;
            tl.v[i] = __builtin_nontemporal_load((const u32x3 *)(vbase + row + voff));
        }
    };

    const float cs = f.scale * kLog2e;
    const int64_t mrow = b * f.m_sb + (h0 + min(l16, gv - 1)) * f.m_sh;
    const half8_t neg_magic = {(_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic,
                               (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic};
    float m = -INFINITY;  // running max of head l16 (log2 domain)
    float lsum = 0.0f;    // running sum of head l16
    f32x4 acc[NB][2];     // O^T[32 blk + 16 h + 4 q4 + i][head l16], unnormalised
#pragma unroll
    for (int t = 0; t < NB; ++t) acc[t][0] = acc[t][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    uint8_t *vt = s_v[w];

    auto compute = [&](int step, const Tile &tl) {
        const int k0 = kbeg + step * kStep + 32 * w;
        // ---- V rows of the step into LDS (k-slot order) with their scales ----
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int r = RPW * i + vrow;
            const int rho = 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
            uint32_t q0, q1, db;
            extract12(tl.v[i], vblk & 1, q0, q1, db);
            *(u32x2 *)(vt + rho * VP + 8 * sub) = u32x2{q0 ^ kFlip, q1 ^ kFlip};
            if (vpart == 0) s_dv[w][vblk][rho] = h2f(db);
        }
        // ---- scores ----
        half8_t ka[2][NB];
        float dk[2][NB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                uint32_t q0, q1, db;
                extract12(tl.k[kb][t], t & 1, q0, q1, db);
                const u32x2 lo = magic4(q0 ^ kFlip), hi = magic4(q1 ^ kFlip);
                ka[kb][t] = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
                dk[kb][t] = h2f(db);
            }
        if (q4 == 0) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int t = 0; t < NB; ++t) s_d[w][16 * kb + l16][t] = dk[kb][t];
        }
        __builtin_amdgcn_wave_barrier();  // LDS written by this wave before it is read
        float sc[2][4];
        float cm = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 sum4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const f32x4 c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][t], qb[t], z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) sum4[i] = fmaf(s_d[w][16 * kb + 4 * q4 + i][t], c4[i] - cq[t], sum4[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + 16 * kb + 4 * q4 + i;
                float x = sum4[i] * cs;
                bool blocked = key >= kend || l16 >= gv;
                if (MASK != 0) {
                    const int64_t mi = mrow + (int64_t)min(key, S - 1) * f.m_ss;
                    if (MASK == 1) blocked = blocked || !((const uint8_t *)f.mask)[mi];
                    else x = fmaf(((const float *)f.mask)[mi], kLog2e, x);
                }
                x = blocked ? -INFINITY : x;
                sc[kb][i] = x;
                cm = fmaxf(cm, x);
            }
        }
        // ---- online softmax of head l16 over the step ----
        cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
        cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
        const float mnew = fmaxf(m, cm);
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = mnew == -INFINITY ? 1.0f : fast_exp2(m - mnew);  // m = -inf: 0
        m = mnew;
        float ps = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[kb][i] = fast_exp2(sc[kb][i] - msub);  // -inf -> 0
                ps += sc[kb][i];
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        lsum = fmaf(lsum, alpha, ps);
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                acc[t][0] *= alpha;
                acc[t][1] *= alpha;
            }
        }
        // ---- P.V on MFMA ----
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const f32x4 dv0 = *(const f32x4 *)&s_dv[w][t][8 * q4], dv1 = *(const f32x4 *)&s_dv[w][t][8 * q4 + 4];
            u32x4 pw;  // k-slot e = 4 kb + i: key 16 kb + 4 q4 + i, scale of k-slot row 8 q4 + e
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                pw[j] = pack_h2(sc[0][2 * j] * dv0[2 * j], sc[0][2 * j + 1] * dv0[2 * j + 1]);
                pw[j + 2] = pack_h2(sc[1][2 * j] * dv1[2 * j], sc[1][2 * j + 1] * dv1[2 * j + 1]);
            }
            const half8_t bp = __builtin_bit_cast(half8_t, pw);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x2 raw = read_tr8(vt + (8 * q4 + (l16 >> 1)) * VP + 32 * t + 16 * h + 8 * (l16 & 1));
                const uint32_t r0 = raw[0], r1 = raw[1];  // through scalars (see extract12's caller)
                const u32x2 lo = magic4(r0), hi = magic4(r1);
                const half8_t av = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
                acc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bp, acc[t][h], 0, 0, 0);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_magic, bp, acc[t][h], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();  // LDS read before the next step overwrites it
    };

    // The loads are unconditional (rows past the split are clamped reads of valid rows): with a
    // branch around them the compiler's load counters cannot tell which loads are in flight and
    // would wait for the prefetched step too.
    Tile ta, tb;
    load(0, ta);
    for (int st = 0; st < nsteps; st += 2) {
        load(st + 1, tb);
        __builtin_amdgcn_sched_barrier(0);
        compute(st, ta);
        load(st + 2, ta);
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < nsteps) compute(st + 1, tb);
    }

    // ---- combine the four waves ----
    if (lane < G) {
        s_m[w][lane] = m;
        s_l[w][lane] = lsum;
    }
    if (l16 < G) {
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_o[w][l16][32 * t + 16 * h + 4 * q4 + i] = acc[t][h][i];
    }
    __syncthreads();
    for (int e = tid; e < gv * D; e += 256) {
        const int h = e / D, d = e % D;
        const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float o = 0.0f, L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float wg = s_m[ww][h] == -INFINITY ? 0.0f : fast_exp2(s_m[ww][h] - M);
            o = fmaf(wg, s_o[ww][h][d], o);
            L = fmaf(wg, s_l[ww][h], L);
        }
        const int64_t row = b * f.H + h0 + h;
        if (a.nsplit == 1) {
            ((_Float16 *)f.o)[row * D + d] = (_Float16)(L > 0.0f ? o / L : 0.0f);
            if (f.lse && d == 0) ((float *)f.lse)[row] = L > 0.0f ? (M + log2f(L)) * kLn2 : INFINITY;
        } else {
            const int64_t pr = row * a.nsplit + split;
            a.part_o[pr * D + d] = o;
            if (d == 0) {
                a.part_ml[pr * 2 + 0] = M;
                a.part_ml[pr * 2 + 1] = L;
            }
        }
    }
    if (a.nsplit > 1 && a.counters) gtdecode::finish_split<_Float16, D>(a, bkg, b * f.H + h0, gv);
}

// Reductions over lanes l, l ^ 16 and l, l ^ 32 with v_permlane16/32_swap (VALU, no LDS).
__device__ inline float max_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float max_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float sum_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Streaming variant: each wavefront's 32 K rows and 32 V rows of a step (34 D / 32 bytes each,
// so a step's rows are one contiguous span per tensor) are read with 16-byte loads, 1 KiB per
// instruction, so every request the memory pipeline sees is a whole run of cache lines, and
// written raw into the wave's LDS tile; the next step's loads are in flight in registers while
// this step is computed from LDS.  Operands come from the raw rows:
//   K (scores): the 12-byte windows of the register variant, read as dwords from LDS;
//   V^T (P.V MFMA A operand): byte e of lane (g = l/16, m = l%16) is row key(g, e) of dim
//     32 blk + 16 h + m, one ds_read_u8 each, packed as fp16 (qs + 1152);
//   the V block scales are read once per (row, block) into a small table, zero for keys past
//     the end (their rows may be clamped copies).
// Needs 16-byte aligned K/V bases and (b, kv head) slices of a multiple of 16 bytes.
template <int D, int G, int MASK>
__global__ __launch_bounds__(256, 2) void decode_q8_lds_kernel(DecodeArgs a) {
    constexpr int NB = D / 32;                // Q8_0 blocks per row
    constexpr int RB = NB * 34;               // bytes per row
    constexpr int TB = 32 * RB;               // bytes of a wave's 32 rows (a multiple of 16)
    constexpr int NL = (TB + 1023) / 1024;    // 16-byte loads per lane and tile
    constexpr int TAIL = (TB % 1024) / 16;    // lanes of the last load that fall inside the tile (0: all)
    constexpr int SV = NB * 32 / 64;          // V scales read per lane and step
    __shared__ __attribute__((aligned(16))) uint8_t s_raw[4][2][NL * 1024];  // [wave][K, V]
    __shared__ __attribute__((aligned(16))) float s_dv[4][NB][32];       // V scales by row
    __shared__ float s_m[4][G], s_l[4][G];
    static_assert(G * D * 4 <= 2 * NL * 1024, "s_o alias");

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    // blockIdx.x = (sequence, kv head, head group), blockIdx.y = split: workgroups are dealt to
    // the XCDs round robin by linear index, so an XCD gets whole (sequence, kv head) slices rather
    // than one split position of every other slice (measured 50.2 against 50.6 us); the kv
    // head's gtot query heads run in groups of G (the last group may hold fewer, gv; its padding
    // columns are blocked)
    const int split = blockIdx.y;
    const int gtot = (int)(f.H / f.Hkv), ngrp = (gtot + G - 1) / G;
    const int64_t bkg = blockIdx.x, bk = bkg / ngrp, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int hg = (int)(bkg % ngrp);
    const int h0 = (int)hk * gtot + hg * G, gv = min(G, gtot - hg * G);
    const int S = (int)f.S;
    const int span = ((S + kStep - 1) / kStep + a.nsplit - 1) / a.nsplit * kStep;
    const int kbeg = split * span, kend = min(attn_decode_end(f, b), kbeg + span);
    const int nsteps = kend > kbeg ? (kend - kbeg + kStep - 1) / kStep : 0;

    half8_t qb[NB];
    f32x4 c0[NB];  // -1152 x the block sums of each head's query: the score MFMA's initial value
    {
        const _Float16 *qr = (const _Float16 *)f.q + b * f.q_sb + (h0 + min(l16, gv - 1)) * f.q_sh + 8 * q4;
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const u32x4 x = *(const u32x4 *)(qr + 32 * t);
            qb[t] = __builtin_bit_cast(half8_t, x);
        }
    }
    const half8_t neg_magic = {(_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic,
                               (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic, (_Float16)-kMagic};
#pragma unroll
    for (int t = 0; t < NB; ++t)
        c0[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_magic, qb[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);

    const int64_t slice = (b * f.Hkv + hk) * (int64_t)S * RB;
    const uint8_t *kbase = (const uint8_t *)f.k + slice;
    const uint8_t *vbase = (const uint8_t *)f.v + slice;
    const uint32_t last16 = (uint32_t)S * RB - 16;  // last 16-byte piece of the slice
    // the lane's pieces of the wave's K and V tiles of `step` (pieces past the slice read its last
    // piece; lanes of the last load past the tile re-read lane 0's line, adding no requests, and land
    // in the LDS tile's slack, never read)
    u32x4 rk[NL], rv[NL];
    auto load = [&](int step) {
        const uint32_t t0 = (uint32_t)(kbeg + step * kStep + 32 * w) * RB;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const bool spare = TAIL != 0 && j == NL - 1 && lane >= TAIL;
            const uint32_t off = min(t0 + 1024u * j + (spare ? 0u : 16u * lane), last16);
            rk[j] = __builtin_nontemporal_load((const u32x4 *)(kbase + off));
            rv[j] = __builtin_nontemporal_load((const u32x4 *)(vbase + off));
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            *(u32x4 *)&s_raw[w][0][1024 * j + 16 * lane] = rk[j];
            *(u32x4 *)&s_raw[w][1][1024 * j + 16 * lane] = rv[j];
        }
    };

    auto in_row = [](int blk, int part) { return 34 * blk + 8 * part - ((blk & 1) ? 2 : 0); };
    const float cs = f.scale * kLog2e;
    const int64_t mrow = b * f.m_sb + (h0 + min(l16, gv - 1)) * f.m_sh;
    float m = -INFINITY, lsum = 0.0f;
    f32x4 acc[NB][2];
#pragma unroll
    for (int t = 0; t < NB; ++t) acc[t][0] = acc[t][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int step) {
        const int k0 = kbeg + step * kStep + 32 * w;
        const uint8_t *kt = s_raw[w][0];
        const uint8_t *vt = s_raw[w][1];
        // ---- V block scales of the step (zero past the end: those rows may be clamped copies) ----
#pragma unroll
        for (int j = 0; j < SV; ++j) {
            const int idx = lane + 64 * j, r = idx & 31, t = idx >> 5;
            const float d = h2f(*(const uint16_t *)(vt + r * RB + 34 * t));
            s_dv[w][t][r] = k0 + r < kend ? d : 0.0f;
        }
        // ---- scores ----
        // K block scales of the C rows (keys 16 kb + 4 q4 + i): d of block 2p is the low half of the
        // dword at 68 p of the row, d of block 2p + 1 the high half of the dword 32 bytes later
        float dk[2][4][NB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t *row = (const uint32_t *)(kt + (16 * kb + 4 * q4 + i) * RB);
#pragma unroll
                for (int p2 = 0; p2 < NB / 2; ++p2) {
                    dk[kb][i][2 * p2] = h2f(row[17 * p2] & 0xffffu);
                    dk[kb][i][2 * p2 + 1] = h2f(row[17 * p2 + 8] >> 16);
                }
            }
        half8_t ka[2][NB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const uint32_t *p = (const uint32_t *)(kt + (16 * kb + l16) * RB + in_row(t, q4));
                const u32x3 win = {p[0], p[1], p[2]};
                uint32_t q0, q1, db;
                extract12(win, t & 1, q0, q1, db);
                const u32x2 lo = magic4(q0 ^ kFlip), hi = magic4(q1 ^ kFlip);
                ka[kb][t] = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
            }
        float sc[2][4];
        float cm = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 sum4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const f32x4 c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][t], qb[t], c0[t], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) sum4[i] = fmaf(dk[kb][i][t], c4[i], sum4[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + 16 * kb + 4 * q4 + i;
                float x = sum4[i] * cs;
                bool blocked = key >= kend || l16 >= gv;
                if (MASK != 0) {
                    const int64_t mi = mrow + (int64_t)min(key, S - 1) * f.m_ss;
                    if (MASK == 1) blocked = blocked || !((const uint8_t *)f.mask)[mi];
                    else x = fmaf(((const float *)f.mask)[mi], kLog2e, x);
                }
                x = blocked ? -INFINITY : x;
                sc[kb][i] = x;
                cm = fmaxf(cm, x);
            }
        }
        cm = max_x16(cm);
        cm = max_x32(cm);
        const float mnew = fmaxf(m, cm);
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = mnew == -INFINITY ? 1.0f : fast_exp2(m - mnew);
        m = mnew;
        float ps = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[kb][i] = fast_exp2(sc[kb][i] - msub);
                ps += sc[kb][i];
            }
        ps = sum_x16(ps);
        ps = sum_x32(ps);
        lsum = fmaf(lsum, alpha, ps);
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                acc[t][0] *= alpha;
                acc[t][1] *= alpha;
            }
        }
        // ---- P.V: k-slot e of lane group q4 is key 16(e/4) + 4 q4 + e%4 ----
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const f32x4 dv0 = *(const f32x4 *)&s_dv[w][t][4 * q4], dv1 = *(const f32x4 *)&s_dv[w][t][16 + 4 * q4];
            u32x4 pw;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                pw[j] = pack_h2(sc[0][2 * j] * dv0[2 * j], sc[0][2 * j + 1] * dv0[2 * j + 1]);
                pw[j + 2] = pack_h2(sc[1][2 * j] * dv1[2 * j], sc[1][2 * j + 1] * dv1[2 * j + 1]);
            }
            const half8_t bp = __builtin_bit_cast(half8_t, pw);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint8_t *col = vt + 34 * t + 2 + 16 * h + l16;
                uint32_t by[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) by[e] = col[(16 * (e >> 2) + 4 * q4 + (e & 3)) * RB];
                u32x4 av;
#pragma unroll
                for (int j = 0; j < 4; ++j) av[j] = (by[2 * j] | (by[2 * j + 1] << 16)) ^ 0x64806480u;
                acc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, av), bp, acc[t][h], 0,
                                                                   0, 0);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_magic, bp, acc[t][h], 0, 0, 0);
        }
    };

    // The wave's LDS tile holds the step being computed; the registers hold the next one in
    // flight.  Inside the loop the loads are unconditional (clamped) so the compiler's load
    // counters stay exact; the last step is peeled off so that no workgroup fetches the rows
    // past its split (the next split's first step, which another XCD's L2 fetches again).
    // Wave priority follows the step (progress_priority: the two workgroups on a CU stay level).
    if (nsteps > 0) {
        load(0);
        __builtin_amdgcn_s_setprio(3);
        for (int st = 0; st + 1 < nsteps; ++st) {
            progress_priority(st + 1);
            __builtin_amdgcn_wave_barrier();  // the previous step's LDS reads come before the overwrite
            stage();
            __builtin_amdgcn_sched_barrier(0);
            load(st + 1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_wave_barrier();
            compute(st);
        }
        __builtin_amdgcn_wave_barrier();
        stage();
        __builtin_amdgcn_wave_barrier();
        compute(nsteps - 1);
    }
    __builtin_amdgcn_s_setprio(3);  // the combine and the merge are the launch's tail

    // ---- combine the four waves (each wave's partial O goes into its own LDS tile) ----
    constexpr int WSTRIDE = 2 * NL * 1024 / 4;  // floats per wave region
    float *my_o = reinterpret_cast<float *>(&s_raw[w][0][0]);
    __builtin_amdgcn_wave_barrier();
    if (lane < G) {
        s_m[w][lane] = m;
        s_l[w][lane] = lsum;
    }
    if (l16 < G) {
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) my_o[l16 * D + 32 * t + 16 * h + 4 * q4 + i] = acc[t][h][i];
    }
    __syncthreads();
    const float *o_all = reinterpret_cast<const float *>(&s_raw[0][0][0]);
    for (int e = tid; e < gv * D; e += 256) {
        const int h = e / D, d = e % D;
        const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float o = 0.0f, L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float wg = s_m[ww][h] == -INFINITY ? 0.0f : fast_exp2(s_m[ww][h] - M);
            o = fmaf(wg, o_all[ww * WSTRIDE + h * D + d], o);
            L = fmaf(wg, s_l[ww][h], L);
        }
        const int64_t row = b * f.H + h0 + h;
        if (a.nsplit == 1) {
            ((_Float16 *)f.o)[row * D + d] = (_Float16)(L > 0.0f ? o / L : 0.0f);
            if (f.lse && d == 0) ((float *)f.lse)[row] = L > 0.0f ? (M + log2f(L)) * kLn2 : INFINITY;
        } else {
            const int64_t pr = row * a.nsplit + split;
            a.part_o[pr * D + d] = o;
            if (d == 0) {
                a.part_ml[pr * 2 + 0] = M;
                a.part_ml[pr * 2 + 1] = L;
            }
        }
    }
    if (a.nsplit > 1 && a.counters) gtdecode::finish_split<_Float16, D>(a, bkg, b * f.H + h0, gv);
}

template <int D, bool LDS>
const void *q8_kernel_d(const AttnFwdArgs &f, int G) {
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
#define GT_QK(K, GG) \
    (mode == 0 ? (const void *)K<D, GG, 0> : mode == 1 ? (const void *)K<D, GG, 1> : (const void *)K<D, GG, 2>)
#define GT_QG(GG) (LDS ? GT_QK(decode_q8_lds_kernel, GG) : GT_QK(decode_q8_mfma_kernel, GG))
    switch (G) {
        case 1: return GT_QG(1);
        case 2: return GT_QG(2);
        case 4: return GT_QG(4);
        case 8: return GT_QG(8);
        default: return nullptr;
    }
#undef GT_QG
#undef GT_QK
}

// The streaming kernel reads 16-byte pieces of each (b, kv head) slice: bases 16-byte aligned and
// slices a multiple of 16 bytes.
bool q8_stream_ok(const AttnFwdArgs &f) {
    const int64_t slice = f.S * (f.D / 32 * 34);
    return slice % 16 == 0 && (uintptr_t)f.k % 16 == 0 && (uintptr_t)f.v % 16 == 0;
}

const void *q8_kernel(const AttnFwdArgs &f) {
    const int G = decode_head_tile(f.H / f.Hkv, kDecodeQ8MaxTile);
    if (q8_stream_ok(f)) return f.D == 128 ? q8_kernel_d<128, true>(f, G) : q8_kernel_d<64, true>(f, G);
    return f.D == 128 ? q8_kernel_d<128, false>(f, G) : q8_kernel_d<64, false>(f, G);
}

// Workgroups of `kernel` the device runs at once (CUs x resident workgroups per CU), cached.
int64_t resident_slots(const void *kernel) {
    static std::mutex mu;
    static std::map<std::pair<int, const void *>, int64_t> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dev, kernel});
    if (it != cache.end()) return it->second;
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, 256, 0) != hipSuccess || per <= 0) per = 2;
    const int64_t slots = (int64_t)cus * per;
    cache[{dev, kernel}] = slots;
    return slots;
}

}  // namespace

// The merge kernel is shared with the fp16 decode path.
hipError_t launch_attn_decode_merge(const DecodeArgs &a, int out_dtype, hipStream_t s);

int attn_decode_q8_splits(const AttnFwdArgs &f) {
    const void *kernel = q8_kernel(f);
    const int64_t slots = kernel ? resident_slots(kernel) : 512;
    const int64_t steps = (f.S + kStep - 1) / kStep;
    return decode_split_count(decode_units(f.B, f.H, f.Hkv, kDecodeQ8MaxTile), steps, slots, std::min<int64_t>(64, steps));
}

bool attn_decode_q8_supported(const AttnFwdArgs &f, int q_dtype) {
    if (q_dtype != GT_F16 || f.out_dtype != GT_F16) return false;
    if (f.L != 1 || f.S <= 0 || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    if (f.S >= (1LL << 30) || f.S * (f.D / 32 * 34) > 0xffffffffLL) return false;  // 32-bit offsets
    // any number of query heads per kv head, in groups of up to 8
    if (decode_units(f.B, f.H, f.Hkv, kDecodeQ8MaxTile) > 65535) return false;  // grid.y (register kernel)
    if (f.q_sh % 8 != 0 || f.q_sb % 8 != 0 || (uintptr_t)f.q % 16 != 0) return false;
    // K/V are whole dense Q8_0 tensors; rows are 4-byte aligned when the base is
    for (const void *p : {f.k, f.v}) if ((uintptr_t)p % 8 != 0) return false;
    return true;
}

hipError_t launch_attn_decode_q8(const DecodeArgs &a, hipStream_t s) {
    const void *kernel = q8_kernel(a.f);
    if (!kernel) return hipErrorInvalidValue;
    const unsigned units = (unsigned)decode_units(a.f.B, a.f.H, a.f.Hkv, kDecodeQ8MaxTile);
    // streaming kernel: (units, splits); register kernel: (splits, units)
    const dim3 grid = q8_stream_ok(a.f) ? dim3(units, (unsigned)a.nsplit) : dim3((unsigned)a.nsplit, units);
    void *args[] = {(void *)&a};
    hipError_t e = hipLaunchKernel(kernel, grid, dim3(256), args, 0, s);
    // one split, or the last split merged in the kernel: the kernel wrote the output
    if (e != hipSuccess || a.nsplit == 1 || a.counters) return e;
    return launch_attn_decode_merge(a, GT_F16, s);
}
