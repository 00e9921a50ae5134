// Fused attention forward on gfx950 MFMA (fp16 / bf16 inputs, fp32 softmax and accumulation).
//
// Replaces the reference's scalar fp64 loop (csrc/gt_ops_nn.cpp:2423-2525) for L > 1 with
// the same semantics: scale, top-left causal mask, bool/additive mask, rows with nothing to
// attend to -> 0, output rounded from fp32 to the input dtype.
//
// Workgroup: 4 wavefronts, query tiles of BM = 128 rows (32 per wavefront), two workgroups per
// CU (two wavefronts per SIMD), so each K/V tile brought into LDS serves 128 queries.  A workgroup runs the query tiles p and
// nq-1-p of one head one after the other: under the causal mask their key ranges add up to
// the same length for every p, so all workgroups carry equal work.  K/V tiles of BN = 64 rows
// stream through NST LDS stages: global_load_lds_dwordx4 writes tile s+NST-1 straight into LDS
// (no staging registers) while tile s is computed, with one barrier per tile; the loads are
// issued after tile s's S MFMAs (2-3% faster on the prefill workload than right after the
// barrier).  Tiles are
// unpadded; 16-byte chunk c of row r sits at chunk c ^ f(r), which keeps both the row reads of
// K (16 rows per LDS cycle) and the transposed reads of V (4 rows x 4 chunks per cycle) free of
// bank conflicts on the 64-bank LDS: f(r) = (r ^ 4r) mod 16 for 16-chunk rows (D = 128),
// f(r) = (2r + r/4) mod 8 for 8-chunk rows (D = 64).
// Per tile and wavefront:
//   S^T (keys x queries) = K . Q^T    v_mfma_f32_32x32x16_{f16,bf16}; Q^T stays in registers
//                                      as the B operand, K rows come from LDS (ds_read_b128).
//   online softmax in the log2 domain: every lane owns one query row (lane % 32) and 32 of
//   its scores, so max/sum are in-lane plus one exchange between the two wave halves
//   (v_permlane32_swap).  O and l are rescaled only when a row's max grows by more than
//   kLazy (the result O / l does not depend on the reference point).
//   O^T (d x queries) += V^T . P^T    P^T is the S^T accumulator converted in place (the
//                                      MFMA's k index is permuted to match the accumulator
//                                      layout); V^T fragments come from the row-major V tile
//                                      through ds_read_b64_tr_b16.
// bf16 P is split into hi + lo bf16 parts (two MFMAs) so the probabilities keep ~16 bits.
// Causal tiles above the diagonal are never loaded.
// Dropout (DROP): P.V takes P times the element's multiplier (gt_philox.h); the 8 scores a lane
// packs for one k-step are two groups of 4 consecutive keys, one Philox block each.  The
// running sum (and the log-sum-exp) keeps the undropped probabilities.

#include "attn_common.h"
#include "gt_internal.h"
#include "mfma_util.h"
#include "lds_dma.h"
#include "gt_rope_math.h"

#include <cmath>
#include <type_traits>

namespace {

// Wavefronts per workgroup and K/V tile stages in LDS.  4 wavefronts (128 query rows) and two
// workgroups per CU: the two run their tiles independently (a workgroup's barrier does not hold
// the other), which overlaps one's softmax with the other's MFMAs better than 8 wavefronts in
// lockstep (measured: 3% for D = 128, 9% for the D = 64 training forward).  LDS per workgroup:
// NST = 2 stages x 2 tiles of BN x D, 64 KB for both head sizes.
template <int D>
constexpr int nw_of() { return 4; }
template <int D>
constexpr int nst_of() { return 2; }
template <int D>
constexpr int bm_of() { return 32 * nw_of<D>(); }  // query rows per tile
// keys per K/V tile: 64, or 128 for head size 64 (a tile of 64 keys x 64 dims is too little work
// per barrier)
template <int D>
constexpr int bn_of() { return D == 64 ? 128 : 64; }
constexpr float kLazy = 8.0f;   // rescale threshold, log2 domain: probabilities stay <= 256

// p = 2^(fma(s, c, -m)) rounds the product s c only once, after subtracting m, while m itself
// comes from the rounded product of the row max; the two differ by up to half an ulp of m.
// That is below 2^-4 while |m| < 2^20 and is ignored there.  Beyond it (an additive mask of
// -1e9 on every key of a row puts m near -1.4e9, where an ulp is 128) the reference point
// moves above the max by |m| 2^-21 (more than that rounding error), and a tile only keeps the
// reference point when its max lies |m| 2^-22 below the usual threshold, so that no
// probability exceeds 2^kLazy: such rows give finite results (0 where every probability
// underflows, the rule for a row with nothing visible).
__device__ inline float huge_margin(float x) {
    const float ax = fabsf(x);
    return ax >= 0x1p20f ? ax * 0x1p-21f : 0.0f;
}
using namespace gtmfma;

template <typename T>
__device__ inline void store4(T *dst, float a, float b, float c, float d) {
    u32x2 v = {Mfma<T>::pack(a, b), Mfma<T>::pack(c, d)};
    *(u32x2 *)dst = v;
}

template <int D>
__device__ inline int swz(int r) {
    if constexpr (D == 128) return (r ^ (r << 2)) & 15;
    return (2 * r + (r >> 2)) & 7;
}

// max of three floats in one v_maximum3_f32 (fmaxf would first quiet each MFMA result with a
// v_max_f32 x, x, x).  Compiler-visible rather than assembly: a VALU read of an MFMA result
// needs wait states that the compiler only places around instructions it can see.  A NaN score
// makes the tile's max NaN (v_max3_f32 would skip it); that row's output is NaN either way.
__device__ inline float max3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// RoPE of the lane's query row as it is loaded (all D dims rotated): q[t] holds dims
// 16t + 8 half + 0..7.  The same float32 rotation and rounding as the rope kernel (gt_rope), so
// the result equals attention of gt_rope's output.  NORMAL pairs (2i, 2i+1) lie inside one
// 8-dim group; NeoX pairs (i, i + D/2) lie D/32 groups apart in the same lane.
template <typename T, int D>
__device__ inline void rope_rows(typename Mfma<T>::V8 *q, const float2 *tab, int neox, int half) {
    constexpr int DT = D / 16, TP = D / 32;
    if (!neox) {
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float2 cs = tab[(16 * t + 8 * half + e) >> 1];
                const float lo = (float)q[t][e], hi = (float)q[t][e + 1];
                q[t][e] = (T)rope_rot_lo(lo, hi, cs);
                q[t][e + 1] = (T)rope_rot_hi(lo, hi, cs);
            }
    } else {
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float2 cs = tab[16 * t + 8 * half + e];
                const float lo = (float)q[t][e], hi = (float)q[t + TP][e];
                q[t][e] = (T)rope_rot_lo(lo, hi, cs);
                q[t + TP][e] = (T)rope_rot_hi(lo, hi, cs);
            }
    }
}

// Keys covered by query tile qt: the sequence's keys, or (causal) up to the tile's last row,
// whose position is qpos + qt*BM + BM-1.
template <bool CAUSAL, int BM, int BN>
__device__ inline int key_tiles(int qt, int nkv, int qpos) {
    const int kv_end = CAUSAL ? min(qt * BM + BM + qpos, nkv) : nkv;
    return kv_end > 0 ? (kv_end + BN - 1) / BN : 0;
}

// MASK: 0 = none, 1 = bool bytes, 2 = additive float, 4 = additive float that does not depend
// on the query row (key padding: the tile's mask row travels to LDS with the K/V tile),
// 5 / 6 = bool / float with contiguous keys and 4-key aligned rows: a lane's 4 consecutive keys
// in one 4- / 16-byte load, issued with the tile's DMA so that they land during S = K.Q^T.
// (dropout with a per-element mask: one workgroup per CU is the guaranteed minimum, so that the
// Philox state does not spill)
// HILO (fp16 training forwards, with and without dropout): P enters P.V as hi + lo fp16 operands
// and the row sums add the float32 probabilities, as the bf16 kernels do, so that the float32
// output (whose rowsum(dO.O) forms dS) and the log-sum-exp the backward recomputes P from are
// exact to ~22 bits instead of fp16's 11.
template <typename T, int D, bool CAUSAL, int MASK, bool ROPE = false, bool DROP = false, bool HILO = false>
__global__ __launch_bounds__(64 * nw_of<D>(), DROP && (MASK == 1 || MASK == 2 || MASK >= 5) ? 1 : 8 / nw_of<D>()) void prefill_fwd_kernel(
    AttnFwdArgs a, int nq, int npairs) {
    constexpr int NW = nw_of<D>(), BM = bm_of<D>(), NST = nst_of<D>(), BN = bn_of<D>();
    constexpr int NKB = BN / 32;  // 32-key blocks per tile
    using M = Mfma<T>;
    using V8 = typename M::V8;
    constexpr int DT = D / 16;             // k-steps of S^T = K.Q^T
    constexpr int DB = D / 32;             // d blocks of O^T
    constexpr int CH = D / 8;              // 16-byte chunks per row
    constexpr int TILE = BN * D;           // elements per tile
    constexpr int NPW = BN * CH / 64 / NW; // 1 KB wave loads per operand, wave and tile
    constexpr bool MROW = MASK == 4;
    constexpr bool MVEC = MASK >= 5;                     // per-element mask, 4 keys per load
    constexpr bool MBOOL = MASK == 1 || MASK == 5;
    constexpr int PER = 2 * NPW + (MROW ? BN / 64 : 0);  // loads per wave and tile (K, V, mask row)
    static_assert(NPW >= 1 && PER * (NST - 2) < 64, "tile split");
    static_assert(BN % 64 == 0, "mask row: one key per lane and load");
    __shared__ __attribute__((aligned(1024))) T sK[NST][TILE];
    __shared__ __attribute__((aligned(1024))) T sV[NST][TILE];
    __shared__ __attribute__((aligned(16))) float sMk[MROW ? NST : 1][BN];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wavefront index, uniform
    const int lrow = lane & 31, half = lane >> 5;
    const int g16 = lane >> 4, i16 = lane & 15;
    const int64_t BH = a.B * a.H;
    // Workgroups are dealt to the 8 XCDs round robin (x % 8); when the heads split evenly,
    // XCD x takes heads [x*BH/8, (x+1)*BH/8), so their K/V stay in its own L2.
    int pair;
    int64_t bh;
    if (BH % 8 == 0) {
        const int64_t hpx = BH / 8, i = blockIdx.x / 8;
        pair = (int)(i % npairs);
        bh = (int64_t)(blockIdx.x % 8) * hpx + i / npairs;
    } else {
        pair = (int)(blockIdx.x % npairs);
        bh = (int64_t)blockIdx.x / npairs;
    }
    const int64_t b = bh / a.H, h = bh % a.H, hk = h / (a.H / a.Hkv);
    const int L = (int)a.L, S = (int)a.S;
    // keys present for this sequence and the position of its query row 0 (KV cache; the
    // reference operator: S and 0)
    const int nkv = attn_kv_len(a, b), qpos = attn_q_pos(a, b);
    const int qa = nq - 1 - pair, qb = pair;  // the heavier tile first
    const int nparts = qa == qb ? 1 : 2;
    const int na = key_tiles<CAUSAL, BM, BN>(qa, nkv, qpos);
    const int total = na + (nparts == 2 ? key_tiles<CAUSAL, BM, BN>(qb, nkv, qpos) : 0);

    const T *kbase = (const T *)a.k + b * a.k_sb + hk * a.k_sh;
    const T *vbase = (const T *)a.v + b * a.v_sb + hk * a.v_sh;
    const float c = a.scale * kLog2e;  // raw score -> log2 domain
    const float inv_scale = 1.0f / a.scale;
    const float dscale = DROP ? (float)a.drop.scale : 1.0f;
    const uint64_t dblocks = (uint64_t)((a.S + 3) / 4);  // Philox blocks per attention row

    // Flat step s (key tile s of part 0, then key tile s - na of part 1) goes to stage s % NST;
    // wave w issues NPW 1 KB loads per operand: lane `lane` of load n fills 16-byte slot
    // (w*NPW + n)*64 + lane = row*CH + (col ^ swz<D>(row)).  Rows past S repeat row S-1 (finite
    // values, masked to -inf / weight 0 below).  Byte offsets from the (b, kv head) base fit
    // 32 bits (checked by the launcher).
    const uint32_t k_row = (uint32_t)a.k_ss * 2, v_row = (uint32_t)a.v_ss * 2;
    int lrow_n[NPW];
    uint32_t lcol_n[NPW];
#pragma unroll
    for (int n = 0; n < NPW; ++n) {
        const int slot = (w * NPW + n) * 64 + lane;
        lrow_n[n] = slot / CH;
        lcol_n[n] = 16u * (uint32_t)((slot % CH) ^ swz<D>(slot / CH));
    }
    uint32_t kofs_n[NPW], vofs_n[NPW];  // lane offsets within a full tile
#pragma unroll
    for (int n = 0; n < NPW; ++n) {
        kofs_n[n] = (uint32_t)lrow_n[n] * k_row + lcol_n[n];
        vofs_n[n] = (uint32_t)lrow_n[n] * v_row + lcol_n[n];
    }
    const float *mrow = MROW ? (const float *)a.mask + b * a.m_sb + h * a.m_sh : nullptr;
    auto issue = [&](int step) {
        const int kt = step < na ? step : step - na;
        const int st = step % NST;
        if constexpr (MROW) {
            // the mask values of keys kt*BN .. +63 (keys past S repeat key S-1); every wave writes
            // the same row, which keeps the loads per wave and tile uniform and needs no exec mask
#pragma unroll
            for (int c = 0; c < BN / 64; ++c)
                lds_dma4(lds_addr(&sMk[st][64 * c]), mrow, (uint32_t)min(kt * BN + 64 * c + lane, S - 1) * (uint32_t)a.m_ss * 4u);
        }
        const uint32_t dk = lds_addr(&sK[st][0]) + w * NPW * 1024;
        const uint32_t dv = lds_addr(&sV[st][0]) + w * NPW * 1024;
        if (kt * BN + BN <= S) {
            // a full tile: its offset goes into the scalar base, the lane offsets are fixed
            const char *kb = (const char *)kbase + (uint64_t)(kt * BN) * k_row;
            const char *vb = (const char *)vbase + (uint64_t)(kt * BN) * v_row;
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                lds_dma16(dk + n * 1024, kb, kofs_n[n]);
                lds_dma16(dv + n * 1024, vb, vofs_n[n]);
            }
        } else {
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                const uint32_t key = (uint32_t)min(kt * BN + lrow_n[n], S - 1);
                lds_dma16(dk + n * 1024, kbase, key * k_row + lcol_n[n]);
                lds_dma16(dv + n * 1024, vbase, key * v_row + lcol_n[n]);
            }
        }
    };

    // LDS element offsets of this lane's fragments within a tile, fixed for the whole kernel:
    //   K, k-step t: row lrow (+32 kb), 16-byte chunk 2t + half (the swizzle of row r only
    //   depends on r mod 32 for both D)
    //   V^T, (kb, hs, db): rows (keys) 32kb + 16hs + 4(g16/2) + i16/4 and +8, column
    //   32db + 16(g16%2) + 4(i16%4); with D = 128 the swizzle only depends on row mod 16, so
    //   (kb, hs) is a constant 16(2kb + hs) rows further.
    // the swizzle repeats every 16 rows (D = 128) or 32 rows (D = 64): offsets of the first
    // period, later (kb, hs) groups a constant number of rows further
    constexpr int NV = D == 128 ? DB : 2 * DB;
    int kofs[DT], vofs0[NV], vofs1[NV];
#pragma unroll
    for (int t = 0; t < DT; ++t) kofs[t] = lrow * D + 8 * ((2 * t + half) ^ swz<D>(lrow));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int db = i % DB, g = i / DB;  // g = 2kb + hs (D = 64)
        const int row = 16 * g + 4 * (g16 >> 1) + (i16 >> 2);
        const int col = 32 * db + 16 * (g16 & 1) + 4 * (i16 & 3);
        const int chunk = col >> 3, within = col & 7;
        vofs0[i] = row * D + 8 * (chunk ^ swz<D>(row)) + within;
        vofs1[i] = (row + 8) * D + 8 * (chunk ^ swz<D>(row + 8)) + within;
    }

#pragma unroll
    for (int st = 0; st < NST - 1; ++st)
        if (st < total) issue(st);

    int step = 0;
    for (int part = 0; part < nparts; ++part) {
        const int qt = part == 0 ? qa : qb;
        const int ntiles = part == 0 ? na : total - na;
        const int q0 = qt * BM;
        const int wq0 = q0 + 32 * w;  // first query row of this wavefront
        const int lq = wq0 + lrow;    // this lane's query row

        // Q^T fragments (B operand): lane holds Q[lq][16t + 8*half + 0..7]; rows past L read row L-1
        V8 qf[DT];
        {
            const T *qr = (const T *)a.q + b * a.q_sb + h * a.q_sh + (int64_t)min(lq, L - 1) * a.q_sl + 8 * half;
#pragma unroll
            for (int t = 0; t < DT; ++t) qf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 16 * t));
            if constexpr (ROPE)
                rope_rows<T, D>(qf, (const float2 *)a.rope_q + (int64_t)min(lq, L - 1) * (D / 2), a.rope_neox, half);
            // Wait for Q here: otherwise the compiler's wait for these loads lands inside the tile
            // loop, where it also waits for every K/V tile prefetch issued since.
#pragma unroll
            for (int t = 0; t < DT; ++t) asm volatile("" ::"v"(qf[t]));
        }

        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
        float m = -INFINITY;     // reference point of this lane's row, log2 domain
        float mthr = -INFINITY;  // a tile whose row max exceeds this moves m
        float lsum = 0.0f;    // this lane's share of the running sum
        // dropout: Philox block of keys 0..3 of this lane's row (rows past L draw unused words)
        const uint64_t drow = DROP ? (uint64_t)(bh * a.L + lq) * dblocks : 0;
        // MVEC: element offset of this lane's mask row
        const int64_t mrb = MVEC ? b * a.m_sb + h * a.m_sh + (int64_t)min(lq, L - 1) * a.m_sl : 0;

        for (int j = 0; j < ntiles; ++j, ++step) {
            const int k0 = j * BN;
            // Tile `step` is complete once at most the loads of the tiles issued after it are
            // outstanding (vector memory loads complete in order); the barrier then makes every
            // wavefront's part visible and guarantees stage (step-1) % NST is no longer read.
            const int later = min(NST - 2, total - 1 - step);
            if (later >= 2) wait_vm<2 * PER>();
            else if (later == 1) wait_vm<PER>();
            else wait_vm<0>();
            __syncthreads();
            // head size 64: priority by progress (training forward 2.5 us faster per step); at 128
            // it measured neutral (the two workgroups even out, but each runs slower)
            if constexpr (D <= 64) progress_priority(step);
            const T *cK = sK[step % NST];
            const T *cV = sV[step % NST];
            // MVEC: keys k0 + 32kb + 8g + 4half + 0..3 of this lane's row (starts past the last
            // 4 keys read those: their scores are blocked below)
            f32x4 mvf[MVEC && !MBOOL ? NKB : 1][4];
            uint32_t mvb[MVEC && MBOOL ? NKB : 1][4];
            if constexpr (MVEC) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int64_t at = mrb + min(k0 + 32 * kb + 8 * g + 4 * half, S - 4);
                        if constexpr (MBOOL) mvb[kb][g] = *(const uint32_t *)((const uint8_t *)a.mask + at);
                        else mvf[kb][g] = *(const f32x4 *)((const float *)a.mask + at);
                    }
            }

            // (causal) a wavefront whose rows all precede this tile still runs it: every score
            // is masked to -inf and p = 0; skipping it makes the compiler copy O on every tile
            // ---- S^T = K . Q^T ----
            // MROW: the key-padding row enters as the accumulator's initial value (mask / scale,
            // the raw-score units of the accumulator), so S^T = K.Q^T + mask costs no VALU add
            f32x16 s[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                V8 kf[DT];
#pragma unroll
                for (int t = 0; t < DT; ++t) kf[t] = *(const V8 *)&cK[kofs[t] + 32 * kb * D];
                if constexpr (MROW) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 mv4 = *(const f32x4 *)&sMk[step % NST][32 * kb + 8 * g + 4 * half];
#pragma unroll
                        for (int e = 0; e < 4; ++e) s[kb][4 * g + e] = mv4[e] * inv_scale;
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[kb][i] = 0.0f;
                }
#pragma unroll
                for (int t = 0; t < DT; ++t) s[kb] = M::mma(kf[t], qf[t], s[kb]);
            }

            // the next tile's loads into the stage every wavefront finished with before the barrier
            if (step + NST - 1 < total) issue(step + NST - 1);

            // ---- masks: s[kb][i] is (key = k0 + 32kb + 8(i/4) + 4half + i%4, query = lq) ----
            const bool edge = k0 + BN > nkv || (CAUSAL && k0 + BN - 1 > wq0 + qpos);
            if ((MASK != 0 && !MROW) || edge) {
                // key k0 + 4half + c (c = 32kb + 8(i/4) + i%4, a constant per entry) is visible
                // to this lane's row when c <= vis: one compare per score
                const int vis = min(nkv - 1, CAUSAL ? lq + qpos : nkv - 1) - (k0 + 4 * half);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * half + (i % 4);
                        float x = s[kb][i];
                        if constexpr (MROW) {
                            // the mask row is already in s
                        } else if constexpr (MVEC) {
                            if constexpr (MBOOL) x = (mvb[kb][i / 4] >> (8 * (i % 4))) & 0xffu ? x : -INFINITY;
                            else x = fmaf(mvf[kb][i / 4][i % 4], inv_scale, x);
                        } else if (MASK != 0) {
                            const int64_t mi = b * a.m_sb + h * a.m_sh + (int64_t)min(lq, L - 1) * a.m_sl +
                                               (int64_t)min(key, S - 1) * a.m_ss;
                            if (MASK == 1) {
                                x = ((const uint8_t *)a.mask)[mi] ? x : -INFINITY;
                            } else {
                                x = fmaf(((const float *)a.mask)[mi], inv_scale, x);
                            }
                        }
                        const bool blocked = 32 * kb + 8 * (i / 4) + (i % 4) > vis;
                        s[kb][i] = blocked ? -INFINITY : x;
                    }
                }
            }

            // ---- online softmax ----
            float tmax = max3(s[0][0], s[0][1], s[0][2]);
#pragma unroll
            for (int i = 3; i < 16 * NKB - 1; i += 2) tmax = max3(tmax, s[i / 16][i % 16], s[(i + 1) / 16][(i + 1) % 16]);
            tmax = max3(tmax, s[NKB - 1][15], s[NKB - 1][15]);
            tmax = xhalf_max(tmax);
            // Lazy rescaling: the reference point m of a row only moves when the tile's max
            // exceeds it by more than kLazy, so p = 2^(s c - m) stays below 2^kLazy.  A row with
            // nothing visible yet keeps m = -inf and p = 0 (no branch: the MFMAs below combine
            // the two lanes of each row and run for the whole wave).
            const float tm = tmax * c;
            const bool move = tm > mthr;
            if (!__all(!move)) {
                const float mnew = move ? tm + huge_margin(tm) : m;
                const float alpha = move ? fast_exp2(m - mnew) : 1.0f;  // m = -inf: 0 (O and l are 0)
                lsum *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
                m = mnew;
                mthr = m + kLazy - 0.5f * huge_margin(m);
            }
            const float msub = m == -INFINITY ? 0.0f : m;

            // P^T as B operands: k-step (kb, hs) takes accumulator entries 8hs .. 8hs+7
            V8 pb[NKB][2], pl[NKB][2];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int hs = 0; hs < 2; ++hs) {
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(s[kb][8 * hs + e], c, -msub));
                    if constexpr (DROP) {
                        // keys k0 + 32kb + 16hs + 4half + (0..3, 8..11): blocks g0 and g0 + 2
                        const uint64_t g0 = drow + (uint64_t)((k0 + 32 * kb + 16 * hs + 4 * half) >> 2);
#pragma unroll
                        for (int e = 0; e < 8; ++e) lsum += p[e];
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            const GtWord4 x = gt_philox4x32_10(g0 + 2 * u, a.drop.offset, a.drop.seed);
#pragma unroll
                            for (int e = 0; e < 4; ++e) p[4 * u + e] *= x.w[e] < a.drop.thresh ? dscale : 0.0f;
                        }
                        if constexpr (HILO) pack8_hilo<T>(p, pb[kb][hs], pl[kb][hs]);
                        else pack8<T>(p, pb[kb][hs], pl[kb][hs]);
                    } else if constexpr (M::kSplit) {
                        // bf16: sum the float32 p first; packing consumes them (the residuals are
                        // formed in place)
                        lsum = sum8<T>(p, pb[kb][hs], lsum);
                        pack8<T>(p, pb[kb][hs], pl[kb][hs]);
                    } else if constexpr (HILO) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) lsum += p[e];
                        pack8_hilo<T>(p, pb[kb][hs], pl[kb][hs]);
                    } else {
                        pack8<T>(p, pb[kb][hs], pl[kb][hs]);
                        lsum = sum8<T>(p, pb[kb][hs], lsum);
                    }
                }
            }

            // ---- O^T += V^T . P^T ----
            // d blocks innermost: consecutive MFMAs accumulate into different O blocks, so none
            // waits for the previous one's result (a dependent 32x32x16 chain issues at ~44
            // cycles per MFMA instead of 32)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int hs = 0; hs < 2; ++hs) {
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const int g = 2 * kb + hs;
                        const V8 av = D == 128 ? read_tr8<T>(&cV[vofs0[db] + 16 * g * D], &cV[vofs1[db] + 16 * g * D])
                                               : read_tr8<T>(&cV[vofs0[(g % 2) * DB + db] + 32 * kb * D],
                                                             &cV[vofs1[(g % 2) * DB + db] + 32 * kb * D]);
                        o[db] = M::mma(av, pb[kb][hs], o[db]);
                        if constexpr (M::kSplit || HILO) o[db] = M::mma(av, pl[kb][hs], o[db]);
                    }
                }
            }
        }

        // ---- epilogue: normalise, store O (B,H,L,D) and the log-sum-exp ----
        const float ltot = xhalf_sum(lsum);
        const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
        if (lq < L) {
            T *orow = (T *)a.o + (bh * a.L + lq) * D;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    store4<T>(orow + 32 * db + 8 * g + 4 * half, o[db][4 * g] * inv, o[db][4 * g + 1] * inv,
                              o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
            if (a.lse && half == 0)
                ((float *)a.lse)[bh * a.L + lq] = ltot > 0.0f ? (m + log2f(ltot)) * kLn2 : INFINITY;
            if (a.o32) {
                float *row32 = (float *)a.o32 + (bh * a.L + lq) * D;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 v = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                         o[db][4 * g + 3] * inv};
                        *(f32x4 *)(row32 + 32 * db + 8 * g + 4 * half) = v;
                    }
            }
        }
    }
}

template <typename T, int D>
hipError_t launch_variant(const AttnFwdArgs &a, int nq, int npairs, int64_t grid, hipStream_t s) {
    const int mode = attn_mask_mode(a);
#define GT_PREFILL_LAUNCH(C, MK) \
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, C, MK>), dim3((unsigned)grid), dim3(64 * nw_of<D>()), 0, s, a, nq, npairs)
#define GT_PREFILL_LAUNCH_R(C, MK) \
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, C, MK, true>), dim3((unsigned)grid), dim3(64 * nw_of<D>()), 0, s, a, nq, npairs)
#define GT_PREFILL_LAUNCH_D(C, MK) \
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, C, MK, false, true, std::is_same<T, _Float16>::value>), dim3((unsigned)grid), dim3(64 * nw_of<D>()), 0, s, a, nq, npairs)
#define GT_PREFILL_LAUNCH_X(C, MK) \
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, C, MK, false, false, true>), dim3((unsigned)grid), dim3(64 * nw_of<D>()), 0, s, a, nq, npairs)
    if (a.dropout) {
        if (a.rope_q) return hipErrorInvalidValue;  // dropout runs on unrotated queries only
        if (a.causal) {
            if (mode == 0) GT_PREFILL_LAUNCH_D(true, 0);
            else if (mode == 1) GT_PREFILL_LAUNCH_D(true, 1);
            else if (mode == 4) GT_PREFILL_LAUNCH_D(true, 4);
            else if (mode == 5) GT_PREFILL_LAUNCH_D(true, 5);
            else if (mode == 6) GT_PREFILL_LAUNCH_D(true, 6);
            else GT_PREFILL_LAUNCH_D(true, 2);
        } else {
            if (mode == 0) GT_PREFILL_LAUNCH_D(false, 0);
            else if (mode == 1) GT_PREFILL_LAUNCH_D(false, 1);
            else if (mode == 4) GT_PREFILL_LAUNCH_D(false, 4);
            else if (mode == 5) GT_PREFILL_LAUNCH_D(false, 5);
            else if (mode == 6) GT_PREFILL_LAUNCH_D(false, 6);
            else GT_PREFILL_LAUNCH_D(false, 2);
        }
    } else if (a.rope_q) {
        // fused query RoPE: no mask or a key-padding row (the host rotates q itself otherwise)
        if (mode != 0 && mode != 4) return hipErrorInvalidValue;
        if (a.causal) {
            if (mode == 0) GT_PREFILL_LAUNCH_R(true, 0);
            else GT_PREFILL_LAUNCH_R(true, 4);
        } else {
            if (mode == 0) GT_PREFILL_LAUNCH_R(false, 0);
            else GT_PREFILL_LAUNCH_R(false, 4);
        }
    } else if (std::is_same<T, _Float16>::value && a.o32) {
        // fp16 training forward (HILO): its float32 output and log-sum-exp feed the backward.  With
        // single fp16 probabilities the row sum is off by up to ~2^-12 where few keys are visible,
        // and dV, dK sum that per-row error over every query row (measured 1.01x the 2e-3 bar).
        if constexpr (std::is_same<T, _Float16>::value) {
            if (a.causal) {
                if (mode == 0) GT_PREFILL_LAUNCH_X(true, 0);
                else if (mode == 1) GT_PREFILL_LAUNCH_X(true, 1);
                else if (mode == 4) GT_PREFILL_LAUNCH_X(true, 4);
                else if (mode == 5) GT_PREFILL_LAUNCH_X(true, 5);
                else if (mode == 6) GT_PREFILL_LAUNCH_X(true, 6);
                else GT_PREFILL_LAUNCH_X(true, 2);
            } else {
                if (mode == 0) GT_PREFILL_LAUNCH_X(false, 0);
                else if (mode == 1) GT_PREFILL_LAUNCH_X(false, 1);
                else if (mode == 4) GT_PREFILL_LAUNCH_X(false, 4);
                else if (mode == 5) GT_PREFILL_LAUNCH_X(false, 5);
                else if (mode == 6) GT_PREFILL_LAUNCH_X(false, 6);
                else GT_PREFILL_LAUNCH_X(false, 2);
            }
        }
    } else if (a.causal) {
        if (mode == 0) GT_PREFILL_LAUNCH(true, 0);
        else if (mode == 1) GT_PREFILL_LAUNCH(true, 1);
        else if (mode == 4) GT_PREFILL_LAUNCH(true, 4);
        else if (mode == 5) GT_PREFILL_LAUNCH(true, 5);
        else if (mode == 6) GT_PREFILL_LAUNCH(true, 6);
        else GT_PREFILL_LAUNCH(true, 2);
    } else {
        if (mode == 0) GT_PREFILL_LAUNCH(false, 0);
        else if (mode == 1) GT_PREFILL_LAUNCH(false, 1);
        else if (mode == 4) GT_PREFILL_LAUNCH(false, 4);
        else if (mode == 5) GT_PREFILL_LAUNCH(false, 5);
        else if (mode == 6) GT_PREFILL_LAUNCH(false, 6);
        else GT_PREFILL_LAUNCH(false, 2);
    }
#undef GT_PREFILL_LAUNCH
#undef GT_PREFILL_LAUNCH_R
#undef GT_PREFILL_LAUNCH_D
#undef GT_PREFILL_LAUNCH_X
    return hipGetLastError();
}

// ---- float32 --------------------------------------------------------------------------------
// Float32 prefill (D = Dv = 64 or 128, no mask or a key-padding row): the structure of
// prefill_fwd_kernel (query tiles of 128 rows in pairs, K/V tiles streamed into LDS by DMA, one
// barrier per tile, the same lazy online softmax and causal / edge handling) on
// v_mfma_f32_32x32x2_f32, whose products and sums are float32 like the generic kernel's.  The
// MFMA's k index is free as long as both operands agree:
//   S^T = K.Q^T: k-step t takes dim t + (D/2)(lane/32), so a lane's Q values are the dims
//   [(D/2)(lane/32), +D/2) of its row, held in registers, and its K values come 4 at a time from
//   one 16-byte LDS read;
//   O^T += V^T.P^T: k-step s takes key 8(s/4) + 4(lane/32) + s%4, the key of the lane's S^T
//   accumulator entry s, so P^T's operand for step s is that entry as it stands.
// 32-key tiles: 16-byte chunk c of tile row r sits at chunk c ^ (r & 15), so the 16 rows one
// quarter-wave reads land on 16 different chunks mod 16 (different LDS banks).
constexpr int F32_NW = 4, F32_BM = 32 * F32_NW, F32_BN = 32, F32_NST = 2;

__device__ inline f32x16 mfma_f32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// DROP: P.V takes P times the element's multiplier (gt_philox.h); the lane's entries 4g .. 4g+3
// are 4 consecutive keys of its row, one Philox block.  The running sum keeps the undropped P.
template <int D, bool CAUSAL, int MASK, bool DROP = false>
__global__ __launch_bounds__(64 * F32_NW, 2) void prefill_f32_kernel(AttnFwdArgs a, int nq, int npairs) {
    constexpr int NW = F32_NW, BM = F32_BM, BN = F32_BN, NST = F32_NST;
    constexpr int CH = D / 4;               // 16-byte chunks per row
    constexpr int TILE = BN * D;            // floats per tile
    constexpr int NPW = BN * CH / 64 / NW;  // 1 KB wave loads per operand, wave and tile
    constexpr int DB = D / 32;              // d blocks of O^T
    constexpr int DH = D / 2;               // dims per lane half in S^T
    constexpr bool MROW = MASK == 4;
    constexpr bool MEL = MASK == 1 || MASK == 2 || MASK >= 5;  // per-element mask
    constexpr bool MVEC = MASK >= 5;                           // 4 keys per mask load
    constexpr bool MBOOL = MASK == 1 || MASK == 5;
    constexpr int PER = 2 * NPW + (MROW ? 1 : 0);  // loads per wave and tile
    static_assert(NPW >= 1 && CH >= 16 && PER < 64, "tile split");
    __shared__ __attribute__((aligned(1024))) float sK[NST][TILE];
    __shared__ __attribute__((aligned(1024))) float sV[NST][TILE];
    __shared__ __attribute__((aligned(16))) float sMk[MROW ? NST : 1][64];  // keys k0 .. k0+63 (32 used)

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t BH = a.B * a.H;
    int pair;
    int64_t bh;
    if (BH % 8 == 0) {
        const int64_t hpx = BH / 8, i = blockIdx.x / 8;
        pair = (int)(i % npairs);
        bh = (int64_t)(blockIdx.x % 8) * hpx + i / npairs;
    } else {
        pair = (int)(blockIdx.x % npairs);
        bh = (int64_t)blockIdx.x / npairs;
    }
    const int64_t b = bh / a.H, h = bh % a.H, hk = h / (a.H / a.Hkv);
    const int L = (int)a.L, S = (int)a.S;
    const int nkv = attn_kv_len(a, b), qpos = attn_q_pos(a, b);
    const int qa = nq - 1 - pair, qb = pair;
    const int nparts = qa == qb ? 1 : 2;
    const int na = key_tiles<CAUSAL, BM, BN>(qa, nkv, qpos);
    const int total = na + (nparts == 2 ? key_tiles<CAUSAL, BM, BN>(qb, nkv, qpos) : 0);

    const float *kbase = (const float *)a.k + b * a.k_sb + hk * a.k_sh;
    const float *vbase = (const float *)a.v + b * a.v_sb + hk * a.v_sh;
    const float c = a.scale * kLog2e;
    const float inv_scale = 1.0f / a.scale;
    const uint32_t k_row = (uint32_t)a.k_ss * 4, v_row = (uint32_t)a.v_ss * 4;
    int lrow_n[NPW];
    uint32_t lcol_n[NPW], kofs_n[NPW], vofs_n[NPW];
#pragma unroll
    for (int n = 0; n < NPW; ++n) {
        const int slot = (w * NPW + n) * 64 + lane;
        lrow_n[n] = slot / CH;
        lcol_n[n] = 16u * (uint32_t)((slot % CH) ^ (lrow_n[n] & 15));
        kofs_n[n] = (uint32_t)lrow_n[n] * k_row + lcol_n[n];
        vofs_n[n] = (uint32_t)lrow_n[n] * v_row + lcol_n[n];
    }
    const float *mrow = MROW ? (const float *)a.mask + b * a.m_sb + h * a.m_sh : nullptr;
    auto issue = [&](int step) {
        const int kt = step < na ? step : step - na;
        const int st = step % NST;
        if constexpr (MROW)
            lds_dma4(lds_addr(&sMk[st][0]), mrow, (uint32_t)min(kt * BN + lane, S - 1) * (uint32_t)a.m_ss * 4u);
        const uint32_t dk = lds_addr(&sK[st][0]) + w * NPW * 1024;
        const uint32_t dv = lds_addr(&sV[st][0]) + w * NPW * 1024;
        if (kt * BN + BN <= S) {
            const char *kb = (const char *)kbase + (uint64_t)(kt * BN) * k_row;
            const char *vb = (const char *)vbase + (uint64_t)(kt * BN) * v_row;
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                lds_dma16(dk + n * 1024, kb, kofs_n[n]);
                lds_dma16(dv + n * 1024, vb, vofs_n[n]);
            }
        } else {
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                const uint32_t key = (uint32_t)min(kt * BN + lrow_n[n], S - 1);
                lds_dma16(dk + n * 1024, kbase, key * k_row + lcol_n[n]);
                lds_dma16(dv + n * 1024, vbase, key * v_row + lcol_n[n]);
            }
        }
    };
    // LDS float offsets of this lane's fragments within a tile, as a per-lane part plus a
    // compile-time part (the XOR swizzle only touches chunk bits 0..3, so it splits):
    //   K, dims 4u .. 4u+3 of its half: row lrow, chunk (u + (D/8) half) ^ (lrow & 15)
    //     = lrow D + (4u ^ 4 ((lrow & 15) ^ (D/8) half))  (u < D/8: u + (D/8) half = u ^ (D/8) half)
    //   V, k-step s, d block db: row r = 8(s/4) + 4half + s%4, float d = 32db + lrow, chunk
    //     (d/4) ^ (r & 15) = (8db ^ 8((s/4) & 1)) + ((lrow/4) ^ 4half ^ (s%4))
    const int kbase0 = lrow * D, kx = 4 * ((lrow & 15) ^ ((D / 8) * half));
    auto kofs = [&](int u) { return kbase0 + ((4 * u) ^ kx); };
    const int vy = (lrow >> 2) ^ (4 * half);
    int vx[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) vx[cc] = 4 * D * half + (lrow & 3) + 4 * (vy ^ cc);
    auto vofs = [&](int s, int db) {
        return vx[s & 3] + 8 * D * (s >> 2) + D * (s & 3) + 4 * ((8 * db) ^ (8 * ((s >> 2) & 1)));
    };

#pragma unroll
    for (int st = 0; st < NST - 1; ++st)
        if (st < total) issue(st);

    int step = 0;
    for (int part = 0; part < nparts; ++part) {
        const int qt = part == 0 ? qa : qb;
        const int ntiles = part == 0 ? na : total - na;
        const int wq0 = qt * BM + 32 * w;
        const int lq = wq0 + lrow;
        // Q^T as B operands: dims (D/2) half .. +D/2 of row lq (rows past L read row L-1)
        float qf[DH];
        {
            const float *qr = (const float *)a.q + b * a.q_sb + h * a.q_sh + (int64_t)min(lq, L - 1) * a.q_sl + DH * half;
#pragma unroll
            for (int u = 0; u < DH / 4; ++u) {
                const f32x4 x = *(const f32x4 *)(qr + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) qf[4 * u + e] = x[e];
            }
#pragma unroll
            for (int u = 0; u < DH; ++u) asm volatile("" ::"v"(qf[u]));
        }
        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
        float m = -INFINITY, mthr = -INFINITY, lsum = 0.0f;
        // dropout: Philox block of keys 0..3 of this lane's row (rows past L draw unused words)
        const uint64_t drow = DROP ? (uint64_t)(bh * a.L + lq) * (uint64_t)((a.S + 3) / 4) : 0;
        // per-element mask: element offset of this lane's mask row
        const int64_t mrb = MEL ? b * a.m_sb + h * a.m_sh + (int64_t)min(lq, L - 1) * a.m_sl : 0;

        for (int j = 0; j < ntiles; ++j, ++step) {
            const int k0 = j * BN;
            const int later = min(NST - 2, total - 1 - step);
            if (later >= 1) wait_vm<PER>();
            else wait_vm<0>();
            __syncthreads();
            const float *cK = sK[step % NST];
            const float *cV = sV[step % NST];
            // MVEC: the mask of keys k0 + 8g + 4half + 0..3 of this lane's row, loaded before the
            // MFMAs (groups past the last 4 keys read those: their scores are blocked below)
            f32x4 mvf[MVEC && !MBOOL ? 4 : 1];
            uint32_t mvb[MVEC && MBOOL ? 4 : 1];
            if constexpr (MVEC) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int64_t at = mrb + min(k0 + 8 * g + 4 * half, S - 4);
                    if constexpr (MBOOL) mvb[g] = *(const uint32_t *)((const uint8_t *)a.mask + at);
                    else mvf[g] = *(const f32x4 *)((const float *)a.mask + at);
                }
            }
            // ---- S^T = K . Q^T: s[i] is key k0 + 8(i/4) + 4half + i%4, query lq ----
            f32x16 s;
            if constexpr (MROW) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 mv4 = *(const f32x4 *)&sMk[step % NST][8 * g + 4 * half];
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[4 * g + e] = mv4[e] * inv_scale;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < DH / 4; ++u) {
                const f32x4 kv = *(const f32x4 *)&cK[kofs(u)];
#pragma unroll
                for (int e = 0; e < 4; ++e) s = mfma_f32x2(kv[e], qf[4 * u + e], s);
            }
            // the next tile's loads into the stage every wavefront finished with before the barrier
            if (step + NST - 1 < total) issue(step + NST - 1);

            const bool edge = k0 + BN > nkv || (CAUSAL && k0 + BN - 1 > wq0 + qpos);
            if (MEL || edge) {
                const int vis = min(nkv - 1, CAUSAL ? lq + qpos : nkv - 1) - (k0 + 4 * half);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float x = s[i];
                    if constexpr (MVEC) {
                        if constexpr (MBOOL) x = (mvb[i / 4] >> (8 * (i % 4))) & 0xffu ? x : -INFINITY;
                        else x = fmaf(mvf[i / 4][i % 4], inv_scale, x);
                    } else if constexpr (MEL) {
                        const int key = min(k0 + 8 * (i / 4) + 4 * half + (i % 4), S - 1);
                        const int64_t mi = mrb + (int64_t)key * a.m_ss;
                        if constexpr (MBOOL) x = ((const uint8_t *)a.mask)[mi] ? x : -INFINITY;
                        else x = fmaf(((const float *)a.mask)[mi], inv_scale, x);
                    }
                    const bool blocked = 8 * (i / 4) + (i % 4) > vis;
                    s[i] = blocked ? -INFINITY : x;
                }
            }
            float tmax = max3(s[0], s[1], s[2]);
#pragma unroll
            for (int i = 3; i < 15; i += 2) tmax = max3(tmax, s[i], s[i + 1]);
            tmax = max3(tmax, s[15], s[15]);
            tmax = xhalf_max(tmax);
            const float tm = tmax * c;
            const bool move = tm > mthr;
            if (!__all(!move)) {
                const float mnew = move ? tm + huge_margin(tm) : m;
                const float alpha = move ? fast_exp2(m - mnew) : 1.0f;
                lsum *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
                m = mnew;
                mthr = m + kLazy - 0.5f * huge_margin(m);
            }
            const float msub = m == -INFINITY ? 0.0f : m;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s[i] = fast_exp2(fmaf(s[i], c, -msub));
                lsum += s[i];
            }
            if constexpr (DROP) {
                const float dscale = (float)a.drop.scale;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const GtWord4 x = gt_philox4x32_10(drow + (uint64_t)((k0 + 8 * g + 4 * half) >> 2), a.drop.offset,
                                                       a.drop.seed);
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[4 * g + e] *= x.w[e] < a.drop.thresh ? dscale : 0.0f;
                }
            }
            // ---- O^T += V^T . P^T ----
#pragma unroll
            for (int st2 = 0; st2 < 16; ++st2)
#pragma unroll
                for (int db = 0; db < DB; ++db) o[db] = mfma_f32x2(cV[vofs(st2, db)], s[st2], o[db]);
        }

        const float ltot = xhalf_sum(lsum);
        const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
        if (lq < L) {
            float *orow = (float *)a.o + (bh * a.L + lq) * D;
            float *row32 = a.o32 ? (float *)a.o32 + (bh * a.L + lq) * D : nullptr;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 v = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                     o[db][4 * g + 3] * inv};
                    *(f32x4 *)(orow + 32 * db + 8 * g + 4 * half) = v;
                    if (row32) *(f32x4 *)(row32 + 32 * db + 8 * g + 4 * half) = v;
                }
            if (a.lse && half == 0)
                ((float *)a.lse)[bh * a.L + lq] = ltot > 0.0f ? (m + log2f(ltot)) * kLn2 : INFINITY;
        }
    }
}

// Float32 prefill for small grids (few heads of short sequences, where prefill_f32_kernel has
// fewer workgroups than the GPU has CUs and each wavefront's walk over the key tiles is the whole
// time): one workgroup per 32 query rows, its 4 wavefronts splitting the key tiles (tile t to
// wavefront t % 4) with an online softmax each, then merging the four (max, sum, O) states
// through LDS.  The operand mapping is prefill_f32_kernel's (S^T = K.Q^T with k-step t = dim
// t + (D/2)(lane/32) and Q in registers; O^T += V^T.P^T with k-step s = the key of accumulator
// entry s), but each wavefront reads its K rows (16-byte pieces) and V^T values straight from
// memory: they are few and stay in L2.  Masks, dropout and KV-cache lengths as prefill_f32_kernel
// takes them (the mask read per score, or 4 keys per load for modes 5 and 6).
template <int D, bool CAUSAL, int MASK, bool DROP>
__global__ __launch_bounds__(256) void prefill_f32_split_kernel(AttnFwdArgs a, int ng) {
    constexpr int DH = D / 2, DB = D / 32, OP = D + 4;  // OP: LDS row pitch of the partial O
    constexpr bool MVEC = MASK >= 5;                    // 4 keys per mask load
    constexpr bool MBOOL = MASK == 1 || MASK == 5;
    __shared__ __attribute__((aligned(16))) float sO[4][32][OP];
    __shared__ float sM[4][32], sL[4][32];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t bh = blockIdx.x / ng;
    const int rg = (int)(blockIdx.x % ng);
    const int64_t b = bh / a.H, h = bh % a.H, hk = h / (a.H / a.Hkv);
    const int L = (int)a.L, S = (int)a.S;
    const int q0 = 32 * rg, lq = q0 + lrow, lqc = min(lq, L - 1);
    const int nkv = attn_kv_len(a, b), qpos = attn_q_pos(a, b);
    const int kv_end = CAUSAL ? min(q0 + 32 + qpos, nkv) : nkv;  // keys any row of the group sees
    const int nt = kv_end > 0 ? (kv_end + 31) / 32 : 0;
    const float c = a.scale * kLog2e;
    // element offset of this lane's mask row (MASK 4: the key-padding row, m_sl = 0)
    const int64_t mrb = MASK != 0 ? b * a.m_sb + h * a.m_sh + (int64_t)lqc * a.m_sl : 0;
    // dropout: Philox block of keys 0..3 of this lane's row (rows past L draw unused words)
    const uint64_t drow = DROP ? (uint64_t)(bh * a.L + lq) * (uint64_t)((a.S + 3) / 4) : 0;

    float qf[DH];  // Q of row lqc, dims DH half .. +DH (B operand of S^T)
    {
        const float *qr = (const float *)a.q + b * a.q_sb + h * a.q_sh + (int64_t)lqc * a.q_sl + DH * half;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(qr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[4 * u + e] = x[e];
        }
    }
    const float *kbase = (const float *)a.k + b * a.k_sb + hk * a.k_sh;
    const float *vbase = (const float *)a.v + b * a.v_sb + hk * a.v_sh;
    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;  // running max (log2 domain) and this half's share of the sum

    for (int t = w; t < nt; t += 4) {
        const int k0 = 32 * t;
        // S^T: s[i] is key k0 + 8(i/4) + 4half + i%4, query lq
        const float *kr = kbase + (int64_t)min(k0 + lrow, S - 1) * a.k_ss + DH * half;
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 kv = *(const f32x4 *)(kr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) s = mfma_f32x2(kv[e], qf[4 * u + e], s);
        }
        const int vis = min(nkv - 1, CAUSAL ? lq + qpos : nkv - 1) - (k0 + 4 * half);
        // MVEC: the mask of keys k0 + 8g + 4half + 0..3 (groups past the last 4 keys read those:
        // their scores are blocked)
        f32x4 mvf[MVEC && !MBOOL ? 4 : 1];
        uint32_t mvb[MVEC && MBOOL ? 4 : 1];
        if constexpr (MVEC) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t at = mrb + min(k0 + 8 * g + 4 * half, S - 4);
                if constexpr (MBOOL) mvb[g] = *(const uint32_t *)((const uint8_t *)a.mask + at);
                else mvf[g] = *(const f32x4 *)((const float *)a.mask + at);
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float x = s[i] * c;
            bool blocked = 8 * (i / 4) + (i % 4) > vis;
            if constexpr (MVEC) {
                if constexpr (MBOOL) blocked = blocked || ((mvb[i / 4] >> (8 * (i % 4))) & 0xffu) == 0u;
                else x = fmaf(mvf[i / 4][i % 4], kLog2e, x);
            } else if constexpr (MASK != 0) {
                const int64_t mi = mrb + (int64_t)min(k0 + 8 * (i / 4) + 4 * half + (i % 4), S - 1) * a.m_ss;
                if constexpr (MBOOL) blocked = blocked || ((const uint8_t *)a.mask)[mi] == 0;
                else x = fmaf(((const float *)a.mask)[mi], kLog2e, x);
            }
            s[i] = blocked ? -INFINITY : x;
            tmax = fmaxf(tmax, s[i]);
        }
        const float mnew = fmaxf(m, xhalf_max(tmax));
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        if (mnew != m) {
            const float alpha = fast_exp2(m - msub);  // m = -inf: 0 (O and the sum are 0)
            lsum *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
            m = mnew;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s[i] = fast_exp2(s[i] - msub);  // -inf -> 0
            lsum += s[i];
        }
        if constexpr (DROP) {
            // entries 4g .. 4g+3 are keys k0 + 8g + 4half + 0..3: one Philox block
            const float dscale = (float)a.drop.scale;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const GtWord4 x = gt_philox4x32_10(drow + (uint64_t)((k0 + 8 * g + 4 * half) >> 2), a.drop.offset,
                                                   a.drop.seed);
#pragma unroll
                for (int e = 0; e < 4; ++e) s[4 * g + e] *= x.w[e] < a.drop.thresh ? dscale : 0.0f;
            }
        }
        // O^T += V^T . P^T: k-step s2 is key k0 + 8(s2/4) + 4half + s2%4, A = V[that key][32 db + lrow]
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) {
            const float *vr = vbase + (int64_t)min(k0 + 8 * (s2 >> 2) + 4 * half + (s2 & 3), S - 1) * a.v_ss + lrow;
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] = mfma_f32x2(vr[32 * db], s[s2], o[db]);
        }
    }

    // ---- merge the four wavefronts' states ----
    const float ltot = xhalf_sum(lsum);
    if (half == 0) {
        sM[w][lrow] = m;
        sL[w][lrow] = ltot;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = {o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
            *(f32x4 *)&sO[w][lrow][32 * db + 8 * g + 4 * half] = v;
        }
    __syncthreads();
    // thread: row r of the group, dims (D/8) part .. +D/8
    const int r = threadIdx.x >> 3, part = threadIdx.x & 7;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sM[ww][r]);
    float wg[4], Lt = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
        wg[ww] = sM[ww][r] == -INFINITY ? 0.0f : fast_exp2(sM[ww][r] - M);
        Lt = fmaf(wg[ww], sL[ww][r], Lt);
    }
    const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
    if (q0 + r < L) {
        float *orow = (float *)a.o + (bh * a.L + q0 + r) * D + (D / 8) * part;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                const f32x4 x = *(const f32x4 *)&sO[ww][r][(D / 8) * part + 4 * j];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = fmaf(wg[ww], x[e], acc[e]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] *= inv;
            *(f32x4 *)(orow + 4 * j) = acc;
        }
        if (a.lse && part == 0) ((float *)a.lse)[bh * a.L + q0 + r] = Lt > 0.0f ? (M + log2f(Lt)) * kLn2 : INFINITY;
    }
}

// The calls prefill_f32_split_kernel takes: at most 64 workgroups of prefill_f32_kernel
// (B * H * query-tile pairs) and at most 4096 keys.  Measured
// against the tiled kernel: faster at every grid of up to 64 of its workgroups (B2 H8 L=S=1024
// D128: 107 against 276 us; B1 H8 L=S=2048 D128 causal: 207 against 295 us), mixed at 128,
// twice as slow at 256 (each 32-row group reads its keys' K and V itself, where the tiled
// kernel shares a tile among 128 rows).
bool prefill_f32_split(const AttnFwdArgs &f) {
    if (f.o32 || f.rope_q || f.S > 4096) return false;
    const int64_t pairs = ((f.L + F32_BM - 1) / F32_BM + 1) / 2;
    return f.B * f.H * pairs <= 64;
}

bool prefill_f32_supported(const AttnFwdArgs &f) {
    if (f.out_dtype != GT_F32 || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    if (f.rope_q) return false;
    const int mode = attn_mask_mode(f);
    // fewer than 16 query rows: one mostly empty 128-row tile per head walking every key; the
    // generic kernel measured as fast or faster there (one row: 1.14 against 2.02 ms at B32
    // H32/8 S4096 D128; 16 rows: even).  The small-grid kernel takes them (32-row groups,
    // 4 wavefronts per key range): 4 rows B1 H32/8 S4096 D128 229 us against the generic 538
    if ((f.L < 16 && !prefill_f32_split(f)) || f.L < 1 || f.S < 1 || !(f.scale > 0.0f)) return false;
    if (f.L >= (1LL << 30) || f.S >= (1LL << 30)) return false;
    const int64_t strides[] = {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 4 != 0 || st < 0) return false;  // 16-byte rows
    for (const void *p : {f.q, f.k, f.v, (const void *)f.o}) if ((uintptr_t)p % 16 != 0) return false;
    if (f.o32 && (uintptr_t)f.o32 % 16 != 0) return false;
    if ((f.S - 1) * f.k_ss * 4 + f.D * 4 > 0xffffffffLL) return false;
    if ((f.S - 1) * f.v_ss * 4 + f.Dv * 4 > 0xffffffffLL) return false;
    if (mode == 4 && (f.m_ss < 0 || (f.S - 1) * f.m_ss * 4 + 4 > 0xffffffffLL)) return false;
    return true;
}

template <int D, bool CAUSAL, bool DROP>
hipError_t launch_prefill_f32_cd(const AttnFwdArgs &a, int nq, int npairs, int64_t grid, hipStream_t s) {
#define GT_F32_LAUNCH(MK) \
    hipLaunchKernelGGL((prefill_f32_kernel<D, CAUSAL, MK, DROP>), dim3((unsigned)grid), dim3(64 * F32_NW), 0, s, a, nq, npairs)
    switch (attn_mask_mode(a)) {
        case 0: GT_F32_LAUNCH(0); break;
        case 1: GT_F32_LAUNCH(1); break;
        case 2: GT_F32_LAUNCH(2); break;
        case 4: GT_F32_LAUNCH(4); break;
        case 5: GT_F32_LAUNCH(5); break;
        case 6: GT_F32_LAUNCH(6); break;
        default: return hipErrorInvalidValue;
    }
#undef GT_F32_LAUNCH
    return hipGetLastError();
}

template <int D>
hipError_t launch_prefill_f32_d(const AttnFwdArgs &a, int nq, int npairs, int64_t grid, hipStream_t s) {
    if (a.dropout)
        return a.causal ? launch_prefill_f32_cd<D, true, true>(a, nq, npairs, grid, s)
                        : launch_prefill_f32_cd<D, false, true>(a, nq, npairs, grid, s);
    return a.causal ? launch_prefill_f32_cd<D, true, false>(a, nq, npairs, grid, s)
                    : launch_prefill_f32_cd<D, false, false>(a, nq, npairs, grid, s);
}

template <int D, bool CAUSAL, bool DROP>
hipError_t launch_split(const AttnFwdArgs &a, dim3 grid, int ng, hipStream_t s) {
#define GT_SPLIT(MK) hipLaunchKernelGGL((prefill_f32_split_kernel<D, CAUSAL, MK, DROP>), grid, dim3(256), 0, s, a, ng)
    switch (attn_mask_mode(a)) {
        case 0: GT_SPLIT(0); break;
        case 1: GT_SPLIT(1); break;
        case 2: GT_SPLIT(2); break;
        case 4: GT_SPLIT(4); break;
        case 5: GT_SPLIT(5); break;
        case 6: GT_SPLIT(6); break;
        default: return hipErrorInvalidValue;
    }
#undef GT_SPLIT
    return hipGetLastError();
}

hipError_t launch_prefill_f32(const AttnFwdArgs &a, hipStream_t s) {
    if (prefill_f32_split(a)) {
        const int ng = (int)((a.L + 31) / 32);
        const dim3 grid((unsigned)(a.B * a.H * ng));
        if (a.D == 128) {
            if (a.dropout) return a.causal ? launch_split<128, true, true>(a, grid, ng, s) : launch_split<128, false, true>(a, grid, ng, s);
            return a.causal ? launch_split<128, true, false>(a, grid, ng, s) : launch_split<128, false, false>(a, grid, ng, s);
        }
        if (a.dropout) return a.causal ? launch_split<64, true, true>(a, grid, ng, s) : launch_split<64, false, true>(a, grid, ng, s);
        return a.causal ? launch_split<64, true, false>(a, grid, ng, s) : launch_split<64, false, false>(a, grid, ng, s);
    }
    const int nq = (int)((a.L + F32_BM - 1) / F32_BM);
    const int npairs = (nq + 1) / 2;
    const int64_t grid = (int64_t)npairs * a.B * a.H;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    return a.D == 128 ? launch_prefill_f32_d<128>(a, nq, npairs, grid, s) : launch_prefill_f32_d<64>(a, nq, npairs, grid, s);
}

}  // namespace

bool attn_prefill_f32_split(const AttnFwdArgs &f, int cd) {
    return cd == GT_F32 && prefill_f32_supported(f) && prefill_f32_split(f);
}

bool attn_prefill_supported(const AttnFwdArgs &f, int cd) {
    if (cd == GT_F32) return prefill_f32_supported(f);
    if (cd != GT_F16 && cd != GT_BF16) return false;
    if (f.rope_q && f.mask && (f.mask_bool || f.m_sl != 0)) return false;  // fused RoPE: no mask or key padding
    if (f.rope_q && f.dropout) return false;
    if (f.out_dtype != cd || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    if (f.L < 1 || f.S < 1 || !(f.scale > 0.0f)) return false;
    if (f.L >= (1LL << 30) || f.S >= (1LL << 30)) return false;  // 32-bit row indices
    const int64_t strides[] = {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 8 != 0 || st < 0) return false;
    for (const void *p : {f.q, f.k, f.v}) if ((uintptr_t)p % 16 != 0) return false;
    // K/V tiles are addressed by 32-bit byte offsets from the (batch, kv head) base
    if ((f.S - 1) * f.k_ss * 2 + f.D * 2 > 0xffffffffLL) return false;
    if ((f.S - 1) * f.v_ss * 2 + f.Dv * 2 > 0xffffffffLL) return false;
    // a query-independent float mask row is addressed the same way
    if (f.mask && !f.mask_bool && f.m_sl == 0 && (f.m_ss < 0 || (f.S - 1) * f.m_ss * 4 + 4 > 0xffffffffLL)) return false;
    return true;
}

hipError_t launch_attn_prefill(const AttnFwdArgs &a, int cd, hipStream_t s) {
    if (cd == GT_F32) return launch_prefill_f32(a, s);
    if (attn_prefill_asm_supported(a, cd)) return launch_attn_prefill_asm(a, s);
    const int BM = a.D == 64 ? bm_of<64>() : bm_of<128>();
    const int nq = (int)((a.L + BM - 1) / BM);
    const int npairs = (nq + 1) / 2;  // query tiles p and nq-1-p share a workgroup
    const int64_t grid = (int64_t)npairs * a.B * a.H;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    if (cd == GT_F16)
        return a.D == 128 ? launch_variant<_Float16, 128>(a, nq, npairs, grid, s)
                          : launch_variant<_Float16, 64>(a, nq, npairs, grid, s);
    return a.D == 128 ? launch_variant<__bf16, 128>(a, nq, npairs, grid, s)
                      : launch_variant<__bf16, 64>(a, nq, npairs, grid, s);
}
