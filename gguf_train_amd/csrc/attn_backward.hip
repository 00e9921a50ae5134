// Recompute-based attention backward on gfx950 MFMA (fp16 / bf16 inputs, fp32 gradients).
//
// Replaces the reference's Python composition (gguf_train/_functions.py:1933-1965), which
// materialises (B,H,L,S) scores, probabilities and their gradients, with two kernels that
// keep everything in registers and LDS and recompute P from the forward's log-sum-exp:
//   dQ:     the forward's structure (a workgroup owns 128 query rows, loops over key tiles);
//           each row first forms D_q = sum_d dO[q,d] * O[q,d] (= sum_s P[q,s] dP[q,s], the
//           rowsum in dS) and writes it for dK/dV, which runs after it:
//             S^T = K.Q^T, dP^T = V.dO^T, dS^T as below, dQ^T += K^T.dS^T
//   dK/dV:  a workgroup owns 128 keys of one kv head (32 per wavefront, K and V rows held in
//           registers) and walks over the query tiles of every query head of its GQA group:
//             S = Q.K^T, dP = dO.V^T          (keys on lanes: the accumulator layout)
//             P = exp2(S*scale*log2e - lse*log2e), dS = P * (dP - D_q)
//             dV += P^T.dO, dK += dS^T.Q      (P, dS feed the MFMA A operand in place; dO and Q
//                                              are read transposed from row-major LDS tiles)
// dK and dV of a GQA group are summed in registers (no atomics).  P and dS are split into hi +
// lo operands so the products keep ~16 bits (bf16) or ~22 (fp16): a single fp16 operand's 2^-12
// rounding accumulates in dV and dK, whose sums run over query rows (measured 1.27x the 2e-3
// bar on fp16 dV), and dQ follows the same rule.  Masks: top-left causal,
// bool / additive (read per element; an additive mask that does not depend on the query row is
// read once per key: per head in dK/dV, staged with the K/V tile in dQ), keys >= S and
// queries >= L contribute nothing.
// Dropout (DROP): dV += (P*m)^T.dO and dP = m * dO.V^T in dS = P * (dP - delta), m the
// element's multiplier (gt_philox.h).  dQ draws its lanes' Philox blocks directly (4 consecutive
// keys of one query per block, as the forward) and writes the decisions as bits, one word per
// (query row, 32 keys); dK/dV, whose lanes hold 16 queries of one key, streams those words in
// with each query step (64 rows x 4 words through LDS) instead of drawing again.  Without that
// buffer (a.dbits null: the caller bounds its size) each dK/dV thread draws its word itself, 8
// Philox blocks per step.

#include "attn_common.h"
#include "gt_internal.h"
#include "mfma_util.h"
#include "lds_dma.h"

#include <cmath>

namespace {

using namespace gtmfma;

constexpr int BKV = 128;  // keys per dK/dV workgroup (32 per wavefront)
constexpr int BQ = 64;    // query rows per dK/dV step
constexpr int BMQ = 128;  // query rows per dQ workgroup (32 per wavefront)
constexpr int BNK = 64;   // key rows per dQ step

// ---- dK, dV ----------------------------------------------------------------------------------

// D = 64 fits two wavefronts per SIMD without spills (with one, the compiler parks values in
// AGPRs and moves them back and forth); D = 128 needs the whole register file.  (Dropout with the
// key-padding row spills ~60 bytes per lane at two per SIMD and is still faster there: 255 against
// 285 us for the training step with dropout.)
template <typename T, int D, bool CAUSAL, int MASK, bool DROP = false>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void bwd_dkdv_kernel(AttnBwdArgs a) {
    using M = Mfma<T>;
    using V8 = typename M::V8;
    constexpr int DT = D / 16, DB = D / 32, CH = D / 8;
    constexpr int QP = D + 16;              // Q / dO tile pitch (transposed reads)
    constexpr int NLD = BQ * CH / 256;      // 16-byte loads per thread per tile and operand
    static_assert(NLD >= 1, "tile split over the threads");
    __shared__ __attribute__((aligned(16))) T sQ[2][BQ * QP];
    __shared__ __attribute__((aligned(16))) T sG[2][BQ * QP];  // dO
    __shared__ __attribute__((aligned(16))) float sL[2][BQ];    // lse * log2(e)
    __shared__ __attribute__((aligned(16))) float sD[2][BQ];    // -delta
    // dropout: word [w][r] = decisions of keys k0 + 32w .. +31 for query qs0 + r (bit j: key 32w + j)
    __shared__ __attribute__((aligned(16))) uint32_t sDm[DROP ? 2 : 1][DROP ? 4 * BQ : 1];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int g16 = lane >> 4, i16 = lane & 15;
    // Key tile major: all workgroups of key tile 0 first.  Under the causal mask tile kt walks
    // the queries from k0 on, so the heaviest workgroups start first and the short ones fill
    // the tail (list scheduling over two rounds of B*Hkv*nkt = 1024 workgroups on 512 slots:
    // makespan 18 steps instead of 28 with key tiles interleaved).  The tiles of one (b, kv
    // head) sit B*Hkv apart, on the same XCD when B*Hkv % 8 == 0.
    const int64_t nbk = f.B * f.Hkv;
    const int kt = (int)(blockIdx.x / nbk);
    const int64_t bk = blockIdx.x % nbk, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int G = (int)(f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int k0 = kt * BKV, wk0 = k0 + 32 * w, key = wk0 + lrow;  // this lane's key (n index)
    const float c = f.scale * kLog2e, inv_scale = 1.0f / f.scale;
    const float dscale = DROP ? (float)f.drop.scale : 1.0f;
    const int64_t dwords = (f.S + 31) / 32;  // decision words per query row

    // K and V rows of this lane's key as B operands (B[k = d][n = key])
    V8 kf[DT], vf[DT];
    {
        const int kk = min(key, S - 1);
        const T *kr = (const T *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)kk * f.k_ss + 8 * half;
        const T *vr = (const T *)f.v + b * f.v_sb + hk * f.v_sh + (int64_t)kk * f.v_ss + 8 * half;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            kf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(kr + 16 * t));
            vf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(vr + 16 * t));
        }
        // Wait for K and V here: otherwise the compiler's wait for these loads lands inside the
        // loop, where (vector memory loads completing in order) it also waits for every Q / dO
        // prefetch issued since, exposing the full global load latency on every step.
#pragma unroll
        for (int t = 0; t < DT; ++t) asm volatile("" ::"v"(kf[t]), "v"(vf[t]));
    }
    f32x16 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dk[db][i] = dv[db][i] = 0.0f;

    // the query steps: every query head of the group, queries that can see a key of this tile
    const int qstart = CAUSAL ? (k0 / BQ) * BQ : 0;
    const int nqs = L > qstart ? (L - qstart + BQ - 1) / BQ : 0;
    const int nsteps = nqs * G;

    u32x4 qreg[NLD], greg[NLD];
    float lreg = 0.0f, dreg = 0.0f;
    uint32_t mreg = 0u;  // dropout: this thread's decision word of the step
    auto load_step = [&](int st) {
        const int hh = st / nqs, qs0 = qstart + (st % nqs) * BQ;
        const int64_t h = hk * G + hh;
        const T *qb = (const T *)f.q + b * f.q_sb + h * f.q_sh;
        const T *gb = (const T *)a.dout + ((b * f.H + h) * f.L) * D;
        if constexpr (DROP) {
            // thread t: row t % 64 of the step, key word t / 64 of the tile (words past the
            // sequence's keys repeat the last one: their keys have P = 0)
            const int r = tid % BQ, wd = min((int)(k0 / 32 + tid / BQ), (int)dwords - 1);
            const int64_t row = (b * f.H + h) * f.L + min(qs0 + r, L - 1);
            if (a.dbits) {
                mreg = a.dbits[row * dwords + wd];
            } else {
                const uint64_t n0 = (uint64_t)row * (uint64_t)((f.S + 3) / 4) + (uint64_t)(8 * wd);
                uint32_t word = 0u;
#pragma unroll 2
                for (int u = 0; u < 8; ++u) {
                    const GtWord4 x = gt_philox4x32_10(n0 + u, f.drop.offset, f.drop.seed);
#pragma unroll
                    for (int e = 0; e < 4; ++e) word |= (x.w[e] < f.drop.thresh ? 1u : 0u) << (4 * u + e);
                }
                mreg = word;
            }
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int cidx = tid + 256 * i, row = cidx / CH, col = cidx % CH;
            const int q = min(qs0 + row, L - 1);
            qreg[i] = *(const u32x4 *)(qb + (int64_t)q * f.q_sl + 8 * col);
            greg[i] = *(const u32x4 *)(gb + (int64_t)q * D + 8 * col);
        }
        if (tid < BQ) {
            // raw values: the arithmetic waits for the loads, so it happens at store time
            const int64_t r = (b * f.H + h) * f.L + min(qs0 + tid, L - 1);
            lreg = ((const float *)f.lse)[r];
            dreg = ((const float *)a.delta)[r];
        }
    };
    auto store_step = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int cidx = tid + 256 * i, row = cidx / CH, col = cidx % CH;
            *(u32x4 *)&sQ[buf][row * QP + 8 * col] = qreg[i];
            *(u32x4 *)&sG[buf][row * QP + 8 * col] = greg[i];
        }
        if (tid < BQ) {
            sL[buf][tid] = lreg * kLog2e;  // lse * log2(e)
            sD[buf][tid] = -dreg;          // -delta
        }
        if constexpr (DROP) sDm[buf][tid] = mreg;  // [tid / 64][tid % 64]
    };

    if (nsteps > 0) {
        load_step(0);
        store_step(0);
        if (nsteps > 1) load_step(1);
    }
    __syncthreads();
    // The first S and dP products accumulate onto (the key's mask term, -delta of each query):
    // S then holds QK^T + mask and dP holds dO.V^T - delta, with no per-element adds.
    f32x16 sinit;  // MASK 4: the mask value of this lane's key for the current head (raw units)
#pragma unroll
    for (int i = 0; i < 16; ++i) sinit[i] = 0.0f;
    for (int st = 0; st < nsteps; ++st) {
        const int buf = st & 1;
        const int hh = st / nqs, qs0 = qstart + (st % nqs) * BQ;
        if constexpr (D <= 64) progress_priority(st);  // two workgroups per CU
        const int64_t h = hk * G + hh;
        const T *cQ = sQ[buf];
        const T *cG = sG[buf];
        if (MASK == 4 && st % nqs == 0) {
            const float madd =
                ((const float *)f.mask)[b * f.m_sb + h * f.m_sh + (int64_t)min(key, S - 1) * f.m_ss] * inv_scale;
#pragma unroll
            for (int i = 0; i < 16; ++i) sinit[i] = madd;
        }
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int q0 = qs0 + 32 * qb;
            if (CAUSAL && q0 + 31 < wk0) continue;  // every query of the block precedes our keys
            // MASK 1 / 2: this lane's 16 mask values of the block (query q0 + 4half + c, c = 8(i/4) +
            // i%4), loaded before the S and dP products so that they land during them; the loads
            // are unconditional (no branch, no wait per element), an invisible element reading
            // the lane's key in the last query row instead
            constexpr bool MFULL = MASK == 1 || MASK == 2;
            float madd[MASK == 2 ? 16 : 1];
            uint32_t mbyte[MASK == 1 ? 16 : 1];
            if constexpr (MFULL) {
                const int64_t mkey = b * f.m_sb + h * f.m_sh + (int64_t)min(key, S - 1) * f.m_ss;
                const int64_t mlane = mkey + (int64_t)(q0 + 4 * half) * f.m_sl;
                const int64_t msafe = mkey + (int64_t)(L - 1) * f.m_sl;
                int lo = (CAUSAL ? key : 0) - (q0 + 4 * half);
                int span = (L - 1 - (q0 + 4 * half)) - lo;
                if (key >= S || span < 0) {
                    lo = 32;
                    span = 0;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int cq = 8 * (i / 4) + (i % 4);
                    const int64_t mi = (uint32_t)(cq - lo) <= (uint32_t)span ? mlane + (int64_t)cq * f.m_sl : msafe;
                    if constexpr (MASK == 2) madd[i] = ((const float *)f.mask)[mi];
                    else mbyte[i] = ((const uint8_t *)f.mask)[mi];
                }
            }
            // s[i], dp[i]: query q0 + 8(i/4) + 4half + i%4, key `key`
            // (dropout: dP starts at 0, -delta is added after the multiplier)
            f32x16 s, dp;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 d4 = *(const f32x4 *)&sD[buf][32 * qb + 8 * g + 4 * half];
#pragma unroll
                for (int e = 0; e < 4; ++e) dp[4 * g + e] = DROP ? 0.0f : d4[e];
            }
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const V8 qa = *(const V8 *)&cQ[(32 * qb + lrow) * QP + 16 * t + 8 * half];
                const V8 ga = *(const V8 *)&cG[(32 * qb + lrow) * QP + 16 * t + 8 * half];
                s = M::mma(qa, kf[t], t == 0 ? sinit : s);
                dp = M::mma(ga, vf[t], dp);
            }
            float p[16], ds[16];
            // every (query, key) of the block visible and no per-element mask: no tests
            const bool interior = (MASK == 0 || MASK == 4) && wk0 + 31 < S && q0 + 31 < L && (!CAUSAL || q0 >= wk0 + 31);
            // dropout: multiplier of entry i (query 32qb + 8(i/4) + 4half + i%4 of the step, this
            // lane's key 32w + lrow of the tile): bit lrow of word [w][query]
            uint32_t dbits = 0u;  // bit i: entry i kept
            if constexpr (DROP) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const u32x4 dw = *(const u32x4 *)&sDm[buf][w * BQ + 32 * qb + 8 * g + 4 * half];
#pragma unroll
                    for (int e = 0; e < 4; ++e) dbits |= ((dw[e] >> lrow) & 1u) << (4 * g + e);
                }
            }
            auto mult = [&](int i) { return (dbits >> i) & 1u ? dscale : 0.0f; };
            if constexpr (DROP) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 d4 = *(const f32x4 *)&sD[buf][32 * qb + 8 * g + 4 * half];
#pragma unroll
                    for (int e = 0; e < 4; ++e) dp[4 * g + e] = fmaf(dp[4 * g + e], mult(4 * g + e), d4[e]);  // m dO.V - delta
                }
            }
            if (interior) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int qi = 32 * qb + 8 * g + 4 * half;
                    const f32x4 l4 = *(const f32x4 *)&sL[buf][qi];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * g + e;
                        const float pv = fast_exp2(fmaf(s[i], c, -l4[e]));
                        p[i] = DROP ? pv * mult(i) : pv;
                        ds[i] = pv * dp[i];
                    }
                }
            } else {
                // query q0 + 4half + c (c = 8(i/4) + i%4) sees this lane's key when lo <= c <= lo + span
                // (key < S, q < L, causal q >= key), as one unsigned compare per score; a
                // per-element mask is read only there, at this lane's offset plus c rows
                int lo = (CAUSAL ? key : 0) - (q0 + 4 * half);
                int span = (L - 1 - (q0 + 4 * half)) - lo;
                if (key >= S || span < 0) {
                    lo = 32;  // no c in 0..27 passes
                    span = 0;
                }
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int qi = 32 * qb + 8 * g + 4 * half;  // 4 consecutive queries
                    const f32x4 l4 = *(const f32x4 *)&sL[buf][qi];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * g + e;
                        float add = 0.0f;  // MASK 4: already in s
                        bool ok = (uint32_t)(8 * g + e - lo) <= (uint32_t)span;
                        if constexpr (MASK == 1) ok = ok && mbyte[i] != 0u;
                        else if constexpr (MASK == 2) add = madd[i] * inv_scale;
                        const float pv = ok ? fast_exp2(fmaf(s[i] + add, c, -l4[e])) : 0.0f;
                        p[i] = DROP ? pv * mult(i) : pv;
                        ds[i] = pv * dp[i];
                    }
                }
            }
            // P and dS as hi + lo operands for both types: dV and dK sum a key's terms over every
            // query row, so the rounding of a single fp16 operand grows with P's column sums (a
            // causal key 0 collects P of every row: measured 1.27x the 2e-3 bar on fp16 dV)
            V8 pa[2], pal[2], da[2], dal[2];
#pragma unroll
            for (int hs = 0; hs < 2; ++hs) {
                pack8_hilo<T>(p + 8 * hs, pa[hs], pal[hs]);
                pack8_hilo<T>(ds + 8 * hs, da[hs], dal[hs]);
            }
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int hs = 0; hs < 2; ++hs) {
                    const int row = 32 * qb + 16 * hs + 4 * (g16 >> 1) + (i16 >> 2);
                    const int col = 32 * db + 16 * (g16 & 1) + 4 * (i16 & 3);
                    const V8 gt = read_tr8<T>(&cG[row * QP + col], &cG[(row + 8) * QP + col]);
                    const V8 qt = read_tr8<T>(&cQ[row * QP + col], &cQ[(row + 8) * QP + col]);
                    dv[db] = M::mma(pa[hs], gt, dv[db]);
                    dk[db] = M::mma(da[hs], qt, dk[db]);
                    dv[db] = M::mma(pal[hs], gt, dv[db]);
                    dk[db] = M::mma(dal[hs], qt, dk[db]);
                }
            }
        }
        if (st + 1 < nsteps) {
            store_step(buf ^ 1);
            if (st + 2 < nsteps) load_step(st + 2);
        }
        __syncthreads();
    }

    // dK[key][d] (scaled) and dV[key][d]: accumulator row = key wk0 + 8(i/4) + 4half + i%4, column d
    float *dkp = (float *)a.dk + (bk * f.S) * D;
    float *dvp = (float *)a.dv + (bk * f.S) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kr = wk0 + 8 * (i / 4) + 4 * half + (i % 4);
            if (kr < S) {
                dkp[(int64_t)kr * D + 32 * db + lrow] = dk[db][i] * f.scale;
                dvp[(int64_t)kr * D + 32 * db + lrow] = dv[db][i];
            }
        }
    }
}

// ---- dQ --------------------------------------------------------------------------------------

// (two per SIMD for D = 64 as in dK/dV, except with a per-element mask, which would spill)
// MASK 5 / 6: bool / float per-element mask with contiguous keys and 4-key aligned rows, read
// as a lane's 4 consecutive keys per load at the start of the tile (as the forward).
template <typename T, int D, bool CAUSAL, int MASK, bool DROP = false>
__global__ __launch_bounds__(256, D <= 64 && (MASK == 0 || MASK == 4) ? 2 : 1) void bwd_dq_kernel(AttnBwdArgs a, int nq) {
    using M = Mfma<T>;
    using V8 = typename M::V8;
    constexpr int DT = D / 16, DB = D / 32, CH = D / 8;
    constexpr int KP = D + 16;  // K tile: row reads and transposed reads
    constexpr int VP = D + 8;   // V tile: row reads
    constexpr int NLD = BNK * CH / 256;
    __shared__ __attribute__((aligned(16))) T sK[2][BNK * KP];
    __shared__ __attribute__((aligned(16))) T sV[2][BNK * VP];
    __shared__ __attribute__((aligned(16))) float sMk[MASK == 4 ? 2 : 1][BNK];  // MASK 4: the tile's mask row

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int g16 = lane >> 4, i16 = lane & 15;
    const int64_t BH = f.B * f.H;
    const int qt = nq - 1 - (int)(blockIdx.x / BH);
    const int64_t bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / f.H, h = bh % f.H, hk = h / (f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = qt * BMQ, wq0 = q0 + 32 * w, lq = wq0 + lrow;
    const int lqc = min(lq, L - 1);
    const float c = f.scale * kLog2e, inv_scale = 1.0f / f.scale;
    const float dscale = DROP ? (float)f.drop.scale : 1.0f;
    // dropout: Philox block of keys 0..3 of this lane's row
    const uint64_t drow = DROP ? (uint64_t)(bh * f.L + lq) * (uint64_t)((f.S + 3) / 4) : 0;

    V8 qf[DT], gf[DT];
    {
        const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)lqc * f.q_sl + 8 * half;
        const T *gr = (const T *)a.dout + (bh * f.L + lqc) * D + 8 * half;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            qf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 16 * t));
            gf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(gr + 16 * t));
        }
    }
    const float lse2 = ((const float *)f.lse)[bh * f.L + lqc] * kLog2e;
    // delta = rowsum(dO * O) of this lane's query (the two lanes of a row each hold half of it;
    // O is the training forward's float32 output when given, else the rounded one), written for
    // the dK/dV kernel that runs next; dP accumulates onto -delta (no per-element subtract)
    f32x16 dinit;
    float dlt;
    {
        float part = 0.0f;
        if (a.o_f32) {
            const float *orow = (const float *)f.o + (bh * f.L + lqc) * D + 8 * half;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const f32x4 o0 = *(const f32x4 *)(orow + 16 * t), o1 = *(const f32x4 *)(orow + 16 * t + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    part = fmaf((float)gf[t][e], o0[e], part);
                    part = fmaf((float)gf[t][e + 4], o1[e], part);
                }
            }
        } else {
            const T *orow = (const T *)f.o + (bh * f.L + lqc) * D + 8 * half;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const V8 ov = __builtin_bit_cast(V8, *(const u32x4 *)(orow + 16 * t));
#pragma unroll
                for (int e = 0; e < 8; ++e) part = fmaf((float)gf[t][e], (float)ov[e], part);
            }
        }
        dlt = xhalf_sum(part);
        if (half == 0 && lq < L) ((float *)a.delta)[bh * f.L + lq] = dlt;
        // (dropout: dP starts at 0, -delta is added after the multiplier)
#pragma unroll
        for (int i = 0; i < 16; ++i) dinit[i] = DROP ? 0.0f : -dlt;
    }

    f32x16 dq[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq[db][i] = 0.0f;

    const T *kbase = (const T *)f.k + b * f.k_sb + hk * f.k_sh;
    const T *vbase = (const T *)f.v + b * f.v_sb + hk * f.v_sh;
    const int kv_end = CAUSAL ? min(q0 + BMQ, S) : S;
    const int ntiles = (kv_end + BNK - 1) / BNK;
    u32x4 kreg[NLD], vreg[NLD];
    float mreg = 0.0f;
    const float *mrow = MASK == 4 ? (const float *)f.mask + b * f.m_sb + h * f.m_sh : nullptr;
    auto load_tile = [&](int j) {
        // the raw mask value: scaled at store time, so that nothing waits for the load here
        if (MASK == 4 && tid < BNK) mreg = mrow[(int64_t)min(j * BNK + tid, S - 1) * f.m_ss];
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int cidx = tid + 256 * i, row = cidx / CH, col = cidx % CH;
            const int kk = min(j * BNK + row, S - 1);
            kreg[i] = *(const u32x4 *)(kbase + (int64_t)kk * f.k_ss + 8 * col);
            vreg[i] = *(const u32x4 *)(vbase + (int64_t)kk * f.v_ss + 8 * col);
        }
    };
    auto store_tile = [&](int buf) {
        if (MASK == 4 && tid < BNK) sMk[buf][tid] = mreg * inv_scale;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int cidx = tid + 256 * i, row = cidx / CH, col = cidx % CH;
            *(u32x4 *)&sK[buf][row * KP + 8 * col] = kreg[i];
            *(u32x4 *)&sV[buf][row * VP + 8 * col] = vreg[i];
        }
    };

    if (ntiles > 0) {
        load_tile(0);
        store_tile(0);
        if (ntiles > 1) load_tile(1);
    }
    __syncthreads();
    for (int j = 0; j < ntiles; ++j) {
        const int buf = j & 1, k0 = j * BNK;
        if constexpr (D <= 64) progress_priority(j);  // two workgroups per CU with MASK 0 / 4 (one otherwise: no effect)
        const T *cK = sK[buf];
        const T *cV = sV[buf];
        if (!CAUSAL || k0 <= wq0 + 31) {
            // MASK 5 / 6: keys k0 + 32kb + 8g + 4half + 0..3 of this lane's row (starts past
            // the last 4 keys read those: their scores are blocked)
            constexpr bool MVEC = MASK >= 5;
            f32x4 mvf[MASK == 6 ? 2 : 1][4];
            uint32_t mvb[MASK == 5 ? 2 : 1][4];
            if constexpr (MVEC) {
                const int64_t mrb = b * f.m_sb + h * f.m_sh + (int64_t)lqc * f.m_sl;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int64_t at = mrb + min(k0 + 32 * kb + 8 * g + 4 * half, S - 4);
                        if constexpr (MASK == 5) mvb[kb][g] = *(const uint32_t *)((const uint8_t *)f.mask + at);
                        else mvf[kb][g] = *(const f32x4 *)((const float *)f.mask + at);
                    }
            }
            // s[kb][i]: key k0 + 32kb + 8(i/4) + 4half + i%4, query lq.  S accumulates onto the
            // tile's mask row (MASK 4: the keys' additive terms), dP onto -delta.
            f32x16 s[2], dp[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                f32x16 sinit;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 mv = MASK == 4 ? *(const f32x4 *)&sMk[buf][32 * kb + 8 * g + 4 * half]
                                               : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int e = 0; e < 4; ++e) sinit[4 * g + e] = mv[e];
                }
#pragma unroll
                for (int t = 0; t < DT; ++t) {
                    const V8 ka = *(const V8 *)&cK[(32 * kb + lrow) * KP + 16 * t + 8 * half];
                    const V8 va = *(const V8 *)&cV[(32 * kb + lrow) * VP + 16 * t + 8 * half];
                    s[kb] = M::mma(ka, qf[t], t == 0 ? sinit : s[kb]);
                    dp[kb] = M::mma(va, gf[t], t == 0 ? dinit : dp[kb]);
                }
            }
            V8 sb[2][2], sl[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                float ds[16];
                // every (query, key) of the block visible and no per-element mask: no tests
                const int kb0 = k0 + 32 * kb;
                if constexpr (DROP) {
                    // entries 4g .. 4g+3: keys kb0 + 8g + 4half + 0..3, one Philox block; the
                    // decisions also go out as bit 8g + 4half + e of the (row, 32 keys) word
                    uint32_t bits = 0u;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const GtWord4 x = gt_philox4x32_10(drow + (uint64_t)((kb0 + 8 * g + 4 * half) >> 2),
                                                           f.drop.offset, f.drop.seed);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const bool keep = x.w[e] < f.drop.thresh;
                            bits |= (keep ? 1u : 0u) << (8 * g + 4 * half + e);
                            dp[kb][4 * g + e] = fmaf(dp[kb][4 * g + e], keep ? dscale : 0.0f, -dlt);
                        }
                    }
                    const auto r = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
                    if (a.dbits && half == 0 && lq < L && kb0 < S)
                        a.dbits[(bh * f.L + lq) * ((f.S + 31) / 32) + kb0 / 32] = r[0] | r[1];
                }
                const bool interior =
                    (MASK == 0 || MASK == 4) && kb0 + 31 < S && wq0 + 31 < L && (!CAUSAL || wq0 >= kb0 + 31);
                if (interior) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) ds[i] = fast_exp2(fmaf(s[kb][i], c, -lse2)) * dp[kb][i];
                } else {
                    // key kb0 + 4half + c (c = 8(i/4) + i%4) is visible to this lane's row when c <= vis
                    const int vis = (lq < L ? (CAUSAL ? min(lq, S - 1) : S - 1) : -1) - (kb0 + 4 * half);
                    // per-element mask: this lane's offset plus c keys where visible, else the
                    // lane's row at the last key (unconditional loads: no branch per element)
                    const int64_t mrow0 = b * f.m_sb + h * f.m_sh + (int64_t)lqc * f.m_sl;
                    const int64_t mlane = mrow0 + (int64_t)(kb0 + 4 * half) * f.m_ss;
                    const int64_t msafe = mrow0 + (int64_t)(S - 1) * f.m_ss;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        float add = 0.0f;  // MASK 4: already in s
                        const int ck = 8 * (i / 4) + (i % 4);
                        bool ok = ck <= vis;
                        if constexpr (MASK == 1 || MASK == 2) {
                            const int64_t mi = ok ? mlane + (int64_t)ck * f.m_ss : msafe;
                            if constexpr (MASK == 1) ok = ok && ((const uint8_t *)f.mask)[mi] != 0;
                            else add = ((const float *)f.mask)[mi] * inv_scale;
                        } else if constexpr (MVEC) {
                            if constexpr (MASK == 5) ok = ok && ((mvb[kb][i / 4] >> (8 * (i % 4))) & 0xffu) != 0;
                            else add = mvf[kb][i / 4][i % 4] * inv_scale;
                        }
                        const float pv = ok ? fast_exp2(fmaf(s[kb][i] + add, c, -lse2)) : 0.0f;
                        ds[i] = pv * dp[kb][i];
                    }
                }
                pack8_hilo<T>(ds, sb[kb][0], sl[kb][0]);
                pack8_hilo<T>(ds + 8, sb[kb][1], sl[kb][1]);
            }
            // dQ^T += K^T . dS^T
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int hs = 0; hs < 2; ++hs) {
                        const int row = 32 * kb + 16 * hs + 4 * (g16 >> 1) + (i16 >> 2);
                        const int col = 32 * db + 16 * (g16 & 1) + 4 * (i16 & 3);
                        const V8 kt = read_tr8<T>(&cK[row * KP + col], &cK[(row + 8) * KP + col]);
                        dq[db] = M::mma(kt, sb[kb][hs], dq[db]);
                        dq[db] = M::mma(kt, sl[kb][hs], dq[db]);
                    }
                }
            }
        }
        if (j + 1 < ntiles) {
            store_tile(buf ^ 1);
            if (j + 2 < ntiles) load_tile(j + 2);
        }
        __syncthreads();
    }
    if (lq < L) {
        float *row = (float *)a.dq + (bh * f.L + lq) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = {dq[db][4 * g] * f.scale, dq[db][4 * g + 1] * f.scale, dq[db][4 * g + 2] * f.scale,
                                 dq[db][4 * g + 3] * f.scale};
                *(f32x4 *)(row + 32 * db + 8 * g + 4 * half) = v;
            }
    }
}

template <typename T, int D, bool CAUSAL, int MASK, bool DROP>
hipError_t launch_bwd_drop(const AttnBwdArgs &a, hipStream_t s) {
    const AttnFwdArgs &f = a.f;
    // dQ first: it computes delta = rowsum(dO * O) per query row, which dK/dV reads
    const int nq = (int)((f.L + BMQ - 1) / BMQ);
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, CAUSAL, MASK, DROP>), dim3((unsigned)(nq * f.B * f.H)), dim3(256), 0, s, a, nq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // dK/dV reads a per-element mask one element per lane (its lanes hold one key each): modes
    // 5 / 6 are 1 / 2 there
    constexpr int MKV = MASK >= 5 ? MASK - 4 : MASK;
    const int nkt = (int)((f.S + BKV - 1) / BKV);
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, D, CAUSAL, MKV, DROP>), dim3((unsigned)(nkt * f.B * f.Hkv)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <typename T, int D, bool CAUSAL, int MASK>
hipError_t launch_bwd_typed(const AttnBwdArgs &a, hipStream_t s) {
    return a.f.dropout ? launch_bwd_drop<T, D, CAUSAL, MASK, true>(a, s) : launch_bwd_drop<T, D, CAUSAL, MASK, false>(a, s);
}

template <typename T, int D>
hipError_t launch_bwd_d(const AttnBwdArgs &a, hipStream_t s) {
    // mode 4: a float mask that does not depend on the query row (key padding); 5 / 6: bool /
    // float per-element masks with contiguous, 4-key aligned keys (attn_mask_mode)
    const int mode = attn_mask_mode(a.f);
    if (a.f.causal) {
        if (mode == 0) return launch_bwd_typed<T, D, true, 0>(a, s);
        if (mode == 1) return launch_bwd_typed<T, D, true, 1>(a, s);
        if (mode == 4) return launch_bwd_typed<T, D, true, 4>(a, s);
        if (mode == 5) return launch_bwd_typed<T, D, true, 5>(a, s);
        if (mode == 6) return launch_bwd_typed<T, D, true, 6>(a, s);
        return launch_bwd_typed<T, D, true, 2>(a, s);
    }
    if (mode == 0) return launch_bwd_typed<T, D, false, 0>(a, s);
    if (mode == 1) return launch_bwd_typed<T, D, false, 1>(a, s);
    if (mode == 4) return launch_bwd_typed<T, D, false, 4>(a, s);
    if (mode == 5) return launch_bwd_typed<T, D, false, 5>(a, s);
    if (mode == 6) return launch_bwd_typed<T, D, false, 6>(a, s);
    return launch_bwd_typed<T, D, false, 2>(a, s);
}

// ---- float32 ----------------------------------------------------------------------------------
// Float32 backward (D = Dv = 64 or 128, no mask or a key-padding row, dropout (DROP)) on
// v_mfma_f32_32x32x2_f32, with the division of work of the kernels above (dQ first, writing
// delta = rowsum(dO.O); then dK/dV) and the float32 forward's operand mapping: a 32-row block's
// row fragments take k-step t = dim t + (D/2)(lane/32), four k-steps per 16-byte LDS read, and the
// products with P or dS take k-step s = the key (dQ) or query (dK/dV) of accumulator entry s,
// 8(s/4) + 4(lane/32) + s%4, so P and dS enter as they stand.  Tiles reach LDS by DMA, 16-byte
// chunk c of tile row r at chunk c ^ (r & 15).  Float32 operands keep 24 bits: no hi/lo split.

// Tile element offsets: float d of tile row r sits at r*D + 4((d/4) ^ (r & 15)) + d%4; the
// 16-byte fragment of dims (D/2) half + 4u .. +3 of row r at r*D + 4(((D/8) half + u) ^ (r & 15)),
// which is r*D + ((4u) ^ 4((r & 15) ^ (D/8) half)) as u < D/8.
// f32_elem_ofs<D>(32m + 8(s/4) + 4 half + s%4, 32 db + lrow), the element k-step s of a 32-row
// block m and column 32 db + lrow, split into a per-lane part (one of four, by s % 4) and a
// compile-time part, so the reads take immediate offsets
template <int D>
__device__ inline int f32_col_lane(int lrow, int half, int c) {
    return 4 * D * half + (lrow & 3) + 4 * (((lrow >> 2) ^ (4 * half)) ^ c);
}
template <int D>
__host__ __device__ constexpr int f32_col_const(int s, int db, int m) {
    return 32 * m * D + 8 * D * (s >> 2) + D * (s & 3) + 4 * ((8 * db) ^ (8 * ((s >> 2) & 1)));
}
__device__ inline f32x16 mma_f32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// dQ: a workgroup owns 128 query rows (32 per wavefront), K/V tiles of 32 keys.
template <int D, bool CAUSAL, int MASK, bool DROP>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void bwd_dq_f32_kernel(AttnBwdArgs a, int nq) {
    constexpr int NW = 4, BM = 128, BN = 32, NST = 2;
    constexpr int CH = D / 4, TILE = BN * D, NPW = BN * CH / 64 / NW, DB = D / 32, DH = D / 2;
    constexpr bool MROW = MASK == 4;
    constexpr bool MEL = MASK == 1 || MASK == 2 || MASK >= 5;  // per-element mask
    constexpr bool MVEC = MASK >= 5;                           // 4 keys per mask load
    constexpr bool MBOOL = MASK == 1 || MASK == 5;
    static_assert(NPW >= 1 && CH >= 16, "tile split");
    __shared__ __attribute__((aligned(1024))) float sK[NST][TILE];
    __shared__ __attribute__((aligned(1024))) float sV[NST][TILE];
    __shared__ __attribute__((aligned(16))) float sMk[MROW ? NST : 1][64];  // keys k0 .. k0+63 (32 used)

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t BH = f.B * f.H;
    const int qt = nq - 1 - (int)(blockIdx.x / BH);
    const int64_t bh = (int64_t)blockIdx.x % BH;
    const int64_t b = bh / f.H, h = bh % f.H, hk = h / (f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = qt * BM, wq0 = q0 + 32 * w, lq = wq0 + lrow, lqc = min(lq, L - 1);
    const float c = f.scale * kLog2e, inv_scale = 1.0f / f.scale;

    // Q and dO of row lq, dims (D/2) half .. +D/2 (B operands of S^T and dP^T)
    float qf[DH], gf[DH];
    float dlt;
    {
        const float *qr = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)lqc * f.q_sl + DH * half;
        const float *gr = (const float *)a.dout + (bh * f.L + lqc) * D + DH * half;
        const float *orow = (const float *)f.o + (bh * f.L + lqc) * D + DH * half;
        float part = 0.0f;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(qr + 4 * u), g = *(const f32x4 *)(gr + 4 * u);
            const f32x4 o4 = *(const f32x4 *)(orow + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qf[4 * u + e] = x[e];
                gf[4 * u + e] = g[e];
                part = fmaf(g[e], o4[e], part);
            }
        }
        // delta = rowsum(dO * O) of this row (the two lanes of a row hold half each), for dK/dV
        dlt = xhalf_sum(part);
        if (half == 0 && lq < L) ((float *)a.delta)[bh * f.L + lq] = dlt;
#pragma unroll
        for (int u = 0; u < DH; ++u) asm volatile("" ::"v"(qf[u]), "v"(gf[u]));
    }
    const float lse2 = ((const float *)f.lse)[bh * f.L + lqc] * kLog2e;
    // dropout: Philox block of keys 0..3 of this lane's row (rows past L draw unused words)
    const uint64_t drow = DROP ? (uint64_t)(bh * f.L + lq) * (uint64_t)((f.S + 3) / 4) : 0;
    const int64_t dwords = (f.S + 31) / 32;  // decision words per row
    // per-element mask: element offset of this lane's mask row
    const int64_t mrb = MEL ? b * f.m_sb + h * f.m_sh + (int64_t)lqc * f.m_sl : 0;
    f32x16 dq[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq[db][i] = 0.0f;

    const float *kbase = (const float *)f.k + b * f.k_sb + hk * f.k_sh;
    const float *vbase = (const float *)f.v + b * f.v_sb + hk * f.v_sh;
    const int kv_end = CAUSAL ? min(q0 + BM, S) : S;
    const int ntiles = (kv_end + BN - 1) / BN;
    const uint32_t k_row = (uint32_t)f.k_ss * 4, v_row = (uint32_t)f.v_ss * 4;
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
    int cx[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) cx[c4] = f32_col_lane<D>(lrow, half, c4);
    const int kx = 4 * ((lrow & 15) ^ ((D / 8) * half));  // row fragments: lrow * D + ((4u) ^ kx)
    const float *mrow = MROW ? (const float *)f.mask + b * f.m_sb + h * f.m_sh : nullptr;
    auto issue = [&](int j) {
        const int st = j % NST;
        if constexpr (MROW)
            lds_dma4(lds_addr(&sMk[st][0]), mrow, (uint32_t)min(j * BN + lane, S - 1) * (uint32_t)f.m_ss * 4u);
        const uint32_t dk = lds_addr(&sK[st][0]) + w * NPW * 1024;
        const uint32_t dv = lds_addr(&sV[st][0]) + w * NPW * 1024;
        if (j * BN + BN <= S) {
            const char *kb = (const char *)kbase + (uint64_t)(j * BN) * k_row;
            const char *vb = (const char *)vbase + (uint64_t)(j * BN) * v_row;
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                lds_dma16(dk + n * 1024, kb, kofs_n[n]);
                lds_dma16(dv + n * 1024, vb, vofs_n[n]);
            }
        } else {
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                const uint32_t key = (uint32_t)min(j * BN + lrow_n[n], S - 1);
                lds_dma16(dk + n * 1024, kbase, key * k_row + lcol_n[n]);
                lds_dma16(dv + n * 1024, vbase, key * v_row + lcol_n[n]);
            }
        }
    };

    if (ntiles > 0) issue(0);
    for (int j = 0; j < ntiles; ++j) {
        wait_vm<0>();
        __syncthreads();
        const int st = j % NST, k0 = j * BN;
        const float *cK = sK[st];
        const float *cV = sV[st];
        if (j + 1 < ntiles) issue(j + 1);  // stage (j+1) % 2 was last read before this barrier
        if (CAUSAL && k0 > wq0 + 31) continue;  // every key of the tile follows the wave's rows
        // MVEC: the mask of keys k0 + 8g + 4half + 0..3 of this lane's row (groups past the last
        // 4 keys read those: their scores are blocked below)
        f32x4 mvf[MVEC && !MBOOL ? 4 : 1];
        uint32_t mvb[MVEC && MBOOL ? 4 : 1];
        if constexpr (MVEC) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t at = mrb + min(k0 + 8 * g + 4 * half, S - 4);
                if constexpr (MBOOL) mvb[g] = *(const uint32_t *)((const uint8_t *)f.mask + at);
                else mvf[g] = *(const f32x4 *)((const float *)f.mask + at);
            }
        }
        // S^T = K.Q^T (onto the key-padding terms), dP^T = V.dO^T (onto -delta):
        // entry i is key k0 + 8(i/4) + 4half + i%4, query lq
        f32x16 sc, dp;
        if constexpr (MROW) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 mv4 = *(const f32x4 *)&sMk[st][8 * g + 4 * half];
#pragma unroll
                for (int e = 0; e < 4; ++e) sc[4 * g + e] = mv4[e] * inv_scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) dp[i] = DROP ? 0.0f : -dlt;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const int o = lrow * D + ((4 * u) ^ kx);
            const f32x4 kv = *(const f32x4 *)&cK[o], vv = *(const f32x4 *)&cV[o];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = mma_f32x2(kv[e], qf[4 * u + e], sc);
                dp = mma_f32x2(vv[e], gf[4 * u + e], dp);
            }
        }
        if constexpr (DROP) {
            // entries 4g .. 4g+3 are keys k0 + 8g + 4half + 0..3: one Philox block; dP = m dO.V - delta
            const float dscale = (float)f.drop.scale;
            uint32_t word = 0u;  // bit k: key k0 + k kept
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const GtWord4 x = gt_philox4x32_10(drow + (uint64_t)((k0 + 8 * g + 4 * half) >> 2), f.drop.offset,
                                                   f.drop.seed);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool keep = x.w[e] < f.drop.thresh;
                    dp[4 * g + e] = fmaf(dp[4 * g + e], keep ? dscale : 0.0f, -dlt);
                    word |= (keep ? 1u : 0u) << (8 * g + 4 * half + e);
                }
            }
            // the row's word for these 32 keys (the two halves hold complementary keys), for dK/dV
            const auto r = __builtin_amdgcn_permlane32_swap(word, word, false, false);
            if (a.dbits && half == 0 && lq < L && k0 < S) a.dbits[(bh * f.L + lq) * dwords + k0 / 32] = r[0] | r[1];
        }
        float ds[16];
        const bool interior = !MEL && k0 + BN - 1 < S && wq0 + 31 < L && (!CAUSAL || wq0 >= k0 + BN - 1);
        if (interior) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ds[i] = fast_exp2(fmaf(sc[i], c, -lse2)) * dp[i];
        } else {
            // key k0 + 4half + (8(i/4) + i%4) is visible to this lane's row when that offset <= vis
            const int vis = (lq < L ? (CAUSAL ? min(lq, S - 1) : S - 1) : -1) - (k0 + 4 * half);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                bool ok = 8 * (i / 4) + (i % 4) <= vis;
                float x = sc[i];
                if constexpr (MVEC) {
                    if constexpr (MBOOL) ok = ok && ((mvb[i / 4] >> (8 * (i % 4))) & 0xffu) != 0u;
                    else x = fmaf(mvf[i / 4][i % 4], inv_scale, x);
                } else if constexpr (MEL) {
                    const int64_t mi = mrb + (int64_t)min(k0 + 8 * (i / 4) + 4 * half + (i % 4), S - 1) * f.m_ss;
                    if constexpr (MBOOL) ok = ok && ((const uint8_t *)f.mask)[mi] != 0;
                    else x = fmaf(((const float *)f.mask)[mi], inv_scale, x);
                }
                ds[i] = (ok ? fast_exp2(fmaf(x, c, -lse2)) : 0.0f) * dp[i];
            }
        }
        // dQ^T += K^T . dS^T: k-step s2 is key 8(s2/4) + 4half + s2%4, A = K[that key][32db + lrow]
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
#pragma unroll
            for (int db = 0; db < DB; ++db)
                dq[db] = mma_f32x2(cK[cx[s2 & 3] + f32_col_const<D>(s2, db, 0)], ds[s2], dq[db]);
    }
    if (lq < L) {
        float *row = (float *)a.dq + (bh * f.L + lq) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = {dq[db][4 * g] * f.scale, dq[db][4 * g + 1] * f.scale, dq[db][4 * g + 2] * f.scale,
                                 dq[db][4 * g + 3] * f.scale};
                *(f32x4 *)(row + 32 * db + 8 * g + 4 * half) = v;
            }
    }
}

// dK, dV: a workgroup owns 128 keys of one kv head (32 per wavefront, K and V rows in registers)
// and walks query steps of 64 rows over every query head of its group; Q, dO, lse and delta of a
// step reach LDS by DMA.
// (head size 64 with dropout and a per-element mask: one workgroup per CU, two would spill)
template <int D, bool CAUSAL, int MASK, bool DROP>
__global__ __launch_bounds__(256, D <= 64 && !(DROP && (MASK == 1 || MASK == 2)) ? 2 : 1) void bwd_dkdv_f32_kernel(AttnBwdArgs a) {
    constexpr int BKV = 128, BQ = 64, NST = 2, NW = 4;
    constexpr int CH = D / 4, TILE = BQ * D, NPW = BQ * CH / 64 / NW, DB = D / 32, DH = D / 2;
    static_assert(NPW >= 1 && CH >= 16, "tile split");
    __shared__ __attribute__((aligned(1024))) float sQ[NST][TILE];
    __shared__ __attribute__((aligned(1024))) float sG[NST][TILE];  // dO
    __shared__ __attribute__((aligned(16))) float sL[NST][BQ];      // lse (natural log)
    __shared__ __attribute__((aligned(16))) float sD[NST][BQ];      // delta
    // dropout decisions: word [w][r] = keys 32w .. 32w+31 of the tile for query r of the step
    __shared__ __attribute__((aligned(16))) uint32_t sDm[DROP ? NST : 1][DROP ? NW * BQ : 1];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t nbk = f.B * f.Hkv;
    const int kt = (int)(blockIdx.x / nbk);
    const int64_t bk = blockIdx.x % nbk, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int G = (int)(f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int k0 = kt * BKV, wk0 = k0 + 32 * w, key = wk0 + lrow;
    const float c = f.scale * kLog2e, inv_scale = 1.0f / f.scale;

    // K and V of this lane's key, dims (D/2) half .. +D/2 (B operands of S and dP)
    float kf[DH], vf[DH];
    {
        const int kk = min(key, S - 1);
        const float *kr = (const float *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)kk * f.k_ss + DH * half;
        const float *vr = (const float *)f.v + b * f.v_sb + hk * f.v_sh + (int64_t)kk * f.v_ss + DH * half;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(kr + 4 * u), y = *(const f32x4 *)(vr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[4 * u + e] = x[e];
                vf[4 * u + e] = y[e];
            }
        }
#pragma unroll
        for (int u = 0; u < DH; ++u) asm volatile("" ::"v"(kf[u]), "v"(vf[u]));
    }
    f32x16 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dk[db][i] = dv[db][i] = 0.0f;

    const int qstart = CAUSAL ? (k0 / BQ) * BQ : 0;
    const int nqs = L > qstart ? (L - qstart + BQ - 1) / BQ : 0;
    const int nsteps = nqs * G;
    const uint32_t q_row = (uint32_t)f.q_sl * 4, g_row = (uint32_t)D * 4;
    int lrow_n[NPW];
    uint32_t lcol_n[NPW], qofs_n[NPW], gofs_n[NPW];
#pragma unroll
    for (int n = 0; n < NPW; ++n) {
        const int slot = (w * NPW + n) * 64 + lane;
        lrow_n[n] = slot / CH;
        lcol_n[n] = 16u * (uint32_t)((slot % CH) ^ (lrow_n[n] & 15));
        qofs_n[n] = (uint32_t)lrow_n[n] * q_row + lcol_n[n];
        gofs_n[n] = (uint32_t)lrow_n[n] * g_row + lcol_n[n];
    }
    int cx[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) cx[c4] = f32_col_lane<D>(lrow, half, c4);
    const int kx = 4 * ((lrow & 15) ^ ((D / 8) * half));  // row fragments: (32m + lrow) * D + ((4u) ^ kx)
    auto issue = [&](int st) {
        const int hh = st / nqs, qs0 = qstart + (st % nqs) * BQ, sg = st % NST;
        const int64_t h = hk * G + hh;
        const float *qb = (const float *)f.q + b * f.q_sb + h * f.q_sh;
        const float *gb = (const float *)a.dout + ((b * f.H + h) * f.L) * D;
        const float *lb = (const float *)f.lse + (b * f.H + h) * f.L;
        const float *db = (const float *)a.delta + (b * f.H + h) * f.L;
        const uint32_t rq = (uint32_t)min(qs0 + lane, L - 1) * 4u;  // lane's row of lse / delta
        lds_dma4(lds_addr(&sL[sg][0]), lb, rq);
        lds_dma4(lds_addr(&sD[sg][0]), db, rq);
        if constexpr (DROP) {
            // the dQ kernel's word (row qs0 + lane, keys of this wave); 32-bit byte offsets
            // (the launcher checks the buffer's size)
            const int64_t dwords = (f.S + 31) / 32;
            const int64_t drow = (b * f.H + h) * f.L + min(qs0 + lane, L - 1);
            const uint32_t off = (uint32_t)((drow * dwords + min((int64_t)(k0 / 32 + w), dwords - 1)) * 4);
            lds_dma4(lds_addr(&sDm[sg][w * BQ]), a.dbits, off);
        }
        const uint32_t dq = lds_addr(&sQ[sg][0]) + w * NPW * 1024;
        const uint32_t dg = lds_addr(&sG[sg][0]) + w * NPW * 1024;
        if (qs0 + BQ <= L) {
            const char *qr = (const char *)qb + (uint64_t)qs0 * q_row;
            const char *gr = (const char *)gb + (uint64_t)qs0 * g_row;
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                lds_dma16(dq + n * 1024, qr, qofs_n[n]);
                lds_dma16(dg + n * 1024, gr, gofs_n[n]);
            }
        } else {
#pragma unroll
            for (int n = 0; n < NPW; ++n) {
                const uint32_t r = (uint32_t)min(qs0 + lrow_n[n], L - 1);
                lds_dma16(dq + n * 1024, qb, r * q_row + lcol_n[n]);
                lds_dma16(dg + n * 1024, gb, r * g_row + lcol_n[n]);
            }
        }
    };

    float madd = 0.0f;  // MASK 4: the key's additive term for the current head (raw units)
    if (nsteps > 0) issue(0);
    for (int st = 0; st < nsteps; ++st) {
        wait_vm<0>();
        __syncthreads();
        const int sg = st % NST;
        const int hh = st / nqs, qs0 = qstart + (st % nqs) * BQ;
        const int64_t h = hk * G + hh;
        if (st + 1 < nsteps) issue(st + 1);  // stage (st+1) % 2 was last read before this barrier
        if (MASK == 4 && st % nqs == 0) {
            madd = ((const float *)f.mask)[b * f.m_sb + h * f.m_sh + (int64_t)min(key, S - 1) * f.m_ss] * inv_scale;
        }
        const float *cQ = sQ[sg];
        const float *cG = sG[sg];
        // per-element mask (MASK 1, 2): element offset of this head's mask at this lane's key
        const int64_t mel0 = MASK == 1 || MASK == 2 ? b * f.m_sb + h * f.m_sh + (int64_t)min(key, S - 1) * f.m_ss : 0;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int q0 = qs0 + 32 * qb;
            if (CAUSAL && q0 + 31 < wk0) continue;  // every query of the block precedes our keys
            // S = Q.K^T (onto the key's mask term), dP = dO.V^T (onto -delta): entry i is query
            // q0 + 8(i/4) + 4half + i%4 (tile row 32qb + 8(i/4) + 4half + i%4), key `key`
            f32x16 sc, dp;
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[i] = madd;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 d4 = *(const f32x4 *)&sD[sg][32 * qb + 8 * g + 4 * half];
#pragma unroll
                for (int e = 0; e < 4; ++e) dp[4 * g + e] = DROP ? 0.0f : -d4[e];
            }
#pragma unroll
            for (int u = 0; u < DH / 4; ++u) {
                const int o = (32 * qb + lrow) * D + ((4 * u) ^ kx);
                const f32x4 qa = *(const f32x4 *)&cQ[o], ga = *(const f32x4 *)&cG[o];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sc = mma_f32x2(qa[e], kf[4 * u + e], sc);
                    dp = mma_f32x2(ga[e], vf[4 * u + e], dp);
                }
            }
            // dropout: multiplier of entry i (query 32qb + 8(i/4) + 4half + i%4 of the step, this
            // lane's key): bit lrow of word [w][query]; dP = m dO.V - delta
            uint32_t keep = 0u;  // bit i: entry i kept
            if constexpr (DROP) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const u32x4 dw = *(const u32x4 *)&sDm[sg][w * BQ + 32 * qb + 8 * g + 4 * half];
                    const f32x4 d4 = *(const f32x4 *)&sD[sg][32 * qb + 8 * g + 4 * half];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t bit = (dw[e] >> lrow) & 1u;
                        keep |= bit << (4 * g + e);
                        dp[4 * g + e] = fmaf(dp[4 * g + e], bit ? (float)f.drop.scale : 0.0f, -d4[e]);
                    }
                }
            }
            float p[16], ds[16];
            const bool interior = MASK != 1 && MASK != 2 && wk0 + 31 < S && q0 + 31 < L && (!CAUSAL || q0 >= wk0 + 31);
            // query q0 + 4half + c (c = 8(i/4) + i%4) sees this lane's key when lo <= c <= lo + span
            int lo = (CAUSAL ? key : 0) - (q0 + 4 * half);
            int span = (L - 1 - (q0 + 4 * half)) - lo;
            if (key >= S || span < 0) {
                lo = 32;  // no c in 0..27 passes
                span = 0;
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 l4 = *(const f32x4 *)&sL[sg][32 * qb + 8 * g + 4 * half];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * g + e;
                    bool ok = interior || (uint32_t)(8 * g + e - lo) <= (uint32_t)span;
                    float x = sc[i];
                    if constexpr (MASK == 1 || MASK == 2) {
                        // per-element mask of query q0 + 8g + 4half + e, this lane's key
                        const int64_t mi = mel0 + (int64_t)min(q0 + 8 * g + 4 * half + e, L - 1) * f.m_sl;
                        if constexpr (MASK == 1) ok = ok && ((const uint8_t *)f.mask)[mi] != 0;
                        else x = fmaf(((const float *)f.mask)[mi], inv_scale, x);
                    }
                    const float pv = ok ? fast_exp2(fmaf(x, c, -l4[e] * kLog2e)) : 0.0f;
                    p[i] = DROP ? ((keep >> i) & 1u ? pv * (float)f.drop.scale : 0.0f) : pv;
                    ds[i] = pv * dp[i];
                }
            }
            // dV += P^T.dO, dK += dS^T.Q: k-step s2 is query 8(s2/4) + 4half + s2%4 of the block
#pragma unroll
            for (int s2 = 0; s2 < 16; ++s2) {
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const int o = cx[s2 & 3] + f32_col_const<D>(s2, db, qb);
                    dv[db] = mma_f32x2(p[s2], cG[o], dv[db]);
                    dk[db] = mma_f32x2(ds[s2], cQ[o], dk[db]);
                }
            }
        }
    }

    // dK[key][d] (scaled) and dV[key][d]: accumulator row = key wk0 + 8(i/4) + 4half + i%4, column d
    float *dkp = (float *)a.dk + (bk * f.S) * D;
    float *dvp = (float *)a.dv + (bk * f.S) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kr = wk0 + 8 * (i / 4) + 4 * half + (i % 4);
            if (kr < S) {
                dkp[(int64_t)kr * D + 32 * db + lrow] = dk[db][i] * f.scale;
                dvp[(int64_t)kr * D + 32 * db + lrow] = dv[db][i];
            }
        }
    }
}

template <int D, bool CAUSAL, int MASK, bool DROP>
hipError_t launch_bwd_f32_cm(const AttnBwdArgs &a, hipStream_t s) {
    const AttnFwdArgs &f = a.f;
    const int nq = (int)((f.L + 127) / 128);
    hipLaunchKernelGGL((bwd_dq_f32_kernel<D, CAUSAL, MASK, DROP>), dim3((unsigned)(nq * f.B * f.H)), dim3(256), 0, s, a, nq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nkt = (int)((f.S + 127) / 128);
    // dK/dV reads a per-element mask one element at a time whatever its layout: modes 5, 6 as 1, 2
    constexpr int MKV = MASK == 5 ? 1 : MASK == 6 ? 2 : MASK;
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, CAUSAL, MKV, DROP>), dim3((unsigned)(nkt * f.B * f.Hkv)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int D, bool CAUSAL, bool DROP>
hipError_t launch_bwd_f32_cd(const AttnBwdArgs &a, hipStream_t s) {
    switch (attn_mask_mode(a.f)) {
        case 0: return launch_bwd_f32_cm<D, CAUSAL, 0, DROP>(a, s);
        case 1: return launch_bwd_f32_cm<D, CAUSAL, 1, DROP>(a, s);
        case 2: return launch_bwd_f32_cm<D, CAUSAL, 2, DROP>(a, s);
        case 4: return launch_bwd_f32_cm<D, CAUSAL, 4, DROP>(a, s);
        case 5: return launch_bwd_f32_cm<D, CAUSAL, 5, DROP>(a, s);
        case 6: return launch_bwd_f32_cm<D, CAUSAL, 6, DROP>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <int D, bool DROP>
hipError_t launch_bwd_f32_dd(const AttnBwdArgs &a, hipStream_t s) {
    return a.f.causal ? launch_bwd_f32_cd<D, true, DROP>(a, s) : launch_bwd_f32_cd<D, false, DROP>(a, s);
}

template <int D>
hipError_t launch_bwd_f32_d(const AttnBwdArgs &a, hipStream_t s) {
    if (!a.f.dropout) return launch_bwd_f32_dd<D, false>(a, s);
    // dropout: the dK/dV kernel reads the dQ kernel's decision words (it does not draw them)
    // through 32-bit byte offsets
    const int64_t bytes = a.f.B * a.f.H * a.f.L * ((a.f.S + 31) / 32) * 4;
    if (!a.dbits || bytes > 0xffffffffLL) return hipErrorInvalidValue;
    return launch_bwd_f32_dd<D, true>(a, s);
}

// ---- float32, small grids ----
// Fewer than 32 dQ workgroups (few heads of one or two sequences) leave the kernels above with a
// long walk per wavefront and most CUs idle.  Here a workgroup owns 32 query rows (dQ) or 32 keys
// (dK/dV) and its 4 wavefronts split the key tiles (dQ) or the (query head, query tile) steps
// (dK/dV), each accumulating its own partial gradient; the partials are summed through LDS.  The
// operand mapping is that of the kernels above; Q, K, V and dO are read straight from memory
// (16-byte row pieces as the row fragments, single floats as the per-element operands), as they
// are few and stay in L2.  Dropout (DROP) as in the kernels above: dQ draws the decisions and
// writes them as one word per (query row, 32 keys), each (row, tile) by the one wavefront that
// owns the tile; dK/dV reads the words of its 32 keys.

// element MASK term of score (q, key) in raw score units (MASK 4: the key's, MASK 2: the
// element's), and whether a bool mask (MASK 1) blocks it
template <int MASK>
__device__ inline float f32s_mask(const AttnFwdArgs &f, int64_t b, int64_t h, int q, int key, bool &ok) {
    if constexpr (MASK == 0) return 0.0f;
    const int64_t mi = b * f.m_sb + h * f.m_sh + (int64_t)q * f.m_sl + (int64_t)key * f.m_ss;
    if constexpr (MASK == 1) {
        ok = ok && ((const uint8_t *)f.mask)[mi] != 0;
        return 0.0f;
    } else {
        return ((const float *)f.mask)[mi] / f.scale;
    }
}

template <int D, bool CAUSAL, int MASK, bool DROP>
__global__ __launch_bounds__(256) void bwd_dq_f32s_kernel(AttnBwdArgs a, int ng) {
    constexpr int DH = D / 2, DB = D / 32, OP = D + 4;
    __shared__ __attribute__((aligned(16))) float sQ[4][32][OP];
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t bh = blockIdx.x / ng;
    const int rg = (int)(blockIdx.x % ng);
    const int64_t b = bh / f.H, h = bh % f.H, hk = h / (f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = 32 * rg, lq = q0 + lrow, lqc = min(lq, L - 1);
    const float c = f.scale * kLog2e;

    float qf[DH], gf[DH];  // Q and dO of row lqc, dims DH half .. +DH
    float dlt;
    {
        const float *qr = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)lqc * f.q_sl + DH * half;
        const float *gr = (const float *)a.dout + (bh * f.L + lqc) * D + DH * half;
        const float *orow = (const float *)f.o + (bh * f.L + lqc) * D + DH * half;
        float part = 0.0f;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(qr + 4 * u), g = *(const f32x4 *)(gr + 4 * u);
            const f32x4 o4 = *(const f32x4 *)(orow + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qf[4 * u + e] = x[e];
                gf[4 * u + e] = g[e];
                part = fmaf(g[e], o4[e], part);
            }
        }
        // delta = rowsum(dO * O), for dK/dV
        dlt = xhalf_sum(part);
        if (w == 0 && half == 0 && lq < L) ((float *)a.delta)[bh * f.L + lq] = dlt;
    }
    const float lse2 = ((const float *)f.lse)[bh * f.L + lqc] * kLog2e;
    const float *kbase = (const float *)f.k + b * f.k_sb + hk * f.k_sh;
    const float *vbase = (const float *)f.v + b * f.v_sb + hk * f.v_sh;
    const int kv_end = CAUSAL ? min(q0 + 32, S) : S;
    const int nt = (kv_end + 31) / 32;
    // dropout: Philox block of keys 0..3 of this lane's row (rows past L draw unused words)
    const uint64_t drow = DROP ? (uint64_t)(bh * f.L + lq) * (uint64_t)((f.S + 3) / 4) : 0;
    const int64_t dwords = (f.S + 31) / 32;  // decision words per row
    f32x16 dq[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq[db][i] = 0.0f;

    for (int t = w; t < nt; t += 4) {
        const int k0 = 32 * t;
        // S^T = K.Q^T, dP^T = V.dO^T - delta: entry i is key k0 + 8(i/4) + 4half + i%4, query lq
        const float *kr = kbase + (int64_t)min(k0 + lrow, S - 1) * f.k_ss + DH * half;
        const float *vr = vbase + (int64_t)min(k0 + lrow, S - 1) * f.v_ss + DH * half;
        f32x16 sc, dp;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sc[i] = 0.0f;
            dp[i] = DROP ? 0.0f : -dlt;
        }
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 kv = *(const f32x4 *)(kr + 4 * u), vv = *(const f32x4 *)(vr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = mma_f32x2(kv[e], qf[4 * u + e], sc);
                dp = mma_f32x2(vv[e], gf[4 * u + e], dp);
            }
        }
        if constexpr (DROP) {
            // entries 4g .. 4g+3 are keys k0 + 8g + 4half + 0..3: one Philox block; dP = m dO.V - delta
            const float dscale = (float)f.drop.scale;
            uint32_t word = 0u;  // bit k: key k0 + k kept
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const GtWord4 x = gt_philox4x32_10(drow + (uint64_t)((k0 + 8 * g + 4 * half) >> 2), f.drop.offset,
                                                   f.drop.seed);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool keep = x.w[e] < f.drop.thresh;
                    dp[4 * g + e] = fmaf(dp[4 * g + e], keep ? dscale : 0.0f, -dlt);
                    word |= (keep ? 1u : 0u) << (8 * g + 4 * half + e);
                }
            }
            // the row's word for these 32 keys (the two halves hold complementary keys)
            const auto rw = __builtin_amdgcn_permlane32_swap(word, word, false, false);
            if (half == 0 && lq < L) a.dbits[(bh * f.L + lq) * dwords + t] = rw[0] | rw[1];
        }
        const int vis = (lq < L ? (CAUSAL ? min(lq, S - 1) : S - 1) : -1) - (k0 + 4 * half);
        float ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            bool ok = 8 * (i / 4) + (i % 4) <= vis;
            const int key = min(k0 + 8 * (i / 4) + 4 * half + (i % 4), S - 1);
            const float x = sc[i] + f32s_mask<MASK>(f, b, h, lqc, key, ok);
            ds[i] = (ok ? fast_exp2(fmaf(x, c, -lse2)) : 0.0f) * dp[i];
        }
        // dQ^T += K^T . dS^T: k-step s2 is key k0 + 8(s2/4) + 4half + s2%4, A = K[that key][32db + lrow]
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) {
            const float *kk = kbase + (int64_t)min(k0 + 8 * (s2 >> 2) + 4 * half + (s2 & 3), S - 1) * f.k_ss + lrow;
#pragma unroll
            for (int db = 0; db < DB; ++db) dq[db] = mma_f32x2(kk[32 * db], ds[s2], dq[db]);
        }
    }
    // sum the four partials: entry i of dq[db] is dim 32db + 8(i/4) + 4half + i%4 of query lrow
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 v = {dq[db][4 * g], dq[db][4 * g + 1], dq[db][4 * g + 2], dq[db][4 * g + 3]};
            *(f32x4 *)&sQ[w][lrow][32 * db + 8 * g + 4 * half] = v;
        }
    __syncthreads();
    const int r = threadIdx.x >> 3, part = threadIdx.x & 7;
    if (q0 + r < L) {
        float *row = (float *)a.dq + (bh * f.L + q0 + r) * D + (D / 8) * part;
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
            f32x4 acc = *(const f32x4 *)&sQ[0][r][(D / 8) * part + 4 * j];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) {
                const f32x4 x = *(const f32x4 *)&sQ[ww][r][(D / 8) * part + 4 * j];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] += x[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] *= f.scale;
            *(f32x4 *)(row + 4 * j) = acc;
        }
    }
}

template <int D, bool CAUSAL, int MASK, bool DROP>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_f32s_kernel(AttnBwdArgs a, int nkg) {
    constexpr int DH = D / 2, DB = D / 32, OP = D + 4;
    __shared__ __attribute__((aligned(16))) float sK[4][32][OP];
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t bk = blockIdx.x / nkg;
    const int kg = (int)(blockIdx.x % nkg);
    const int64_t b = bk / f.Hkv, hk = bk % f.Hkv;
    const int G = (int)(f.H / f.Hkv);
    const int L = (int)f.L, S = (int)f.S;
    const int k0 = 32 * kg, key = k0 + lrow, kc = min(key, S - 1);
    const float c = f.scale * kLog2e;

    float kf[DH], vf[DH];  // K and V of this lane's key, dims DH half .. +DH
    {
        const float *kr = (const float *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)kc * f.k_ss + DH * half;
        const float *vr = (const float *)f.v + b * f.v_sb + hk * f.v_sh + (int64_t)kc * f.v_ss + DH * half;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(kr + 4 * u), y = *(const f32x4 *)(vr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[4 * u + e] = x[e];
                vf[4 * u + e] = y[e];
            }
        }
    }
    f32x16 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dk[db][i] = dv[db][i] = 0.0f;

    // steps: (query head hh of the group, 32-row query tile) for the tiles that can see these keys
    const int qt0 = CAUSAL ? k0 / 32 : 0;
    const int nqt = max(0, (L + 31) / 32 - qt0);
    for (int j = w; j < G * nqt; j += 4) {
        const int hh = j / nqt, q0 = 32 * (qt0 + j % nqt);
        const int64_t h = hk * G + hh, bh = b * f.H + h;
        // S = Q.K^T, dP = dO.V^T - delta: entry i is query q0 + 8(i/4) + 4half + i%4, this lane's key
        const float *qr = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)min(q0 + lrow, L - 1) * f.q_sl + DH * half;
        const float *gr = (const float *)a.dout + (bh * f.L + min(q0 + lrow, L - 1)) * D + DH * half;
        f32x16 sc, dp;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int q = min(q0 + 8 * (i / 4) + 4 * half + (i % 4), L - 1);
            sc[i] = 0.0f;
            dp[i] = DROP ? 0.0f : -((const float *)a.delta)[bh * f.L + q];
        }
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 qa = *(const f32x4 *)(qr + 4 * u), ga = *(const f32x4 *)(gr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = mma_f32x2(qa[e], kf[4 * u + e], sc);
                dp = mma_f32x2(ga[e], vf[4 * u + e], dp);
            }
        }
        float p[16], ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int qq = q0 + 8 * (i / 4) + 4 * half + (i % 4), q = min(qq, L - 1);
            bool ok = key < S && qq < L && (!CAUSAL || qq >= key);
            const float x = sc[i] + f32s_mask<MASK>(f, b, h, q, kc, ok);
            const float ls = ((const float *)f.lse)[bh * f.L + q] * kLog2e;
            const float pv = ok ? fast_exp2(fmaf(x, c, -ls)) : 0.0f;
            if constexpr (DROP) {
                // the dQ kernel's decision for (query q, this lane's key): bit lrow of its word
                const bool keep = (a.dbits[(bh * f.L + q) * ((f.S + 31) / 32) + kg] >> lrow) & 1u;
                const float m = keep ? (float)f.drop.scale : 0.0f;
                dp[i] = fmaf(dp[i], m, -((const float *)a.delta)[bh * f.L + q]);
                p[i] = pv * m;
            } else {
                p[i] = pv;
            }
            ds[i] = pv * dp[i];
        }
        // dV += P^T.dO, dK += dS^T.Q: k-step s2 is query q0 + 8(s2/4) + 4half + s2%4
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) {
            const int q = min(q0 + 8 * (s2 >> 2) + 4 * half + (s2 & 3), L - 1);
            const float *qq = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)q * f.q_sl + lrow;
            const float *gg = (const float *)a.dout + (bh * f.L + q) * D + lrow;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                dv[db] = mma_f32x2(p[s2], gg[32 * db], dv[db]);
                dk[db] = mma_f32x2(ds[s2], qq[32 * db], dk[db]);
            }
        }
    }
    // sum the four partials (dK, then dV through the same buffer): entry i of dk[db] is key
    // 8(i/4) + 4half + i%4 of the group, dim 32db + lrow
    const int r = threadIdx.x >> 3, part = threadIdx.x & 7;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        if (which) __syncthreads();  // the dK sums are read before dV overwrites the buffer
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                sK[w][8 * (i / 4) + 4 * half + (i % 4)][32 * db + lrow] = which ? dv[db][i] : dk[db][i];
        __syncthreads();
        if (k0 + r < S) {
            float *row = (float *)(which ? a.dv : a.dk) + (bk * f.S + k0 + r) * D + (D / 8) * part;
            const float mul = which ? 1.0f : f.scale;
#pragma unroll
            for (int j = 0; j < D / 32; ++j) {
                f32x4 acc = *(const f32x4 *)&sK[0][r][(D / 8) * part + 4 * j];
#pragma unroll
                for (int ww = 1; ww < 4; ++ww) {
                    const f32x4 x = *(const f32x4 *)&sK[ww][r][(D / 8) * part + 4 * j];
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] += x[e];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] *= mul;
                *(f32x4 *)(row + 4 * j) = acc;
            }
        }
    }
}

template <int D, bool CAUSAL, int MASK, bool DROP>
hipError_t launch_bwd_f32s_cmd(const AttnBwdArgs &a, hipStream_t s) {
    const AttnFwdArgs &f = a.f;
    const int ng = (int)((f.L + 31) / 32), nkg = (int)((f.S + 31) / 32);
    hipLaunchKernelGGL((bwd_dq_f32s_kernel<D, CAUSAL, MASK, DROP>), dim3((unsigned)(f.B * f.H * ng)), dim3(256), 0, s, a, ng);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_dkdv_f32s_kernel<D, CAUSAL, MASK, DROP>), dim3((unsigned)(f.B * f.Hkv * nkg)), dim3(256), 0, s, a, nkg);
    return hipGetLastError();
}

template <int D, bool CAUSAL, int MASK>
hipError_t launch_bwd_f32s_cm(const AttnBwdArgs &a, hipStream_t s) {
    if (!a.f.dropout) return launch_bwd_f32s_cmd<D, CAUSAL, MASK, false>(a, s);
    if (!a.dbits) return hipErrorInvalidValue;  // dK/dV reads the dQ kernel's decision words
    return launch_bwd_f32s_cmd<D, CAUSAL, MASK, true>(a, s);
}

template <int D, bool CAUSAL>
hipError_t launch_bwd_f32s_c(const AttnBwdArgs &a, hipStream_t s) {
    switch (attn_mask_mode(a.f)) {
        case 0: return launch_bwd_f32s_cm<D, CAUSAL, 0>(a, s);
        case 1: case 5: return launch_bwd_f32s_cm<D, CAUSAL, 1>(a, s);
        case 2: case 6: return launch_bwd_f32s_cm<D, CAUSAL, 2>(a, s);
        case 4: return launch_bwd_f32s_cm<D, CAUSAL, 2>(a, s);  // the key-padding row as a float mask with m_sl = 0
        default: return hipErrorInvalidValue;
    }
}

// fewer than 128 dQ workgroups of the kernels above (and at most 4096 query rows and keys):
// measured faster there (B2 H4 L=S=512 D64 causal 60 against 149 us, B1 H8 L=S=512 D128 142
// against 261, B1 H24 L=S=512 D64 125 against 149), mixed at 128 (B2 H8 L=S=1024 D64 227
// against 288 us, B1 H8 L=S=2048 D128 1022 against 958), slower from 192 on (B2 H16 L=S=1024
// D64 418 against 284 us): each 32-row or 32-key workgroup reads its operands itself
bool bwd_f32_small(const AttnFwdArgs &f) {
    return f.B * f.H * ((f.L + 127) / 128) < 128 && f.L <= 4096 && f.S <= 4096;
}

bool bwd_f32_supported(const AttnBwdArgs &a) {
    const AttnFwdArgs &f = a.f;
    if (f.D != f.Dv || (f.D != 64 && f.D != 128) || f.kv_len || f.q_pos) return false;
    const int mode = attn_mask_mode(f);
    // as the forward: fewer than 16 query rows take the small-grid kernels or the generic ones
    if ((f.L < 16 && !bwd_f32_small(f)) || f.L < 1 || f.S < 1 || !(f.scale > 0.0f) || !f.o || !f.lse)
        return false;  // f.o: float32 output
    // small grids take the small-grid kernels (bwd_f32_small)
    if (f.L >= (1LL << 30) || f.S >= (1LL << 30)) return false;
    const int64_t strides[] = {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 4 != 0 || st < 0) return false;  // 16-byte rows
    for (const void *p : {f.q, f.k, f.v, (const void *)a.dout, (const void *)f.o, (const void *)a.dq})
        if ((uintptr_t)p % 16 != 0) return false;
    // 32-bit byte offsets from the per-head bases: K/V rows (dQ tiles), Q and dO rows (dK/dV steps)
    if ((f.S - 1) * f.k_ss * 4 + f.D * 4 > 0xffffffffLL || (f.S - 1) * f.v_ss * 4 + f.D * 4 > 0xffffffffLL) return false;
    if ((f.L - 1) * f.q_sl * 4 + f.D * 4 > 0xffffffffLL || (f.L - 1) * f.D * 4 + f.D * 4 > 0xffffffffLL) return false;
    if (mode == 4 && (f.m_ss < 0 || (f.S - 1) * f.m_ss * 4 + 4 > 0xffffffffLL)) return false;
    return true;
}

}  // namespace

bool attn_bwd_mfma_supported(const AttnBwdArgs &a, int cd) {
    const AttnFwdArgs &f = a.f;
    if (cd == GT_F32) return bwd_f32_supported(a);
    if (cd != GT_F16 && cd != GT_BF16) return false;
    if (f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    if (f.L < 1 || f.S < 1 || !(f.scale > 0.0f) || !f.o || !f.lse) return false;
    if (f.L >= (1LL << 30) || f.S >= (1LL << 30)) return false;
    const int64_t strides[] = {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 8 != 0) return false;
    for (const void *p : {f.q, f.k, f.v, (const void *)a.dout, (const void *)f.o})
        if ((uintptr_t)p % 16 != 0) return false;
    return true;
}

bool attn_bwd_f32_split(const AttnBwdArgs &a) { return bwd_f32_small(a.f); }

hipError_t launch_attn_bwd_mfma(const AttnBwdArgs &a, int cd, hipStream_t s) {
    if (cd == GT_F32 && attn_bwd_f32_split(a)) {
        if (a.f.D == 128) return a.f.causal ? launch_bwd_f32s_c<128, true>(a, s) : launch_bwd_f32s_c<128, false>(a, s);
        return a.f.causal ? launch_bwd_f32s_c<64, true>(a, s) : launch_bwd_f32s_c<64, false>(a, s);
    }
    if (cd == GT_F32) return a.f.D == 128 ? launch_bwd_f32_d<128>(a, s) : launch_bwd_f32_d<64>(a, s);
    if (cd == GT_F16) return a.f.D == 128 ? launch_bwd_d<_Float16, 128>(a, s) : launch_bwd_d<_Float16, 64>(a, s);
    return a.f.D == 128 ? launch_bwd_d<__bf16, 128>(a, s) : launch_bwd_d<__bf16, 64>(a, s);
}
