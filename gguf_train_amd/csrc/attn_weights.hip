// Explicit attention weights (MultiheadAttention with need_weights=True).
//
// The reference materialises them with ggml ops (gguf_train/nn/modules/transformer.py:153-166:
// scores = q.k^T * scale (+ causal, + mask), weights = softmax(scores), optionally averaged over
// the heads).  Here they are recomputed from the log-sum-exp of the fused forward, which has
// already produced the attention output: P[l, s] = exp(scores[l, s] - lse[l]), written in the
// dtype of q.  Causally excluded and masked-out positions get weight 0, a row with nothing to
// attend to is all zeros (as the fused forward's output row).
//
// float16 / bfloat16, head size 64 or 128: S = Q.K^T on v_mfma_f32_32x32x16, a wavefront owns 32
// query rows (Q in registers as the A operand) and walks the key tiles of 32; K rows are the B
// operand straight from memory (each 16-byte piece feeds one MFMA).  The accumulator holds
// S[query = 8(i/4) + 4half + i%4][key = lane % 32], so the 32 lanes of a half store 32
// consecutive keys of one query row.  HBM-bound: the weights written dominate the traffic.
// Averaged weights: a workgroup walks all H heads of its rows and writes the mean once.
// float32, head size 64 or 128: the same on v_mfma_f32_32x32x2_f32 (attn_weights_f32_kernel).
// Other dtypes / head sizes: one thread per (query, key) in the compute precision.
// Dropout (f.dropout): the weights are those the dropout forward multiplied V by, P * m with the
// element's multiplier m (gt_philox.h); computed by the per-element kernel.

#include "attn_common.h"
#include "gt_internal.h"
#include "mfma_util.h"

#include <algorithm>
#include <cmath>

namespace {

using namespace gtmfma;

constexpr int WQ = 4;  // wavefronts per workgroup: 128 query rows

template <typename T>
__device__ inline void store1(void *o, int64_t i, float v) {
    ((T *)o)[i] = (T)v;
}

template <int MASK>
__device__ inline float mask_term(const AttnFwdArgs &f, int64_t b, int64_t h, int64_t q, int64_t s, bool &blocked) {
    if (MASK == 0) return 0.0f;
    const int64_t mi = b * f.m_sb + h * f.m_sh + q * f.m_sl + s * f.m_ss;
    if (MASK == 1) {
        blocked = blocked || !((const uint8_t *)f.mask)[mi];
        return 0.0f;
    }
    return ((const float *)f.mask)[mi];
}

// grid: (row blocks of 128 queries) x (B*H, or B when averaging)
template <typename T, int D, bool CAUSAL, int MASK, bool AVG>
__global__ __launch_bounds__(64 * WQ) void attn_weights_kernel(AttnFwdArgs f, void *wout, int64_t nrb) {
    using M = Mfma<T>;
    using V8 = typename M::V8;
    constexpr int DT = D / 16;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t rb = blockIdx.x % nrb, g = blockIdx.x / nrb;
    const int64_t b = AVG ? g : g / f.H;
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = (int)rb * 32 * WQ + 32 * w;  // first query row of this wavefront
    const float c = f.scale * kLog2e;
    const int nh = AVG ? (int)f.H : 1;
    const float inv_h = 1.0f / (float)nh;
    const int kv_end = CAUSAL ? min(q0 + 32, S) : S;  // keys any of the wave's rows can see
    const int nkt = (S + 31) / 32;
    // log2(e) * lse of this lane's 16 rows (one head: loaded once)
    float lsv[16];
    if (!AVG) {
        const float *lse = (const float *)f.lse + g * f.L;
#pragma unroll
        for (int i = 0; i < 16; ++i) lsv[i] = lse[min(q0 + 8 * (i / 4) + 4 * half + (i % 4), L - 1)] * kLog2e;
    }
    for (int kt = blockIdx.y; kt < nkt; kt += gridDim.y) {  // key tiles split over blockIdx.y
        const int k0 = kt * 32;
        f32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
        if (k0 < kv_end) {
            for (int hh = 0; hh < nh; ++hh) {
                const int64_t h = AVG ? hh : g % f.H;
                const int64_t hk = h / (f.H / f.Hkv);
                // A = Q rows (query lrow of the wave, d = 16t + 8half + 0..7); B = K rows
                const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)min(q0 + lrow, L - 1) * f.q_sl + 8 * half;
                const T *kr = (const T *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)min(k0 + lrow, S - 1) * f.k_ss + 8 * half;
                f32x16 s;
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
                for (int t = 0; t < DT; ++t) {
                    const V8 qa = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 16 * t));
                    const V8 kb = __builtin_bit_cast(V8, *(const u32x4 *)(kr + 16 * t));
                    s = M::mma(qa, kb, s);
                }
                // s[i]: query q0 + 8(i/4) + 4half + i%4, key k0 + lrow
                const int key = k0 + lrow;
                const float *lse = (const float *)f.lse + (b * f.H + h) * f.L;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int q = q0 + 8 * (i / 4) + 4 * half + (i % 4);
                    bool blocked = key >= S || q >= L || (CAUSAL && key > q);
                    const float add = mask_term<MASK>(f, b, h, min(q, L - 1), min(key, S - 1), blocked);
                    const float ls = AVG ? lse[min(q, L - 1)] * kLog2e : lsv[i];
                    // lse = +inf (nothing visible): weight 0
                    const float p = blocked ? 0.0f : exp2f(fmaf(s[i], c, add * kLog2e - ls));
                    acc[i] += AVG ? p * inv_h : p;
                }
            }
        }
        // store: for fixed i, the 32 lanes of a half write 32 consecutive keys of one row
        const int key = k0 + lrow;
        if (key < S) {
            const int64_t base = AVG ? b * f.L : g * f.L;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int q = q0 + 8 * (i / 4) + 4 * half + (i % 4);
                if (q < L) store1<T>(wout, (base + q) * f.S + key, acc[i]);
            }
        }
    }
}

// The same weights for S % 8 == 0 and a 16-byte aligned output: key tiles of 64 (two 32-key
// blocks), S^T = K.Q^T so that a lane holds one query row (its log-sum-exp in one register) and
// four consecutive keys per register group, Q in registers when there is one head, blocks with
// every weight visible and no mask computed without the per-element tests, and the wavefront's
// 32 x 64 tile transposed through LDS (8-byte writes, rows padded by 16 bytes) so that each lane
// stores 16-byte pieces: 8 lanes write a row's 64 keys (128 bytes) where attn_weights_kernel
// stores 2 bytes per lane.  The same operations per weight, so the same bits.
template <typename T, int D, bool CAUSAL, int MASK, bool AVG>
__global__ __launch_bounds__(64 * WQ) void attn_weights_vec_kernel(AttnFwdArgs f, void *wout, int64_t nrb) {
    using M = Mfma<T>;
    using V8 = typename M::V8;
    constexpr int DT = D / 16;
    constexpr int RP = 64 + 8;  // LDS row pitch (elements): 64 keys and 16 bytes of padding
    __shared__ __attribute__((aligned(16))) T tile[WQ][32 * RP];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t rb = blockIdx.x % nrb, g = blockIdx.x / nrb;
    const int64_t b = AVG ? g : g / f.H;
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = (int)rb * 32 * WQ + 32 * w;  // first query row of this wavefront
    const int q = q0 + lrow;                    // this lane's query row
    const int qc = min(q, L - 1);
    const float c = f.scale * kLog2e;
    const int nh = AVG ? (int)f.H : 1;
    const float inv_h = 1.0f / (float)nh;
    const int kv_end = CAUSAL ? min(q0 + 32, S) : S;  // keys any of the wave's rows can see
    const int nkt = (S + 63) / 64;
    T *tw = tile[w];
    // one head: its Q fragments (query row lrow, d = 16t + 8half + 0..7) and log2(e) * lse
    V8 qf[DT];
    float ls1 = 0.0f;
    if (!AVG) {
        const int64_t h = g % f.H;
        const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)qc * f.q_sl + 8 * half;
#pragma unroll
        for (int t = 0; t < DT; ++t) qf[t] = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 16 * t));
        ls1 = ((const float *)f.lse)[g * f.L + qc] * kLog2e;
    }
    const int64_t base = AVG ? b * f.L : g * f.L;
    for (int kt = blockIdx.y; kt < nkt; kt += gridDim.y) {  // key tiles split over blockIdx.y
        const int k0 = kt * 64;
        f32x16 acc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[kb][i] = 0.0f;
        for (int hh = 0; hh < nh; ++hh) {
            const int64_t h = AVG ? hh : g % f.H;
            const int64_t hk = h / (f.H / f.Hkv);
            V8 qa[DT];
            float ls = ls1;
            if constexpr (AVG) {
                const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)qc * f.q_sl + 8 * half;
#pragma unroll
                for (int t = 0; t < DT; ++t) qa[t] = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 16 * t));
                ls = ((const float *)f.lse)[(b * f.H + h) * f.L + qc] * kLog2e;
            } else {
#pragma unroll
                for (int t = 0; t < DT; ++t) qa[t] = qf[t];
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int kb0 = k0 + 32 * kb;
                if (kb0 >= kv_end) continue;  // every weight of the block is 0 (acc stays 0)
                // A = K rows (key kb0 + lrow), B = Q rows: sc[i] is key kb0 + 8(i/4) + 4half + i%4, query q
                const T *kr = (const T *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)min(kb0 + lrow, S - 1) * f.k_ss + 8 * half;
                f32x16 sc;
#pragma unroll
                for (int i = 0; i < 16; ++i) sc[i] = 0.0f;
#pragma unroll
                for (int t = 0; t < DT; ++t) sc = M::mma(__builtin_bit_cast(V8, *(const u32x4 *)(kr + 16 * t)), qa[t], sc);
                const bool interior = MASK == 0 && kb0 + 31 < S && q0 + 31 < L && (!CAUSAL || kb0 + 31 <= q0);
                if (interior) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float p = exp2f(fmaf(sc[i], c, 0.0f * kLog2e - ls));
                        acc[kb][i] += AVG ? p * inv_h : p;
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = kb0 + 8 * (i / 4) + 4 * half + (i % 4);
                        bool blocked = key >= S || q >= L || (CAUSAL && key > q);
                        const float add = mask_term<MASK>(f, b, h, qc, min(key, S - 1), blocked);
                        const float p = blocked ? 0.0f : exp2f(fmaf(sc[i], c, add * kLog2e - ls));
                        acc[kb][i] += AVG ? p * inv_h : p;
                    }
                }
            }
        }
        // the tile into LDS as rows (query) x keys, four keys per 8-byte write, then 16-byte pieces
        // out: piece u * 64 + lane is row (u * 64 + lane) / 8, keys 8 * (lane % 8) .. +7
        __builtin_amdgcn_wave_barrier();  // the previous tile's reads are done
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                T v4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = (T)acc[kb][4 * gq + e];
                *(u32x2 *)&tw[lrow * RP + 32 * kb + 8 * gq + 4 * half] = __builtin_bit_cast(u32x2, v4);
            }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pc = u * 64 + lane, row = pc >> 3, key0 = k0 + 8 * (pc & 7);
            const u32x4 piece = *(const u32x4 *)&tw[row * RP + 8 * (pc & 7)];
            if (q0 + row < L && key0 < S) *(u32x4 *)((T *)wout + (base + q0 + row) * f.S + key0) = piece;
        }
    }
}

// Float32 weights, head size 64 or 128: the structure of attn_weights_vec_kernel on
// v_mfma_f32_32x32x2_f32.  S^T = K.Q^T with k-step (u, e) = dim (D/2)(lane/32) + 4u + e: a lane's
// Q values are half of its query row (D/2 floats in registers) and its K values come four
// k-steps at a time from one 16-byte load of key row lrow.  The wavefront's 32 x 64 tile goes
// through LDS (16-byte writes, rows padded by 16 bytes) and out as 16-byte pieces when S % 4 == 0
// and the output is 16-byte aligned (VEC), else as 4-byte stores of 64 consecutive keys.
template <int D, bool CAUSAL, int MASK, bool AVG, bool VEC>
__global__ __launch_bounds__(64 * WQ) void attn_weights_f32_kernel(AttnFwdArgs f, void *wout, int64_t nrb) {
    constexpr int DH = D / 2;
    constexpr int RP = 64 + 4;  // LDS row pitch (floats): 64 keys and 16 bytes of padding
    __shared__ __attribute__((aligned(16))) float tile[WQ][32 * RP];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lrow = lane & 31, half = lane >> 5;
    const int64_t rb = blockIdx.x % nrb, g = blockIdx.x / nrb;
    const int64_t b = AVG ? g : g / f.H;
    const int L = (int)f.L, S = (int)f.S;
    const int q0 = (int)rb * 32 * WQ + 32 * w;  // first query row of this wavefront
    const int q = q0 + lrow;                    // this lane's query row
    const int qc = min(q, L - 1);
    const float c = f.scale * kLog2e;
    const int nh = AVG ? (int)f.H : 1;
    const float inv_h = 1.0f / (float)nh;
    const int kv_end = CAUSAL ? min(q0 + 32, S) : S;  // keys any of the wave's rows can see
    const int nkt = (S + 63) / 64;
    float *tw = tile[w];
    // one head: its Q values (query row qc, dims DH half .. +DH) and log2(e) * lse
    float qf[DH];
    float ls1 = 0.0f;
    if (!AVG) {
        const int64_t h = g % f.H;
        const float *qr = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)qc * f.q_sl + DH * half;
#pragma unroll
        for (int u = 0; u < DH / 4; ++u) {
            const f32x4 x = *(const f32x4 *)(qr + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[4 * u + e] = x[e];
        }
        ls1 = ((const float *)f.lse)[g * f.L + qc] * kLog2e;
    }
    const int64_t base = AVG ? b * f.L : g * f.L;
    for (int kt = blockIdx.y; kt < nkt; kt += gridDim.y) {  // key tiles split over blockIdx.y
        const int k0 = kt * 64;
        f32x16 acc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[kb][i] = 0.0f;
        for (int hh = 0; hh < nh; ++hh) {
            const int64_t h = AVG ? hh : g % f.H;
            const int64_t hk = h / (f.H / f.Hkv);
            float ls = ls1;
            if constexpr (AVG) {
                const float *qr = (const float *)f.q + b * f.q_sb + h * f.q_sh + (int64_t)qc * f.q_sl + DH * half;
#pragma unroll
                for (int u = 0; u < DH / 4; ++u) {
                    const f32x4 x = *(const f32x4 *)(qr + 4 * u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) qf[4 * u + e] = x[e];
                }
                ls = ((const float *)f.lse)[(b * f.H + h) * f.L + qc] * kLog2e;
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int kb0 = k0 + 32 * kb;
                if (kb0 >= kv_end) continue;  // every weight of the block is 0 (acc stays 0)
                // A = K rows (key kb0 + lrow), B = Q: sc[i] is key kb0 + 8(i/4) + 4half + i%4, query q
                const float *kr =
                    (const float *)f.k + b * f.k_sb + hk * f.k_sh + (int64_t)min(kb0 + lrow, S - 1) * f.k_ss + DH * half;
                f32x16 sc;
#pragma unroll
                for (int i = 0; i < 16; ++i) sc[i] = 0.0f;
#pragma unroll
                for (int u = 0; u < DH / 4; ++u) {
                    const f32x4 kv = *(const f32x4 *)(kr + 4 * u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[e], qf[4 * u + e], sc, 0, 0, 0);
                }
                const bool interior = MASK == 0 && kb0 + 31 < S && q0 + 31 < L && (!CAUSAL || kb0 + 31 <= q0);
                if (interior) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float p = exp2f(fmaf(sc[i], c, 0.0f * kLog2e - ls));
                        acc[kb][i] += AVG ? p * inv_h : p;
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = kb0 + 8 * (i / 4) + 4 * half + (i % 4);
                        bool blocked = key >= S || q >= L || (CAUSAL && key > q);
                        const float add = mask_term<MASK>(f, b, h, qc, min(key, S - 1), blocked);
                        const float p = blocked ? 0.0f : exp2f(fmaf(sc[i], c, add * kLog2e - ls));
                        acc[kb][i] += AVG ? p * inv_h : p;
                    }
                }
            }
        }
        // the tile into LDS as rows (query) x keys, four keys per 16-byte write
        __builtin_amdgcn_wave_barrier();  // the previous tile's reads are done
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const f32x4 v4 = {acc[kb][4 * gq], acc[kb][4 * gq + 1], acc[kb][4 * gq + 2], acc[kb][4 * gq + 3]};
                *(f32x4 *)&tw[lrow * RP + 32 * kb + 8 * gq + 4 * half] = v4;
            }
        __builtin_amdgcn_wave_barrier();
        if constexpr (VEC) {
            // piece u * 64 + lane: row (u * 64 + lane) / 16, keys 4 * (lane % 16) .. +3
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int pc = u * 64 + lane, row = pc >> 4, key0 = k0 + 4 * (pc & 15);
                const f32x4 piece = *(const f32x4 *)&tw[row * RP + 4 * (pc & 15)];
                if (q0 + row < L && key0 < S) *(f32x4 *)((float *)wout + (base + q0 + row) * f.S + key0) = piece;
            }
        } else {
            // row r: lanes write its 64 keys
#pragma unroll 4
            for (int r = 0; r < 32; ++r) {
                const int key = k0 + lane;
                if (q0 + r < L && key < S) ((float *)wout)[(base + q0 + r) * f.S + key] = tw[r * RP + lane];
            }
        }
    }
}

// Generic: one thread per (query, key), any float dtype, accumulation in A (double for float64).
template <typename T, typename A, bool AVG>
__global__ __launch_bounds__(256) void attn_weights_generic_kernel(AttnFwdArgs f, void *wout) {
    const int64_t nrow = AVG ? f.B * f.L : f.B * f.H * f.L;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nrow * f.S) return;
    const int64_t s = i % f.S, r = i / f.S;
    const int64_t l = r % f.L, g = r / f.L;
    const int64_t b = AVG ? g : g / f.H;
    const int nh = AVG ? (int)f.H : 1;
    A sum = 0;
    for (int hh = 0; hh < nh; ++hh) {
        const int64_t h = AVG ? hh : g % f.H, hk = h / (f.H / f.Hkv);
        if (s >= attn_kv_len(f, b) || (f.causal && s > l + attn_q_pos(f, b))) continue;
        const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + l * f.q_sl;
        const T *kr = (const T *)f.k + b * f.k_sb + hk * f.k_sh + s * f.k_ss;
        A dot = 0;
        for (int64_t d = 0; d < f.D; ++d) dot += (A)(float)qr[d] * (A)(float)kr[d];
        A x = dot * (A)f.scale;
        if (f.mask) {
            const int64_t mi = b * f.m_sb + h * f.m_sh + l * f.m_sl + s * f.m_ss;
            if (f.mask_bool) {
                if (!((const uint8_t *)f.mask)[mi]) continue;
            } else {
                x += sizeof(A) == 8 ? (A)((const double *)f.mask)[mi] : (A)((const float *)f.mask)[mi];
            }
        }
        const int64_t row = (b * f.H + h) * f.L + l;
        const A ls = sizeof(A) == 8 ? (A)((const double *)f.lse)[row] : (A)((const float *)f.lse)[row];
        A p = sizeof(A) == 8 ? (A)exp((double)(x - ls)) : (A)expf((float)(x - ls));
        if (f.dropout) p *= gt_dropout_mult<A>(f.drop, row, f.S, s, (A)f.drop.scale);
        sum += p;
    }
    if (AVG) sum /= (A)nh;
    switch (f.out_dtype) {
        case GT_F64: ((double *)wout)[i] = (double)sum; break;
        case GT_F32: ((float *)wout)[i] = (float)sum; break;
        case GT_F16: ((_Float16 *)wout)[i] = (_Float16)(float)sum; break;
        case GT_BF16: ((__bf16 *)wout)[i] = (__bf16)(float)sum; break;
        default: break;
    }
}

// One thread per Philox block (4 consecutive keys of one row).
__global__ __launch_bounds__(256) void dropout_mask_kernel(GtDropout d, int keep_all, int64_t rows, int64_t S,
                                                          uint8_t *out) {
    const int64_t nb = (S + 3) / 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t row = i / nb, s0 = 4 * (i % nb);
    const GtWord4 x = gt_philox4x32_10(gt_dropout_block(row, S, s0 / 4), d.offset, d.seed);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (s0 + j < S) out[row * S + s0 + j] = keep_all || x.w[j] < d.thresh ? 1 : 0;
}

// Averaged weights run every head inside one workgroup, whose grid (query blocks x B) can be
// far smaller than the GPU: their key tiles are split over blockIdx.y up to ~1024 workgroups.
// Each weight is still computed and written by one workgroup, in the same order: the same bits.
unsigned key_splits(int64_t grid, int64_t nkt, bool avg) {
    if (!avg || grid <= 0) return 1;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(nkt, (1024 + grid - 1) / grid));
}

template <typename T, int D, bool AVG>
hipError_t launch_mfma(const AttnFwdArgs &f, void *w, hipStream_t st) {
    const int64_t nrb = (f.L + 32 * WQ - 1) / (32 * WQ);
    const int64_t grid = nrb * (AVG ? f.B : f.B * f.H);
    if (grid > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
    // whole 16-byte pieces of every row: the LDS-transposed kernel
    const bool vec = f.S % 8 == 0 && (uintptr_t)w % 16 == 0;
    const unsigned ny = key_splits(grid, vec ? (f.S + 63) / 64 : (f.S + 31) / 32, AVG);
#define GT_W(C, MK)                                                                                                     \
    do {                                                                                                                \
        if (vec) hipLaunchKernelGGL((attn_weights_vec_kernel<T, D, C, MK, AVG>), dim3((unsigned)grid, ny), dim3(64 * WQ), 0, st, f, w, nrb); \
        else hipLaunchKernelGGL((attn_weights_kernel<T, D, C, MK, AVG>), dim3((unsigned)grid, ny), dim3(64 * WQ), 0, st, f, w, nrb); \
    } while (0)
    if (f.causal) {
        if (mode == 0) GT_W(true, 0);
        else if (mode == 1) GT_W(true, 1);
        else GT_W(true, 2);
    } else {
        if (mode == 0) GT_W(false, 0);
        else if (mode == 1) GT_W(false, 1);
        else GT_W(false, 2);
    }
#undef GT_W
    return hipGetLastError();
}

template <int D, bool AVG>
hipError_t launch_f32(const AttnFwdArgs &f, void *w, hipStream_t st) {
    const int64_t nrb = (f.L + 32 * WQ - 1) / (32 * WQ);
    const int64_t grid = nrb * (AVG ? f.B : f.B * f.H);
    if (grid > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
    const bool vec = f.S % 4 == 0 && (uintptr_t)w % 16 == 0;
    const unsigned ny = key_splits(grid, (f.S + 63) / 64, AVG);
#define GT_WF(C, MK)                                                                                                    \
    do {                                                                                                                \
        if (vec) hipLaunchKernelGGL((attn_weights_f32_kernel<D, C, MK, AVG, true>), dim3((unsigned)grid, ny), dim3(64 * WQ), 0, st, f, w, nrb); \
        else hipLaunchKernelGGL((attn_weights_f32_kernel<D, C, MK, AVG, false>), dim3((unsigned)grid, ny), dim3(64 * WQ), 0, st, f, w, nrb); \
    } while (0)
    if (f.causal) {
        if (mode == 0) GT_WF(true, 0);
        else if (mode == 1) GT_WF(true, 1);
        else GT_WF(true, 2);
    } else {
        if (mode == 0) GT_WF(false, 0);
        else if (mode == 1) GT_WF(false, 1);
        else GT_WF(false, 2);
    }
#undef GT_WF
    return hipGetLastError();
}

template <typename T, typename A>
hipError_t launch_generic(const AttnFwdArgs &f, void *w, bool avg, hipStream_t st) {
    const int64_t n = (avg ? f.B * f.L : f.B * f.H * f.L) * f.S;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    if (avg) hipLaunchKernelGGL((attn_weights_generic_kernel<T, A, true>), dim3((unsigned)blocks), dim3(256), 0, st, f, w);
    else hipLaunchKernelGGL((attn_weights_generic_kernel<T, A, false>), dim3((unsigned)blocks), dim3(256), 0, st, f, w);
    return hipGetLastError();
}

}  // namespace

// `f` as for the forward (q, k, mask, lse of the same call; out_dtype = dtype of the weights);
// `w` receives (B,H,L,S), or (B,L,S) when averaging over the heads.
bool attn_weights_mfma(const AttnFwdArgs &f, int cd) {
    if ((cd != GT_F16 && cd != GT_BF16 && cd != GT_F32) || (f.D != 64 && f.D != 128) || f.out_dtype != cd) return false;
    if (f.kv_len || f.q_pos || f.dropout || (uintptr_t)f.q % 16 != 0 || (uintptr_t)f.k % 16 != 0) return false;
    const int64_t rows = cd == GT_F32 ? 4 : 8;  // 16-byte rows
    for (int64_t st : {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss})
        if (st % rows != 0) return false;
    return true;
}

hipError_t launch_attn_weights(const AttnFwdArgs &f, int cd, void *w, bool average, hipStream_t st) {
    if (f.B * f.L * f.S == 0 || f.H == 0) return hipSuccess;
    const bool mfma = attn_weights_mfma(f, cd);
    if (mfma && cd == GT_F32) {
        if (f.D == 128) return average ? launch_f32<128, true>(f, w, st) : launch_f32<128, false>(f, w, st);
        return average ? launch_f32<64, true>(f, w, st) : launch_f32<64, false>(f, w, st);
    }
    if (mfma) {
        if (cd == GT_F16) {
            if (f.D == 128) return average ? launch_mfma<_Float16, 128, true>(f, w, st) : launch_mfma<_Float16, 128, false>(f, w, st);
            return average ? launch_mfma<_Float16, 64, true>(f, w, st) : launch_mfma<_Float16, 64, false>(f, w, st);
        }
        if (f.D == 128) return average ? launch_mfma<__bf16, 128, true>(f, w, st) : launch_mfma<__bf16, 128, false>(f, w, st);
        return average ? launch_mfma<__bf16, 64, true>(f, w, st) : launch_mfma<__bf16, 64, false>(f, w, st);
    }
    switch (cd) {
        case GT_F64: return launch_generic<double, double>(f, w, average, st);
        case GT_F16: return launch_generic<_Float16, float>(f, w, average, st);
        case GT_BF16: return launch_generic<__bf16, float>(f, w, average, st);
        default: return launch_generic<float, float>(f, w, average, st);
    }
}

hipError_t launch_dropout_mask(const GtDropout &d, bool keep_all, int64_t rows, int64_t S, uint8_t *out, hipStream_t st) {
    const int64_t n = rows * ((S + 3) / 4);
    if (n == 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(dropout_mask_kernel, dim3((unsigned)blocks), dim3(256), 0, st, d, keep_all ? 1 : 0, rows, S, out);
    return hipGetLastError();
}
