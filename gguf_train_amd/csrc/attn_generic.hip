// Generic attention kernels: any head size, any float dtype (float32, float16, bfloat16 with
// float accumulation; float64 with double accumulation), any mask.  They carry the exact
// semantics of the reference's fused forward (csrc/gt_ops_nn.cpp:2423-2525) and of its
// backward composition (gguf_train/_functions.py:1933-1965) for the shapes the MFMA kernels
// do not take (tiny or odd head sizes, float32/float64, mixed dtypes).
//
// Forward: one wavefront per query row.  Keys are processed 64 at a time, one per lane, with
// an online softmax; the P.V product runs with lanes over the value dimension.
// Backward: a row kernel (dQ and delta = rowsum(P*dP)) and a column kernel (dK, dV) with one
// wavefront per key; both recompute P from the saved log-sum-exp.

#include "attn_common.h"
#include "gt_internal.h"

#include <cmath>

namespace {

constexpr int kRowsPerBlock = 4;  // one wavefront per row, 4 wavefronts per workgroup
constexpr int kDvChunk = 256;     // value dims handled per pass (4 per lane)

template <typename A>
__device__ inline A neg_inf() {
    return -__builtin_huge_val();
}
template <>
__device__ inline float neg_inf<float>() {
    return -__builtin_huge_valf();
}

__device__ inline float to_acc(float x, float) { return x; }
__device__ inline float to_acc(_Float16 x, float) { return (float)x; }
__device__ inline float to_acc(__bf16 x, float) { return (float)x; }
__device__ inline double to_acc(double x, double) { return x; }

__device__ inline float acc_exp(float x) { return expf(x); }
__device__ inline double acc_exp(double x) { return exp(x); }
__device__ inline float acc_log(float x) { return logf(x); }
__device__ inline double acc_log(double x) { return log(x); }

template <typename A>
__device__ inline A wave_max(A v) {
    for (int off = 32; off >= 1; off >>= 1) {
        const A o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}
template <typename A>
__device__ inline A wave_sum(A v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Applies the mask to a finite-or-not score: bool 0 -> -inf, additive -> score + value.
template <typename A>
__device__ inline A apply_mask(const AttnFwdArgs &a, A sc, int64_t b, int64_t h, int64_t l, int64_t s) {
    if (!a.mask) return sc;
    const int64_t mi = b * a.m_sb + h * a.m_sh + l * a.m_sl + s * a.m_ss;
    if (a.mask_bool) return ((const uint8_t *)a.mask)[mi] ? sc : neg_inf<A>();
    return sc + ((const A *)a.mask)[mi];
}

template <typename A>
__device__ inline void store_out(void *o, int dtype, int64_t i, A v) {
    switch (dtype) {
        case GT_F32: ((float *)o)[i] = (float)v; break;
        case GT_F64: ((double *)o)[i] = (double)v; break;
        case GT_F16: ((_Float16 *)o)[i] = (_Float16)(float)v; break;
        case GT_BF16: ((__bf16 *)o)[i] = (__bf16)(float)v; break;
        default: break;
    }
}

// Score of (l, s) for lane-private use: -inf when causally or mask-blocked.
template <typename T, typename A>
__device__ inline A score_of(const AttnFwdArgs &a, const T *qr, const T *kb, int64_t b, int64_t h, int64_t l,
                             int64_t s) {
    if (s >= attn_kv_len(a, b) || (a.causal && s > l + attn_q_pos(a, b))) return neg_inf<A>();
    const T *kr = kb + s * a.k_ss;
    A dot = 0;
    for (int64_t d = 0; d < a.D; ++d) dot += to_acc(qr[d], A()) * to_acc(kr[d], A());
    A sc = dot * (A)a.scale;
    return apply_mask<A>(a, sc, b, h, l, s);
}

template <typename T, typename A>
__global__ __launch_bounds__(256) void generic_fwd_kernel(AttnFwdArgs a, int64_t row_blocks) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int64_t bh = blockIdx.x / row_blocks;
    const int64_t l = (blockIdx.x % row_blocks) * kRowsPerBlock + w;
    if (l >= a.L) return;
    const int64_t b = bh / a.H, h = bh % a.H, g = h / (a.H / a.Hkv);
    const T *qr = (const T *)a.q + b * a.q_sb + h * a.q_sh + l * a.q_sl;
    const T *kb = (const T *)a.k + b * a.k_sb + g * a.k_sh;
    const T *vb = (const T *)a.v + b * a.v_sb + g * a.v_sh;
    const int64_t row = bh * a.L + l;
    const A ninf = neg_inf<A>();

    for (int64_t dv0 = 0;; dv0 += kDvChunk) {
        A m = ninf, lsum = 0;
        A acc[kDvChunk / 64];
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) acc[j] = 0;
        for (int64_t s0 = 0; s0 < a.S; s0 += 64) {
            const int64_t s = s0 + lane;
            const A sc = s < a.S ? score_of<T, A>(a, qr, kb, b, h, l, s) : ninf;
            const A cm = wave_max(sc);
            if (!(cm > ninf)) continue;  // the whole chunk is blocked
            const A mn = cm > m ? cm : m;
            const A corr = m > ninf ? acc_exp(m - mn) : (A)0;
            lsum *= corr;
#pragma unroll
            for (int j = 0; j < kDvChunk / 64; ++j) acc[j] *= corr;
            m = mn;
            const A p = sc > ninf ? acc_exp(sc - m) : (A)0;
            lsum += wave_sum(p);
            const int nt = (int)((a.S - s0) < 64 ? (a.S - s0) : 64);
            for (int t = 0; t < nt; ++t) {
                const A pt = __shfl(p, t, 64);
                if (pt == (A)0) continue;  // the reference skips p == 0 (gt_ops_nn.cpp:2515)
                const T *vr = vb + (s0 + t) * a.v_ss;
#pragma unroll
                for (int j = 0; j < kDvChunk / 64; ++j) {
                    const int64_t d = dv0 + lane + 64 * j;
                    if (d < a.Dv) acc[j] += pt * to_acc(vr[d], A());
                }
            }
        }
        const A inv = lsum > (A)0 ? (A)1 / lsum : (A)0;
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) {
            const int64_t d = dv0 + lane + 64 * j;
            if (d < a.Dv) {
                store_out<A>(a.o, a.out_dtype, row * a.Dv + d, acc[j] * inv);
                if (a.o32) store_out<A>(a.o32, GT_F32, row * a.Dv + d, acc[j] * inv);
            }
        }
        if (dv0 == 0 && a.lse && lane == 0) {
            ((A *)a.lse)[row] = lsum > (A)0 ? m + acc_log(lsum) : (A)__builtin_huge_val();
        }
        if (dv0 + kDvChunk >= a.Dv) break;
    }
}

// dO . V[s] for lane-private use.
template <typename T, typename A>
__device__ inline A dprob_of(const AttnFwdArgs &a, const T *dor, const T *vb, int64_t s) {
    const T *vr = vb + s * a.v_ss;
    A dot = 0;
    for (int64_t d = 0; d < a.Dv; ++d) dot += to_acc(dor[d], A()) * to_acc(vr[d], A());
    return dot;
}

// Row kernel: delta[l] = sum_s P*dP, then dQ[l] = scale * sum_s P*(dP - delta) * K[s].
template <typename T, typename A>
__global__ __launch_bounds__(256) void generic_bwd_rows_kernel(AttnBwdArgs a, int64_t row_blocks) {
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int64_t bh = blockIdx.x / row_blocks;
    const int64_t l = (blockIdx.x % row_blocks) * kRowsPerBlock + w;
    if (l >= f.L) return;
    const int64_t b = bh / f.H, h = bh % f.H, g = h / (f.H / f.Hkv);
    const int64_t row = bh * f.L + l;
    const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + l * f.q_sl;
    const T *kb = (const T *)f.k + b * f.k_sb + g * f.k_sh;
    const T *vb = (const T *)f.v + b * f.v_sb + g * f.v_sh;
    const T *dor = (const T *)a.dout + row * f.Dv;
    const A lse = ((const A *)f.lse)[row];
    const A ninf = neg_inf<A>();

    A delta = 0;
    for (int64_t s0 = 0; s0 < f.S; s0 += 64) {
        const int64_t s = s0 + lane;
        A c = 0;
        if (s < f.S) {
            const A sc = score_of<T, A>(f, qr, kb, b, h, l, s);
            if (sc > ninf) c = acc_exp(sc - lse) * dprob_of<T, A>(f, dor, vb, s);
        }
        delta += wave_sum(c);
    }
    if (lane == 0) ((A *)a.delta)[row] = delta;

    for (int64_t d0 = 0;; d0 += kDvChunk) {
        A acc[kDvChunk / 64];
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) acc[j] = 0;
        for (int64_t s0 = 0; s0 < f.S; s0 += 64) {
            const int64_t s = s0 + lane;
            A ds = 0;
            if (s < f.S) {
                const A sc = score_of<T, A>(f, qr, kb, b, h, l, s);
                if (sc > ninf) {
                    const A p = acc_exp(sc - lse);
                    ds = p * (dprob_of<T, A>(f, dor, vb, s) - delta);
                }
            }
            const int nt = (int)((f.S - s0) < 64 ? (f.S - s0) : 64);
            for (int t = 0; t < nt; ++t) {
                const A dst = __shfl(ds, t, 64);
                if (dst == (A)0) continue;
                const T *kr = kb + (s0 + t) * f.k_ss;
#pragma unroll
                for (int j = 0; j < kDvChunk / 64; ++j) {
                    const int64_t d = d0 + lane + 64 * j;
                    if (d < f.D) acc[j] += dst * to_acc(kr[d], A());
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) {
            const int64_t d = d0 + lane + 64 * j;
            if (d < f.D) ((A *)a.dq)[row * f.D + d] = acc[j] * (A)f.scale;
        }
        if (d0 + kDvChunk >= f.D) break;
    }
}

// Column kernel: for key s of kv head g, sum over the group's query heads and rows:
//   dV[s] = sum P * dO[l],  dK[s] = scale * sum P*(dP - delta[l]) * Q[l].
template <typename T, typename A>
__global__ __launch_bounds__(256) void generic_bwd_cols_kernel(AttnBwdArgs a, int64_t col_blocks) {
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int64_t bg = blockIdx.x / col_blocks;
    const int64_t s = (blockIdx.x % col_blocks) * kRowsPerBlock + w;
    if (s >= f.S) return;
    const int64_t b = bg / f.Hkv, g = bg % f.Hkv;
    const int64_t group = f.H / f.Hkv;
    const T *kb = (const T *)f.k + b * f.k_sb + g * f.k_sh;
    const T *vb = (const T *)f.v + b * f.v_sb + g * f.v_sh;
    const int64_t col = bg * f.S + s;
    const A ninf = neg_inf<A>();
    const int64_t Dmax = f.D > f.Dv ? f.D : f.Dv;

    for (int64_t d0 = 0;; d0 += kDvChunk) {
        A adk[kDvChunk / 64], adv[kDvChunk / 64];
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) adk[j] = adv[j] = 0;
        for (int64_t hh = 0; hh < group; ++hh) {
            const int64_t h = g * group + hh;
            const int64_t bh = b * f.H + h;
            for (int64_t l0 = 0; l0 < f.L; l0 += 64) {
                const int64_t l = l0 + lane;
                A p = 0, ds = 0;
                if (l < f.L) {
                    const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + l * f.q_sl;
                    const A sc = score_of<T, A>(f, qr, kb, b, h, l, s);
                    if (sc > ninf) {
                        const int64_t row = bh * f.L + l;
                        p = acc_exp(sc - ((const A *)f.lse)[row]);
                        const T *dor = (const T *)a.dout + row * f.Dv;
                        ds = p * (dprob_of<T, A>(f, dor, vb, s) - ((const A *)a.delta)[row]);
                    }
                }
                const int nt = (int)((f.L - l0) < 64 ? (f.L - l0) : 64);
                for (int t = 0; t < nt; ++t) {
                    const A pt = __shfl(p, t, 64);
                    const A dst = __shfl(ds, t, 64);
                    if (pt == (A)0 && dst == (A)0) continue;
                    const int64_t row = bh * f.L + l0 + t;
                    const T *dor = (const T *)a.dout + row * f.Dv;
                    const T *qr = (const T *)f.q + b * f.q_sb + h * f.q_sh + (l0 + t) * f.q_sl;
#pragma unroll
                    for (int j = 0; j < kDvChunk / 64; ++j) {
                        const int64_t d = d0 + lane + 64 * j;
                        if (d < f.Dv) adv[j] += pt * to_acc(dor[d], A());
                        if (d < f.D) adk[j] += dst * to_acc(qr[d], A());
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kDvChunk / 64; ++j) {
            const int64_t d = d0 + lane + 64 * j;
            if (d < f.Dv) ((A *)a.dv)[col * f.Dv + d] = adv[j];
            if (d < f.D) ((A *)a.dk)[col * f.D + d] = adk[j] * (A)f.scale;
        }
        if (d0 + kDvChunk >= Dmax) break;
    }
}

template <typename T, typename A>
hipError_t launch_fwd(const AttnFwdArgs &a, hipStream_t s) {
    const int64_t row_blocks = (a.L + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t grid = row_blocks * a.B * a.H;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL((generic_fwd_kernel<T, A>), dim3((unsigned)grid), dim3(256), 0, s, a, row_blocks);
    return hipGetLastError();
}

template <typename T, typename A>
hipError_t launch_bwd(const AttnBwdArgs &a, hipStream_t s) {
    const AttnFwdArgs &f = a.f;
    const int64_t row_blocks = (f.L + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t rgrid = row_blocks * f.B * f.H;
    if (rgrid > 0) {
        hipLaunchKernelGGL((generic_bwd_rows_kernel<T, A>), dim3((unsigned)rgrid), dim3(256), 0, s, a, row_blocks);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int64_t col_blocks = (f.S + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t cgrid = col_blocks * f.B * f.Hkv;
    if (cgrid > 0) {
        hipLaunchKernelGGL((generic_bwd_cols_kernel<T, A>), dim3((unsigned)cgrid), dim3(256), 0, s, a, col_blocks);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_generic_fwd(const AttnFwdArgs &a, int cd, hipStream_t s) {
    switch (cd) {
        case GT_F32: return launch_fwd<float, float>(a, s);
        case GT_F16: return launch_fwd<_Float16, float>(a, s);
        case GT_BF16: return launch_fwd<__bf16, float>(a, s);
        case GT_F64: return launch_fwd<double, double>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_generic_bwd(const AttnBwdArgs &a, int cd, hipStream_t s) {
    switch (cd) {
        case GT_F32: return launch_bwd<float, float>(a, s);
        case GT_F16: return launch_bwd<_Float16, float>(a, s);
        case GT_BF16: return launch_bwd<__bf16, float>(a, s);
        case GT_F64: return launch_bwd<double, double>(a, s);
        default: return hipErrorInvalidValue;
    }
}
