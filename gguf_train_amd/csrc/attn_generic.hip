// Generic attention kernels: any head size, any float dtype (float32, float16, bfloat16 with
// float accumulation; float64 with double accumulation), any mask.  They carry the exact
// semantics of the reference's fused forward (csrc/gt_ops_nn.cpp:2423-2525) and of its
// backward composition (gguf_train/_functions.py:1933-1965) for the shapes the MFMA kernels
// do not take (tiny or odd head sizes, float32/float64, mixed dtypes).
//
// Forward: one wavefront per query row.  Keys are processed in chunks, with an online softmax;
// the P.V product runs with lanes over the value dimension.  When a chunk of K and V fits in
// LDS (head sizes up to a few hundred), the 4 rows of a workgroup share chunks staged there
// (generic_fwd_lds_kernel); otherwise each lane reads its key row from global memory.
// Backward: a row kernel (dQ and delta = rowsum(P*dP)) and a column kernel (dK, dV) with one
// wavefront per key; both recompute P from the saved log-sum-exp.
// Dropout (a.dropout): the forward's P.V takes P * m (m = the element's multiplier, 0 or
// 1/(1-p), gt_philox.h) while the normaliser sums P; the backward uses dV = (P*m)^T.dO and
// dP = m * dO.V^T in dS = P * (dP - delta), delta = rowsum(P * dP) = rowsum(dO * O).

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

// Dropout multiplier of element (row, s) (1 without dropout).
template <typename A>
__device__ inline A drop_mult(const AttnFwdArgs &a, int64_t row, int64_t s) {
    if (!a.dropout) return (A)1;
    return gt_dropout_mult<A>(a.drop, row, a.S, s, (A)a.drop.scale);
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
            const A pd = sc > ninf ? p * drop_mult<A>(a, row, s) : (A)0;  // P.V weight
            const int nt = (int)((a.S - s0) < 64 ? (a.S - s0) : 64);
            for (int t = 0; t < nt; ++t) {
                const A pt = __shfl(pd, t, 64);
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

// Wave-wide max / sum whose result every lane holds: DPP within rows of 16 (quad swaps, then
// the half-row and row mirrors), then the row and half swaps (v_permlane16/32_swap); all in
// registers.  Max keeps generic_fwd_kernel's comparison (a NaN on the right is not taken).
template <int CTRL>
__device__ inline float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ inline float max_by(float a, float b) { return b > a ? b : a; }
__device__ inline float wave_max_reg(float v) {
    v = max_by(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
    v = max_by(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
    v = max_by(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = max_by(v, dpp_mov<0x140>(v));  // row_mirror
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = max_by(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max_by(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_sum_reg(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline double wave_max_reg(double v) { return wave_max(v); }
__device__ inline double wave_sum_reg(double v) { return wave_sum(v); }
// v of lane t (t wave-uniform)
__device__ inline float lane_value(float v, int t) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), t));
}
__device__ inline double lane_value(double v, int t) {
    const int64_t x = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, t);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), t);
    return __longlong_as_double((int64_t)(((uint64_t)hi << 32) | lo));
}

// Copies rows [0, nk) of a row-major block (row r at base + r * rs, D values each) into LDS
// through put(r, d, value), and zeros for rows nk .. NR - 1.  Thread t owns column t % D of
// rows t / D, t / D + 256 / D, ... (D <= 256; columns t, t + 256, ... of every row otherwise):
// the loads of 8 rows are issued before their stores, so their latencies overlap.
template <int NR, typename T, typename A, typename F>
__device__ inline void stage_rows(const T *base, int64_t rs, int nk, int D, int tid, F put) {
    const bool narrow = D <= 256;
    const int rstep = narrow ? 256 / D : 1;
    const int r0 = narrow ? tid / D : 0;
    if (r0 >= rstep) return;
    for (int d = narrow ? tid % D : tid; d < D; d += narrow ? D : 256) {
        for (int rb = r0; rb < NR; rb += 8 * rstep) {
            A buf[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int r = rb + u * rstep;
                buf[u] = r < nk ? to_acc(base[(int64_t)r * rs + d], A()) : (A)0;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int r = rb + u * rstep;
                if (r < NR) put(r, d, buf[u]);
            }
        }
    }
}

// Forward with the key/value chunks staged in LDS: the 4 query rows of a workgroup share each
// chunk of NK keys (64, 32 or 16, the largest whose K and V fit; LPK = 64 / NK lanes per key).
// The chunk is read once, coalesced, converted to the accumulation type; K is stored transposed
// (Kt[d][key], rows of NK + 1) so that the lanes of a key column read consecutive words and the
// transposing stores of consecutive dims land in distinct banks.  Lane (key = lane % NK,
// part = lane / NK) sums dims [part*DP, part*DP + DP) of its key's dot product; shuffles across
// the parts complete it.  Then the same online softmax and P.V as generic_fwd_kernel (lanes over
// the value dims, terms with p == 0 skipped), with register-only reductions and broadcasts.
template <typename T, typename A, int NK, int NJ>
__global__ __launch_bounds__(256) void generic_fwd_lds_kernel(AttnFwdArgs a, int64_t row_blocks) {
    constexpr int LPK = 64 / NK, KT = NK + 1;
    extern __shared__ __attribute__((aligned(16))) unsigned char g_lds[];
    A *Kt = reinterpret_cast<A *>(g_lds);  // [D][KT]
    A *Vs = Kt + a.D * KT;                 // [NK][Dv]
    A *Qs = Vs + NK * a.Dv;                // [kRowsPerBlock][D]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int key = lane % NK, part = lane / NK;
    const int D = (int)a.D, Dv = (int)a.Dv;
    const int DP = (D + LPK - 1) / LPK;
    const int d_lo = min(part * DP, D), d_hi = min(d_lo + DP, D);
    const int64_t bh = blockIdx.x / row_blocks;
    const int64_t l0 = (blockIdx.x % row_blocks) * kRowsPerBlock;
    const int64_t l = l0 + w;
    const bool active = l < a.L;
    const int64_t b = bh / a.H, h = bh % a.H, g = h / (a.H / a.Hkv);
    const T *kb = (const T *)a.k + b * a.k_sb + g * a.k_sh;
    const T *vb = (const T *)a.v + b * a.v_sb + g * a.v_sh;
    const int64_t row = bh * a.L + l;
    const A ninf = neg_inf<A>();
    const int64_t kvn = attn_kv_len(a, b), qpos = attn_q_pos(a, b);
    // keys this workgroup needs: its last row's causal limit
    const int64_t l_last = min(l0 + kRowsPerBlock - 1, a.L - 1);
    const int64_t kend = min(kvn, a.causal ? l_last + qpos + 1 : a.S);
    const int64_t my_end = active ? min(kvn, a.causal ? l + qpos + 1 : a.S) : 0;

    // the query rows (zeros past L: those wavefronts compute nothing)
    stage_rows<kRowsPerBlock, T, A>((const T *)a.q + b * a.q_sb + h * a.q_sh + l0 * a.q_sl, a.q_sl,
                                    (int)min((int64_t)kRowsPerBlock, a.L - l0), D, tid,
                                    [&](int r, int d, A x) { Qs[r * D + d] = x; });
    // value dims lane, lane + 64, ... (NJ blocks of 64 cover Dv; the last one's reads clamp to
    // column Dv - 1 and its results past Dv are not stored)
    int dcol[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) dcol[j] = min(lane + 64 * j, Dv - 1);
    A m = ninf, lsum = 0;
    A acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = 0;
    // Chunk staging through registers: thread t holds column t % D of rows t / D + u * (256 / D)
    // (at most PR of them: NK * D <= 256 * PR), likewise for V.  The next chunk's loads are
    // issued before the current chunk is computed and stored to LDS after the next barrier.
    constexpr int PR = 16;
    const int kstep = 256 / D, kr0 = tid / D, kd = tid % D;
    const int vstep = 256 / Dv, vr0 = tid / Dv, vd = tid % Dv;
    A kreg[PR], vreg[PR];
    auto load_chunk = [&](int64_t c0, int n) {
#pragma unroll
        for (int u = 0; u < PR; ++u) {
            const int rk = kr0 + u * kstep, rv = vr0 + u * vstep;
            kreg[u] = (kr0 < kstep && rk < n) ? to_acc(kb[(c0 + rk) * a.k_ss + kd], A()) : (A)0;
            vreg[u] = (vr0 < vstep && rv < n) ? to_acc(vb[(c0 + rv) * a.v_ss + vd], A()) : (A)0;
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int u = 0; u < PR; ++u) {
            const int rk = kr0 + u * kstep, rv = vr0 + u * vstep;
            if (kr0 < kstep && rk < NK) Kt[kd * KT + rk] = kreg[u];
            if (vr0 < vstep && rv < NK) Vs[rv * Dv + vd] = vreg[u];
        }
    };
    if (kend > 0) load_chunk(0, (int)min((int64_t)NK, kend));
    for (int64_t s0 = 0; s0 < kend; s0 += NK) {
        const int nk = (int)min((int64_t)NK, kend - s0);
        __syncthreads();  // the previous chunk is no longer read (and Qs is written)
        store_chunk();
        __syncthreads();
        if (s0 + NK < kend) load_chunk(s0 + NK, (int)min((int64_t)NK, kend - s0 - NK));
        if (s0 >= my_end) continue;  // this row sees none of the chunk (wave-uniform)
        const int64_t s = s0 + key;
        A dot = 0;
        {
            const A *kc = Kt + key;
            const A *qr = Qs + w * D;
#pragma unroll 8
            for (int d = d_lo; d < d_hi; ++d) dot += qr[d] * kc[d * KT];
        }
#pragma unroll
        for (int off = NK; off < 64; off <<= 1) dot += __shfl_xor(dot, off, 64);
        A sc = ninf;
        if (s < my_end) sc = apply_mask<A>(a, dot * (A)a.scale, b, h, l, s);
        const A cm = wave_max_reg(sc);
        if (!(cm > ninf)) continue;  // the whole chunk is blocked for this row
        const A mn = cm > m ? cm : m;
        const A corr = m > ninf ? acc_exp(m - mn) : (A)0;
        lsum *= corr;
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[j] *= corr;
        m = mn;
        A p = sc > ninf ? acc_exp(sc - m) : (A)0;
        lsum += wave_sum_reg(part == 0 ? p : (A)0);
        if (a.dropout && p != (A)0 && part == 0) p *= drop_mult<A>(a, row, s);  // P.V weight
        // P.V over 8 keys at a time: their V words are read first; a key with p == 0 adds nothing
        // (its V word is replaced by 0, so an inf / NaN there is never touched, as the reference
        // skips such terms, gt_ops_nn.cpp:2515).  Keys past nk have p == 0 and zero rows.
        for (int t0 = 0; t0 < nk; t0 += 8) {
            A pp[8], vv[8][NJ];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                pp[u] = lane_value(p, t0 + u);  // lane t holds key t (part 0)
#pragma unroll
                for (int j = 0; j < NJ; ++j) vv[u][j] = Vs[(t0 + u) * Dv + dcol[j]];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[j] += pp[u] * (pp[u] != (A)0 ? vv[u][j] : (A)0);
        }
    }
    if (!active) return;
    const A inv = lsum > (A)0 ? (A)1 / lsum : (A)0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int64_t d = lane + 64 * j;
        if (d < Dv) {
            store_out<A>(a.o, a.out_dtype, row * Dv + d, acc[j] * inv);
            if (a.o32) store_out<A>(a.o32, GT_F32, row * Dv + d, acc[j] * inv);
        }
    }
    if (a.lse && lane == 0) ((A *)a.lse)[row] = lsum > (A)0 ? m + acc_log(lsum) : (A)__builtin_huge_val();
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
            if (sc > ninf) c = acc_exp(sc - lse) * dprob_of<T, A>(f, dor, vb, s) * drop_mult<A>(f, row, s);
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
                    ds = p * (dprob_of<T, A>(f, dor, vb, s) * drop_mult<A>(f, row, s) - delta);
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
                        const A mlt = drop_mult<A>(f, row, s);
                        ds = p * (dprob_of<T, A>(f, dor, vb, s) * mlt - ((const A *)a.delta)[row]);
                        p *= mlt;  // dV takes the dropped weight
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

// Backward with LDS staging (head sizes up to 256), the structure of generic_fwd_lds_kernel:
//   rows: the 4 query rows of a workgroup share chunks of NK keys (K and V transposed in LDS);
//         one pass per row accumulates U = sum_s P dP K[s], W = sum_s P K[s] and
//         delta = sum_s P dP, then dQ = scale (U - delta W) = scale sum_s P (dP - delta) K[s];
//   cols: the 4 keys of a workgroup share chunks of NK query rows (Q and dO transposed, with
//         their lse and delta) of every query head of the kv head's group:
//         dV[s] = sum_l P dO[l], dK[s] = scale sum_l P (dP - delta[l]) Q[l].
// Terms with P == 0 (dS == 0 for dK) are skipped, as the reference's loops skip them.  NJ
// blocks of 64 output dims per lane.
template <typename T, typename A, int NK, int NJ>
__global__ __launch_bounds__(256) void generic_bwd_rows_lds_kernel(AttnBwdArgs a, int64_t row_blocks) {
    constexpr int LPK = 64 / NK, KT = NK + 1;
    const AttnFwdArgs &f = a.f;
    extern __shared__ __attribute__((aligned(16))) unsigned char g_lds[];
    const int D = (int)f.D, Dv = (int)f.Dv;
    A *Kt = reinterpret_cast<A *>(g_lds);  // [D][KT]
    A *Vt = Kt + D * KT;                   // [Dv][KT]
    A *Qs = Vt + Dv * KT;                  // [kRowsPerBlock][D]
    A *Gs = Qs + kRowsPerBlock * D;        // [kRowsPerBlock][Dv]: dO rows
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int key = lane % NK, part = lane / NK;
    const int DPq = (D + LPK - 1) / LPK, DPv = (Dv + LPK - 1) / LPK;
    const int q_lo = min(part * DPq, D), q_hi = min(q_lo + DPq, D);
    const int v_lo = min(part * DPv, Dv), v_hi = min(v_lo + DPv, Dv);
    const int64_t bh = blockIdx.x / row_blocks;
    const int64_t l0 = (blockIdx.x % row_blocks) * kRowsPerBlock;
    const int64_t l = l0 + w;
    const bool active = l < f.L;
    const int64_t b = bh / f.H, h = bh % f.H, g = h / (f.H / f.Hkv);
    const T *kb = (const T *)f.k + b * f.k_sb + g * f.k_sh;
    const T *vb = (const T *)f.v + b * f.v_sb + g * f.v_sh;
    const int64_t row = bh * f.L + l;
    const A ninf = neg_inf<A>();
    const int64_t kvn = attn_kv_len(f, b), qpos = attn_q_pos(f, b);
    const int64_t l_last = min(l0 + kRowsPerBlock - 1, f.L - 1);
    const int64_t kend = min(kvn, f.causal ? l_last + qpos + 1 : f.S);
    const int64_t my_end = active ? min(kvn, f.causal ? l + qpos + 1 : f.S) : 0;
    const A lse = active ? ((const A *)f.lse)[row] : (A)0;

    const int nrows = (int)min((int64_t)kRowsPerBlock, f.L - l0);
    stage_rows<kRowsPerBlock, T, A>((const T *)f.q + b * f.q_sb + h * f.q_sh + l0 * f.q_sl, f.q_sl, nrows, D, tid,
                                    [&](int r, int d, A x) { Qs[r * D + d] = x; });
    stage_rows<kRowsPerBlock, T, A>((const T *)a.dout + (bh * f.L + l0) * Dv, Dv, nrows, Dv, tid,
                                    [&](int r, int d, A x) { Gs[r * Dv + d] = x; });
    int dcol[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) dcol[j] = min(lane + 64 * j, D - 1);
    A U[NJ], W[NJ], delta = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) U[j] = W[j] = 0;
    for (int64_t s0 = 0; s0 < kend; s0 += NK) {
        const int nk = (int)min((int64_t)NK, kend - s0);
        __syncthreads();  // the previous chunk is no longer read (and Qs / Gs are written)
        stage_rows<NK, T, A>(kb + s0 * f.k_ss, f.k_ss, nk, D, tid, [&](int r, int d, A x) { Kt[d * KT + r] = x; });
        stage_rows<NK, T, A>(vb + s0 * f.v_ss, f.v_ss, nk, Dv, tid, [&](int r, int d, A x) { Vt[d * KT + r] = x; });
        __syncthreads();
        if (s0 >= my_end) continue;  // this row sees none of the chunk (wave-uniform)
        const int64_t s = s0 + key;
        A dot = 0, dpd = 0;
        {
            const A *qr = Qs + w * D;
            const A *gr = Gs + w * Dv;
#pragma unroll 8
            for (int d = q_lo; d < q_hi; ++d) dot += qr[d] * Kt[d * KT + key];
#pragma unroll 8
            for (int d = v_lo; d < v_hi; ++d) dpd += gr[d] * Vt[d * KT + key];
        }
#pragma unroll
        for (int off = NK; off < 64; off <<= 1) {
            dot += __shfl_xor(dot, off, 64);
            dpd += __shfl_xor(dpd, off, 64);
        }
        A p = 0;
        if (s < my_end) {
            const A sc = apply_mask<A>(f, dot * (A)f.scale, b, h, l, s);
            if (sc > ninf) p = acc_exp(sc - lse);
        }
        if (f.dropout && p != (A)0 && part == 0) dpd *= drop_mult<A>(f, row, s);  // dP = m * dO.V
        const A pdp = p * dpd;
        delta += wave_sum_reg(part == 0 ? pdp : (A)0);
        for (int t0 = 0; t0 < nk; t0 += 8) {
            A pp[8], qq[8], kv[8][NJ];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                pp[u] = lane_value(p, t0 + u);  // lane t holds key t (part 0)
                qq[u] = lane_value(pdp, t0 + u);
#pragma unroll
                for (int j = 0; j < NJ; ++j) kv[u][j] = Kt[dcol[j] * KT + t0 + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const A x = pp[u] != (A)0 ? kv[u][j] : (A)0;
                    W[j] += pp[u] * x;
                    U[j] += qq[u] * x;
                }
        }
    }
    if (!active) return;
    if (lane == 0) ((A *)a.delta)[row] = delta;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        if (d < D) ((A *)a.dq)[row * D + d] = (U[j] - delta * W[j]) * (A)f.scale;
    }
}

template <typename T, typename A, int NQ, int NJ>
__global__ __launch_bounds__(256) void generic_bwd_cols_lds_kernel(AttnBwdArgs a, int64_t col_blocks) {
    constexpr int LPQ = 64 / NQ, QT = NQ + 1;
    const AttnFwdArgs &f = a.f;
    extern __shared__ __attribute__((aligned(16))) unsigned char g_lds[];
    const int D = (int)f.D, Dv = (int)f.Dv;
    A *Qt = reinterpret_cast<A *>(g_lds);  // [D][QT]
    A *Gt = Qt + D * QT;                   // [Dv][QT]: dO rows, transposed
    A *Ks = Gt + Dv * QT;                  // [kRowsPerBlock][D]
    A *Vs = Ks + kRowsPerBlock * D;        // [kRowsPerBlock][Dv]
    A *Ls = Vs + kRowsPerBlock * Dv;       // [NQ] lse of the chunk's rows
    A *Ds = Ls + NQ;                       // [NQ] delta of the chunk's rows
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % NQ, part = lane / NQ;
    const int DPq = (D + LPQ - 1) / LPQ, DPv = (Dv + LPQ - 1) / LPQ;
    const int q_lo = min(part * DPq, D), q_hi = min(q_lo + DPq, D);
    const int v_lo = min(part * DPv, Dv), v_hi = min(v_lo + DPv, Dv);
    const int64_t bg = blockIdx.x / col_blocks;
    const int64_t k0 = (blockIdx.x % col_blocks) * kRowsPerBlock;
    const int64_t s = k0 + w;
    const bool active = s < f.S;
    const int64_t b = bg / f.Hkv, g = bg % f.Hkv;
    const int64_t group = f.H / f.Hkv;
    const T *kb = (const T *)f.k + b * f.k_sb + g * f.k_sh;
    const T *vb = (const T *)f.v + b * f.v_sb + g * f.v_sh;
    const A ninf = neg_inf<A>();
    const int64_t kvn = attn_kv_len(f, b), qpos = attn_q_pos(f, b);
    const bool live = active && s < kvn;  // keys at or past the sequence's length are never seen

    const int nkeys = (int)min((int64_t)kRowsPerBlock, f.S - k0);
    stage_rows<kRowsPerBlock, T, A>(kb + k0 * f.k_ss, f.k_ss, nkeys, D, tid, [&](int rr, int d, A x) { Ks[rr * D + d] = x; });
    stage_rows<kRowsPerBlock, T, A>(vb + k0 * f.v_ss, f.v_ss, nkeys, Dv, tid, [&](int rr, int d, A x) { Vs[rr * Dv + d] = x; });
    int qcol[NJ], vcol[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        qcol[j] = min(lane + 64 * j, D - 1);
        vcol[j] = min(lane + 64 * j, Dv - 1);
    }
    A adk[NJ], adv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) adk[j] = adv[j] = 0;
    // (causal) rows l with l + qpos < k0 see none of the workgroup's keys
    const int64_t lstart = f.causal ? max((int64_t)0, k0 - qpos) / NQ * NQ : 0;
    const int64_t lfirst = k0 < kvn ? lstart : f.L;
    for (int64_t hh = 0; hh < group; ++hh) {
        const int64_t h = g * group + hh;
        const int64_t bh = b * f.H + h;
        for (int64_t c0 = lfirst; c0 < f.L; c0 += NQ) {
            const int nq = (int)min((int64_t)NQ, f.L - c0);
            __syncthreads();  // the previous chunk is no longer read (and Ks / Vs are written)
            stage_rows<NQ, T, A>((const T *)f.q + b * f.q_sb + h * f.q_sh + c0 * f.q_sl, f.q_sl, nq, D, tid,
                                 [&](int rr, int d, A x) { Qt[d * QT + rr] = x; });
            stage_rows<NQ, T, A>((const T *)a.dout + (bh * f.L + c0) * Dv, Dv, nq, Dv, tid,
                                 [&](int rr, int d, A x) { Gt[d * QT + rr] = x; });
            if (tid < NQ) {
                Ls[tid] = tid < nq ? ((const A *)f.lse)[bh * f.L + c0 + tid] : (A)0;
                Ds[tid] = tid < nq ? ((const A *)a.delta)[bh * f.L + c0 + tid] : (A)0;
            }
            __syncthreads();
            if (!live) continue;  // wave-uniform
            const int64_t l = c0 + r;
            A dot = 0, dpd = 0;
            {
                const A *kr = Ks + w * D;
                const A *vr = Vs + w * Dv;
#pragma unroll 8
                for (int d = q_lo; d < q_hi; ++d) dot += kr[d] * Qt[d * QT + r];
#pragma unroll 8
                for (int d = v_lo; d < v_hi; ++d) dpd += vr[d] * Gt[d * QT + r];
            }
#pragma unroll
            for (int off = NQ; off < 64; off <<= 1) {
                dot += __shfl_xor(dot, off, 64);
                dpd += __shfl_xor(dpd, off, 64);
            }
            A p = 0, ds = 0;
            if (r < nq && (!f.causal || s <= l + qpos)) {
                const A sc = apply_mask<A>(f, dot * (A)f.scale, b, h, l, s);
                if (sc > ninf) {
                    p = acc_exp(sc - Ls[r]);
                    const A mlt = drop_mult<A>(f, bh * f.L + l, s);
                    ds = p * (dpd * mlt - Ds[r]);
                    p *= mlt;  // dV takes the dropped weight
                }
            }
            for (int t0 = 0; t0 < nq; t0 += 8) {
                A pp[8], dd[8], gv[8][NJ], qv[8][NJ];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    pp[u] = lane_value(p, t0 + u);  // lane t holds row t (part 0)
                    dd[u] = lane_value(ds, t0 + u);
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        gv[u][j] = Gt[vcol[j] * QT + t0 + u];
                        qv[u][j] = Qt[qcol[j] * QT + t0 + u];
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        adv[j] += pp[u] * (pp[u] != (A)0 ? gv[u][j] : (A)0);
                        adk[j] += dd[u] * (dd[u] != (A)0 ? qv[u][j] : (A)0);
                    }
            }
        }
    }
    if (!active) return;
    const int64_t col = bg * f.S + s;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        if (d < Dv) ((A *)a.dv)[col * Dv + d] = adv[j];
        if (d < D) ((A *)a.dk)[col * D + d] = adk[j] * (A)f.scale;
    }
}

template <typename T, typename A, int NK>
hipError_t launch_lds(int nj, int64_t grid, size_t bytes, const AttnFwdArgs &a, int64_t row_blocks, hipStream_t s) {
    if (nj == 1)
        hipLaunchKernelGGL((generic_fwd_lds_kernel<T, A, NK, 1>), dim3((unsigned)grid), dim3(256), bytes, s, a, row_blocks);
    else if (nj == 2)
        hipLaunchKernelGGL((generic_fwd_lds_kernel<T, A, NK, 2>), dim3((unsigned)grid), dim3(256), bytes, s, a, row_blocks);
    else
        hipLaunchKernelGGL((generic_fwd_lds_kernel<T, A, NK, 4>), dim3((unsigned)grid), dim3(256), bytes, s, a, row_blocks);
    return hipGetLastError();
}

template <typename T, typename A>
hipError_t launch_fwd(const AttnFwdArgs &a, hipStream_t s) {
    const int64_t row_blocks = (a.L + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t grid = row_blocks * a.B * a.H;
    if (grid <= 0) return hipSuccess;
    // LDS-staged chunks (head sizes up to 256): NK keys per chunk, the largest whose K and V fit
    // in 48 KB of LDS and whose rows per staging thread (rows / (256 / D)) fit its 16 registers
    if (a.Dv <= 256 && a.D <= 256 && a.D > 0 && a.Dv > 0) {
        auto bytes = [&](int nk) { return (size_t)(a.D * (nk + 1) + nk * a.Dv + kRowsPerBlock * a.D) * sizeof(A); };
        auto rows_per_thread = [](int nk, int64_t d) { return (nk + 256 / d - 1) / (256 / d); };
        auto fits = [&](int nk) {
            return bytes(nk) <= 48 * 1024 && rows_per_thread(nk, a.D) <= 16 && rows_per_thread(nk, a.Dv) <= 16;
        };
        const int nj = a.Dv <= 64 ? 1 : a.Dv <= 128 ? 2 : 4;
        if (fits(64))
            return launch_lds<T, A, 64>(nj, grid, bytes(64), a, row_blocks, s);
        if (fits(32))
            return launch_lds<T, A, 32>(nj, grid, bytes(32), a, row_blocks, s);
        if (fits(16))
            return launch_lds<T, A, 16>(nj, grid, bytes(16), a, row_blocks, s);
    }
    hipLaunchKernelGGL((generic_fwd_kernel<T, A>), dim3((unsigned)grid), dim3(256), 0, s, a, row_blocks);
    return hipGetLastError();
}

template <typename T, typename A, int NK, int NJ>
void launch_bwd_lds(const AttnBwdArgs &a, int64_t rgrid, int64_t row_blocks, int64_t cgrid, int64_t col_blocks,
                    size_t rbytes, size_t cbytes, hipStream_t s) {
    if (rgrid > 0)
        hipLaunchKernelGGL((generic_bwd_rows_lds_kernel<T, A, NK, NJ>), dim3((unsigned)rgrid), dim3(256), rbytes, s, a,
                           row_blocks);
    if (cgrid > 0)
        hipLaunchKernelGGL((generic_bwd_cols_lds_kernel<T, A, NK, NJ>), dim3((unsigned)cgrid), dim3(256), cbytes, s, a,
                           col_blocks);
}

template <typename T, typename A, int NK>
void launch_bwd_lds_nj(int nj, const AttnBwdArgs &a, int64_t rgrid, int64_t row_blocks, int64_t cgrid,
                       int64_t col_blocks, size_t rbytes, size_t cbytes, hipStream_t s) {
    if (nj == 1) launch_bwd_lds<T, A, NK, 1>(a, rgrid, row_blocks, cgrid, col_blocks, rbytes, cbytes, s);
    else if (nj == 2) launch_bwd_lds<T, A, NK, 2>(a, rgrid, row_blocks, cgrid, col_blocks, rbytes, cbytes, s);
    else launch_bwd_lds<T, A, NK, 4>(a, rgrid, row_blocks, cgrid, col_blocks, rbytes, cbytes, s);
}

template <typename T, typename A>
hipError_t launch_bwd(const AttnBwdArgs &a, hipStream_t s) {
    const AttnFwdArgs &f = a.f;
    const int64_t row_blocks = (f.L + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t rgrid = row_blocks * f.B * f.H;
    const int64_t col_blocks = (f.S + kRowsPerBlock - 1) / kRowsPerBlock;
    const int64_t cgrid = col_blocks * f.B * f.Hkv;
    // LDS-staged kernels (head sizes up to 256): chunks of 64, 32 or 16 keys (rows for dK/dV),
    // the largest whose transposed K and V (Q and dO) fit in 48 KB
    if (f.D <= 256 && f.Dv <= 256 && f.D > 0 && f.Dv > 0) {
        const size_t dd = (size_t)(f.D + f.Dv);
        auto rbytes = [&](int nk) { return (dd * (nk + 1) + kRowsPerBlock * dd) * sizeof(A); };
        auto cbytes = [&](int nk) { return (dd * (nk + 1) + kRowsPerBlock * dd + 2 * (size_t)nk) * sizeof(A); };
        const int64_t dm = f.D > f.Dv ? f.D : f.Dv;
        const int nj = dm <= 64 ? 1 : dm <= 128 ? 2 : 4;
        constexpr size_t kMax = 48 * 1024;
        if (cbytes(64) <= kMax) launch_bwd_lds_nj<T, A, 64>(nj, a, rgrid, row_blocks, cgrid, col_blocks, rbytes(64), cbytes(64), s);
        else if (cbytes(32) <= kMax) launch_bwd_lds_nj<T, A, 32>(nj, a, rgrid, row_blocks, cgrid, col_blocks, rbytes(32), cbytes(32), s);
        else if (cbytes(16) <= kMax) launch_bwd_lds_nj<T, A, 16>(nj, a, rgrid, row_blocks, cgrid, col_blocks, rbytes(16), cbytes(16), s);
        else goto unstaged;
        return hipGetLastError();
    }
unstaged:
    if (rgrid > 0) {
        hipLaunchKernelGGL((generic_bwd_rows_kernel<T, A>), dim3((unsigned)rgrid), dim3(256), 0, s, a, row_blocks);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
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
