// Single-query (decode) attention: split-K over the KV length with every query head of a GQA
// group in one workgroup, so each K/V byte is read from HBM exactly once.
//
// The reference has no decode kernel: decode is gt_flash_attention with L = 1
// (csrc/gt_ops_nn.cpp:2423-2525), whose loop reads a kv head once per query head.  Semantics
// kept: scale, additive/bool mask, top-left causal (only key 0 when L = 1), empty rows -> 0.
//
// Work decomposition (HBM-bound; bytes per launch = K + V + Q + O):
//   workgroup = (kv head of one sequence, chunk of kChunk keys), 256 threads;
//   a key row of D values is read by D/8 lanes with one 16-byte load each, so a wave reads
//   64*16 bytes of consecutive rows per load instruction (fully coalesced);
//   every lane issues all of its row loads for the chunk before using any of them;
//   scores use v_dot2_f32_{f16,bf16}: products exact, fp32 sums; the chunk softmax runs in the
//   log2 domain (exp2); P.V accumulates in fp32.
// A second kernel merges the per-chunk (max, sum, unnormalised O) partials of each row.

#include "attn_common.h"
#include "gt_internal.h"

#include <cmath>

namespace {

constexpr int kChunk = 256;  // keys per workgroup = threads per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Pack;
template <>
struct Pack<_Float16> {
    typedef half2_t T2;
    static __device__ inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
    }
    static __device__ inline float lo(uint32_t a) { return (float)__builtin_bit_cast(half2_t, a)[0]; }
    static __device__ inline float hi(uint32_t a) { return (float)__builtin_bit_cast(half2_t, a)[1]; }
};
template <>
struct Pack<__bf16> {
    typedef bf162_t T2;
    static __device__ inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a), __builtin_bit_cast(bf162_t, b), c, false);
    }
    static __device__ inline float lo(uint32_t a) { return __uint_as_float(a << 16); }
    static __device__ inline float hi(uint32_t a) { return __uint_as_float(a & 0xffff0000u); }
};

__device__ inline float wave_max(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ inline float wave_sum(float v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Score of key `key` for query head `h` after scale and mask, in the log2 domain.
__device__ inline float finish_score(const AttnFwdArgs &f, float dot, int64_t b, int64_t h, int64_t key) {
    if (key >= f.S || (f.causal && key > 0)) return -INFINITY;
    float s = dot * (f.scale * kLog2e);
    if (f.mask) {
        const int64_t mi = b * f.m_sb + h * f.m_sh + key * f.m_ss;
        if (f.mask_bool) {
            if (!((const uint8_t *)f.mask)[mi]) return -INFINITY;
        } else {
            s += ((const float *)f.mask)[mi] * kLog2e;
        }
    }
    return s;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
    using P = Pack<T>;
    constexpr int LPR = D / 8;        // lanes per key row
    constexpr int RPW = 64 / LPR;     // rows per wave per load
    constexpr int RPB = 4 * RPW;      // rows per workgroup per load
    constexpr int NR = kChunk / RPB;  // rows per lane
    static_assert(G <= LPR, "one lane per head writes the scores");
    __shared__ float s_p[G][kChunk];
    __shared__ float s_red[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int sub = lane % LPR, rg = w * RPW + lane / LPR;
    const int split = blockIdx.x;
    const int64_t bk = blockIdx.y, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int64_t s0 = (int64_t)split * kChunk;

    // the G query rows of this kv head, 8 values per lane
    uint32_t q2[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const T *qr = (const T *)f.q + b * f.q_sb + (hk * G + h) * f.q_sh + 8 * sub;
        const u32x4 x = *(const u32x4 *)qr;
        q2[h][0] = x[0];
        q2[h][1] = x[1];
        q2[h][2] = x[2];
        q2[h][3] = x[3];
    }

    // K rows of the chunk: all loads first
    const T *kb = (const T *)f.k + b * f.k_sb + hk * f.k_sh + 8 * sub;
    u32x4 kr[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int64_t key = s0 + rg + RPB * i;
        kr[i] = key < f.S ? *(const u32x4 *)(kb + key * f.k_ss) : u32x4{0, 0, 0, 0};
    }
    float sc[NR][G];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) s = P::dot2(kr[i][j], q2[h][j], s);
            sc[i][h] = s;
        }
    }
    // V loads do not depend on the scores: issue them now
    const T *vb = (const T *)f.v + b * f.v_sb + hk * f.v_sh + 8 * sub;
    u32x4 vr[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int64_t key = s0 + rg + RPB * i;
        vr[i] = key < f.S ? *(const u32x4 *)(vb + key * f.v_ss) : u32x4{0, 0, 0, 0};
    }
    // sum the partial dots over the LPR lanes of each row
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 1; m < LPR; m <<= 1) sc[i][h] += __shfl_xor(sc[i][h], m, 64);
    // lane `sub` of a row stores head `sub`
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) v = (sub == h) ? sc[i][h] : v;
        if (sub < G) {
            const int slot = rg + RPB * i;
            s_p[sub][slot] = finish_score(f, v, b, hk * G + sub, s0 + slot);
        }
    }
    __syncthreads();

    // chunk softmax: thread `tid` owns key slot `tid`
    float mx[G], sum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float m = wave_max(s_p[h][tid]);
        if (lane == 0) s_red[w][h] = m;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) mx[h] = fmaxf(fmaxf(s_red[0][h], s_red[1][h]), fmaxf(s_red[2][h], s_red[3][h]));
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float s = s_p[h][tid];
        const float p = (s == -INFINITY) ? 0.0f : exp2f(s - mx[h]);
        s_p[h][tid] = p;
        const float t = wave_sum(p);
        if (lane == 0) s_red[w][h] = t;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) sum[h] = (s_red[0][h] + s_red[1][h]) + (s_red[2][h] + s_red[3][h]);

    // P.V over this lane's rows
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int slot = rg + RPB * i;
        float vf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vf[2 * j] = P::lo(vr[i][j]);
            vf[2 * j + 1] = P::hi(vr[i][j]);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float p = s_p[h][slot];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(p, vf[j], acc[h][j]);
        }
    }
    // rows of a wave -> one partial per wave
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int m = LPR; m < 64; m <<= 1) acc[h][j] += __shfl_xor(acc[h][j], m, 64);
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) s_o[w][h][8 * sub + j] = acc[h][j];
    }
    __syncthreads();
    const int64_t row0 = (b * f.H + hk * G) * a.nsplit + split;  // (b, head hk*G, split)
    for (int e = tid; e < G * D; e += 256) {
        const int h = e / D, d = e % D;
        const float o = (s_o[0][h][d] + s_o[1][h][d]) + (s_o[2][h][d] + s_o[3][h][d]);
        a.part_o[(row0 + (int64_t)h * a.nsplit) * D + d] = o;
    }
    if (tid < G) {
        a.part_ml[(row0 + (int64_t)tid * a.nsplit) * 2 + 0] = mx[tid];
        a.part_ml[(row0 + (int64_t)tid * a.nsplit) * 2 + 1] = sum[tid];
    }
}

template <typename T>
__device__ inline void store_t(void *o, int64_t i, float v);
template <>
__device__ inline void store_t<_Float16>(void *o, int64_t i, float v) {
    ((_Float16 *)o)[i] = (_Float16)v;
}
template <>
__device__ inline void store_t<__bf16>(void *o, int64_t i, float v) {
    ((__bf16 *)o)[i] = (__bf16)v;
}
template <>
__device__ inline void store_t<float>(void *o, int64_t i, float v) {
    ((float *)o)[i] = v;
}

// One wave per (b, h) row: out = sum_i 2^(m_i - M) O_i / sum_i 2^(m_i - M) l_i.
template <typename TO, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + w;
    if (row >= f.B * f.H) return;
    const float *ml = a.part_ml + row * a.nsplit * 2;
    float M = -INFINITY;
    for (int i = lane; i < a.nsplit; i += 64) M = fmaxf(M, ml[2 * i]);
    M = wave_max(M);
    constexpr int NJ = (D + 63) / 64;
    float o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[j] = 0.0f;
    float L = 0.0f;
    for (int i = 0; i < a.nsplit; ++i) {
        const float m = ml[2 * i];
        const float wgt = (m == -INFINITY) ? 0.0f : exp2f(m - M);
        L = fmaf(wgt, ml[2 * i + 1], L);
        const float *po = a.part_o + (row * a.nsplit + i) * D;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int d = lane + 64 * j;
            if (d < D) o[j] = fmaf(wgt, po[d], o[j]);
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        if (d < D) store_t<TO>(f.o, row * D + d, o[j] * inv);
    }
    if (f.lse && lane == 0) ((float *)f.lse)[row] = L > 0.0f ? (M + log2f(L)) * kLn2 : INFINITY;
}

template <typename T, int D, int G>
hipError_t launch_typed(const DecodeArgs &a, hipStream_t s) {
    dim3 grid((unsigned)a.nsplit, (unsigned)(a.f.B * a.f.Hkv));
    hipLaunchKernelGGL((decode_split_kernel<T, D, G>), grid, dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t rows = a.f.B * a.f.H;
    hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_g(const DecodeArgs &a, int G, hipStream_t s) {
    switch (G) {
        case 1: return launch_typed<T, D, 1>(a, s);
        case 2: return launch_typed<T, D, 2>(a, s);
        case 4: return launch_typed<T, D, 4>(a, s);
        case 8: return launch_typed<T, D, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t launch_d(const DecodeArgs &a, int G, hipStream_t s) {
    switch (a.f.D) {
        case 64: return launch_g<T, 64>(a, G, s);
        case 128: return launch_g<T, 128>(a, G, s);
        case 256: return launch_g<T, 256>(a, G, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename TO>
hipError_t launch_merge_t(const DecodeArgs &a, hipStream_t s) {
    const int64_t rows = a.f.B * a.f.H;
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch (a.f.D) {
        case 64: hipLaunchKernelGGL((decode_merge_kernel<TO, 64>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((decode_merge_kernel<TO, 128>), grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL((decode_merge_kernel<TO, 256>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_decode_merge(const DecodeArgs &a, int out_dtype, hipStream_t s) {
    if (out_dtype == GT_F16) return launch_merge_t<_Float16>(a, s);
    if (out_dtype == GT_BF16) return launch_merge_t<__bf16>(a, s);
    if (out_dtype == GT_F32) return launch_merge_t<float>(a, s);
    return hipErrorInvalidValue;
}

int attn_decode_splits(int64_t S) { return (int)((S + kChunk - 1) / kChunk); }

bool attn_decode_supported(const AttnFwdArgs &f, int cd) {
    if (cd != GT_F16 && cd != GT_BF16) return false;
    if (f.L != 1 || f.S <= 0 || f.D != f.Dv) return false;
    if (f.D != 64 && f.D != 128 && f.D != 256) return false;
    const int64_t G = f.H / f.Hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return false;
    if (f.D / 8 < G) return false;
    // 16-byte row loads: every row start must be 16-byte aligned
    const int64_t strides[] = {f.q_sb, f.q_sh, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 8 != 0) return false;
    for (const void *p : {f.q, f.k, f.v}) if ((uintptr_t)p % 16 != 0) return false;
    return true;
}

hipError_t launch_attn_decode(const DecodeArgs &a, int cd, hipStream_t s) {
    const int G = (int)(a.f.H / a.f.Hkv);
    if (cd == GT_F16) return launch_d<_Float16>(a, G, s);
    if (cd == GT_BF16) return launch_d<__bf16>(a, G, s);
    return hipErrorInvalidValue;
}
