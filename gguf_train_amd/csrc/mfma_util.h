// gfx950 MFMA helpers shared by the attention kernels.
//
// v_mfma_f32_32x32x16_{f16,bf16} operand layouts (lane l of a 64-lane wavefront):
//   A (32 x 16, M x K): lane holds A[m = l % 32][k = 8 (l / 32) + 0..7]
//   B (16 x 32, K x N): lane holds B[k = 8 (l / 32) + 0..7][n = l % 32]
//   C (32 x 32):        lane holds C[m = 8 (i / 4) + 4 (l / 32) + i % 4][n = l % 32], i = 0..15
// The k index of one MFMA may be permuted freely as long as A and B use the same permutation;
// the kernels use that to feed an accumulator (16 values of one column n per lane) back as an
// operand without moving data between lanes: k-slot e (0..7) of lane half h, for k-step hs,
// is accumulator row 16 hs + 8 (e / 4) + 4 h + e % 4.
//
// ds_read_b64_tr_b16: 16 lanes each address 8 bytes; lanes 4r .. 4r+3 address 16 consecutive
// 16-bit values of "row" r (r = 0..3); lane i of the group receives value i of rows 0..3.
// With rows = 4 consecutive rows of a row-major tile this reads a column fragment (4 rows of
// one column per lane), which is how a row-major LDS tile becomes a transposed operand.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gtmfma {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
    typedef half8 V8;
    static constexpr bool kSplit = false;  // fp16 keeps 11 bits: one operand where sums run along normalised rows (pack8_hilo elsewhere)
    static __device__ inline f32x16 mma(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
    static __device__ inline uint32_t pack(float x, float y) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h2 v = {(_Float16)x, (_Float16)y};
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ inline float round(float x) { return (float)(_Float16)x; }
};
template <>
struct Mfma<__bf16> {
    typedef bf16x8 V8;
    static constexpr bool kSplit = true;  // bf16 keeps 8 bits: operands built on the fly are split hi + lo
    static __device__ inline f32x16 mma(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
    static __device__ inline uint32_t pack(float x, float y) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        b2 v = {(__bf16)x, (__bf16)y};
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ inline float round(float x) { return (float)(__bf16)x; }
};

// Packs 8 floats as an MFMA operand; `lo` receives the rounding residuals when the type splits.
// bf16: the residual x - hi of each element comes from the packed pair itself with one
// v_dot2_f32_bf16 (hi pair . (-1, 0) + x, or . (0, -1)): the products are exact and x - hi is
// exactly representable, so the result is the exact residual, in one instruction instead of
// widening hi back to float and subtracting.
template <typename T>
__device__ inline void pack8(const float *x, typename Mfma<T>::V8 &hi, typename Mfma<T>::V8 &lo) {
    using M = Mfma<T>;
    u32x4 h = {M::pack(x[0], x[1]), M::pack(x[2], x[3]), M::pack(x[4], x[5]), M::pack(x[6], x[7])};
    hi = __builtin_bit_cast(typename M::V8, h);
    if constexpr (M::kSplit) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        // (-1, 0) and (0, -1), element 0 in the low half, kept opaque: the compiler folds the
        // constant pair (-1, 0) into the inline constant -1.0, whose bits 0xbf800000 are (0, -1)
        uint32_t nf_bits = 0x0000bf80u, ns_bits = 0xbf800000u;
        asm("" : "+v"(nf_bits), "+v"(ns_bits));
        const b2 neg_first = __builtin_bit_cast(b2, nf_bits), neg_second = __builtin_bit_cast(b2, ns_bits);
        float r[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t hj = h[j];  // through a scalar: bit-casting a vector element reads element 0
            const b2 pair = __builtin_bit_cast(b2, hj);
            r[2 * j] = __builtin_amdgcn_fdot2_f32_bf16(pair, neg_first, x[2 * j], false);
            r[2 * j + 1] = __builtin_amdgcn_fdot2_f32_bf16(pair, neg_second, x[2 * j + 1], false);
        }
        u32x4 l = {M::pack(r[0], r[1]), M::pack(r[2], r[3]), M::pack(r[4], r[5]), M::pack(r[6], r[7])};
        lo = __builtin_bit_cast(typename M::V8, l);
    }
}

// pack8 with a residual operand for either type: `lo` = x - hi rounded to T, so that hi + lo
// carries about twice T's significand.  For sums whose terms are not normalised per row (dV =
// P^T.dO and dK = dS^T.Q add a key's contributions over every query row), where a single fp16
// operand's 2^-12 relative rounding accumulates with the column sums of P.  fp16: the residual of
// each element is exact, from the packed pair with one v_dot2_f32_f16 ((hi0, hi1) . (-1, 0) + x0).
template <typename T>
__device__ inline void pack8_hilo(const float *x, typename Mfma<T>::V8 &hi, typename Mfma<T>::V8 &lo) {
    using M = Mfma<T>;
    if constexpr (M::kSplit) {
        pack8<T>(x, hi, lo);
    } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        u32x4 h = {M::pack(x[0], x[1]), M::pack(x[2], x[3]), M::pack(x[4], x[5]), M::pack(x[6], x[7])};
        hi = __builtin_bit_cast(typename M::V8, h);
        // (-1, 0) and (0, -1), element 0 in the low half, kept opaque (see pack8)
        uint32_t nf_bits = 0x0000bc00u, ns_bits = 0xbc000000u;
        asm("" : "+v"(nf_bits), "+v"(ns_bits));
        const h2 neg_first = __builtin_bit_cast(h2, nf_bits), neg_second = __builtin_bit_cast(h2, ns_bits);
        float r[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t hj = h[j];  // through a scalar: bit-casting a vector element reads element 0
            const h2 pair = __builtin_bit_cast(h2, hj);
            r[2 * j] = __builtin_amdgcn_fdot2(pair, neg_first, x[2 * j], false);
            r[2 * j + 1] = __builtin_amdgcn_fdot2(pair, neg_second, x[2 * j + 1], false);
        }
        u32x4 l = {M::pack(r[0], r[1]), M::pack(r[2], r[3]), M::pack(r[4], r[5]), M::pack(r[6], r[7])};
        lo = __builtin_bit_cast(typename M::V8, l);
    }
}

// acc + the sum of 8 probabilities x whose operand form is `hi` (pack8).  fp16: the rounded
// values the MFMA consumes, summed pairwise with v_dot2_f32_f16 (products by 1 are exact, fp32
// accumulation), 4 instructions instead of 8; bf16: the fp32 values.
template <typename T>
__device__ inline float sum8(const float *x, typename Mfma<T>::V8 hi, float acc) {
    if constexpr (Mfma<T>::kSplit) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += x[e];
    } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        const u32x4 u = __builtin_bit_cast(u32x4, hi);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t ue = u[e];  // through a scalar: bit-casting a vector element reads element 0
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ue), one, acc, false);
        }
    }
    return acc;
}

// Column fragment of a row-major LDS tile: rows row0 .. row0+3 and row0+8 .. row0+11 (8 values)
// of one column per lane, as laid out by the caller's addressing (see the header comment).
template <typename T>
__device__ inline typename Mfma<T>::V8 read_tr8(const T *p0, const T *p1) {
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(__attribute__((address_space(3))) char *)p0);
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(__attribute__((address_space(3))) char *)p1);
    const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
    return __builtin_bit_cast(typename Mfma<T>::V8, u32x4{w0[0], w0[1], w1[0], w1[1]});
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of v over lanes l and l ^ 32
__device__ inline float xhalf_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xhalf_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace gtmfma
