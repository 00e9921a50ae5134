// Element conversion / layout copy kernels and the GGUF Q8_0 codec.
//
// Conversion follows the reference's per-element semantics (csrc/gt_internal.h:243-301): a
// value is read as double and written back through float for float16/bfloat16, so a float64
// source is rounded twice (double -> float -> half) exactly as the reference does.
//
// Q8_0 (ggml block_q8_0, 34 bytes: fp16 d, int8 qs[32]) follows ggml's reference quantizer
// (quantize_row_q8_0_ref in ggml-quants.c, reached from ggml_quantize_chunk,
// csrc/gt_core.cpp:819-832) and its to_float (csrc/gt_core.cpp:800-808):
//   amax = max|x|, d = amax/127, id = d ? 1/d : 0, qs = roundf(x*id), d stored as fp16 (RNE);
//   y = (float)qs * (float)d.
// HBM-bound byte work: one wave handles two blocks with one lane per value, so loads and
// stores are coalesced; no LDS is needed.

#include "gt_internal.h"
#include "gt_rope_math.h"

#include <cmath>

namespace {

__device__ inline uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ inline float u2f(uint32_t u) { return __uint_as_float(u); }

// IEEE binary16 <-> binary32, round to nearest even (bit-exact with the host converter).
__device__ inline uint16_t d_f32_to_f16_bits(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

// The same rounding by the hardware (v_cvt_f16_f32 in the default round-to-nearest-even mode,
// half subnormals kept), a few times cheaper than the bit-level routine; a NaN keeps the
// routine's payload rule.  The two agree on every non-NaN input (a GPU test checks every Q8_0
// value q * d: all 2^16 scale bit patterns times all 256 quants).
__device__ inline uint16_t d_f32_to_f16(float f) {
    if (f != f) return d_f32_to_f16_bits(f);
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ inline float d_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            e = 113;
            while (!(m & 0x400u)) {
                m <<= 1;
                --e;
            }
            x = sign | (e << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    return u2f(x);
}

__device__ inline uint16_t d_f32_to_bf16(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ inline double read_elem(const void *p, int dtype, int64_t i) {
    switch (dtype) {
        case GT_F32: return ((const float *)p)[i];
        case GT_F64: return ((const double *)p)[i];
        case GT_F16: return d_f16_to_f32(((const uint16_t *)p)[i]);
        case GT_BF16: return u2f((uint32_t)((const uint16_t *)p)[i] << 16);
        case GT_I8: return ((const int8_t *)p)[i];
        case GT_U8: return ((const uint8_t *)p)[i];
        case GT_I16: return ((const int16_t *)p)[i];
        case GT_I32: return ((const int32_t *)p)[i];
        case GT_I64: return (double)((const int64_t *)p)[i];
        case GT_BOOL: return ((const uint8_t *)p)[i] ? 1.0 : 0.0;
        default: return 0.0;
    }
}

__device__ inline void write_elem(void *p, int dtype, int64_t i, double v) {
    switch (dtype) {
        case GT_F32: ((float *)p)[i] = (float)v; break;
        case GT_F64: ((double *)p)[i] = v; break;
        case GT_F16: ((uint16_t *)p)[i] = d_f32_to_f16((float)v); break;
        case GT_BF16: ((uint16_t *)p)[i] = d_f32_to_bf16((float)v); break;
        case GT_I8: ((int8_t *)p)[i] = (int8_t)v; break;
        case GT_U8: ((uint8_t *)p)[i] = (uint8_t)v; break;
        case GT_I16: ((int16_t *)p)[i] = (int16_t)v; break;
        case GT_I32: ((int32_t *)p)[i] = (int32_t)v; break;
        case GT_I64: ((int64_t *)p)[i] = (int64_t)v; break;
        case GT_BOOL: ((uint8_t *)p)[i] = v != 0.0 ? 1 : 0; break;
        default: break;
    }
}

__device__ inline bool is_int(int dt) {
    return dt == GT_I8 || dt == GT_U8 || dt == GT_I16 || dt == GT_I32 || dt == GT_I64;
}

__device__ inline int64_t read_int(const void *p, int dtype, int64_t i) {
    switch (dtype) {
        case GT_I8: return ((const int8_t *)p)[i];
        case GT_U8: return ((const uint8_t *)p)[i];
        case GT_I16: return ((const int16_t *)p)[i];
        case GT_I32: return ((const int32_t *)p)[i];
        default: return ((const int64_t *)p)[i];
    }
}

__device__ inline void write_int(void *p, int dtype, int64_t i, int64_t v) {
    switch (dtype) {
        case GT_I8: ((int8_t *)p)[i] = (int8_t)v; break;
        case GT_U8: ((uint8_t *)p)[i] = (uint8_t)v; break;
        case GT_I16: ((int16_t *)p)[i] = (int16_t)v; break;
        case GT_I32: ((int32_t *)p)[i] = (int32_t)v; break;
        default: ((int64_t *)p)[i] = v; break;
    }
}

__device__ inline int64_t offset_of(const gt_layout &l, int64_t linear) {
    int64_t off = 0;
    for (int d = l.ndim - 1; d >= 0; --d) {
        const int64_t c = linear % l.shape[d];
        linear /= l.shape[d];
        off += c * l.strides[d];
    }
    return off;
}

__device__ inline void copy_bytes(void *dst, const void *src, int n) {
    switch (n) {
        case 1: *(uint8_t *)dst = *(const uint8_t *)src; break;
        case 2: *(uint16_t *)dst = *(const uint16_t *)src; break;
        case 4: *(uint32_t *)dst = *(const uint32_t *)src; break;
        default: *(uint64_t *)dst = *(const uint64_t *)src; break;
    }
}

__global__ void convert_kernel(const void *__restrict__ src, int sdt, gt_layout sl, void *__restrict__ dst, int ddt,
                               gt_layout dl, int64_t numel, int es) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += stride) {
        const int64_t so = offset_of(sl, i), doff = offset_of(dl, i);
        if (sdt == ddt) {
            copy_bytes((char *)dst + doff * es, (const char *)src + so * es, es);
        } else if (is_int(sdt) && is_int(ddt)) {
            write_int(dst, ddt, doff, read_int(src, sdt, so));  // exact beyond 2^53
        } else {
            write_elem(dst, ddt, doff, read_elem(src, sdt, so));
        }
    }
}

// One Q8_0 block, one lane per value: value j (= lane % 32) of the block at `b`, quantized
// with the other 31 lanes of its wave half.  Every lane of the wave calls it (the max is a
// cross-lane exchange); `live` lanes write.
__device__ inline void q8_0_quantize_lane(float v, bool live, uint8_t *b, int j) {
    float amax = fabsf(v);
    // max over the 32 lanes of this half (xor offsets < 32 stay inside the half)
    for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    if (!live) return;
    const float x0 = v * id;
    b[2 + j] = (uint8_t)(int8_t)roundf(x0);
    if (j == 0) {
        const uint16_t h = d_f32_to_f16(d);
        b[0] = (uint8_t)(h & 0xff);
        b[1] = (uint8_t)(h >> 8);
    }
}

// 64 blocks per workgroup of 256 threads, four threads per block: thread t quantizes values
// 8 (t % 4) .. +7 of block t / 4 (two 16-byte loads; the block's |x| max over its four threads
// by two lane exchanges), with the same operations as q8_0_quantize_lane.  A full tile whose
// output starts 16-byte aligned (34 * 64 = 2176 bytes) is assembled in LDS and written with
// 16-byte stores; otherwise every thread stores its bytes directly.
__global__ __launch_bounds__(256) void q8_0_quantize_kernel(const float *__restrict__ x, uint8_t *__restrict__ out,
                                                            int64_t nblocks) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[64 * 34];
    const int tid = threadIdx.x, part = tid & 3;
    const int64_t blk0 = (int64_t)blockIdx.x * 64, blk = blk0 + (tid >> 2);
    const bool live = blk < nblocks;
    float v[8];
    const float *src = x + (live ? blk : 0) * 32 + 8 * part;
    if ((uintptr_t)x % 16 == 0) {
        const float4 a = ((const float4 *)src)[0], b = ((const float4 *)src)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = src[e];
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    // the four threads of a block are lanes 4k .. 4k+3 of one wavefront
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e >> 2] |= (uint32_t)(uint8_t)(int8_t)roundf(v[e] * id) << (8 * (e & 3));
    const uint16_t h = d_f32_to_f16(d);
    // uniform over the workgroup: every thread takes the same branch (the barrier is inside one)
    if (blk0 + 64 <= nblocks && (uintptr_t)out % 16 == 0) {
        uint16_t *tb = (uint16_t *)&tile[34 * (tid >> 2)];  // 2-byte aligned: 34 is even
        if (part == 0) tb[0] = h;
#pragma unroll
        for (int i = 0; i < 4; ++i) tb[1 + 4 * part + i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
        __syncthreads();
        if (tid < 136) *(uint4 *)(out + blk0 * 34 + 16 * tid) = *(const uint4 *)&tile[16 * tid];
    } else if (live) {
        uint8_t *b = out + blk * 34;
        if (part == 0) {
            b[0] = (uint8_t)(h & 0xff);
            b[1] = (uint8_t)(h >> 8);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) b[2 + 8 * part + e] = (uint8_t)(w[e >> 2] >> (8 * (e & 3)));
    }
}

// KV-cache append: row (b, h, t) of src (B, Hkv, T, D), any strides, goes to row pos[b] + t of
// the cache (B, Hkv, cap, D).  A float cache receives converted elements (one thread each); a
// Q8_0 cache receives the row quantized block by block (two blocks per wave, as above).
// With a RoPE table (gt_rope_apply), element d < n_dims is first rotated with its partner (d ^ 1,
// or d -/+ n_dims/2 for NeoX) read from the same source row, in float32 as gt_rope does, and
// rounded to the source dtype, so the cache holds what gt_rope followed by the append stores.
__global__ void kv_append_kernel(const void *__restrict__ src, int sdt, int64_t s_sb, int64_t s_sh, int64_t s_st,
                                 int64_t s_sd, void *__restrict__ dst, int ddt, const int32_t *__restrict__ pos,
                                 int64_t Hkv, int64_t T, int64_t D, int64_t cap, int64_t n,
                                 const float2 *__restrict__ rope_table, int n_dims, int neox) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // value index (b, h, t, d)
    const bool live = i < n;
    const int64_t ic = live ? i : 0;
    const int64_t d = ic % D, t = (ic / D) % T, h = (ic / (D * T)) % Hkv, b = ic / (D * T * Hkv);
    const int64_t src_row = b * s_sb + h * s_sh + t * s_st;
    double x = read_elem(src, sdt, src_row + d * s_sd);
    if (rope_table && d < n_dims) {
        const int half = n_dims / 2;
        const bool lo = neox ? d < half : (d & 1) == 0;
        const int64_t pd = neox ? (lo ? d + half : d - half) : (d ^ 1);
        const int pair = neox ? (int)(lo ? d : pd) : (int)(d >> 1);
        const float v = (float)x, w = (float)read_elem(src, sdt, src_row + pd * s_sd);
        const float2 cs = rope_table[(b * T + t) * half + pair];
        float r = lo ? rope_rot_lo(v, w, cs) : rope_rot_hi(w, v, cs);
        if (sdt == GT_F16) r = d_f16_to_f32(d_f32_to_f16(r));
        else if (sdt == GT_BF16) r = u2f((uint32_t)d_f32_to_bf16(r) << 16);
        x = r;
    }
    const int64_t row = (b * Hkv + h) * cap + pos[b] + t;
    if (ddt == GT_Q8_0) {
        // D % 32 == 0 and n % 32 == 0, so a wave half is one whole block of one row
        q8_0_quantize_lane((float)x, live, (uint8_t *)dst + (row * (D / 32) + d / 32) * 34, (int)(d % 32));
    } else if (live) {
        write_elem(dst, ddt, row * D + d, x);
    }
}

// float16 bits -> float32: the hardware conversion (exact) except for NaNs, which keep
// d_f16_to_f32's payload rule
__device__ inline float d_f16_to_f32_fast(uint16_t h) {
    if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)) return d_f16_to_f32(h);
    return (float)__builtin_bit_cast(_Float16, h);
}

// 8 consecutive elements of a float32 / float16 / bfloat16 source as float32 (exact), from a
// 16-byte aligned address.
template <int SDT>
__device__ inline void load8(const void *base, int64_t e0, float *v) {
    if constexpr (SDT == GT_F32) {
        const float4 a = ((const float4 *)((const float *)base + e0))[0];
        const float4 c = ((const float4 *)((const float *)base + e0))[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
        const uint4 q = *(const uint4 *)((const uint16_t *)base + e0);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (SDT == GT_F16) {
                v[2 * i] = d_f16_to_f32_fast((uint16_t)(w[i] & 0xffffu));
                v[2 * i + 1] = d_f16_to_f32_fast((uint16_t)(w[i] >> 16));
            } else {
                v[2 * i] = u2f(w[i] << 16);
                v[2 * i + 1] = u2f(w[i] & 0xffff0000u);
            }
        }
    }
}

// KV-cache append, fast path: source rows of D contiguous float32 / float16 / bfloat16 elements
// starting 16-byte aligned (and, with RoPE, n_dims a multiple of 16, so that no 8-element chunk
// straddles n_dims or a NeoX half).  One thread per 8 consecutive elements of a row: 16- or
// 32-byte loads and stores, 32-bit index arithmetic below the row.  Same values and bytes as
// kv_append_kernel: the rotation in float32 rounded to the source dtype, then the cache dtype;
// a Q8_0 cache quantizes with four threads per block (the block's |x| max by two lane
// exchanges) and the operations of q8_0_quantize_lane.
template <int SDT, int DDT>
__global__ __launch_bounds__(256) void kv_append_vec_kernel(const void *__restrict__ src, int64_t s_sb, int64_t s_sh,
                                                            int64_t s_st, void *__restrict__ dst,
                                                            const int32_t *__restrict__ pos, int Hkv, int T, int D,
                                                            int64_t cap, int64_t n8, const float2 *__restrict__ rope_table,
                                                            int n_dims, int neox) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < n8;
    const int64_t ic = live ? i : 0;
    const int per = D / 8;
    const int j = (int)(ic % per);
    const int64_t r = ic / per;  // source row (b, h, t)
    const int t = (int)(r % T);
    const int64_t bh = r / T;
    const int h = (int)(bh % Hkv);
    const int64_t b = bh / Hkv;
    const int d0 = 8 * j;
    const int64_t srow = b * s_sb + h * s_sh + (int64_t)t * s_st;
    float v[8];
    load8<SDT>(src, srow + d0, v);
    if (rope_table && d0 < n_dims) {
        const int half = n_dims / 2;
        const bool lo_chunk = d0 < half;  // NeoX: the whole chunk is on one side of half
        float w[8];
        if (neox) load8<SDT>(src, srow + (lo_chunk ? d0 + half : d0 - half), w);
        float rr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = d0 + e;
            const bool lo = neox ? lo_chunk : (e & 1) == 0;
            const float other = neox ? w[e] : v[e ^ 1];
            const int pair = neox ? (lo ? d : d - half) : (d >> 1);
            const float2 cs = rope_table[((int64_t)b * T + t) * half + pair];
            float x = lo ? rope_rot_lo(v[e], other, cs) : rope_rot_hi(other, v[e], cs);
            if constexpr (SDT == GT_F16) x = d_f16_to_f32(d_f32_to_f16(x));
            else if constexpr (SDT == GT_BF16) x = u2f((uint32_t)d_f32_to_bf16(x) << 16);
            rr[e] = x;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = rr[e];
    }
    const int64_t row = ((int64_t)b * Hkv + h) * cap + pos[b] + t;
    if constexpr (DDT == GT_Q8_0) {
        // the four threads of a block are lanes 4k .. 4k+3 (D / 8 is a multiple of 4), all live or
        // none (n8 is too)
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        if (!live) return;
        uint16_t *blk = (uint16_t *)((uint8_t *)dst + (row * (D / 32) + d0 / 32) * 34);  // 34 is even
        const int part = j & 3;
        if (part == 0) blk[0] = d_f32_to_f16(d);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t q0 = (uint8_t)(int8_t)roundf(v[e] * id), q1 = (uint8_t)(int8_t)roundf(v[e + 1] * id);
            blk[1 + 4 * part + e / 2] = (uint16_t)(q0 | (q1 << 8));
        }
    } else {
        if (!live) return;
        const int64_t o = row * D + d0;
        if constexpr (DDT == GT_F32) {
            ((float4 *)((float *)dst + o))[0] = make_float4(v[0], v[1], v[2], v[3]);
            ((float4 *)((float *)dst + o))[1] = make_float4(v[4], v[5], v[6], v[7]);
        } else {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t a = DDT == GT_F16 ? d_f32_to_f16(v[2 * k]) : d_f32_to_bf16(v[2 * k]);
                const uint32_t c = DDT == GT_F16 ? d_f32_to_f16(v[2 * k + 1]) : d_f32_to_bf16(v[2 * k + 1]);
                w[k] = a | (c << 16);
            }
            *(uint4 *)((uint16_t *)dst + o) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

// KV-cache append of rows that are already Q8_0: row (b, h, t) of the dense Q8_0 src
// (B, Hkv, T, D) is copied, block bytes unchanged, to row pos[b] + t of the Q8_0 cache.  A row is
// D / 32 blocks of 34 bytes; one thread moves one 16-bit half-word of it.
__global__ void kv_append_blocks_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst,
                                        const int32_t *__restrict__ pos, int64_t Hkv, int64_t T, int64_t hpr,
                                        int64_t cap, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / hpr, j = i % hpr;  // source row (b, h, t) and half-word in it
    const int64_t t = r % T, bh = r / T, b = bh / Hkv;
    dst[(bh * cap + pos[b] + t) * hpr + j] = src[i];
}

// Block blk of the output reads source block blk, or, with group_blocks > 0, the blocks of each
// group of group_blocks consecutive output blocks read from a source group src_group_blocks
// blocks long (the first rows of every (sequence, kv head) of a KV cache).
__global__ void q8_0_dequantize_kernel(const uint8_t *__restrict__ in, void *__restrict__ out, int dst_dtype,
                                       int64_t nblocks, int64_t group_blocks, int64_t src_group_blocks) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t blk = wave * 2 + (lane >> 5);
    const int j = lane & 31;
    if (blk >= nblocks) return;
    const int64_t sblk = group_blocks > 0 ? blk / group_blocks * src_group_blocks + blk % group_blocks : blk;
    const uint8_t *b = in + sblk * 34;
    const float d = d_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    const float y = (float)(int8_t)b[2 + j] * d;
    const int64_t i = blk * 32 + j;
    switch (dst_dtype) {
        case GT_F32: ((float *)out)[i] = y; break;
        case GT_F64: ((double *)out)[i] = (double)y; break;
        case GT_F16: ((uint16_t *)out)[i] = d_f32_to_f16(y); break;
        case GT_BF16: ((uint16_t *)out)[i] = d_f32_to_bf16(y); break;
        default: write_elem(out, dst_dtype, i, (double)y); break;
    }
}

// The same for float32 / float16 / bfloat16 outputs: thread t dequantizes values 8 (t % 4) .. +7
// of block t / 4 (the scale and four 16-bit quant loads: a block starts at an even byte) and
// writes them with 16-byte stores.  Same values as q8_0_dequantize_kernel.
template <int DT>
__global__ void q8_0_dequantize_vec_kernel(const uint8_t *__restrict__ in, void *__restrict__ out, int64_t nblocks,
                                           int64_t group_blocks, int64_t src_group_blocks) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = t >> 2;
    const int part = (int)(t & 3);
    if (blk >= nblocks) return;
    const int64_t sblk = group_blocks > 0 ? blk / group_blocks * src_group_blocks + blk % group_blocks : blk;
    const uint16_t *b = (const uint16_t *)(in + sblk * 34);
    const float d = d_f16_to_f32(b[0]);
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t two = b[1 + 4 * part + i];
        y[2 * i] = (float)(int8_t)(two & 0xffu) * d;
        y[2 * i + 1] = (float)(int8_t)(two >> 8) * d;
    }
    const int64_t i0 = blk * 32 + 8 * part;
    if constexpr (DT == GT_F32) {
        float4 *o = (float4 *)((float *)out + i0);
        o[0] = make_float4(y[0], y[1], y[2], y[3]);
        o[1] = make_float4(y[4], y[5], y[6], y[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = DT == GT_F16 ? d_f32_to_f16(y[2 * i]) : d_f32_to_bf16(y[2 * i]);
            const uint32_t hi = DT == GT_F16 ? d_f32_to_f16(y[2 * i + 1]) : d_f32_to_bf16(y[2 * i + 1]);
            w[i] = lo | (hi << 16);
        }
        *(uint4 *)((uint16_t *)out + i0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Bool mask bytes -> additive float mask: 0 (attend) or -inf (blocked).
__global__ void bool_to_bias_kernel(const uint8_t *__restrict__ src, float *__restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[i] ? 0.0f : -INFINITY;
}

// Zero fill of `bytes` bytes at p, as a kernel so that a stream under graph capture records a
// kernel node, not a memset node: 16-byte stores over the first n16 chunks, byte stores for the
// remaining bytes (all of them when p is not 16-byte aligned: n16 = 0).
__global__ void fill_zero_kernel(uint8_t *__restrict__ p, int64_t n16, int64_t bytes) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n = n16 + (bytes - 16 * n16);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        if (i < n16) *(uint4 *)(p + 16 * i) = make_uint4(0u, 0u, 0u, 0u);
        else p[16 * n16 + (i - n16)] = 0;
    }
}

// Rows of a 4-D tensor (rows (b, h, l) at b*sb + h*sh + l*sl, D contiguous elements of ES bytes)
// into a dense (B*H*L, Dp) buffer, dims D .. Dp-1 set to zero; or back (unpad: the first D of
// every Dp).  One thread per destination element.
template <typename E>
__global__ void pad_rows_kernel(const E *__restrict__ src, int64_t sb, int64_t sh, int64_t sl, int64_t H, int64_t L,
                                int64_t D, E *__restrict__ dst, int64_t Dp, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / Dp, d = i % Dp;
        const int64_t l = r % L, bh = r / L, h = bh % H, b = bh / H;
        dst[i] = d < D ? src[b * sb + h * sh + l * sl + d] : E(0);
    }
}
template <typename E>
__global__ void unpad_rows_kernel(const E *__restrict__ src, int64_t Dp, E *__restrict__ dst, int64_t D, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[(i / D) * Dp + i % D];
}

// The same two copies with 8 elements of ES bytes (16 or 32 bytes) per thread, for D % 8 == 0
// and 16-byte aligned rows: a destination chunk of pad_rows is all source or all zero, and
// every chunk starts at a 16-byte boundary on both sides.
template <int ES>
__global__ void pad_rows_vec_kernel(const uint8_t *__restrict__ src, int64_t sb, int64_t sh, int64_t sl, int64_t H,
                                    int64_t L, int D, uint8_t *__restrict__ dst, int Dp, int64_t n8) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int per = Dp / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const int64_t r = i / per;
        const int d0 = 8 * (int)(i - r * per);
        const int64_t l = r % L, bh = r / L, h = bh % H, b = bh / H;
        uint4 x[ES / 2];
#pragma unroll
        for (int k = 0; k < ES / 2; ++k) x[k] = make_uint4(0u, 0u, 0u, 0u);
        if (d0 < D) {
            const uint4 *sp = (const uint4 *)(src + (b * sb + h * sh + l * sl + d0) * ES);
#pragma unroll
            for (int k = 0; k < ES / 2; ++k) x[k] = sp[k];
        }
        uint4 *dp = (uint4 *)(dst + i * 8 * ES);
#pragma unroll
        for (int k = 0; k < ES / 2; ++k) dp[k] = x[k];
    }
}
template <int ES>
__global__ void unpad_rows_vec_kernel(const uint8_t *__restrict__ src, int Dp, uint8_t *__restrict__ dst, int D,
                                      int64_t n8) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int per = D / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const int64_t r = i / per;
        const int d0 = 8 * (int)(i - r * per);
        const uint4 *sp = (const uint4 *)(src + (r * Dp + d0) * ES);
        uint4 *dp = (uint4 *)(dst + i * 8 * ES);
#pragma unroll
        for (int k = 0; k < ES / 2; ++k) dp[k] = sp[k];
    }
}

inline unsigned grid_for(int64_t n, int block) {
    const int64_t g = (n + block - 1) / block;
    return (unsigned)(g < 65536 * 16 ? (g > 0 ? g : 1) : 65536 * 16);
}

}  // namespace

hipError_t gt_launch_convert(const void *src, int src_dtype, const gt_layout &src_layout, void *dst, int dst_dtype,
                             const gt_layout &dst_layout, int64_t numel, hipStream_t stream) {
    if (numel <= 0) return hipSuccess;
    const int es = (int)gt_elem_bytes(src_dtype);
    hipLaunchKernelGGL(convert_kernel, dim3(grid_for(numel, 256)), dim3(256), 0, stream, src, src_dtype, src_layout, dst,
                       dst_dtype, dst_layout, numel, es);
    return hipGetLastError();
}

hipError_t gt_launch_q8_0_quantize(const float *src, void *dst, int64_t nblocks, hipStream_t stream) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t wgs = (nblocks + 63) / 64;
    if (wgs > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(q8_0_quantize_kernel, dim3((unsigned)wgs), dim3(256), 0, stream, src, (uint8_t *)dst, nblocks);
    return hipGetLastError();
}

hipError_t gt_launch_q8_0_dequantize(const void *src, void *dst, int dst_dtype, int64_t nblocks, hipStream_t stream) {
    return gt_launch_q8_0_dequantize_rows(src, dst, dst_dtype, nblocks, 0, 0, stream);
}

hipError_t gt_launch_q8_0_dequantize_rows(const void *src, void *dst, int dst_dtype, int64_t nblocks,
                                          int64_t group_blocks, int64_t src_group_blocks, hipStream_t stream) {
    if (nblocks <= 0) return hipSuccess;
    if (dst_dtype == GT_F32 || dst_dtype == GT_F16 || dst_dtype == GT_BF16) {
        // four threads per block, eight values each, one or two 16-byte stores
        const int64_t wgs = (nblocks * 4 + 255) / 256;
        if (wgs > 0x7fffffffLL) return hipErrorInvalidConfiguration;
        if (dst_dtype == GT_F32)
            hipLaunchKernelGGL(q8_0_dequantize_vec_kernel<GT_F32>, dim3((unsigned)wgs), dim3(256), 0, stream,
                               (const uint8_t *)src, dst, nblocks, group_blocks, src_group_blocks);
        else if (dst_dtype == GT_F16)
            hipLaunchKernelGGL(q8_0_dequantize_vec_kernel<GT_F16>, dim3((unsigned)wgs), dim3(256), 0, stream,
                               (const uint8_t *)src, dst, nblocks, group_blocks, src_group_blocks);
        else
            hipLaunchKernelGGL(q8_0_dequantize_vec_kernel<GT_BF16>, dim3((unsigned)wgs), dim3(256), 0, stream,
                               (const uint8_t *)src, dst, nblocks, group_blocks, src_group_blocks);
        return hipGetLastError();
    }
    const int64_t waves = (nblocks + 1) / 2;
    if ((waves + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(q8_0_dequantize_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream,
                       (const uint8_t *)src, dst, dst_dtype, nblocks, group_blocks, src_group_blocks);
    return hipGetLastError();
}

hipError_t gt_launch_bool_to_bias(const void *src, float *dst, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(bool_to_bias_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, (const uint8_t *)src, dst, n);
    return hipGetLastError();
}

hipError_t gt_launch_fill_zero(void *p, int64_t bytes, hipStream_t stream) {
    if (bytes <= 0) return hipSuccess;
    const int64_t n16 = (uintptr_t)p % 16 == 0 ? bytes / 16 : 0;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n16 + (bytes - 16 * n16), 256)), dim3(256), 0, stream,
                       (uint8_t *)p, n16, bytes);
    return hipGetLastError();
}

template <int SDT>
hipError_t launch_kv_append_vec(const void *src, const int64_t *st, void *dst, int ddt, const int32_t *pos, int64_t Hkv,
                                int64_t T, int64_t D, int64_t cap, int64_t n8, const gt_rope_apply *rope,
                                hipStream_t stream) {
    const dim3 grid((unsigned)((n8 + 255) / 256));
    const float2 *tab = rope ? (const float2 *)rope->table : nullptr;
    const int nd = rope ? rope->n_dims : 0, nx = rope ? rope->neox : 0;
#define GT_KV_APPEND_VEC(DDT)                                                                                          \
    hipLaunchKernelGGL((kv_append_vec_kernel<SDT, DDT>), grid, dim3(256), 0, stream, src, st[0], st[1], st[2], dst, pos, \
                       (int)Hkv, (int)T, (int)D, cap, n8, tab, nd, nx)
    if (ddt == GT_F32) GT_KV_APPEND_VEC(GT_F32);
    else if (ddt == GT_F16) GT_KV_APPEND_VEC(GT_F16);
    else if (ddt == GT_BF16) GT_KV_APPEND_VEC(GT_BF16);
    else GT_KV_APPEND_VEC(GT_Q8_0);
#undef GT_KV_APPEND_VEC
    return hipGetLastError();
}

hipError_t gt_launch_kv_append(const void *src, int src_dtype, const int64_t *src_strides, void *dst, int dst_dtype,
                               const int32_t *pos, int64_t B, int64_t Hkv, int64_t T, int64_t D, int64_t cap,
                               const gt_rope_apply *rope, hipStream_t stream) {
    const int64_t n = B * Hkv * T * D;
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    if (rope && (rope->n_dims < 2 || rope->n_dims % 2 != 0 || rope->n_dims > D)) return hipErrorInvalidValue;
    // fast path: contiguous rows of a float32 / float16 / bfloat16 source starting 16-byte aligned
    const int es = src_dtype == GT_F32 ? 4 : 2;
    const bool vec_src = src_dtype == GT_F32 || src_dtype == GT_F16 || src_dtype == GT_BF16;
    const bool vec_dst = dst_dtype == GT_F32 || dst_dtype == GT_F16 || dst_dtype == GT_BF16 || dst_dtype == GT_Q8_0;
    if (vec_src && vec_dst && src_strides[3] == 1 && D % 8 == 0 && (uintptr_t)src % 16 == 0 &&
        (src_strides[0] * es) % 16 == 0 && (src_strides[1] * es) % 16 == 0 && (src_strides[2] * es) % 16 == 0 &&
        (uintptr_t)dst % 16 == 0 && (!rope || rope->n_dims % 16 == 0) && T < (1LL << 31) && D < (1LL << 31) &&
        Hkv < (1LL << 31) && (dst_dtype != GT_Q8_0 || D % 32 == 0)) {
        const int64_t n8 = n / 8;
        if ((n8 + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidConfiguration;
        if (src_dtype == GT_F32) return launch_kv_append_vec<GT_F32>(src, src_strides, dst, dst_dtype, pos, Hkv, T, D, cap, n8, rope, stream);
        if (src_dtype == GT_F16) return launch_kv_append_vec<GT_F16>(src, src_strides, dst, dst_dtype, pos, Hkv, T, D, cap, n8, rope, stream);
        return launch_kv_append_vec<GT_BF16>(src, src_strides, dst, dst_dtype, pos, Hkv, T, D, cap, n8, rope, stream);
    }
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, src, src_dtype, src_strides[0],
                       src_strides[1], src_strides[2], src_strides[3], dst, dst_dtype, pos, Hkv, T, D, cap, n,
                       rope ? (const float2 *)rope->table : nullptr, rope ? rope->n_dims : 0, rope ? rope->neox : 0);
    return hipGetLastError();
}

hipError_t gt_launch_kv_append_blocks(const void *src, void *dst, const int32_t *pos, int64_t B, int64_t Hkv,
                                      int64_t T, int64_t D, int64_t cap, hipStream_t stream) {
    const int64_t hpr = D / 32 * 17;  // half-words per row
    const int64_t n = B * Hkv * T * hpr;
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    if (D % 32 != 0 || blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(kv_append_blocks_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint16_t *)src,
                       (uint16_t *)dst, pos, Hkv, T, hpr, cap, n);
    return hipGetLastError();
}

hipError_t gt_launch_pad_rows(const void *src, int elem_bytes, const int64_t *strides, int64_t B, int64_t H, int64_t L,
                              int64_t D, void *dst, int64_t Dp, hipStream_t stream) {
    const int64_t n = B * H * L * Dp;
    if (n <= 0) return hipSuccess;
    const bool vec = (elem_bytes == 2 || elem_bytes == 4) && D % 8 == 0 && Dp % 8 == 0 && (uintptr_t)src % 16 == 0 &&
                     (uintptr_t)dst % 16 == 0 && (strides[0] * elem_bytes) % 16 == 0 &&
                     (strides[1] * elem_bytes) % 16 == 0 && (strides[2] * elem_bytes) % 16 == 0 && Dp < (1LL << 30);
    if (vec) {
        if (elem_bytes == 2)
            hipLaunchKernelGGL(pad_rows_vec_kernel<2>, dim3(grid_for(n / 8, 256)), dim3(256), 0, stream,
                               (const uint8_t *)src, strides[0], strides[1], strides[2], H, L, (int)D, (uint8_t *)dst,
                               (int)Dp, n / 8);
        else
            hipLaunchKernelGGL(pad_rows_vec_kernel<4>, dim3(grid_for(n / 8, 256)), dim3(256), 0, stream,
                               (const uint8_t *)src, strides[0], strides[1], strides[2], H, L, (int)D, (uint8_t *)dst,
                               (int)Dp, n / 8);
        return hipGetLastError();
    }
    if (elem_bytes == 2)
        hipLaunchKernelGGL(pad_rows_kernel<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0, stream, (const uint16_t *)src,
                           strides[0], strides[1], strides[2], H, L, D, (uint16_t *)dst, Dp, n);
    else if (elem_bytes == 4)
        hipLaunchKernelGGL(pad_rows_kernel<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0, stream, (const uint32_t *)src,
                           strides[0], strides[1], strides[2], H, L, D, (uint32_t *)dst, Dp, n);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t gt_launch_unpad_rows(const void *src, int elem_bytes, int64_t rows, int64_t Dp, void *dst, int64_t D,
                                hipStream_t stream) {
    const int64_t n = rows * D;
    if (n <= 0) return hipSuccess;
    if ((elem_bytes == 2 || elem_bytes == 4) && D % 8 == 0 && Dp % 8 == 0 && (uintptr_t)src % 16 == 0 &&
        (uintptr_t)dst % 16 == 0 && Dp < (1LL << 30)) {
        if (elem_bytes == 2)
            hipLaunchKernelGGL(unpad_rows_vec_kernel<2>, dim3(grid_for(n / 8, 256)), dim3(256), 0, stream,
                               (const uint8_t *)src, (int)Dp, (uint8_t *)dst, (int)D, n / 8);
        else
            hipLaunchKernelGGL(unpad_rows_vec_kernel<4>, dim3(grid_for(n / 8, 256)), dim3(256), 0, stream,
                               (const uint8_t *)src, (int)Dp, (uint8_t *)dst, (int)D, n / 8);
        return hipGetLastError();
    }
    if (elem_bytes == 2)
        hipLaunchKernelGGL(unpad_rows_kernel<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0, stream,
                           (const uint16_t *)src, Dp, (uint16_t *)dst, D, n);
    else if (elem_bytes == 4)
        hipLaunchKernelGGL(unpad_rows_kernel<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0, stream,
                           (const uint32_t *)src, Dp, (uint32_t *)dst, D, n);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}
