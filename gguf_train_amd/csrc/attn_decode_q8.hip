// Single-query (decode) attention over a GGUF Q8_0 K/V cache, fp16 query.
//
// The reference reads a Q8_0 tensor only after gt_dequantize (ggml to_float,
// csrc/gt_core.cpp:800-808: y = qs * d); passed straight to gt_flash_attention it would read
// zeros (csrc/gt_internal.h:243-259).  This kernel computes attention over exactly the
// dequantized values without materialising them: HBM traffic is the 34-byte blocks
// (1.0625 bytes per value), read once per kv head.
//
// Same split-K decomposition as the fp16 decode kernel (workgroup = kv head x chunk of 256
// keys, all query heads of the GQA group together, a merge kernel combines the chunks).
// The chunk's raw block bytes are staged in LDS with coalesced 8-byte loads.
//
// Exact int8 -> fp16 conversion without a convert per value: for u = qs ^ 0x80 (= qs + 128),
// the fp16 bit pattern 0x6400 | u is exactly 1024 + u = qs + 1152.  One v_perm_b32 places two
// bytes under a 0x00 high byte, one logic op sets the 0x64 exponent (and flips the sign bit),
// and v_dot2_f32_f16 multiplies two such values by two fp16 operands with exact products:
//   sum_i q_i * qs_i            = dot2-sum(q, qs + 1152) - 1152 * sum_i q_i
//   sum_k p'_k * qs_k (p' = p*d) = dot2-sum(p', qs + 1152) - 1152 * sum_k p'_k
// where the second uses the fp16-rounded p' on both sides, so the offset cancels exactly.

#include "attn_common.h"
#include "gt_internal.h"

#include <cmath>

namespace {

constexpr int kChunk = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMagic = 1152.0f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}
__device__ inline float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }

// Two int8 values -> packed fp16 (qs + 1152): bytes (lo, hi) selected by `sel` from {x1:x0}
// into the low bytes of each half, then 0x64 exponent and sign flip.
__device__ inline uint32_t magic2(uint32_t x1, uint32_t x0, uint32_t sel) {
    return __builtin_amdgcn_perm(x1, x0, sel) ^ 0x64806480u;
}
// selectors: bytes (b0,b1) and (b2,b3) of x0 into the two halves (0x0c = zero byte)
constexpr uint32_t kSelLo = 0x0c010c00u;
constexpr uint32_t kSelHi = 0x0c030c02u;

__device__ inline float wave_max(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ inline float wave_sum(float v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

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

// The 32 quantized values of block j of key `key` in the staged chunk, as 8 dwords, and its
// scale.  Rows are RB = NB*34 bytes; block j starts at byte 34j of its row: 4-byte aligned
// (then d sits in the first half word) when j is even, 2 mod 4 when j is odd.
template <int NB>
__device__ inline float read_block(const uint8_t *s_kv, int key, int j, uint32_t qs[8]) {
    constexpr int RB = NB * 34;
    const int off = key * RB + 34 * j;
    const uint32_t *p = (const uint32_t *)(s_kv + (off & ~3));
    if ((off & 3) == 0) {
        uint32_t w[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) w[i] = p[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) qs[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        return h2f(w[0] & 0xffffu);
    }
    const uint32_t w0 = p[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) qs[i] = p[i + 1];
    return h2f(w0 >> 16);
}

template <int D, int G>
__global__ __launch_bounds__(256) void decode_q8_split_kernel(DecodeArgs a) {
    constexpr int NB = D / 32;            // blocks per row
    constexpr int RB = NB * 34;           // bytes per row
    constexpr int BYTES = kChunk * RB;    // bytes per chunk
    constexpr int UNITS = BYTES / 8;      // 8-byte units per chunk (RB is a multiple of 4; 256 rows)
    constexpr int NLD = (UNITS + 255) / 256;  // staging loads per thread
    constexpr int KG = 256 / NB;          // key groups of the score phase
    constexpr int NOCT = D / 8;           // 8-value slices of a row (value phase)
    constexpr int VKG = 256 / NOCT;       // key groups of the value phase
    constexpr int VKEYS = kChunk / VKG;   // keys per thread in the value phase (even)
    __shared__ __attribute__((aligned(16))) uint8_t s_kv[BYTES];
    __shared__ float s_p[G][kChunk];
    __shared__ __attribute__((aligned(16))) _Float16 s_pq[G][NB][kChunk];  // fp16(p * d)
    __shared__ float s_pqsum[G][NB];
    __shared__ float s_red[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x;
    const int64_t bk = blockIdx.y, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int64_t s0 = (int64_t)split * kChunk;
    const int64_t valid = (f.S - s0) < kChunk ? (f.S - s0) : kChunk;  // keys of this chunk < S
    const int64_t vbytes = valid * RB;

    // ---- stage the K chunk (coalesced 8-byte loads; bytes past S are zero) ----
    const uint8_t *kchunk = (const uint8_t *)f.k + (bk * f.S + s0) * RB;
    const uint8_t *vchunk = (const uint8_t *)f.v + (bk * f.S + s0) * RB;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int u = tid + 256 * i, o = 8 * u;
        if (u < UNITS) *(u32x2 *)(s_kv + o) = o < vbytes ? *(const u32x2 *)(kchunk + o) : u32x2{0, 0};
    }
    if (tid < G * NB) (&s_pqsum[0][0])[tid] = 0.0f;

    // ---- this thread's query values: block j of every head (fp16 pairs) and their sums ----
    const int j = tid % NB, kg = tid / NB;
    uint32_t q2[G][16];
    float qsum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const _Float16 *qr = (const _Float16 *)f.q + b * f.q_sb + (hk * G + h) * f.q_sh + 32 * j;
        float sacc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 x = *(const u32x4 *)(qr + 8 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // through a scalar: bit-casting a vector element directly reads element 0
                const uint32_t xe = x[e];
                q2[h][4 * i + e] = xe;
                const half2_t hv = __builtin_bit_cast(half2_t, xe);
                sacc += (float)hv[0] + (float)hv[1];
            }
        }
        qsum[h] = sacc;
    }
    // V chunk loads go out now and land while the scores are computed
    u32x2 vreg[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int o = 8 * (tid + 256 * i);
        vreg[i] = o < vbytes ? *(const u32x2 *)(vchunk + o) : u32x2{0, 0};  // o < vbytes implies u < UNITS
    }
    __syncthreads();

    // ---- scores: thread (kg, j) takes block j of keys kg + KG*i ----
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int key = kg + KG * i;
        uint32_t qs[8];
        const float d = read_block<NB>(s_kv, key, j, qs);
        float acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t lo = magic2(0u, qs[e], kSelLo), hi = magic2(0u, qs[e], kSelHi);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                acc[h] = dot2(q2[h][2 * e], lo, acc[h]);
                acc[h] = dot2(q2[h][2 * e + 1], hi, acc[h]);
            }
        }
        float part[G];
#pragma unroll
        for (int h = 0; h < G; ++h) part[h] = d * (acc[h] - kMagic * qsum[h]);
        // sum over the NB lanes holding the blocks of this key (adjacent lanes)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int mm = 1; mm < NB; mm <<= 1) part[h] += __shfl_xor(part[h], mm, 64);
        if (j == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) s_p[h][key] = finish_score(f, part[h], b, hk * G + h, s0 + key);
        }
    }
    __syncthreads();

    // ---- V chunk into LDS; chunk softmax (thread = key slot) ----
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int u = tid + 256 * i;
        if (u < UNITS) *(u32x2 *)(s_kv + 8 * u) = vreg[i];
    }
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
    float pk[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float s = s_p[h][tid];
        pk[h] = (s == -INFINITY) ? 0.0f : exp2f(s - mx[h]);
        const float t = wave_sum(pk[h]);
        if (lane == 0) s_red[w][h] = t;
    }
    // p' = fp16(p * d_block) per (head, block) and the sums of the rounded values
    {
        const int key = tid;
#pragma unroll
        for (int jj = 0; jj < NB; ++jj) {
            const int off = key * RB + 34 * jj;
            const uint16_t dbits = *(const uint16_t *)(s_kv + off);
            const float d = h2f(dbits);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const _Float16 pq = (_Float16)(pk[h] * d);
                s_pq[h][jj][key] = pq;
                const float t = wave_sum((float)pq);
                if (lane == 0) atomicAdd(&s_pqsum[h][jj], t);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) sum[h] = (s_red[0][h] + s_red[1][h]) + (s_red[2][h] + s_red[3][h]);

    // ---- P.V: thread (vkg, oct) owns values 8*oct .. 8*oct+7 of keys vkg*VKEYS .. +VKEYS-1 ----
    const int oct = tid % NOCT, vkg = tid / NOCT;
    const int jb = oct / 4, part8 = oct % 4;  // block and 8-value slice inside it
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
#pragma unroll 2
    for (int kk = 0; kk < VKEYS; kk += 2) {
        const int k0 = vkg * VKEYS + kk;
        // 8 quantized values of each key: byte offset key*RB + 34jb + 2 + 8*part8
        uint32_t x0[2], x1[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int off = (k0 + r) * RB + 34 * jb + 2 + 8 * part8;
            const uint32_t *p = (const uint32_t *)(s_kv + (off & ~3));
            uint32_t lo, hi;
            if ((off & 3) == 0) {
                lo = p[0];
                hi = p[1];
            } else {
                lo = __builtin_amdgcn_alignbyte(p[1], p[0], 2);
                hi = __builtin_amdgcn_alignbyte(p[2], p[1], 2);
            }
            (r == 0 ? x0 : x1)[0] = lo;
            (r == 0 ? x0 : x1)[1] = hi;
        }
        // pairs (key k0, key k0+1) of value e, packed as fp16 (qs + 1152)
        uint32_t f2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t a0 = x0[e / 4], a1 = x1[e / 4];
            const uint32_t bsel = e % 4;  // byte of the dword
            // byte bsel of a0 -> byte 0, byte bsel of a1 -> byte 2 (selector 4+ picks a1)
            const uint32_t sel = 0x0c000c00u | bsel | ((4u + bsel) << 16);
            f2[e] = magic2(a1, a0, sel);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const uint32_t pq2 = *(const uint32_t *)&s_pq[h][jb][k0];  // (p'_k0, p'_k0+1)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = dot2(pq2, f2[e], acc[h][e]);
        }
    }
    // remove the 1152 offset, reduce the key groups of a wave (lanes NOCT apart), then across waves
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float off = kMagic * s_pqsum[h][jb] / (float)VKG;  // each key group carries 1/VKG of it
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[h][e] - off;
#pragma unroll
            for (int mm = NOCT; mm < 64; mm <<= 1) v += __shfl_xor(v, mm, 64);
            acc[h][e] = v;
        }
    }
    if (lane < NOCT) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) s_o[w][h][8 * oct + e] = acc[h][e];
    }
    __syncthreads();
    const int64_t row0 = (b * f.H + hk * G) * a.nsplit + split;
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

template <int D, int G>
hipError_t launch_q8(const DecodeArgs &a, hipStream_t s) {
    dim3 grid((unsigned)a.nsplit, (unsigned)(a.f.B * a.f.Hkv));
    hipLaunchKernelGGL((decode_q8_split_kernel<D, G>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

// The merge kernel is shared with the fp16 decode path.
hipError_t launch_attn_decode_merge(const DecodeArgs &a, int out_dtype, hipStream_t s);

bool attn_decode_q8_supported(const AttnFwdArgs &f, int q_dtype) {
    if (q_dtype != GT_F16 || f.out_dtype != GT_F16) return false;
    if (f.L != 1 || f.S <= 0 || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    const int64_t G = f.H / f.Hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return false;
    if (f.q_sh % 8 != 0 || f.q_sb % 8 != 0 || (uintptr_t)f.q % 16 != 0) return false;
    // K/V are whole dense Q8_0 tensors; rows are 8-byte aligned when the base is
    for (const void *p : {f.k, f.v}) if ((uintptr_t)p % 8 != 0) return false;
    return true;
}

hipError_t launch_attn_decode_q8(const DecodeArgs &a, hipStream_t s) {
    const int G = (int)(a.f.H / a.f.Hkv);
    hipError_t e = hipErrorInvalidValue;
#define GT_Q8_CASE(DD)                                   \
    switch (G) {                                         \
        case 1: e = launch_q8<DD, 1>(a, s); break;       \
        case 2: e = launch_q8<DD, 2>(a, s); break;       \
        case 4: e = launch_q8<DD, 4>(a, s); break;       \
        case 8: e = launch_q8<DD, 8>(a, s); break;       \
        default: break;                                  \
    }
    if (a.f.D == 128) {
        GT_Q8_CASE(128)
    } else {
        GT_Q8_CASE(64)
    }
#undef GT_Q8_CASE
    if (e != hipSuccess) return e;
    return launch_attn_decode_merge(a, GT_F16, s);
}
