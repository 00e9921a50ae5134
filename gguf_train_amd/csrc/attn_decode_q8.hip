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

// Two int8 values -> packed fp16 (qs + 1152): bytes selected by `sel` from x into the low byte
// of each half, then the 0x64 exponent and the sign flip.
__device__ inline uint32_t magic2(uint32_t x, uint32_t sel) { return __builtin_amdgcn_perm(0u, x, sel) ^ 0x64806480u; }
// selectors: bytes (b0,b1) and (b2,b3) of x into the two halves (0x0c = zero byte)
constexpr uint32_t kSelLo = 0x0c010c00u;
constexpr uint32_t kSelHi = 0x0c030c02u;

// 12 loaded bytes -> the 8 quantized values as 4 packed fp16 (qs + 1152) and the raw scale
// bits (meaningful in the block's first lane).  `odd`: block index odd (see the header).
__device__ inline void unpack12(u32x3 w, bool odd, u32x4 &mag, uint32_t &dbits) {
    uint32_t q0, q1;
    if (odd) {
        q0 = w[1];
        q1 = w[2];
        dbits = w[0] >> 16;
    } else {
        q0 = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
        q1 = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
        dbits = w[0] & 0xffffu;
    }
    mag[0] = magic2(q0, kSelLo);
    mag[1] = magic2(q0, kSelHi);
    mag[2] = magic2(q1, kSelLo);
    mag[3] = magic2(q1, kSelHi);
}

// MASK: 0 = none, 1 = bool bytes, 2 = additive float.
template <int D, int G, int MASK>
__global__ __launch_bounds__(256, 2) void decode_q8_stream_kernel(DecodeArgs a) {
    constexpr int NB = D / 32;     // Q8_0 blocks per row = k-steps of the score MFMA
    constexpr int RB = NB * 34;    // bytes per row
    constexpr int LPR = D / 8;     // lanes per V row (8 values each)
    constexpr int RPW = 64 / LPR;  // V rows per wave load
    constexpr int NV = 32 / RPW;   // V loads per lane and step
    __shared__ __attribute__((aligned(16))) float s_p[4][32][G];   // per-wave probabilities
    __shared__ __attribute__((aligned(16))) float s_d[4][32][NB];  // per-wave K block scales
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int sub = lane % LPR, vrow = lane / LPR;
    const int vblk = sub >> 2, vpart = sub & 3;  // V: block and 8-value part of this lane
    const int split = blockIdx.x;
    const int64_t bk = blockIdx.y, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int S = (int)f.S;
    const int span = ((S + kStep - 1) / kStep + a.nsplit - 1) / a.nsplit * kStep;
    const int kbeg = split * span, kend = min(attn_decode_end(f, b), kbeg + span);
    const int nsteps = kend > kbeg ? (kend - kbeg + kStep - 1) / kStep : 0;

    // B operand (Q^T, fp16): lane holds Q[head l16][32t + 8 q4 + 0..7]; columns l16 >= G repeat
    // head G-1 and are discarded.  cq[t]: sum of block t of head l16's query.
    half8_t qb[NB];
    float cq[NB];
    {
        const _Float16 *qr = (const _Float16 *)f.q + b * f.q_sb + (hk * G + min(l16, G - 1)) * f.q_sh + 8 * q4;
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
        const int k0 = kbeg + step * kStep + 32 * w;
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
    const int64_t mrow = b * f.m_sb + (hk * G + min(l16, G - 1)) * f.m_sh;
    float m = -INFINITY;  // running max of head l16 (log2 domain)
    float lsum = 0.0f;    // running sum of head l16
    float acc[G][8];      // unnormalised sum of p d (qs + 1152), dims 8 sub .. +7, this lane's rows
    float csum[G];        // sum of p d over this lane's rows (the offset to remove)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        csum[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
    }

    auto compute = [&](int step, const Tile &tl) {
        const int k0 = kbeg + step * kStep + 32 * w;
        // K operands and scales
        half8_t ka[2][NB];
        float dk[2][NB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                u32x4 mag;
                uint32_t db;
                unpack12(tl.k[kb][t], t & 1, mag, db);
                ka[kb][t] = __builtin_bit_cast(half8_t, mag);
                dk[kb][t] = h2f(db);
            }
        if (q4 == 0) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int t = 0; t < NB; ++t) s_d[w][16 * kb + l16][t] = dk[kb][t];
        }
        __builtin_amdgcn_wave_barrier();  // s_d written by this wave before it is read
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
                bool blocked = key >= kend || l16 >= G;
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
        if (l16 < G) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_p[w][16 * kb + 4 * q4 + i][l16] = sc[kb][i];
        }
        float al[G];
#pragma unroll
        for (int h = 0; h < G; ++h) al[h] = __shfl(alpha, h, 64);
        __builtin_amdgcn_wave_barrier();  // s_p written by this wave before it is read
#pragma unroll
        for (int h = 0; h < G; ++h) {
            csum[h] *= al[h];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] *= al[h];
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int r = RPW * i + vrow;
            u32x4 mag;
            uint32_t db;
            unpack12(tl.v[i], vblk & 1, mag, db);
            // the block's scale sits in the first lane of each group of 4 (quad broadcast)
            const float dv = h2f((uint32_t)__builtin_amdgcn_mov_dpp((int)db, 0x00, 0xf, 0xf, false));
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float pd = s_p[w][r][h] * dv;
                csum[h] += pd;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t mj = mag[j];
                    acc[h][2 * j] = fmaf(pd, hlo(mj), acc[h][2 * j]);
                    acc[h][2 * j + 1] = fmaf(pd, hhi(mj), acc[h][2 * j + 1]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // s_p / s_d read before the next step overwrites them
    };

    Tile ta, tb;
    if (nsteps > 0) load(0, ta);
    for (int st = 0; st < nsteps; st += 2) {
        if (st + 1 < nsteps) load(st + 1, tb);
        __builtin_amdgcn_sched_barrier(0);
        compute(st, ta);
        if (st + 1 < nsteps) {
            if (st + 2 < nsteps) load(st + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            compute(st + 1, tb);
        }
    }

    // ---- remove the offset, combine the four waves ----
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[h][j] = fmaf(-kMagic, csum[h], acc[h][j]);
#pragma unroll
            for (int mm = LPR; mm < 64; mm <<= 1) acc[h][j] += __shfl_xor(acc[h][j], mm, 64);
        }
    if (lane < G) {
        s_m[w][lane] = m;
        s_l[w][lane] = lsum;
    }
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) s_o[w][h][8 * sub + j] = acc[h][j];
    }
    __syncthreads();
    for (int e = tid; e < G * D; e += 256) {
        const int h = e / D, d = e % D;
        const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float o = 0.0f, L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float wg = s_m[ww][h] == -INFINITY ? 0.0f : fast_exp2(s_m[ww][h] - M);
            o = fmaf(wg, s_o[ww][h][d], o);
            L = fmaf(wg, s_l[ww][h], L);
        }
        const int64_t row = b * f.H + hk * G + h;
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
}

template <int D>
const void *q8_kernel_d(const AttnFwdArgs &f, int G) {
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
#define GT_QK(GG) \
    (mode == 0 ? (const void *)decode_q8_stream_kernel<D, GG, 0> \
               : mode == 1 ? (const void *)decode_q8_stream_kernel<D, GG, 1> : (const void *)decode_q8_stream_kernel<D, GG, 2>)
    switch (G) {
        case 1: return GT_QK(1);
        case 2: return GT_QK(2);
        case 4: return GT_QK(4);
        case 8: return GT_QK(8);
        default: return nullptr;
    }
#undef GT_QK
}

const void *q8_kernel(const AttnFwdArgs &f) {
    const int G = (int)(f.H / f.Hkv);
    return f.D == 128 ? q8_kernel_d<128>(f, G) : q8_kernel_d<64>(f, G);
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
    const int64_t wgs = f.B * f.Hkv;
    const int64_t maxs = std::min<int64_t>(64, (f.S + kStep - 1) / kStep);
    int best = 1;
    double best_cost = 1e30;
    for (int64_t n = 1; n <= maxs; ++n) {
        const double cost = (double)((wgs * n + slots - 1) / slots) / (double)n + (n > 1 ? 0.02 * (double)n : 0.0);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = (int)n;
        }
    }
    return best;
}

bool attn_decode_q8_supported(const AttnFwdArgs &f, int q_dtype) {
    if (q_dtype != GT_F16 || f.out_dtype != GT_F16) return false;
    if (f.L != 1 || f.S <= 0 || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
    if (f.S >= (1LL << 30) || f.S * (f.D / 32 * 34) > 0xffffffffLL) return false;  // 32-bit offsets
    const int64_t G = f.H / f.Hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return false;
    if (f.q_sh % 8 != 0 || f.q_sb % 8 != 0 || (uintptr_t)f.q % 16 != 0) return false;
    // K/V are whole dense Q8_0 tensors; rows are 4-byte aligned when the base is
    for (const void *p : {f.k, f.v}) if ((uintptr_t)p % 8 != 0) return false;
    return true;
}

hipError_t launch_attn_decode_q8(const DecodeArgs &a, hipStream_t s) {
    const void *kernel = q8_kernel(a.f);
    if (!kernel) return hipErrorInvalidValue;
    dim3 grid((unsigned)a.nsplit, (unsigned)(a.f.B * a.f.Hkv));
    void *args[] = {(void *)&a};
    hipError_t e = hipLaunchKernel(kernel, grid, dim3(256), args, 0, s);
    if (e != hipSuccess || a.nsplit == 1) return e;  // one split: the kernel wrote the output
    return launch_attn_decode_merge(a, GT_F16, s);
}
