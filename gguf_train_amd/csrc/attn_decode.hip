// Single-query (decode) attention: split-K over the KV length with every query head of a GQA
// group in one workgroup, so each K/V byte is read from HBM exactly once.
//
// The reference has no decode kernel: decode is gt_flash_attention with L = 1
// (csrc/gt_ops_nn.cpp:2423-2525), whose loop reads a kv head once per query head.  Semantics
// kept: scale, additive/bool mask, top-left causal (only key 0 when L = 1), empty rows -> 0.
//
// Work decomposition (HBM-bound; bytes per launch = K + V + Q + O):
//   workgroup = (kv head of one sequence, chunk of kChunk keys), 256 threads; every lane
//   issues all of its K and V loads for the chunk before using any of them.
//   D = 64, 128: the scores S^T (keys x heads) = K . Q^T run on v_mfma_f32_16x16x32_{f16,bf16}
//   with the G query heads as MFMA columns: lane l holds K[key l%16][32t + 8(l/16) .. +7] as the
//   A operand straight from memory (4 lanes read 64 consecutive bytes of a row), so no
//   cross-lane reduction is needed for a dot product.  D = 256: a key row is split over D/8
//   lanes, dot products with v_dot2_f32_{f16,bf16} summed across those lanes.
//   The chunk softmax runs in the log2 domain (exp2); P.V is a VALU fp32 accumulation over
//   coalesced V rows (D/8 lanes per row, 16-byte loads), reduced across lanes once per chunk.
// A second kernel merges the per-chunk (max, sum, unnormalised O) partials of each row.

#include "attn_common.h"
#include "decode_merge.h"
#include "gt_internal.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>

namespace {

constexpr int kChunk = 256;  // keys per workgroup = threads per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
    if (key >= attn_decode_end(f, b)) return -INFINITY;
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

template <typename T>
struct Mfma16;
template <>
struct Mfma16<_Float16> {
    typedef _Float16 V8 __attribute__((ext_vector_type(8)));
    static __device__ inline f32x4 mma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <>
struct Mfma16<__bf16> {
    typedef __bf16 V8 __attribute__((ext_vector_type(8)));
    static __device__ inline f32x4 mma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

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

// D = 64, 128: streaming kernel.  Workgroup = (kv head of one sequence, split); the split's
// keys are walked in steps of kStep = 128 keys, the loads of step s+1 in flight while step s is
// computed.  Wave w owns keys [32w, 32w + 32) of every step end to end (scores, softmax, P.V)
// and keeps its own online-softmax state, so steps need no workgroup barrier; the four waves
// are combined once at the end.  With a single split the kernel writes the output itself.
// v_mfma_f32_16x16x32 layouts (lane l): A[m = l%16][k = 8(l/16) + 0..7], B[k = 8(l/16) + 0..7][n = l%16],
// C[m = 4(l/16) + i][n = l%16], i = 0..3.
constexpr int kStep = 128;  // keys per step of a workgroup (32 per wave)

// MASK: 0 = none, 1 = bool bytes, 2 = additive float.
template <typename T, int D, int G, int MASK>
__global__ __launch_bounds__(256, 2) void decode_stream_kernel(DecodeArgs a) {
    using P = Pack<T>;
    using MM = Mfma16<T>;
    using V8 = typename MM::V8;
    constexpr int NT = D / 32;     // k-steps of the score MFMA
    constexpr int LPR = D / 8;     // lanes per V row (16 bytes each)
    constexpr int RPW = 64 / LPR;  // V rows per wave load
    constexpr int NV = 32 / RPW;   // V loads per lane and step
    // G = 8, 16: P.V on MFMA with the heads as its columns, A = V^T gathered from the wave's V
    // rows staged in LDS; G <= 4: P.V on VALU over the V rows in registers, the probabilities
    // shared through LDS
    constexpr bool PVM = G >= 8;
    constexpr int VS = D + 8;  // row stride (halfs) of the staged V rows
    __shared__ __attribute__((aligned(16))) float s_p[4][PVM ? 1 : 32][G];  // per-wave probabilities
    __shared__ __attribute__((aligned(16))) uint16_t s_v[PVM ? 4 : 1][32][PVM ? VS : 8];
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int sub = lane % LPR, vrow = lane / LPR;
    // The other grid dimension is (sequence, kv head, head group): the kv head's gtot query heads
    // run in groups of G (the last group may hold fewer, gv; its padding columns are blocked).
    // Workgroups go to the XCDs round robin by linear index.  Groups of up to 8 heads take the
    // splits along blockIdx.y, so an XCD gets whole (sequence, kv head) slices rather than one
    // split position of every other slice (benchmark shape: 86.0 -> 85.1 us).  16-head groups
    // keep the splits along blockIdx.x: the other head group of the kv head then runs on the
    // same XCD at the same time, and its re-read of the keys hits that L2.
    constexpr bool kSplitsY = G <= 8;
    const int split = kSplitsY ? blockIdx.y : blockIdx.x;
    const int gtot = (int)(f.H / f.Hkv), ngrp = (gtot + G - 1) / G;
    const int64_t bkg = kSplitsY ? blockIdx.x : blockIdx.y, bk = bkg / ngrp, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int hg = (int)(bkg % ngrp);
    const int h0 = (int)hk * gtot + hg * G, gv = min(G, gtot - hg * G);
    const int S = (int)f.S;
    const int span = ((S + kStep - 1) / kStep + a.nsplit - 1) / a.nsplit * kStep;  // keys per split
    const int kbeg = split * span, kend = min(attn_decode_end(f, b), kbeg + span);
    const int nsteps = kend > kbeg ? (kend - kbeg + kStep - 1) / kStep : 0;

    // B operand (Q^T): lane holds Q[head h0 + l16][32t + 8 q4 + 0..7]; columns l16 >= gv repeat
    // head h0 + gv - 1 and are discarded
    V8 qb[NT];
    {
        const T *qr = (const T *)f.q + b * f.q_sb + (h0 + min(l16, gv - 1)) * f.q_sh + 8 * q4;
#pragma unroll
        for (int t = 0; t < NT; ++t) qb[t] = __builtin_bit_cast(V8, *(const u32x4 *)(qr + 32 * t));
    }
    // K/V rows of a step; keys past S read row S-1 (finite; masked to -inf / weight 0).  Byte
    // offsets from the (b, kv head) bases fit 32 bits (checked by the launcher).  Every byte is
    // read once: nontemporal loads keep it from displacing useful lines in the caches.
    const char *kbase = (const char *)((const T *)f.k + b * f.k_sb + hk * f.k_sh);
    const char *vbase = (const char *)((const T *)f.v + b * f.v_sb + hk * f.v_sh);
    const uint32_t krow = (uint32_t)f.k_ss * (uint32_t)sizeof(T), vrowb = (uint32_t)f.v_ss * (uint32_t)sizeof(T);
    struct Tile {
        V8 k[2][NT];   // A operands: block kb = keys 16kb + l16 of the wave's 32
        u32x4 v[NV];   // V rows RPW*i + vrow of the wave's 32, dims 8 sub .. +7
    };
    // (16-head groups: plain loads, so that the other head groups of the kv head, which run at the
    // same time on the same XCD, find the lines in its L2)
    auto ld = [](const char *p) -> u32x4 {
        if constexpr (G > 8) return *(const u32x4 *)p;
        else return __builtin_nontemporal_load((const u32x4 *)p);
    };
    auto load = [&](int step, Tile &tl) {
        const int k0 = kbeg + step * kStep + 32 * w;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const uint32_t off = (uint32_t)min(k0 + 16 * kb + l16, S - 1) * krow + 16u * q4;
#pragma unroll
            for (int t = 0; t < NT; ++t) tl.k[kb][t] = __builtin_bit_cast(V8, ld(kbase + off + 64 * t));
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t off = (uint32_t)min(k0 + RPW * i + vrow, S - 1) * vrowb + 16u * sub;
            tl.v[i] = ld(vbase + off);
        }
    };

    const float cs = f.scale * kLog2e;
    const int64_t mrow = b * f.m_sb + (h0 + min(l16, gv - 1)) * f.m_sh;
    float m = -INFINITY;  // running max of head l16 (log2 domain), same in the 4 lanes of a head
    float lsum = 0.0f;    // running sum of head l16
    float acc[PVM ? 1 : G][8];  // VALU P.V: unnormalised O of every head, dims 8 sub .. +7, this lane's rows
#pragma unroll
    for (int h = 0; h < (PVM ? 1 : G); ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
    f32x4 accm[PVM ? D / 16 : 1];  // MFMA P.V: C[dim 16 blk + 4 q4 + i][head l16]
#pragma unroll
    for (int blk = 0; blk < (PVM ? D / 16 : 1); ++blk) accm[blk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int step, const Tile &tl) {
        const int k0 = kbeg + step * kStep + 32 * w;
        float sc[2][4];
        float cm = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < NT; ++t) c4 = MM::mma(tl.k[kb][t], qb[t], c4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + 16 * kb + 4 * q4 + i;
                float x = c4[i] * cs;
                bool blocked = key >= kend || l16 >= gv;
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
        if constexpr (PVM) {
            // the wave's 32 V rows into LDS, then per block of 16 dims one MFMA: A[dim][k-slot]
            // = V^T, B[k-slot][head] = P, k-slot e of lane group q4 being key 16(e/4) + 4 q4 + e%4
            // (this lane's sc[e/4][e%4])
#pragma unroll
            for (int i = 0; i < NV; ++i) *(u32x4 *)&s_v[w][RPW * i + vrow][8 * sub] = tl.v[i];
            if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
                for (int blk = 0; blk < D / 16; ++blk) accm[blk] *= alpha;  // head l16's factor
            }
            // bf16 keeps 8 bits of a probability: P goes in as hi + lo bf16 operands (two MFMAs,
            // ~16 bits, as lsum's fp32 P), fp16 as one operand (11 bits)
            constexpr bool kSplitP = __is_same(T, __bf16);
            V8 bp, bpl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = sc[e >> 2][e & 3];
                const T xh = (T)x;
                bp[e] = xh;
                if constexpr (kSplitP) bpl[e] = (T)(x - (float)xh);
            }
            __builtin_amdgcn_wave_barrier();  // s_v written by this wave before it is read
#pragma unroll
            for (int blk = 0; blk < D / 16; ++blk) {
                const uint16_t *col = &s_v[w][4 * q4][16 * blk + l16];
                u32x4 av;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 16 * (j >> 1) + 2 * (j & 1);  // k-slots 2j, 2j + 1: rows r, r + 1 past 4 q4
                    av[j] = (uint32_t)col[r * VS] | ((uint32_t)col[(r + 1) * VS] << 16);
                }
                accm[blk] = MM::mma(__builtin_bit_cast(V8, av), bp, accm[blk]);
                if constexpr (kSplitP) accm[blk] = MM::mma(__builtin_bit_cast(V8, av), bpl, accm[blk]);
            }
            __builtin_amdgcn_wave_barrier();  // s_v read before the next step overwrites it
        } else {
            if (l16 < G) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s_p[w][16 * kb + 4 * q4 + i][l16] = sc[kb][i];
            }
            // the head-h rescale factor sits in lane h
            float al[G];
#pragma unroll
            for (int h = 0; h < G; ++h) al[h] = __shfl(alpha, h, 64);
            __builtin_amdgcn_wave_barrier();  // s_p written by this wave before it is read
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[h][j] *= al[h];
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int r = RPW * i + vrow;
                float vf[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    vf[2 * j] = P::lo(tl.v[i][j]);
                    vf[2 * j + 1] = P::hi(tl.v[i][j]);
                }
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float p = s_p[w][r][h];
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(p, vf[j], acc[h][j]);
                }
            }
            __builtin_amdgcn_wave_barrier();  // s_p read before the next step overwrites it
        }
    };

    // two tiles in flight, unrolled by two so they swap roles without copies.  (Measured: issuing
    // the prefetch under these branches, which makes the compiler wait for it as well, is faster
    // on this kernel than keeping it in flight across the compute.)  Wave priority follows the
    // step (progress_priority: the two workgroups on a CU stay level).
    Tile ta, tb;
    if (nsteps > 0) load(0, ta);
    for (int st = 0; st < nsteps; st += 2) {
        progress_priority(st);
        if (st + 1 < nsteps) load(st + 1, tb);
        __builtin_amdgcn_sched_barrier(0);
        compute(st, ta);
        if (st + 1 < nsteps) {
            progress_priority(st + 1);
            if (st + 2 < nsteps) load(st + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            compute(st + 1, tb);
        }
    }
    __builtin_amdgcn_s_setprio(3);

    // ---- combine the four waves ----
    if (lane < G) {
        s_m[w][lane] = m;
        s_l[w][lane] = lsum;
    }
    if constexpr (PVM) {
        if (l16 < G) {
#pragma unroll
            for (int blk = 0; blk < D / 16; ++blk)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_o[w][l16][16 * blk + 4 * q4 + i] = accm[blk][i];
        }
    } else {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int mm = LPR; mm < 64; mm <<= 1) acc[h][j] += __shfl_xor(acc[h][j], mm, 64);
        if (lane < LPR) {
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) s_o[w][h][8 * sub + j] = acc[h][j];
        }
    }
    __syncthreads();
    for (int e = tid; e < gv * D; e += 256) {
        const int h = e / D, d = e % D;
        const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float o = 0.0f, L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float wg = s_m[ww][h] == -INFINITY ? 0.0f : fast_exp2(s_m[ww][h] - M);
            o = fmaf(wg, s_o[ww][h][d], o);
            L = fmaf(wg, s_l[ww][h], L);
        }
        const int64_t row = b * f.H + h0 + h;
        if (a.nsplit == 1) {
            // the whole key range: normalise and store
            store_t<T>(f.o, row * D + d, L > 0.0f ? o / L : 0.0f);
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
    if (a.nsplit > 1 && a.counters) gtdecode::finish_split<T, D>(a, bkg, b * f.H + h0, gv);
}

// Float32 K/V, D = 64, 128: the streaming kernel's decomposition (workgroup = (sequence, kv
// head, head group) x split; each wave owns its keys of every step end to end; the waves combine
// once at the end; the last split merges in the kernel) with float32 operands and 16 keys per
// wave and step.  Scores S^T = K.Q^T on v_mfma_f32_16x16x4_f32 with the heads as its columns:
// lane (l16, q4) reads 16 bytes of key l16's row at dims 16t + 4q4 .. +3 (four lanes read 64
// consecutive bytes), and MFMA (t, e) takes k index q4 as dim 16t + 4q4 + e, the same dim in the
// lane's Q^T operand; accumulator entry i is key 4q4 + i, head l16.  P.V on the VALU in float32
// over 16-byte V rows, the probabilities shared through LDS.  Groups of up to 8 heads.
// v_mfma_f32_16x16x4_f32 layouts (lane l): A[m = l%16][k = l/16], B[k = l/16][n = l%16],
// C[m = 4(l/16) + i][n = l%16], i = 0..3.
constexpr int kStepF32 = 64;  // keys per step of a workgroup (16 per wave)

// D = 128 with 8 heads holds two 16 KB tiles, Q and acc[8][4] per lane: one workgroup per CU
// (512 registers; two would spill), whose 4 waves x 2 tiles in flight still cover the CU's
// share of the memory latency.
template <int D, int G, int MASK>
__global__ __launch_bounds__(256, (D == 128 && G == 8) ? 1 : 2) void decode_f32_kernel(DecodeArgs a) {
    constexpr int NT = D / 16;     // 16-byte K pieces per lane and key block (4 MFMAs each)
    constexpr int LPR = D / 4;     // lanes per V row (16 bytes each)
    constexpr int RPW = 64 / LPR;  // V rows per wave load
    constexpr int NV = 16 / RPW;   // V loads per lane and step
    static_assert(G <= kDecodeF32MaxTile && NV >= 1, "decode_f32 tile");
    __shared__ __attribute__((aligned(16))) float s_p[4][16][G];  // per-wave probabilities
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_o[4][G][D];

    const AttnFwdArgs &f = a.f;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int sub = lane % LPR, vrow = lane / LPR;
    // blockIdx.x = (sequence, kv head, head group), blockIdx.y = split (an XCD gets whole slices)
    const int split = blockIdx.y;
    const int gtot = (int)(f.H / f.Hkv), ngrp = (gtot + G - 1) / G;
    const int64_t bkg = blockIdx.x, bk = bkg / ngrp, b = bk / f.Hkv, hk = bk % f.Hkv;
    const int hg = (int)(bkg % ngrp);
    const int h0 = (int)hk * gtot + hg * G, gv = min(G, gtot - hg * G);
    const int S = (int)f.S;
    const int span = ((S + kStepF32 - 1) / kStepF32 + a.nsplit - 1) / a.nsplit * kStepF32;  // keys per split
    const int kbeg = split * span, kend = min(attn_decode_end(f, b), kbeg + span);
    const int nsteps = kend > kbeg ? (kend - kbeg + kStepF32 - 1) / kStepF32 : 0;

    // B operand (Q^T): lane holds Q[head h0 + l16][16t + 4q4 .. +3]; columns l16 >= gv repeat
    // head h0 + gv - 1 and are discarded
    f32x4 qb[NT];
    {
        const float *qr = (const float *)f.q + b * f.q_sb + (h0 + min(l16, gv - 1)) * f.q_sh + 4 * q4;
#pragma unroll
        for (int t = 0; t < NT; ++t) qb[t] = *(const f32x4 *)(qr + 16 * t);
    }
    // K/V rows of a step; keys past S read row S-1 (finite; masked to -inf / weight 0).  Byte
    // offsets from the (b, kv head) bases fit 32 bits (checked by the launcher); nontemporal
    // loads, every byte is read once.
    const char *kbase = (const char *)((const float *)f.k + b * f.k_sb + hk * f.k_sh);
    const char *vbase = (const char *)((const float *)f.v + b * f.v_sb + hk * f.v_sh);
    const uint32_t krow = (uint32_t)f.k_ss * 4u, vrowb = (uint32_t)f.v_ss * 4u;
    struct Tile {
        f32x4 k[NT];  // K[key l16 of the wave's 16][16t + 4q4 .. +3]
        f32x4 v[NV];  // V rows RPW*i + vrow of the wave's 16, dims 4 sub .. +3
    };
    auto load = [&](int step, Tile &tl) {
        const int k0 = kbeg + step * kStepF32 + 16 * w;
        const uint32_t koff = (uint32_t)min(k0 + l16, S - 1) * krow + 16u * q4;
#pragma unroll
        for (int t = 0; t < NT; ++t) tl.k[t] = __builtin_nontemporal_load((const f32x4 *)(kbase + koff + 64 * t));
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t off = (uint32_t)min(k0 + RPW * i + vrow, S - 1) * vrowb + 16u * sub;
            tl.v[i] = __builtin_nontemporal_load((const f32x4 *)(vbase + off));
        }
    };

    const float cs = f.scale * kLog2e;
    const int64_t mrow = b * f.m_sb + (h0 + min(l16, gv - 1)) * f.m_sh;
    float m = -INFINITY;  // running max of head l16 (log2 domain), same in the 4 lanes of a head
    float lsum = 0.0f;    // running sum of head l16
    float acc[G][4];      // unnormalised O of every head, dims 4 sub .. +3, this lane's rows
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[h][j] = 0.0f;

    auto compute = [&](int step, const Tile &tl) {
        const int k0 = kbeg + step * kStepF32 + 16 * w;
        // two accumulators (even and odd pieces) halve the dependent MFMA chain
        f32x4 ca = {0.0f, 0.0f, 0.0f, 0.0f}, cb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < NT; t += 2)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ca = __builtin_amdgcn_mfma_f32_16x16x4f32(tl.k[t][e], qb[t][e], ca, 0, 0, 0);
                cb = __builtin_amdgcn_mfma_f32_16x16x4f32(tl.k[t + 1][e], qb[t + 1][e], cb, 0, 0, 0);
            }
        float sc[4];
        float cm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = k0 + 4 * q4 + i;
            float x = (ca[i] + cb[i]) * cs;
            bool blocked = key >= kend || l16 >= gv;
            if (MASK != 0) {
                const int64_t mi = mrow + (int64_t)min(key, S - 1) * f.m_ss;
                if (MASK == 1) blocked = blocked || !((const uint8_t *)f.mask)[mi];
                else x = fmaf(((const float *)f.mask)[mi], kLog2e, x);
            }
            x = blocked ? -INFINITY : x;
            sc[i] = x;
            cm = fmaxf(cm, x);
        }
        cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
        cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
        const float mnew = fmaxf(m, cm);
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = mnew == -INFINITY ? 1.0f : fast_exp2(m - mnew);  // m = -inf: 0
        m = mnew;
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = fast_exp2(sc[i] - msub);  // -inf -> 0
            ps += sc[i];
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        lsum = fmaf(lsum, alpha, ps);
        if (l16 < G) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s_p[w][4 * q4 + i][l16] = sc[i];
        }
        // the head-h rescale factor sits in lane h
        float al[G];
#pragma unroll
        for (int h = 0; h < G; ++h) al[h] = __shfl(alpha, h, 64);
        __builtin_amdgcn_wave_barrier();  // s_p written by this wave before it is read
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[h][j] *= al[h];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int r = RPW * i + vrow;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = s_p[w][r][h];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[h][j] = fmaf(p, tl.v[i][j], acc[h][j]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // s_p read before the next step overwrites it
    };

    // two tiles in flight, unrolled by two so they swap roles without copies; wave priority
    // follows the step (the two workgroups on a CU stay level)
    Tile ta, tb;
    if (nsteps > 0) load(0, ta);
    for (int st = 0; st < nsteps; st += 2) {
        progress_priority(st);
        if (st + 1 < nsteps) load(st + 1, tb);
        __builtin_amdgcn_sched_barrier(0);
        compute(st, ta);
        if (st + 1 < nsteps) {
            progress_priority(st + 1);
            if (st + 2 < nsteps) load(st + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            compute(st + 1, tb);
        }
    }
    __builtin_amdgcn_s_setprio(3);

    // ---- combine the four waves ----
    if (lane < G) {
        s_m[w][lane] = m;
        s_l[w][lane] = lsum;
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mm = LPR; mm < 64; mm <<= 1) acc[h][j] += __shfl_xor(acc[h][j], mm, 64);
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) s_o[w][h][4 * sub + j] = acc[h][j];
    }
    __syncthreads();
    for (int e = tid; e < gv * D; e += 256) {
        const int h = e / D, d = e % D;
        const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float o = 0.0f, L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float wg = s_m[ww][h] == -INFINITY ? 0.0f : fast_exp2(s_m[ww][h] - M);
            o = fmaf(wg, s_o[ww][h][d], o);
            L = fmaf(wg, s_l[ww][h], L);
        }
        const int64_t row = b * f.H + h0 + h;
        if (a.nsplit == 1) {
            store_t<float>(f.o, row * D + d, L > 0.0f ? o / L : 0.0f);
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
    if (a.nsplit > 1 && a.counters) gtdecode::finish_split<float, D>(a, bkg, b * f.H + h0, gv);
}

// D = 256: a key row is split over D/8 lanes (16-byte loads), dot products reduced across lanes.
template <typename T, int D, int G>
__global__ __launch_bounds__(256) void decode_rows_kernel(DecodeArgs a) {
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

// One wave per (b, h) row: out = sum_i 2^(m_i - M) O_i / sum_i 2^(m_i - M) l_i.  A split's
// partial O row is read as 16-byte pieces by D/4 lanes, 64/(D/4) splits per wave load, eight
// independent loads per lane in flight.
template <typename TO, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int LPS = D / 4;     // lanes per partial row
    constexpr int SPW = 64 / LPS;  // partial rows per wave load
    constexpr int U = 8;           // loads in flight per lane
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + w;
    if (row >= f.B * f.H) return;
    const int ns = a.nsplit;
    const float *ml = a.part_ml + row * ns * 2;
    float M = -INFINITY;
    for (int i = lane; i < ns; i += 64) M = fmaxf(M, ml[2 * i]);
    M = wave_max(M);
    float L = 0.0f;
    for (int i = lane; i < ns; i += 64) {
        const float m = ml[2 * i];
        L += m == -INFINITY ? 0.0f : fast_exp2(m - M) * ml[2 * i + 1];
    }
    L = wave_sum(L);
    const int sub = lane % LPS, sp = lane / LPS;
    const float *po = a.part_o + row * ns * D + 4 * sub;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < ns; i0 += SPW * U) {
        f32x4 x[U];
        float wgt[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(i0 + SPW * u + sp, ns - 1);
            x[u] = *(const f32x4 *)(po + (int64_t)i * D);
            const float m = ml[2 * i];
            wgt[u] = (i0 + SPW * u + sp >= ns || m == -INFINITY) ? 0.0f : fast_exp2(m - M);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += wgt[u] * x[u];
    }
#pragma unroll
    for (int m = LPS; m < 64; m <<= 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += __shfl_xor(acc[j], m, 64);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (lane < LPS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) store_t<TO>(f.o, row * D + 4 * sub + j, acc[j] * inv);
    }
    if (f.lse && lane == 0) ((float *)f.lse)[row] = L > 0.0f ? (M + log2f(L)) * kLn2 : INFINITY;
}

template <typename T, int D, int G>
hipError_t launch_typed(const DecodeArgs &a, hipStream_t s) {
    dim3 grid((unsigned)a.nsplit, (unsigned)decode_units(a.f.B, a.f.H, a.f.Hkv, kDecodeMaxTile));
    if constexpr (D <= 128) {
        if constexpr (G <= 8) grid = dim3(grid.y, grid.x);  // the stream kernel's split axis (kSplitsY)
        const int mode = !a.f.mask ? 0 : (a.f.mask_bool ? 1 : 2);
        if (mode == 0) hipLaunchKernelGGL((decode_stream_kernel<T, D, G, 0>), grid, dim3(256), 0, s, a);
        else if (mode == 1) hipLaunchKernelGGL((decode_stream_kernel<T, D, G, 1>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((decode_stream_kernel<T, D, G, 2>), grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((decode_rows_kernel<T, D, G>), grid, dim3(256), 0, s, a);
    }
    hipError_t e = hipGetLastError();
    // one split of the streaming kernel, or its last split merged in the kernel: it wrote the output
    if (e != hipSuccess || (D <= 128 && (a.nsplit == 1 || a.counters))) return e;
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
        case 16:
            if constexpr (D <= 128) return launch_typed<T, D, 16>(a, s);
            return hipErrorInvalidValue;
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

template <int D, int G>
hipError_t launch_f32_g(const DecodeArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)decode_units(a.f.B, a.f.H, a.f.Hkv, kDecodeF32MaxTile), (unsigned)a.nsplit);
    const int mode = !a.f.mask ? 0 : (a.f.mask_bool ? 1 : 2);
    if (mode == 0) hipLaunchKernelGGL((decode_f32_kernel<D, G, 0>), grid, dim3(256), 0, s, a);
    else if (mode == 1) hipLaunchKernelGGL((decode_f32_kernel<D, G, 1>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((decode_f32_kernel<D, G, 2>), grid, dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    // one split, or the last split merged in the kernel: it wrote the output
    if (e != hipSuccess || a.nsplit == 1 || a.counters) return e;
    const int64_t rows = a.f.B * a.f.H;
    hipLaunchKernelGGL((decode_merge_kernel<float, D>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int D>
hipError_t launch_f32_d(const DecodeArgs &a, hipStream_t s) {
    switch (decode_head_tile(a.f.H / a.f.Hkv, kDecodeF32MaxTile)) {
        case 1: return launch_f32_g<D, 1>(a, s);
        case 2: return launch_f32_g<D, 2>(a, s);
        case 4: return launch_f32_g<D, 4>(a, s);
        case 8: return launch_f32_g<D, 8>(a, s);
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

namespace {

// The streaming kernel instance a launch of `f` uses (compute dtype cd).
template <typename T, int D>
const void *stream_kernel_d(const AttnFwdArgs &f, int G) {
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
#define GT_SK(GG) \
    (mode == 0 ? (const void *)decode_stream_kernel<T, D, GG, 0> \
               : mode == 1 ? (const void *)decode_stream_kernel<T, D, GG, 1> : (const void *)decode_stream_kernel<T, D, GG, 2>)
    switch (G) {
        case 1: return GT_SK(1);
        case 2: return GT_SK(2);
        case 4: return GT_SK(4);
        case 8: return GT_SK(8);
        case 16: return GT_SK(16);
        default: return nullptr;
    }
#undef GT_SK
}

template <int D>
const void *f32_kernel_d(const AttnFwdArgs &f, int G) {
    const int mode = !f.mask ? 0 : (f.mask_bool ? 1 : 2);
#define GT_FK(GG) \
    (mode == 0 ? (const void *)decode_f32_kernel<D, GG, 0> \
               : mode == 1 ? (const void *)decode_f32_kernel<D, GG, 1> : (const void *)decode_f32_kernel<D, GG, 2>)
    switch (G) {
        case 1: return GT_FK(1);
        case 2: return GT_FK(2);
        case 4: return GT_FK(4);
        case 8: return GT_FK(8);
        default: return nullptr;
    }
#undef GT_FK
}

const void *stream_kernel(const AttnFwdArgs &f, int cd) {
    if (cd == GT_F32) {
        const int G = decode_head_tile(f.H / f.Hkv, kDecodeF32MaxTile);
        return f.D == 128 ? f32_kernel_d<128>(f, G) : f32_kernel_d<64>(f, G);
    }
    const int G = decode_head_tile(f.H / f.Hkv, kDecodeMaxTile);
    if (cd == GT_F16) return f.D == 128 ? stream_kernel_d<_Float16, 128>(f, G) : stream_kernel_d<_Float16, 64>(f, G);
    return f.D == 128 ? stream_kernel_d<__bf16, 128>(f, G) : stream_kernel_d<__bf16, 64>(f, G);
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

int attn_decode_splits(const AttnFwdArgs &f, int cd) {
    if (f.D > 128) return (int)((f.S + kChunk - 1) / kChunk);  // one 256-key chunk per workgroup
    // Streaming kernel: workgroups of equal length, as many splits as keep every CU busy
    // without a partial last round; each extra split costs a little merge work.
    const void *kernel = stream_kernel(f, cd);
    const int64_t slots = kernel ? resident_slots(kernel) : 512;
    const int64_t step = cd == GT_F32 ? kStepF32 : kStep;
    const int64_t steps = (f.S + step - 1) / step;
    return decode_split_count(decode_units(f.B, f.H, f.Hkv, attn_decode_max_tile(cd)), steps, slots,
                              std::min<int64_t>(64, steps));
}

int attn_decode_max_tile(int cd) { return cd == GT_F32 ? kDecodeF32MaxTile : kDecodeMaxTile; }

bool attn_decode_supported(const AttnFwdArgs &f, int cd) {
    if (cd == GT_F32) {
        if (f.L != 1 || f.S <= 0 || f.D != f.Dv || (f.D != 64 && f.D != 128)) return false;
        if (f.S >= (1LL << 30)) return false;  // 32-bit key indices
        if ((f.S - 1) * f.k_ss * 4 + f.D * 4 > 0xffffffffLL || (f.S - 1) * f.v_ss * 4 + f.D * 4 > 0xffffffffLL) return false;
        if (decode_units(f.B, f.H, f.Hkv, kDecodeF32MaxTile) >= (1LL << 31)) return false;  // grid.x
        // 16-byte row loads: every row start must be 16-byte aligned
        const int64_t strides[] = {f.q_sb, f.q_sh, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
        for (int64_t st : strides) if (st % 4 != 0) return false;
        for (const void *p : {f.q, f.k, f.v}) if ((uintptr_t)p % 16 != 0) return false;
        return true;
    }
    if (cd != GT_F16 && cd != GT_BF16) return false;
    if (f.L != 1 || f.S <= 0 || f.D != f.Dv) return false;
    if (f.S >= (1LL << 30)) return false;  // 32-bit key indices
    // 32-bit byte offsets of K/V rows from the (batch, kv head) base
    if ((f.S - 1) * f.k_ss * 2 + f.D * 2 > 0xffffffffLL || (f.S - 1) * f.v_ss * 2 + f.D * 2 > 0xffffffffLL) return false;
    if (f.D != 64 && f.D != 128 && f.D != 256) return false;
    // any number of query heads per kv head on the streaming kernel (D <= 128), in groups of
    // up to 16; the D = 256 kernel takes 1, 2, 4 or 8
    const int64_t G = f.H / f.Hkv;
    if (f.D == 256 && G != 1 && G != 2 && G != 4 && G != 8) return false;
    if (decode_units(f.B, f.H, f.Hkv, kDecodeMaxTile) > 65535) return false;  // grid.y
    // 16-byte row loads: every row start must be 16-byte aligned
    const int64_t strides[] = {f.q_sb, f.q_sh, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh, f.v_ss};
    for (int64_t st : strides) if (st % 8 != 0) return false;
    for (const void *p : {f.q, f.k, f.v}) if ((uintptr_t)p % 16 != 0) return false;
    return true;
}

hipError_t launch_attn_decode(const DecodeArgs &a, int cd, hipStream_t s) {
    const int G = decode_head_tile(a.f.H / a.f.Hkv, kDecodeMaxTile);
    if (cd == GT_F16) return launch_d<_Float16>(a, G, s);
    if (cd == GT_BF16) return launch_d<__bf16>(a, G, s);
    if (cd == GT_F32) return a.f.D == 128 ? launch_f32_d<128>(a, s) : launch_f32_d<64>(a, s);
    return hipErrorInvalidValue;
}
