// Parameters shared by the attention kernels and the host-side dispatcher.
//
// Layouts (elements, innermost dimension contiguous):
//   q  (B, H,   L, D)   element (b,h,l,d)  at q + b*q_sb + h*q_sh + l*q_sl + d
//   k  (B, Hkv, S, D)   element (b,g,s,d)  at k + b*k_sb + g*k_sh + s*k_ss + d
//   v  (B, Hkv, S, Dv)  element (b,g,s,d)  at v + b*v_sb + g*v_sh + s*v_ss + d
//   o  (B, H,   L, Dv)  dense
//   lse (B, H, L)       dense, natural-log log-sum-exp of the scaled, masked scores
//   mask                element (b,h,l,s) at mask + b*m_sb + h*m_sh + l*m_sl + s*m_ss; a
//                       broadcast dimension has stride 0.  mask_bool: bytes, 0 = blocked;
//                       otherwise values of the compute precision (float, or double for the
//                       float64 path) added to the scores.
// Query head h reads kv head h / (H / Hkv) (csrc/gt_ops_nn.cpp:2432,2471).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gt_philox.h"

struct AttnFwdArgs {
    const void *q;
    const void *k;
    const void *v;
    const void *mask;
    void *o;
    void *lse;  // float (double on the float64 path) or null
    void *o32;  // optional float32 copy of o before rounding (training forward), or null
    int64_t B, H, Hkv, L, S, D, Dv;
    int64_t q_sb, q_sh, q_sl;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t m_sb, m_sh, m_sl, m_ss;
    float scale;
    int causal;
    int mask_bool;
    int out_dtype;  // gt_dtype of o
    // Per-sequence key lengths and query positions (a KV cache; both null for the reference
    // operator): key s of batch b is present when s < kv_len[b], and the causal test is
    // s <= q_pos[b] + l (null: s < S, and q_pos = 0, the reference's top-left alignment).
    const int32_t *kv_len;
    const int32_t *q_pos;
    // RoPE of the queries (all D dims) applied as the prefill kernel loads them (null: none):
    // (cos, sin) of pair i of query row l at rope_q[l * D / 2 + i]; rope_neox: NeoX pairing.
    const void *rope_q;  // float2
    int rope_neox;
    // Dropout of the probabilities (dropout != 0): P.V uses P * multiplier (gt_philox.h), the
    // log-sum-exp stays that of the undropped scores.  Decode kernels never see it.
    int dropout;
    GtDropout drop;
};

// Mask mode of the MFMA kernels: 0 none; 1 bool bytes, 2 additive float (per element, any
// strides); 4 additive float that does not depend on the query row (key padding); 5 / 6 bool /
// float per element with contiguous keys, rows and broadcast strides of whole 4-key groups and
// an aligned base (4-key loads).
inline int attn_mask_mode(const AttnFwdArgs &a) {
    if (!a.mask) return 0;
    if (!a.mask_bool && a.m_sl == 0) return 4;
    const bool vec = a.m_ss == 1 && a.S >= 4 && a.S % 4 == 0 && a.m_sb % 4 == 0 && a.m_sh % 4 == 0 &&
                     a.m_sl % 4 == 0 && (uintptr_t)a.mask % (a.mask_bool ? 4 : 16) == 0;
    if (a.mask_bool) return vec ? 5 : 1;
    return vec ? 6 : 2;
}

__device__ inline int attn_kv_len(const AttnFwdArgs &a, int64_t b) { return a.kv_len ? a.kv_len[b] : (int)a.S; }
__device__ inline int attn_q_pos(const AttnFwdArgs &a, int64_t b) { return a.q_pos ? a.q_pos[b] : 0; }
// Wave priority by progress: 3, 2, 1, 0 for steps 0, 1, 2, 3 (mod 4) of a kernel's step loop.
// Two workgroups resident on one CU share its SIMDs, and among waves of equal priority a SIMD
// issues the older one first, so the first-dispatched workgroup streams ahead (measured 10-15%
// faster) and the other finishes alone at the end of the launch; with this a wave one to three
// steps behind outranks the one ahead.  It changes only the issue order, never a result.
__device__ inline void progress_priority(int step) {
    switch (step & 3) {
        case 0: __builtin_amdgcn_s_setprio(3); break;
        case 1: __builtin_amdgcn_s_setprio(2); break;
        case 2: __builtin_amdgcn_s_setprio(1); break;
        default: __builtin_amdgcn_s_setprio(0); break;
    }
}

// Keys [0, end) are visible to a single query row (L == 1) of batch b.
__device__ inline int attn_decode_end(const AttnFwdArgs &a, int64_t b) {
    const int n = attn_kv_len(a, b);
    return a.causal ? min(n, attn_q_pos(a, b) + 1) : n;
}

struct AttnBwdArgs {
    AttnFwdArgs f;         // q/k/v/mask/o/lse as in the forward (o and lse are inputs here)
    const void *dout;      // (B,H,L,Dv) dense, compute dtype
    int o_f32;             // f.o is float32 (the training forward's unrounded output)
    void *dq;              // (B,H,L,D) dense, float (double on the float64 path)
    void *dk;              // (B,Hkv,S,D) dense
    void *dv;              // (B,Hkv,S,Dv) dense
    void *delta;           // (B,H,L) scratch: rowsum(P * dP)
    // dropout, MFMA kernels: (B,H,L, ceil(S/32)) words, bit j of word [row][w] = decision of key
    // 32w + j; written by the dQ kernel (which draws them), read by the dK/dV kernel
    uint32_t *dbits;
};

// Query heads per decode workgroup: a kv head's gtot query heads (GQA / MQA) run in groups of
// 1, 2, 4, 8 or 16 heads (at most max_tile), the 16 MFMA columns holding one group; more heads
// take several workgroups over the same keys, each re-reading them.
constexpr int kDecodeMaxTile = 16;   // fp16/bf16 streaming kernel (16 heads: P.V on MFMA)
constexpr int kDecodeQ8MaxTile = 8;  // Q8_0 kernels (16 measured slower: half the workgroups)
constexpr int kDecodeF32MaxTile = 8; // float32 kernel (VALU P.V: acc[G][4] per lane)
inline int decode_head_tile(int64_t gtot, int max_tile) {
    const int t = gtot > 8 ? 16 : gtot > 4 ? 8 : gtot > 2 ? 4 : (int)gtot;
    return t < max_tile ? t : max_tile;
}

// Workgroups along blockIdx.y of a decode launch, (sequence, kv head, head group); also the
// number of arrival counters its splits use.
inline int64_t decode_units(int64_t B, int64_t H, int64_t Hkv, int max_tile) {
    const int64_t gtot = H / Hkv, tile = decode_head_tile(gtot, max_tile);
    return B * Hkv * ((gtot + tile - 1) / tile);
}

// Split count of a split-K decode launch over `units` (sequence, kv head, head group) of `steps` key
// steps each on `slots` resident workgroups: the n in 1 .. max_splits with the smallest time in
// key steps, rounds(n) x (steps per split + 1, a workgroup's fixed cost: query load, first
// load latency, epilogue) + n / 32 (each split's share of the merge).  A fixed per-split
// penalty would starve short batches: one sequence of 8 kv heads and 32768 keys needs all 64
// splits (512 workgroups) to cover the GPU.
inline int decode_split_count(int64_t units, int64_t steps, int64_t slots, int64_t max_splits) {
    int best = 1;
    double best_cost = 1e300;
    for (int64_t n = 1; n <= max_splits; ++n) {
        const int64_t rounds = (units * n + slots - 1) / slots;
        const int64_t per = (steps + n - 1) / n;
        const double cost = (double)rounds * (double)(per + 1) + (double)n / 32.0;
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = (int)n;
        }
    }
    return best;
}

// Single-query (L == 1) split-K decode: per-chunk partials, then a merge.
struct DecodeArgs {
    AttnFwdArgs f;
    float *part_o;   // (B*H, nsplit, D) unnormalised chunk outputs
    float *part_ml;  // (B*H, nsplit, 2) chunk max (log2 domain) and sum of exp2
    int nsplit;
    int *counters;   // (decode_units) zeroed arrival counters in uncached memory (part_o / part_ml too):
                     // the last split merges in the kernel; null: a merge launch
};


// Launchers.  `cd` is the compute dtype of q/k/v (GT_F32/GT_F16/GT_BF16/GT_F64).
hipError_t launch_attn_generic_fwd(const AttnFwdArgs &a, int cd, hipStream_t s);
hipError_t launch_attn_generic_bwd(const AttnBwdArgs &a, int cd, hipStream_t s);

bool attn_decode_supported(const AttnFwdArgs &f, int cd);
int attn_decode_splits(const AttnFwdArgs &f, int cd);
int attn_decode_max_tile(int cd);  // query heads per workgroup at most (decode_units' max_tile)
hipError_t launch_attn_decode(const DecodeArgs &a, int cd, hipStream_t s);

bool attn_prefill_supported(const AttnFwdArgs &f, int cd);
// (launch_attn_prefill runs the software-pipelined fp16 head-size-128 kernel where
// attn_prefill_asm_supported holds, the HIP prefill kernel otherwise)
hipError_t launch_attn_prefill(const AttnFwdArgs &a, int cd, hipStream_t s);
bool attn_prefill_asm_supported(const AttnFwdArgs &f, int cd);
bool attn_prefill_f32_split(const AttnFwdArgs &f, int cd);  // float32: the small-grid kernel
hipError_t launch_attn_prefill_asm(const AttnFwdArgs &a, hipStream_t s);

bool attn_decode_q8_supported(const AttnFwdArgs &f, int q_dtype);
int attn_decode_q8_splits(const AttnFwdArgs &f);
hipError_t launch_attn_decode_q8(const DecodeArgs &a, hipStream_t s);
hipError_t launch_attn_decode_merge(const DecodeArgs &a, int out_dtype, hipStream_t s);

// Explicit attention weights from the forward's log-sum-exp: (B,H,L,S), or (B,L,S) averaged
// over the heads, in f.out_dtype.
hipError_t launch_attn_weights(const AttnFwdArgs &f, int cd, void *w, bool average, hipStream_t s);
bool attn_weights_mfma(const AttnFwdArgs &f, int cd);  // the MFMA weights kernels take `f`
// Dropout decisions of `rows` attention rows of S keys as bytes (1 = kept; all 1 when keep_all).
hipError_t launch_dropout_mask(const GtDropout &d, bool keep_all, int64_t rows, int64_t S, uint8_t *out, hipStream_t s);

bool attn_bwd_mfma_supported(const AttnBwdArgs &a, int cd);
bool attn_bwd_f32_split(const AttnBwdArgs &a);  // float32: the small-grid backward kernels
hipError_t launch_attn_bwd_mfma(const AttnBwdArgs &a, int cd, hipStream_t s);
