// Split-K finish for the single-query (decode) kernels, done inside the split kernel instead of
// a second launch: every workgroup of a (sequence, kv head) writes its partial (max, sum,
// unnormalised O) rows, then counts itself in; the last one to arrive merges the partials of
// that kv head's G query rows and resets the counter to zero for the next launch.
//
// The partials and the counters live in uncached device memory (a persistent per-stream
// workspace), which every XCD reads and writes at the memory itself: no L2 write-back or
// invalidation is needed, only the order of each workgroup's own accesses.  A workgroup waits
// for its partial stores to complete (vmcnt(0)) before it counts itself in, and the counters are
// relaxed device-scope atomics.  Launches on one stream run one after another, so they never
// share a workspace while running.
#pragma once

#include "attn_common.h"

#include <hip/hip_runtime.h>

namespace gtdecode {

template <typename TO>
__device__ inline void store_out(void *o, int64_t i, float v) {
    if constexpr (sizeof(TO) == 4) ((float *)o)[i] = v;
    else ((TO *)o)[i] = (TO)v;  // float16 / bfloat16: round to nearest even
}

__device__ inline float wmax(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ inline float wsum(float v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Merges the nsplit partials of output rows row0 .. row0 + nrows - 1 (one wavefront per row).
// MEMORY INVARIANT: part_o / part_ml are written by other workgroups of this launch, possibly on
// other XCDs, and read here with plain loads and no acquire fence.  That is correct only because
// they live in uncached device memory (hipDeviceMallocUncached, gt_decode_workspace): no L2
// holds a stale or dirty copy.  In ordinary (cached) memory these loads could miss stores still
// sitting in another XCD's L2; such buffers must use the two-launch merge (counters == null).
// Every load of a row (the splits' (max, sum) pairs and their first SPW * U output pieces) is
// issued before any is used: each uncached load is a round trip to the memory, and this runs at
// the tail of the kernel.  The sums run in the order of the merge kernel (decode_merge_kernel),
// so both merges give the same bits.
template <typename TO, int D>
__device__ inline void merge_rows(const DecodeArgs &a, int64_t row0, int nrows) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int LPS = D / 4;     // lanes per partial row
    constexpr int SPW = 64 / LPS;  // partial rows per wave load
    constexpr int U = 8;           // partial rows per lane and batch
    const AttnFwdArgs &f = a.f;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int ns = a.nsplit;  // <= 64 (decode_split_count)
    const int sub = lane % LPS, sp = lane / LPS;
    for (int r = w; r < nrows; r += nw) {
        const int64_t row = row0 + r;
        const float *ml = a.part_ml + row * ns * 2;
        const float *po = a.part_o + row * ns * D + 4 * sub;
        // all loads first: split `lane`'s (max, sum) and the first batch of output pieces
        const float mi = lane < ns ? ml[2 * lane] : -INFINITY;
        const float li = lane < ns ? ml[2 * lane + 1] : 0.0f;
        f32x4 x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = *(const f32x4 *)(po + (int64_t)min(SPW * u + sp, ns - 1) * D);
        const float M = wmax(mi);
        const float L = wsum(mi == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mi - M) * li);
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i0 = 0; i0 < ns; i0 += SPW * U) {
            if (i0 > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u) x[u] = *(const f32x4 *)(po + (int64_t)min(i0 + SPW * u + sp, ns - 1) * D);
            }
            float wgt[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + SPW * u + sp;
                const float m = __shfl(mi, min(i, ns - 1), 64);  // split i's max sits in lane i
                wgt[u] = (i >= ns || m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M);
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
            for (int j = 0; j < 4; ++j) store_out<TO>(f.o, row * D + 4 * sub + j, acc[j] * inv);
        }
        if (f.lse && lane == 0) ((float *)f.lse)[row] = L > 0.0f ? (M + log2f(L)) * 0.6931471805599453f : INFINITY;
    }
}

// Called by every thread of a split workgroup after its partial stores (nsplit > 1, counters
// set).  `bk` is the (sequence, kv head) index, rows row0 .. row0 + nrows - 1 its query rows.
// MEMORY INVARIANT (see merge_rows): counters, part_o and part_ml are uncached device memory.
// The order "partial stores complete, then the counter increment" is given by vmcnt(0) plus the
// barrier, not by a release fence; with uncached memory a completed store is in memory and
// visible to every XCD.  The relaxed agent-scope atomics are then enough for the count.
template <typename TO, int D>
__device__ inline void finish_split(const DecodeArgs &a, int64_t bk, int64_t row0, int nrows) {
    __shared__ int s_last;
    // this thread's partial stores have completed (reached the uncached memory)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&a.counters[bk], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 a.nsplit - 1;
    __syncthreads();
    if (!s_last) return;
    merge_rows<TO, D>(a, row0, nrows);
    if (threadIdx.x == 0) __hip_atomic_store(&a.counters[bk], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace gtdecode
