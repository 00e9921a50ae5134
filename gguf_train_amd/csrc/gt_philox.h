// Counter-based random numbers for attention dropout.
//
// Philox4x32-10 (J. Salmon, M. Moraes, R. Dror, D. Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC 2011): a 128-bit counter and a 64-bit key map to four 32-bit words through ten
// rounds of two 32x32 -> 64-bit products; the key is bumped by the Weyl constants between
// rounds.  Any element's word is computed on its own, so every kernel that needs the dropout
// decision of an element (the forward, both backward kernels, the explicit weights) recomputes
// it from the element's coordinates instead of storing a mask.
//
// Element (row, s) of an attention matrix with S keys, row = (b*H + h)*L + l, takes word
// s % 4 of the block
//     counter = (n mod 2^32, n / 2^32, offset mod 2^32, offset / 2^32),  n = row*ceil(S/4) + s/4
//     key     = (seed mod 2^32, seed / 2^32)
// and is kept when that word is below `thresh`; a kept probability is multiplied by `scale`.
// Four consecutive keys of a row (aligned to 4) share one block.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

struct GtDropout {
    uint64_t seed;    // Philox key
    uint64_t offset;  // high half of the counter: separates the draws of one seed
    uint32_t thresh;  // keep when the word < thresh: floor((1 - p) * 2^32), 0 for p = 1
    double scale;     // 1 / (1 - p), 0 for p = 1 (float kernels round it to float once)
};

struct GtWord4 {
    uint32_t w[4];
};

__host__ __device__ inline GtWord4 gt_philox4x32_10(uint64_t n, uint64_t offset, uint64_t seed) {
    uint32_t c0 = (uint32_t)n, c1 = (uint32_t)(n >> 32), c2 = (uint32_t)offset, c3 = (uint32_t)(offset >> 32);
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return GtWord4{{c0, c1, c2, c3}};
}

// Block index of keys 4*s4 .. 4*s4 + 3 of `row` (s4 = s / 4).
__host__ __device__ inline uint64_t gt_dropout_block(int64_t row, int64_t S, int64_t s4) {
    return (uint64_t)row * (uint64_t)((S + 3) / 4) + (uint64_t)s4;
}

// Multipliers of keys 4*s4 .. 4*s4 + 3 of `row`: `scale` when kept, 0 when dropped.
template <typename A>
__device__ inline void gt_dropout_mult4(const GtDropout &d, int64_t row, int64_t S, int64_t s4, A scale, A m[4]) {
    const GtWord4 x = gt_philox4x32_10(gt_dropout_block(row, S, s4), d.offset, d.seed);
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = x.w[j] < d.thresh ? scale : (A)0;
}

// Multiplier of element (row, s): `scale` when kept, 0 when dropped.
template <typename A>
__device__ inline A gt_dropout_mult(const GtDropout &d, int64_t row, int64_t S, int64_t s, A scale) {
    const GtWord4 x = gt_philox4x32_10(gt_dropout_block(row, S, s >> 2), d.offset, d.seed);
    const int j = (int)(s & 3);  // selects, not an indexed load: keeps the words in registers
    const uint32_t w = j == 0 ? x.w[0] : j == 1 ? x.w[1] : j == 2 ? x.w[2] : x.w[3];
    return w < d.thresh ? scale : (A)0;
}
