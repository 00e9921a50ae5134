// Software-pipelined fused attention forward for fp16, head size 128 (gfx950).
//
// Replaces the reference's scalar loop (csrc/gt_ops_nn.cpp:2468-2522) for the plain SDPA case:
// fp16 q/k/v, D = Dv = 128, no mask, no dropout, scale > 0, K and V rows of one stride, keys in
// whole pairs of 64-key tiles (causal: L == S, a multiple of 128; otherwise S a multiple of 128,
// at least 256).  Same semantics as the HIP prefill kernel (attn_prefill.hip): top-left causal
// mask, fp32 softmax and accumulation, output rounded to fp16, natural-log log-sum-exp.
//
// The kernel body is one inline-assembly statement written by prefill_asm_gen.py (its header
// describes the schedule); this file supplies the workgroup -> (head, query tile pair) mapping,
// the per-head base addresses and the LDS allocation, and the launcher.  The body uses every
// vector and accumulation register but v0 (the thread index), and s40-s83.

#include "attn_common.h"
#include "gt_internal.h"
#include "prefill_asm_body.inc"

#include <cstring>

namespace {

constexpr int kRows = 128;  // query rows per tile (2 wavefronts x 64)

template <bool CAUSAL>
__global__ __launch_bounds__(128, 1) void prefill_asm_kernel(AttnFwdArgs a, int nq, int npairs, uint32_t cbits) {
    __shared__ __attribute__((aligned(1024))) char lds[65536];
    // Workgroups are dealt to the 8 XCDs round robin (x % 8); when the heads split evenly, XCD x
    // takes heads [x*BH/8, (x+1)*BH/8), so their K/V stay in its own L2 (as attn_prefill.hip).
    const int64_t BH = a.B * a.H;
    int pair;
    int64_t bh;
    if (BH % 8 == 0) {
        const int64_t hpx = BH / 8, i = blockIdx.x / 8;
        pair = (int)(i % npairs);
        bh = (int64_t)(blockIdx.x % 8) * hpx + i / npairs;
    } else {
        pair = (int)(blockIdx.x % npairs);
        bh = (int64_t)blockIdx.x / npairs;
    }
    const int64_t b = bh / a.H, h = bh % a.H, hk = h / (a.H / a.Hkv);
    const uint32_t qa = (uint32_t)(nq - 1 - pair), qb = (uint32_t)pair;
    const uint32_t np = qa == qb ? 1u : 2u;
    const uint64_t q = (uint64_t)((const _Float16 *)a.q + b * a.q_sb + h * a.q_sh);
    const uint64_t k = (uint64_t)((const _Float16 *)a.k + b * a.k_sb + hk * a.k_sh);
    const uint64_t v = (uint64_t)((const _Float16 *)a.v + b * a.v_sb + hk * a.v_sh);
    const uint64_t o = (uint64_t)((_Float16 *)a.o + bh * a.L * 128);
    const uint64_t lse = a.lse ? (uint64_t)((float *)a.lse + bh * a.L) : 0;
    const uint32_t qsl = (uint32_t)(a.q_sl * 2), kvrow = (uint32_t)(a.k_ss * 2);
    const uint32_t L = (uint32_t)a.L, ntk = (uint32_t)(a.S / 64);
    const uint32_t ldsaddr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
    uint32_t tid = threadIdx.x;
    if constexpr (CAUSAL) {
        asm volatile(GT_PREFILL_ASM_CAUSAL
                     : [tid] "+v"(tid)
                     : [q] "s"(q), [k] "s"(k), [v] "s"(v), [o] "s"(o), [lse] "s"(lse),
                       [qsl] "s"(qsl), [kvrow] "s"(kvrow), [L] "s"(L), [ntk] "s"(ntk), [c] "s"(cbits),
                       [qa] "s"(qa), [qb] "s"(qb), [np] "s"(np), [lds] "s"(ldsaddr)
                     : GT_PREFILL_ASM_CLOBBERS);
    } else {
        asm volatile(GT_PREFILL_ASM_FULL
                     : [tid] "+v"(tid)
                     : [q] "s"(q), [k] "s"(k), [v] "s"(v), [o] "s"(o), [lse] "s"(lse),
                       [qsl] "s"(qsl), [kvrow] "s"(kvrow), [L] "s"(L), [ntk] "s"(ntk), [c] "s"(cbits),
                       [qa] "s"(qa), [qb] "s"(qb), [np] "s"(np), [lds] "s"(ldsaddr)
                     : GT_PREFILL_ASM_CLOBBERS);
    }
}

// Switched off, with no way to enable it: the first GPU run of this kernel (causal, L = S = 128)
// did not finish, while every path of the same instruction stream runs to completion with
// correct results in a functional model of the documented instruction semantics (alignment, LDS
// bounds, waits and barriers included).  Until the cause is known the HIP prefill kernel serves
// every call; the kernel stays compiled so that the generator's output is built and checked.
bool asm_enabled() { return false; }

}  // namespace

bool attn_prefill_asm_supported(const AttnFwdArgs &f, int cd) {
    if (!asm_enabled()) return false;
    if (cd != GT_F16 || f.out_dtype != GT_F16 || f.D != 128 || f.Dv != 128) return false;
    if (f.mask || f.dropout || f.rope_q || f.o32 || f.kv_len || f.q_pos) return false;
    if (!(f.scale > 0.0f) || f.L < 1) return false;
    if (f.causal) {
        if (f.L != f.S || f.L % kRows != 0) return false;
    } else if (f.S % 128 != 0 || f.S < 256) {
        return false;
    }
    if (f.k_ss != f.v_ss) return false;  // one set of tile-load offsets serves K and V
    const int64_t strides[] = {f.q_sb, f.q_sh, f.q_sl, f.k_sb, f.k_sh, f.k_ss, f.v_sb, f.v_sh};
    for (int64_t st : strides) if (st % 8 != 0 || st < 0) return false;
    for (const void *p : {(const void *)f.q, (const void *)f.k, (const void *)f.v, (const void *)f.o})
        if ((uintptr_t)p % 16 != 0) return false;
    // 32-bit byte offsets from the per-head bases: q rows, K/V rows, o rows, lse
    if ((f.L - 1) * f.q_sl * 2 + 256 > 0xffffffffLL) return false;
    if ((f.S - 1) * f.k_ss * 2 + 256 > 0xffffffffLL) return false;
    if (f.L * 256 > 0xffffffffLL) return false;
    return (f.B * f.H) * ((f.L + kRows - 1) / kRows + 1) / 2 <= 0x7fffffffLL;
}

hipError_t launch_attn_prefill_asm(const AttnFwdArgs &a, hipStream_t s) {
    const int nq = (int)((a.L + kRows - 1) / kRows);
    const int npairs = (nq + 1) / 2;  // query tiles p and nq-1-p share a workgroup
    const int64_t grid = (int64_t)npairs * a.B * a.H;
    if (grid <= 0) return hipSuccess;
    // raw score -> log2 domain, as the HIP kernel's c (computed here: the kernel body takes it
    // in a scalar register)
    const float cf = a.scale * 1.4426950408889634f;
    uint32_t cbits;
    std::memcpy(&cbits, &cf, 4);
    if (a.causal)
        hipLaunchKernelGGL((prefill_asm_kernel<true>), dim3((unsigned)grid), dim3(128), 0, s, a, nq, npairs, cbits);
    else
        hipLaunchKernelGGL((prefill_asm_kernel<false>), dim3((unsigned)grid), dim3(128), 0, s, a, nq, npairs, cbits);
    return hipGetLastError();
}
