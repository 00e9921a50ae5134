// The rotation step of RoPE, shared by the rope kernel (gt_rope.hip) and the RoPE-on-append of
// the KV cache (gt_convert.hip) so that both produce the same bits.  For a pair (lo, hi) and the
// angle's (cos, sin) = (c, s):  y_lo = lo*c - hi*s,  y_hi = lo*s + hi*c  (ggml's rotation,
// csrc/gt_ops_nn.cpp:2388-2391 -> ggml_rope_ext).  Each is one product rounded to float32 and one
// fused multiply-add, written out so that the compiler's contraction choices cannot differ
// between the call sites.  The float32 result is pinned in a register: the reference rounds it to
// float32 and then to the tensor's dtype, and without the pin the compiler may fuse the multiply-add
// with a conversion to float16 (v_fma_mix*_f16), which rounds once and differs in rare halfway cases.
#pragma once

#include <hip/hip_runtime.h>

__device__ inline float rope_rot_lo(float lo, float hi, float2 cs) {
    float r = __fmaf_rn(lo, cs.x, -(hi * cs.y));
    asm volatile("" : "+v"(r));
    return r;
}
__device__ inline float rope_rot_hi(float lo, float hi, float2 cs) {
    float r = __fmaf_rn(hi, cs.x, lo * cs.y);
    asm volatile("" : "+v"(r));
    return r;
}
