// The rotation step of RoPE, shared by the rope kernel (gt_rope.hip) and the RoPE-on-append of
// the KV cache (gt_convert.hip) so that both produce the same bits.  For a pair (lo, hi) and the
// angle's (cos, sin) = (c, s):  y_lo = lo*c - hi*s,  y_hi = lo*s + hi*c  (ggml's rotation,
// csrc/gt_ops_nn.cpp:2388-2391 -> ggml_rope_ext).  Each is one product rounded to float32 and one
// fused multiply-add, written out so that the compiler's contraction choices cannot differ
// between the two call sites.
#pragma once

#include <hip/hip_runtime.h>

__device__ inline float rope_rot_lo(float lo, float hi, float2 cs) { return __fmaf_rn(lo, cs.x, -(hi * cs.y)); }
__device__ inline float rope_rot_hi(float lo, float hi, float2 cs) { return __fmaf_rn(hi, cs.x, lo * cs.y); }
