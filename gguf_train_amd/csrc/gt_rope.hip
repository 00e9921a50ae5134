// RoPE (rotary position embedding): GGUF_train's gt_rope / gt_rope_backward
// (csrc/gt_ops_nn.cpp:2298-2421), which run ggml_rope_ext / ggml_rope_ext_back with ext_factor 0,
// attn_factor 1 and no frequency factors.  With those arguments the operation is:
//   theta_scale = powf(freq_base, -2 / n_dims)            (computed on the host, C library powf)
//   pair i at position p: theta_0 = (float)p, theta_{i+1} = theta_i * theta_scale (float32, one
//   rounding per step), angle_i = freq_scale * theta_i, (c, s) = (cos, sin)(angle_i); the backward
//   uses -s (the inverse rotation).
//   NORMAL (mode 0) rotates elements (2i, 2i+1), NEOX (mode 2) rotates (i, i + n_dims/2), for
//   i < n_dims/2; elements from n_dims on pass through.  y_lo = x_lo c - x_hi s,
//   y_hi = x_lo s + x_hi c in float32, on inputs converted to float32, rounded to the output type.
//
// Two kernels: the angle table (one (cos, sin) pair per position and pair index, computed once per
// call and shared by every head), then the rotation, which is HBM-bound element work: one thread
// per VEC consecutive elements of a row (16-byte loads and stores for dense rows); a NeoX thread
// also loads its partner group from the other half of the same row, cache lines the neighbouring
// threads of the wave load anyway, so HBM sees each byte once.

#include "gt_internal.h"
#include "gt_rope_math.h"

#include <cmath>

namespace {

struct RopeArgs {
    const void *x;
    int64_t sb, sh, ss, sd;   // element strides of x (B, H, S, D)
    void *y;                  // dense (B, H, S, D) output
    const float2 *table;      // (table row, pair) -> (cos, sin)
    int64_t tb;               // table row of (b, s) = b * tb + s
    int64_t H, S, D;
    int n_dims, half, neox;
    int64_t ngroups;          // B * H * S * D / VEC
};

template <typename T>
__device__ inline float to_f(T v) {
    return (float)v;
}
template <typename T>
__device__ inline T from_f(float v) {
    return (T)v;  // float16 / bfloat16: round to nearest even; float64: exact
}

// (cos, sin) of every (table row, pair): row r is position pos[r], or base[r / T] + r % T when
// base is given (rows appended after what each sequence holds).
__global__ void rope_table_kernel(const int32_t *__restrict__ pos, const int32_t *__restrict__ base, int64_t T,
                                  int64_t rows, int half, float theta_scale, float freq_scale, float sin_sign,
                                  float2 *__restrict__ table) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * half) return;
    const int64_t r = idx / half;
    const int i = (int)(idx - r * half);
    const int32_t p = base ? base[r / T] + (int32_t)(r % T) : pos[r];
    float theta = (float)p;
    for (int j = 0; j < i; ++j) theta *= theta_scale;  // the same chain of float32 products as ggml
    const float angle = freq_scale * theta;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    table[idx] = make_float2(cs, sin_sign * sn);
}

template <typename T, int VEC>
__device__ inline void load_group(const T *row, int d, int64_t sd, float *v) {
    if constexpr (VEC == 1) {
        v[0] = to_f(row[d * sd]);
    } else {
        struct alignas(sizeof(T) * VEC) G {
            T e[VEC];
        };
        const G g = *reinterpret_cast<const G *>(row + d);
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[j] = to_f(g.e[j]);
    }
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256) rope_kernel(RopeArgs a) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= a.ngroups) return;
    const int64_t gpr = a.D / VEC;
    const int64_t row = g / gpr;
    const int d0 = (int)(g - row * gpr) * VEC;
    const int64_t s = row % a.S, bh = row / a.S, h = bh % a.H, b = bh / a.H;
    const T *xr = static_cast<const T *>(a.x) + b * a.sb + h * a.sh + s * a.ss;
    const float2 *tab = a.table + (b * a.tb + s) * a.half;
    float v[VEC], o[VEC];
    load_group<T, VEC>(xr, d0, a.sd, v);
    if (d0 >= a.n_dims) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) o[j] = v[j];
    } else if (!a.neox) {
        if constexpr (VEC == 1) {
            // the pair (d0 & ~1, d0 | 1); n_dims is even, so both are rotated
            float w;
            load_group<T, 1>(xr, d0 ^ 1, a.sd, &w);
            const float2 cs = tab[d0 >> 1];
            o[0] = (d0 & 1) ? rope_rot_hi(w, v[0], cs) : rope_rot_lo(v[0], w, cs);
        } else {
#pragma unroll
            for (int j = 0; j < VEC; j += 2) {
                const float2 cs = tab[(d0 + j) >> 1];
                o[j] = rope_rot_lo(v[j], v[j + 1], cs);
                o[j + 1] = rope_rot_hi(v[j], v[j + 1], cs);
            }
        }
    } else {
        const bool lo = d0 < a.half;
        const int pd = lo ? d0 + a.half : d0 - a.half;
        float w[VEC];
        load_group<T, VEC>(xr, pd, a.sd, w);
        const int i0 = lo ? d0 : pd;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const float2 cs = tab[i0 + j];
            o[j] = lo ? rope_rot_lo(v[j], w[j], cs) : rope_rot_hi(w[j], v[j], cs);
        }
    }
    T *yr = static_cast<T *>(a.y) + row * a.D + d0;
    if constexpr (VEC == 1) {
        yr[0] = from_f<T>(o[0]);
    } else {
        struct alignas(sizeof(T) * VEC) G {
            T e[VEC];
        };
        G out;
#pragma unroll
        for (int j = 0; j < VEC; ++j) out.e[j] = from_f<T>(o[j]);
        *reinterpret_cast<G *>(yr) = out;
    }
}

template <typename T, int VEC>
hipError_t launch_rotation(RopeArgs a, int64_t numel, hipStream_t stream) {
    a.ngroups = numel / VEC;
    const int64_t blocks = (a.ngroups + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((rope_kernel<T, VEC>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// 16-byte groups when every row starts on a group boundary and a group never straddles n_dims
// or (NeoX) the half of the rotated part.
template <typename T>
hipError_t dispatch_rotation(const RopeArgs &a, int64_t numel, hipStream_t stream) {
    constexpr int V = 16 / (int)sizeof(T);
    const bool vec = V > 1 && a.sd == 1 && a.D % V == 0 && a.n_dims % V == 0 && (!a.neox || a.half % V == 0) &&
                     a.sb % V == 0 && a.sh % V == 0 && a.ss % V == 0 && ((uintptr_t)a.x % 16) == 0;
    if constexpr (V > 1) {
        if (vec) return launch_rotation<T, V>(a, numel, stream);
    }
    return launch_rotation<T, 1>(a, numel, stream);
}

}  // namespace

hipError_t gt_launch_rope_table(const int32_t *pos, const int32_t *base, int64_t T, int64_t rows, int n_dims,
                                float theta_scale, float freq_scale, int backward, void *table, hipStream_t stream) {
    const int half = n_dims / 2;
    const int64_t n = rows * half;
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, pos, base, T, rows, half,
                       theta_scale, freq_scale, backward ? -1.0f : 1.0f, (float2 *)table);
    return hipGetLastError();
}

hipError_t gt_launch_rope(const void *x, int dtype, const int64_t *strides, void *y, const void *table,
                          int64_t table_b_stride, int64_t B, int64_t H, int64_t S, int64_t D, int n_dims, int mode,
                          hipStream_t stream) {
    const int64_t numel = B * H * S * D;
    if (numel <= 0) return hipSuccess;
    RopeArgs a{};
    a.x = x;
    a.sb = strides[0];
    a.sh = strides[1];
    a.ss = strides[2];
    a.sd = strides[3];
    a.y = y;
    a.table = (const float2 *)table;
    a.tb = table_b_stride;
    a.H = H;
    a.S = S;
    a.D = D;
    a.n_dims = n_dims;
    a.half = n_dims / 2;
    a.neox = mode == 2;
    switch (dtype) {
        case GT_F32: return dispatch_rotation<float>(a, numel, stream);
        case GT_F16: return dispatch_rotation<_Float16>(a, numel, stream);
        case GT_BF16: return dispatch_rotation<__bf16>(a, numel, stream);
        case GT_F64: return dispatch_rotation<double>(a, numel, stream);
        default: return hipErrorInvalidValue;
    }
}
