// Internal declarations of libgt_attn.so: tensor handle, storage, device memory pool, errors,
// and the launchers each .hip translation unit exports to the host-side API code.
//
// The handle carries the same field meanings as the reference's gt_tensor
// (csrc/gt_internal.h:30-70): shape/strides in elements, element offset, dtype code, device,
// shared storage.  The struct layout itself is private; callers only hold pointers.
#pragma once

#include "../../include/gt_attn.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>

// ---- errors (thread-local message, csrc/gt_core.cpp:7-23) ---------------------------------
void gt_set_error(const std::string &msg);
// Records a HIP failure as "<what>: <hip error string>" and returns false.
bool gt_hip_check(hipError_t e, const char *what);

// ---- devices / streams ----------------------------------------------------------------------
// True when HIP device `idx` exists; otherwise sets the error message and returns false.
bool gt_device_ok(int idx);
// The calling thread's current stream (gt_set_stream).
hipStream_t gt_stream();

// ---- storage ----------------------------------------------------------------------------------
enum gt_storage_kind { GT_STORE_HOST = 0, GT_STORE_DEVICE = 1, GT_STORE_EXTERNAL = 2 };

struct gt_storage {
    void *ptr = nullptr;     // first byte (host or device address)
    size_t nbytes = 0;       // bytes reachable from ptr
    size_t capacity = 0;     // bytes actually allocated (pool block size)
    int64_t numel = 0;       // elements reachable (bounds of views)
    int device_type = GT_DEV_CPU;
    int device_index = 0;
    int kind = GT_STORE_HOST;
    uint64_t token = 0;      // external memory: reported by gt_external_released
    hipStream_t stream = nullptr;  // stream the pool may reuse a device block on
    ~gt_storage();
};

struct gt_tensor {
    int ndim = 0;
    int64_t shape[GT_MAX_DIMS] = {};
    int64_t strides[GT_MAX_DIMS] = {};
    int64_t offset = 0;
    int64_t numel = 1;
    int dtype = GT_F32;
    int device_type = GT_DEV_CPU;
    int device_index = 0;
    std::shared_ptr<gt_storage> storage;
};

// ---- dtype helpers ----------------------------------------------------------------------------
size_t gt_elem_bytes(int dtype);  // 0 for unknown and quantized dtypes
inline bool gt_is_quantized(int dtype) { return dtype >= GT_Q_BASE; }
inline bool gt_is_float(int dtype) {
    return dtype == GT_F32 || dtype == GT_F16 || dtype == GT_BF16 || dtype == GT_F64;
}
// Bytes of `numel` elements of `dtype` (Q8_0: numel/32 blocks of 34 bytes).
size_t gt_dtype_nbytes(int dtype, int64_t numel);
const char *gt_dtype_name(int dtype);

inline int64_t gt_numel_of(int ndim, const int64_t *shape) {
    int64_t n = 1;
    for (int i = 0; i < ndim; ++i) n *= shape[i];
    return n;
}
void gt_default_strides(int ndim, const int64_t *shape, int64_t *strides);
bool gt_is_dense(const gt_tensor *t);  // contiguous row-major (size-1 dims ignored)

// New tensor with fresh storage (pool-backed on the device).  Sets the error on failure.
gt_tensor *gt_new_tensor(int ndim, const int64_t *shape, int dtype, int device_type, int device_index);
// Base address of element 0 of `t` (storage ptr + offset * element size).
void *gt_data(const gt_tensor *t);

// Device-resident, element-converted copy helpers used by the op layer.  Each returns a new
// tensor on device `dev` or NULL (error set).
//   gt_to_device_dense: contiguous copy on the device, converted to `dtype` (-1 keeps it).
gt_tensor *gt_to_device_dense(const gt_tensor *t, int dev, int dtype);
// Copies the device tensor `src` into host tensor `dst` (same shape, dense), waiting for it.
bool gt_copy_device_to_host(gt_tensor *dst, const gt_tensor *src);

// `dev_t` itself, or (to_host) a new host tensor with its contents, `dev_t` freed; NULL on error.
gt_tensor *gt_deliver(gt_tensor *dev_t, bool to_host);

// Workspace of the decode kernels' in-kernel split merge on stream `s` of device `dev`, in
// uncached device memory: `n_counters` zeroed arrival counters (the kernels leave them zero),
// then at least `part_bytes` bytes for the partials, 256-byte aligned.  Cached per stream and
// never freed (uncached memory a kernel has read is kept until the process ends); null on failure.
struct gt_decode_ws {
    int *counters;
    void *parts;
};
bool gt_decode_workspace(int dev, hipStream_t s, int64_t n_counters, size_t part_bytes, gt_decode_ws &ws);

// Stream-ordered scratch memory from the pool (freed back to the pool in stream order).
struct gt_scratch {
    std::shared_ptr<gt_storage> st;
    void *ptr() const { return st ? st->ptr : nullptr; }
};
bool gt_scratch_alloc(gt_scratch &s, size_t nbytes, int dev);

// ---- launchers (defined in the .hip files) -------------------------------------------------
struct gt_layout {
    int ndim;
    int64_t shape[GT_MAX_DIMS];
    int64_t strides[GT_MAX_DIMS];
};
// Element-wise copy with conversion between two layouts of the same shape (any strides, any
// supported dtype): dst[dst_layout(i)] = convert(src[src_layout(i)]) for i < numel.
hipError_t gt_launch_convert(const void *src, int src_dtype, const gt_layout &src_layout, void *dst, int dst_dtype,
                             const gt_layout &dst_layout, int64_t numel, hipStream_t stream);
// KV-cache append: rows (b, h, t) of the 4-D src (element strides src_strides) are written at
// row pos[b] + t (pos: device int32 per batch) of the dense (B, Hkv, cap, D) cache of dtype
// dst_dtype (float32/float16/bfloat16, or GT_Q8_0 quantized row by row; D % 32 == 0 then).
// With `rope` (non-null) the rows are rotated on the way in: element d of row (b, h, t) becomes
// RoPE(src row)[d] with the angles of table row b * T + t (positions pos[b] + t), rounded to
// src_dtype first, so the cache holds exactly what gt_rope followed by the append would store.
struct gt_rope_apply {
    const void *table;  // float2 (cos, sin) per (row, pair), from gt_launch_rope_table
    int n_dims;
    int neox;
};
hipError_t gt_launch_kv_append(const void *src, int src_dtype, const int64_t *src_strides, void *dst, int dst_dtype,
                               const int32_t *pos, int64_t B, int64_t Hkv, int64_t T, int64_t D, int64_t cap,
                               const gt_rope_apply *rope, hipStream_t stream);
// KV-cache append of Q8_0 rows: the dense Q8_0 src (B, Hkv, T, D), D % 32 == 0, copied block by
// block (bytes unchanged) to rows pos[b] + t of the Q8_0 cache (B, Hkv, cap, D).
hipError_t gt_launch_kv_append_blocks(const void *src, void *dst, const int32_t *pos, int64_t B, int64_t Hkv,
                                      int64_t T, int64_t D, int64_t cap, hipStream_t stream);
// RoPE angle table: (cos, sin) of pair i < n_dims/2 for `rows` positions, row r at position pos[r],
// or base[r / T] + r % T when base is non-null; float2 per entry, sin negated when backward.
hipError_t gt_launch_rope_table(const int32_t *pos, const int32_t *base, int64_t T, int64_t rows, int n_dims,
                                float theta_scale, float freq_scale, int backward, void *table, hipStream_t stream);
// RoPE rotation of x (B, H, S, D; element strides) into the dense y of the same float dtype, with
// the angles of table row b * table_b_stride + s; mode 0 NORMAL, 2 NEOX.
hipError_t gt_launch_rope(const void *x, int dtype, const int64_t *strides, void *y, const void *table,
                          int64_t table_b_stride, int64_t B, int64_t H, int64_t S, int64_t D, int n_dims, int mode,
                          hipStream_t stream);
// ---- RoPE argument checks (gt_rope_ops.cpp) ----------------------------------------------------
// mode 0/2, even n_dims in [2, head_dim], positive finite freq_base, finite freq_scale; the
// reference's messages prefixed with `who`.
bool gt_rope_check_args(const char *who, int64_t head_dim, int n_dims, int mode, float freq_base, float freq_scale);
// powf(freq_base, -2 / n_dims), as ggml computes it.
float gt_rope_theta_scale(float freq_base, int n_dims);
// Zero fill of `bytes` bytes at p on `stream` (a kernel, not hipMemsetAsync, so that a captured
// stream records no memset node).
hipError_t gt_launch_fill_zero(void *p, int64_t bytes, hipStream_t stream);
// Dense bool bytes -> dense float additive mask (0 where true, -inf where false).
hipError_t gt_launch_bool_to_bias(const void *src, float *dst, int64_t n, hipStream_t stream);
// Head padding for the MFMA kernels: rows of a 4-D (B,H,L,D) tensor (element strides
// strides[0..2], innermost contiguous, 2- or 4-byte elements) into a dense (B,H,L,Dp) buffer with
// zero dims D .. Dp-1; and the first D of each dense Dp-row back into a dense (rows, D) buffer.
hipError_t gt_launch_pad_rows(const void *src, int elem_bytes, const int64_t *strides, int64_t B, int64_t H, int64_t L,
                              int64_t D, void *dst, int64_t Dp, hipStream_t stream);
hipError_t gt_launch_unpad_rows(const void *src, int elem_bytes, int64_t rows, int64_t Dp, void *dst, int64_t D,
                                hipStream_t stream);
// Q8_0 (ggml block_q8_0) quantize `nrows` rows of `row_len` floats (row_len % 32 == 0).
hipError_t gt_launch_q8_0_quantize(const float *src, void *dst, int64_t nblocks, hipStream_t stream);
// Q8_0 dequantize into `dst_dtype` (f32/f16/bf16/f64).
hipError_t gt_launch_q8_0_dequantize(const void *src, void *dst, int dst_dtype, int64_t nblocks, hipStream_t stream);
// Dequantizes nblocks blocks: output block i reads source block i / group_blocks *
// src_group_blocks + i % group_blocks (group_blocks 0: block i).
hipError_t gt_launch_q8_0_dequantize_rows(const void *src, void *dst, int dst_dtype, int64_t nblocks,
                                          int64_t group_blocks, int64_t src_group_blocks, hipStream_t stream);
