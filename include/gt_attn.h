/*
 * gt_attn.h - C ABI of libgt_attn.so, the MI355X (gfx950) attention library.
 *
 * The entry points below carry the names, argument meanings, return conventions and error
 * behaviour of GGUF_train's native ABI (csrc/gguf_train.h), so the reference's ctypes loader
 * (gguf_train/_C.py) can bind them unchanged.  Every declaration cites the reference
 * declaration it replaces; entry points the reference does not have say so.
 *
 * Conventions shared with the reference:
 *   - a tensor is an opaque `gt_tensor *` handle: shape and strides counted in elements, an
 *     element offset, a dtype code and a device (csrc/gt_internal.h:30-70);
 *   - a function returning `gt_tensor *` returns a NEW handle owned by the caller (release it
 *     with gt_tensor_free) or NULL on failure; a function returning `int` returns 0 on success;
 *   - on failure the message is stored per thread and read with gt_last_error()
 *     (csrc/gt_core.cpp:7-23); nothing throws or aborts across this boundary.
 *
 * Devices: GT_DEV_CPU tensors live in host memory, GT_DEV_CUDA tensors in HIP device memory
 * (the reference files HIP/ROCm GPUs under GT_DEV_CUDA, csrc/gt_core.cpp:86-87).  All compute
 * runs on the GPU: host inputs are copied to the device and host outputs copied back, the
 * reverse of the reference's device->host staging (csrc/gt_core.cpp:314-329).  There is no
 * CPU compute path: without a HIP device every compute entry point fails with a message.
 *
 * Ordering: work is enqueued on the calling thread's current stream (gt_set_stream; the null
 * stream by default).  Device results may still be in flight when a call returns; every call
 * that hands bytes to the host (gt_tensor_copy_to_host, host outputs) waits for them.
 */
#ifndef GT_ATTN_H
#define GT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GT_API __attribute__((visibility("default")))

/* csrc/gguf_train.h:20 */
#define GT_MAX_DIMS 12

/* dtype codes: csrc/gguf_train.h:22-36.  Quantized types are GT_Q_BASE + ggml type id. */
enum gt_dtype {
    GT_F32 = 0,
    GT_F16 = 1,
    GT_BF16 = 2,
    GT_F64 = 3,
    GT_I8 = 4,
    GT_U8 = 5,
    GT_I16 = 6,
    GT_I32 = 7,
    GT_I64 = 8,
    GT_BOOL = 9,
    GT_C64 = 10,
    GT_C128 = 11,
    GT_Q_BASE = 100
};
/* GGUF Q8_0: blocks of 32 values, {fp16 d, int8 qs[32]} = 34 bytes (ggml type 8;
 * gguf_train/_dtype.py:85 names it 108). */
#define GT_Q8_0 (GT_Q_BASE + 8)

/* device codes: csrc/gguf_train.h:38-44 */
enum gt_device_type {
    GT_DEV_CPU = 0,
    GT_DEV_CUDA = 1,
    GT_DEV_MPS = 2,
    GT_DEV_VULKAN = 3,
    GT_DEV_META = 4
};

typedef struct gt_tensor gt_tensor;

/* ---- runtime / errors ------------------------------------------------------------------ */

/* csrc/gguf_train.h:170.  Idempotent; called by every entry point that needs it. */
GT_API void gt_init(void);
/* csrc/gguf_train.h:175.  Number of HIP devices for GT_DEV_CUDA, 1 for GT_DEV_CPU. */
GT_API int gt_device_count(int device_type);
/* csrc/gguf_train.h:176 */
GT_API void gt_device_name(int device_type, int idx, char *buf, int buf_len);
/* csrc/gguf_train.h:177 */
GT_API void gt_device_memory(int device_type, int idx, size_t *free_bytes, size_t *total_bytes);
/* csrc/gguf_train.h:178.  Waits for all work this library enqueued on the device. */
GT_API void gt_synchronize(int device_type, int idx);
/* csrc/gguf_train.h:182-185 */
GT_API const char *gt_last_error(void);
GT_API void gt_clear_error(void);
GT_API void gt_set_last_error(const char *msg);

/* No counterpart in the reference (its calls are synchronous and stream-less).  Sets the HIP
 * stream (a hipStream_t, NULL = the null stream) that this thread's calls enqueue on, so a
 * host that keeps its own current stream (e.g. PyTorch) stays ordered with this library. */
GT_API void gt_set_stream(void *stream);
GT_API void *gt_get_stream(void);

/* No counterpart in the reference: the SHA-256 (hex) of the sources the library was built from
 * (csrc/ and this header), so a loader can refuse a library that does not match its tree. */
GT_API const char *gt_source_hash(void);

/* No counterpart in the reference (a diagnostic): the kernels the last attention call made on
 * this thread launched, "; "-separated, e.g. "decode q8_0 D=128 heads_per_group=4 splits=4
 * units=128 merge=in-kernel" or "prefill f16 D=128 B=4 H=32 L=2048 S=2048".  Valid until this
 * thread's next attention call; "" before the first. */
GT_API const char *gt_last_launch(void);

/* ---- tensor lifecycle & metadata: csrc/gguf_train.h:188-227 ----------------------------- */

GT_API gt_tensor *gt_tensor_empty(int ndim, const int64_t *shape, int dtype, int device_type, int device_index);
GT_API gt_tensor *gt_tensor_from_data(int ndim, const int64_t *shape, int dtype, int device_type, int device_index,
                                      const void *data, size_t nbytes);
/* csrc/gguf_train.h:191-198: host memory owned by the caller, nothing copied; `token` is
 * reported by gt_external_released() once the last handle on that memory is gone. */
GT_API gt_tensor *gt_tensor_from_external(int ndim, const int64_t *shape, const int64_t *strides, int dtype,
                                          void *data, uint64_t token);
GT_API int64_t gt_external_released(uint64_t *tokens, int64_t capacity);
/* No counterpart in the reference: device memory owned by the caller (e.g. a PyTorch CUDA
 * tensor), borrowed without a copy.  The caller keeps the memory alive while any handle on
 * it exists; `token` (non-zero) is reported by gt_external_released() like host memory. */
GT_API gt_tensor *gt_tensor_from_device_ptr(int ndim, const int64_t *shape, const int64_t *strides, int dtype,
                                            int device_index, void *data, uint64_t token);
GT_API gt_tensor *gt_tensor_clone(const gt_tensor *t);
GT_API gt_tensor *gt_tensor_view(const gt_tensor *t, int ndim, const int64_t *shape, const int64_t *strides,
                                 int64_t offset);
GT_API gt_tensor *gt_tensor_contiguous(const gt_tensor *t);
GT_API gt_tensor *gt_tensor_to_dtype(const gt_tensor *t, int dtype);
GT_API gt_tensor *gt_tensor_to_device(const gt_tensor *t, int device_type, int device_index);
GT_API void gt_tensor_free(gt_tensor *t);

GT_API int gt_tensor_ndim(const gt_tensor *t);
GT_API void gt_tensor_shape(const gt_tensor *t, int64_t *out);
GT_API void gt_tensor_strides(const gt_tensor *t, int64_t *out);
GT_API int64_t gt_tensor_offset(const gt_tensor *t);
GT_API int64_t gt_tensor_numel(const gt_tensor *t);
GT_API int gt_tensor_dtype(const gt_tensor *t);
GT_API int gt_tensor_device_type(const gt_tensor *t);
GT_API int gt_tensor_device_index(const gt_tensor *t);
GT_API int gt_tensor_is_contiguous(const gt_tensor *t);
GT_API uint64_t gt_tensor_data_ptr(const gt_tensor *t);
GT_API size_t gt_tensor_storage_nbytes(const gt_tensor *t);
GT_API size_t gt_tensor_nbytes(const gt_tensor *t);
GT_API size_t gt_tensor_elem_size(int dtype);

/* csrc/gguf_train.h:222-224: dense row-major copies; they wait for the device. */
GT_API int gt_tensor_copy_to_host(const gt_tensor *t, void *dst, size_t dst_bytes);
GT_API int gt_tensor_copy_from_host(gt_tensor *t, const void *src, size_t src_bytes);
GT_API int gt_tensor_copy_inplace(gt_tensor *dst, const gt_tensor *src);

/* No counterpart in the reference: a DLPack (DLManagedTensor, unversioned ABI) describing the
 * tensor's memory without a copy; it holds a reference on the storage until its deleter runs.
 * Returns NULL on failure.  Lets hosts such as PyTorch adopt results zero-copy. */
GT_API void *gt_tensor_to_dlpack(const gt_tensor *t);

/* ---- attention ------------------------------------------------------------------------ */

/* csrc/gguf_train.h:311 (implementation csrc/gt_ops_nn.cpp:2423-2525).
 * q (B,H,L,D), k (B,Hkv,S,D), v (B,Hkv,S,Dv); H % Hkv == 0, head h reads kv head h/(H/Hkv).
 * mask: NULL, (L,S) or 4-D, every dim 1 or full; bool = may attend, other dtypes are added.
 * scale <= 0 means 1/sqrt(D).  is_causal masks s > l (top-left aligned).  A row with nothing
 * to attend to yields 0.  Output (B,H,L,Dv) contiguous, dtype of q, device of q.
 * k and v may also be GT_Q8_0 (contiguous), read as their dequantized values. */
GT_API gt_tensor *gt_flash_attention(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                     const gt_tensor *mask, float scale, int is_causal);

/* No counterpart in the reference: gt_flash_attention that also returns the per-row
 * log-sum-exp of the scaled, masked scores (B,H,L) float32 (+inf for a row with nothing to
 * attend to), the residual the backward needs.  Out-params follow gt_layer_norm_backward's
 * convention (csrc/gguf_train.h:284).  Returns 0 on success. */
GT_API int gt_flash_attention_lse(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v, const gt_tensor *mask,
                                  float scale, int is_causal, gt_tensor **out, gt_tensor **lse);

/* No counterpart in the reference: the training forward.  As gt_flash_attention_lse, plus
 * out32 = the float32 output before it is rounded to float16/bfloat16 (for float32/float64
 * inputs out32 is NULL and `out` itself is exact).  Pass out32 as the backward's `out`: its
 * rowsum(dO * O) is then exact without recomputing anything.  Returns 0 on success. */
GT_API int gt_flash_attention_train(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v, const gt_tensor *mask,
                                    float scale, int is_causal, gt_tensor **out, gt_tensor **lse, gt_tensor **out32);

/* Replaces the Python composition FlashAttentionFn.backward (gguf_train/_functions.py:1933-1965)
 * with a native recompute-based backward.  dq (B,H,L,D), dk (B,Hkv,S,D), dv (B,Hkv,S,Dv) are
 * float32 for float16/bfloat16/float32 inputs and float64 for float64 inputs; gradients of
 * a GQA group are summed into its kv head.  `out` (the forward's output) and `lse` may be NULL:
 * they are recomputed; for float16/bfloat16 inputs an `out` that is not the float32 copy from
 * gt_flash_attention_train also makes the backward recompute that copy (one forward pass), so
 * the result does not depend on the output's rounding.  Returns 0 on success. */
GT_API int gt_flash_attention_backward(const gt_tensor *grad_out, const gt_tensor *q, const gt_tensor *k,
                                       const gt_tensor *v, const gt_tensor *mask, const gt_tensor *out,
                                       const gt_tensor *lse, float scale, int is_causal, gt_tensor **dq,
                                       gt_tensor **dk, gt_tensor **dv);
/* (out may be NULL together with lse: the forward is then recomputed.  A float32 out, from
 * gt_flash_attention_train, is used as is.) */

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): gt_flash_attention
 * written into `out`, a dense (B,H,L,Dv) device tensor of q's dtype that the caller owns, with no
 * device allocation and no hipMalloc / hipFree.  q, k, v, mask and out must be on the same HIP
 * device; q, k, v of one dtype with a contiguous innermost dimension (or q float16 with q8_0
 * k/v and L = 1); mask NULL, bool, or float32 (float64 for float64 inputs), read in place.
 * Inputs that would need staging or conversion are refused with an error.  The split-K
 * partials of single-query calls go to a fixed 16 MiB device array per GPU (held until the
 * process ends); a call whose partials (B*H*splits*(D+2)*4 bytes) exceed it is refused.  Calls
 * that overlap in time on one GPU share that array and race: serialise them.  A call that would
 * write the array while the previous such call, made on another stream, has not finished is
 * refused with an error (not checked for streams under graph capture).  Asynchronous on the
 * current stream (gt_set_stream).  Returns 0 on success, -1 with gt_last_error() set. */
GT_API int gt_flash_attention_noalloc(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                      const gt_tensor *mask, float scale, int is_causal, gt_tensor *out);

/* Replaces the explicit weights of MultiheadAttention(need_weights=True), which the reference
 * computes with ggml ops (gguf_train/nn/modules/transformer.py:153-166): softmax(q.k^T*scale +
 * mask) with the causal mask, recomputed from `lse`, the (B,H,L) log-sum-exp of the forward of
 * the same q, k, mask, scale, is_causal (gt_flash_attention_lse).  Returns (B,H,L,S), or
 * (B,L,S) averaged over the heads when average_heads != 0, dtype and device of q.  Positions
 * that are causally or mask-blocked weigh 0; a row with nothing to attend to is all zeros. */
GT_API gt_tensor *gt_attention_weights(const gt_tensor *q, const gt_tensor *k, const gt_tensor *mask,
                                       const gt_tensor *lse, float scale, int is_causal, int average_heads);

/* ---- dropout ---------------------------------------------------------------------------- */

/* Replaces the reference's dropout composition in scaled_dot_product_attention
 * (gguf_train/nn/functional.py:750-767: softmax(q.k^T*scale + masks), then probs * (rand < 1-p)
 * / (1-p), then .matmul(v)) with the fused training forward: as gt_flash_attention_train, with
 * the probabilities multiplied by 1/(1-p) where kept and by 0 where dropped before P.V; lse is
 * that of the undropped scores.  The decisions come from Philox4x32-10 keyed by `seed`, counter
 * (element block, `offset`) (gt_philox.h: element (b,h,l,s) uses word s%4 of block
 * ((b*H + h)*L + l)*ceil(S/4) + s/4 and is kept when the word < floor((1-p)*2^32)), not from the
 * reference's sequential mt19937_64 draws.  0 <= dropout_p <= 1 (0: no dropout, 1: all dropped).
 * The causal mask and bool masks block with -inf where the reference adds -1e9: identical
 * except for a row with nothing to attend to, which yields 0 here.  Returns 0 on success. */
GT_API int gt_flash_attention_dropout(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                      const gt_tensor *mask, float scale, int is_causal, double dropout_p,
                                      uint64_t seed, uint64_t offset, gt_tensor **out, gt_tensor **lse,
                                      gt_tensor **out32);

/* The backward of gt_flash_attention_dropout with the same (dropout_p, seed, offset): the
 * gradients of the reference's composition under the same dropout decisions, as
 * gt_flash_attention_backward otherwise (out / lse may be NULL: recomputed). */
GT_API int gt_flash_attention_dropout_backward(const gt_tensor *grad_out, const gt_tensor *q, const gt_tensor *k,
                                               const gt_tensor *v, const gt_tensor *mask, const gt_tensor *out,
                                               const gt_tensor *lse, float scale, int is_causal, double dropout_p,
                                               uint64_t seed, uint64_t offset, gt_tensor **dq, gt_tensor **dk,
                                               gt_tensor **dv);

/* Replaces MultiheadAttention's dropout on its explicit weights
 * (gguf_train/nn/modules/transformer.py:162-163): gt_attention_weights multiplied by the dropout
 * multipliers of the same (dropout_p, seed, offset) as gt_flash_attention_dropout, i.e. the
 * weights that forward multiplied V by (averaged over the heads after the dropout). */
GT_API gt_tensor *gt_attention_weights_dropout(const gt_tensor *q, const gt_tensor *k, const gt_tensor *mask,
                                               const gt_tensor *lse, float scale, int is_causal, int average_heads,
                                               double dropout_p, uint64_t seed, uint64_t offset);

/* No counterpart in the reference: the dropout decisions of (dropout_p, seed, offset) for a
 * (B,H,L,S) attention, as a bool tensor on HIP device `device_index` (1 = kept, scaled by
 * 1/(1-p)).  What the dropout kernels use, element for element. */
GT_API gt_tensor *gt_attention_dropout_mask(int64_t B, int64_t H, int64_t L, int64_t S, double dropout_p,
                                            uint64_t seed, uint64_t offset, int device_index);

/* ---- RoPE ------------------------------------------------------------------------------ */

/* csrc/gguf_train.h:309-310 (implementation csrc/gt_ops_nn.cpp:2298-2421, ggml_rope_ext /
 * ggml_rope_ext_back with ext_factor 0, attn_factor 1).  x (batch, heads, seq_len, head_dim) or
 * (heads, seq_len, head_dim), any float dtype and strides; pos 1-D with at least seq_len
 * positions (the first seq_len are used), any integer or float dtype, read as int32.  mode 0
 * (NORMAL: pairs (2i, 2i+1)) or 2 (NeoX: pairs (i, i + n_dims/2)); n_dims even in
 * [2, head_dim]; elements from n_dims on pass through.  Angle of pair i at position p:
 * freq_scale * p * theta_scale^i in float32 (theta_scale = powf(freq_base, -2/n_dims), the
 * power taken by repeated float32 products), rotation in float32, result rounded to x's dtype.
 * The backward rotates by the negated angle.  n_ctx_orig is accepted and unused (YaRN only).
 * Result: a new dense tensor of x's shape, dtype and device; NULL with the reference's message
 * on bad arguments. */
GT_API gt_tensor *gt_rope(const gt_tensor *x, const gt_tensor *pos, int n_dims, int mode, int n_ctx_orig,
                          float freq_base, float freq_scale);
GT_API gt_tensor *gt_rope_backward(const gt_tensor *grad_out, const gt_tensor *pos, int n_dims, int mode,
                                   int n_ctx_orig, float freq_base, float freq_scale);

/* No counterpart in the reference (there: gt_rope of q and of k, then gt_flash_attention, the
 * composition of csrc/gt_ops_nn.cpp:2298-2525): attention of gt_rope(q, pos) and gt_rope(k, pos)
 * (q rows at the first L positions, k rows at the first S), gt_flash_attention's other arguments
 * and semantics, gt_rope's checks and arithmetic; pos needs max(L, S) positions.  The keys are
 * rotated in one pass; for float16/bfloat16 q, k, v of one dtype with n_dims = D (64 or 128),
 * L > 1 and no mask or a key-padding mask, the prefill kernel rotates each query row as it loads
 * it (the same bits as gt_rope).  Output as gt_flash_attention. */
GT_API gt_tensor *gt_flash_attention_rope(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                          const gt_tensor *mask, float scale, int is_causal, const gt_tensor *pos,
                                          int n_dims, int mode, float freq_base, float freq_scale);

/* ---- GGUF Q8_0 ------------------------------------------------------------------------ */

/* csrc/gguf_train.h:381 (gt_tensor_to_dtype, csrc/gt_core.cpp:784-847): quantizes rows of
 * last-dim length (one flat row when that is not a multiple of 32).  Only GT_Q8_0
 * (ggml_type_id 8) is supported. */
GT_API gt_tensor *gt_quantize(const gt_tensor *t, int ggml_type_id);
/* csrc/gguf_train.h:382: y = float(qs[j]) * float(d), then converted to out_dtype. */
GT_API gt_tensor *gt_dequantize(const gt_tensor *t, int out_dtype);

/* ---- GGUF files ----------------------------------------------------------------------- */

/* csrc/gguf_train.h:363-379 (csrc/gt_ops_extra.cpp:1811-1990), read side.  The reader parses the
 * file itself (no ggml); a file ggml would refuse fails with "Failed to open GGUF file: <why>".
 * Tensors come back with the reference's dtype and shape rules, including the recorded
 * "gguf_train.shape.<name>" / "gguf_train.dtype.<name>" keys.  Stored types: f32, f16, bf16,
 * f64, i8, i16, i32, i64 and q8_0; other quantized types and complex tensors are refused by
 * gt_gguf_get_tensor with a message naming the tensor.  The file stays open (and must not
 * change) until gt_gguf_close; tensor bytes are read when a tensor is asked for. */
typedef struct gt_gguf_file gt_gguf_file;
GT_API gt_gguf_file *gt_gguf_open(const char *path);
GT_API void gt_gguf_close(gt_gguf_file *f);
GT_API int64_t gt_gguf_n_tensors(const gt_gguf_file *f);
GT_API const char *gt_gguf_tensor_name(const gt_gguf_file *f, int64_t idx);
/* A new host tensor; dequantize_f32 turns a q8_0 tensor into float32. */
GT_API gt_tensor *gt_gguf_get_tensor(const gt_gguf_file *f, const char *name, int dequantize_f32);
/* No counterpart in the reference ABI (there, gt_gguf_get_tensor then gt_tensor_to_device): the
 * same tensor streamed from the file into memory of HIP device `device_index` through pinned
 * staging, on the calling thread's stream, complete on return.  A q8_0 tensor stays in its
 * 34-byte blocks (ready for gt_flash_attention as k / v) unless dequantize_f32 asks for float32,
 * which is done on the device. */
GT_API gt_tensor *gt_gguf_get_tensor_device(const gt_gguf_file *f, const char *name, int dequantize_f32,
                                            int device_index);
GT_API int64_t gt_gguf_n_kv(const gt_gguf_file *f);
GT_API const char *gt_gguf_kv_key(const gt_gguf_file *f, int64_t idx);
/* A gguf_type (0 u8 .. 12 f64; 8 string, 9 array), -1 for a bad index. */
GT_API int gt_gguf_kv_type(const gt_gguf_file *f, int64_t idx);
/* The value as text; returns its full length (as snprintf does), so a result >= buf_len means it
 * was cut short.  A null buffer asks for the length. */
GT_API int gt_gguf_kv_val_str(const gt_gguf_file *f, int64_t idx, char *buf, int buf_len);
/* Arrays: element gguf_type (-1 when the value is not an array), element count, packed
 * elements (null for string arrays; bools one byte each), and the i-th string of a string array. */
GT_API int gt_gguf_kv_arr_type(const gt_gguf_file *f, int64_t idx);
GT_API int64_t gt_gguf_kv_arr_n(const gt_gguf_file *f, int64_t idx);
GT_API const void *gt_gguf_kv_arr_data(const gt_gguf_file *f, int64_t idx);
GT_API const char *gt_gguf_kv_arr_str(const gt_gguf_file *f, int64_t idx, int64_t i);

/* ---- KV cache ------------------------------------------------------------------------- */

/* No counterpart in the reference ABI: the reference's decode cache is llama.cpp's, reached
 * through LlamaContext (gt_llama_forward_logits, csrc/llama_bridge.cpp:245-296; clear_kv,
 * gguf_train/llama/__init__.py:174-190).  This is the same behaviour for attention on the
 * device: a cache of `batch` sequences with n_head_kv heads of head_dim values and room for
 * `capacity` tokens each, stored as GT_F32, GT_F16, GT_BF16 or GT_Q8_0 (rows quantized on
 * append exactly as gt_quantize does; head_dim % 32 == 0).  Returns NULL on failure. */
typedef struct gt_kv_cache gt_kv_cache;
GT_API gt_kv_cache *gt_kv_cache_create(int64_t batch, int64_t n_head_kv, int64_t capacity, int64_t head_dim,
                                       int dtype, int device_index);
GT_API void gt_kv_cache_free(gt_kv_cache *c);
/* Empties sequence `seq`, or every sequence when seq < 0 (LlamaContext.clear_kv). */
GT_API int gt_kv_cache_clear(gt_kv_cache *c, int64_t seq);
/* Tokens held by sequence `seq` (-1 on error). */
GT_API int64_t gt_kv_cache_length(const gt_kv_cache *c, int64_t seq);
GT_API int64_t gt_kv_cache_capacity(const gt_kv_cache *c);
/* New handles sharing the cache's K / V storage, (batch, n_head_kv, capacity, head_dim). */
GT_API gt_tensor *gt_kv_cache_keys(const gt_kv_cache *c);
GT_API gt_tensor *gt_kv_cache_values(const gt_kv_cache *c);
/* Appends T tokens to every sequence: k, v (batch, n_head_kv, T, head_dim), any float dtype
 * and strides, or dense q8_0 (e.g. from gt_gguf_get_tensor_device; copied block for block into a
 * q8_0 cache, dequantized into a float one), host or device.  pos_offset < 0 appends after what each sequence holds;
 * otherwise it must equal every sequence's length (positions continue the cache, as
 * gt_llama_forward_logits requires).  Fails without writing when a sequence would pass the
 * capacity.  Returns 0 on success. */
GT_API int gt_kv_cache_append(gt_kv_cache *c, const gt_tensor *k, const gt_tensor *v, int64_t pos_offset);
/* No counterpart in the reference ABI (there, gt_rope of the keys, then the cache write inside
 * llama.cpp): gt_kv_cache_append with the keys rotated on the way in, each key row at its cache
 * position (the sequence's length + t), with gt_rope's arguments and arithmetic; the cache then
 * holds exactly what gt_rope followed by gt_kv_cache_append would store.  Values are not
 * rotated.  q8_0 keys are dequantized, rotated and quantized again. */
GT_API int gt_kv_cache_append_rope(gt_kv_cache *c, const gt_tensor *k, const gt_tensor *v, int64_t pos_offset,
                                   int n_dims, int mode, float freq_base, float freq_scale);
/* Attention of q (batch, H, L, head_dim), H % n_head_kv == 0, over each sequence's cached
 * tokens, query row l of sequence b being its token len_b - L + l (the last L appended).
 * is_causal: a query attends to its own position and the ones before it; otherwise to every
 * cached token.  scale <= 0 means 1/sqrt(head_dim).  Output (batch, H, L, head_dim), dtype
 * and device of q. */
GT_API gt_tensor *gt_kv_cache_attention(gt_kv_cache *c, const gt_tensor *q, float scale, int is_causal);

#ifdef __cplusplus
}
#endif

#endif /* GT_ATTN_H */
