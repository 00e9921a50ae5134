// RoPE entry points of libgt_attn.so: gt_rope / gt_rope_backward with the contract of the
// reference's operators (csrc/gt_ops_nn.cpp:2298-2421, declared at csrc/gguf_train.h:309-310):
// the same argument checks and error text, x of shape (batch, heads, seq_len, head_dim) or
// (heads, seq_len, head_dim) in any float dtype and any strides, positions read as int32 (any
// integer or float dtype, any strides, at least seq_len of them; the first seq_len are used),
// the result a new dense tensor of x's dtype on x's device.  The arithmetic (float32 angles and
// rotation, see gt_rope.hip) runs on the GPU; host tensors are staged through it.

#include "gt_internal.h"

#include <cmath>
#include <string>

namespace {

std::string shape_str(const gt_tensor *t) {
    std::string s = "[";
    for (int i = 0; i < t->ndim; ++i) s += (i ? ", " : "") + std::to_string(t->shape[i]);
    return s + "]";
}

struct RopeLayout {
    int64_t B = 1, H = 0, S = 0, D = 0;
    int64_t sb = 0, sh = 0, ss = 0, sd = 0;  // element strides of x as (B, H, S, D)
};

}  // namespace

// Checks of csrc/gt_ops_nn.cpp:2311-2349 (the reference turns every argument ggml would assert
// on, or loop forever on, into an error), shared with the RoPE-on-append of the KV cache.
bool gt_rope_check_args(const char *who, int64_t head_dim, int n_dims, int mode, float freq_base, float freq_scale) {
    if (mode != 0 && mode != 2) {
        gt_set_error(std::string(who) + ": mode must be 0 (normal) or 2 (NeoX), got " + std::to_string(mode) +
                     "; the multi-dimensional modes need per-section position ids and are not supported");
        return false;
    }
    if (n_dims < 2 || n_dims % 2 != 0 || n_dims > head_dim) {
        gt_set_error(std::string(who) + ": n_dims must be an even number between 2 and the head dimension " +
                     std::to_string(head_dim) + ", got " + std::to_string(n_dims));
        return false;
    }
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base) || !std::isfinite(freq_scale)) {
        gt_set_error(std::string(who) + ": freq_base must be positive and finite, and freq_scale finite");
        return false;
    }
    return true;
}

// ggml's theta_scale = powf(freq_base, -2/n_dims), computed on the host as ggml's CPU rope does.
float gt_rope_theta_scale(float freq_base, int n_dims) { return powf(freq_base, -2.0f / (float)n_dims); }

namespace {

bool rope_check(const gt_tensor *x, const gt_tensor *pos, int n_dims, int mode, float freq_base, float freq_scale,
                RopeLayout &L) {
    if (!x || !pos) {
        gt_set_error("rope: x and pos are required");
        return false;
    }
    if (x->ndim < 3 || x->ndim > 4) {
        gt_set_error("rope: expected x of shape (batch, heads, seq_len, head_dim) or (heads, seq_len, head_dim), got " +
                     shape_str(x));
        return false;
    }
    if (!gt_is_float(x->dtype)) {
        gt_set_error("rope: x must be a floating point tensor");
        return false;
    }
    const int o = x->ndim == 4 ? 1 : 0;
    L.B = o ? x->shape[0] : 1;
    L.H = x->shape[o];
    L.S = x->shape[o + 1];
    L.D = x->shape[o + 2];
    L.sb = o ? x->strides[0] : 0;
    L.sh = x->strides[o];
    L.ss = x->strides[o + 1];
    L.sd = x->strides[o + 2];
    if (!gt_rope_check_args("rope", L.D, n_dims, mode, freq_base, freq_scale)) return false;
    if (pos->ndim != 1 || pos->shape[0] < L.S) {
        gt_set_error("rope: pos must be a 1-D tensor with a position for each of the " + std::to_string(L.S) +
                     " sequence elements, got shape " + shape_str(pos));
        return false;
    }
    if (gt_is_quantized(pos->dtype)) {
        gt_set_error(std::string("rope: pos must hold integer or float positions, got ") + gt_dtype_name(pos->dtype));
        return false;
    }
    return true;
}

gt_tensor *rope_run(const gt_tensor *x, const gt_tensor *pos, const RopeLayout &L, int n_dims, int mode,
                    float freq_base, float freq_scale, bool backward) {
    if (x->numel == 0) return gt_tensor_empty(x->ndim, x->shape, x->dtype, x->device_type, x->device_index);
    const int dev = x->device_type == GT_DEV_CUDA ? x->device_index : 0;
    if (!gt_device_ok(dev)) return nullptr;
    gt_tensor *xs_owned = nullptr, *ps_owned = nullptr;
    const gt_tensor *xs = x;
    RopeLayout l = L;
    if (x->device_type != GT_DEV_CUDA || x->device_index != dev) {
        xs = xs_owned = gt_to_device_dense(x, dev, -1);
        if (!xs) return nullptr;
        l.sd = 1;
        l.ss = L.D;
        l.sh = L.S * L.D;
        l.sb = x->ndim == 4 ? L.H * L.S * L.D : 0;
    }
    // positions: a dense int32 device copy of the first S (integer or float -> int32 as a C cast)
    const gt_tensor *ps = pos;
    if (!(pos->device_type == GT_DEV_CUDA && pos->device_index == dev && pos->dtype == GT_I32 && gt_is_dense(pos))) {
        ps = ps_owned = gt_to_device_dense(pos, dev, GT_I32);
    }
    gt_tensor *out = ps ? gt_new_tensor(x->ndim, x->shape, x->dtype, GT_DEV_CUDA, dev) : nullptr;
    gt_scratch table;
    bool ok = out && gt_scratch_alloc(table, (size_t)L.S * (size_t)(n_dims / 2) * 2 * sizeof(float), dev);
    if (ok) {
        const float theta_scale = gt_rope_theta_scale(freq_base, n_dims);
        const int64_t strides[4] = {l.sb, l.sh, l.ss, l.sd};
        ok = gt_hip_check(gt_launch_rope_table((const int32_t *)gt_data(ps), nullptr, 1, L.S, n_dims, theta_scale,
                                               freq_scale, backward ? 1 : 0, table.ptr(), gt_stream()),
                          "rope table kernel") &&
             gt_hip_check(gt_launch_rope(gt_data(xs), x->dtype, strides, gt_data(out), table.ptr(), 0, L.B, L.H, L.S,
                                         L.D, n_dims, mode, gt_stream()),
                          "rope kernel");
    }
    gt_tensor_free(xs_owned);
    gt_tensor_free(ps_owned);
    if (!ok) {
        gt_tensor_free(out);
        return nullptr;
    }
    return gt_deliver(out, x->device_type != GT_DEV_CUDA);
}

}  // namespace

extern "C" gt_tensor *gt_rope(const gt_tensor *x, const gt_tensor *pos, int n_dims, int mode, int n_ctx_orig,
                              float freq_base, float freq_scale) {
    (void)n_ctx_orig;  // only used by YaRN (ext_factor != 0), which the reference never enables
    RopeLayout L;
    if (!rope_check(x, pos, n_dims, mode, freq_base, freq_scale, L)) return nullptr;
    return rope_run(x, pos, L, n_dims, mode, freq_base, freq_scale, false);
}

extern "C" gt_tensor *gt_rope_backward(const gt_tensor *grad_out, const gt_tensor *pos, int n_dims, int mode,
                                       int n_ctx_orig, float freq_base, float freq_scale) {
    (void)n_ctx_orig;
    RopeLayout L;
    if (!rope_check(grad_out, pos, n_dims, mode, freq_base, freq_scale, L)) return nullptr;
    return rope_run(grad_out, pos, L, n_dims, mode, freq_base, freq_scale, true);
}
