// Attention entry points of libgt_attn.so: argument validation with the reference's messages,
// operand staging onto the device, kernel selection, and the Q8_0 codec entry points.
//
// gt_flash_attention keeps the contract of csrc/gt_ops_nn.cpp:2423-2525; the kernels it
// dispatches to live in attn_generic.hip (any dtype/shape), attn_decode.hip (single-query
// split-K over the KV length, fp16/bf16/Q8_0 K/V) and attn_prefill.hip (fp16/bf16 MFMA).

#include "attn_common.h"
#include "gt_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

namespace {

// What the current (outermost) attention call on this thread launched, for gt_last_launch: one
// entry per kernel family, "; "-separated.  A call that starts while none is running clears it.
thread_local std::string t_launches;
thread_local int t_call_depth = 0;

struct LaunchScope {
    LaunchScope() {
        if (t_call_depth++ == 0) t_launches.clear();
    }
    ~LaunchScope() { --t_call_depth; }
};

void note_launch(const std::string &s) {
    if (!t_launches.empty()) t_launches += "; ";
    t_launches += s;
}

const char *dtype_tag(int cd) { return cd == GT_F16 ? "f16" : cd == GT_BF16 ? "bf16" : cd == GT_F32 ? "f32" : "f64"; }

// Owns the temporaries of one call.
struct Temps {
    std::vector<gt_tensor *> list;
    gt_tensor *keep(gt_tensor *t) {
        if (t) list.push_back(t);
        return t;
    }
    ~Temps() {
        for (gt_tensor *t : list) gt_tensor_free(t);
    }
};

bool inner_contiguous(const gt_tensor *t) { return t->ndim == 0 || t->shape[t->ndim - 1] <= 1 || t->strides[t->ndim - 1] == 1; }

// A device view of `t` in dtype `cd` whose innermost dimension is contiguous: `t` itself when
// it already is one, otherwise a dense converted copy (kept in `tmp`).
const gt_tensor *stage(const gt_tensor *t, int dev, int cd, Temps &tmp) {
    if (t->device_type == GT_DEV_CUDA && t->device_index == dev && t->dtype == cd && inner_contiguous(t)) return t;
    return tmp.keep(gt_to_device_dense(t, dev, cd));
}

// Same checks and messages as csrc/gt_ops_nn.cpp:2425-2454.
bool validate(const char *who, const gt_tensor *q, const gt_tensor *k, const gt_tensor *v, const gt_tensor *mask) {
    if (!q || !k || !v || q->ndim != 4 || k->ndim != 4 || v->ndim != 4) {
        gt_set_error("flash_attention expects 4D q, k, v tensors (B, H, L, D)");
        return false;
    }
    const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], D = q->shape[3];
    const int64_t Hkv = k->shape[1], S = k->shape[2];
    if (Hkv == 0 || H % Hkv != 0) {
        gt_set_error("flash_attention: num_heads must be divisible by num_kv_heads");
        return false;
    }
    if (k->shape[0] != B || v->shape[0] != B || v->shape[1] != Hkv || v->shape[2] != S || k->shape[3] != D) {
        gt_set_error("flash_attention: q (B, H, L, D), k (B, H_kv, S, D) and v (B, H_kv, S, Dv) do not fit together");
        return false;
    }
    if (mask) {
        const int64_t want[4] = {B, H, L, S};
        bool fits = mask->ndim == 2 || mask->ndim == 4;
        for (int i = 0; fits && i < mask->ndim; ++i) {
            const int64_t m = mask->shape[i];
            fits = (m == 1 || m == want[4 - mask->ndim + i]);
        }
        if (!fits) {
            std::string shape = "[";
            for (int i = 0; i < mask->ndim; ++i) shape += (i ? ", " : "") + std::to_string(mask->shape[i]);
            gt_set_error("flash_attention: attn_mask of shape " + shape + "] cannot be broadcast to the attention weights [" +
                         std::to_string(B) + ", " + std::to_string(H) + ", " + std::to_string(L) + ", " +
                         std::to_string(S) + "]");
            return false;
        }
        if (gt_is_quantized(mask->dtype)) {
            gt_set_error(std::string(who) + ": a quantized attn_mask is not supported");
            return false;
        }
    }
    if (!gt_is_float(q->dtype)) {
        gt_set_error(std::string(who) + ": q must be float32, float16, bfloat16 or float64, got " + gt_dtype_name(q->dtype));
        return false;
    }
    for (const gt_tensor *t : {k, v}) {
        if (!gt_is_float(t->dtype) && t->dtype != GT_Q8_0) {
            gt_set_error(std::string(who) + ": k and v must be float32, float16, bfloat16, float64 or q8_0, got " +
                         gt_dtype_name(t->dtype));
            return false;
        }
        if (t->dtype == GT_Q8_0 && (t->shape[3] % 32 != 0 || !gt_is_dense(t) || t->offset != 0)) {
            gt_set_error(std::string(who) + ": a q8_0 k/v must be contiguous with a head size that is a multiple of 32");
            return false;
        }
    }
    return true;
}

// Compute dtype of q/k/v: float64 if any operand is float64; the common dtype when all agree
// on float32/float16/bfloat16; float32 otherwise (every such widening is exact).  A Q8_0 k/v
// counts as float16 when q is float16 (its dequantized values, rounded once to float16, 2^-12
// relative, feed the MFMA kernels), as float32 otherwise (exact values: rounded to bfloat16
// the keys would move the scores by ~2^-9 relative, more than the bfloat16 bar allows).
int compute_dtype(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v) {
    const int q8_as = q->dtype == GT_F16 ? GT_F16 : GT_F32;
    const int dq = q->dtype, dk = k->dtype == GT_Q8_0 ? q8_as : k->dtype, dv = v->dtype == GT_Q8_0 ? q8_as : v->dtype;
    if (dq == GT_F64 || dk == GT_F64 || dv == GT_F64) return GT_F64;
    if (dq == dk && dk == dv) return dq;
    return GT_F32;
}

// Fills the mask fields of `a`: a bool mask is read as bytes; any other dtype is staged as
// additive values of the compute precision.  Broadcast dimensions get stride 0.
bool stage_mask(const gt_tensor *mask, int dev, int cd, AttnFwdArgs &a, Temps &tmp) {
    a.mask = nullptr;
    a.mask_bool = 0;
    a.m_sb = a.m_sh = a.m_sl = a.m_ss = 0;
    if (!mask) return true;
    const int want = mask->dtype == GT_BOOL ? GT_BOOL : (cd == GT_F64 ? GT_F64 : GT_F32);
    const gt_tensor *m = mask;
    if (!(m->device_type == GT_DEV_CUDA && m->device_index == dev && m->dtype == want)) {
        m = tmp.keep(gt_to_device_dense(mask, dev, want));
        if (!m) return false;
    }
    // A bool mask that does not depend on the query row (key padding, (L, S) with L == 1 or a
    // broadcast query dimension) becomes the equivalent additive mask (0 / -inf): x + 0 = x and
    // x + -inf = -inf, so the scores, the blocked positions and the all-blocked rows are the same,
    // and the kernels read it once per key instead of once per (query, key).
    const bool row_bcast = m->ndim < 2 || m->shape[m->ndim - 2] == 1;
    if (want == GT_BOOL && cd != GT_F64 && row_bcast) {
        const gt_tensor *dense = gt_is_dense(m) && m->offset == 0 ? m : tmp.keep(gt_to_device_dense(m, dev, GT_BOOL));
        if (!dense) return false;
        gt_tensor *bias = tmp.keep(gt_new_tensor(dense->ndim, dense->shape, GT_F32, GT_DEV_CUDA, dev));
        if (!bias) return false;
        if (!gt_hip_check(gt_launch_bool_to_bias(gt_data(dense), (float *)gt_data(bias), dense->numel, gt_stream()),
                          "flash_attention: mask conversion"))
            return false;
        m = bias;
    }
    int64_t st[4] = {0, 0, 0, 0}, sh[4] = {1, 1, 1, 1};
    for (int i = 0; i < m->ndim; ++i) {
        sh[4 - m->ndim + i] = m->shape[i];
        st[4 - m->ndim + i] = m->strides[i];
    }
    for (int i = 0; i < 4; ++i) if (sh[i] == 1) st[i] = 0;
    a.mask = gt_data(m);
    a.mask_bool = m->dtype == GT_BOOL;
    a.m_sb = st[0];
    a.m_sh = st[1];
    a.m_sl = st[2];
    a.m_ss = st[3];
    return true;
}

void fill_qkv(AttnFwdArgs &a, const gt_tensor *q, const gt_tensor *k, const gt_tensor *v) {
    a.q = gt_data(q);
    a.k = gt_data(k);
    a.v = gt_data(v);
    a.B = q->shape[0];
    a.H = q->shape[1];
    a.L = q->shape[2];
    a.D = q->shape[3];
    a.Hkv = k->shape[1];
    a.S = k->shape[2];
    a.Dv = v->shape[3];
    a.q_sb = q->strides[0];
    a.q_sh = q->strides[1];
    a.q_sl = q->strides[2];
    if (k->dtype == GT_Q8_0) {  // dense block rows: strides counted in elements of the logical tensor
        a.k_sb = k->shape[1] * k->shape[2] * k->shape[3];
        a.k_sh = k->shape[2] * k->shape[3];
        a.k_ss = k->shape[3];
    } else {
        a.k_sb = k->strides[0];
        a.k_sh = k->strides[1];
        a.k_ss = k->strides[2];
    }
    if (v->dtype == GT_Q8_0) {
        a.v_sb = v->shape[1] * v->shape[2] * v->shape[3];
        a.v_sh = v->shape[2] * v->shape[3];
        a.v_ss = v->shape[3];
    } else {
        a.v_sb = v->strides[0];
        a.v_sh = v->strides[1];
        a.v_ss = v->strides[2];
    }
}

// Memory for the split partials of a decode launch (da.nsplit set): with several splits, the
// per-stream uncached workspace whose counters (`units`: one per blockIdx.y of the launch) let
// the last split merge in the kernel; otherwise
// (or when that workspace is unavailable) stream-ordered scratch, merged by a second launch.
bool decode_partials(DecodeArgs &da, int64_t units, int dev, gt_scratch &scratch) {
    const AttnFwdArgs &a = da.f;
    const size_t rows = (size_t)(a.B * a.H) * (size_t)da.nsplit;
    const size_t bytes = rows * (size_t)(a.D + 2) * sizeof(float);
    gt_decode_ws ws{};
    if (da.nsplit > 1 && gt_decode_workspace(dev, gt_stream(), units, bytes, ws)) {
        da.counters = ws.counters;
        da.part_o = (float *)ws.parts;
    } else {
        if (!gt_scratch_alloc(scratch, bytes, dev)) return false;
        da.part_o = (float *)scratch.ptr();
    }
    da.part_ml = da.part_o + rows * (size_t)a.D;
    return true;
}

// Picks the kernel for a staged forward: split-K decode for single-query rows, the MFMA
// prefill kernel for fp16/bf16 with head size 64/128, the generic kernel otherwise.
// Launch-log entry of a split-K decode launch.
std::string decode_note(const char *kind, const DecodeArgs &da, int max_tile) {
    const AttnFwdArgs &a = da.f;
    const bool merged_in_kernel = da.counters && da.nsplit > 1 && a.D <= 128;
    return std::string(kind) + " D=" + std::to_string(a.D) +
           " heads_per_group=" + std::to_string(decode_head_tile(a.H / a.Hkv, max_tile)) +
           " splits=" + std::to_string(da.nsplit) + " units=" + std::to_string(decode_units(a.B, a.H, a.Hkv, max_tile)) +
           " merge=" + (da.nsplit == 1 && a.D <= 128 ? "none" : merged_in_kernel ? "in-kernel" : "second-launch");
}

std::string prefill_note(const AttnFwdArgs &a, int cd) {
    return std::string(attn_prefill_asm_supported(a, cd) ? "prefill pipelined " : "prefill ") + dtype_tag(cd) + " D=" + std::to_string(a.D) + " B=" + std::to_string(a.B) +
           " H=" + std::to_string(a.H) + " L=" + std::to_string(a.L) + " S=" + std::to_string(a.S) +
           (attn_prefill_f32_split(a, cd) ? " split" : "");
}

bool dispatch_forward(const AttnFwdArgs &a, int cd, int dev) {
    if (a.out_dtype == cd && !a.o32 && !a.dropout && attn_decode_supported(a, cd)) {
        DecodeArgs da{};
        da.f = a;
        da.nsplit = attn_decode_splits(a, cd);
        gt_scratch ws;
        const int tile = attn_decode_max_tile(cd);
        if (!decode_partials(da, decode_units(a.B, a.H, a.Hkv, tile), dev, ws)) return false;
        note_launch(decode_note((std::string("decode ") + dtype_tag(cd)).c_str(), da, tile));
        return gt_hip_check(launch_attn_decode(da, cd, gt_stream()), "flash_attention decode kernel");
    }
    if (attn_prefill_supported(a, cd)) {
        note_launch(prefill_note(a, cd));
        return gt_hip_check(launch_attn_prefill(a, cd, gt_stream()), "flash_attention prefill kernel");
    }
    note_launch(std::string("generic ") + dtype_tag(cd));
    return gt_hip_check(launch_attn_generic_fwd(a, cd, gt_stream()), "flash_attention kernel");
}

// Moves a device result into a new host tensor when the caller's q lives on the host.
gt_tensor *deliver(gt_tensor *dev_t, bool to_host) { return gt_deliver(dev_t, to_host); }

// Single-query attention straight from Q8_0 K/V blocks.  Returns 1 when it ran, 0 when the
// shapes do not suit the kernel (the caller then dequantizes), -1 on error.
int run_q8_decode(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v, const gt_tensor *mask, float scale,
                  int is_causal, int dev, gt_tensor *o, gt_tensor *lse, Temps &tmp, const int32_t *kv_len = nullptr,
                  const int32_t *q_pos = nullptr) {
    const gt_tensor *qs = stage(q, dev, GT_F16, tmp);
    const gt_tensor *ks = k->device_type == GT_DEV_CUDA && k->device_index == dev ? k : tmp.keep(gt_to_device_dense(k, dev, -1));
    const gt_tensor *vs = v->device_type == GT_DEV_CUDA && v->device_index == dev ? v : tmp.keep(gt_to_device_dense(v, dev, -1));
    if (!qs || !ks || !vs) return -1;
    AttnFwdArgs a{};
    fill_qkv(a, qs, ks, vs);
    a.o = gt_data(o);
    a.lse = lse ? gt_data(lse) : nullptr;
    a.scale = scale;
    a.causal = is_causal ? 1 : 0;
    a.out_dtype = GT_F16;
    a.kv_len = kv_len;
    a.q_pos = q_pos;
    if (!attn_decode_q8_supported(a, GT_F16)) return 0;
    if (!stage_mask(mask, dev, GT_F16, a, tmp)) return -1;
    DecodeArgs da{};
    da.f = a;
    da.nsplit = attn_decode_q8_splits(a);
    gt_scratch ws;
    if (!decode_partials(da, decode_units(a.B, a.H, a.Hkv, kDecodeQ8MaxTile), dev, ws)) return -1;
    note_launch(decode_note("decode q8_0", da, kDecodeQ8MaxTile));
    return gt_hip_check(launch_attn_decode_q8(da, gt_stream()), "flash_attention q8_0 decode kernel") ? 1 : -1;
}

// Dropout of the attention probabilities: the Philox key/counter and the keep threshold of
// probability p (gt_philox.h).  p = 0 leaves `on` false (plain attention); p outside [0, 1] is an
// error.  thresh = floor((1 - p) * 2^32) and scale = 1 / (1 - p) in double precision, 0 for p = 1.
struct Dropout {
    bool on = false;
    GtDropout d{};
};

bool make_dropout(const char *who, double p, uint64_t seed, uint64_t offset, Dropout &out) {
    if (!(p >= 0.0 && p <= 1.0)) {
        gt_set_error(std::string(who) + ": dropout probability has to be between 0 and 1, but got " + std::to_string(p));
        return false;
    }
    out = Dropout{};
    if (p == 0.0) return true;
    out.on = true;
    out.d.seed = seed;
    out.d.offset = offset;
    const double t = std::floor((1.0 - p) * 4294967296.0);
    out.d.thresh = t >= 4294967295.0 ? 4294967295u : (uint32_t)t;
    out.d.scale = p < 1.0 ? 1.0 / (1.0 - p) : 0.0;
    return true;
}

// Largest buffer of dropout decision bits the backward allocates (B*H*L*ceil(S/32)*4 bytes):
// 512 MiB, or GT_ATTN_DROPOUT_BITS_MAX bytes when set; beyond it the dK/dV kernel draws the
// decisions itself (bounded memory, more Philox work).
size_t dropout_bits_max() {
    const char *v = std::getenv("GT_ATTN_DROPOUT_BITS_MAX");
    return v && *v ? (size_t)std::strtoull(v, nullptr, 10) : ((size_t)512 << 20);
}

void apply_dropout(AttnFwdArgs &a, const Dropout *drop) {
    if (drop && drop->on) {
        a.dropout = 1;
        a.drop = drop->d;
    }
}

// ---- head padding ----------------------------------------------------------------------------
// The MFMA kernels take head sizes 64 and 128.  Attention with another head size up to 128 and
// more than one query row runs on them with q, k, v (and in the backward dO and the output)
// zero-padded to 64 or 128 dims: the zero dims add nothing to Q.K^T (the scale stays that of the
// real head size), padded V columns give output columns that are dropped, and the padded columns
// of dQ, dK, dV are zero and dropped.  Single-query rows keep their kernels (padding would copy
// the whole K/V).  Float32 pads only calls its MFMA kernels take (16 query rows or more, no KV
// cache lengths: f32_pads; the backward also 32 dQ workgroups), the rest keep the generic kernels
// unpadded.
int64_t mfma_head(int64_t d) { return d <= 0 ? 0 : d <= 64 ? 64 : d <= 128 ? 128 : 0; }

int64_t padded_head(int cd, int64_t L, int64_t D, int64_t Dv) {
    if ((cd != GT_F16 && cd != GT_BF16 && cd != GT_F32) || L <= 1) return 0;
    if (cd == GT_F32 && L < 16) return 0;
    if (D == Dv && (D == 64 || D == 128)) return 0;
    if (!mfma_head(D) || !mfma_head(Dv)) return 0;
    return std::max(mfma_head(D), mfma_head(Dv));
}

// Float32 calls whose padded form the float32 MFMA kernels take (masks staged, dropout applied).
bool f32_pads(const AttnFwdArgs &a) { return !a.kv_len && !a.q_pos; }

// A dense (d0, d1, d2, Dp) copy of the 4-D device tensor t (innermost contiguous, 2- or 4-byte
// elements) whose dims past t's last are zero; kept in tmp.
const gt_tensor *pad_heads(const gt_tensor *t, int64_t Dp, int dev, Temps &tmp) {
    const int64_t sh[4] = {t->shape[0], t->shape[1], t->shape[2], Dp};
    gt_tensor *p = tmp.keep(gt_new_tensor(4, sh, t->dtype, GT_DEV_CUDA, dev));
    if (!p || !gt_hip_check(gt_launch_pad_rows(gt_data(t), (int)gt_elem_bytes(t->dtype), t->strides, sh[0], sh[1],
                                               sh[2], t->shape[3], gt_data(p), Dp, gt_stream()),
                            "head padding kernel"))
        return nullptr;
    return p;
}

// The first t->shape[3] dims of every row of the dense padded buffer `src` into the dense t.
bool unpad_heads(const gt_tensor *src, gt_tensor *t) {
    const int64_t rows = t->shape[0] * t->shape[1] * t->shape[2];
    return gt_hip_check(gt_launch_unpad_rows(gt_data(src), (int)gt_elem_bytes(t->dtype), rows, src->shape[3],
                                             gt_data(t), t->shape[3], gt_stream()),
                        "head padding kernel");
}

// RoPE of the queries fused into the prefill kernel: the (cos, sin) table of the L query rows.
struct QRope {
    const void *table;  // float2 (L, D/2) on the device
    int neox;
};

int attention_forward(const char *who, const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                      const gt_tensor *mask, float scale, int is_causal, gt_tensor **out_o, gt_tensor **out_lse,
                      gt_tensor **out_o32 = nullptr, const QRope *qrope = nullptr, const Dropout *drop = nullptr) {
    LaunchScope scope;
    if (out_o) *out_o = nullptr;
    if (out_lse) *out_lse = nullptr;
    if (out_o32) *out_o32 = nullptr;
    if (!validate(who, q, k, v, mask)) return -1;
    const int dev = q->device_type == GT_DEV_CUDA ? q->device_index : 0;
    const bool host_io = q->device_type != GT_DEV_CUDA;
    if (!gt_device_ok(dev)) return -1;
    const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], D = q->shape[3];
    const int64_t Dv = v->shape[3];
    if (scale <= 0.0f) scale = 1.0f / std::sqrt((float)D);  // csrc/gt_ops_nn.cpp:2433

    const int cd = compute_dtype(q, k, v);
    const int lse_dtype = cd == GT_F64 ? GT_F64 : GT_F32;
    const int64_t osh[4] = {B, H, L, Dv}, lsh[3] = {B, H, L};
    gt_tensor *o = gt_new_tensor(4, osh, q->dtype, GT_DEV_CUDA, dev);
    gt_tensor *lse = out_lse ? gt_new_tensor(3, lsh, lse_dtype, GT_DEV_CUDA, dev) : nullptr;
    // the unrounded float32 output, for a training forward of a float16/bfloat16 call
    const bool want32 = out_o32 && (q->dtype == GT_F16 || q->dtype == GT_BF16);
    gt_tensor *o32 = want32 ? gt_new_tensor(4, osh, GT_F32, GT_DEV_CUDA, dev) : nullptr;
    if (!o || (out_lse && !lse) || (want32 && !o32)) {
        gt_tensor_free(o);
        gt_tensor_free(lse);
        gt_tensor_free(o32);
        return -1;
    }
    Temps tmp;
    bool ok = true;
    int q8 = 0;  // 1: the Q8_0 decode kernel ran
    if ((o->numel > 0 || (lse && lse->numel > 0)) && k->dtype == GT_Q8_0 && v->dtype == GT_Q8_0 &&
        q->dtype == GT_F16 && L == 1 && !o32 && !(drop && drop->on)) {
        q8 = run_q8_decode(q, k, v, mask, scale, is_causal, dev, o, lse, tmp);
        ok = q8 >= 0;
    }
    if (q8 == 0 && (o->numel > 0 || (lse && lse->numel > 0))) {
        // Q8_0 K/V are dequantized to the compute dtype: float16 for float16 queries (values
        // rounded once; the MFMA kernels run), float32 otherwise (exact values)
        const gt_tensor *qs = stage(q, dev, cd, tmp);
        if (k->dtype == GT_Q8_0 || v->dtype == GT_Q8_0) note_launch("dequantize q8_0 k/v");
        // Causal without a mask or dropout: keys >= L are visible to no query row (top-left
        // alignment), so only the first L rows of Q8_0 K/V are dequantized and attended.
        const int64_t S = k->shape[2];
        const int64_t Sq = is_causal && !mask && !(drop && drop->on) && L < S && k->dtype == GT_Q8_0 &&
                                   v->dtype == GT_Q8_0 ? L : S;
        auto dequant = [&](const gt_tensor *t) -> const gt_tensor * {
            if (Sq == S) return tmp.keep(gt_dequantize(t, cd));
            const gt_tensor *src = t->device_type == GT_DEV_CUDA ? t : tmp.keep(gt_to_device_dense(t, dev, GT_Q8_0));
            const int64_t sh[4] = {t->shape[0], t->shape[1], Sq, t->shape[3]}, rb = t->shape[3] / 32;
            gt_tensor *d = src ? tmp.keep(gt_new_tensor(4, sh, cd, GT_DEV_CUDA, dev)) : nullptr;
            if (!d || !gt_hip_check(gt_launch_q8_0_dequantize_rows(gt_data(src), gt_data(d), cd, sh[0] * sh[1] * Sq * rb,
                                                                   Sq * rb, S * rb, gt_stream()),
                                    "q8_0 dequantize kernel"))
                return nullptr;
            return d;
        };
        const gt_tensor *ks = k->dtype == GT_Q8_0 ? dequant(k) : stage(k, dev, cd, tmp);
        const gt_tensor *vs = v->dtype == GT_Q8_0 ? dequant(v) : stage(v, dev, cd, tmp);
        if (ks && ks->device_type != GT_DEV_CUDA) ks = stage(ks, dev, cd, tmp);
        if (vs && vs->device_type != GT_DEV_CUDA) vs = stage(vs, dev, cd, tmp);
        ok = qs && ks && vs;
        AttnFwdArgs a{};
        if (ok) {
            fill_qkv(a, qs, ks, vs);
            ok = stage_mask(mask, dev, cd, a, tmp);
        }
        if (ok) {
            a.o = gt_data(o);
            a.lse = lse ? gt_data(lse) : nullptr;
            a.o32 = o32 ? gt_data(o32) : nullptr;
            a.scale = scale;
            a.causal = is_causal ? 1 : 0;
            a.out_dtype = q->dtype;
            apply_dropout(a, drop);
            // heads padded to the MFMA kernels' sizes (output and float32 output unpadded after)
            const gt_tensor *po = nullptr, *po32 = nullptr;
            const int64_t Dp = qrope || a.out_dtype != cd || (cd == GT_F32 && !f32_pads(a)) ? 0 : padded_head(cd, L, D, Dv);
            if (Dp) {
                const gt_tensor *qp = pad_heads(qs, Dp, dev, tmp), *kp = pad_heads(ks, Dp, dev, tmp);
                const gt_tensor *vp = pad_heads(vs, Dp, dev, tmp);
                const int64_t psh[4] = {B, H, L, Dp};
                po = tmp.keep(gt_new_tensor(4, psh, q->dtype, GT_DEV_CUDA, dev));
                po32 = o32 ? tmp.keep(gt_new_tensor(4, psh, GT_F32, GT_DEV_CUDA, dev)) : nullptr;
                ok = qp && kp && vp && po && (!o32 || po32);
                if (ok) {
                    fill_qkv(a, qp, kp, vp);
                    a.o = const_cast<void *>(gt_data(po));
                    a.o32 = po32 ? const_cast<void *>(gt_data(po32)) : nullptr;
                }
            }
            if (qrope) {
                a.rope_q = qrope->table;
                a.rope_neox = qrope->neox;
                if (!attn_prefill_supported(a, cd)) {
                    // only the prefill kernel applies the rotation: the caller rotates q itself
                    gt_tensor_free(o);
                    gt_tensor_free(lse);
                    gt_tensor_free(o32);
                    return 1;
                }
            }
            ok = ok && dispatch_forward(a, cd, dev);
            if (ok && po) ok = unpad_heads(po, o) && (!po32 || unpad_heads(po32, o32));
        }
    }
    if (!ok) {
        gt_tensor_free(o);
        gt_tensor_free(lse);
        gt_tensor_free(o32);
        return -1;
    }
    o = deliver(o, host_io);
    if (lse) lse = deliver(lse, host_io);
    if (o32) o32 = deliver(o32, host_io);
    if (!o || (out_lse && !lse) || (want32 && !o32)) {
        gt_tensor_free(o);
        gt_tensor_free(lse);
        gt_tensor_free(o32);
        return -1;
    }
    if (out_o) *out_o = o; else gt_tensor_free(o);
    if (out_lse) *out_lse = lse;
    if (out_o32) *out_o32 = o32;
    return 0;
}

}  // namespace

extern "C" const char *gt_last_launch(void) { return t_launches.c_str(); }

extern "C" gt_tensor *gt_flash_attention(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                         const gt_tensor *mask, float scale, int is_causal) {
    gt_tensor *o = nullptr;
    if (attention_forward("flash_attention", q, k, v, mask, scale, is_causal, &o, nullptr) != 0) return nullptr;
    return o;
}

// Attention of RoPE-rotated queries and keys: gt_rope(q, pos) and gt_rope(k, pos) (first L / S
// positions) followed by gt_flash_attention.  The keys are rotated in one pass (each is read by
// every query tile); the queries are rotated by the prefill kernel as it loads them when it runs
// (float16/bfloat16 q, k, v of one dtype, n_dims = D, L > 1, no mask or a key-padding row),
// otherwise in a pass of their own.
extern "C" gt_tensor *gt_flash_attention_rope(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                              const gt_tensor *mask, float scale, int is_causal, const gt_tensor *pos,
                                              int n_dims, int mode, float freq_base, float freq_scale) {
    const char *who = "flash_attention_rope";
    LaunchScope scope;
    if (!validate(who, q, k, v, mask)) return nullptr;
    const int64_t L = q->shape[2], S = k->shape[2], D = q->shape[3];
    if (!gt_rope_check_args(who, D, n_dims, mode, freq_base, freq_scale)) return nullptr;
    const int64_t need = std::max(L, S);
    if (!pos || pos->ndim != 1 || pos->shape[0] < need || gt_is_quantized(pos->dtype)) {
        gt_set_error(std::string(who) + ": pos must be a 1-D tensor with a position for each of the " +
                     std::to_string(need) + " sequence elements");
        return nullptr;
    }
    if (k->dtype == GT_Q8_0) {
        gt_set_error(std::string(who) + ": k must be a floating point tensor (RoPE of q8_0 keys: dequantize first)");
        return nullptr;
    }
    const int dev = q->device_type == GT_DEV_CUDA ? q->device_index : 0;
    if (!gt_device_ok(dev)) return nullptr;
    Temps tmp;
    const gt_tensor *kd =
        k->device_type == GT_DEV_CUDA && k->device_index == dev ? k : tmp.keep(gt_to_device_dense(k, dev, -1));
    if (!kd) return nullptr;
    gt_tensor *o = nullptr;
    const bool key_padding = !mask || (mask->dtype != GT_BOOL && mask->shape[mask->ndim - 2] == 1);
    if ((q->dtype == GT_F16 || q->dtype == GT_BF16) && k->dtype == q->dtype && v->dtype == q->dtype &&
        q->device_type == GT_DEV_CUDA && n_dims == D && (D == 64 || D == 128) && L > 1 && key_padding &&
        kd->ndim == 4) {
        // one int32 copy of the positions and one (cos, sin) table for the first max(L, S) of them:
        // the keys are rotated with it here, the prefill kernel rotates the queries (rows 0..L-1)
        // as it loads them; the same values as gt_rope's own table for either
        const gt_tensor *pd = (pos->device_type == GT_DEV_CUDA && pos->device_index == dev && pos->dtype == GT_I32 &&
                               gt_is_dense(pos))
                                  ? pos
                                  : tmp.keep(gt_to_device_dense(pos, dev, GT_I32));
        gt_scratch table;
        gt_tensor *kr = pd ? tmp.keep(gt_new_tensor(4, kd->shape, kd->dtype, GT_DEV_CUDA, dev)) : nullptr;
        if (!kr || !gt_scratch_alloc(table, (size_t)need * (size_t)(D / 2) * 2 * sizeof(float), dev) ||
            !gt_hip_check(gt_launch_rope_table((const int32_t *)gt_data(pd), nullptr, 1, need, n_dims,
                                               gt_rope_theta_scale(freq_base, n_dims), freq_scale, 0, table.ptr(),
                                               gt_stream()),
                          "rope table kernel") ||
            !gt_hip_check(gt_launch_rope(gt_data(kd), kd->dtype, kd->strides, gt_data(kr), table.ptr(), 0, kd->shape[0],
                                         kd->shape[1], S, D, n_dims, mode, gt_stream()),
                          "rope kernel"))
            return nullptr;
        const QRope qr{table.ptr(), mode == 2 ? 1 : 0};
        const int rc = attention_forward(who, q, kr, v, mask, scale, is_causal, &o, nullptr, nullptr, &qr);
        if (rc < 0) return nullptr;
        if (rc == 0) return o;
        // the kernel declined the rotated-query form (rc > 0): rotate q and attend below
        const gt_tensor *qr2 = tmp.keep(gt_rope(q, pd, n_dims, mode, 0, freq_base, freq_scale));
        if (!qr2 || attention_forward(who, qr2, kr, v, mask, scale, is_causal, &o, nullptr) != 0) return nullptr;
        return o;
    }
    const gt_tensor *kr = tmp.keep(gt_rope(kd, pos, n_dims, mode, 0, freq_base, freq_scale));
    const gt_tensor *qr = kr ? tmp.keep(gt_rope(q, pos, n_dims, mode, 0, freq_base, freq_scale)) : nullptr;
    if (!qr || attention_forward(who, qr, kr, v, mask, scale, is_causal, &o, nullptr) != 0) return nullptr;
    return o;
}

extern "C" int gt_flash_attention_lse(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v, const gt_tensor *mask,
                                      float scale, int is_causal, gt_tensor **out, gt_tensor **lse) {
    if (!out || !lse) {
        gt_set_error("flash_attention_lse: out and lse must not be NULL");
        return -1;
    }
    return attention_forward("flash_attention_lse", q, k, v, mask, scale, is_causal, out, lse);
}

extern "C" int gt_flash_attention_train(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                        const gt_tensor *mask, float scale, int is_causal, gt_tensor **out,
                                        gt_tensor **lse, gt_tensor **out32) {
    if (!out || !lse || !out32) {
        gt_set_error("flash_attention_train: out, lse and out32 must not be NULL");
        return -1;
    }
    return attention_forward("flash_attention_train", q, k, v, mask, scale, is_causal, out, lse, out32);
}

namespace {

int attention_backward(const char *who, const gt_tensor *grad_out, const gt_tensor *q, const gt_tensor *k,
                       const gt_tensor *v, const gt_tensor *mask, const gt_tensor *out, const gt_tensor *lse,
                       float scale, int is_causal, const Dropout *drop, gt_tensor **dq, gt_tensor **dk,
                       gt_tensor **dv) {
    LaunchScope scope;
    if (!dq || !dk || !dv) {
        gt_set_error(std::string(who) + ": dq, dk and dv must not be NULL");
        return -1;
    }
    *dq = *dk = *dv = nullptr;
    if (!validate(who, q, k, v, mask)) return -1;
    if (k->dtype == GT_Q8_0 || v->dtype == GT_Q8_0) {
        gt_set_error(std::string(who) + ": q8_0 k/v have no gradient");
        return -1;
    }
    const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], D = q->shape[3];
    const int64_t Hkv = k->shape[1], S = k->shape[2], Dv = v->shape[3];
    if (!grad_out || grad_out->ndim != 4 || grad_out->shape[0] != B || grad_out->shape[1] != H ||
        grad_out->shape[2] != L || grad_out->shape[3] != Dv) {
        gt_set_error(std::string(who) + ": grad_out must have the output's shape (B, H, L, Dv)");
        return -1;
    }
    if (lse && (lse->ndim != 3 || lse->shape[0] != B || lse->shape[1] != H || lse->shape[2] != L)) {
        gt_set_error(std::string(who) + ": lse must have shape (B, H, L)");
        return -1;
    }
    const int dev = q->device_type == GT_DEV_CUDA ? q->device_index : 0;
    const bool host_io = q->device_type != GT_DEV_CUDA;
    if (!gt_device_ok(dev)) return -1;
    if (scale <= 0.0f) scale = 1.0f / std::sqrt((float)D);
    const int cd = compute_dtype(q, k, v);
    const int gd = cd == GT_F64 ? GT_F64 : GT_F32;
    Temps tmp;

    // the forward's residuals (output and log-sum-exp): given, or recomputed by a forward pass.
    // The fp16/bf16 MFMA backward forms rowsum(dP * P) as rowsum(dO * O), exact with the float32
    // output the training forward keeps; an output rounded to fp16/bf16 would carry its rounding
    // into every dS, so that case recomputes the float32 output (the forward is deterministic:
    // it is the training forward's copy bit for bit).
    const gt_tensor *lse_s = nullptr, *out_s = nullptr;
    int64_t Dp = padded_head(cd, L, D, Dv);  // heads padded for the MFMA kernels (0: none)
    const bool mfma_shape = ((cd == GT_F16 || cd == GT_BF16) && D == Dv && (D == 64 || D == 128)) || Dp != 0;
    if (!lse || !out || (mfma_shape && out->dtype != GT_F32)) {
        gt_tensor *o2 = nullptr, *l2 = nullptr, *o32 = nullptr;
        if (attention_forward(who, q, k, v, mask, scale, is_causal, &o2, &l2, mfma_shape ? &o32 : nullptr, nullptr,
                              drop) != 0)
            return -1;
        tmp.keep(o2);
        tmp.keep(l2);
        tmp.keep(o32);
        if (!lse) lse = l2;
        out = o32 ? o32 : o2;
    }
    lse_s = (lse->device_type == GT_DEV_CUDA && lse->device_index == dev && lse->dtype == gd && gt_is_dense(lse))
                ? lse
                : tmp.keep(gt_to_device_dense(lse, dev, gd));
    // a float32 `out` (the training forward's unrounded output) gives the exact rowsum(dO * O)
    const int od = (out->dtype == GT_F32 && cd != GT_F64) ? GT_F32 : cd;
    out_s = (out->device_type == GT_DEV_CUDA && out->device_index == dev && out->dtype == od && gt_is_dense(out))
                ? out
                : tmp.keep(gt_to_device_dense(out, dev, od));
    if (!lse_s || !out_s) return -1;
    const int64_t qsh[4] = {B, H, L, D}, ksh[4] = {B, Hkv, S, D}, vsh[4] = {B, Hkv, S, Dv}, rsh[3] = {B, H, L};
    gt_tensor *gq = gt_new_tensor(4, qsh, gd, GT_DEV_CUDA, dev);
    gt_tensor *gk = gt_new_tensor(4, ksh, gd, GT_DEV_CUDA, dev);
    gt_tensor *gv = gt_new_tensor(4, vsh, gd, GT_DEV_CUDA, dev);
    gt_tensor *delta = tmp.keep(gt_new_tensor(3, rsh, gd, GT_DEV_CUDA, dev));
    const gt_tensor *qs = stage(q, dev, cd, tmp), *ks = stage(k, dev, cd, tmp), *vs = stage(v, dev, cd, tmp);
    const gt_tensor *gos = grad_out->device_type == GT_DEV_CUDA && grad_out->device_index == dev &&
                                   grad_out->dtype == cd && gt_is_dense(grad_out)
                               ? grad_out
                               : tmp.keep(gt_to_device_dense(grad_out, dev, cd));
    bool ok = gq && gk && gv && delta && qs && ks && vs && gos && lse_s;
    AttnBwdArgs a{};
    if (ok) {
        fill_qkv(a.f, qs, ks, vs);
        ok = stage_mask(mask, dev, cd, a.f, tmp);
    }
    if (ok) {
        a.f.lse = gt_data(lse_s);
        a.f.scale = scale;
        a.f.causal = is_causal ? 1 : 0;
        a.f.out_dtype = cd;
        a.dout = gt_data(gos);
        a.dq = gt_data(gq);
        a.dk = gt_data(gk);
        a.dv = gt_data(gv);
        a.delta = gt_data(delta);
        a.f.o = const_cast<void *>(gt_data(out_s));
        a.o_f32 = od == GT_F32 && cd != GT_F32;
        apply_dropout(a.f, drop);
        // heads padded to the MFMA kernels' sizes: padded inputs, padded gradients unpadded after.
        // Float32: only where its MFMA backward takes the padded call
        if (cd == GT_F32 && !f32_pads(a.f)) Dp = 0;
        const gt_tensor *pq = nullptr, *pk = nullptr, *pv = nullptr;
        if (Dp) {
            const gt_tensor *qp = pad_heads(qs, Dp, dev, tmp), *kp = pad_heads(ks, Dp, dev, tmp);
            const gt_tensor *vp = pad_heads(vs, Dp, dev, tmp), *gp = pad_heads(gos, Dp, dev, tmp);
            const gt_tensor *op = pad_heads(out_s, Dp, dev, tmp);
            const int64_t qsh2[4] = {B, H, L, Dp}, ksh2[4] = {B, Hkv, S, Dp};
            pq = tmp.keep(gt_new_tensor(4, qsh2, gd, GT_DEV_CUDA, dev));
            pk = tmp.keep(gt_new_tensor(4, ksh2, gd, GT_DEV_CUDA, dev));
            pv = tmp.keep(gt_new_tensor(4, ksh2, gd, GT_DEV_CUDA, dev));
            ok = qp && kp && vp && gp && op && pq && pk && pv;
            if (ok) {
                fill_qkv(a.f, qp, kp, vp);
                a.dout = gt_data(gp);
                a.f.o = const_cast<void *>(gt_data(op));
                a.dq = const_cast<void *>(gt_data(pq));
                a.dk = const_cast<void *>(gt_data(pk));
                a.dv = const_cast<void *>(gt_data(pv));
            }
        }
        gt_scratch bits;  // dropout on the MFMA kernels: the dQ kernel's decisions for dK/dV, 1 bit each
        const size_t nbits = (size_t)(B * H * L) * (size_t)((S + 31) / 32) * sizeof(uint32_t);
        // the float32 dK/dV kernel takes dropout only with those bits (it does not draw its own),
        // addressed by 32-bit byte offsets
        const bool f32_drop_ok = cd != GT_F32 || !a.f.dropout || (nbits <= dropout_bits_max() && nbits <= 0xffffffffull);
        if (ok && f32_drop_ok && attn_bwd_mfma_supported(a, cd)) {
            if (a.f.dropout && nbits <= dropout_bits_max()) {
                ok = gt_scratch_alloc(bits, nbits, dev);
                a.dbits = (uint32_t *)bits.ptr();
            }
            if (ok)
                note_launch(std::string("backward mfma ") + dtype_tag(cd) + " D=" + std::to_string(a.f.D) +
                            (cd == GT_F32 && attn_bwd_f32_split(a) ? " split" : ""));
            ok = ok && gt_hip_check(launch_attn_bwd_mfma(a, cd, gt_stream()), "flash_attention_backward kernel");
        } else if (ok) {
            note_launch(std::string("backward generic ") + dtype_tag(cd));
            ok = gt_hip_check(launch_attn_generic_bwd(a, cd, gt_stream()), "flash_attention_backward kernel");
        }
        if (ok && Dp) ok = unpad_heads(pq, gq) && unpad_heads(pk, gk) && unpad_heads(pv, gv);
    }
    if (ok) {
        gq = deliver(gq, host_io);
        gk = deliver(gk, host_io);
        gv = deliver(gv, host_io);
        ok = gq && gk && gv;
    }
    if (!ok) {
        gt_tensor_free(gq);
        gt_tensor_free(gk);
        gt_tensor_free(gv);
        return -1;
    }
    *dq = gq;
    *dk = gk;
    *dv = gv;
    return 0;
}

}  // namespace

extern "C" int gt_flash_attention_backward(const gt_tensor *grad_out, const gt_tensor *q, const gt_tensor *k,
                                           const gt_tensor *v, const gt_tensor *mask, const gt_tensor *out,
                                           const gt_tensor *lse, float scale, int is_causal, gt_tensor **dq,
                                           gt_tensor **dk, gt_tensor **dv) {
    return attention_backward("flash_attention_backward", grad_out, q, k, v, mask, out, lse, scale, is_causal, nullptr,
                              dq, dk, dv);
}

// ---- dropout ------------------------------------------------------------------------------------
// The reference's scaled_dot_product_attention with dropout_p > 0 composes explicit ops
// (gguf_train/nn/functional.py:750-767: scores, softmax, dropout by rand_like(probs) < 1 - p,
// scaled by 1 / (1 - p), then probs.matmul(v)); MultiheadAttention does the same on its explicit
// weights (gguf_train/nn/modules/transformer.py:153-166).  Here the fused kernels take the dropout
// decisions from a counter-based generator instead (gt_philox.h), so the forward, the backward
// and the weights of one (seed, offset) agree element for element without storing a mask.

extern "C" int gt_flash_attention_dropout(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                          const gt_tensor *mask, float scale, int is_causal, double dropout_p,
                                          uint64_t seed, uint64_t offset, gt_tensor **out, gt_tensor **lse,
                                          gt_tensor **out32) {
    const char *who = "flash_attention_dropout";
    if (!out || !lse || !out32) {
        gt_set_error("flash_attention_dropout: out, lse and out32 must not be NULL");
        return -1;
    }
    *out = *lse = *out32 = nullptr;
    Dropout drop;
    if (!make_dropout(who, dropout_p, seed, offset, drop)) return -1;
    return attention_forward(who, q, k, v, mask, scale, is_causal, out, lse, out32, nullptr, &drop);
}

extern "C" int gt_flash_attention_dropout_backward(const gt_tensor *grad_out, const gt_tensor *q, const gt_tensor *k,
                                                   const gt_tensor *v, const gt_tensor *mask, const gt_tensor *out,
                                                   const gt_tensor *lse, float scale, int is_causal, double dropout_p,
                                                   uint64_t seed, uint64_t offset, gt_tensor **dq, gt_tensor **dk,
                                                   gt_tensor **dv) {
    const char *who = "flash_attention_dropout_backward";
    if (dq) *dq = nullptr;
    if (dk) *dk = nullptr;
    if (dv) *dv = nullptr;
    Dropout drop;
    if (!make_dropout(who, dropout_p, seed, offset, drop)) return -1;
    return attention_backward(who, grad_out, q, k, v, mask, out, lse, scale, is_causal, &drop, dq, dk, dv);
}

// The dropout decisions themselves, (B,H,L,S) bool on device `device_index` (1 = kept): the
// elements the dropout kernels of the same (p, seed, offset) keep.
extern "C" gt_tensor *gt_attention_dropout_mask(int64_t B, int64_t H, int64_t L, int64_t S, double dropout_p,
                                                uint64_t seed, uint64_t offset, int device_index) {
    const char *who = "attention_dropout_mask";
    if (B < 0 || H < 0 || L < 0 || S < 0) {
        gt_set_error("attention_dropout_mask: negative dimension");
        return nullptr;
    }
    Dropout drop;
    if (!make_dropout(who, dropout_p, seed, offset, drop)) return nullptr;
    if (!gt_device_ok(device_index)) return nullptr;
    const int64_t sh[4] = {B, H, L, S};
    gt_tensor *m = gt_new_tensor(4, sh, GT_BOOL, GT_DEV_CUDA, device_index);
    if (!m) return nullptr;
    // p = 0: every element kept
    if (!gt_hip_check(launch_dropout_mask(drop.d, !drop.on, B * H * L, S, (uint8_t *)gt_data(m), gt_stream()),
                      "dropout mask kernel")) {
        gt_tensor_free(m);
        return nullptr;
    }
    return m;
}

// ---------------------------------------------------------------------------------------------
// Attention that allocates nothing (no counterpart in the reference)
// ---------------------------------------------------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc): gt_flash_attention into an output the caller owns.
// The only device memory beyond the inputs and the output is the split-K partials of the
// decode kernels, and those live in `scratch`, a fixed array of device memory that each GPU
// the library runs on holds until the process ends.  The decode launch then merges its splits
// with a second kernel (the in-kernel merge of gt_flash_attention needs the uncached
// workspace, which is allocated); every split writes all of its partial rows before the merge
// reads them, so nothing in `scratch` needs clearing between calls.  All calls on one GPU share
// its array: calls that overlap in time on one GPU (different streams, different threads)
// race on it and must be serialised by the caller.  A call that would write it while the last
// call that did, on another stream, has not finished is refused (scratch_claim below); calls on
// one stream are ordered by the stream, and streams under graph capture are not checked.

namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// Device address of this GPU's `scratch` (the name is a host-side stand-in in host code), looked
// up once per device with that device current; null with the error set on failure.
char *noalloc_scratch(int dev) {
    static std::mutex mu;
    static std::vector<char *> ptrs;
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)dev >= ptrs.size()) ptrs.resize((size_t)dev + 1, nullptr);
    if (!ptrs[(size_t)dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            gt_set_error(std::string("flash_attention_noalloc: hipGetSymbolAddress of the scratch array failed: ") +
                         hipGetErrorString(e));
            (void)hipGetLastError();
            return nullptr;
        }
        ptrs[(size_t)dev] = (char *)p;
    }
    return ptrs[(size_t)dev];
}

bool on_device(const gt_tensor *t, int dev) { return t->device_type == GT_DEV_CUDA && t->device_index == dev; }

// Overlap detection for the calls that use `scratch`: the last such call's stream and an event
// recorded after its launches, per device.  A call on another stream while that event is still
// pending would race on the array, so it is refused.  (Calls on one stream are ordered by the
// stream; a stream under graph capture is not checked: its launches run when the graph does.)
struct ScratchUse {
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;
    bool used = false;
};

std::mutex g_scratch_mu;
std::vector<ScratchUse> g_scratch_use;

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return st != hipStreamCaptureStatusNone;
}

// Before a launch into `scratch` on the current stream: false (error set) when the previous
// such launch, on another stream, may still be running.  On success `held` keeps the lock until
// scratch_release has recorded this call's launches, so that two threads cannot both pass the
// check before either has launched.
bool scratch_claim(const char *who, int dev, std::unique_lock<std::mutex> &held) {
    const hipStream_t s = gt_stream();
    if (capturing(s)) return true;
    held = std::unique_lock<std::mutex>(g_scratch_mu);
    if ((size_t)dev >= g_scratch_use.size()) g_scratch_use.resize((size_t)dev + 1);
    ScratchUse &u = g_scratch_use[(size_t)dev];
    if (u.used && u.stream != s) {
        const hipError_t e = hipEventQuery(u.done);
        if (e == hipErrorNotReady) {
            (void)hipGetLastError();
            gt_set_error(std::string(who) + ": a call on another stream that uses this GPU's scratch array may still "
                         "be running; calls that overlap in time on one GPU race on it (serialise them)");
            return false;
        }
        if (e != hipSuccess) (void)hipGetLastError();
    }
    return true;
}

// After the launches: records where the scratch array was last written, then lets the next
// claim in (the lock taken by scratch_claim; none under graph capture).
void scratch_release(int dev, std::unique_lock<std::mutex> &held) {
    if (!held.owns_lock()) return;
    const hipStream_t s = gt_stream();
    std::unique_lock<std::mutex> lock(std::move(held));
    ScratchUse &u = g_scratch_use[(size_t)dev];
    if (!u.done && hipEventCreateWithFlags(&u.done, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        u.done = nullptr;
        u.used = false;
        return;
    }
    if (hipEventRecord(u.done, s) != hipSuccess) {
        (void)hipGetLastError();
        u.used = false;
        return;
    }
    u.stream = s;
    u.used = true;
}

}  // namespace

extern "C" int gt_flash_attention_noalloc(const gt_tensor *q, const gt_tensor *k, const gt_tensor *v,
                                          const gt_tensor *mask, float scale, int is_causal, gt_tensor *out) {
    const char *who = "flash_attention_noalloc";
    LaunchScope scope;
    if (!validate(who, q, k, v, mask)) return -1;
    const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], D = q->shape[3], Dv = v->shape[3];
    const int dev = q->device_type == GT_DEV_CUDA ? q->device_index : 0;
    for (const gt_tensor *t : {q, k, v, mask, (const gt_tensor *)out}) {
        if (t && !on_device(t, dev)) {
            gt_set_error(std::string(who) + ": q, k, v, mask and out must all be on HIP device " + std::to_string(dev) +
                         " (nothing is staged: staging would allocate)");
            return -1;
        }
    }
    if (!out || out->ndim != 4 || out->shape[0] != B || out->shape[1] != H || out->shape[2] != L ||
        out->shape[3] != Dv || out->dtype != q->dtype || !gt_is_dense(out)) {
        gt_set_error(std::string(who) + ": out must be a dense (B, H, L, Dv) = [" + std::to_string(B) + ", " +
                     std::to_string(H) + ", " + std::to_string(L) + ", " + std::to_string(Dv) + "] tensor of q's dtype");
        return -1;
    }
    const bool q8 = k->dtype == GT_Q8_0 || v->dtype == GT_Q8_0;
    if (q8 && !(k->dtype == GT_Q8_0 && v->dtype == GT_Q8_0 && q->dtype == GT_F16 && L == 1)) {
        gt_set_error(std::string(who) + ": q8_0 k/v need float16 q with one query row (L = 1); other q8_0 "
                     "calls dequantize, which allocates");
        return -1;
    }
    const int cd = q8 ? GT_F16 : q->dtype;
    if (!q8 && (k->dtype != cd || v->dtype != cd)) {
        gt_set_error(std::string(who) + ": q, k and v must have one dtype (converting them would allocate), got " +
                     gt_dtype_name(q->dtype) + ", " + gt_dtype_name(k->dtype) + ", " + gt_dtype_name(v->dtype));
        return -1;
    }
    for (const gt_tensor *t : {q, k, v}) {
        if (t->dtype != GT_Q8_0 && !inner_contiguous(t)) {
            gt_set_error(std::string(who) + ": q, k and v need a contiguous innermost dimension (a copy would allocate)");
            return -1;
        }
    }
    const int mask_want = cd == GT_F64 ? GT_F64 : GT_F32;
    if (mask && mask->dtype != GT_BOOL && mask->dtype != mask_want) {
        gt_set_error(std::string(who) + ": the mask must be bool or " + gt_dtype_name(mask_want) + " (got " +
                     gt_dtype_name(mask->dtype) + "; converting it would allocate)");
        return -1;
    }
    if (!gt_device_ok(dev)) return -1;
    if (scale <= 0.0f) scale = 1.0f / std::sqrt((float)D);  // csrc/gt_ops_nn.cpp:2433
    if (out->numel == 0) return 0;

    AttnFwdArgs a{};
    fill_qkv(a, q, k, v);
    a.o = gt_data(out);
    a.scale = scale;
    a.causal = is_causal ? 1 : 0;
    a.out_dtype = q->dtype;
    if (mask) {
        // read in place through broadcast strides (a bool mask as bytes, not turned into a bias)
        int64_t st[4] = {0, 0, 0, 0}, sh[4] = {1, 1, 1, 1};
        for (int i = 0; i < mask->ndim; ++i) {
            sh[4 - mask->ndim + i] = mask->shape[i];
            st[4 - mask->ndim + i] = mask->strides[i];
        }
        a.mask = gt_data(mask);
        a.mask_bool = mask->dtype == GT_BOOL;
        a.m_sb = sh[0] == 1 ? 0 : st[0];
        a.m_sh = sh[1] == 1 ? 0 : st[1];
        a.m_sl = sh[2] == 1 ? 0 : st[2];
        a.m_ss = sh[3] == 1 ? 0 : st[3];
    }

    const bool dec = q8 ? attn_decode_q8_supported(a, GT_F16) : attn_decode_supported(a, cd);
    if (q8 && !dec) {
        gt_set_error(std::string(who) + ": these q8_0 shapes need the dequantizing path, which allocates");
        return -1;
    }
    if (dec) {
        DecodeArgs da{};
        da.f = a;
        da.nsplit = q8 ? attn_decode_q8_splits(a) : attn_decode_splits(a, cd);
        da.counters = nullptr;  // splits merged by a second launch
        // partials: (B*H, nsplit, D) outputs then (B*H, nsplit, 2) (max, sum); the streaming
        // kernels write the output themselves when there is one split
        const bool partials = da.nsplit > 1 || (!q8 && D > 128);
        std::unique_lock<std::mutex> held;  // the scratch check's lock, until the launch is recorded
        if (partials) {
            const size_t rows = (size_t)(B * H) * (size_t)da.nsplit;
            const size_t need = rows * (size_t)(D + 2) * sizeof(float);
            if (need > kNoAllocScratchBytes) {
                gt_set_error(std::string(who) + ": the split partials of this call need " + std::to_string(need) +
                             " bytes, more than the " + std::to_string(kNoAllocScratchBytes) +
                             "-byte scratch array (B*H*splits*(D+2)*4 bytes); use gt_flash_attention");
                return -1;
            }
            char *base = noalloc_scratch(dev);
            if (!base || !scratch_claim(who, dev, held)) return -1;
            da.part_o = (float *)base;
            da.part_ml = da.part_o + rows * (size_t)D;
        }
        note_launch(q8 ? decode_note("decode q8_0", da, kDecodeQ8MaxTile)
                       : decode_note((std::string("decode ") + dtype_tag(cd)).c_str(), da, attn_decode_max_tile(cd)));
        const hipError_t e = q8 ? launch_attn_decode_q8(da, gt_stream()) : launch_attn_decode(da, cd, gt_stream());
        if (partials) scratch_release(dev, held);
        return gt_hip_check(e, "flash_attention_noalloc decode kernel") ? 0 : -1;
    }
    if (attn_prefill_supported(a, cd)) {
        note_launch(prefill_note(a, cd));
        return gt_hip_check(launch_attn_prefill(a, cd, gt_stream()), "flash_attention_noalloc prefill kernel") ? 0 : -1;
    }
    note_launch(std::string("generic ") + dtype_tag(cd));
    return gt_hip_check(launch_attn_generic_fwd(a, cd, gt_stream()), "flash_attention_noalloc kernel") ? 0 : -1;
}

// ---------------------------------------------------------------------------------------------
// Q8_0 codec (csrc/gt_ops_extra.cpp:2002-2009 -> csrc/gt_core.cpp:784-847)
// ---------------------------------------------------------------------------------------------

extern "C" gt_tensor *gt_quantize(const gt_tensor *t, int ggml_type_id) {
    if (!t) {
        gt_set_error("quantize: NULL tensor");
        return nullptr;
    }
    if (ggml_type_id != GT_Q8_0 - GT_Q_BASE) {
        gt_set_error("quantize: only q8_0 (ggml type 8) is supported, got ggml type " + std::to_string(ggml_type_id));
        return nullptr;
    }
    if (gt_is_quantized(t->dtype)) {
        gt_set_error("quantize: the tensor is already quantized");
        return nullptr;
    }
    if (t->numel % 32 != 0) {
        gt_set_error("Tensor size must be a multiple of ggml quantization block size");
        return nullptr;
    }
    const int dev = t->device_type == GT_DEV_CUDA ? t->device_index : 0;
    if (!gt_device_ok(dev)) return nullptr;
    Temps tmp;
    const gt_tensor *f = (t->device_type == GT_DEV_CUDA && t->dtype == GT_F32 && gt_is_dense(t))
                             ? t
                             : tmp.keep(gt_to_device_dense(t, dev, GT_F32));
    if (!f) return nullptr;
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, GT_Q8_0, GT_DEV_CUDA, dev);
    if (!out) return nullptr;
    if (!gt_hip_check(gt_launch_q8_0_quantize((const float *)gt_data(f), gt_data(out), t->numel / 32, gt_stream()),
                      "q8_0 quantize kernel")) {
        gt_tensor_free(out);
        return nullptr;
    }
    return deliver(out, t->device_type != GT_DEV_CUDA);
}

extern "C" gt_tensor *gt_dequantize(const gt_tensor *t, int out_dtype) {
    if (!t) {
        gt_set_error("dequantize: NULL tensor");
        return nullptr;
    }
    if (t->dtype != GT_Q8_0) {
        gt_set_error(std::string("dequantize: expected a q8_0 tensor, got ") + gt_dtype_name(t->dtype));
        return nullptr;
    }
    if (out_dtype != GT_F32 && out_dtype != GT_F16 && out_dtype != GT_BF16 && out_dtype != GT_F64) {
        gt_set_error(std::string("dequantize: unsupported output dtype ") + gt_dtype_name(out_dtype));
        return nullptr;
    }
    const int dev = t->device_type == GT_DEV_CUDA ? t->device_index : 0;
    if (!gt_device_ok(dev)) return nullptr;
    Temps tmp;
    const gt_tensor *src = t->device_type == GT_DEV_CUDA ? t : tmp.keep(gt_to_device_dense(t, dev, GT_Q8_0));
    if (!src) return nullptr;
    gt_tensor *out = gt_new_tensor(t->ndim, t->shape, out_dtype, GT_DEV_CUDA, dev);
    if (!out) return nullptr;
    if (!gt_hip_check(gt_launch_q8_0_dequantize(gt_data(src), gt_data(out), out_dtype, t->numel / 32, gt_stream()),
                      "q8_0 dequantize kernel")) {
        gt_tensor_free(out);
        return nullptr;
    }
    return deliver(out, t->device_type != GT_DEV_CUDA);
}

// ---- explicit attention weights ----------------------------------------------------------------
// MultiheadAttention(need_weights=True) in the reference materialises softmax(q.k^T*scale +
// masks) with ggml ops (gguf_train/nn/modules/transformer.py:153-166).  Here the fused forward
// gives the output and the log-sum-exp; this entry point recomputes the weights from them.

namespace {

gt_tensor *attention_weights(const gt_tensor *q, const gt_tensor *k, const gt_tensor *mask, const gt_tensor *lse,
                             float scale, int is_causal, int average_heads, const Dropout *drop) {
    LaunchScope scope;
    if (!validate("attention_weights", q, k, k, mask)) return nullptr;
    if (!lse || lse->ndim != 3 || lse->shape[0] != q->shape[0] || lse->shape[1] != q->shape[1] ||
        lse->shape[2] != q->shape[2]) {
        gt_set_error("attention_weights: lse must be (B, H, L), the log-sum-exp of the same forward");
        return nullptr;
    }
    if (k->dtype == GT_Q8_0) {
        gt_set_error("attention_weights: q8_0 keys are not supported (dequantize them first)");
        return nullptr;
    }
    const int dev = q->device_type == GT_DEV_CUDA ? q->device_index : 0;
    if (!gt_device_ok(dev)) return nullptr;
    const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], D = q->shape[3], S = k->shape[2];
    if (scale <= 0.0f) scale = 1.0f / std::sqrt((float)D);
    const int cd = compute_dtype(q, k, k);
    Temps tmp;
    const gt_tensor *qs = stage(q, dev, cd, tmp), *ks = stage(k, dev, cd, tmp);
    const int ld = cd == GT_F64 ? GT_F64 : GT_F32;
    const gt_tensor *ls = lse->device_type == GT_DEV_CUDA && lse->device_index == dev && lse->dtype == ld && gt_is_dense(lse) &&
                                  lse->offset == 0
                              ? lse
                              : tmp.keep(gt_to_device_dense(lse, dev, ld));
    if (!qs || !ks || !ls) return nullptr;
    AttnFwdArgs a{};
    fill_qkv(a, qs, ks, ks);
    if (!stage_mask(mask, dev, cd, a, tmp)) return nullptr;
    a.lse = gt_data(ls);
    a.scale = scale;
    a.causal = is_causal ? 1 : 0;
    a.out_dtype = q->dtype;
    apply_dropout(a, drop);
    const int64_t wsh4[4] = {B, H, L, S}, wsh3[3] = {B, L, S};
    gt_tensor *w = average_heads ? gt_new_tensor(3, wsh3, q->dtype, GT_DEV_CUDA, dev)
                                 : gt_new_tensor(4, wsh4, q->dtype, GT_DEV_CUDA, dev);
    if (!w) return nullptr;
    note_launch(std::string("weights ") + (attn_weights_mfma(a, cd) ? "mfma " : "generic ") + dtype_tag(cd) +
                " D=" + std::to_string(D));
    if (!gt_hip_check(launch_attn_weights(a, cd, gt_data(w), average_heads != 0, gt_stream()),
                      "attention weights kernel")) {
        gt_tensor_free(w);
        return nullptr;
    }
    return deliver(w, q->device_type != GT_DEV_CUDA);
}

}  // namespace

extern "C" gt_tensor *gt_attention_weights(const gt_tensor *q, const gt_tensor *k, const gt_tensor *mask,
                                           const gt_tensor *lse, float scale, int is_causal, int average_heads) {
    return attention_weights(q, k, mask, lse, scale, is_causal, average_heads, nullptr);
}

extern "C" gt_tensor *gt_attention_weights_dropout(const gt_tensor *q, const gt_tensor *k, const gt_tensor *mask,
                                                   const gt_tensor *lse, float scale, int is_causal, int average_heads,
                                                   double dropout_p, uint64_t seed, uint64_t offset) {
    Dropout drop;
    if (!make_dropout("attention_weights_dropout", dropout_p, seed, offset, drop)) return nullptr;
    return attention_weights(q, k, mask, lse, scale, is_causal, average_heads, &drop);
}

// ---- KV cache --------------------------------------------------------------------------------
// The per-sequence K/V store of a decoding loop.  In the reference it is llama.cpp's cache
// behind LlamaContext.forward_logits (csrc/llama_bridge.cpp:245-296, gguf_train/llama/__init__.py:
// 174-190): tokens are appended at the positions that continue what a sequence holds
// (pos_offset), the context has a fixed capacity (n_ctx), clear_kv() empties it, and a query
// attends to its own position and everything before it.  Here the cache lives in HBM as dense
// (B, Hkv, capacity, D) tensors, float16/bfloat16/float32 or GGUF Q8_0 (quantized on append
// with the same steps as gt_quantize), with per-sequence lengths; attention over it runs the
// same kernels as gt_flash_attention, given each sequence's length and query position.

struct gt_kv_cache {
    int64_t B = 0, Hkv = 0, cap = 0, D = 0;
    int dtype = GT_F16;
    int dev = 0;
    gt_tensor *k = nullptr, *v = nullptr;  // (B, Hkv, cap, D), zero-filled at creation
    std::vector<int32_t> len;              // tokens held per sequence (the authoritative copy)
    gt_tensor *len_dev = nullptr;          // device copy of len (int32, B)
    gt_tensor *pos_dev = nullptr;          // position of query row 0 per sequence (int32, B)
};

namespace {

bool kv_upload(gt_tensor *dst, const std::vector<int32_t> &src) {
    // pageable source: returns once the bytes are staged, so `src` may change afterwards
    return gt_hip_check(hipMemcpyAsync(gt_data(dst), src.data(), src.size() * sizeof(int32_t), hipMemcpyHostToDevice,
                                       gt_stream()),
                        "kv cache: length upload");
}

bool kv_zero(gt_tensor *t) {
    return gt_hip_check(gt_launch_fill_zero(gt_data(t), (int64_t)gt_dtype_nbytes(t->dtype, t->numel), gt_stream()),
                        "kv cache: zero fill");
}

bool kv_check_rows(const char *who, const gt_kv_cache *c, const gt_tensor *t, const char *name) {
    if (!t || t->ndim != 4) {
        gt_set_error(std::string(who) + ": " + name + " must be a 4-D tensor (B, Hkv, T, D)");
        return false;
    }
    if (t->shape[0] != c->B || t->shape[1] != c->Hkv || t->shape[3] != c->D || t->shape[2] < 1) {
        gt_set_error(std::string(who) + ": " + name + " of shape [" + std::to_string(t->shape[0]) + ", " +
                     std::to_string(t->shape[1]) + ", " + std::to_string(t->shape[2]) + ", " +
                     std::to_string(t->shape[3]) + "] does not match the cache [" + std::to_string(c->B) + ", " +
                     std::to_string(c->Hkv) + ", T, " + std::to_string(c->D) + "]");
        return false;
    }
    if (t->dtype == GT_Q8_0) {
        // Q8_0 rows (e.g. read from a GGUF file): whole blocks along head_dim
        if (c->D % 32 != 0 || !gt_is_dense(t) || t->offset != 0) {
            gt_set_error(std::string(who) + ": a q8_0 " + name + " must be dense with head_dim a multiple of 32");
            return false;
        }
        return true;
    }
    if (!gt_is_float(t->dtype)) {
        gt_set_error(std::string(who) + ": " + name + " must be float32, float16, bfloat16, float64 or q8_0, got " +
                     gt_dtype_name(t->dtype));
        return false;
    }
    return true;
}

}  // namespace

extern "C" gt_kv_cache *gt_kv_cache_create(int64_t batch, int64_t n_head_kv, int64_t capacity, int64_t head_dim,
                                           int dtype, int device_index) {
    gt_init();
    if (batch < 1 || n_head_kv < 1 || capacity < 1 || head_dim < 1) {
        gt_set_error("kv_cache_create: batch, n_head_kv, capacity and head_dim must be positive");
        return nullptr;
    }
    if (dtype != GT_F32 && dtype != GT_F16 && dtype != GT_BF16 && dtype != GT_Q8_0) {
        gt_set_error(std::string("kv_cache_create: dtype must be float32, float16, bfloat16 or q8_0, got ") +
                     gt_dtype_name(dtype));
        return nullptr;
    }
    if (dtype == GT_Q8_0 && head_dim % 32 != 0) {
        gt_set_error("kv_cache_create: a q8_0 cache needs a head_dim that is a multiple of 32, got " +
                     std::to_string(head_dim));
        return nullptr;
    }
    if (capacity >= (1LL << 30)) {
        gt_set_error("kv_cache_create: capacity must be below 2^30");
        return nullptr;
    }
    if (!gt_device_ok(device_index)) return nullptr;
    auto *c = new gt_kv_cache();
    c->B = batch;
    c->Hkv = n_head_kv;
    c->cap = capacity;
    c->D = head_dim;
    c->dtype = dtype;
    c->dev = device_index;
    c->len.assign((size_t)batch, 0);
    const int64_t sh[4] = {batch, n_head_kv, capacity, head_dim}, lsh[1] = {batch};
    c->k = gt_new_tensor(4, sh, dtype, GT_DEV_CUDA, device_index);
    c->v = c->k ? gt_new_tensor(4, sh, dtype, GT_DEV_CUDA, device_index) : nullptr;
    c->len_dev = c->v ? gt_new_tensor(1, lsh, GT_I32, GT_DEV_CUDA, device_index) : nullptr;
    c->pos_dev = c->len_dev ? gt_new_tensor(1, lsh, GT_I32, GT_DEV_CUDA, device_index) : nullptr;
    // rows past a sequence's length are read (and weighted 0) by the kernels: keep them finite
    if (!c->pos_dev || !kv_zero(c->k) || !kv_zero(c->v) || !kv_upload(c->len_dev, c->len) ||
        !kv_upload(c->pos_dev, c->len)) {
        gt_kv_cache_free(c);
        return nullptr;
    }
    return c;
}

extern "C" void gt_kv_cache_free(gt_kv_cache *c) {
    if (!c) return;
    gt_tensor_free(c->k);
    gt_tensor_free(c->v);
    gt_tensor_free(c->len_dev);
    gt_tensor_free(c->pos_dev);
    delete c;
}

extern "C" int gt_kv_cache_clear(gt_kv_cache *c, int64_t seq) {
    if (!c) {
        gt_set_error("kv_cache_clear: NULL cache");
        return -1;
    }
    if (seq >= c->B) {
        gt_set_error("kv_cache_clear: sequence " + std::to_string(seq) + " out of range for " + std::to_string(c->B) +
                     " sequences");
        return -1;
    }
    if (seq < 0) std::fill(c->len.begin(), c->len.end(), 0);
    else c->len[(size_t)seq] = 0;
    return kv_upload(c->len_dev, c->len) ? 0 : -1;
}

extern "C" int64_t gt_kv_cache_length(const gt_kv_cache *c, int64_t seq) {
    if (!c || seq < 0 || seq >= c->B) {
        gt_set_error("kv_cache_length: invalid cache or sequence");
        return -1;
    }
    return c->len[(size_t)seq];
}

extern "C" int64_t gt_kv_cache_capacity(const gt_kv_cache *c) { return c ? c->cap : -1; }

extern "C" gt_tensor *gt_kv_cache_keys(const gt_kv_cache *c) {
    if (!c) {
        gt_set_error("kv_cache_keys: NULL cache");
        return nullptr;
    }
    auto *t = new gt_tensor(*c->k);  // shares the storage
    return t;
}

extern "C" gt_tensor *gt_kv_cache_values(const gt_kv_cache *c) {
    if (!c) {
        gt_set_error("kv_cache_values: NULL cache");
        return nullptr;
    }
    auto *t = new gt_tensor(*c->v);
    return t;
}

namespace {

struct KvRope {
    int n_dims, mode;
    float freq_base, freq_scale;
};

// Appends k/v rows at each sequence's length; with `rope` the key rows are rotated at their cache
// positions (length + t) on the way in.
int kv_append(const char *who, gt_kv_cache *c, const gt_tensor *k, const gt_tensor *v, int64_t pos_offset,
              const KvRope *rope) {
    if (!c) {
        gt_set_error(std::string(who) + ": NULL cache");
        return -1;
    }
    if (!kv_check_rows(who, c, k, "k") || !kv_check_rows(who, c, v, "v")) return -1;
    if (rope && !gt_rope_check_args(who, c->D, rope->n_dims, rope->mode, rope->freq_base, rope->freq_scale)) return -1;
    const int64_t T = k->shape[2];
    if (v->shape[2] != T) {
        gt_set_error("kv_cache_append: k and v hold different numbers of tokens (" + std::to_string(T) + " and " +
                     std::to_string(v->shape[2]) + ")");
        return -1;
    }
    for (int64_t b = 0; b < c->B; ++b) {
        const int64_t n = c->len[(size_t)b];
        const int64_t p0 = pos_offset < 0 ? n : pos_offset;
        if (pos_offset >= 0 && pos_offset != n) {
            gt_set_error("kv_cache_append: positions " + std::to_string(p0) + ".." + std::to_string(p0 + T - 1) +
                         " do not continue what sequence " + std::to_string(b) + " holds (" + std::to_string(n) +
                         " tokens; see kv_cache_clear)");
            return -1;
        }
        if (p0 + T > c->cap) {
            gt_set_error("kv_cache_append: positions " + std::to_string(p0) + ".." + std::to_string(p0 + T - 1) +
                         " of sequence " + std::to_string(b) + " do not fit the cache (capacity = " +
                         std::to_string(c->cap) + ")");
            return -1;
        }
    }
    if (!gt_device_ok(c->dev)) return -1;
    Temps tmp;
    const int32_t *pos = (const int32_t *)gt_data(c->len_dev);
    gt_scratch table;
    gt_rope_apply ra{};
    if (rope && T > 0) {
        // (cos, sin) of table row b * T + t at position len[b] + t
        if (!gt_scratch_alloc(table, (size_t)(c->B * T) * (size_t)(rope->n_dims / 2) * 2 * sizeof(float), c->dev) ||
            !gt_hip_check(gt_launch_rope_table(nullptr, pos, T, c->B * T, rope->n_dims,
                                               gt_rope_theta_scale(rope->freq_base, rope->n_dims), rope->freq_scale, 0,
                                               table.ptr(), gt_stream()),
                          "rope table kernel"))
            return -1;
        ra.table = table.ptr();
        ra.n_dims = rope->n_dims;
        ra.neox = rope->mode == 2;
    }
    for (const gt_tensor *src : {k, v}) {
        const bool rotate = rope && src == k;
        const gt_tensor *s = src->device_type == GT_DEV_CUDA && src->device_index == c->dev
                                 ? src
                                 : tmp.keep(gt_to_device_dense(src, c->dev, -1));
        if (!s) return -1;
        // Q8_0 rows go into a Q8_0 cache unchanged; a float cache takes their dequantized values,
        // and so do rotated keys (rotated, then quantized again for a Q8_0 cache)
        if (s->dtype == GT_Q8_0 && (c->dtype != GT_Q8_0 || rotate) && !(s = tmp.keep(gt_dequantize(s, GT_F32))))
            return -1;
        gt_tensor *dst = src == k ? c->k : c->v;
        // the rows go to each sequence's current length (len_dev), before it is advanced
        const hipError_t e =
            s->dtype == GT_Q8_0
                ? gt_launch_kv_append_blocks(gt_data(s), gt_data(dst), pos, c->B, c->Hkv, T, c->D, c->cap, gt_stream())
                : gt_launch_kv_append(gt_data(s), s->dtype, s->strides, gt_data(dst), c->dtype, pos, c->B, c->Hkv, T,
                                      c->D, c->cap, rotate && T > 0 ? &ra : nullptr, gt_stream());
        if (!gt_hip_check(e, "kv cache append kernel")) return -1;
    }
    for (auto &n : c->len) n += (int32_t)T;
    return kv_upload(c->len_dev, c->len) ? 0 : -1;
}

}  // namespace

extern "C" int gt_kv_cache_append(gt_kv_cache *c, const gt_tensor *k, const gt_tensor *v, int64_t pos_offset) {
    return kv_append("kv_cache_append", c, k, v, pos_offset, nullptr);
}

extern "C" int gt_kv_cache_append_rope(gt_kv_cache *c, const gt_tensor *k, const gt_tensor *v, int64_t pos_offset,
                                       int n_dims, int mode, float freq_base, float freq_scale) {
    const KvRope r{n_dims, mode, freq_base, freq_scale};
    return kv_append("kv_cache_append_rope", c, k, v, pos_offset, &r);
}

extern "C" gt_tensor *gt_kv_cache_attention(gt_kv_cache *c, const gt_tensor *q, float scale, int is_causal) {
    LaunchScope scope;
    if (!c) {
        gt_set_error("kv_cache_attention: NULL cache");
        return nullptr;
    }
    if (!q || q->ndim != 4 || q->shape[0] != c->B || q->shape[3] != c->D || q->shape[1] < 1 ||
        q->shape[1] % c->Hkv != 0) {
        gt_set_error("kv_cache_attention: q must be (B, H, L, D) with B = " + std::to_string(c->B) + ", D = " +
                     std::to_string(c->D) + " and H a multiple of " + std::to_string(c->Hkv));
        return nullptr;
    }
    if (!gt_is_float(q->dtype)) {
        gt_set_error(std::string("kv_cache_attention: q must be a float tensor, got ") + gt_dtype_name(q->dtype));
        return nullptr;
    }
    const int64_t B = c->B, H = q->shape[1], L = q->shape[2], D = c->D;
    // query row l of sequence b is token len[b] - L + l
    std::vector<int32_t> pos((size_t)B);
    int64_t maxlen = 0;
    for (int64_t b = 0; b < B; ++b) {
        const int64_t n = c->len[(size_t)b];
        if (n < L) {
            gt_set_error("kv_cache_attention: sequence " + std::to_string(b) + " holds " + std::to_string(n) +
                         " tokens, fewer than the " + std::to_string(L) + " query rows (append them first)");
            return nullptr;
        }
        pos[(size_t)b] = (int32_t)(n - L);
        maxlen = std::max<int64_t>(maxlen, n);
    }
    if (scale <= 0.0f) scale = 1.0f / std::sqrt((float)D);
    const int dev = c->dev;
    if (!gt_device_ok(dev) || !kv_upload(c->pos_dev, pos)) return nullptr;
    const int32_t *kv_len = (const int32_t *)gt_data(c->len_dev), *q_pos = (const int32_t *)gt_data(c->pos_dev);
    const bool host_io = q->device_type != GT_DEV_CUDA;
    const int64_t osh[4] = {B, H, L, D};
    gt_tensor *o = gt_new_tensor(4, osh, q->dtype, GT_DEV_CUDA, dev);
    if (!o) return nullptr;
    Temps tmp;
    bool ok = true;
    int q8 = 0;
    if (o->numel > 0 && c->dtype == GT_Q8_0 && q->dtype == GT_F16 && L == 1) {
        q8 = run_q8_decode(q, c->k, c->v, nullptr, scale, is_causal, dev, o, nullptr, tmp, kv_len, q_pos);
        ok = q8 >= 0;
    }
    if (ok && q8 == 0 && o->numel > 0) {
        // the float cache is read in place through a view of its first maxlen rows; of a Q8_0
        // cache only those rows are dequantized, to float16 for float16 queries (the MFMA
        // kernels run) or to float32 / float64 (exact values), as gt_flash_attention does
        const gt_tensor *kv_views[2] = {nullptr, nullptr};
        const int64_t vsh[4] = {B, c->Hkv, maxlen, D};
        if (c->dtype == GT_Q8_0) {
            const int kd = q->dtype == GT_F16 ? GT_F16 : q->dtype == GT_F64 ? GT_F64 : GT_F32;
            note_launch("dequantize q8_0 cache rows");
            for (int i = 0; i < 2 && ok; ++i) {
                gt_tensor *d = tmp.keep(gt_new_tensor(4, vsh, kd, GT_DEV_CUDA, dev));
                const int64_t rb = D / 32;  // blocks per row
                ok = d && gt_hip_check(gt_launch_q8_0_dequantize_rows(gt_data(i == 0 ? c->k : c->v), gt_data(d), kd,
                                                                      B * c->Hkv * maxlen * rb, maxlen * rb,
                                                                      c->cap * rb, gt_stream()),
                                       "q8_0 dequantize kernel");
                kv_views[i] = ok ? d : nullptr;
            }
        } else {
            for (int i = 0; i < 2; ++i) {
                const gt_tensor *base = i == 0 ? c->k : c->v;
                kv_views[i] = tmp.keep(gt_tensor_view(base, 4, vsh, base->strides, base->offset));
            }
        }
        const gt_tensor *kv = kv_views[0], *vv = kv_views[1];
        ok = kv && vv;
        const int cd = ok ? compute_dtype(q, kv, vv) : GT_F32;
        const gt_tensor *qs = ok ? stage(q, dev, cd, tmp) : nullptr;
        const gt_tensor *ks = ok ? stage(kv, dev, cd, tmp) : nullptr;
        const gt_tensor *vs = ok ? stage(vv, dev, cd, tmp) : nullptr;
        ok = qs && ks && vs;
        // heads padded to the MFMA kernels' sizes (the cache's first maxlen rows are copied)
        const gt_tensor *po = nullptr;
        const int64_t Dp = ok && q->dtype == cd ? padded_head(cd, L, D, D) : 0;
        if (Dp) {
            const gt_tensor *qp = pad_heads(qs, Dp, dev, tmp), *kp = pad_heads(ks, Dp, dev, tmp);
            const gt_tensor *vp = pad_heads(vs, Dp, dev, tmp);
            const int64_t psh[4] = {B, H, L, Dp};
            po = tmp.keep(gt_new_tensor(4, psh, q->dtype, GT_DEV_CUDA, dev));
            ok = qp && kp && vp && po;
            if (ok) {
                qs = qp;
                ks = kp;
                vs = vp;
            }
        }
        if (ok) {
            AttnFwdArgs a{};
            fill_qkv(a, qs, ks, vs);
            a.o = const_cast<void *>(gt_data(po ? po : o));
            a.scale = scale;
            a.causal = is_causal ? 1 : 0;
            a.out_dtype = q->dtype;
            a.kv_len = kv_len;
            a.q_pos = q_pos;
            ok = dispatch_forward(a, cd, dev);
            if (ok && po) ok = unpad_heads(po, o);
        }
    }
    if (!ok) {
        gt_tensor_free(o);
        return nullptr;
    }
    return deliver(o, host_io);
}
