/*
 * oracle_attn.c - CPU ORACLE.  TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, float64 restatement of GGUF_train's attention path, the parity reference for the
 * HIP library.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only to check or to time the CPU baseline; the library never calls it and has no CPU
 * compute path.
 *
 * Functions and the reference code each one follows:
 *   oracle_read_f64 / oracle_write_f64   csrc/gt_internal.h:243-277 (per-element dtype reads;
 *                                        writes go double -> float -> half/bfloat16)
 *   oracle_f32_to_f16 / _f16_to_f32      IEEE binary16, round to nearest even (ggml's
 *   oracle_f32_to_bf16 / _bf16_to_f32    fp16/bf16 helpers used by the lines above)
 *   oracle_flash_attention               csrc/gt_ops_nn.cpp:2423-2525 (gt_flash_attention)
 *   oracle_flash_attention_backward      gguf_train/_functions.py:1933-1965
 *                                        (FlashAttentionFn.backward) in float64
 *   oracle_q8_0_quantize / _dequantize   csrc/gt_core.cpp:800-832 -> ggml quantize_row_q8_0_ref
 *                                        and dequantize_row_q8_0 (ggml @ f3b407ca, tag b12283,
 *                                        not vendored: restated from its published algorithm)
 *   oracle_rope                          csrc/gt_ops_nn.cpp:2298-2421 -> ggml_rope_ext(_back)
 *                                        (same ggml, restated from its published algorithm)
 *   oracle_attention_dropout(_backward)  gguf_train/nn/functional.py:750-767 (the dropout path of
 *                                        scaled_dot_product_attention: scores, -1e9 fills,
 *                                        softmax, probs * keep / (1 - p), .matmul(v)) and its
 *                                        autograd gradients, in float64, for a given keep mask
 *
 * How each is pinned (tests/test_oracle.py): the converters against numpy float16 and torch
 * bfloat16 over every 16-bit pattern and edge values; the forward against the closed form
 * softmax(QK^T*s + M).V computed by torch.float64 on the CPU, hand-computed cases, the
 * fully-masked-row and causal rules, GQA = explicit head repetition; the backward against
 * central finite differences of the forward and against torch.autograd in float64; the Q8_0
 * codec against hand-computed blocks (amax = 127 gives exact integers, d = 0, ties away from
 * zero) and the reference's own accuracy checks (tests/test_numpy_interop.py:443-454); RoPE
 * against the reference's own known-answer test (tests/test_losses_and_rope.py:254-291, the
 * closed form in float64), the closed form at large positions within the float32 angle
 * chain's error bound, position 0 = identity, backward = inverse and adjoint, norm kept, NeoX =
 * NORMAL under the pair permutation, pass-through beyond n_dims (tests/test_oracle_rope.py).
 * The dropout composition against torch.autograd in float64 with the same keep mask, and the
 * keep mask's generator (Philox4x32-10, oracle/__init__.py) against the Random123 known answers
 * and rocRAND's engine (tests/golden/philox4x32_10.json).
 * Parity unpinned: the byte output of ggml_quantize_chunk itself (ggml cannot be built here),
 * bfloat16 results whose magnitude is below 2^-126 (ggml versions differ on flushing them).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype codes of csrc/gguf_train.h:22-36 */
enum { O_F32 = 0, O_F16 = 1, O_BF16 = 2, O_F64 = 3, O_I8 = 4, O_U8 = 5, O_I16 = 6, O_I32 = 7, O_I64 = 8, O_BOOL = 9 };

static uint32_t f_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float bits_f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even; overflow -> inf; NaN stays NaN. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mag = x & 0x7fffffffu;
    int32_t e = (int32_t)(mag >> 23) - 127; /* unbiased exponent */
    uint32_t mant = mag & 0x7fffffu;
    if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | (mant >> 13));
    if (mag == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    if (mag == 0) return (uint16_t)sign;
    /* value = 1.mant * 2^e (normal) or mant * 2^-149 (subnormal f32) */
    uint64_t sig;   /* integer significand */
    int32_t exp2v;  /* value = sig * 2^exp2v */
    if ((mag >> 23) == 0) {
        sig = mant;
        exp2v = -149;
    } else {
        sig = (uint64_t)(mant | 0x800000u);
        exp2v = e - 23;
    }
    /* target: half with unit 2^(E-10) for normal E in [-14,15], or 2^-24 for subnormals */
    int32_t E = e;
    if ((mag >> 23) == 0) { /* f32 subnormal: far below half range */
        return (uint16_t)sign;
    }
    int32_t unit_exp = (E < -14) ? -24 : E - 10;
    /* q = sig * 2^(exp2v - unit_exp), rounded to nearest even */
    int32_t sh = unit_exp - exp2v; /* >= 13 for normals */
    uint64_t q, rem, halfw;
    if (sh >= 64) {
        q = 0;
        rem = sig;
        halfw = 0; /* unreachable for finite f32 inputs with E >= -149 */
        (void)rem;
        return (uint16_t)sign;
    }
    q = sig >> sh;
    rem = sig & ((1ull << sh) - 1ull);
    halfw = 1ull << (sh - 1);
    if (rem > halfw || (rem == halfw && (q & 1ull))) q++;
    if (E < -14) {
        /* subnormal half: q counts 2^-24 units; q == 1024 rounds up into the smallest normal */
        return (uint16_t)(sign | (uint32_t)q);
    }
    /* normal: q in [1024, 2048]; 2048 means carry into the next binade */
    if (q == 2048) {
        q = 1024;
        E += 1;
    }
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)(E + 15) << 10) | ((uint32_t)q - 1024u));
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15);
    uint32_t E = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (E == 0) v = ldexpf((float)m, -24);
    else if (E == 31) v = m ? bits_f(0x7fc00000u | (m << 13)) : INFINITY;
    else v = ldexpf((float)(m | 0x400u), (int)E - 25);
    return sign ? -v : v;
}

/* binary32 -> bfloat16, round to nearest even; NaN -> quiet NaN. */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t hi = u >> 16, lo = u & 0xffffu;
    if (lo > 0x8000u || (lo == 0x8000u && (hi & 1u))) hi += 1u;
    return (uint16_t)hi;
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f((uint32_t)b << 16); }

void oracle_f32_to_f16_array(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}
void oracle_f16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f16_to_f32(x[i]);
}
void oracle_f32_to_bf16_array(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}
void oracle_bf16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_bf16_to_f32(x[i]);
}

/* csrc/gt_internal.h:243-259 */
double oracle_read_f64(const void *p, int dtype, int64_t i) {
    switch (dtype) {
        case O_F32: return (double)((const float *)p)[i];
        case O_F64: return ((const double *)p)[i];
        case O_F16: return (double)oracle_f16_to_f32(((const uint16_t *)p)[i]);
        case O_BF16: return (double)oracle_bf16_to_f32(((const uint16_t *)p)[i]);
        case O_I8: return (double)((const int8_t *)p)[i];
        case O_U8: return (double)((const uint8_t *)p)[i];
        case O_I16: return (double)((const int16_t *)p)[i];
        case O_I32: return (double)((const int32_t *)p)[i];
        case O_I64: return (double)((const int64_t *)p)[i];
        case O_BOOL: return ((const uint8_t *)p)[i] ? 1.0 : 0.0;
        default: return 0.0;
    }
}

/* csrc/gt_internal.h:261-277 */
void oracle_write_f64(void *p, int dtype, int64_t i, double v) {
    switch (dtype) {
        case O_F32: ((float *)p)[i] = (float)v; break;
        case O_F64: ((double *)p)[i] = v; break;
        case O_F16: ((uint16_t *)p)[i] = oracle_f32_to_f16((float)v); break;
        case O_BF16: ((uint16_t *)p)[i] = oracle_f32_to_bf16((float)v); break;
        default: break;
    }
}

/* Mask element for (b, h, l, s) of a dense mask of mask_ndim (2 or 4) dims, each 1 or full:
 * csrc/gt_ops_nn.cpp:2486-2494. */
static int64_t mask_index(int mask_ndim, const int64_t *ms, int64_t b, int64_t h, int64_t l, int64_t s) {
    if (mask_ndim == 2) return (ms[0] > 1 ? l : 0) * ms[1] + (ms[1] > 1 ? s : 0);
    int64_t mb = ms[0] > 1 ? b : 0, mh = ms[1] > 1 ? h : 0;
    return ((mb * ms[1] + mh) * ms[2] + (ms[2] > 1 ? l : 0)) * ms[3] + (ms[3] > 1 ? s : 0);
}

/*
 * gt_flash_attention (csrc/gt_ops_nn.cpp:2423-2525), dense inputs:
 *   q (B,H,L,D), k (B,Hkv,S,D), v (B,Hkv,S,Dv) in their own dtypes; mask dense with
 *   mask_ndim dims of shape mask_shape (or NULL); out dense (B,H,L,Dv) in out_dtype.
 * lse (optional, B*H*L doubles) receives max + log(sum exp), +inf for a fully blocked row.
 * nthreads > 0 sets the OpenMP team size.  Returns 0, or -1 for inconsistent shapes.
 */
int oracle_flash_attention(const void *q, int q_dtype, const void *k, int k_dtype, const void *v, int v_dtype,
                           const void *mask, int mask_dtype, int mask_ndim, const int64_t *mask_shape, int64_t B,
                           int64_t H, int64_t Hkv, int64_t L, int64_t S, int64_t D, int64_t Dv, float scale,
                           int is_causal, void *out, int out_dtype, double *lse, int nthreads) {
    if (Hkv <= 0 || H % Hkv != 0) return -1;
    if (mask && mask_ndim != 2 && mask_ndim != 4) return -1;
    const int64_t group = H / Hkv;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)D);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for collapse(2) if (B * H > 4) schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < H; ++h) {
            const int64_t hk = h / group;
            double *scores = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
            for (int64_t l = 0; l < L; ++l) {
                double mx = -INFINITY;
                for (int64_t s = 0; s < S; ++s) {
                    if (is_causal && s > l) {
                        scores[s] = -INFINITY;
                        continue;
                    }
                    double dot = 0.0;
                    const int64_t qo = ((b * H + h) * L + l) * D, ko = ((b * Hkv + hk) * S + s) * D;
                    for (int64_t d = 0; d < D; ++d)
                        dot += oracle_read_f64(q, q_dtype, qo + d) * oracle_read_f64(k, k_dtype, ko + d);
                    dot *= (double)scale;
                    if (mask) {
                        const int64_t mi = mask_index(mask_ndim, mask_shape, b, h, l, s);
                        if (mask_dtype == O_BOOL) {
                            if (((const uint8_t *)mask)[mi] == 0) dot = -INFINITY;
                        } else {
                            dot += oracle_read_f64(mask, mask_dtype, mi);
                        }
                    }
                    scores[s] = dot;
                    if (dot > mx) mx = dot;
                }
                double sum_e = 0.0;
                for (int64_t s = 0; s < S; ++s) {
                    if (isinf(scores[s]) && scores[s] < 0) {
                        scores[s] = 0.0;
                    } else {
                        scores[s] = exp(scores[s] - mx);
                        sum_e += scores[s];
                    }
                }
                const double inv_se = sum_e > 0.0 ? 1.0 / sum_e : 0.0;
                if (lse) lse[(b * H + h) * L + l] = sum_e > 0.0 ? mx + log(sum_e) : INFINITY;
                const int64_t oo = ((b * H + h) * L + l) * Dv;
                for (int64_t dv = 0; dv < Dv; ++dv) {
                    double acc = 0.0;
                    for (int64_t s = 0; s < S; ++s) {
                        const double p = scores[s] * inv_se;
                        if (p == 0.0) continue;
                        acc += p * oracle_read_f64(v, v_dtype, ((b * Hkv + hk) * S + s) * Dv + dv);
                    }
                    oracle_write_f64(out, out_dtype, oo + dv, acc);
                }
            }
            free(scores);
        }
    }
    return 0;
}

/*
 * FlashAttentionFn.backward (gguf_train/_functions.py:1933-1965) in float64:
 *   scores = q.k^T * scale; causal adds -1e9 above the diagonal; a bool mask fills blocked
 *   positions with -1e9, a float mask is added; P = softmax(scores); dV = P^T.dO;
 *   dP = dO.V^T; dS = P*(dP - rowsum(dP*P)); dQ = dS.K*scale; dK = dS^T.Q*scale; a GQA group's
 *   dK/dV are summed into its kv head.
 * Inputs dense in their dtypes; dq (B,H,L,D), dk (B,Hkv,S,D), dv (B,Hkv,S,Dv) are float64.
 */
int oracle_flash_attention_backward(const void *dout, int dout_dtype, const void *q, int q_dtype, const void *k,
                                    int k_dtype, const void *v, int v_dtype, const void *mask, int mask_dtype,
                                    int mask_ndim, const int64_t *mask_shape, int64_t B, int64_t H, int64_t Hkv,
                                    int64_t L, int64_t S, int64_t D, int64_t Dv, float scale, int is_causal,
                                    double *dq, double *dk, double *dv, int nthreads) {
    if (Hkv <= 0 || H % Hkv != 0) return -1;
    if (mask && mask_ndim != 2 && mask_ndim != 4) return -1;
    const int64_t group = H / Hkv;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)D);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    memset(dk, 0, sizeof(double) * (size_t)(B * Hkv * S * D));
    memset(dv, 0, sizeof(double) * (size_t)(B * Hkv * S * Dv));
    /* one (b, kv head) per iteration so the group's dK/dV sums stay private */
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t hk = 0; hk < Hkv; ++hk) {
            double *P = (double *)malloc(sizeof(double) * (size_t)(L * S > 0 ? L * S : 1));
            double *dP = (double *)malloc(sizeof(double) * (size_t)(L * S > 0 ? L * S : 1));
            for (int64_t h = hk * group; h < (hk + 1) * group; ++h) {
                for (int64_t l = 0; l < L; ++l) {
                    double mx = -INFINITY;
                    for (int64_t s = 0; s < S; ++s) {
                        double dot = 0.0;
                        const int64_t qo = ((b * H + h) * L + l) * D, ko = ((b * Hkv + hk) * S + s) * D;
                        for (int64_t d = 0; d < D; ++d)
                            dot += oracle_read_f64(q, q_dtype, qo + d) * oracle_read_f64(k, k_dtype, ko + d);
                        double sc = dot * (double)scale;
                        if (is_causal && s > l) sc += -1e9;
                        if (mask) {
                            const int64_t mi = mask_index(mask_ndim, mask_shape, b, h, l, s);
                            if (mask_dtype == O_BOOL) {
                                if (((const uint8_t *)mask)[mi] == 0) sc = -1e9;
                            } else {
                                sc += oracle_read_f64(mask, mask_dtype, mi);
                            }
                        }
                        P[l * S + s] = sc;
                        if (sc > mx) mx = sc;
                    }
                    double se = 0.0;
                    for (int64_t s = 0; s < S; ++s) {
                        P[l * S + s] = exp(P[l * S + s] - mx);
                        se += P[l * S + s];
                    }
                    for (int64_t s = 0; s < S; ++s) P[l * S + s] /= se;
                    double rs = 0.0;
                    for (int64_t s = 0; s < S; ++s) {
                        double acc = 0.0;
                        const int64_t go = ((b * H + h) * L + l) * Dv, vo = ((b * Hkv + hk) * S + s) * Dv;
                        for (int64_t d = 0; d < Dv; ++d)
                            acc += oracle_read_f64(dout, dout_dtype, go + d) * oracle_read_f64(v, v_dtype, vo + d);
                        dP[l * S + s] = acc;
                        rs += acc * P[l * S + s];
                    }
                    for (int64_t s = 0; s < S; ++s) dP[l * S + s] = P[l * S + s] * (dP[l * S + s] - rs); /* dS */
                }
                for (int64_t l = 0; l < L; ++l) {
                    for (int64_t d = 0; d < D; ++d) {
                        double acc = 0.0;
                        for (int64_t s = 0; s < S; ++s)
                            acc += dP[l * S + s] * oracle_read_f64(k, k_dtype, ((b * Hkv + hk) * S + s) * D + d);
                        dq[((b * H + h) * L + l) * D + d] = acc * (double)scale;
                    }
                }
                for (int64_t s = 0; s < S; ++s) {
                    for (int64_t d = 0; d < D; ++d) {
                        double acc = 0.0;
                        for (int64_t l = 0; l < L; ++l)
                            acc += dP[l * S + s] * oracle_read_f64(q, q_dtype, ((b * H + h) * L + l) * D + d);
                        dk[((b * Hkv + hk) * S + s) * D + d] += acc * (double)scale;
                    }
                    for (int64_t d = 0; d < Dv; ++d) {
                        double acc = 0.0;
                        for (int64_t l = 0; l < L; ++l)
                            acc += P[l * S + s] * oracle_read_f64(dout, dout_dtype, ((b * H + h) * L + l) * Dv + d);
                        dv[((b * Hkv + hk) * S + s) * Dv + d] += acc;
                    }
                }
            }
            free(P);
            free(dP);
        }
    }
    return 0;
}

/*
 * scaled_dot_product_attention with dropout_p > 0 (gguf_train/nn/functional.py:750-767) in
 * float64, dense inputs, for a given keep mask (B,H,L,S bytes, 1 = kept):
 *   scores = q.k^T * scale; causal adds -1e9 above the diagonal; a bool mask fills blocked
 *   positions with -1e9, a float mask is added; P = softmax(scores); Pd = P * keep / (1 - p)
 *   (0 for p = 1, where the reference's dropout returns zeros); out = Pd.v.
 * Backward (grad_out given, dq/dk/dv float64): dV = Pd^T.dO; dPd = dO.V^T; dP = dPd * keep /
 * (1 - p); dS = P * (dP - rowsum(dP * P)); dQ = dS.K * scale; dK = dS^T.Q * scale; a GQA
 * group's dK/dV are summed into its kv head (repeat_interleave's gradient).
 * out (forward) in out_dtype; either of out / dq may be NULL to skip that half.
 */
static void dropout_probs(const void *q, int q_dtype, const void *k, int k_dtype, const void *mask, int mask_dtype,
                          int mask_ndim, const int64_t *mask_shape, int64_t b, int64_t h, int64_t hk, int64_t H,
                          int64_t Hkv, int64_t L, int64_t S, int64_t D, float scale, int is_causal, double *P) {
    for (int64_t l = 0; l < L; ++l) {
        double mx = -INFINITY;
        for (int64_t s = 0; s < S; ++s) {
            double dot = 0.0;
            const int64_t qo = ((b * H + h) * L + l) * D, ko = ((b * Hkv + hk) * S + s) * D;
            for (int64_t d = 0; d < D; ++d) dot += oracle_read_f64(q, q_dtype, qo + d) * oracle_read_f64(k, k_dtype, ko + d);
            double sc = dot * (double)scale;
            if (is_causal && s > l) sc += -1e9;
            if (mask) {
                const int64_t mi = mask_index(mask_ndim, mask_shape, b, h, l, s);
                if (mask_dtype == O_BOOL) {
                    if (((const uint8_t *)mask)[mi] == 0) sc = -1e9;
                } else {
                    sc += oracle_read_f64(mask, mask_dtype, mi);
                }
            }
            P[l * S + s] = sc;
            if (sc > mx) mx = sc;
        }
        double se = 0.0;
        for (int64_t s = 0; s < S; ++s) {
            P[l * S + s] = exp(P[l * S + s] - mx);
            se += P[l * S + s];
        }
        for (int64_t s = 0; s < S; ++s) P[l * S + s] /= se;
    }
}

int oracle_attention_dropout(const void *q, int q_dtype, const void *k, int k_dtype, const void *v, int v_dtype,
                             const void *mask, int mask_dtype, int mask_ndim, const int64_t *mask_shape,
                             const uint8_t *keep, double p, const void *dout, int dout_dtype, int64_t B, int64_t H,
                             int64_t Hkv, int64_t L, int64_t S, int64_t D, int64_t Dv, float scale, int is_causal,
                             void *out, int out_dtype, double *dq, double *dk, double *dv, int nthreads) {
    if (Hkv <= 0 || H % Hkv != 0) return -1;
    if (mask && mask_ndim != 2 && mask_ndim != 4) return -1;
    if (dq && !dout) return -1;
    const int64_t group = H / Hkv;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)D);
    const double r = p < 1.0 ? 1.0 / (1.0 - p) : 0.0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    if (dk) memset(dk, 0, sizeof(double) * (size_t)(B * Hkv * S * D));
    if (dv) memset(dv, 0, sizeof(double) * (size_t)(B * Hkv * S * Dv));
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t hk = 0; hk < Hkv; ++hk) {
            const size_t n = (size_t)(L * S > 0 ? L * S : 1);
            double *P = (double *)malloc(sizeof(double) * n);
            double *Pd = (double *)malloc(sizeof(double) * n);
            double *dS = (double *)malloc(sizeof(double) * n);
            for (int64_t h = hk * group; h < (hk + 1) * group; ++h) {
                dropout_probs(q, q_dtype, k, k_dtype, mask, mask_dtype, mask_ndim, mask_shape, b, h, hk, H, Hkv, L, S, D,
                              scale, is_causal, P);
                const uint8_t *kp = keep + (b * H + h) * L * S;
                for (int64_t i = 0; i < L * S; ++i) Pd[i] = kp[i] ? P[i] * r : 0.0;
                if (out) {
                    for (int64_t l = 0; l < L; ++l)
                        for (int64_t d = 0; d < Dv; ++d) {
                            double acc = 0.0;
                            for (int64_t s = 0; s < S; ++s)
                                acc += Pd[l * S + s] * oracle_read_f64(v, v_dtype, ((b * Hkv + hk) * S + s) * Dv + d);
                            oracle_write_f64(out, out_dtype, ((b * H + h) * L + l) * Dv + d, acc);
                        }
                }
                if (!dq) continue;
                for (int64_t l = 0; l < L; ++l) {
                    double rs = 0.0;
                    const int64_t go = ((b * H + h) * L + l) * Dv;
                    for (int64_t s = 0; s < S; ++s) {
                        double acc = 0.0;
                        const int64_t vo = ((b * Hkv + hk) * S + s) * Dv;
                        for (int64_t d = 0; d < Dv; ++d)
                            acc += oracle_read_f64(dout, dout_dtype, go + d) * oracle_read_f64(v, v_dtype, vo + d);
                        dS[l * S + s] = kp[l * S + s] ? acc * r : 0.0; /* dP */
                        rs += dS[l * S + s] * P[l * S + s];
                    }
                    for (int64_t s = 0; s < S; ++s) dS[l * S + s] = P[l * S + s] * (dS[l * S + s] - rs);
                }
                for (int64_t l = 0; l < L; ++l)
                    for (int64_t d = 0; d < D; ++d) {
                        double acc = 0.0;
                        for (int64_t s = 0; s < S; ++s)
                            acc += dS[l * S + s] * oracle_read_f64(k, k_dtype, ((b * Hkv + hk) * S + s) * D + d);
                        dq[((b * H + h) * L + l) * D + d] = acc * (double)scale;
                    }
                for (int64_t s = 0; s < S; ++s) {
                    for (int64_t d = 0; d < D; ++d) {
                        double acc = 0.0;
                        for (int64_t l = 0; l < L; ++l)
                            acc += dS[l * S + s] * oracle_read_f64(q, q_dtype, ((b * H + h) * L + l) * D + d);
                        dk[((b * Hkv + hk) * S + s) * D + d] += acc * (double)scale;
                    }
                    for (int64_t d = 0; d < Dv; ++d) {
                        double acc = 0.0;
                        for (int64_t l = 0; l < L; ++l)
                            acc += Pd[l * S + s] * oracle_read_f64(dout, dout_dtype, ((b * H + h) * L + l) * Dv + d);
                        dv[((b * Hkv + hk) * S + s) * Dv + d] += acc;
                    }
                }
            }
            free(P);
            free(Pd);
            free(dS);
        }
    }
    return 0;
}

/* ggml block_q8_0: { ggml_half d; int8_t qs[32]; } = 34 bytes. */
void oracle_q8_0_quantize(const float *x, uint8_t *out, int64_t nblocks) {
    for (int64_t i = 0; i < nblocks; ++i) {
        const float *xb = x + i * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = oracle_f32_to_f16(d);
        uint8_t *ob = out + i * 34;
        ob[0] = (uint8_t)(dh & 0xffu);
        ob[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 32; ++j) {
            const float x0 = xb[j] * id;
            ob[2 + j] = (uint8_t)(int8_t)roundf(x0);
        }
    }
}

void oracle_q8_0_dequantize(const uint8_t *in, float *y, int64_t nblocks) {
    for (int64_t i = 0; i < nblocks; ++i) {
        const uint8_t *b = in + i * 34;
        const float d = oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        for (int j = 0; j < 32; ++j) y[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
    }
}

/* RoPE: csrc/gt_ops_nn.cpp:2298-2421 (gt_rope / gt_rope_backward) -> ggml_rope_ext /
 * ggml_rope_ext_back with ext_factor 0, attn_factor 1, no frequency factors (ggml @ f3b407ca, not
 * vendored; restated from its published CPU algorithm, ggml_rope_cache_init + rope_yarn):
 *   theta_scale = powf(freq_base, -2/n_dims); for position p: theta = (float)p, and for pair i
 *   (i < n_dims/2) angle_i = freq_scale * theta then theta *= theta_scale (float32 each step);
 *   (c, s) = (cosf, sinf)(angle_i), s negated for the backward.
 *   NORMAL (mode 0) rotates (x[2i], x[2i+1]), NEOX (mode 2) rotates (x[i], x[i + n_dims/2]):
 *   y_lo = x_lo*c - x_hi*s, y_hi = x_lo*s + x_hi*c; elements from n_dims on are copied.
 * x is read as float32 (the reference converts its input to float32) and the result written in
 * x's dtype.  The two products of each output are formed in double and rounded once to float
 * (ggml's float32 expression differs from this by at most an ulp of its terms).
 * x (B, H, S, D) dense; pos[s] is the position of sequence element s. */
int oracle_rope(const void *x, int x_dtype, int64_t B, int64_t H, int64_t S, int64_t D, const int32_t *pos,
                int n_dims, int mode, float freq_base, float freq_scale, int backward, void *y) {
    if (n_dims < 2 || n_dims % 2 || n_dims > D || (mode != 0 && mode != 2)) return -1;
    const int half = n_dims / 2;
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float *cs = (float *)malloc(sizeof(float) * 2 * (size_t)(half > 0 ? half : 1));
    if (!cs) return -1;
    for (int64_t si = 0; si < S; ++si) {
        float theta = (float)pos[si];
        for (int i = 0; i < half; ++i) {
            const float angle = freq_scale * theta;
            cs[2 * i] = cosf(angle);
            cs[2 * i + 1] = backward ? -sinf(angle) : sinf(angle);
            theta *= theta_scale;
        }
        for (int64_t bh = 0; bh < B * H; ++bh) {
            const int64_t row = (bh * S + si) * D;
            for (int64_t d = n_dims; d < D; ++d)
                oracle_write_f64(y, x_dtype, row + d, (double)(float)oracle_read_f64(x, x_dtype, row + d));
            for (int i = 0; i < half; ++i) {
                const int64_t a = mode == 2 ? i : 2 * i, b = mode == 2 ? i + half : 2 * i + 1;
                const double xa = (float)oracle_read_f64(x, x_dtype, row + a);
                const double xb = (float)oracle_read_f64(x, x_dtype, row + b);
                const double c = cs[2 * i], sn = cs[2 * i + 1];
                oracle_write_f64(y, x_dtype, row + a, (double)(float)(xa * c - xb * sn));
                oracle_write_f64(y, x_dtype, row + b, (double)(float)(xa * sn + xb * c));
            }
        }
    }
    free(cs);
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
