/* CPU oracle of the int8 Qwen3 decoder -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product path never does. A plain sequential restatement of
 * qwen3::serve::Engine's step tape (crates/qwen3/src/serve.rs:1194-1310)
 * for one token at a time per sequence (causal prefill == feeding the
 * prompt token by token, because every op is row-wise except attention,
 * which reads only earlier positions):
 *
 * With kv_int8, K and V are stored as int8 codes with one scale per (token,
 * kv head): scale = min(max|x|, clip)/127 (1 if 0), code =
 * clamp(round_even(x/scale)) (paged_kv_append_i8_clipped_batched.wgsl; the
 * clip table per (layer, kv head) is FLT_MAX unless given); scores use
 * (q . f32(code)) * kscale * hd^-1/2 and the context (p * f32(code)) * vscale
 * (paged_decode_{scores,apply}_i8_batched.wgsl).
 *
 *   x = tok[t]                                   embed.wgsl
 *   per layer:
 *     xn = rmsnorm(x, ln1)                       rmsnorm_rows.wgsl:24-44
 *     q,k,v = lin(xn, wq|wk|wv)                  serve.rs:1242-1247
 *     q,k = rmsnorm per head (q_norm/k_norm)     serve.rs:1253-1254
 *     q,k = rope(pos)                            rope_paged.wgsl:27-38
 *     K[pos],V[pos] = k,v                        paged_kv_append_batched.wgsl
 *     s_j = (q . K_j) * hd^-1/2, j <= pos        paged_decode_scores_wg.wgsl
 *     p = softmax(s)                             decode_softmax_batched.wgsl
 *     ctx = sum_j p_j V_j                        paged_decode_apply_batched.wgsl
 *     x = x + lin(ctx, wo)                       add2.wgsl
 *     xn = rmsnorm(x, ln2)
 *     h = silu(lin(xn, gate)) * lin(xn, up)      silu_mul.wgsl
 *     x = x + lin(h, down)
 *   logits = lin(rmsnorm(x, norm), head)          serve.rs:1297, 1358-1367
 *   next = argmax(logits)                         argmax_row.wgsl
 *
 * lin() is the int8 path when int8 != 0: per-token activation quant
 * (or_max_abs_row / or_quant_pack), weights quantized per output row
 * (or_quantize_weight), exact integer accumulation and the (f32(acc)*sx)*sw
 * epilogue, all from brain_oracle.c. With int8 == 0 it is an f32 linear
 * (double accumulation, rounded once): the fp32 model the int8 path is
 * bounded against (crates/qwen3/src/model.rs:2638-2661, rel-L2 < 0.10).
 *
 * Parameters arrive as one f32 blob in decoder_param_list order
 * (crates/qwen3/src/serve.rs:320-340), then lm_head.weight when untied.
 *
 * Pinned by tests/test_qwen3_oracle.py: an independent numpy float64 forward
 * of the fp32 model, the int8-vs-fp32 bound, and argmax tie/NaN cases.
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "brain_oracle.h"
#include "qwen3_oracle.h"
#include "kv8_oracle.h"

typedef struct {
    const float *ln1, *wq, *wk, *wv, *qn, *kn, *wo, *ln2, *gate, *up, *down;
} layer_t;

typedef struct {
    uint32_t *packed; /* NULL in fp32 mode */
    float *scale;
    const float *w;
    uint32_t n, k;
} lin_t;

static void lin_init(lin_t *l, const float *w, uint32_t n, uint32_t k, int int8) {
    l->w = w;
    l->n = n;
    l->k = k;
    l->packed = NULL;
    l->scale = NULL;
    if (int8) {
        l->packed = (uint32_t *)malloc((size_t)n * k);
        l->scale = (float *)malloc((size_t)n * 4);
        or_quantize_weight(w, n, k, l->packed, l->scale);
    }
}

static void lin_free(lin_t *l) {
    free(l->packed);
    free(l->scale);
}

/* out[n] = lin(x[k]) for one token row. */
static void lin_apply(const lin_t *l, const float *x, float *out) {
    const uint32_t n = l->n, k = l->k;
    if (l->packed) {
        if (k >= 133143u) abort();
        float sx;
        uint32_t *xq = (uint32_t *)malloc((size_t)k);
        or_max_abs_row(x, 1, k, &sx);
        or_quant_pack(x, &sx, 1, k, xq);
        const int8_t *a = (const int8_t *)xq;
        /* Output rows are independent and each keeps its own order: threads
         * only change the speed. */
#pragma omp parallel for schedule(static)
        for (uint32_t j = 0; j < n; ++j) {
            const int8_t *b = (const int8_t *)(l->packed + (size_t)j * (k / 4));
            /* |acc| <= 127 * 127 * k: exact in i32 for k < 133143 (checked
             * below), so the (vectorised) sum equals the int64 one. */
            int32_t acc = 0;
#pragma omp simd reduction(+ : acc)
            for (uint32_t c = 0; c < k; ++c) acc += (int32_t)a[c] * (int32_t)b[c];
            const float v = (float)(int32_t)acc * sx;
            out[j] = v * l->scale[j];
        }
        free(xq);
    } else {
#pragma omp parallel for schedule(static)
        for (uint32_t j = 0; j < n; ++j) {
            const float *w = l->w + (size_t)j * k;
            double acc = 0.0;
            for (uint32_t c = 0; c < k; ++c) acc += (double)x[c] * (double)w[c];
            out[j] = (float)acc;
        }
    }
}

static void rmsnorm(const float *x, const float *w, uint32_t d, float eps, float *out) {
    float ss = 0.0f;
    for (uint32_t c = 0; c < d; ++c) ss += x[c] * x[c];
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (uint32_t c = 0; c < d; ++c) out[c] = x[c] * inv * w[c];
}

static void rope(float *h, uint32_t hd, uint32_t pos, float theta) {
    const uint32_t half = hd / 2;
    for (uint32_t m = 0; m < half; ++m) {
        const float angle = (float)pos * powf(theta, -(float)(2 * m) / (float)hd);
        const float c = cosf(angle), s = sinf(angle);
        const float x0 = h[m], x1 = h[m + half];
        h[m] = x0 * c - x1 * s;
        h[m + half] = x1 * c + x0 * s;
    }
}

uint32_t or_argmax_row(const float *x, uint32_t n) {
    uint32_t best = 0;
    float bv = -FLT_MAX;
    for (uint32_t j = 0; j < n; ++j)
        if (x[j] > bv) {
            bv = x[j];
            best = j;
        }
    return best;
}

uint64_t or_qwen3_param_count(const or_qwen3_config *c) {
    const uint64_t d = c->d_model, ff = c->d_ff, hd = c->head_dim;
    const uint64_t hq = (uint64_t)c->n_heads * hd, hkv = (uint64_t)c->n_kv_heads * hd;
    const uint64_t per = d + hq * d + 2 * hkv * d + 2 * hd + d * hq + d + 3 * ff * d;
    uint64_t n = per * c->n_layers + d + (uint64_t)c->vocab * d;
    if (!c->tie_embeddings) n += (uint64_t)c->vocab * d;
    return n;
}

int or_qwen3_generate(const or_qwen3_config *c, const float *params, int int8, const uint32_t *prompts,
                      uint32_t batch, uint32_t len, uint32_t steps, uint32_t *out_tokens, float *out_logits) {
    return or_qwen3_generate_clip(c, params, int8, prompts, batch, len, steps, out_tokens, out_logits, NULL, NULL);
}

int or_qwen3_generate_clip(const or_qwen3_config *c, const float *params, int int8, const uint32_t *prompts,
                           uint32_t batch, uint32_t len, uint32_t steps, uint32_t *out_tokens, float *out_logits,
                           const float *kclip, const float *vclip) {
    const uint32_t d = c->d_model, ff = c->d_ff, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    const uint32_t hq = nh * hd, hkv = nkv * hd, G = nh / nkv, L = c->n_layers, V = c->vocab;
    if (!len || nh % nkv || hd % 2) return -1;
    const uint32_t T = len + steps;
    const float *p = params;
    layer_t *ly = (layer_t *)calloc(L, sizeof(layer_t));
    for (uint32_t l = 0; l < L; ++l) {
        ly[l].ln1 = p; p += d;
        ly[l].wq = p; p += (size_t)hq * d;
        ly[l].wk = p; p += (size_t)hkv * d;
        ly[l].wv = p; p += (size_t)hkv * d;
        ly[l].qn = p; p += hd;
        ly[l].kn = p; p += hd;
        ly[l].wo = p; p += (size_t)d * hq;
        ly[l].ln2 = p; p += d;
        ly[l].gate = p; p += (size_t)ff * d;
        ly[l].up = p; p += (size_t)ff * d;
        ly[l].down = p; p += (size_t)d * ff;
    }
    const float *norm = p; p += d;
    const float *tok = p; p += (size_t)V * d;
    const float *head_w = c->tie_embeddings ? tok : p;

    lin_t *lq = (lin_t *)calloc(L * 7, sizeof(lin_t));
#pragma omp parallel for schedule(dynamic)
    for (uint32_t l = 0; l < L; ++l) {
        lin_init(&lq[7 * l + 0], ly[l].wq, hq, d, int8);
        lin_init(&lq[7 * l + 1], ly[l].wk, hkv, d, int8);
        lin_init(&lq[7 * l + 2], ly[l].wv, hkv, d, int8);
        lin_init(&lq[7 * l + 3], ly[l].wo, d, hq, int8);
        lin_init(&lq[7 * l + 4], ly[l].gate, ff, d, int8);
        lin_init(&lq[7 * l + 5], ly[l].up, ff, d, int8);
        lin_init(&lq[7 * l + 6], ly[l].down, d, ff, int8);
    }
    lin_t head;
    lin_init(&head, head_w, V, d, int8);

    float *K = (float *)malloc(sizeof(float) * L * T * hkv);
    float *Vc = (float *)malloc(sizeof(float) * L * T * hkv);
    float *KS = (float *)malloc(sizeof(float) * L * T * nkv); /* kv_int8 scales; K/Vc then hold codes */
    float *VS = (float *)malloc(sizeof(float) * L * T * nkv);
    float *x = (float *)malloc(sizeof(float) * d), *xn = (float *)malloc(sizeof(float) * d);
    float *q = (float *)malloc(sizeof(float) * hq), *k = (float *)malloc(sizeof(float) * hkv);
    float *v = (float *)malloc(sizeof(float) * hkv), *ctx = (float *)malloc(sizeof(float) * hq);
    float *o = (float *)malloc(sizeof(float) * d), *g = (float *)malloc(sizeof(float) * ff);
    float *u = (float *)malloc(sizeof(float) * ff), *s = (float *)malloc(sizeof(float) * T);
    float *logits = (float *)malloc(sizeof(float) * V), *tmp = (float *)malloc(sizeof(float) * hd);
    const float scale = 1.0f / sqrtf((float)hd);

    for (uint32_t b = 0; b < batch; ++b) {
        uint32_t cur = prompts[(size_t)b * len];
        for (uint32_t pos = 0; pos < T; ++pos) {
            memcpy(x, tok + (size_t)cur * d, sizeof(float) * d);
            for (uint32_t l = 0; l < L; ++l) {
                float *Kl = K + (size_t)l * T * hkv, *Vl = Vc + (size_t)l * T * hkv;
                rmsnorm(x, ly[l].ln1, d, c->rms_eps, xn);
                lin_apply(&lq[7 * l + 0], xn, q);
                lin_apply(&lq[7 * l + 1], xn, k);
                lin_apply(&lq[7 * l + 2], xn, v);
                for (uint32_t h = 0; h < nh; ++h) {
                    if (c->qk_norm) {
                        rmsnorm(q + h * hd, ly[l].qn, hd, c->rms_eps, tmp);
                        memcpy(q + h * hd, tmp, sizeof(float) * hd);
                    }
                    rope(q + h * hd, hd, pos, c->rope_theta);
                }
                for (uint32_t h = 0; h < nkv; ++h) {
                    if (c->qk_norm) {
                        rmsnorm(k + h * hd, ly[l].kn, hd, c->rms_eps, tmp);
                        memcpy(k + h * hd, tmp, sizeof(float) * hd);
                    }
                    rope(k + h * hd, hd, pos, c->rope_theta);
                }
                memcpy(Kl + (size_t)pos * hkv, k, sizeof(float) * hkv);
                memcpy(Vl + (size_t)pos * hkv, v, sizeof(float) * hkv);
                float *KSl = KS + (size_t)l * T * nkv, *VSl = VS + (size_t)l * T * nkv;
                if (c->kv_int8) {
                    /* paged_kv_append_i8_clipped_batched.wgsl:56-77 (or_kv8_code): the
                     * scale is min(max|x|, clip[l][h]) / 127, 1 when that is 0. */
                    for (uint32_t h = 0; h < nkv; ++h)
                        for (int which = 0; which < 2; ++which) {
                            float *xr = (which ? Vl : Kl) + (size_t)pos * hkv + h * hd;
                            const float *ct = which ? vclip : kclip;
                            float mxa = 0.0f;
                            for (uint32_t e = 0; e < hd; ++e) mxa = fmaxf(mxa, fabsf(xr[e]));
                            float sc = fminf(mxa, ct ? ct[(size_t)l * nkv + h] : FLT_MAX) / 127.0f;
                            if (sc == 0.0f) sc = 1.0f;
                            for (uint32_t e = 0; e < hd; ++e) xr[e] = (float)or_kv8_code(xr[e], sc);
                            (which ? VSl : KSl)[(size_t)pos * nkv + h] = sc;
                        }
                }
                for (uint32_t h = 0; h < nh; ++h) {
                    const uint32_t kh = h / G;
                    float mx = -3.4e38f;
                    for (uint32_t j = 0; j <= pos; ++j) {
                        float acc = 0.0f;
                        const float *kr = Kl + (size_t)j * hkv + kh * hd;
                        for (uint32_t e = 0; e < hd; ++e) acc += q[h * hd + e] * kr[e];
                        if (c->kv_int8) acc = acc * KSl[(size_t)j * nkv + kh];
                        s[j] = acc * scale;
                        if (s[j] > mx) mx = s[j];
                    }
                    float sum = 0.0f;
                    for (uint32_t j = 0; j <= pos; ++j) sum += expf(s[j] - mx);
                    const float inv = 1.0f / sum;
                    for (uint32_t j = 0; j <= pos; ++j) s[j] = expf(s[j] - mx) * inv;
                    for (uint32_t e = 0; e < hd; ++e) {
                        float acc = 0.0f;
                        for (uint32_t j = 0; j <= pos; ++j) {
                            const float pv = s[j] * Vl[(size_t)j * hkv + kh * hd + e];
                            acc += c->kv_int8 ? pv * VSl[(size_t)j * nkv + kh] : pv;
                        }
                        ctx[h * hd + e] = acc;
                    }
                }
                lin_apply(&lq[7 * l + 3], ctx, o);
                for (uint32_t e = 0; e < d; ++e) x[e] = x[e] + o[e];
                rmsnorm(x, ly[l].ln2, d, c->rms_eps, xn);
                lin_apply(&lq[7 * l + 4], xn, g);
                lin_apply(&lq[7 * l + 5], xn, u);
                for (uint32_t e = 0; e < ff; ++e) g[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
                lin_apply(&lq[7 * l + 6], g, o);
                for (uint32_t e = 0; e < d; ++e) x[e] = x[e] + o[e];
            }
            if (pos + 1 < len) {
                cur = prompts[(size_t)b * len + pos + 1];
                continue;
            }
            rmsnorm(x, norm, d, c->rms_eps, xn);
            lin_apply(&head, xn, logits);
            const uint32_t gen = pos + 1 - len; /* 0: the token after the prompt */
            cur = or_argmax_row(logits, V);
            if (out_tokens) out_tokens[(size_t)gen * batch + b] = cur;
            if (out_logits) memcpy(out_logits + ((size_t)gen * batch + b) * V, logits, sizeof(float) * V);
            if (pos + 1 == T) break;
        }
    }
    free(K); free(Vc); free(KS); free(VS); free(x); free(xn); free(q); free(k); free(v); free(ctx); free(o);
    free(g); free(u); free(s); free(logits); free(tmp);
    for (uint32_t i = 0; i < 7 * L; ++i) lin_free(&lq[i]);
    lin_free(&head);
    free(lq);
    free(ly);
    return 0;
}

/* ---------------------------------------------------------------------------
 * CPU baseline of one int8 decode step at the real shape (bench only).
 * The linears run backend-cpu's restated int8 GEMV (or_cpu_gemv_packed: one
 * workgroup per output column, OpenMP over columns, as rayon over
 * available_parallelism), each activation quantized once per distinct input
 * (crates/qwen3/src/serve.rs:1059-1066). RMSNorm, RoPE and attention are f32
 * loops, attention parallel over heads. Weights are random int8 with small
 * scales, since only time is measured. The KV cache holds `ctx` random
 * positions, then `steps` greedy steps are timed at batch 1. Returns the
 * seconds of the timed steps. */
#include <omp.h>

static uint64_t xs_next(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return *s = x;
}

static void fill_i8(uint32_t *p, size_t words, uint64_t seed) {
#pragma omp parallel
    {
        uint64_t s = seed * 0x9E3779B97F4A7C15ull + (uint64_t)omp_get_thread_num() * 0xBF58476D1CE4E5B9ull + 1;
#pragma omp for schedule(static)
        for (long long i = 0; i < (long long)words; ++i) {
            s ^= (uint64_t)i;
            p[i] = (uint32_t)xs_next(&s) & 0x7f7f7f7fu;  /* bytes in [0,127]: no -128 */
        }
    }
}

typedef struct {
    uint32_t *w;
    float *s;
    uint32_t n, k;
} plin_t;

static void plin_make(plin_t *l, uint32_t n, uint32_t k, uint64_t seed) {
    l->n = n;
    l->k = k;
    l->w = (uint32_t *)malloc((size_t)n * k);
    l->s = (float *)malloc((size_t)n * 4);
    fill_i8(l->w, (size_t)n * k / 4, seed);
    for (uint32_t i = 0; i < n; ++i) l->s[i] = 1.0f / (64.0f * sqrtf((float)k));
}

static void plin_run(const plin_t *l, const uint32_t *xq, const float *sx, int threads, float *out) {
    or_cpu_gemv_packed(xq, l->w, sx, l->s, 1, l->k / 4, l->n, threads, out);
}

static void quant1(const float *x, uint32_t k, float *sx, uint32_t *xq) {
    or_max_abs_row(x, 1, k, sx);
    or_quant_pack(x, sx, 1, k, xq);
}

double or_qwen3_cpu_decode(const or_qwen3_config *c, uint64_t seed, int threads, uint32_t ctx, uint32_t steps) {
    const uint32_t d = c->d_model, ff = c->d_ff, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    const uint32_t hq = nh * hd, hkv = nkv * hd, G = nh / nkv, L = c->n_layers, V = c->vocab;
    const uint32_t T = ctx + steps;
    omp_set_num_threads(threads);
    plin_t *q = (plin_t *)calloc(L * 7, sizeof(plin_t)), head;
    for (uint32_t l = 0; l < L; ++l) {
        plin_make(&q[7 * l + 0], hq, d, seed + 7 * l + 0);
        plin_make(&q[7 * l + 1], hkv, d, seed + 7 * l + 1);
        plin_make(&q[7 * l + 2], hkv, d, seed + 7 * l + 2);
        plin_make(&q[7 * l + 3], d, hq, seed + 7 * l + 3);
        plin_make(&q[7 * l + 4], ff, d, seed + 7 * l + 4);
        plin_make(&q[7 * l + 5], ff, d, seed + 7 * l + 5);
        plin_make(&q[7 * l + 6], d, ff, seed + 7 * l + 6);
    }
    plin_make(&head, V, d, seed + 7 * L);
    float *K = (float *)malloc(sizeof(float) * (size_t)L * T * hkv);
    float *Vc = (float *)malloc(sizeof(float) * (size_t)L * T * hkv);
    uint64_t rs = seed | 1;
    for (size_t i = 0; i < (size_t)L * T * hkv; ++i) {
        K[i] = (float)(int32_t)(xs_next(&rs) & 0xffff) / 65536.0f - 0.5f;
        Vc[i] = (float)(int32_t)(xs_next(&rs) & 0xffff) / 65536.0f - 0.5f;
    }
    float *gain = (float *)malloc(sizeof(float) * (d > hd ? d : hd));
    for (uint32_t i = 0; i < (d > hd ? d : hd); ++i) gain[i] = 1.0f;
    float *x = (float *)malloc(4 * d), *xn = (float *)malloc(4 * d), *qv = (float *)malloc(4 * hq);
    float *kv = (float *)malloc(4 * hkv), *vv = (float *)malloc(4 * hkv), *cx = (float *)malloc(4 * hq);
    float *o = (float *)malloc(4 * d), *g = (float *)malloc(4 * ff), *u = (float *)malloc(4 * ff);
    float *lg = (float *)malloc(4 * (size_t)V), *tmp = (float *)malloc(4 * hd);
    uint32_t *xq = (uint32_t *)malloc(ff > d ? ff : (hq > d ? hq : d));
    float sx;
    const float scale = 1.0f / sqrtf((float)hd);
    uint32_t cur = 1;
    const double t0 = omp_get_wtime();
    for (uint32_t pos = ctx; pos < T; ++pos) {
        for (uint32_t e = 0; e < d; ++e) x[e] = (float)((cur * 2654435761u + e * 40503u) & 1023) / 1024.0f - 0.5f;
        for (uint32_t l = 0; l < L; ++l) {
            float *Kl = K + (size_t)l * T * hkv, *Vl = Vc + (size_t)l * T * hkv;
            rmsnorm(x, gain, d, c->rms_eps, xn);
            quant1(xn, d, &sx, xq);
            plin_run(&q[7 * l + 0], xq, &sx, threads, qv);
            plin_run(&q[7 * l + 1], xq, &sx, threads, kv);
            plin_run(&q[7 * l + 2], xq, &sx, threads, vv);
            for (uint32_t h = 0; h < nh; ++h) {
                rmsnorm(qv + h * hd, gain, hd, c->rms_eps, tmp);
                memcpy(qv + h * hd, tmp, 4 * hd);
                rope(qv + h * hd, hd, pos, c->rope_theta);
            }
            for (uint32_t h = 0; h < nkv; ++h) {
                rmsnorm(kv + h * hd, gain, hd, c->rms_eps, tmp);
                memcpy(kv + h * hd, tmp, 4 * hd);
                rope(kv + h * hd, hd, pos, c->rope_theta);
            }
            memcpy(Kl + (size_t)pos * hkv, kv, 4 * hkv);
            memcpy(Vl + (size_t)pos * hkv, vv, 4 * hkv);
#pragma omp parallel for schedule(static)
            for (int h = 0; h < (int)nh; ++h) {
                const uint32_t kh = (uint32_t)h / G;
                float *s = (float *)malloc(4 * (size_t)(pos + 1));
                float mx = -3.4e38f;
                for (uint32_t j = 0; j <= pos; ++j) {
                    float acc = 0.0f;
                    for (uint32_t e = 0; e < hd; ++e) acc += qv[h * hd + e] * Kl[(size_t)j * hkv + kh * hd + e];
                    s[j] = acc * scale;
                    if (s[j] > mx) mx = s[j];
                }
                float sum = 0.0f;
                for (uint32_t j = 0; j <= pos; ++j) sum += (s[j] = expf(s[j] - mx));
                const float inv = 1.0f / sum;
                for (uint32_t e = 0; e < hd; ++e) {
                    float acc = 0.0f;
                    for (uint32_t j = 0; j <= pos; ++j) acc += s[j] * inv * Vl[(size_t)j * hkv + kh * hd + e];
                    cx[h * hd + e] = acc;
                }
                free(s);
            }
            quant1(cx, hq, &sx, xq);
            plin_run(&q[7 * l + 3], xq, &sx, threads, o);
            for (uint32_t e = 0; e < d; ++e) x[e] += o[e];
            rmsnorm(x, gain, d, c->rms_eps, xn);
            quant1(xn, d, &sx, xq);
            plin_run(&q[7 * l + 4], xq, &sx, threads, g);
            plin_run(&q[7 * l + 5], xq, &sx, threads, u);
            for (uint32_t e = 0; e < ff; ++e) g[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
            quant1(g, ff, &sx, xq);
            plin_run(&q[7 * l + 6], xq, &sx, threads, o);
            for (uint32_t e = 0; e < d; ++e) x[e] += o[e];
        }
        rmsnorm(x, gain, d, c->rms_eps, xn);
        quant1(xn, d, &sx, xq);
        plin_run(&head, xq, &sx, threads, lg);
        cur = or_argmax_row(lg, V);
    }
    const double secs = omp_get_wtime() - t0;
    for (uint32_t i = 0; i < 7 * L; ++i) {
        free(q[i].w);
        free(q[i].s);
    }
    free(q);
    free(head.w); free(head.s);
    free(K); free(Vc); free(gain); free(x); free(xn); free(qv); free(kv); free(vv); free(cx);
    free(o); free(g); free(u); free(lg); free(tmp); free(xq);
    return secs;
}
