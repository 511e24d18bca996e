/* CPU oracle of the int8 Qwen3 decoder -- TEST INFRASTRUCTURE ONLY (see qwen3_oracle.c). */
#ifndef QWEN3_ORACLE_H
#define QWEN3_ORACLE_H
#include <stdint.h>

typedef struct {
    uint32_t vocab, n_layers, d_model, n_heads, n_kv_heads, head_dim, d_ff;
    float rope_theta, rms_eps;
    uint32_t tie_embeddings, qk_norm;
    uint32_t kv_int8; /* int8 KV cache (paged_kv_append_i8_clipped_batched; clip tables via or_qwen3_generate_clip) */
} or_qwen3_config;

/* argmax_row.wgsl: first index of the largest value strictly above -FLT_MAX, else 0. */
uint32_t or_argmax_row(const float *x, uint32_t n);
/* Floats in the parameter blob (decoder_param_list order, + lm_head when untied). */
uint64_t or_qwen3_param_count(const or_qwen3_config *c);
/* Greedy generation for `batch` prompts [batch][len]: out_tokens[(steps+1)][batch]
 * (index 0 = the token after the prompt), out_logits[(steps+1)][batch][vocab]
 * (either may be NULL). int8: 1 = int8 linears, 0 = f32 linears. */
int or_qwen3_generate(const or_qwen3_config *c, const float *params, int int8, const uint32_t *prompts,
                      uint32_t batch, uint32_t len, uint32_t steps, uint32_t *out_tokens, float *out_logits);
/* The same with per-(layer, kv head) clip ceilings of the int8 KV cache,
 * kclip/vclip [n_layers][n_kv_heads] (NULL: FLT_MAX, no clipping). */
int or_qwen3_generate_clip(const or_qwen3_config *c, const float *params, int int8, const uint32_t *prompts,
                           uint32_t batch, uint32_t len, uint32_t steps, uint32_t *out_tokens, float *out_logits,
                           const float *kclip, const float *vclip);
/* CPU baseline (bench only): seconds for `steps` int8 decode steps at batch 1
 * after `ctx` cached positions, backend-cpu's restated int8 GEMV on `threads`
 * OpenMP threads, random int8 weights at the config's shapes. */
double or_qwen3_cpu_decode(const or_qwen3_config *c, uint64_t seed, int threads, uint32_t ctx, uint32_t steps);
#endif
