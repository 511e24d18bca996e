/* CPU oracle of the int8 paged KV kernels -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/ load this (through liboracle.so); the product path never does.
 * Sequential restatements, one output at a time in the WGSL kernels' own
 * loop order, so every f32 sum is the reference's:
 *   or_paged_kv_append_i8_clipped  crates/kernels/wgsl/paged_kv_append_i8_clipped_batched.wgsl:46-77
 *   or_paged_decode_scores_i8      crates/kernels/wgsl/paged_decode_scores_i8_batched.wgsl:28-54
 *   or_paged_decode_apply_i8       crates/kernels/wgsl/paged_decode_apply_i8_batched.wgsl:28-53
 * The WGSL `round` is ties-to-even and `i32(f32)` saturates with NaN -> 0
 * (their CPU lowering: crates/wgsl-cpu/src/lib.rs:1448, 1554).
 *
 * Pinning (tests/test_kv8_oracle.py): scale = max|x|/127 in closed form and
 * the code round trip |code*scale - x| <= scale/2 without a clip; a clip
 * below max|x| gives scale = clip/127 and saturated +-127 codes; ties-to-even
 * known answers at scale 1 (x/scale = k + 1/2 exactly); a zero row gives
 * scale 1 and zero codes; the slot arithmetic against hand-built block
 * tables; scores and context against exact integer-valued cases (every sum
 * exact, so the order cannot matter) and against float64 on random data. */
#ifndef KV8_ORACLE_H
#define KV8_ORACLE_H
#include <stdint.h>

/* params [batch, kv_stride, block_size, head_dim]; bindings src [batch][kv_stride],
 * blocks [batch], offsets [batch], clip [n_kv], pool (u32 words of int8), scales. */
void or_paged_kv_append_i8_clipped(const float *src, const uint32_t *blocks, const uint32_t *offsets,
                                   const float *clip, uint32_t *pool, float *scales, uint32_t batch,
                                   uint32_t kv_stride, uint32_t block_size, uint32_t head_dim);
/* params [batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt, scale];
 * scores [batch][n_heads][cap]; entries j >= seq_lens[b] are left untouched. */
void or_paged_decode_scores_i8(const float *q, const uint32_t *pool, const uint32_t *block_tables,
                               const uint32_t *seq_lens, const float *scales, float *scores, uint32_t batch,
                               uint32_t n_heads, uint32_t group, uint32_t head_dim, uint32_t block_size,
                               uint32_t kv_stride, uint32_t cap, uint32_t max_bt, float scale);
/* params [batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt];
 * probs [batch][n_heads][cap], ctx [batch][n_heads*head_dim]. */
void or_paged_decode_apply_i8(const float *probs, const uint32_t *pool, const uint32_t *block_tables,
                              const uint32_t *seq_lens, const float *scales, float *ctx, uint32_t batch,
                              uint32_t n_heads, uint32_t group, uint32_t head_dim, uint32_t block_size,
                              uint32_t kv_stride, uint32_t cap, uint32_t max_bt);
/* One KV code: clamp(i32(round(x / scale)), -127, 127) as an int8. */
int8_t or_kv8_code(float x, float scale);
#endif
