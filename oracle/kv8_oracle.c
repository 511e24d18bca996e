/* CPU oracle of the int8 paged KV kernels -- TEST INFRASTRUCTURE ONLY.
 * See kv8_oracle.h for what each function restates and how it is pinned. */
#include "kv8_oracle.h"

#include <math.h>

/* i32(f32) as crates/wgsl-cpu/src/lib.rs:1554 lowers it (fcvt_to_sint_sat):
 * truncation toward zero, saturating, NaN -> 0. */
static int32_t f32_to_i32_sat(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v < -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* paged_kv_append_i8_clipped_batched.wgsl:72: round() ties-to-even
 * (lib.rs:1448 `nearest`), then i32() and clamp. */
int8_t or_kv8_code(float x, float scale) {
    int32_t q = f32_to_i32_sat(nearbyintf(x / scale));
    if (q < -127) q = -127;
    if (q > 127) q = 127;
    return (int8_t)q;
}

/* paged_kv_append_i8_clipped_batched.wgsl:46-77 */
void or_paged_kv_append_i8_clipped(const float *src, const uint32_t *blocks, const uint32_t *offsets,
                                   const float *clip, uint32_t *pool, float *scales, uint32_t batch,
                                   uint32_t kv_stride, uint32_t block_size, uint32_t head_dim) {
    const uint32_t n_kv = kv_stride / head_dim;
    for (uint32_t idx = 0; idx < batch * n_kv; ++idx) {
        const uint32_t b = idx / n_kv, head = idx % n_kv, hd = head_dim;
        const uint32_t kbase = b * kv_stride + head * hd;
        float mx = 0.0f;
        for (uint32_t i = 0; i < hd; ++i) mx = fmaxf(mx, fabsf(src[kbase + i]));
        const float capped = fminf(mx, clip[head]);
        float scale = capped / 127.0f;
        if (scale == 0.0f) scale = 1.0f;
        const uint32_t slot = blocks[b] * block_size + offsets[b];
        scales[slot * n_kv + head] = scale;
        const uint32_t base_i8 = slot * kv_stride + head * hd;
        for (uint32_t i = 0; i < hd; i += 4) {
            uint32_t packed = 0;
            for (uint32_t j = 0; j < 4; ++j)
                packed |= ((uint32_t)(uint8_t)or_kv8_code(src[kbase + i + j], scale)) << (8 * j);
            pool[(base_i8 + i) / 4] = packed;
        }
    }
}

static float code_at(const uint32_t *pool, uint32_t e) {
    const uint32_t byte = (pool[e / 4] >> (8 * (e % 4))) & 0xffu;
    return (float)(int32_t)(byte > 127 ? (int32_t)byte - 256 : (int32_t)byte);
}

/* paged_decode_scores_i8_batched.wgsl:28-54 */
void or_paged_decode_scores_i8(const float *q, const uint32_t *pool, const uint32_t *block_tables,
                               const uint32_t *seq_lens, const float *scales, float *scores, uint32_t batch,
                               uint32_t n_heads, uint32_t group, uint32_t head_dim, uint32_t block_size,
                               uint32_t kv_stride, uint32_t cap, uint32_t max_bt, float scale) {
    const uint32_t hd = head_dim, n_kv = kv_stride / hd;
    for (uint32_t idx = 0; idx < batch * n_heads * cap; ++idx) {
        const uint32_t b = idx / (n_heads * cap), rem = idx % (n_heads * cap);
        const uint32_t h = rem / cap, j = rem % cap;
        if (j >= seq_lens[b]) continue;
        const uint32_t kvh = h / group;
        const uint32_t physical = block_tables[b * max_bt + j / block_size];
        const uint32_t slot = physical * block_size + (j % block_size);
        const float qscale = scales[slot * n_kv + kvh];
        const uint32_t base_i8 = slot * kv_stride + kvh * hd;
        const uint32_t qb = (b * n_heads + h) * hd;
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) acc = acc + q[qb + d] * code_at(pool, base_i8 + d);
        scores[(b * n_heads + h) * cap + j] = acc * qscale * scale;
    }
}

/* paged_decode_apply_i8_batched.wgsl:28-53. The sum runs over
 * j < min(seq_lens[b], cap): the WGSL loops to seq_lens[b], and past cap it
 * would read the next row's probabilities (or, at the buffer end, whatever
 * robust access returns), which no caller relies on since probs rows are cap
 * wide. The HIP kernel clamps the same way; both are pinned by a test with
 * seq_lens > cap. */
void or_paged_decode_apply_i8(const float *probs, const uint32_t *pool, const uint32_t *block_tables,
                              const uint32_t *seq_lens, const float *scales, float *ctx, uint32_t batch,
                              uint32_t n_heads, uint32_t group, uint32_t head_dim, uint32_t block_size,
                              uint32_t kv_stride, uint32_t cap, uint32_t max_bt) {
    const uint32_t hd = head_dim, n_kv = kv_stride / hd;
    for (uint32_t idx = 0; idx < batch * n_heads * hd; ++idx) {
        const uint32_t b = idx / (n_heads * hd), rem = idx % (n_heads * hd);
        const uint32_t h = rem / hd, d = rem % hd;
        const uint32_t t = seq_lens[b] < cap ? seq_lens[b] : cap, kvh = h / group, pbase = (b * n_heads + h) * cap;
        float acc = 0.0f;
        for (uint32_t j = 0; j < t; ++j) {
            const uint32_t physical = block_tables[b * max_bt + j / block_size];
            const uint32_t slot = physical * block_size + (j % block_size);
            const float qscale = scales[slot * n_kv + kvh];
            acc = acc + probs[pbase + j] * code_at(pool, slot * kv_stride + kvh * hd + d) * qscale;
        }
        ctx[b * (n_heads * hd) + h * hd + d] = acc;
    }
}
