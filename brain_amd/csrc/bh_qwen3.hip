// The int8 Qwen3 decoder on gfx950: the host step tape of
// qwen3::serve::Engine (crates/qwen3/src/serve.rs:1194-1310) with int8
// weights, rebuilt around fused row kernels, the library's int8 GEMV/GEMM, and
// one HIP graph per decode step.
//
// Per layer (rows = tokens in flight; decode: one per sequence, prefill: one
// per prompt position):
//   norm_quant      [residual add +] RMSNorm + per-token int8 quant of the
//                   result (rmsnorm_rows.wgsl + max_abs_row + quant_pack)
//   linear qkv      one int8 linear over the q|k|v weights stacked by rows
//                   (the reference runs three; per-row weight scales make the
//                   stacked product column-for-column identical)
//   qk_rope_append  per head: QK-norm, RoPE (rope_paged.wgsl), K/V append
//   attention       causal GQA over the f32 cache split over key chunks
//                   (flash-decoding): per (row, kv head, 32 keys) scores,
//                   chunk softmax statistics and weighted V, then one
//                   combine per row that also quantizes the context
//                   (paged_decode_scores_wg / decode_softmax_batched /
//                   paged_decode_apply_batched + max_abs_row/quant_pack)
//   linear o
//   norm_quant      residual add + RMSNorm + quant
//   linear gate|up  stacked like qkv
//   swiglu_quant    silu(g)*u (silu_mul.wgsl) + quant
//   linear down     (its residual add is fused into the next norm_quant)
// then norm_quant (final norm, only the rows whose logits are wanted), the
// int8 head and a two-stage greedy argmax that also advances the position and
// records the token, so decode steps chain on the device.
//
// The attention reductions, RMSNorm sums and transcendental functions are
// evaluated in a different order / with different libm than the reference's
// shaders, so activations agree to f32 rounding, not bit for bit; every int8
// linear is the bit-exact path of the rest of the library.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "../../include/brain_hip.h"
#include "bh_attn.h"
#include "bh_common.h"
#include "bh_st.h"

namespace bh {
hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, float* sx, uint32_t* xq);
hipError_t launch_quantize_weight(hipStream_t s, const float* w, int n, int k, uint32_t* packed, float* sw);
hipError_t launch_gemv_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n,
                          bool keep_cached = false, float* am_v = nullptr, uint32_t* am_i = nullptr,
                          uint32_t* am_n = nullptr, int am_stride = 0);
hipError_t gemm_reserve(hipStream_t s, int m, int kg, int n);
hipError_t launch_gemm_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n);
hipError_t launch_gemv_i8_pre(hipStream_t s, int mode, const uint32_t* pre_tok, const float* pre_emb,
                              const float* pre_a, const float* pre_b, const float* pre_w, float* res_out, float eps,
                              const uint32_t* wq, const float* sw, float* out, int m, int kg, int n);
hipError_t launch_gemv_i8_merge(hipStream_t s, const float* part_o, const float* part_ml, const uint32_t* pos, int nh,
                                int hd, int splits, const uint32_t* wq, const float* sw, float* out, int m, int kg,
                                int n);

int tuned_variant(uint32_t m, uint32_t n, uint32_t k);

namespace {

constexpr int RT = 256;       // threads of the row kernels
constexpr int AM_CH = 64;     // argmax chunks per row
constexpr int AM_PARTS = 4096;  // argmax partials per row from the streaming LM head (one per wave)
constexpr int MAX_GROUP = 8;  // query heads per kv head
constexpr uint32_t NO_INDEX = 0xffffffffu;

__device__ __forceinline__ float wave_sum(float v) {
    v = xor_sum<32>(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = xor_max<32>(v);
    return v;
}
// Block-wide reductions over RT threads; `red` holds RT/64 floats. Safe to
// call back to back (the leading barrier retires the previous use of red).
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < RT / 64; ++w) s += red[w];
    return s;
}
// LEAD = false: red has not been used before in this block (no leading barrier).
template <int NT = RT, bool LEAD = true>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    if constexpr (LEAD) __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) s = fmaxf(s, red[w]);
    return s;
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ __forceinline__ float absmax4(float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); }

// Per-token quantization of a row held in registers (G float4 per thread):
// sx = max(max|y|, 1e-8)/127, q = clamp(rne(y * (1/sx))) as quant_pack.
// NT: threads of the block (the row's max is exact in any order, so the
// result does not depend on it).
template <int G, int NT = RT, bool LEAD = true>
__device__ __forceinline__ void quant_row(const float4 (&y)[G], int d4, float* red, float* sx, uint32_t* xq) {
    float am = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (threadIdx.x + g * NT < d4) am = fmaxf(am, absmax4(y[g]));
    am = block_max<NT, LEAD>(am, red);
    const float s = fmaxf(am, 1e-8f) / 127.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int i = threadIdx.x + g * NT;
        if (i < d4) xq[i] = quant_word(y[g], inv);
    }
    if (threadIdx.x == 0) *sx = s;
}

struct NormQuantArgs {
    const float* a;        // x = a[ir] (+ b[ir]) ...
    const float* b;
    const uint32_t* tok;   // ... or x = emb[tok[ir]]
    const float* emb;
    const int* row_map;    // ir = row_map[r] (null: ir = r)
    float* res_out;        // x written back at row ir (may alias a)
    const float* w;        // RMSNorm gain [d]
    float eps;
    int d;
    float* sx;             // [rows]
    uint32_t* xq;          // [rows, xq_words]
    int xq_words;
};

// rmsnorm_rows.wgsl:24-44 (y = x * (1/sqrt(mean(x^2) + eps)) * w) on x = a + b
// (add2.wgsl) or an embedding row (embed.wgsl), then the row's int8 quant.
template <int G>
__global__ __launch_bounds__(RT) void norm_quant_kernel(NormQuantArgs p) {
    __shared__ float red[RT / 64];
    const int r = blockIdx.x;
    const int ir = p.row_map ? p.row_map[r] : r;
    const int d4 = p.d >> 2;
    const float4* src = p.tok ? reinterpret_cast<const float4*>(p.emb + (size_t)p.tok[ir] * p.d)
                              : reinterpret_cast<const float4*>(p.a + (size_t)ir * p.d);
    const float4* add = p.b ? reinterpret_cast<const float4*>(p.b + (size_t)ir * p.d) : nullptr;
    // The gains go out first (unconditional, clamped), so they are not a
    // second memory round trip after the sum's barriers.
    const float4* w4 = reinterpret_cast<const float4*>(p.w);
    float4 wv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) wv[g] = w4[min((int)threadIdx.x + g * RT, d4 - 1)];
    float4 x[G];
    float ss = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int i = threadIdx.x + g * RT;
        x[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < d4) {
            float4 v = src[i];
            if (add) v = add4(v, add[i]);
            x[g] = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }
    if (p.res_out) {
        float4* o = reinterpret_cast<float4*>(p.res_out + (size_t)ir * p.d);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int i = threadIdx.x + g * RT;
            if (i < d4) o[i] = x[g];
        }
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)p.d + p.eps);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int i = threadIdx.x + g * RT;
        if (i < d4)
            x[g] = make_float4(x[g].x * inv * wv[g].x, x[g].y * inv * wv[g].y, x[g].z * inv * wv[g].z,
                               x[g].w * inv * wv[g].w);
    }
    __shared__ float red2[RT / 64];  // the max's own array: no barrier to retire the sum's
    quant_row<G, RT, false>(x, d4, red2, p.sx + r, p.xq + (size_t)r * p.xq_words);
}

// silu_mul.wgsl (h = g / (1 + exp(-g)) * u) over the stacked gate|up output,
// then the row's int8 quant.
template <int G, int NT = RT>
__global__ __launch_bounds__(NT) void swiglu_quant_kernel(const float* gu, int ff, float* sx, uint32_t* xq, int xq_words) {
    __shared__ float red[NT / 64];
    const int r = blockIdx.x;
    const int d4 = ff >> 2;
    const float4* g4 = reinterpret_cast<const float4*>(gu + (size_t)r * 2 * ff);
    const float4* u4 = g4 + d4;
    float4 h[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int i = threadIdx.x + g * NT;
        h[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < d4) {
            const float4 a = g4[i], b = u4[i];
            h[g] = make_float4(a.x / (1.0f + expf(-a.x)) * b.x, a.y / (1.0f + expf(-a.y)) * b.y,
                               a.z / (1.0f + expf(-a.z)) * b.z, a.w / (1.0f + expf(-a.w)) * b.w);
        }
    }
    quant_row<G, NT, false>(h, d4, red, sx + r, xq + (size_t)r * xq_words);
}

// Where position `pos` of sequence `seq` lives in a layer's cache: the token
// slot whose K (V) row is [slot][hkv] and whose KV8 scales are [slot][nkv].
// Contiguous slabs (bs == 0): slot = seq * max_seq + pos. Paged pool
// (crates/qwen3/src/serve.rs:349-356, the layout of
// paged_kv_append_i8_clipped_batched.wgsl:46-77): slot = block * bs + pos % bs
// with block = bt[seq * max_bt + pos / bs]; bs is a multiple of the attention
// chunk, so a chunk of keys lies inside one block. A table entry outside the
// pool (an unallocated block) maps to block 0: only chunks past a row's
// position read it (their reads are issued before the position is known and
// never used), and the host refuses to run a row whose used blocks are not
// allocated.
struct KvMap {
    const uint32_t* bt;  // [max_batch][max_bt] physical blocks (paged)
    int max_bt, bs, nblk, max_seq;
    __device__ __forceinline__ size_t slot(size_t seq, int pos) const {
        if (bs == 0) return seq * max_seq + pos;
        const uint32_t blk = bt[seq * max_bt + pos / bs];
        return (size_t)(blk < (uint32_t)nblk ? blk : 0u) * bs + pos % bs;
    }
};

struct RopeArgs {
    const float* qkv;  // [rows, hq + 2 hkv]
    float* q;          // [rows, hq]
    void* kc;          // this layer's K cache [slots, hkv] (f32, or int8 with KV8)
    void* vc;
    float* ks;         // KV8: per (token slot, kv head) scales [slots, nkv]
    float* vs;
    const float* kclip;  // KV8: per kv head ceilings (FLT_MAX: no clipping)
    const float* vclip;
    const float* qn;   // q_norm / k_norm gains [hd]
    const float* kn;
    const uint32_t* pos;
    const uint32_t* seq;
    int nh, nkv, hd, hq, hkv, max_seq, qk_norm;
    float eps, theta;
    const float2* cs;  // [max_seq][hd/2] (cos, sin) of the rotation angles, rope_table_kernel
    KvMap map;         // (seq, pos) -> cache slot
};

// The rotation of pair m at position pos, angle pos * theta^(-2m/hd)
// (rope_paged.wgsl:27-38), as (cos, sin): evaluated once per engine for every
// position the cache holds, so decode reads it with the row instead of
// spending the transcendental latency on every step.
__global__ __launch_bounds__(256) void rope_table_kernel(float2* cs, int max_seq, int hd, float theta) {
    const int half = hd >> 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)max_seq * half) return;
    const int pos = (int)(i / half), m = (int)(i - (int64_t)pos * half);
    const float angle = (float)pos * powf(theta, -(float)(2 * m) / (float)hd);
    cs[i] = make_float2(cosf(angle), sinf(angle));
}

// One int8 KV code: clamp(round_even(v / scale), -127, 127)
// (paged_kv_append_i8_clipped_batched.wgsl).

// One head of the q|k|v row through the per-head RMSNorm and the
// rotate-half RoPE of rope_paged.wgsl:27-38 (pair (m, m+hd/2), angle
// pos * theta^(-2m/hd)) when `rot` (queries and keys), else unchanged
// (values). One wave; lane l holds pairs m = l and l + 64 (hd <= 256).
__device__ __forceinline__ void rope_head(const RopeArgs& p, const float* src, const float* nw, bool rot, uint32_t pos,
                                          int lane, float (&y0)[2], float (&y1)[2]) {
    const int half = p.hd >> 1;
    const bool norm = rot && p.qk_norm;
    float ss = 0.0f, w0[2] = {0.0f, 0.0f}, w1[2] = {0.0f, 0.0f};
    float2 cs[2] = {make_float2(1.0f, 0.0f), make_float2(1.0f, 0.0f)};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = lane + 64 * u;
        y0[u] = y1[u] = 0.0f;
        if (m < half) {
            y0[u] = src[m];
            y1[u] = src[m + half];
            // The norm weights and the rotation go out with the row, not
            // after the reduction.
            if (norm) {
                w0[u] = nw[m];
                w1[u] = nw[m + half];
            }
            if (rot) cs[u] = p.cs[(size_t)pos * half + m];
            ss += y0[u] * y0[u] + y1[u] * y1[u];
        }
    }
    if (!rot) return;
    float inv = 1.0f;
    if (p.qk_norm) {
        ss = wave_sum(ss);
        inv = 1.0f / sqrtf(ss / (float)p.hd + p.eps);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = lane + 64 * u;
        if (m >= half) continue;
        float a = y0[u], b = y1[u];
        if (p.qk_norm) {
            a = a * inv * w0[u];
            b = b * inv * w1[u];
        }
        const float c = cs[u].x, s = cs[u].y;
        y0[u] = a * c - b * s;
        y1[u] = b * c + a * s;
    }
}

// rope_head split in two for the decode attention launch: the loads (every
// one unconditional: lanes past half the head repeat its last element and
// are zeroed by rope_apply; a missing norm table reads the row instead, and
// the value head reads the first (cos, sin) row) so they can go out ahead of
// the cache reads, then the same arithmetic in the same order.
struct RopeIn {
    float y0[2], y1[2], w0[2], w1[2];
    float2 cs[2];
};
__device__ __forceinline__ void rope_load(const RopeArgs& p, const float* src, const float* nw, bool rot, uint32_t pos,
                                          int lane, RopeIn& in) {
    const int half = p.hd >> 1;
    const float* w = (rot && p.qk_norm) ? nw : src;
    const size_t cs_row = rot ? (size_t)pos * half : 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = min(lane + 64 * u, half - 1);
        in.y0[u] = src[m];
        in.y1[u] = src[m + half];
        in.w0[u] = w[m];
        in.w1[u] = w[m + half];
        in.cs[u] = p.cs[cs_row + m];
    }
}
__device__ __forceinline__ void rope_apply(const RopeArgs& p, bool rot, int lane, const RopeIn& in, float (&y0)[2],
                                           float (&y1)[2]) {
    const int half = p.hd >> 1;
    const bool norm = rot && p.qk_norm;
    float ss = 0.0f, w0[2] = {0.0f, 0.0f}, w1[2] = {0.0f, 0.0f};
    float2 cs[2] = {make_float2(1.0f, 0.0f), make_float2(1.0f, 0.0f)};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = lane + 64 * u;
        y0[u] = y1[u] = 0.0f;
        if (m < half) {
            y0[u] = in.y0[u];
            y1[u] = in.y1[u];
            if (norm) {
                w0[u] = in.w0[u];
                w1[u] = in.w1[u];
            }
            if (rot) cs[u] = in.cs[u];
            ss += y0[u] * y0[u] + y1[u] * y1[u];
        }
    }
    if (!rot) return;
    float inv = 1.0f;
    if (p.qk_norm) {
        ss = wave_sum(ss);
        inv = 1.0f / sqrtf(ss / (float)p.hd + p.eps);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = lane + 64 * u;
        if (m >= half) continue;
        float a = y0[u], b = y1[u];
        if (p.qk_norm) {
            a = a * inv * w0[u];
            b = b * inv * w1[u];
        }
        const float c = cs[u].x, s = cs[u].y;
        y0[u] = a * c - b * s;
        y1[u] = b * c + a * s;
    }
}

// Appends one key or value head at cache slot `tok`: f32 as is, or (KV8)
// int8 codes with one scale per (token, kv head), min(max|x|, clip) / 127
// (1 when that is 0), as paged_kv_append_i8_clipped_batched.wgsl. With KV8
// the values are replaced by their codes (as floats) and the scale returned,
// which is what a reader of the cache sees.
template <bool KV8>
__device__ __forceinline__ float kv_append(const RopeArgs& p, bool is_k, int kh, size_t tok, int lane, float (&y0)[2],
                                           float (&y1)[2]) {
    const int half = p.hd >> 1;
    if constexpr (!KV8) {
        float* dst = static_cast<float*>(is_k ? p.kc : p.vc) + tok * p.hkv + kh * p.hd;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int m = lane + 64 * u;
            if (m >= half) continue;
            dst[m] = y0[u];
            dst[m + half] = y1[u];
        }
        return 1.0f;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (lane + 64 * u < half) mx = fmaxf(mx, fmaxf(fabsf(y0[u]), fabsf(y1[u])));
        mx = wave_max(mx);
        float scale = fminf(mx, (is_k ? p.kclip : p.vclip)[kh]) / 127.0f;
        if (scale == 0.0f) scale = 1.0f;
        uint8_t* d8 = static_cast<uint8_t*>(is_k ? p.kc : p.vc) + tok * p.hkv + kh * p.hd;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int m = lane + 64 * u;
            if (m >= half) continue;
            const uint8_t c0 = kv8_code(y0[u], scale), c1 = kv8_code(y1[u], scale);
            d8[m] = c0;
            d8[m + half] = c1;
            y0[u] = (float)(int8_t)c0;
            y1[u] = (float)(int8_t)c1;
        }
        if (lane == 0) (is_k ? p.ks : p.vs)[tok * p.nkv + kh] = scale;
        return scale;
    }
}

// One wave per (row, head): heads [0,nh) are queries, [nh, nh+nkv) keys,
// [nh+nkv, nh+2nkv) values. Queries and keys get rope_head; keys and values
// land in the cache at (seq, pos) (paged_kv_append_batched.wgsl with a
// contiguous slab per sequence), queries in q.
template <bool KV8>
__global__ __launch_bounds__(64) void qk_rope_append_kernel(RopeArgs p) {
    const int r = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int W = p.hq + 2 * p.hkv;
    const uint32_t pos = p.pos[r];
    const size_t tok = p.map.slot(p.seq[r], (int)pos);
    const bool is_q = h < p.nh, is_k = !is_q && h < p.nh + p.nkv;
    const int kh = is_q ? 0 : (is_k ? h - p.nh : h - p.nh - p.nkv);
    const float* src = p.qkv + (size_t)r * W +
                       (is_q ? h * p.hd : (is_k ? p.hq + kh * p.hd : p.hq + p.hkv + kh * p.hd));
    float y0[2], y1[2];
    rope_head(p, src, is_q ? p.qn : p.kn, is_q || is_k, pos, lane, y0, y1);
    if (!is_q) {
        (void)kv_append<KV8>(p, is_k, kh, tok, lane, y0, y1);
        return;
    }
    const int half = p.hd >> 1;
    float* dst = p.q + (size_t)r * p.hq + h * p.hd;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int m = lane + 64 * u;
        if (m >= half) continue;
        dst[m] = y0[u];
        dst[m + half] = y1[u];
    }
}

constexpr int KCH = ATTN_KCH;  // keys per attention workgroup

struct AttnArgs {
    const float* q;    // [rows, hq]
    const void* kc;    // this layer's caches (f32, or int8 with KV8)
    const void* vc;
    const float* ks;   // KV8 scales [max_batch, max_seq, nkv]
    const float* vs;
    const uint32_t* pos;
    const uint32_t* seq;
    float* part_o;     // [rows, nh, splits, hd]  sum_k exp(s_k - m) v_k over one chunk
    float* part_ml;    // [rows, nh, splits, 2]   (m, sum_k exp(s_k - m))
    int nh, nkv, hd, hq, hkv, max_seq, splits;
    float scale;
    RopeArgs ro;       // ROPE: the q|k|v row, norms and cache of this step
};

// Causal GQA, split over the keys (flash-decoding): one workgroup per (row,
// kv head, chunk of KCH keys); a row attends positions 0..pos of its sequence,
// so chunks starting past pos exit at once. Scores q.k * scale for every
// query head of the group (8 lanes per key, float4 along head_dim), then the
// chunk's own softmax statistics and its unnormalized weighted sum of V.
// attn_combine_quant_kernel merges the chunks: the same softmax as
// paged_decode_scores_wg -> decode_softmax_batched -> paged_decode_apply_batched
// up to f32 rounding order.
// KV8 (paged_decode_scores_i8_batched / paged_decode_apply_i8_batched): the
// score is (q . f32(k8)) * kscale * scale, the weighted sum adds
// (p * f32(v8)) * vscale.
__device__ __forceinline__ float4 i8x4(uint32_t w) {
    return make_float4((float)(int8_t)(w & 0xffu), (float)(int8_t)((w >> 8) & 0xffu),
                       (float)(int8_t)((w >> 16) & 0xffu), (float)(int8_t)(w >> 24));
}

// ROPE (decode, one new token per row, rows in distinct sequences): the
// workgroup also does this step's qk_rope_append work for its kv head. Every
// workgroup rotates the G query heads it reads; the one whose chunk ends at
// pos (the new key) also rotates the new key, appends key and value to the
// cache, and takes them from LDS instead of reading the cache back. Same
// arithmetic, in the same order, as the separate kernels.
// HDT, GT (decode): head_dim and query heads per kv head fixed at compile
// time (0: read from the arguments), so the per-lane loops cover exactly the
// head's pieces and the group's heads.
// PF (decode at many rows, where the cache reads bound the launch): the
// row's position is read first, and a workgroup whose chunk lies past the
// row exits before it reads any of the cache.
template <bool KV8, bool ROPE = false, int HDT = 0, int GT = 0, bool PF = false>
__global__ __launch_bounds__(RT) void attn_split_kernel(AttnArgs p) {
    __shared__ float es[MAX_GROUP * KCH];
    __shared__ float ml[MAX_GROUP * 2];
    __shared__ float ksc[KCH], vsc[KCH];  // KV8: this chunk's per-key scales
    __shared__ float newsc[2];
    // Sized by attn_lds_bytes: the G query heads, the new key and value
    // (ROPE; KV8: codes), and this chunk's V rows read from the cache (f32,
    // or KV8 codes as bytes). Sized to head_dim, not its 256 maximum, so
    // more workgroups fit on a CU.
    extern __shared__ __attribute__((aligned(16))) float attn_dyn[];
    const int r = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z, tid = threadIdx.x;
    // Decode (ROPE) rows are sequences 0..rows-1 in order, so the sequence
    // needs no load there; elsewhere its load goes out with the position's.
    const size_t sq = ROPE ? (size_t)r : (size_t)p.seq[r];
    const int j0 = sp * KCH;
    const int G = GT ? GT : p.nh / p.nkv;
    const int hd = HDT ? HDT : p.hd;
    constexpr int MG = GT ? GT : MAX_GROUP;
    float* qs = attn_dyn;
    float* nk = qs + G * hd;
    float* nv = nk + hd;
    float* vls = nv + hd;
    const size_t tok0 = p.ro.map.slot(sq, j0);  // cache slot of this chunk's first key
    const size_t cb = tok0 * p.hkv + (size_t)kh * hd;  // element of this chunk's first key, this head

    // Every cache read of the chunk is issued first, so its latency overlaps
    // the query rotation: this lane's K pieces (8 lanes per key, float4
    // along head_dim, at most 8 pieces for head_dim <= 256), the V rows
    // (4 elements per piece) and the KV8 scales, for the first `lim` keys.
    const int kk = tid >> 3, l8 = tid & 7;
    constexpr int KP = (HDT ? HDT : 256) / 32;
    float4 kv[KP];
    uint32_t k8[KV8 ? KP : 1];
    // V is staged into LDS on the decode path only (prefill launches
    // thousands of these workgroups and reads V from the cache). The staging
    // is a direct global->LDS load (no registers): piece q (4 elements) of
    // the chunk, key q / (hd/4), lands at byte 16q (f32) or 4q (int8 codes)
    // of vls, i.e. row-major [KCH][hd], so one wave instruction fills 64
    // consecutive pieces. Completion is awaited with an explicit vmcnt wait
    // before the barrier that publishes vls.
    constexpr bool VST = ROPE;
    constexpr int VPT = VST ? KCH * (HDT ? HDT : 256) / 4 / RT : 0;
    const int hd4 = hd >> 2;
    const size_t vbo = cb;
    const uint32_t vls_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)vls;
    float scl = 0.0f;  // KV8: ksc[tid] (tid < KCH) or vsc[tid - KCH]
    // The loads are unconditional, at indices clamped into the first `lim`
    // (>= 1) keys, so none sits behind a branch: a load under a condition
    // has its value moved at the join, which waits for it before the next
    // load goes out. Lanes past `lim` get a repeat of a valid key, masked
    // (K) or never used (V, scales).
    auto load_chunk = [&](int lim) {
        const size_t kro = cb + (size_t)min(kk, lim - 1) * p.hkv;
#pragma unroll
        for (int u = 0; u < KP; ++u) {
            // Pieces past head_dim repeat its last piece (masked below).
            const int c = min(l8 * 4 + 32 * u, hd - 4);
            if constexpr (KV8) k8[u] = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.kc) + kro + c);
            else kv[u] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.kc) + kro + c);
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) {
            const int q0 = tid + u * RT;
            if (q0 - (tid & 63) >= KCH * hd4) break;  // whole waves past the chunk (uniform per wave)
            if (q0 >= KCH * hd4) continue;
            const int q = min(q0, lim * hd4 - 1);  // pieces past `lim` keys repeat a valid one (never read)
            const int k = q / hd4, c = (q - k * hd4) * 4;
            const uint32_t dst = __builtin_amdgcn_readfirstlane(vls_lds + (uint32_t)(q0 - (tid & 63)) * (KV8 ? 4u : 16u));
            if constexpr (KV8) {
                const uint8_t* src = static_cast<const uint8_t*>(p.vc) + vbo + (size_t)k * p.hkv + c;
                asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                             :
                             : "v"(src), "s"(dst)
                             : "memory", "m0");
            } else {
                const float* src = static_cast<const float*>(p.vc) + vbo + (size_t)k * p.hkv + c;
                asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                             :
                             : "v"(src), "s"(dst)
                             : "memory", "m0");
            }
        }
        if constexpr (KV8) {
            const int k = min(tid < KCH ? tid : tid - KCH, lim - 1);
            scl = (tid < KCH ? p.ks : p.vs)[(tok0 + k) * p.nkv + kh];
        }
    };
    // Decode (ROPE): the chunk's addresses do not depend on the row's
    // position, so its reads go out before the position arrives, over every
    // key slot of the chunk inside the cache.
    // One rotated head per wave (the group's query heads, the new key and
    // value: G + 2 <= 4): its loads go out first, ahead of the cache reads,
    // so the rotation runs while those are in flight (vmcnt completes in
    // order: a rotation waiting on loads issued after the cache reads would
    // wait for the cache reads too).
    // The row's position is read once, here, ahead of the cache reads (a
    // scalar load; read again after the DMA's memory clobber it would be a
    // vector load, and waiting for it would wait for every cache read).
    const bool one_head = ROPE && G + 2 <= RT / 64;
    RopeIn rin;
    uint32_t pos_r = 0;
    if constexpr (ROPE) {
        pos_r = p.pos[r];
        if constexpr (PF)
            if (j0 >= (int)pos_r + 1) return;
        if (one_head) {
            const int wave = tid >> 6, lane = tid & 63;
            const RopeArgs& ro = p.ro;
            const uint32_t pos = pos_r;
            const float* row = ro.qkv + (size_t)r * (ro.hq + 2 * ro.hkv);
            const int h = min(wave, G + 1);
            const float* src = h < G ? row + (size_t)(kh * G + h) * hd
                                     : row + ro.hq + (h == G ? 0 : ro.hkv) + kh * hd;
            rope_load(ro, src, h < G ? ro.qn : ro.kn, h <= G, pos, lane, rin);
        }
        load_chunk(min(KCH, p.max_seq - j0));
        // Keeps the loads above the early exit below (the compiler would
        // otherwise sink them past it, behind the position's load).
        asm volatile("" ::: "memory");
    }
    const int t = (int)(ROPE ? pos_r : p.pos[r]) + 1;
    if (j0 >= t) {
        // A chunk past the row: nothing to do, but its V staging loads still
        // write this workgroup's LDS, so they land before the workgroup ends
        // and its LDS can go to another.
        if constexpr (VST) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        return;
    }
    const int n = min(KCH, t - j0);
    const bool last = ROPE && j0 + n == t;  // this chunk ends at the new key
    const int nc = last ? n - 1 : n;        // keys read from the cache
    if constexpr (!ROPE) load_chunk(nc);
    if constexpr (ROPE) {
        const int wave = tid >> 6, lane = tid & 63, half = hd >> 1;
        const RopeArgs& ro = p.ro;
        const uint32_t pos = pos_r;
        const float* row = ro.qkv + (size_t)r * (ro.hq + 2 * ro.hkv);
        for (int h = wave; h < G + 2; h += RT / 64) {
            if (h >= G && !last) continue;
            float y0[2], y1[2];
            float* dst;
            if (h < G) {
                if (one_head) rope_apply(ro, true, lane, rin, y0, y1);
                else rope_head(ro, row + (size_t)(kh * G + h) * hd, ro.qn, true, pos, lane, y0, y1);
                dst = qs + h * hd;
            } else {
                const bool is_k = h == G;
                if (one_head) rope_apply(ro, is_k, lane, rin, y0, y1);
                else rope_head(ro, row + ro.hq + (is_k ? 0 : ro.hkv) + kh * hd, ro.kn, is_k, pos, lane, y0, y1);
                const float sc = kv_append<KV8>(ro, is_k, kh, ro.map.slot(sq, (int)pos), lane, y0, y1);
                dst = is_k ? nk : nv;
                if (lane == 0) newsc[is_k ? 0 : 1] = sc;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int m = lane + 64 * u;
                if (m >= half) continue;
                dst[m] = y0[u];
                dst[m + half] = y1[u];
            }
        }
    } else {
        for (int i = tid; i < G * hd; i += RT) qs[i] = p.q[(size_t)r * p.hq + (size_t)kh * G * hd + i];
    }
    // The V staging loads (and every other load of this wave) have landed.
    if constexpr (VST) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();  // qs, nk, nv, newsc, vls
    if constexpr (KV8) {
        if (tid < KCH) ksc[tid] = tid < n ? (tid < nc ? scl : newsc[0]) : 0.0f;
        else if (tid < 2 * KCH) vsc[tid - KCH] = tid - KCH < n ? (tid - KCH < nc ? scl : newsc[1]) : 0.0f;
    }
    // Keys past the cached ones contribute zeros (done after the rotation,
    // which would otherwise wait for these registers' loads first).
#pragma unroll
    for (int u = 0; u < KP; ++u) {
        const int c = l8 * 4 + 32 * u;
        if constexpr (KV8) kv[u] = i8x4(k8[u]);
        if (kk >= nc || c >= hd) kv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (last && kk == n - 1) {
#pragma unroll
        for (int u = 0; u < KP; ++u) {
            const int c = l8 * 4 + 32 * u;
            if (c < hd) kv[u] = *reinterpret_cast<const float4*>(nk + c);
        }
    }
    if constexpr (KV8) __syncthreads();  // ksc, vsc
    {
        float acc[MG];
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[g] = 0.0f;
#pragma unroll
        for (int u = 0; u < KP; ++u) {
            const int c = l8 * 4 + 32 * u;
            if (c >= hd) break;
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                if (g >= G) break;
                const float4 qv = *reinterpret_cast<const float4*>(qs + g * hd + c);
                acc[g] += qv.x * kv[u].x + qv.y * kv[u].y + qv.z * kv[u].z + qv.w * kv[u].w;
            }
        }
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            if (g >= G) break;
            float v = acc[g];
            v += xor_lane<4>(v);
            v += xor_lane<2>(v);
            v += xor_lane<1>(v);
            if (KV8 && kk < n) v = v * ksc[kk];
            if (l8 == 0) es[g * KCH + kk] = v * p.scale;
        }
    }
    __syncthreads();
    {
        // One 32-lane half-wave per query head: the chunk's max and sum of exp.
        const int g = tid / KCH, k = tid % KCH;
        const bool live = g < G && k < n;
        const float s = live ? es[g * KCH + k] : -INFINITY;
        float m = s;
        m = xor_max<KCH / 2>(m);
        const float e = live ? expf(s - m) : 0.0f;
        float l = e;
        l = xor_sum<KCH / 2>(l);
        __syncthreads();
        if (g < G) es[g * KCH + k] = e;
        if (g < G && k == 0) {
            ml[2 * g] = m;
            ml[2 * g + 1] = l;
        }
    }
    __syncthreads();
    for (int i = tid; i < G * hd; i += RT) {
        const int g = i / hd, d = i - g * hd;
        float acc = 0.0f;
        // Cache rows from LDS (VST) or straight from the cache, same order.
        const size_t vstride = VST ? (size_t)hd : (size_t)p.hkv;
        if constexpr (KV8) {
            const int8_t* vb = VST ? reinterpret_cast<const int8_t*>(vls) : reinterpret_cast<const int8_t*>(p.vc) + vbo;
#pragma unroll 8
            for (int k = 0; k < nc; ++k) acc += es[g * KCH + k] * (float)vb[k * vstride + d] * vsc[k];
            if (last) acc += es[g * KCH + nc] * nv[d] * vsc[nc];
        } else {
            const float* vb = VST ? vls : static_cast<const float*>(p.vc) + vbo;
#pragma unroll 8
            for (int k = 0; k < nc; ++k) acc += es[g * KCH + k] * vb[k * vstride + d];
            if (last) acc += es[g * KCH + nc] * nv[d];
        }
        const size_t slot = ((size_t)r * p.nh + kh * G + g) * p.splits + sp;
        p.part_o[slot * hd + d] = acc;
        if (d == 0) {
            p.part_ml[2 * slot] = ml[2 * g];
            p.part_ml[2 * slot + 1] = ml[2 * g + 1];
        }
    }
}

// Prefill attention over query blocks: one workgroup per (sequence, block
// of QB consecutive rows of that sequence, chunk of 32 keys; kv head), QB*G =
// 32 query vectors (row i, head g). The chunk's K and V go through LDS once
// for all 32 queries (attn_split_kernel reloads them per row). Like the split
// kernel it writes, per (row, head, chunk), the chunk's softmax statistics
// (max m, sum l) and its unnormalized weighted sum of V; attn_combine_quant
// merges the chunks. A query's numbers depend only on its own row and the
// chunk, not on the rows it shares a block with, so any chunking of the
// prompt gives the same bits.
constexpr int PQ = 32;  // query vectors per prefill workgroup
template <bool KV8, int HD>
__global__ __launch_bounds__(RT) void attn_prefill_kernel(AttnArgs p, int rows_per_seq) {
    extern __shared__ __attribute__((aligned(16))) float pf_dyn[];
    constexpr int hd = HD, hd4 = hd >> 2, ks = hd + 4;  // K rows padded for the LDS banks
    constexpr int NP = PQ * hd / 4 / RT;                // float4 pieces per thread (Q, K, V alike)
    static_assert(NP >= 1 && NP * RT * 4 == PQ * hd && KCH * hd4 == NP * RT, "whole pieces per thread");
    constexpr int ow = hd >> 3;                         // head_dim slice per thread in P.V
    const int G = p.nh / p.nkv, QB = PQ / G;
    const int nqb = (rows_per_seq + QB - 1) / QB;
    const int sp = blockIdx.x % p.splits, bq = blockIdx.x / p.splits;
    const int b = bq / nqb, qb = bq - b * nqb, kh = blockIdx.y, tid = threadIdx.x;
    const int i0 = qb * QB, nrow = min(QB, rows_per_seq - i0);
    const int r0 = b * rows_per_seq + i0;  // first row of the block
    const int j0 = sp * KCH;
    // Rows are consecutive positions: the last row holds the largest.
    const int maxpos = (int)p.pos[r0 + nrow - 1];
    if (j0 > maxpos) return;
    const int nk = min(KCH, maxpos + 1 - j0);
    float* Qs = pf_dyn;         // [PQ][hd]
    float* Ks = Qs + PQ * hd;   // [32][hd + 4]
    float* Vs = Ks + KCH * ks;  // [32][hd]
    __shared__ float Ps[PQ][KCH + 1];
    __shared__ float mls[PQ][2];
    __shared__ int posq[PQ];
    __shared__ float ksc[KCH], vsc[KCH];
    const size_t seq = p.seq[r0];
    const size_t tok0 = p.ro.map.slot(seq, j0);  // cache slot of this chunk's first key
    const size_t base = tok0 * p.hkv + (size_t)kh * hd;
    // Every global read is issued before the first use.
    float4 qv[NP], kf[KV8 ? 1 : NP], vf[KV8 ? 1 : NP];
    uint32_t k8[KV8 ? NP : 1], v8[KV8 ? NP : 1];
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        const int idx = tid + u * RT, q = idx / hd4, c = (idx - q * hd4) * 4, i = q / G, g = q - i * G;
        qv[u] = i < nrow ? *reinterpret_cast<const float4*>(p.q + (size_t)(r0 + i) * p.hq + (size_t)(kh * G + g) * hd + c)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
        const int k = idx / hd4;  // the same piece index over the K / V chunk
        const bool live = k < nk;
        const size_t o = base + (size_t)k * p.hkv + c;
        if constexpr (KV8) {
            k8[u] = live ? *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.kc) + o) : 0u;
            v8[u] = live ? *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.vc) + o) : 0u;
        } else {
            kf[u] = live ? *reinterpret_cast<const float4*>(static_cast<const float*>(p.kc) + o) : make_float4(0.f, 0.f, 0.f, 0.f);
            vf[u] = live ? *reinterpret_cast<const float4*>(static_cast<const float*>(p.vc) + o) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float scl = 0.0f;
    if constexpr (KV8) {
        const int k = tid < KCH ? tid : tid - KCH;
        if (tid < 2 * KCH && k < nk) scl = (tid < KCH ? p.ks : p.vs)[(tok0 + k) * p.nkv + kh];
    }
    if (tid < PQ) {
        const int i = tid / G;
        posq[tid] = i < nrow ? (int)p.pos[r0 + i] : -1;
    }
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        const int idx = tid + u * RT, q = idx / hd4, c = (idx - q * hd4) * 4;
        *reinterpret_cast<float4*>(Qs + q * hd + c) = qv[u];
        if constexpr (KV8) {
            *reinterpret_cast<float4*>(Ks + q * ks + c) = i8x4(k8[u]);
            *reinterpret_cast<float4*>(Vs + q * hd + c) = i8x4(v8[u]);
        } else {
            *reinterpret_cast<float4*>(Ks + q * ks + c) = kf[u];
            *reinterpret_cast<float4*>(Vs + q * hd + c) = vf[u];
        }
    }
    if constexpr (KV8) {
        if (tid < KCH) ksc[tid] = scl;
        else if (tid < 2 * KCH) vsc[tid - KCH] = scl;
    }
    __syncthreads();
    // Scores: thread -> queries 2*(t>>4)+{0,1} x keys 2*(t&15)+{0,1}, each dot
    // product in head_dim order, then (KV8: x kscale) x 1/sqrt(hd).
    {
        const int q0 = 2 * (tid >> 4), k0 = 2 * (tid & 15);
        float s00 = 0.f, s01 = 0.f, s10 = 0.f, s11 = 0.f;
        const float* qa = Qs + q0 * hd;
        const float* qb2 = qa + hd;
        const float* ka = Ks + k0 * ks;
        const float* kb = ka + ks;
#pragma unroll 8
        for (int c = 0; c < hd; c += 4) {
            const float4 a0 = *reinterpret_cast<const float4*>(qa + c), a1 = *reinterpret_cast<const float4*>(qb2 + c);
            const float4 b0 = *reinterpret_cast<const float4*>(ka + c), b1 = *reinterpret_cast<const float4*>(kb + c);
            s00 += a0.x * b0.x + a0.y * b0.y + a0.z * b0.z + a0.w * b0.w;
            s01 += a0.x * b1.x + a0.y * b1.y + a0.z * b1.z + a0.w * b1.w;
            s10 += a1.x * b0.x + a1.y * b0.y + a1.z * b0.z + a1.w * b0.w;
            s11 += a1.x * b1.x + a1.y * b1.y + a1.z * b1.z + a1.w * b1.w;
        }
        const float sv[2][2] = {{s00, s01}, {s10, s11}};
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int q = q0 + a, k = k0 + c;
                float v = sv[a][c];
                if (KV8) v = v * ksc[k];
                v = v * p.scale;
                const bool live = k < nk && posq[q] >= 0 && j0 + k <= posq[q];
                Ps[q][k] = live ? v : -INFINITY;
            }
    }
    __syncthreads();
    // The chunk's statistics: 8 lanes per query, 4 keys each; max and sum
    // over the 8 lanes by xor shuffles (a fixed order per query).
    {
        const int q = tid >> 3, k4 = (tid & 7) * 4;
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            sv[c] = Ps[q][k4 + c];
            mx = fmaxf(mx, sv[c]);
        }
        mx = fmaxf(mx, xor_lane<1>(mx));
        mx = fmaxf(mx, xor_lane<2>(mx));
        mx = fmaxf(mx, xor_lane<4>(mx));
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            sv[c] = sv[c] == -INFINITY ? 0.0f : expf(sv[c] - mx);
            sum += sv[c];
        }
        sum += xor_lane<1>(sum);
        sum += xor_lane<2>(sum);
        sum += xor_lane<4>(sum);
#pragma unroll
        for (int c = 0; c < 4; ++c) Ps[q][k4 + c] = sv[c];
        if ((tid & 7) == 0) {
            mls[q][0] = mx;
            mls[q][1] = sum;
        }
    }
    __syncthreads();
    // o = sum_k p_k v_k over the chunk's keys in order.
    const int oq = tid >> 3, od = (tid & 7) * ow;
    const int i = oq / G, g = oq - i * G;
    if (i >= nrow || j0 > posq[oq]) return;  // no key of this chunk is visible to the query
    float O[ow];
#pragma unroll
    for (int u = 0; u < ow; ++u) O[u] = 0.0f;
#pragma unroll 4
    for (int k = 0; k < nk; ++k) {
        const float pk = Ps[oq][k];
        float vk[ow];
#pragma unroll
        for (int u = 0; u < ow; u += 4) {
            const float4 x = *reinterpret_cast<const float4*>(Vs + k * hd + od + u);
            vk[u] = x.x; vk[u + 1] = x.y; vk[u + 2] = x.z; vk[u + 3] = x.w;
        }
        if constexpr (KV8) {
            const float vs = vsc[k];
#pragma unroll
            for (int u = 0; u < ow; ++u) O[u] += pk * vk[u] * vs;
        } else {
#pragma unroll
            for (int u = 0; u < ow; ++u) O[u] += pk * vk[u];
        }
    }
    const size_t slot = ((size_t)(r0 + i) * p.nh + kh * G + g) * p.splits + sp;
#pragma unroll
    for (int u = 0; u < ow; u += 4)
        *reinterpret_cast<float4*>(p.part_o + slot * hd + od + u) = make_float4(O[u], O[u + 1], O[u + 2], O[u + 3]);
    if ((tid & 7) == 0) {
        p.part_ml[2 * slot] = mls[oq][0];
        p.part_ml[2 * slot + 1] = mls[oq][1];
    }
}

// Merge the key chunks of every head of row r: M = max m_s,
// L = sum l_s e^(m_s - M), ctx = sum o_s e^(m_s - M) / L; then quantize the
// whole context row for the output projection (quant_pack semantics).
// H32: head_dim 128, one group per thread (2048 context elements on 512
// threads) and at most ATTN_SB chunks: attn_combine_head32, the chunk
// statistics one per lane and each chunk weight evaluated once.
template <int GQ, int NT = RT, bool H32 = false>
__global__ __launch_bounds__(NT) void attn_combine_quant_kernel(const float* part_o, const float* part_ml,
                                                                const uint32_t* pos, int nh, int hd, int hq,
                                                                int splits, float* sx, uint32_t* xq) {
    __shared__ float red[NT / 64];
    const int r = blockIdx.x;
    const int q4 = hq >> 2;
    // The partial loads of up to two groups go out before the row's position
    // (the number of live chunks) is read; wider rows (more than 2048
    // context elements) take their groups one at a time, as the registers
    // of more preloaded groups would spill.
    constexpr int PRE = GQ <= 2 ? GQ : 1;
    float4 y[GQ];
    AttnFirst4 fb[PRE];
    auto group = [&](int g, size_t& hs, int& d) {
        const int i = threadIdx.x + g * NT;
        const int e = (i < q4 ? i : 0) * 4, h = e / hd;
        d = e - h * hd;
        hs = ((size_t)r * nh + h) * splits;
        return i < q4;
    };
    if constexpr (H32) {
        static_assert(GQ == 1, "one group per thread");
        size_t hs;
        int d;
        (void)group(0, hs, d);
        // Only the row's live chunks (its position is read first).
        const int ns = ((int)pos[r] + ATTN_KCH) / ATTN_KCH;
        attn_load_first4_o(part_o, hs, min(ns, splits), d, hd, fb[0]);
        const float2 mlq = reinterpret_cast<const float2*>(part_ml)[hs + min((int)(threadIdx.x & 31), splits - 1)];
        y[0] = attn_combine_head32(mlq, ns, fb[0]);
    } else if constexpr (PRE == GQ) {
        size_t hs[GQ];
        int dd[GQ];
        bool live[GQ];
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            live[g] = group(g, hs[g], dd[g]);
            attn_load_first4(part_o, part_ml, hs[g], live[g] ? splits : 0, dd[g], hd, fb[g]);
        }
        const int ns = ((int)pos[r] + ATTN_KCH) / ATTN_KCH;
#pragma unroll
        for (int g = 0; g < GQ; ++g)
            y[g] = live[g] ? attn_combine_first4(part_o, part_ml, hs[g], ns, dd[g], hd, fb[g]) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        const int ns = ((int)pos[r] + ATTN_KCH) / ATTN_KCH;
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            size_t hs;
            int d;
            const bool live = group(g, hs, d);
            attn_load_first4(part_o, part_ml, hs, live ? splits : 0, d, hd, fb[0]);
            y[g] = live ? attn_combine_first4(part_o, part_ml, hs, ns, d, hd, fb[0]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    quant_row<GQ, NT, false>(y, q4, red, sx + r, xq + (size_t)r * q4);
}

// Greedy argmax, stage 1: chunk c of row b -> (value, index) with the
// argmax_row.wgsl rule (first index of the largest value strictly above
// -FLT_MAX; NaN never wins).
__device__ __forceinline__ bool am_better(float v, uint32_t i, float bv, uint32_t bi) {
    if (i == NO_INDEX) return false;
    if (bi == NO_INDEX) return true;
    return v > bv || (v == bv && i < bi);
}
template <int OFF>
__device__ __forceinline__ void am_step(float& v, uint32_t& i) {
    const float ov = xor_lane<OFF>(v);
    const uint32_t oi = xor_lane_u<OFF>(i);
    if (am_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}
__device__ __forceinline__ void am_wave(float& v, uint32_t& i) {
    am_step<32>(v, i);
    am_step<16>(v, i);
    am_step<8>(v, i);
    am_step<4>(v, i);
    am_step<2>(v, i);
    am_step<1>(v, i);
}
__global__ __launch_bounds__(RT) void argmax_part_kernel(const float* logits, int vocab, float* pv, uint32_t* pi) {
    __shared__ float rv[RT / 64];
    __shared__ uint32_t ri[RT / 64];
    const int b = blockIdx.y, c = blockIdx.x;
    const int chunk = (vocab + AM_CH - 1) / AM_CH;
    const int lo = c * chunk, hi = min(vocab, lo + chunk);
    const float* row = logits + (size_t)b * vocab;
    float bv = -FLT_MAX;
    uint32_t bi = NO_INDEX;
    for (int j = lo + threadIdx.x; j < hi; j += RT) {
        const float v = row[j];
        if (v > bv) {
            bv = v;
            bi = (uint32_t)j;
        }
    }
    am_wave(bv, bi);
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < RT / 64; ++w)
            if (am_better(rv[w], ri[w], bv, bi)) {
                bv = rv[w];
                bi = ri[w];
            }
        pv[b * AM_CH + c] = bv;
        pi[b * AM_CH + c] = bi;
    }
}

// Stage 2: fold the chunks; tok[b] = winner (0 when nothing beat -FLT_MAX, as
// argmax_row.wgsl). With `hist`, also record the token at generation index
// pos[b] - ctl[0] and advance pos[b] (decode_feed / decode_advance).
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* pv, const uint32_t* pi, uint32_t* tok,
                                                          uint32_t* pos, uint32_t* hist, const uint32_t* ctl,
                                                          int batch) {
    const int b = blockIdx.x, lane = threadIdx.x;
    float v = pv[b * AM_CH + lane];
    uint32_t i = pi[b * AM_CH + lane];
    am_wave(v, i);
    if (lane == 0) {
        const uint32_t idx = i == NO_INDEX ? 0u : i;
        tok[b] = idx;
        if (hist) {
            const uint32_t p = pos[b];
            const uint32_t k = p - ctl[0];
            if (k < ctl[1]) hist[(size_t)k * batch + b] = idx;
            pos[b] = p + 1;
        }
    }
}

// Stage 2 over the LM head's own partials (one per wave of the streaming
// kernel, *np of them per row, stride AM_PARTS); otherwise as above. 256
// threads, every thread's loads issued before the first comparison.
constexpr int AMF_T = 256, AMF_L = 4;  // threads, loads per thread and round
__global__ __launch_bounds__(AMF_T) void argmax_final_parts_kernel(const float* pv, const uint32_t* pi,
                                                                   const uint32_t* np, uint32_t* tok, uint32_t* pos,
                                                                   uint32_t* hist, const uint32_t* ctl, int batch) {
    const int b = blockIdx.x, t = threadIdx.x;
    const int nparts = (int)*np;
    float v = -FLT_MAX;
    uint32_t i = NO_INDEX;
    for (int w0 = 0; w0 < nparts; w0 += AMF_T * AMF_L) {
        float ov[AMF_L];
        uint32_t oi[AMF_L];
#pragma unroll
        for (int k = 0; k < AMF_L; ++k) {
            const int w = min(w0 + t + AMF_T * k, nparts - 1);  // clamped repeats never win over themselves
            ov[k] = pv[(size_t)b * AM_PARTS + w];
            oi[k] = pi[(size_t)b * AM_PARTS + w];
        }
#pragma unroll
        for (int k = 0; k < AMF_L; ++k)
            if (am_better(ov[k], oi[k], v, i)) {
                v = ov[k];
                i = oi[k];
            }
    }
    am_wave(v, i);
    __shared__ float rv[AMF_T / 64];
    __shared__ uint32_t ri[AMF_T / 64];
    if ((t & 63) == 0) {
        rv[t >> 6] = v;
        ri[t >> 6] = i;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < AMF_T / 64; ++w)
            if (am_better(rv[w], ri[w], v, i)) {
                v = rv[w];
                i = ri[w];
            }
        const uint32_t idx = i == NO_INDEX ? 0u : i;
        tok[b] = idx;
        if (hist) {
            const uint32_t p = pos[b];
            const uint32_t k = p - ctl[0];
            if (k < ctl[1]) hist[(size_t)k * batch + b] = idx;
            pos[b] = p + 1;
        }
    }
}

// Counter-based normal generator for the random init: SplitMix64 of
// (key + i), two 24-bit uniforms, Box-Muller.
__device__ __forceinline__ uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void init_normal_kernel(float* w, size_t n, uint64_t key, float stdv) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t z = splitmix(key + i);
        const float u1 = (float)((z >> 40) + 1) * (1.0f / 16777216.0f);
        const float u2 = (float)((z >> 16) & 0xffffffull) * (1.0f / 16777216.0f);
        w[i] = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2) * stdv;
    }
}
__global__ void fill_kernel(float* w, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = v;
}

unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 8192); }

}  // namespace
}  // namespace bh

using namespace bh;

struct bh_qwen3 {
    bh_qwen3_config c{};
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t max_batch = 0, max_seq = 0, max_rows = 0;
    uint32_t hq = 0, hkv = 0, W = 0, xq_words = 0;

    struct Layer {
        float *ln1, *ln2, *qn, *kn;
        uint32_t *wqkv, *wo, *wgu, *wdown;
        float *sqkv, *so, *sgu, *sdown;
    };
    std::vector<Layer> L;
    float* emb = nullptr;
    float* norm = nullptr;
    uint32_t* head = nullptr;
    float* shead = nullptr;
    void *kc = nullptr, *vc = nullptr;  // f32 or int8 elements
    float *kscale = nullptr, *vscale = nullptr;  // KV8: [L][slots][nkv]
    // Cache addressing: slabs (kv_bs 0, slots = max_batch * max_seq) or a
    // paged pool of kv_nblk blocks of kv_bs positions (slots = kv_nblk *
    // kv_bs) through the block table bt [max_batch][kv_max_bt] (host mirror
    // bt_host; BH_QWEN3_NO_BLOCK marks an unallocated entry).
    uint32_t kv_bs = 0, kv_nblk = 0, kv_max_bt = 0;
    size_t slots = 0;
    uint32_t* bt = nullptr;
    std::vector<uint32_t> bt_host;
    float *kclip = nullptr, *vclip = nullptr;    // KV8: [L][nkv], FLT_MAX = no clipping
    float2* rope_cs = nullptr;                   // [max_seq][hd/2] rotation (cos, sin)
    size_t layer_kv = 0;  // elements per layer per cache
    size_t kv_elem = 4;   // bytes per cache element

    float *res = nullptr, *res2 = nullptr, *qkv = nullptr, *q = nullptr, *proj = nullptr, *gu = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;  // attention chunk partials
    uint32_t max_splits = 0;
    const uint32_t* cur_pos = nullptr;
    float *sx = nullptr, *logits = nullptr, *tmpw = nullptr, *am_v = nullptr;
    uint32_t *xq = nullptr, *am_i = nullptr, *am_n = nullptr;  // xq: every producer writes rows of width/4 words
    uint32_t *tok_rows = nullptr, *pos_rows = nullptr, *seq_rows = nullptr;
    int* row_map = nullptr;
    uint32_t *tok_dec = nullptr, *pos_dec = nullptr, *seq_dec = nullptr, *hist = nullptr, *ctl = nullptr;
    size_t tmpw_floats = 0;

    uint32_t batch = 0, prompt_len = 0, decoded = 0;
    hipGraphExec_t graph = nullptr;
    uint32_t graph_batch = 0;
    bool nofuse = false;        // BH_QWEN3_UNFUSED for the current decode call
    bool graph_nofuse = false;  // the mode the captured step was recorded in
    std::vector<void*> allocs;
    std::vector<size_t> alloc_bytes;  // parallel to allocs

    ~bh_qwen3() {
        (void)hipSetDevice(device);
        if (graph) (void)hipGraphExecDestroy(graph);
        if (stream) (void)hipStreamSynchronize(stream);
        for (void* p : allocs) (void)hipFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

template <typename T>
int dalloc(bh_qwen3* e, T** p, size_t count) {
    void* v = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    if (hipMalloc(&v, bytes) != hipSuccess) return fail(BH_ERR_NOMEM, "bh_qwen3: hipMalloc of %zu bytes failed", bytes);
    e->allocs.push_back(v);
    e->alloc_bytes.push_back(bytes);
    if (hipMemset(v, 0, bytes) != hipSuccess) return fail(BH_ERR_HIP, "bh_qwen3: hipMemset failed");
    *p = static_cast<T*>(v);
    return BH_OK;
}

// Host-side guard for every copy between the engine's device buffers and the
// caller: [p, p + bytes) must lie inside one engine allocation. The copies
// below are sized from max_batch / max_seq / the live batch; a slip there
// would read or write past an allocation, so it is refused instead.
int check_span(const bh_qwen3* e, const void* p, size_t bytes, const char* what) {
    const uintptr_t a = (uintptr_t)p;
    for (size_t i = 0; i < e->allocs.size(); ++i) {
        const uintptr_t b = (uintptr_t)e->allocs[i];
        if (a >= b && a < b + e->alloc_bytes[i])
            return bytes <= b + e->alloc_bytes[i] - a
                       ? BH_OK
                       : fail(BH_ERR_INVALID, "bh_qwen3: %s: %zu bytes at offset %zu of a %zu-byte buffer", what,
                              bytes, (size_t)(a - b), e->alloc_bytes[i]);
    }
    return fail(BH_ERR_INVALID, "bh_qwen3: %s: pointer outside the engine's buffers", what);
}

#define BH_TRY(x)                 \
    do {                          \
        int _rc = (x);            \
        if (_rc != BH_OK) return _rc; \
    } while (0)
#define BH_HIP(x, what)                                                                        \
    do {                                                                                       \
        hipError_t _e = (x);                                                                   \
        if (_e != hipSuccess) return fail(BH_ERR_HIP, "bh_qwen3: %s: %s", what, hipGetErrorString(_e)); \
    } while (0)

// Sizes the split-K workspace of the engine's stream for every GEMM-routed
// linear of `rows` rows, so a captured step never needs to allocate.
int reserve_linears(bh_qwen3* e, int rows) {
    const int d = (int)e->c.d_model, ff = (int)e->c.d_ff;
    const int shapes[5][2] = {{d, (int)e->W}, {(int)e->hq, d}, {d, 2 * ff}, {ff, d}, {d, (int)e->c.vocab}};
    for (const auto& kn : shapes) {
        const int tuned = tuned_variant((uint32_t)rows, (uint32_t)kn[1], (uint32_t)kn[0]);
        const bool gemv = tuned ? tuned == BH_VARIANT_WORKGROUP_PER_OUTPUT : rows <= 32;
        if (!gemv) BH_HIP(gemm_reserve(e->stream, rows, kn[0] / 4, kn[1]), "split-K workspace");
    }
    return BH_OK;
}

int launch_linear(bh_qwen3* e, const uint32_t* w, const float* sw, float* out, int m, int k, int n,
                  bool keep_cached = false) {
    const int tuned = tuned_variant((uint32_t)m, (uint32_t)n, (uint32_t)k);
    const bool gemv = tuned ? tuned == BH_VARIANT_WORKGROUP_PER_OUTPUT : m <= 32;
    hipError_t err = gemv ? launch_gemv_i8(e->stream, e->xq, w, e->sx, sw, nullptr, out, OUT_F32, m, k / 4, n,
                                           keep_cached)
                             : launch_gemm_i8(e->stream, e->xq, w, e->sx, sw, nullptr, out, OUT_F32, m, k / 4, n);
    BH_HIP(err, "int8 linear launch");
    return BH_OK;
}

int launch_norm_quant(bh_qwen3* e, const NormQuantArgs& a, int rows) {
    const int groups = (a.d / 4 + RT - 1) / RT;
    if (groups <= 1) norm_quant_kernel<1><<<rows, RT, 0, e->stream>>>(a);
    else if (groups <= 2) norm_quant_kernel<2><<<rows, RT, 0, e->stream>>>(a);
    else if (groups <= 4) norm_quant_kernel<4><<<rows, RT, 0, e->stream>>>(a);
    else norm_quant_kernel<8><<<rows, RT, 0, e->stream>>>(a);
    BH_HIP(hipGetLastError(), "norm_quant launch");
    return BH_OK;
}

int launch_swiglu_quant(bh_qwen3* e, int rows) {
    const int ff = (int)e->c.d_ff;
    const int groups = (ff / 4 + RT - 1) / RT;
    if (groups <= 1) swiglu_quant_kernel<1><<<rows, RT, 0, e->stream>>>(e->gu, ff, e->sx, e->xq, ff / 4);
    else if (groups <= 2) swiglu_quant_kernel<2><<<rows, RT, 0, e->stream>>>(e->gu, ff, e->sx, e->xq, ff / 4);
    else if (groups <= 4) swiglu_quant_kernel<1, 4 * RT><<<rows, 4 * RT, 0, e->stream>>>(e->gu, ff, e->sx, e->xq, ff / 4);
    else swiglu_quant_kernel<8><<<rows, RT, 0, e->stream>>>(e->gu, ff, e->sx, e->xq, ff / 4);
    BH_HIP(hipGetLastError(), "swiglu_quant launch");
    return BH_OK;
}

// The layer stack over `rows` token rows (tok/pos/seq per row), then, if
// n_out > 0, the final norm of rows out_map[0..n_out) (null: rows 0..n_out),
// the head and the argmax into tok_dec (advancing pos_dec and recording into
// hist when `decode`).
int launch_combine_quant(bh_qwen3* e, int rows, int splits) {
    const int hq = (int)e->hq, groups = (hq / 4 + RT - 1) / RT;
    const int nh = (int)e->c.n_heads, hd = (int)e->c.head_dim;
    const uint32_t* pos = e->cur_pos;
    if (groups <= 1) attn_combine_quant_kernel<1><<<rows, RT, 0, e->stream>>>(e->part_o, e->part_ml, pos, nh, hd, hq, splits, e->sx, e->xq);
    else if (groups <= 2 && hd == 128 && hq == 4 * 2 * RT && splits <= ATTN_SB)
        attn_combine_quant_kernel<1, 2 * RT, true><<<rows, 2 * RT, 0, e->stream>>>(e->part_o, e->part_ml, pos, nh, hd, hq, splits, e->sx, e->xq);
    else if (groups <= 2) attn_combine_quant_kernel<1, 2 * RT><<<rows, 2 * RT, 0, e->stream>>>(e->part_o, e->part_ml, pos, nh, hd, hq, splits, e->sx, e->xq);
    else if (groups <= 4) attn_combine_quant_kernel<4><<<rows, RT, 0, e->stream>>>(e->part_o, e->part_ml, pos, nh, hd, hq, splits, e->sx, e->xq);
    else attn_combine_quant_kernel<8><<<rows, RT, 0, e->stream>>>(e->part_o, e->part_ml, pos, nh, hd, hq, splits, e->sx, e->xq);
    BH_HIP(hipGetLastError(), "attention combine launch");
    return BH_OK;
}

// The fused producer + GEMV paths, up to 4 rows each. Every workgroup redoes
// the producer for all rows, re-reading their inputs from L2 (for the RMSNorm
// 2 x 4 KB per row, for the SwiGLU 24 KB per row). Measured at batch 8
// (step time, HIP graph): the norm fused at 8 rows 1.317 ms per step against
// 1.221 with the separate norm kernel, so both stay at 4 rows; at batch 1
// fusing is 10% faster. BH_QWEN3_FUSE_ROWS / BH_QWEN3_FUSE_SWIGLU_ROWS
// override the two limits for measurements. K a multiple of 16 up to 4096
// (64 for the SwiGLU), and no measured preference for the MFMA tile at this
// shape.
static int env_rows(const char* name, int dflt) {
    const char* v = getenv(name);
    return v ? atoi(v) : dflt;
}
bool fused_ok(int rows, int k, int n, int max_rows) {
    if (rows < 1 || rows > max_rows || k % 16 != 0 || k > 4096) return false;
    return tuned_variant((uint32_t)rows, (uint32_t)n, (uint32_t)k) != BH_VARIANT_PACKED_INT8;
}
int fuse_norm_rows() {
    static const int v = env_rows("BH_QWEN3_FUSE_ROWS", 4);
    return v;
}
// Decode rows from which the attention reads the position before the cache
// (BH_ATTN_POSFIRST_ROWS overrides).
static int attn_posfirst_rows() {
    static const int v = env_rows("BH_ATTN_POSFIRST_ROWS", 8);
    return v;
}
int fuse_swiglu_rows() {
    static const int v = env_rows("BH_QWEN3_FUSE_SWIGLU_ROWS", 4);
    return v;
}
// BH_QWEN3_ARGMAX_SEPARATE=1: the argmax's first stage as its own kernel
// even where the streaming head could carry it (for measurement).
static bool am_separate() {
    static const int v = env_rows("BH_QWEN3_ARGMAX_SEPARATE", 0);
    return v != 0;
}

// `splits`: key chunks of KCH covering the longest row of this launch (the
// workspace stride; chunks past a row's position exit immediately).
// `rows_per_seq` > 0: the rows are whole runs of consecutive positions, one
// run of that many rows per sequence (a prefill chunk), which the
// query-block attention kernel needs.
int run_rows(bh_qwen3* e, int rows, const uint32_t* tok, const uint32_t* pos, const uint32_t* seq, int n_out,
             const int* out_map, bool decode, int splits, int rows_per_seq = 0) {
    e->cur_pos = pos;
    const bh_qwen3_config& c = e->c;
    const int d = (int)c.d_model, ff = (int)c.d_ff, hd = (int)c.head_dim;
    float* cur = e->res;
    float* nxt = e->res2;
    const int nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    // Query-block prefill attention: whole per-sequence runs, 32 query vectors
    // a workgroup (G divides 32), head_dim 64 or 128 (the kernel is built for
    // those; its LDS image stays within 64 KB).
    const bool qblock = !decode && rows_per_seq > 0 && rows % rows_per_seq == 0 && PQ % (nh / nkv) == 0 &&
                        (hd == 64 || hd == 128);
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const bh_qwen3::Layer& Ly = e->L[l];
        void* kc = static_cast<uint8_t*>(e->kc) + l * e->layer_kv * e->kv_elem;
        void* vc = static_cast<uint8_t*>(e->vc) + l * e->layer_kv * e->kv_elem;
        const size_t lsc = (size_t)l * e->slots * nkv;
        float* ksl = e->c.kv_int8 ? e->kscale + lsc : nullptr;
        float* vsl = e->c.kv_int8 ? e->vscale + lsc : nullptr;
        // Residual stream ping-pongs between res and res2 (two swaps per
        // layer): a fused producer's workgroup 0 writes the new residual while
        // other workgroups still read the old one.
        const bool fuse = !e->nofuse && fused_ok(rows, d, (int)e->W, fuse_norm_rows()) &&
                          fused_ok(rows, d, 2 * ff, fuse_norm_rows());
        const bool fuse_sw = !e->nofuse && ff % 64 == 0 && fused_ok(rows, ff, d, fuse_swiglu_rows());
        if (fuse) {
            BH_HIP(launch_gemv_i8_pre(e->stream, 3, l == 0 ? tok : nullptr, e->emb, l == 0 ? nullptr : cur,
                                      l == 0 ? nullptr : e->proj, Ly.ln1, nxt, c.rms_eps, Ly.wqkv, Ly.sqkv, e->qkv,
                                      rows, d / 4, (int)e->W),
                   "fused norm + qkv launch");
        } else {
            NormQuantArgs na{};
            if (l == 0) {
                na.tok = tok;
                na.emb = e->emb;
            } else {
                na.a = cur;
                na.b = e->proj;  // previous layer's down projection
            }
            na.res_out = nxt;
            na.w = Ly.ln1;
            na.eps = c.rms_eps;
            na.d = d;
            na.sx = e->sx;
            na.xq = e->xq;
            na.xq_words = d / 4;
            BH_TRY(launch_norm_quant(e, na, rows));
            BH_TRY(launch_linear(e, Ly.wqkv, Ly.sqkv, e->qkv, rows, d, (int)e->W));
        }
        std::swap(cur, nxt);
        RopeArgs ra{e->qkv, e->q, kc, vc, ksl, vsl, e->kclip + (size_t)l * nkv, e->vclip + (size_t)l * nkv, Ly.qn,
                    Ly.kn, pos, seq, nh, nkv, hd, (int)e->hq, (int)e->hkv, (int)e->max_seq, (int)c.qk_norm,
                    c.rms_eps, c.rope_theta, e->rope_cs,
                    KvMap{e->bt, (int)e->kv_max_bt, (int)e->kv_bs, (int)e->kv_nblk, (int)e->max_seq}};
        AttnArgs aa{e->q, kc, vc, ksl, vsl, pos, seq, e->part_o, e->part_ml, nh, nkv, hd, (int)e->hq,
                    (int)e->hkv, (int)e->max_seq, splits, scale, ra};
        const dim3 agrid(rows, nkv, splits);
        const size_t alds_pre = ((size_t)(nh / nkv) * hd + 2 * hd) * 4;                     // no V staging
        const size_t alds = alds_pre + (size_t)KCH * hd * (c.kv_int8 ? 1 : 4);                 // decode
        if (decode && !e->nofuse) {
            // One new token per row, each row its own sequence: the rotation
            // and cache append run inside the attention launch.
            const bool fixed = hd == 128 && nh == 2 * nkv;
            const bool pf = rows >= attn_posfirst_rows();
            if (c.kv_int8 && fixed && pf) attn_split_kernel<true, true, 128, 2, true><<<agrid, RT, alds, e->stream>>>(aa);
            else if (c.kv_int8 && fixed) attn_split_kernel<true, true, 128, 2><<<agrid, RT, alds, e->stream>>>(aa);
            else if (c.kv_int8) attn_split_kernel<true, true><<<agrid, RT, alds, e->stream>>>(aa);
            else if (fixed && pf) attn_split_kernel<false, true, 128, 2, true><<<agrid, RT, alds, e->stream>>>(aa);
            else if (fixed) attn_split_kernel<false, true, 128, 2><<<agrid, RT, alds, e->stream>>>(aa);
            else attn_split_kernel<false, true><<<agrid, RT, alds, e->stream>>>(aa);
            BH_HIP(hipGetLastError(), "attention launch");
        } else {
            if (c.kv_int8) qk_rope_append_kernel<true><<<dim3(rows, nh + 2 * nkv), 64, 0, e->stream>>>(ra);
            else qk_rope_append_kernel<false><<<dim3(rows, nh + 2 * nkv), 64, 0, e->stream>>>(ra);
            BH_HIP(hipGetLastError(), "qk_rope_append launch");
            if (qblock) {
                const int nqb = (rows_per_seq + PQ / (nh / nkv) - 1) / (PQ / (nh / nkv));
                const dim3 pgrid(rows / rows_per_seq * nqb * splits, nkv);
                const size_t plds = ((size_t)PQ * hd + (size_t)KCH * (hd + 4) + (size_t)KCH * hd) * 4;
                if (hd == 128) {
                    if (c.kv_int8) attn_prefill_kernel<true, 128><<<pgrid, RT, plds, e->stream>>>(aa, rows_per_seq);
                    else attn_prefill_kernel<false, 128><<<pgrid, RT, plds, e->stream>>>(aa, rows_per_seq);
                } else {
                    if (c.kv_int8) attn_prefill_kernel<true, 64><<<pgrid, RT, plds, e->stream>>>(aa, rows_per_seq);
                    else attn_prefill_kernel<false, 64><<<pgrid, RT, plds, e->stream>>>(aa, rows_per_seq);
                }
            } else {
                if (c.kv_int8) attn_split_kernel<true><<<agrid, RT, alds_pre, e->stream>>>(aa);
                else attn_split_kernel<false><<<agrid, RT, alds_pre, e->stream>>>(aa);
            }
            BH_HIP(hipGetLastError(), "attention launch");
        }
        // One row (batch-1 decode): the merge runs inside the output
        // projection's prologue. Every GEMV workgroup re-reads the row's
        // partials (tens of KB from L2), one 4-element context group per
        // thread with the loads issued before the position read, which costs
        // less than a launch. With more rows each workgroup merges them one
        // after another (measured slower from 2 rows: batch 4 1.19 -> 1.43 ms).
        if (fuse && rows == 1 && fused_ok(rows, (int)e->hq, d, 1) && e->hq <= 2048) {
            // The merge of the chunks inside the output projection's prologue.
            BH_HIP(launch_gemv_i8_merge(e->stream, e->part_o, e->part_ml, e->cur_pos, nh, hd, splits, Ly.wo, Ly.so,
                                        e->proj, rows, (int)e->hq / 4, d),
                   "fused merge + output projection launch");
        } else {
            BH_TRY(launch_combine_quant(e, rows, splits));
            BH_TRY(launch_linear(e, Ly.wo, Ly.so, e->proj, rows, (int)e->hq, d));
        }
        if (fuse) {
            BH_HIP(launch_gemv_i8_pre(e->stream, 3, nullptr, nullptr, cur, e->proj, Ly.ln2, nxt, c.rms_eps, Ly.wgu,
                                      Ly.sgu, e->gu, rows, d / 4, 2 * ff),
                   "fused norm + gate/up launch");
            std::swap(cur, nxt);
        } else {
            NormQuantArgs nb{};
            nb.a = cur;
            nb.b = e->proj;
            nb.res_out = nxt;
            nb.w = Ly.ln2;
            nb.eps = c.rms_eps;
            nb.d = d;
            nb.sx = e->sx;
            nb.xq = e->xq;
            nb.xq_words = d / 4;
            BH_TRY(launch_norm_quant(e, nb, rows));
            std::swap(cur, nxt);
            BH_TRY(launch_linear(e, Ly.wgu, Ly.sgu, e->gu, rows, d, 2 * ff));
        }
        if (fuse_sw) {
            BH_HIP(launch_gemv_i8_pre(e->stream, 4, nullptr, nullptr, e->gu, nullptr, nullptr, nullptr, 0.0f, Ly.wdown,
                                      Ly.sdown, e->proj, rows, ff / 4, d),
                   "fused swiglu + down launch");
        } else {
            BH_TRY(launch_swiglu_quant(e, rows));
            BH_TRY(launch_linear(e, Ly.wdown, Ly.sdown, e->proj, rows, ff, d));
        }
    }
    if (n_out <= 0) return BH_OK;
    NormQuantArgs nf{};
    nf.a = cur;
    nf.b = e->proj;
    nf.row_map = out_map;
    nf.w = e->norm;
    nf.eps = c.rms_eps;
    nf.d = d;
    nf.sx = e->sx;
    nf.xq = e->xq;
    nf.xq_words = d / 4;
    BH_TRY(launch_norm_quant(e, nf, n_out));
    // The head's weights are re-read every step and fit the Infinity Cache
    // (measured: batch-1 step 0.861 ms with ordinary loads, 0.863-0.864 with
    // the streaming form that is faster on cold weights).
    // The argmax's first stage rides in the streaming head GEMV when that is
    // the kernel the head runs on (one partial per wave); otherwise its own
    // kernel over the logits.
    const int tuned = tuned_variant((uint32_t)n_out, c.vocab, (uint32_t)d);
    const bool head_gemv = tuned ? tuned == BH_VARIANT_WORKGROUP_PER_OUTPUT : n_out <= 32;
    hipError_t herr = hipErrorNotSupported;
    if (head_gemv && !am_separate())
        herr = launch_gemv_i8(e->stream, e->xq, e->head, e->sx, e->shead, nullptr, e->logits, OUT_F32, n_out, d / 4,
                              (int)c.vocab, true, e->am_v, e->am_i, e->am_n, AM_PARTS);
    if (herr == hipSuccess) {
        argmax_final_parts_kernel<<<n_out, AMF_T, 0, e->stream>>>(e->am_v, e->am_i, e->am_n, e->tok_dec,
                                                                  e->pos_dec, decode ? e->hist : nullptr, e->ctl,
                                                                  n_out);
        BH_HIP(hipGetLastError(), "argmax_final launch");
        return BH_OK;
    }
    if (herr != hipErrorNotSupported) BH_HIP(herr, "int8 head launch");
    BH_TRY(launch_linear(e, e->head, e->shead, e->logits, n_out, d, (int)c.vocab, true));
    argmax_part_kernel<<<dim3(AM_CH, n_out), RT, 0, e->stream>>>(e->logits, (int)c.vocab, e->am_v, e->am_i);
    BH_HIP(hipGetLastError(), "argmax_part launch");
    argmax_final_kernel<<<n_out, 64, 0, e->stream>>>(e->am_v, e->am_i, e->tok_dec, e->pos_dec,
                                                     decode ? e->hist : nullptr, e->ctl, n_out);
    BH_HIP(hipGetLastError(), "argmax_final launch");
    return BH_OK;
}

int quantize_into(bh_qwen3* e, const float* dev_w, uint32_t n, uint32_t k, uint32_t* packed, float* sw) {
    BH_HIP(launch_quantize_weight(e->stream, dev_w, (int)n, (int)k, packed, sw), "weight quantization");
    return BH_OK;
}

// Where a named parameter lives: f32 destination (norm gains, embedding) or
// an int8 slice (packed rows + scales) of a stacked weight.
struct Target {
    float* f32 = nullptr;
    uint32_t* packed = nullptr;
    float* scale = nullptr;
    uint64_t n = 0, k = 0;  // int8: rows x cols; f32: numel in n
    bool is_emb = false;
    float init_std = 0.0f;  // random init: 0 -> gain of 1
};

int resolve(bh_qwen3* e, const std::string& name, Target* t) {
    const bh_qwen3_config& c = e->c;
    const uint64_t d = c.d_model, ff = c.d_ff, hq = e->hq, hkv = e->hkv, hd = c.head_dim;
    const float std0 = 0.02f, stdp = 0.02f / sqrtf(2.0f * (float)c.n_layers);
    if (name == "tok.weight") {
        t->f32 = e->emb;
        t->n = (uint64_t)c.vocab * d;
        t->is_emb = true;
        t->init_std = std0;
        return BH_OK;
    }
    if (name == "norm.weight") {
        t->f32 = e->norm;
        t->n = d;
        return BH_OK;
    }
    if (name == "lm_head.weight") {
        if (c.tie_embeddings) return fail(BH_ERR_INVALID, "bh_qwen3: lm_head.weight with tied embeddings");
        t->packed = e->head;
        t->scale = e->shead;
        t->n = c.vocab;
        t->k = d;
        t->init_std = std0;
        return BH_OK;
    }
    unsigned l = 0;
    int used = 0;
    char rest[64] = {0};
    if (sscanf(name.c_str(), "blocks.%u.%63s%n", &l, rest, &used) != 2 || l >= c.n_layers || (size_t)used != name.size())
        return fail(BH_ERR_INVALID, "bh_qwen3: unknown parameter '%s'", name.c_str());
    bh_qwen3::Layer& Ly = e->L[l];
    const std::string s(rest);
    auto lin = [&](uint32_t* base, float* sbase, uint64_t row0, uint64_t n, uint64_t k, float sd) {
        t->packed = base + row0 * (k / 4);
        t->scale = sbase + row0;
        t->n = n;
        t->k = k;
        t->init_std = sd;
        return BH_OK;
    };
    if (s == "ln1.weight") { t->f32 = Ly.ln1; t->n = d; return BH_OK; }
    if (s == "ln2.weight") { t->f32 = Ly.ln2; t->n = d; return BH_OK; }
    if (s == "attn.q_norm.weight") { t->f32 = Ly.qn; t->n = hd; return BH_OK; }
    if (s == "attn.k_norm.weight") { t->f32 = Ly.kn; t->n = hd; return BH_OK; }
    if (s == "attn.wq.weight") return lin(Ly.wqkv, Ly.sqkv, 0, hq, d, std0);
    if (s == "attn.wk.weight") return lin(Ly.wqkv, Ly.sqkv, hq, hkv, d, std0);
    if (s == "attn.wv.weight") return lin(Ly.wqkv, Ly.sqkv, hq + hkv, hkv, d, std0);
    if (s == "attn.wo.weight") return lin(Ly.wo, Ly.so, 0, d, hq, stdp);
    if (s == "mlp.gate.weight") return lin(Ly.wgu, Ly.sgu, 0, ff, d, std0);
    if (s == "mlp.up.weight") return lin(Ly.wgu, Ly.sgu, ff, ff, d, std0);
    if (s == "mlp.down.weight") return lin(Ly.wdown, Ly.sdown, 0, d, ff, stdp);
    return fail(BH_ERR_INVALID, "bh_qwen3: unknown parameter '%s'", name.c_str());
}

std::vector<std::string> param_names(const bh_qwen3_config& c) {
    std::vector<std::string> v;
    static const char* per_layer[] = {"ln1.weight", "attn.wq.weight", "attn.wk.weight", "attn.wv.weight",
                                      "attn.q_norm.weight", "attn.k_norm.weight", "attn.wo.weight", "ln2.weight",
                                      "mlp.gate.weight", "mlp.up.weight", "mlp.down.weight"};
    for (uint32_t l = 0; l < c.n_layers; ++l)
        for (const char* s : per_layer) v.push_back("blocks." + std::to_string(l) + "." + s);
    v.push_back("norm.weight");
    v.push_back("tok.weight");
    if (!c.tie_embeddings) v.push_back("lm_head.weight");
    return v;
}

uint64_t splitmix_host(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char ch : s) h = (h ^ ch) * 0x100000001b3ull;
    return h;
}

// Paged pool: every block the first `npos` positions of sequences 0..batch-1
// use must be allocated (inside the pool) and owned by one sequence only.
int check_blocks(const bh_qwen3* e, uint32_t batch, uint64_t npos, const char* who) {
    if (!e->kv_bs) return BH_OK;
    const uint64_t nb = (npos + e->kv_bs - 1) / e->kv_bs;
    std::vector<uint8_t> seen(e->kv_nblk, 0);
    for (uint32_t b = 0; b < batch; ++b)
        for (uint64_t i = 0; i < nb; ++i) {
            const uint32_t blk = e->bt_host[(size_t)b * e->kv_max_bt + i];
            if (blk >= e->kv_nblk)
                return fail(BH_ERR_INVALID, "%s: sequence %u position %llu has no block (table entry %u, pool of %u)",
                            who, b, (unsigned long long)(i * e->kv_bs), blk, e->kv_nblk);
            if (seen[blk]++)
                return fail(BH_ERR_INVALID, "%s: block %u is used by two sequences (or twice by one)", who, blk);
        }
    return BH_OK;
}

int sync(bh_qwen3* e) {
    BH_HIP(hipStreamSynchronize(e->stream), "stream synchronize");
    return BH_OK;
}

}  // namespace

extern "C" {

int bh_qwen3_create(const bh_qwen3_config* cfg, uint32_t max_batch, uint32_t max_seq, uint32_t max_rows, int device,
                    bh_qwen3** out) {
    if (!cfg || !out) return fail(BH_ERR_INVALID, "bh_qwen3_create: null argument");
    *out = nullptr;
    const bh_qwen3_config& c = *cfg;
    if (!c.vocab || !c.n_layers || !c.d_model || !c.n_heads || !c.n_kv_heads || !c.head_dim || !c.d_ff)
        return fail(BH_ERR_INVALID, "bh_qwen3_create: zero dimension");
    if (c.head_dim % 64 || c.head_dim > 256 || c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > MAX_GROUP)
        return fail(BH_ERR_INVALID, "bh_qwen3_create: head_dim %u / heads %u / kv heads %u unsupported", c.head_dim,
                    c.n_heads, c.n_kv_heads);
    const uint64_t hq = (uint64_t)c.n_heads * c.head_dim;
    if (c.d_model % 4 || c.d_ff % 4 || c.d_model > 8192 || c.d_ff > 8192 || hq > 8192)
        return fail(BH_ERR_INVALID, "bh_qwen3_create: widths must be multiples of 4 and <= 8192");
    if (!max_batch || !max_seq || max_rows < max_batch)
        return fail(BH_ERR_INVALID, "bh_qwen3_create: max_batch %u max_seq %u max_rows %u", max_batch, max_seq, max_rows);
    if (max_seq > 65536) return fail(BH_ERR_INVALID, "bh_qwen3_create: max_seq %u above 65536", max_seq);
    if (c.kv_block_size % KCH || (!c.kv_block_size && c.kv_num_blocks))
        return fail(BH_ERR_INVALID, "bh_qwen3_create: kv_block_size %u must be a multiple of %d (0: slabs, then "
                    "kv_num_blocks 0)", c.kv_block_size, KCH);
    if (c.kv_block_size && (uint64_t)(c.kv_num_blocks ? c.kv_num_blocks : max_batch * ((max_seq + c.kv_block_size - 1) /
                                                                                      c.kv_block_size)) *
                                   c.kv_block_size > (1ull << 31))
        return fail(BH_ERR_INVALID, "bh_qwen3_create: paged pool above 2^31 slots");
    if (hipSetDevice(device) != hipSuccess) return fail(BH_ERR_HIP, "bh_qwen3_create: hipSetDevice(%d)", device);
    bh_qwen3* e = new bh_qwen3();
    e->c = c;
    e->device = device;
    e->max_batch = max_batch;
    e->max_seq = max_seq;
    e->max_rows = max_rows;
    e->hq = (uint32_t)hq;
    e->hkv = c.n_kv_heads * c.head_dim;
    e->W = e->hq + 2 * e->hkv;
    e->xq_words = std::max(std::max(c.d_model, e->hq), c.d_ff) / 4;
    e->max_splits = (max_seq + KCH - 1) / KCH;
    auto bail = [&](int rc) {
        delete e;
        return rc;
    };
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(BH_ERR_HIP, "bh_qwen3_create: stream"));
    const uint64_t d = c.d_model, ff = c.d_ff;
    e->L.resize(c.n_layers);
    int rc = BH_OK;
    for (auto& Ly : e->L) {
        if ((rc = dalloc(e, &Ly.ln1, d)) || (rc = dalloc(e, &Ly.ln2, d)) || (rc = dalloc(e, &Ly.qn, c.head_dim)) ||
            (rc = dalloc(e, &Ly.kn, c.head_dim)) || (rc = dalloc(e, &Ly.wqkv, (uint64_t)e->W * d / 4)) ||
            (rc = dalloc(e, &Ly.sqkv, e->W)) || (rc = dalloc(e, &Ly.wo, d * hq / 4)) || (rc = dalloc(e, &Ly.so, d)) ||
            (rc = dalloc(e, &Ly.wgu, 2 * ff * d / 4)) || (rc = dalloc(e, &Ly.sgu, 2 * ff)) ||
            (rc = dalloc(e, &Ly.wdown, d * ff / 4)) || (rc = dalloc(e, &Ly.sdown, d)))
            return bail(rc);
    }
    if (c.kv_block_size) {
        e->kv_bs = c.kv_block_size;
        e->kv_max_bt = (max_seq + e->kv_bs - 1) / e->kv_bs;
        e->kv_nblk = c.kv_num_blocks ? c.kv_num_blocks : max_batch * e->kv_max_bt;
        e->slots = (size_t)e->kv_nblk * e->kv_bs;
    } else {
        e->slots = (size_t)max_batch * max_seq;
    }
    e->layer_kv = e->slots * e->hkv;
    e->kv_elem = c.kv_int8 ? 1 : 4;
    e->tmpw_floats = std::max<uint64_t>(std::max<uint64_t>((uint64_t)e->W * d, 2 * ff * d), d * std::max<uint64_t>(hq, ff));
    if (!c.tie_embeddings) e->tmpw_floats = std::max<uint64_t>(e->tmpw_floats, (uint64_t)c.vocab * d);
    const uint64_t R = max_rows;
    if ((rc = dalloc(e, &e->emb, (uint64_t)c.vocab * d)) || (rc = dalloc(e, &e->norm, d)) ||
        (rc = dalloc(e, &e->head, (uint64_t)c.vocab * d / 4)) || (rc = dalloc(e, &e->shead, c.vocab)) ||
        (rc = dalloc(e, (uint8_t**)&e->kc, e->layer_kv * c.n_layers * e->kv_elem)) ||
        (rc = dalloc(e, (uint8_t**)&e->vc, e->layer_kv * c.n_layers * e->kv_elem)) ||
        (rc = dalloc(e, &e->kscale, c.kv_int8 ? (uint64_t)c.n_layers * e->slots * c.n_kv_heads : 1)) ||
        (rc = dalloc(e, &e->vscale, c.kv_int8 ? (uint64_t)c.n_layers * e->slots * c.n_kv_heads : 1)) ||
        (rc = dalloc(e, &e->bt, (uint64_t)max_batch * std::max<uint32_t>(e->kv_max_bt, 1))) ||
        (rc = dalloc(e, &e->kclip, (uint64_t)c.n_layers * c.n_kv_heads)) ||
        (rc = dalloc(e, &e->vclip, (uint64_t)c.n_layers * c.n_kv_heads)) ||
        (rc = dalloc(e, &e->rope_cs, (uint64_t)max_seq * (c.head_dim / 2))) ||
        (rc = dalloc(e, &e->res, R * d)) || (rc = dalloc(e, &e->res2, R * d)) || (rc = dalloc(e, &e->qkv, R * e->W)) || (rc = dalloc(e, &e->q, R * hq)) ||
        (rc = dalloc(e, &e->part_o, R * c.n_heads * e->max_splits * c.head_dim)) || (rc = dalloc(e, &e->part_ml, R * c.n_heads * e->max_splits * 2)) || (rc = dalloc(e, &e->proj, R * d)) || (rc = dalloc(e, &e->gu, R * 2 * ff)) ||
        (rc = dalloc(e, &e->sx, R)) || (rc = dalloc(e, &e->xq, R * e->xq_words)) ||
        (rc = dalloc(e, &e->logits, (uint64_t)max_batch * c.vocab)) || (rc = dalloc(e, &e->tmpw, e->tmpw_floats)) ||
        (rc = dalloc(e, &e->am_v, (uint64_t)max_batch * AM_PARTS)) || (rc = dalloc(e, &e->am_i, (uint64_t)max_batch * AM_PARTS)) ||
        (rc = dalloc(e, &e->am_n, 1)) ||
        (rc = dalloc(e, &e->tok_rows, R)) || (rc = dalloc(e, &e->pos_rows, R)) || (rc = dalloc(e, &e->seq_rows, R)) ||
        (rc = dalloc(e, &e->row_map, max_batch)) || (rc = dalloc(e, &e->tok_dec, max_batch)) ||
        (rc = dalloc(e, &e->pos_dec, max_batch)) || (rc = dalloc(e, &e->seq_dec, max_batch)) ||
        (rc = dalloc(e, &e->hist, (uint64_t)max_seq * max_batch)) || (rc = dalloc(e, &e->ctl, 2)))
        return bail(rc);
    {
        const int64_t nrot = (int64_t)max_seq * (c.head_dim / 2);
        rope_table_kernel<<<(unsigned)((nrot + 255) / 256), 256, 0, e->stream>>>(e->rope_cs, (int)max_seq,
                                                                               (int)c.head_dim, c.rope_theta);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(e->stream) != hipSuccess)
            return bail(fail(BH_ERR_HIP, "bh_qwen3_create: rotation table"));
    }
    std::vector<float> clip((size_t)c.n_layers * c.n_kv_heads, FLT_MAX);
    if (hipMemcpy(e->kclip, clip.data(), clip.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(e->vclip, clip.data(), clip.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(BH_ERR_HIP, "bh_qwen3_create: upload"));
    if (e->kv_bs) {
        // Default table: sequence b owns blocks b * max_bt .. b * max_bt +
        // max_bt - 1 when the pool holds them (the slab layout, paged), else
        // nothing is allocated until bh_qwen3_set_block_table.
        e->bt_host.assign((size_t)max_batch * e->kv_max_bt, BH_QWEN3_NO_BLOCK);
        if ((uint64_t)e->kv_nblk >= (uint64_t)max_batch * e->kv_max_bt)
            for (size_t i = 0; i < e->bt_host.size(); ++i) e->bt_host[i] = (uint32_t)i;
        if (hipMemcpy(e->bt, e->bt_host.data(), e->bt_host.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(BH_ERR_HIP, "bh_qwen3_create: block table upload"));
    }
    std::vector<uint32_t> seq(max_batch);
    for (uint32_t b = 0; b < max_batch; ++b) seq[b] = b;
    if (hipMemcpy(e->seq_dec, seq.data(), max_batch * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(BH_ERR_HIP, "bh_qwen3_create: upload"));
    *out = e;
    return BH_OK;
}

void bh_qwen3_destroy(bh_qwen3* e) { delete e; }

void* bh_qwen3_stream(bh_qwen3* e) { return e ? (void*)e->stream : nullptr; }

int bh_qwen3_set_weight(bh_qwen3* e, const char* name, const float* host, uint64_t numel) {
    if (!e || !name || !host) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight: null argument");
    (void)hipSetDevice(e->device);
    Target t;
    BH_TRY(resolve(e, name, &t));
    if (t.f32) {
        if (numel != t.n) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight: %s has %llu elements, got %llu", name,
                                      (unsigned long long)t.n, (unsigned long long)numel);
        BH_HIP(hipMemcpyAsync(t.f32, host, numel * 4, hipMemcpyHostToDevice, e->stream), "upload");
        if (t.is_emb && e->c.tie_embeddings)
            BH_TRY(quantize_into(e, e->emb, e->c.vocab, e->c.d_model, e->head, e->shead));
        return sync(e);
    }
    if (numel != t.n * t.k) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight: %s has %llu elements, got %llu", name,
                                        (unsigned long long)(t.n * t.k), (unsigned long long)numel);
    BH_HIP(hipMemcpyAsync(e->tmpw, host, numel * 4, hipMemcpyHostToDevice, e->stream), "upload");
    BH_TRY(quantize_into(e, e->tmpw, (uint32_t)t.n, (uint32_t)t.k, t.packed, t.scale));
    return sync(e);
}

int bh_qwen3_set_weight_i8(bh_qwen3* e, const char* name, const uint32_t* packed, const float* scale, uint32_t n,
                           uint32_t k) {
    if (!e || !name || !packed || !scale) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight_i8: null argument");
    (void)hipSetDevice(e->device);
    Target t;
    BH_TRY(resolve(e, name, &t));
    if (!t.packed) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight_i8: %s is not an int8 linear", name);
    if (n != t.n || k != t.k) return fail(BH_ERR_INVALID, "bh_qwen3_set_weight_i8: %s is [%llu,%llu], got [%u,%u]", name,
                                          (unsigned long long)t.n, (unsigned long long)t.k, n, k);
    BH_HIP(hipMemcpyAsync(t.packed, packed, (size_t)n * k, hipMemcpyHostToDevice, e->stream), "upload");
    BH_HIP(hipMemcpyAsync(t.scale, scale, (size_t)n * 4, hipMemcpyHostToDevice, e->stream), "upload");
    return sync(e);
}

// dequantize_weight (crates/model/src/int8.rs:70-87) on the device:
// w[r, 4g+b] = f32(int8 byte b of packed[r, g]) * sw[r].
__global__ void dequantize_rows_kernel(const uint32_t* packed, const float* sw, uint64_t n, uint64_t kg, float* w) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n * kg; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / kg;
        const uint32_t word = packed[i];
        const float s = sw[r];
        const float4 v = make_float4((float)(int8_t)(uint8_t)word * s, (float)(int8_t)(uint8_t)(word >> 8) * s,
                                     (float)(int8_t)(uint8_t)(word >> 16) * s, (float)(int8_t)(uint8_t)(word >> 24) * s);
        reinterpret_cast<float4*>(w)[i] = v;
    }
}

static int upload_chunked(bh_qwen3* e, void* dst, const uint8_t* src, size_t bytes) {
    constexpr size_t CH = 64u << 20;
    for (size_t off = 0; off < bytes; off += CH) {
        const size_t len = std::min(CH, bytes - off);
        BH_HIP(hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, src + off, len, hipMemcpyHostToDevice, e->stream),
               "checkpoint upload");
        BH_TRY(sync(e));
    }
    return BH_OK;
}

int bh_qwen3_load(bh_qwen3* e, const char* path) {
    if (!e || !path) return fail(BH_ERR_INVALID, "bh_qwen3_load: null argument");
    (void)hipSetDevice(e->device);
    bh::StFile f;
    std::string err;
    if (!f.open(path, &err)) return fail(BH_ERR_INVALID, "bh_qwen3_load: %s", err.c_str());
    for (const std::string& name : param_names(e->c)) {
        Target t;
        BH_TRY(resolve(e, name, &t));
        const bh::StTensor* st = f.find(name);
        if (!st) return fail(BH_ERR_INVALID, "bh_qwen3_load: %s has no tensor '%s'", path, name.c_str());
        uint64_t elems = 1;
        for (uint64_t d : st->shape) elems *= d;
        if (t.is_emb && st->dtype == bh::ST_U32) {
            // A quantized embedding, as the reference's importer writes it
            // (should_quantize takes every rank-2 tensor with k % 4 == 0,
            // crates/qwen3omnimoe/src/import.rs:349-351, 622-623): the gather
            // table is its dequantization (crates/model/src/int8.rs:70-87) and
            // a tied head takes the packed words and scales as they are.
            const uint64_t d = e->c.d_model, vocab = e->c.vocab;
            const bh::StTensor* sc = f.find(name + ".scale");
            if (st->shape.size() != 2 || st->shape[0] != vocab || st->shape[1] * 4 != d)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: packed '%s' must be U32 [%llu, %llu]", name.c_str(),
                            (unsigned long long)vocab, (unsigned long long)(d / 4));
            if (!sc || sc->dtype != bh::ST_F32 || sc->shape.size() != 1 || sc->shape[0] != vocab)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: '%s.scale' must be F32 [%llu]", name.c_str(),
                            (unsigned long long)vocab);
            // Tied: straight into the head's buffers. Untied: staged in tmpw
            // (vocab*d floats hold the vocab*d code bytes and the vocab scales).
            uint32_t* pk = e->c.tie_embeddings ? e->head : reinterpret_cast<uint32_t*>(e->tmpw);
            float* sv = e->c.tie_embeddings ? e->shead : e->tmpw + vocab * d / 4;
            BH_TRY(upload_chunked(e, pk, f.bytes(*st), vocab * d));
            BH_TRY(upload_chunked(e, sv, f.bytes(*sc), vocab * 4));
            dequantize_rows_kernel<<<grid_for(vocab * d / 4), 256, 0, e->stream>>>(pk, sv, vocab, d / 4, e->emb);
            BH_HIP(hipGetLastError(), "dequantize launch");
            continue;
        }
        if (t.f32) {
            if (st->dtype != bh::ST_F32 || elems != t.n)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: '%s' must be F32 with %llu elements", name.c_str(),
                            (unsigned long long)t.n);
            BH_TRY(upload_chunked(e, t.f32, f.bytes(*st), elems * 4));
            if (t.is_emb && e->c.tie_embeddings)
                BH_TRY(quantize_into(e, e->emb, e->c.vocab, e->c.d_model, e->head, e->shead));
            continue;
        }
        if (st->dtype == bh::ST_U32) {
            const bh::StTensor* sc = f.find(name + ".scale");
            if (st->shape.size() != 2 || st->shape[0] != t.n || st->shape[1] * 4 != t.k)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: packed '%s' must be U32 [%llu, %llu]", name.c_str(),
                            (unsigned long long)t.n, (unsigned long long)(t.k / 4));
            if (!sc || sc->dtype != bh::ST_F32 || sc->shape.size() != 1 || sc->shape[0] != t.n)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: '%s.scale' must be F32 [%llu]", name.c_str(),
                            (unsigned long long)t.n);
            BH_TRY(upload_chunked(e, t.packed, f.bytes(*st), t.n * t.k));
            BH_TRY(upload_chunked(e, t.scale, f.bytes(*sc), t.n * 4));
        } else if (st->dtype == bh::ST_F32) {
            if (st->shape.size() != 2 || st->shape[0] != t.n || st->shape[1] != t.k)
                return fail(BH_ERR_INVALID, "bh_qwen3_load: '%s' must be [%llu, %llu]", name.c_str(),
                            (unsigned long long)t.n, (unsigned long long)t.k);
            BH_TRY(upload_chunked(e, e->tmpw, f.bytes(*st), elems * 4));
            BH_TRY(quantize_into(e, e->tmpw, (uint32_t)t.n, (uint32_t)t.k, t.packed, t.scale));
        } else {
            return fail(BH_ERR_INVALID, "bh_qwen3_load: '%s' has an unsupported dtype", name.c_str());
        }
    }
    return sync(e);
}

int bh_qwen3_autotune(bh_qwen3* e, uint32_t reps) {
    if (!e) return fail(BH_ERR_INVALID, "bh_qwen3_autotune: null engine");
    const char* off = getenv("BRAIN_NO_AUTOTUNE");
    if (off && strcmp(off, "1") == 0) return 0;
    (void)hipSetDevice(e->device);
    const uint32_t d = e->c.d_model, ff = e->c.d_ff;
    const uint32_t shapes[5][2] = {{e->W, d}, {d, e->hq}, {2 * ff, d}, {d, ff}, {e->c.vocab, d}};  // (n, k)
    int measured = 0;
    for (uint32_t m = 1; m <= 32 && m <= std::max<uint32_t>(1, e->max_batch); m <<= 1)
        for (const auto& sh : shapes) {
            int v = 0;
            float ms[2];
            BH_TRY(bh_tune_i8(e->stream, m, sh[1], sh[0], reps ? reps : 8, &v, ms));
            ++measured;
        }
    if (e->graph) {  // the captured step baked in the old choices
        (void)hipGraphExecDestroy(e->graph);
        e->graph = nullptr;
    }
    return measured;
}

int bh_qwen3_set_kv_clip(bh_qwen3* e, uint32_t layer, uint32_t which, const float* clip) {
    if (!e || !clip || layer >= e->c.n_layers || which > 1)
        return fail(BH_ERR_INVALID, "bh_qwen3_set_kv_clip: bad argument");
    (void)hipSetDevice(e->device);
    float* dst = (which ? e->vclip : e->kclip) + (size_t)layer * e->c.n_kv_heads;
    BH_HIP(hipMemcpyAsync(dst, clip, e->c.n_kv_heads * 4, hipMemcpyHostToDevice, e->stream), "upload");
    return sync(e);
}

int bh_qwen3_init_random(bh_qwen3* e, uint64_t seed) {
    if (!e) return fail(BH_ERR_INVALID, "bh_qwen3_init_random: null engine");
    (void)hipSetDevice(e->device);
    for (const std::string& name : param_names(e->c)) {
        Target t;
        BH_TRY(resolve(e, name, &t));
        const uint64_t key = splitmix_host(seed ^ fnv1a(name));
        if (t.f32) {
            if (t.is_emb) {
                init_normal_kernel<<<grid_for(t.n), 256, 0, e->stream>>>(t.f32, t.n, key, t.init_std);
                if (e->c.tie_embeddings) BH_TRY(quantize_into(e, e->emb, e->c.vocab, e->c.d_model, e->head, e->shead));
            } else {
                fill_kernel<<<grid_for(t.n), 256, 0, e->stream>>>(t.f32, t.n, 1.0f);
            }
        } else {
            const uint64_t n = t.n * t.k;
            if (n > e->tmpw_floats) return fail(BH_ERR_INVALID, "bh_qwen3_init_random: %s exceeds the staging buffer", name.c_str());
            init_normal_kernel<<<grid_for(n), 256, 0, e->stream>>>(e->tmpw, n, key, t.init_std);
            BH_TRY(quantize_into(e, e->tmpw, (uint32_t)t.n, (uint32_t)t.k, t.packed, t.scale));
        }
        BH_HIP(hipGetLastError(), "init launch");
    }
    return sync(e);
}

int bh_qwen3_prefill(bh_qwen3* e, const uint32_t* tokens, uint32_t batch, uint32_t len, uint32_t* next) {
    if (!e || !tokens || !next) return fail(BH_ERR_INVALID, "bh_qwen3_prefill: null argument");
    if (!batch || batch > e->max_batch || !len || len > e->max_seq)
        return fail(BH_ERR_INVALID, "bh_qwen3_prefill: batch %u (max %u), len %u (max %u)", batch, e->max_batch, len,
                    e->max_seq);
    e->nofuse = false;  // the decode flag does not carry over
    BH_TRY(check_blocks(e, batch, len, "bh_qwen3_prefill"));
    for (uint64_t i = 0; i < (uint64_t)batch * len; ++i)
        if (tokens[i] >= e->c.vocab) return fail(BH_ERR_INVALID, "bh_qwen3_prefill: token %u outside the vocabulary (%u)", tokens[i], e->c.vocab);
    (void)hipSetDevice(e->device);
    const uint32_t chunk = std::max<uint32_t>(1, e->max_rows / batch);
    std::vector<uint32_t> tok, pos, seq;
    std::vector<int> map(batch);
    for (uint32_t p0 = 0; p0 < len; p0 += chunk) {
        const uint32_t cc = std::min(chunk, len - p0);
        const uint32_t rows = batch * cc;
        tok.resize(rows);
        pos.resize(rows);
        seq.resize(rows);
        for (uint32_t b = 0; b < batch; ++b)
            for (uint32_t i = 0; i < cc; ++i) {
                const uint32_t r = b * cc + i;
                tok[r] = tokens[(size_t)b * len + p0 + i];
                pos[r] = p0 + i;
                seq[r] = b;
            }
        const bool last = p0 + cc == len;
        for (uint32_t b = 0; b < batch; ++b) map[b] = (int)(b * cc + cc - 1);
        BH_TRY(check_span(e, e->tok_rows, rows * 4, "prefill rows"));
        if (last) BH_TRY(check_span(e, e->row_map, batch * 4, "prefill row map"));
        BH_HIP(hipMemcpyAsync(e->tok_rows, tok.data(), rows * 4, hipMemcpyHostToDevice, e->stream), "upload");
        BH_HIP(hipMemcpyAsync(e->pos_rows, pos.data(), rows * 4, hipMemcpyHostToDevice, e->stream), "upload");
        BH_HIP(hipMemcpyAsync(e->seq_rows, seq.data(), rows * 4, hipMemcpyHostToDevice, e->stream), "upload");
        if (last) BH_HIP(hipMemcpyAsync(e->row_map, map.data(), batch * 4, hipMemcpyHostToDevice, e->stream), "upload");
        BH_TRY(run_rows(e, (int)rows, e->tok_rows, e->pos_rows, e->seq_rows, last ? (int)batch : 0, e->row_map, false,
                        (int)((p0 + cc + KCH - 1) / KCH), (int)cc));
        BH_TRY(sync(e));  // the host vectors are reused by the next chunk
    }
    std::vector<uint32_t> pdec(batch, len);
    const uint32_t ctl[2] = {len, e->max_seq};
    BH_TRY(check_span(e, e->pos_dec, batch * 4, "prefill positions"));
    BH_TRY(check_span(e, e->tok_dec, batch * 4, "prefill tokens"));
    BH_HIP(hipMemcpyAsync(e->pos_dec, pdec.data(), batch * 4, hipMemcpyHostToDevice, e->stream), "upload");
    BH_HIP(hipMemcpyAsync(e->ctl, ctl, sizeof ctl, hipMemcpyHostToDevice, e->stream), "upload");
    BH_HIP(hipMemcpyAsync(next, e->tok_dec, batch * 4, hipMemcpyDeviceToHost, e->stream), "download");
    BH_TRY(sync(e));
    e->batch = batch;
    e->prompt_len = len;
    e->decoded = 0;
    return BH_OK;
}

int bh_qwen3_decode(bh_qwen3* e, uint32_t steps, uint32_t flags, uint32_t* out) {
    if (!e || (steps && !out)) return fail(BH_ERR_INVALID, "bh_qwen3_decode: null argument");
    if (!e->batch) return fail(BH_ERR_INVALID, "bh_qwen3_decode: no live sequences (call bh_qwen3_prefill)");
    if ((uint64_t)e->prompt_len + e->decoded + steps > e->max_seq)
        return fail(BH_ERR_INVALID, "bh_qwen3_decode: %u more steps exceed max_seq %u", steps, e->max_seq);
    if (!steps) return BH_OK;
    BH_TRY(check_blocks(e, e->batch, (uint64_t)e->prompt_len + e->decoded + steps, "bh_qwen3_decode"));
    (void)hipSetDevice(e->device);
    const int b = (int)e->batch;
    e->nofuse = (flags & BH_QWEN3_UNFUSED) != 0;
    if (flags & BH_QWEN3_EAGER) {
        for (uint32_t s = 0; s < steps; ++s)
            BH_TRY(run_rows(e, b, e->tok_dec, e->pos_dec, e->seq_dec, b, nullptr, true, (int)e->max_splits));
    } else {
        if (!e->graph || e->graph_batch != e->batch || e->graph_nofuse != e->nofuse) {
            if (e->graph) {
                (void)hipGraphExecDestroy(e->graph);
                e->graph = nullptr;
            }
            BH_TRY(reserve_linears(e, b));
            hipGraph_t g = nullptr;
            BH_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "begin capture");
            const int rc = run_rows(e, b, e->tok_dec, e->pos_dec, e->seq_dec, b, nullptr, true, (int)e->max_splits);
            const hipError_t ce = hipStreamEndCapture(e->stream, &g);
            if (rc != BH_OK) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            BH_HIP(ce, "end capture");
            const hipError_t ie = hipGraphInstantiate(&e->graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            BH_HIP(ie, "graph instantiate");
            e->graph_batch = e->batch;
            e->graph_nofuse = e->nofuse;
        }
        for (uint32_t s = 0; s < steps; ++s) BH_HIP(hipGraphLaunch(e->graph, e->stream), "graph launch");
    }
    BH_TRY(check_span(e, e->hist + (size_t)e->decoded * b, (size_t)steps * b * 4, "decoded tokens"));
    BH_HIP(hipMemcpyAsync(out, e->hist + (size_t)e->decoded * b, (size_t)steps * b * 4, hipMemcpyDeviceToHost, e->stream),
           "download");
    BH_TRY(sync(e));
    e->decoded += steps;
    return BH_OK;
}

int bh_qwen3_logits(bh_qwen3* e, float* out, uint64_t n) {
    if (!e || !out) return fail(BH_ERR_INVALID, "bh_qwen3_logits: null argument");
    const uint64_t want = (uint64_t)e->batch * e->c.vocab;
    if (!e->batch || n < want) return fail(BH_ERR_INVALID, "bh_qwen3_logits: need %llu floats", (unsigned long long)want);
    (void)hipSetDevice(e->device);
    BH_TRY(check_span(e, e->logits, want * 4, "logits"));
    BH_HIP(hipMemcpyAsync(out, e->logits, want * 4, hipMemcpyDeviceToHost, e->stream), "download");
    return sync(e);
}

int bh_qwen3_kv_read(bh_qwen3* e, uint32_t layer, uint32_t seq, uint32_t which, uint32_t pos0, uint32_t npos,
                     void* data, float* scales) {
    if (!e || !data || which > 1 || layer >= e->c.n_layers || seq >= e->max_batch ||
        (uint64_t)pos0 + npos > e->max_seq)
        return fail(BH_ERR_INVALID, "bh_qwen3_kv_read: bad argument");
    (void)hipSetDevice(e->device);
    const size_t nkv = e->c.n_kv_heads, row = (size_t)e->hkv * e->kv_elem;
    const uint8_t* cache = static_cast<const uint8_t*>(which ? e->vc : e->kc) + (size_t)layer * e->layer_kv * e->kv_elem;
    const float* sc = (which ? e->vscale : e->kscale) + (size_t)layer * e->slots * nkv;
    // Runs of positions that are contiguous in the cache: the whole range
    // with slabs, one block at a time in a paged pool.
    for (uint32_t p = pos0; p < pos0 + npos;) {
        size_t tok;
        uint32_t run;
        if (e->kv_bs) {
            const uint32_t blk = e->bt_host[(size_t)seq * e->kv_max_bt + p / e->kv_bs];
            if (blk >= e->kv_nblk)
                return fail(BH_ERR_INVALID, "bh_qwen3_kv_read: position %u of sequence %u has no block", p, seq);
            tok = (size_t)blk * e->kv_bs + p % e->kv_bs;
            run = std::min(pos0 + npos - p, e->kv_bs - p % e->kv_bs);
        } else {
            tok = (size_t)seq * e->max_seq + p;
            run = pos0 + npos - p;
        }
        uint8_t* dst = static_cast<uint8_t*>(data) + (size_t)(p - pos0) * row;
        BH_TRY(check_span(e, cache + tok * row, (size_t)run * row, "kv read"));
        BH_HIP(hipMemcpyAsync(dst, cache + tok * row, (size_t)run * row, hipMemcpyDeviceToHost, e->stream), "kv read");
        if (e->c.kv_int8 && scales) {
            BH_TRY(check_span(e, sc + tok * nkv, (size_t)run * nkv * 4, "kv scale read"));
            BH_HIP(hipMemcpyAsync(scales + (size_t)(p - pos0) * nkv, sc + tok * nkv, (size_t)run * nkv * 4,
                                  hipMemcpyDeviceToHost, e->stream),
                   "kv scale read");
        }
        p += run;
    }
    return sync(e);
}

int bh_qwen3_kv_pool(bh_qwen3* e, uint32_t layer, uint32_t which, void** pool, uint64_t* pool_words, float** scales,
                     uint64_t* n_scales) {
    if (!e || !pool || !pool_words || !scales || !n_scales || which > 1 || layer >= e->c.n_layers)
        return fail(BH_ERR_INVALID, "bh_qwen3_kv_pool: bad argument");
    *pool = static_cast<uint8_t*>(which ? e->vc : e->kc) + (size_t)layer * e->layer_kv * e->kv_elem;
    *pool_words = e->layer_kv * e->kv_elem / 4;
    *scales = e->c.kv_int8 ? (which ? e->vscale : e->kscale) + (size_t)layer * e->slots * e->c.n_kv_heads : nullptr;
    *n_scales = e->c.kv_int8 ? e->slots * e->c.n_kv_heads : 0;
    return BH_OK;
}

int bh_qwen3_set_block_table(bh_qwen3* e, const uint32_t* table, uint32_t rows, uint32_t max_blocks_per_seq) {
    if (!e || !table) return fail(BH_ERR_INVALID, "bh_qwen3_set_block_table: null argument");
    if (!e->kv_bs) return fail(BH_ERR_INVALID, "bh_qwen3_set_block_table: the engine keeps slabs (kv_block_size 0)");
    if (rows > e->max_batch || max_blocks_per_seq != e->kv_max_bt)
        return fail(BH_ERR_INVALID, "bh_qwen3_set_block_table: %u rows of %u blocks (engine: up to %u rows of %u)",
                    rows, max_blocks_per_seq, e->max_batch, e->kv_max_bt);
    for (uint64_t i = 0; i < (uint64_t)rows * max_blocks_per_seq; ++i)
        if (table[i] >= e->kv_nblk && table[i] != BH_QWEN3_NO_BLOCK)
            return fail(BH_ERR_INVALID, "bh_qwen3_set_block_table: entry %u outside the pool of %u blocks", table[i],
                        e->kv_nblk);
    (void)hipSetDevice(e->device);
    std::copy(table, table + (size_t)rows * max_blocks_per_seq, e->bt_host.begin());
    std::fill(e->bt_host.begin() + (size_t)rows * max_blocks_per_seq, e->bt_host.end(), BH_QWEN3_NO_BLOCK);
    // Ordered on the engine's stream after any step still reading the table.
    BH_HIP(hipMemcpyAsync(e->bt, e->bt_host.data(), e->bt_host.size() * 4, hipMemcpyHostToDevice, e->stream),
           "block table upload");
    return sync(e);
}

int bh_qwen3_lengths(bh_qwen3* e, uint32_t* len, uint32_t batch) {
    if (!e || !len || batch < e->batch) return fail(BH_ERR_INVALID, "bh_qwen3_lengths: bad argument");
    for (uint32_t b = 0; b < e->batch; ++b) len[b] = e->prompt_len + e->decoded;
    return BH_OK;
}

}  // extern "C"
