// Split-KV decode attention: the merge of the per-chunk partials.
#pragma once

#include "bh_common.h"

namespace bh {

constexpr int ATTN_KCH = 32;  // keys per attention workgroup (one split)

// Merge of the key chunks of one head, for the four context elements
// d..d+3: M = max m_s, L = sum l_s e^(m_s - M), ctx = sum o_s e^(m_s - M) / L
// over the ns chunks at part_* slot hs..hs+ns-1 (part_o [.., hd] per slot,
// part_ml (m, l) per slot). Up to SB chunks (512 positions) are loaded in
// one batch, all before use, so the merge costs one memory round trip; longer
// rows loop over batches (max first, then the sums), with the same result.
__device__ __forceinline__ float4 attn_combine4(const float* part_o, const float* part_ml, size_t hs, int ns, int d,
                                                int hd) {
    constexpr int SB = 16;
    if (ns <= SB) {
        float mv[SB], lv[SB];
        float4 ov[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const bool live = j < ns;
            mv[j] = live ? part_ml[2 * (hs + j)] : -INFINITY;
            lv[j] = live ? part_ml[2 * (hs + j) + 1] : 0.0f;
            ov[j] = live ? *reinterpret_cast<const float4*>(part_o + (hs + j) * hd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < SB; ++j) M = fmaxf(M, mv[j]);
        float L = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            if (j >= ns) continue;
            const float w = expf(mv[j] - M);
            L += lv[j] * w;
            o = make_float4(o.x + ov[j].x * w, o.y + ov[j].y * w, o.z + ov[j].z * w, o.w + ov[j].w * w);
        }
        const float inv = 1.0f / L;
        return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    }
    float M = -INFINITY;
    for (int s0 = 0; s0 < ns; s0 += SB) {
        float mv[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) mv[j] = s0 + j < ns ? part_ml[2 * (hs + s0 + j)] : -INFINITY;
#pragma unroll
        for (int j = 0; j < SB; ++j) M = fmaxf(M, mv[j]);
    }
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < ns; s0 += SB) {
        float mv[SB], lv[SB];
        float4 ov[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const bool live = s0 + j < ns;
            mv[j] = live ? part_ml[2 * (hs + s0 + j)] : -INFINITY;
            lv[j] = live ? part_ml[2 * (hs + s0 + j) + 1] : 0.0f;
            ov[j] = live ? *reinterpret_cast<const float4*>(part_o + (hs + s0 + j) * hd + d)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            if (s0 + j >= ns) continue;
            const float w = expf(mv[j] - M);
            L += lv[j] * w;
            o = make_float4(o.x + ov[j].x * w, o.y + ov[j].y * w, o.z + ov[j].z * w, o.w + ov[j].w * w);
        }
    }
    const float inv = 1.0f / L;
    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// Context element group i (4 elements) of row r: head i*4/hd, chunks
// holding positions 0..pos.
__device__ __forceinline__ float4 attn_combine_row4(const float* part_o, const float* part_ml, int r, uint32_t pos,
                                                    int nh, int hd, int splits, int i) {
    const int e = i * 4, h = e / hd, d = e - h * hd;
    const size_t hs = ((size_t)r * nh + h) * splits;
    const int ns = ((int)pos + ATTN_KCH) / ATTN_KCH;
    return attn_combine4(part_o, part_ml, hs, ns, d, hd);
}

}  // namespace bh
