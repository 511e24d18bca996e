// Split-KV decode attention: the merge of the per-chunk partials.
#pragma once

#include "bh_common.h"

namespace bh {

constexpr int ATTN_KCH = 32;  // keys per attention workgroup (one split)
constexpr int ATTN_SB = 16;   // chunks merged in one batch of loads

// Merge of the key chunks of one head, for the four context elements
// d..d+3: M = max m_s, L = sum l_s e^(m_s - M), ctx = sum o_s e^(m_s - M) / L
// over the ns chunks at part_* slot hs..hs+ns-1 (part_o [.., hd] per slot,
// part_ml (m, l) per slot). Up to SB chunks (512 positions) are loaded in
// one batch, all before use, so the merge costs one memory round trip; longer
// rows loop over batches (max first, then the sums), with the same result.
__device__ __forceinline__ float4 attn_combine4(const float* part_o, const float* part_ml, size_t hs, int ns, int d,
                                                int hd) {
    constexpr int SB = ATTN_SB;
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

// The first batch of one head's merge (chunk slots hs..hs+SB-1 below
// `splits`, all in bounds), loaded before the row's position is known so the
// loads overlap the position's; attn_combine_first4 masks the slots past the
// row's chunk count.
struct AttnFirst4 {
    float mv[ATTN_SB], lv[ATTN_SB];
    float4 ov[ATTN_SB];
};
__device__ __forceinline__ void attn_load_first4(const float* part_o, const float* part_ml, size_t hs, int splits, int d,
                                                 int hd, AttnFirst4& b) {
#pragma unroll
    for (int j = 0; j < ATTN_SB; ++j) {
        const bool ld = j < splits;
        b.mv[j] = ld ? part_ml[2 * (hs + j)] : -INFINITY;
        b.lv[j] = ld ? part_ml[2 * (hs + j) + 1] : 0.0f;
        b.ov[j] = ld ? *reinterpret_cast<const float4*>(part_o + (hs + j) * hd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// The context pieces only of attn_load_first4 (HEAD32 merge: the chunk
// statistics are loaded one per lane).
__device__ __forceinline__ void attn_load_first4_o(const float* part_o, size_t hs, int splits, int d, int hd,
                                                   AttnFirst4& b) {
#pragma unroll
    for (int j = 0; j < ATTN_SB; ++j)
        b.ov[j] = j < splits ? *reinterpret_cast<const float4*>(part_o + (hs + j) * hd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// attn_combine_first4 for a head held by one 32-lane half of a wave (head_dim
// 128: 4 context elements per lane) whose chunk statistics sit one per lane:
// lane q of the half holds (m, l) of chunk q (mlq). Every chunk's weight
// e^(m_q - M) is evaluated once, on lane q, instead of on all 32 lanes, and
// read by the others with v_readlane; M is the same maximum, and L and the
// context sum the same products in the same chunk order, so the result is
// attn_combine_first4's bit for bit. ns <= ATTN_SB; whole wave active.
__device__ __forceinline__ float4 attn_combine_head32(float2 mlq, int ns, const AttnFirst4& b) {
    const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int q = (int)(lane & 31u);
    const float mq = q < ns ? mlq.x : -INFINITY;
    const float M = xor_max<16>(mq);
    const float wq = q < ns ? expf(mq - M) : 0.0f;
    const float lwq = mlq.y * wq;
    const bool hi = lane >= 32u;
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < ATTN_SB; ++j) {
        if (j >= ns) continue;
        const float wl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wq), j));
        const float wh = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wq), 32 + j));
        const float ll = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lwq), j));
        const float lh = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lwq), 32 + j));
        const float w = hi ? wh : wl;
        L += hi ? lh : ll;
        o = make_float4(o.x + b.ov[j].x * w, o.y + b.ov[j].y * w, o.z + b.ov[j].z * w, o.w + b.ov[j].w * w);
        // Keeps each chunk's reads next to their use (hoisted, the 64 scalar
        // results outgrow the scalar registers and spill).
        __builtin_amdgcn_sched_barrier(0);
    }
    const float inv = 1.0f / L;
    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// attn_combine4 over ns chunks from a preloaded first batch: the same
// operations in the same order (the one-batch form when ns <= SB, else the
// batched form, which reloads).
__device__ __forceinline__ float4 attn_combine_first4(const float* part_o, const float* part_ml, size_t hs, int ns,
                                                      int d, int hd, const AttnFirst4& b) {
    if (ns > ATTN_SB) return attn_combine4(part_o, part_ml, hs, ns, d, hd);
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < ATTN_SB; ++j) M = fmaxf(M, j < ns ? b.mv[j] : -INFINITY);
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < ATTN_SB; ++j) {
        if (j >= ns) continue;
        const float w = expf(b.mv[j] - M);
        L += b.lv[j] * w;
        o = make_float4(o.x + b.ov[j].x * w, o.y + b.ov[j].y * w, o.z + b.ov[j].z * w, o.w + b.ov[j].w * w);
    }
    const float inv = 1.0f / L;
    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

}  // namespace bh
