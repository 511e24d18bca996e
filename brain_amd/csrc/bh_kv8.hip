// The int8 paged KV cache kernels of brain's int8 serving path, as Backend
// step names and typed calls:
//   paged_kv_append_i8_clipped_batched  crates/kernels/wgsl/paged_kv_append_i8_clipped_batched.wgsl:46-77
//   paged_decode_scores_i8_batched      crates/kernels/wgsl/paged_decode_scores_i8_batched.wgsl:28-54
//   paged_decode_apply_i8_batched       crates/kernels/wgsl/paged_decode_apply_i8_batched.wgsl:28-53
// The pool holds int8 codes (4 per u32 word, little-endian) at slot
// physical*block_size + offset, kv_stride bytes per slot; one f32 scale per
// (slot, kv head).
//
// Each output keeps the reference's own summation order (a score sums its
// head_dim products in order, a context element its positions in order), so
// the f32 results are the reference's bit for bit; the parallelism is across
// outputs. Block tables, offsets and sequence lengths are read on the device,
// so the slots they name are checked there against the pool and scale
// lengths the caller passes: an entry outside them is skipped (nothing
// stored, nothing added) instead of the reference's out-of-bounds access.
#include "bh_common.h"
#include "bh_kv8.h"

namespace bh {

// One wave per (sequence, kv head); lane l owns word l of the head (head_dim
// <= 256). The head's absmax is exact in any order.
__global__ __launch_bounds__(64) void paged_kv_append_i8_kernel(const float* src, const uint32_t* blocks,
                                                                const uint32_t* offsets, const float* clip,
                                                                uint32_t* pool, uint64_t pool_words, float* scales,
                                                                uint64_t n_scales, uint32_t kv_stride, uint32_t bs,
                                                                uint32_t hd) {
    const uint32_t n_kv = kv_stride / hd;
    const uint32_t b = blockIdx.x / n_kv, head = blockIdx.x % n_kv;
    const uint32_t lane = threadIdx.x;
    const bool live = 4 * lane < hd;
    const float* x = src + (uint64_t)b * kv_stride + (uint64_t)head * hd + 4 * lane;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    float mx = 0.0f;
    if (live) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = x[j];
            mx = fmaxf(mx, fabsf(v[j]));
        }
    }
    mx = xor_max<32>(mx);
    float scale = fminf(mx, clip[head]) / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const uint64_t slot = (uint64_t)blocks[b] * bs + offsets[b];
    const uint64_t base = slot * kv_stride + (uint64_t)head * hd;  // a multiple of 4
    if (slot * n_kv + head >= n_scales || (base + hd) / 4 > pool_words) return;
    if (lane == 0) scales[slot * n_kv + head] = scale;
    if (live) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w |= (uint32_t)kv8_code(v[j], scale) << (8 * j);
        pool[base / 4 + lane] = w;
    }
}

__device__ __forceinline__ float code_f(uint32_t w, int e) { return (float)(int8_t)(uint8_t)(w >> (8 * e)); }


// Slot of position j of sequence b, or false when the tables name one
// outside the pool.
__device__ __forceinline__ bool slot_of(const PagedReadArgs& a, uint32_t b, uint32_t j, uint32_t kvh, uint64_t& slot) {
    const uint32_t blk = j / a.bs;
    if (blk >= a.max_bt) return false;
    slot = (uint64_t)a.bt[(uint64_t)b * a.max_bt + blk] * a.bs + j % a.bs;
    const uint32_t n_kv = a.kv_stride / a.hd;
    return slot * n_kv + kvh < a.n_scales && (slot * a.kv_stride + (uint64_t)kvh * a.hd + a.hd + 3) / 4 <= a.pool_words;
}

// One thread per score (b, h, j): q . f32(codes) in head_dim order, then
// (acc * kscale) * scale. A workgroup takes 64 consecutive positions of one
// (b, h), so q is the same for the whole workgroup. Positions at or past the
// sequence length are not written.
template <bool VEC>
__global__ __launch_bounds__(64) void paged_decode_scores_i8_kernel(PagedReadArgs a) {
    const uint32_t nchunk = (a.cap + 63) / 64;
    const uint32_t bh = blockIdx.x / nchunk;
    const uint32_t j = (blockIdx.x % nchunk) * 64 + threadIdx.x;
    const uint32_t b = bh / a.n_heads, h = bh % a.n_heads;
    if (j >= a.cap || j >= a.seq_lens[b]) return;
    const uint32_t kvh = h / a.group;
    uint64_t slot;
    if (!slot_of(a, b, j, kvh, slot)) return;
    const float qscale = a.scales[slot * (a.kv_stride / a.hd) + kvh];
    const uint64_t base = slot * a.kv_stride + (uint64_t)kvh * a.hd;
    const float* q = a.in + (uint64_t)bh * a.hd;
    float acc = 0.0f;
    if constexpr (VEC) {  // base and hd multiples of 16 bytes, pool 16-byte aligned
        const uint4* p = reinterpret_cast<const uint4*>(a.pool) + base / 16;
        for (uint32_t d = 0; d < a.hd; d += 16) {
            const uint4 w = p[d / 16];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = acc + q[d + 4 * i + e] * code_f(ws[i], e);
        }
    } else {
        for (uint32_t d = 0; d < a.hd; d += 4) {
            const uint32_t w = a.pool[(base + d) / 4];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = acc + q[d + e] * code_f(w, e);
        }
    }
    a.out[(uint64_t)bh * a.cap + j] = acc * qscale * a.scale;
}

// One thread per context element (b, h, d): the sum over positions j in
// order of (p_j * f32(code)) * vscale. A workgroup takes 64 consecutive d
// of one (b, h): the probabilities, table entries and scales it reads are
// the same for every lane. Loads for 8 positions go out before their adds.
__global__ __launch_bounds__(64) void paged_decode_apply_i8_kernel(PagedReadArgs a) {
    const uint32_t nchunk = (a.hd + 63) / 64;
    const uint32_t bh = blockIdx.x / nchunk;
    const uint32_t d = (blockIdx.x % nchunk) * 64 + threadIdx.x;
    const uint32_t b = bh / a.n_heads, h = bh % a.n_heads;
    const uint32_t kvh = h / a.group, n_kv = a.kv_stride / a.hd;
    const uint32_t t = min(a.seq_lens[b], a.cap);
    const float* pr = a.in + (uint64_t)bh * a.cap;
    const uint8_t* pool8 = reinterpret_cast<const uint8_t*>(a.pool);
    const bool live = d < a.hd;
    float acc = 0.0f;
    constexpr int U = 8;
    for (uint32_t j0 = 0; j0 < t; j0 += U) {
        float pv[U], sv[U], cv[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint64_t slot = 0;
            ok[u] = j0 + u < t && slot_of(a, b, j0 + u, kvh, slot);
            pv[u] = ok[u] ? pr[j0 + u] : 0.0f;
            sv[u] = ok[u] ? a.scales[slot * n_kv + kvh] : 0.0f;
            cv[u] = ok[u] && live ? (float)(int8_t)pool8[slot * a.kv_stride + (uint64_t)kvh * a.hd + d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (ok[u]) acc = acc + pv[u] * cv[u] * sv[u];
    }
    if (live) a.out[(uint64_t)b * a.n_heads * a.hd + (uint64_t)h * a.hd + d] = acc;
}

hipError_t launch_paged_kv_append_i8(hipStream_t s, const float* src, const uint32_t* blocks, const uint32_t* offsets,
                                     const float* clip, uint32_t* pool, uint64_t pool_words, float* scales,
                                     uint64_t n_scales, uint32_t batch, uint32_t kv_stride, uint32_t bs, uint32_t hd) {
    const uint64_t grid = (uint64_t)batch * (kv_stride / hd);
    if (grid == 0) return hipSuccess;
    paged_kv_append_i8_kernel<<<(unsigned)grid, 64, 0, s>>>(src, blocks, offsets, clip, pool, pool_words, scales,
                                                            n_scales, kv_stride, bs, hd);
    return hipGetLastError();
}

hipError_t launch_paged_decode_i8(hipStream_t s, bool apply, const PagedReadArgs& a, uint32_t batch) {
    if (!apply) {
        const uint64_t grid = (uint64_t)batch * a.n_heads * ((a.cap + 63) / 64);
        if (grid == 0) return hipSuccess;
        const bool vec = a.hd % 16 == 0 && a.kv_stride % 16 == 0 && (reinterpret_cast<uintptr_t>(a.pool) & 15) == 0;
        if (vec) paged_decode_scores_i8_kernel<true><<<(unsigned)grid, 64, 0, s>>>(a);
        else paged_decode_scores_i8_kernel<false><<<(unsigned)grid, 64, 0, s>>>(a);
    } else {
        const uint64_t grid = (uint64_t)batch * a.n_heads * ((a.hd + 63) / 64);
        if (grid == 0) return hipSuccess;
        paged_decode_apply_i8_kernel<<<(unsigned)grid, 64, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace bh
