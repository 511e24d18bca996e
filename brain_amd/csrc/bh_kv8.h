// Internal interface of bh_kv8.hip (the int8 paged KV kernels).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bh {

struct PagedReadArgs {
    const float* in;  // q [batch][n_heads][hd] (scores) or probs [batch][n_heads][cap] (apply)
    const uint32_t* pool;
    uint64_t pool_words;
    const uint32_t* bt;
    const uint32_t* seq_lens;
    const float* scales;
    uint64_t n_scales;
    float* out;  // scores [batch][n_heads][cap] or ctx [batch][n_heads*hd]
    uint32_t n_heads, group, hd, bs, kv_stride, cap, max_bt;
    float scale;
};

hipError_t launch_paged_kv_append_i8(hipStream_t s, const float* src, const uint32_t* blocks, const uint32_t* offsets,
                                     const float* clip, uint32_t* pool, uint64_t pool_words, float* scales,
                                     uint64_t n_scales, uint32_t batch, uint32_t kv_stride, uint32_t bs, uint32_t hd);
hipError_t launch_paged_decode_i8(hipStream_t s, bool apply, const PagedReadArgs& a, uint32_t batch);

}  // namespace bh
