// Per-token activation quantization and per-channel weight quantization on gfx950.
//
// Reference semantics restated here (paths under the swedishembedded/brain tree):
//   max_abs_row  crates/kernels/wgsl/max_abs_row.wgsl:27-34 (== max_abs_rows.wgsl:60-84)
//       sx[m] = max(max_k |x[m,k]|, 1e-8) / 127
//   quant_pack   crates/kernels/wgsl/quant_pack.wgsl:29-44
//       inv = 1/sx[m]; q = clamp(round_ties_even(x*inv), -127, 127); 4 bytes per u32, LE along K
//   quantize_weight crates/model/src/int8.rs:33-59 (host; rounding ties AWAY from zero)
//
// `max` is exact, so any reduction order gives the same scale; 1/sx is an
// IEEE-correct division (the library is built with correctly rounded fp32
// divide) and x*inv is a single rounded product, so the packed bytes are
// bit-identical to a serial host evaluation.
#include "bh_common.h"

namespace bh {

constexpr int QT = 256;  // threads per row block (4 wave64)

// Row max|x| over `k` floats with a block of QT threads. VEC: float4 loads
// (row base 16-byte aligned, k % 4 == 0).
template <bool VEC>
__device__ __forceinline__ float row_absmax(const float* __restrict__ row, int k) {
    float a = 0.0f;
    if constexpr (VEC) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
        for (int i = threadIdx.x; i < (k >> 2); i += QT) {
            float4 v = r4[i];
            a = fmaxf(a, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int i = threadIdx.x; i < k; i += QT) a = fmaxf(a, fabsf(row[i]));
    }
    a = xor_max<32>(a);
    __shared__ float red[QT / 64];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = a;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < QT / 64; ++w) m = fmaxf(m, red[w]);
    return m;
}

template <bool VEC>
__global__ __launch_bounds__(QT) void max_abs_rows_kernel(const float* __restrict__ x, int m, int k,
                                                          float* __restrict__ sx) {
    const int row = blockIdx.x;
    if (row >= m) return;
    float a = row_absmax<VEC>(x + (int64_t)row * k, k);
    if (threadIdx.x == 0) sx[row] = fmaxf(a, 1e-8f) / 127.0f;
}

// One thread per packed output word (M*K/4 words), as quant_pack.wgsl.
template <bool VEC>
__global__ __launch_bounds__(QT) void quant_pack_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ sx, int m, int k,
                                                        uint32_t* __restrict__ xq) {
    const int kg = k >> 2;
    const int64_t total = (int64_t)m * kg;
    for (int64_t idx = (int64_t)blockIdx.x * QT + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * QT) {
        const int64_t r = idx / kg;
        const float inv = 1.0f / sx[r];
        float4 v;
        if constexpr (VEC) {
            v = reinterpret_cast<const float4*>(x)[idx];  // row r, group g: floats 4*idx
        } else {
            const float* p = x + idx * 4;
            v = make_float4(p[0], p[1], p[2], p[3]);
        }
        xq[idx] = quant_word(v, inv);
    }
}

// max_abs_row and quant_pack fused, single pass: one block per row, each
// thread keeps its NV float4s of the row in registers across the block max,
// so the row is read from memory once. Same arithmetic as the pair.
template <int NV>
__global__ __launch_bounds__(QT) void quantize_rows_reg_kernel(const float* __restrict__ x, int m, int k,
                                                               float* __restrict__ sx, uint32_t* __restrict__ xq) {
    const int row = blockIdx.x;
    if (row >= m) return;
    const int kg = k >> 2;
    const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)row * k);
    float4 v[NV];
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + i * QT;
        v[i] = g < kg ? xr[g] : make_float4(0.f, 0.f, 0.f, 0.f);
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    a = xor_max<32>(a);
    __shared__ float red[QT / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < QT / 64; ++w) mx = fmaxf(mx, red[w]);
    const float s = fmaxf(mx, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sx[row] = s;
    const float inv = 1.0f / s;
    uint32_t* q = xq + (int64_t)row * kg;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + i * QT;
        if (g < kg) q[g] = quant_word(v[i], inv);
    }
}

// max_abs_row and quant_pack fused, two passes (long or unaligned rows): the
// row is read twice (the second read hits L2), sx written once.
// One wave per row, four rows per block (rows of at most 64*NV float4): the
// row max is a wave reduction with no block barrier, and a
// block carries four rows' worth of loads. The same arithmetic as the block
// kernel above (the max is exact in any order).
template <int NV>
__global__ __launch_bounds__(QT) void quantize_rows_wave_kernel(const float* __restrict__ x, int m, int k,
                                                                float* __restrict__ sx, uint32_t* __restrict__ xq) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (QT / 64) + (threadIdx.x >> 6);
    if (row >= m) return;
    const int kg = k >> 2;
    const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)row * k);
    float4 v[NV];
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = lane + i * 64;
        v[i] = g < kg ? xr[g] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i)
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    a = xor_max<32>(a);
    const float s = fmaxf(a, 1e-8f) / 127.0f;
    if (lane == 0) sx[row] = s;
    const float inv = 1.0f / s;
    uint32_t* q = xq + (int64_t)row * kg;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = lane + i * 64;
        if (g < kg) q[g] = quant_word(v[i], inv);
    }
}

template <bool VEC>
__global__ __launch_bounds__(QT) void quantize_rows_kernel(const float* __restrict__ x, int m, int k,
                                                           float* __restrict__ sx,
                                                           uint32_t* __restrict__ xq) {
    const int row = blockIdx.x;
    if (row >= m) return;
    const float* xr = x + (int64_t)row * k;
    float a = row_absmax<VEC>(xr, k);
    const float s = fmaxf(a, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sx[row] = s;
    const float inv = 1.0f / s;
    const int kg = k >> 2;
    uint32_t* q = xq + (int64_t)row * kg;
    for (int g = threadIdx.x; g < kg; g += QT) {
        float4 v;
        if constexpr (VEC) v = reinterpret_cast<const float4*>(xr)[g];
        else v = make_float4(xr[4 * g], xr[4 * g + 1], xr[4 * g + 2], xr[4 * g + 3]);
        q[g] = quant_word(v, inv);
    }
}

// Per-token quantization of bf16 activations: widening bf16 to f32 is exact
// (the bits shifted up by 16), so this is quantize_rows on f32(x), bit for
// bit. Register version: each thread keeps NV 16-byte groups (8 values) of the
// row; k % 8 == 0, x 16-byte aligned, k <= 8 * QT * NV.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int NV>
__global__ __launch_bounds__(QT) void quantize_rows_bf16_kernel(const uint16_t* __restrict__ x, int m, int k,
                                                                float* __restrict__ sx, uint32_t* __restrict__ xq) {
    const int row = blockIdx.x;
    if (row >= m) return;
    const int k8 = k >> 3;
    const uint4* xr = reinterpret_cast<const uint4*>(x + (int64_t)row * k);
    uint4 v[NV];
    float a = 0.0f;
    // Every load of the row first, at clamped indices (k8 >= 1), so none
    // waits at a branch join; then the masks and the max.
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = xr[min((int)(threadIdx.x + i * QT), k8 - 1)];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + i * QT;
        if (g >= k8) v[i] = make_uint4(0u, 0u, 0u, 0u);
        const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) a = fmaxf(a, fmaxf(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
    }
    a = xor_max<32>(a);
    __shared__ float red[QT / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < QT / 64; ++w) mx = fmaxf(mx, red[w]);
    const float s = fmaxf(mx, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sx[row] = s;
    const float inv = 1.0f / s;
    uint2* q = reinterpret_cast<uint2*>(xq + (int64_t)row * (k >> 2));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + i * QT;
        if (g >= k8) continue;
        const uint32_t lo = quant_word(make_float4(bf16_lo(v[i].x), bf16_hi(v[i].x), bf16_lo(v[i].y), bf16_hi(v[i].y)), inv);
        const uint32_t hi = quant_word(make_float4(bf16_lo(v[i].z), bf16_hi(v[i].z), bf16_lo(v[i].w), bf16_hi(v[i].w)), inv);
        q[g] = make_uint2(lo, hi);
    }
}

// Any k % 4 == 0 and alignment: two passes of scalar loads.
__global__ __launch_bounds__(QT) void quantize_rows_bf16_any_kernel(const uint16_t* __restrict__ x, int m, int k,
                                                                    float* __restrict__ sx,
                                                                    uint32_t* __restrict__ xq) {
    const int row = blockIdx.x;
    if (row >= m) return;
    const uint16_t* xr = x + (int64_t)row * k;
    float a = 0.0f;
    for (int i = threadIdx.x; i < k; i += QT) a = fmaxf(a, fabsf(__uint_as_float((uint32_t)xr[i] << 16)));
    a = xor_max<32>(a);
    __shared__ float red[QT / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < QT / 64; ++w) mx = fmaxf(mx, red[w]);
    const float s = fmaxf(mx, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sx[row] = s;
    const float inv = 1.0f / s;
    uint32_t* q = xq + (int64_t)row * (k >> 2);
    for (int g = threadIdx.x; g < (k >> 2); g += QT) {
        const float4 v = make_float4(__uint_as_float((uint32_t)xr[4 * g] << 16), __uint_as_float((uint32_t)xr[4 * g + 1] << 16),
                                     __uint_as_float((uint32_t)xr[4 * g + 2] << 16), __uint_as_float((uint32_t)xr[4 * g + 3] << 16));
        q[g] = quant_word(v, inv);
    }
}

// Per-output-row weight quantization (crates/model/src/int8.rs:33-59):
// sw = max(max|w|, 1e-8)/127, q = clamp(round_half_away(w*(1/sw)), +-127),
// NaN -> 0 (Rust's saturating `as i32`).
__device__ __forceinline__ uint32_t wquant_byte(float v, float inv) {
    float q = roundf(v * inv);
    if (q != q) return 0u;
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return (uint32_t)((int)q & 0xff);
}

// One wave per weight row, the row held in registers (K <= 256 NV): read
// once instead of twice, and four short rows per block. The same arithmetic
// as quantize_weight_kernel (the row max is exact in any order).
template <int NV>
__global__ __launch_bounds__(QT) void quantize_weight_wave_kernel(const float* __restrict__ w, int n, int k,
                                                                  uint32_t* __restrict__ packed,
                                                                  float* __restrict__ sw) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (QT / 64) + (threadIdx.x >> 6);
    if (row >= n) return;
    const int kg = k >> 2;
    const float4* wr = reinterpret_cast<const float4*>(w + (int64_t)row * k);
    float4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = lane + i * 64;
        v[i] = g < kg ? wr[g] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    a = xor_max<32>(a);
    const float s = fmaxf(a, 1e-8f) / 127.0f;
    if (lane == 0) sw[row] = s;
    const float inv = 1.0f / s;
    uint32_t* q = packed + (int64_t)row * kg;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = lane + i * 64;
        if (g < kg)
            q[g] = wquant_byte(v[i].x, inv) | (wquant_byte(v[i].y, inv) << 8) | (wquant_byte(v[i].z, inv) << 16) |
                   (wquant_byte(v[i].w, inv) << 24);
    }
}

template <bool VEC>
__global__ __launch_bounds__(QT) void quantize_weight_kernel(const float* __restrict__ w, int n, int k,
                                                             uint32_t* __restrict__ packed,
                                                             float* __restrict__ sw) {
    const int row = blockIdx.x;
    if (row >= n) return;
    const float* wr = w + (int64_t)row * k;
    float a = row_absmax<VEC>(wr, k);
    const float s = fmaxf(a, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sw[row] = s;
    const float inv = 1.0f / s;
    const int kg = k >> 2;
    uint32_t* q = packed + (int64_t)row * kg;
    for (int g = threadIdx.x; g < kg; g += QT) {
        float4 v;
        if constexpr (VEC) v = reinterpret_cast<const float4*>(wr)[g];
        else v = make_float4(wr[4 * g], wr[4 * g + 1], wr[4 * g + 2], wr[4 * g + 3]);
        q[g] = wquant_byte(v.x, inv) | (wquant_byte(v.y, inv) << 8) | (wquant_byte(v.z, inv) << 16) |
               (wquant_byte(v.w, inv) << 24);
    }
}

static inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch_max_abs_rows(hipStream_t s, const float* x, int m, int k, float* sx) {
    if (m <= 0) return hipSuccess;
    const bool vec = (k % 4 == 0) && al16(x);
    if (vec) max_abs_rows_kernel<true><<<m, QT, 0, s>>>(x, m, k, sx);
    else max_abs_rows_kernel<false><<<m, QT, 0, s>>>(x, m, k, sx);
    return hipGetLastError();
}

hipError_t launch_quant_pack(hipStream_t s, const float* x, const float* sx, int m, int k, uint32_t* xq) {
    const int64_t total = (int64_t)m * (k / 4);
    if (total <= 0) return hipSuccess;
    int64_t blocks = (total + QT - 1) / QT;
    if (blocks > 65536) blocks = 65536;
    if (al16(x)) quant_pack_kernel<true><<<(unsigned)blocks, QT, 0, s>>>(x, sx, m, k, xq);
    else quant_pack_kernel<false><<<(unsigned)blocks, QT, 0, s>>>(x, sx, m, k, xq);
    return hipGetLastError();
}

hipError_t launch_quantize_rows_bf16(hipStream_t s, const uint16_t* x, int m, int k, float* sx, uint32_t* xq) {
    if (m <= 0) return hipSuccess;
    const int k8 = k / 8;
    if (k % 8 == 0 && al16(x) && k8 >= 1 && k8 <= 8 * QT) {
        if (k8 <= QT) quantize_rows_bf16_kernel<1><<<m, QT, 0, s>>>(x, m, k, sx, xq);
        else if (k8 <= 2 * QT) quantize_rows_bf16_kernel<2><<<m, QT, 0, s>>>(x, m, k, sx, xq);
        else if (k8 <= 4 * QT) quantize_rows_bf16_kernel<4><<<m, QT, 0, s>>>(x, m, k, sx, xq);
        else if (k8 <= 5 * QT) quantize_rows_bf16_kernel<5><<<m, QT, 0, s>>>(x, m, k, sx, xq);  // K = 10240: no clamped repeats
        else quantize_rows_bf16_kernel<8><<<m, QT, 0, s>>>(x, m, k, sx, xq);
    } else {
        quantize_rows_bf16_any_kernel<<<m, QT, 0, s>>>(x, m, k, sx, xq);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, float* sx, uint32_t* xq) {
    if (m <= 0) return hipSuccess;
    const int kg = k / 4;
    // Short rows, many of them: a wave per row (measured at K = 1024: 12.4 ->
    // 9.8 us for 8192 rows, 4.7 -> 4.5 us for 2048; slower than a block per
    // row from K = 3072 and for few rows).
    if (al16(x) && kg <= 4 * 64 && m >= 1024) {
        quantize_rows_wave_kernel<4><<<(m + QT / 64 - 1) / (QT / 64), QT, 0, s>>>(x, m, k, sx, xq);
    } else if (al16(x) && kg <= 4 * QT) {
        if (kg <= QT) quantize_rows_reg_kernel<1><<<m, QT, 0, s>>>(x, m, k, sx, xq);
        else if (kg <= 2 * QT) quantize_rows_reg_kernel<2><<<m, QT, 0, s>>>(x, m, k, sx, xq);
        else if (kg <= 3 * QT) quantize_rows_reg_kernel<3><<<m, QT, 0, s>>>(x, m, k, sx, xq);  // K = 3072
        else quantize_rows_reg_kernel<4><<<m, QT, 0, s>>>(x, m, k, sx, xq);
    } else if (al16(x)) quantize_rows_kernel<true><<<m, QT, 0, s>>>(x, m, k, sx, xq);
    else quantize_rows_kernel<false><<<m, QT, 0, s>>>(x, m, k, sx, xq);
    return hipGetLastError();
}

hipError_t launch_quantize_weight(hipStream_t s, const float* w, int n, int k, uint32_t* packed, float* sw) {
    if (n <= 0) return hipSuccess;
    const int kg = k / 4;
    // Rows of up to 4096: a wave per row, held in registers (measured 48.8 ->
    // 37.3 us at 11008x4096, 219 -> 138 us at 151936x1024).
    if (al16(w) && k % 4 == 0 && kg >= 1 && kg <= 16 * 64) {
        const int grid = (n + QT / 64 - 1) / (QT / 64);
        if (kg <= 4 * 64) quantize_weight_wave_kernel<4><<<grid, QT, 0, s>>>(w, n, k, packed, sw);
        else if (kg <= 8 * 64) quantize_weight_wave_kernel<8><<<grid, QT, 0, s>>>(w, n, k, packed, sw);
        else quantize_weight_wave_kernel<16><<<grid, QT, 0, s>>>(w, n, k, packed, sw);
    } else if (al16(w)) quantize_weight_kernel<true><<<n, QT, 0, s>>>(w, n, k, packed, sw);
    else quantize_weight_kernel<false><<<n, QT, 0, s>>>(w, n, k, packed, sw);
    return hipGetLastError();
}

}  // namespace bh
