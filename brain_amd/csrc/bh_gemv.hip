// Decode-regime W8A8 GEMV (M <= 32) on gfx950 matrix cores.
//
// Computes the same thing as crates/kernels/wgsl/matmul_i8_gemv.wgsl:39-76:
//   out[m,n] = (f32(sum_k xq[m,k]*wq[n,k]) * sx[m]) * sw[n]
// with xq [M,K/4] u32 and wq [N,K/4] u32 (4 int8 per word, little-endian
// along K), optional bias[n] added after the dequant, f32 or bf16 output.
//
// Design: the weight stream is the only thing that matters (N*K bytes from
// HBM; x is M*K bytes and stays in L2). Instead of the reference's scalar
// DP4A + 64-partial LDS fold, one v_mfma_i32_16x16x64_i8 consumes a 16-column
// x 64-byte slab of W per wave (A = 16 activation rows, B = 16 weight rows),
// so the K-reduction happens inside the matrix core and no cross-lane
// shuffles are needed. M is padded to 16 (or 32 with two A fragments) with
// zero activation rows.
//   block  = 4 waves, one 16-column group, K split across the 4 waves in
//            interleaved 64-byte chunks (the block reads a contiguous 16*K
//            byte region of W; each lane does 16-byte dwordx4 loads)
//   reduce = 4 partial 16x16 i32 tiles summed through LDS (exact: integers)
//   epilogue fused: dequant, bias, bf16 RNE.
#include "bh_common.h"

namespace bh {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = GV_WAVES * 64;
constexpr int GV_UNROLL = 4;  // chunks in flight per wave per iteration

// MT: number of 16-row activation tiles (1 => M<=16, 2 => M<=32).
template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED>
__global__ __launch_bounds__(GV_THREADS) void gemv_i8_kernel(
    const uint32_t* __restrict__ xq, const uint32_t* __restrict__ wq, const float* __restrict__ sx,
    const float* __restrict__ sw, const float* __restrict__ bias, void* __restrict__ out, int m, int kg,
    int n) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col0 = blockIdx.x * 16;
    const int kbytes = kg * 4;
    const int nchunks = (kbytes + 63) >> 6;

    // B operand rows: weight row col0 + lane%16 (clamped so loads stay in bounds;
    // clamped columns are never stored).
    int wrow = col0 + (lane & 15);
    if (wrow > n - 1) wrow = n - 1;
    const uint8_t* wp = reinterpret_cast<const uint8_t*>(wq) + (int64_t)wrow * kbytes;
    // A operand rows: activation row lane%16 (+16 for the second tile), zero past m.
    const uint8_t* xp[MT];
    bool xvalid[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int r = (lane & 15) + 16 * t;
        xvalid[t] = r < m;
        xp[t] = reinterpret_cast<const uint8_t*>(xq) + (int64_t)(xvalid[t] ? r : 0) * kbytes;
    }
    const int ksub = (lane >> 4) * 16;  // this lane's 16-byte slice of a 64-byte chunk

    v4i acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};

    for (int c0 = wave; c0 < nchunks; c0 += GV_WAVES * GV_UNROLL) {
        v4i wf[GV_UNROLL];
        v4i xf[GV_UNROLL][MT];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kb = (c0 + u * GV_WAVES) * 64 + ksub;
            wf[u] = load_k16<ALIGNED>(wp, kb, kbytes);
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kb = (c0 + u * GV_WAVES) * 64 + ksub;
#pragma unroll
            for (int t = 0; t < MT; ++t)
                xf[u][t] = xvalid[t] ? load_k16<ALIGNED>(xp[t], kb, kbytes) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xf[u][t], wf[u], acc[t], 0, 0, 0);
    }

    // Cross-wave reduction of the 4 partial tiles. Lane l, register i of a
    // 16x16 i32 MFMA result holds row 4*(l/16)+i, column l%16.
    __shared__ int red[GV_WAVES][MT * 4][64];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][t * 4 + i][lane] = acc[t][i];
    __syncthreads();

    const int col = col0 + (lane & 15);
    for (int ri = wave; ri < MT * 4; ri += GV_WAVES) {
        int s = 0;
#pragma unroll
        for (int w = 0; w < GV_WAVES; ++w) s += red[w][ri][lane];
        const int t = ri >> 2, i = ri & 3;
        const int row = 16 * t + 4 * (lane >> 4) + i;
        if (row < m && col < n) {
            if constexpr (OUT == OUT_I32) {
                reinterpret_cast<int*>(out)[(int64_t)row * n + col] = s;
                continue;
            }
            float v = dequant(s, sx[row], sw[col]);
            if constexpr (HAS_BIAS) v = v + bias[col];
            store_out<OUT>(out, (int64_t)row * n + col, v);
        }
    }
}

template <int MT, int OUT, bool HAS_BIAS>
static hipError_t gemv_dispatch_aligned(hipStream_t s, bool aligned, const uint32_t* xq, const uint32_t* wq,
                                        const float* sx, const float* sw, const float* bias, void* out,
                                        int m, int kg, int n) {
    dim3 grid((n + 15) / 16);
    if (aligned)
        gemv_i8_kernel<MT, OUT, HAS_BIAS, true><<<grid, GV_THREADS, 0, s>>>(xq, wq, sx, sw, bias, out, m, kg, n);
    else
        gemv_i8_kernel<MT, OUT, HAS_BIAS, false><<<grid, GV_THREADS, 0, s>>>(xq, wq, sx, sw, bias, out, m, kg, n);
    return hipGetLastError();
}

template <int MT>
static hipError_t gemv_dispatch_mt(hipStream_t s, bool aligned, const uint32_t* xq, const uint32_t* wq,
                                   const float* sx, const float* sw, const float* bias, void* out, int out_dtype,
                                   int m, int kg, int n) {
    if (out_dtype == OUT_I32)
        return gemv_dispatch_aligned<MT, OUT_I32, false>(s, aligned, xq, wq, sx, sw, nullptr, out, m, kg, n);
    if (out_dtype == OUT_F32) {
        if (bias) return gemv_dispatch_aligned<MT, OUT_F32, true>(s, aligned, xq, wq, sx, sw, bias, out, m, kg, n);
        return gemv_dispatch_aligned<MT, OUT_F32, false>(s, aligned, xq, wq, sx, sw, bias, out, m, kg, n);
    }
    if (bias) return gemv_dispatch_aligned<MT, OUT_BF16, true>(s, aligned, xq, wq, sx, sw, bias, out, m, kg, n);
    return gemv_dispatch_aligned<MT, OUT_BF16, false>(s, aligned, xq, wq, sx, sw, bias, out, m, kg, n);
}

// Host launcher. Preconditions are checked by the C-ABI layer: 1 <= m <= 32,
// kg >= 0, n >= 1.
hipError_t launch_gemv_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n) {
    const bool aligned = ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
                         ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
    if (m <= 16) return gemv_dispatch_mt<1>(s, aligned, xq, wq, sx, sw, bias, out, out_dtype, m, kg, n);
    return gemv_dispatch_mt<2>(s, aligned, xq, wq, sx, sw, bias, out, out_dtype, m, kg, n);
}

}  // namespace bh
