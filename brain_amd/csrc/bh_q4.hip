// W4A8 decode GEMV on gfx950: matmul_q4_gemv (crates/kernels/wgsl/matmul_q4_gemv.wgsl),
//   out[m,n] = (f32(sum_k xq[m,k] * w4[n,k]) * sx[m]) * sw[n]
// with xq [M, K/4] u32 (the int8 activation, unchanged from the int8 tier)
// and w4 [N, K/8] u32 (8 int4 nibbles per word, nibble b = K index 8g+b,
// crates/model/src/int4.rs:46-67). K is passed raw (the q4 family's own param
// contract, crates/model/src/dispatch.rs:132-178).
//
// HBM-bound on N*K/2 weight bytes. Like the int8 GEMV, the K reduction runs in
// v_mfma_i32_16x16x64_i8. A wave owns 16 columns; per 128-K chunk each lane
// loads 16 bytes of int4 (K 32q..32q+31 of its column, q = lane/16), unpacks
// them to two 16-byte int8 fragments and feeds two MFMAs. The activation
// fragments take the same K slices, so each MFMA pairs lane-quarter q's
// activation bytes with the weights of the same K: a permutation of K inside
// the chunk, applied to both operands, so the integer sum is exact. NW waves
// of a workgroup split K in interleaved chunks and sum their 16x16 partials
// through LDS.
#include "bh_common.h"

namespace bh {

hipError_t launch_gemv_q4_stream(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                 const float* sw, const float* bias, void* out, int out_dtype, int m, int k, int n);

struct GemvQ4Args {
    const uint32_t* xq;
    const uint32_t* wq;
    const float* sx;
    const float* sw;
    const float* bias;
    void* out;
    int m, k, n;
};

// NW waves per workgroup: SL column groups ("slots") of NW/SL waves each,
// the waves of a slot splitting K.
template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED, int NW, int U, int SL = 1>
__global__ __launch_bounds__(NW * 64) void gemv_q4_kernel(GemvQ4Args a) {
    constexpr int KS = NW / SL;  // waves per column group
    __shared__ int red[KS > 1 ? NW : 1][MT * 4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = wave / KS, ks = wave % KS;
    const int m = a.m, n = a.n;
    const int xbytes = a.k, wbytes = a.k >> 1;
    const int nchunks = (a.k + 127) >> 7;
    const int q = lane >> 4;
    const int g = blockIdx.x * SL + slot;  // 16-column group
    int wr = g * 16 + (lane & 15);
    wr = wr < n ? wr : n - 1;  // clamped rows are loaded but never stored
    const uint8_t* wp = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)wr * wbytes;
    const uint8_t* xp[MT];
    bool xlive[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int r = (lane & 15) + 16 * t;
        xlive[t] = r < m;
        xp[t] = reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)(r < m ? r : 0) * xbytes;
    }
    // Epilogue operands fetched up front, off the critical path.
    float sxr[MT * 4], swc = 0.0f, bc = 0.0f;
    const int col = g * 16 + (lane & 15);
#pragma unroll
    for (int ri = 0; ri < MT * 4; ++ri) {
        const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
        sxr[ri] = (OUT != OUT_I32 && row < m) ? a.sx[row] : 0.0f;
    }
    if constexpr (OUT != OUT_I32) swc = col < n ? a.sw[col] : 0.0f;
    if constexpr (HAS_BIAS) bc = col < n ? a.bias[col] : 0.0f;

    v4i acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll 1
    for (int j0 = ks; j0 < nchunks; j0 += KS * U) {
        v4i w16[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + KS * u;
            w16[u] = j < nchunks ? load_k16<ALIGNED>(wp, j * 64 + q * 16, wbytes) : v4i{0, 0, 0, 0};
        }
        v4i x0[U][MT], x1[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + KS * u;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const bool live = xlive[t] && j < nchunks;
                x0[u][t] = live ? load_k16<ALIGNED>(xp[t], j * 128 + q * 32, xbytes) : v4i{0, 0, 0, 0};
                x1[u][t] = live ? load_k16<ALIGNED>(xp[t], j * 128 + q * 32 + 16, xbytes) : v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v4i b0, b1;
            unpack_q4x4(w16[u], b0, b1);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0[u][t], b0, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1[u][t], b1, acc[t], 0, 0, 0);
            }
        }
    }
    auto emit = [&](int ri, int s) {
        const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
        if (row < m && col < n) {
            const int64_t idx = (int64_t)row * n + col;
            if constexpr (OUT == OUT_I32) {
                reinterpret_cast<int*>(a.out)[idx] = s;
            } else {
                float v = dequant(s, sxr[ri], swc);
                if constexpr (HAS_BIAS) v = v + bc;
                store_out<OUT>(a.out, idx, v);
            }
        }
    };
    if constexpr (KS == 1) {
#pragma unroll
        for (int ri = 0; ri < MT * 4; ++ri) emit(ri, acc[ri >> 2][ri & 3]);
    } else {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][t * 4 + i][lane] = acc[t][i];
        __syncthreads();
        // Lane l, register i of a 16x16 result: row 4*(l/16)+i, column l%16.
        for (int ri = ks; ri < MT * 4; ri += KS) {
            int s = 0;
#pragma unroll
            for (int w = 0; w < KS; ++w) s += red[slot * KS + w][ri][lane];
            emit(ri, s);
        }
    }
}

template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED>
static hipError_t q4_go(hipStream_t s, const GemvQ4Args& a) {
    const int groups = (a.n + 15) / 16;
    const int nchunks = (a.k + 127) / 128;
    // Wide N (the LM head) with few rows: one wave per column group over all
    // of K, 4 groups per workgroup, no reduction (with more rows each wave's
    // activation reads outgrow its weight reads). Otherwise K is split across the waves of a
    // workgroup so enough waves stream the weights, up to 4 chunks per pass.
    if (groups >= 1024 && nchunks <= 16 && a.m <= 4)
        gemv_q4_kernel<MT, OUT, HAS_BIAS, ALIGNED, 4, 8, 4><<<(groups + 3) / 4, 256, 0, s>>>(a);
    // Narrow N: 8 waves per column group. Measured (cold, per launch) against
    // 4 waves: K = 3072 4.04 -> 3.45 us at M = 1, 4.96 -> 4.39 at M = 16 (8
    // waves of 3 chunks; 4 waves of 6: 3.6 / 4.6); K = 1024 2.87 -> 2.67 and
    // 3.26 -> 3.04 (8 waves of 1 chunk; 4 waves of 2: 2.70 / 3.10).
    else if (nchunks >= 32) gemv_q4_kernel<MT, OUT, HAS_BIAS, ALIGNED, 8, 4><<<groups, 512, 0, s>>>(a);
    else if (nchunks > 16) gemv_q4_kernel<MT, OUT, HAS_BIAS, ALIGNED, 8, 3><<<groups, 512, 0, s>>>(a);
    else gemv_q4_kernel<MT, OUT, HAS_BIAS, ALIGNED, 8, 1><<<groups, 512, 0, s>>>(a);
    return hipGetLastError();
}

template <int MT, int OUT, bool HAS_BIAS>
static hipError_t q4_align(hipStream_t s, bool aligned, const GemvQ4Args& a) {
    if (aligned) return q4_go<MT, OUT, HAS_BIAS, true>(s, a);
    return q4_go<MT, OUT, HAS_BIAS, false>(s, a);
}

template <int MT>
static hipError_t q4_out(hipStream_t s, bool aligned, int out_dtype, const GemvQ4Args& a) {
    if (out_dtype == OUT_I32) return q4_align<MT, OUT_I32, false>(s, aligned, a);
    if (out_dtype == OUT_F32) {
        if (a.bias) return q4_align<MT, OUT_F32, true>(s, aligned, a);
        return q4_align<MT, OUT_F32, false>(s, aligned, a);
    }
    if (a.bias) return q4_align<MT, OUT_BF16, true>(s, aligned, a);
    return q4_align<MT, OUT_BF16, false>(s, aligned, a);
}

hipError_t launch_gemv_q4(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                          const float* bias, void* out, int out_dtype, int m, int k, int n) {
    // Wide N at K = 1024 (the LM head): the streaming kernel (activation
    // staged once per workgroup in LDS, each wave streaming many column
    // groups), as for int8.
    if (m <= 16 && (n + 15) / 16 >= 1024 && k == 1024) {
        const hipError_t e = launch_gemv_q4_stream(s, xq, wq, sx, sw, bias, out, out_dtype, m, k, n);
        if (e != hipErrorNotSupported) return e;
    }
    GemvQ4Args a{xq, wq, sx, sw, bias, out, m, k, n};
    // Aligned loads need whole 16-byte pieces in every row of both operands.
    const bool aligned = (k % 32) == 0 && ((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15u) == 0;
    if (m <= 16) return q4_out<1>(s, aligned, out_dtype, a);
    return q4_out<2>(s, aligned, out_dtype, a);
}

}  // namespace bh
