// Decode-regime W8A8 GEMV (M <= 32) on gfx950 matrix cores.
//
// Computes the same thing as crates/kernels/wgsl/matmul_i8_gemv.wgsl:39-76:
//   out[m,n] = (f32(sum_k xq[m,k]*wq[n,k]) * sx[m]) * sw[n]
// with xq [M,K/4] u32 and wq [N,K/4] u32 (4 int8 per word, little-endian
// along K), optional bias[n] added after the dequant, f32 / bf16 / raw-i32 out.
//
// The weight stream (N*K bytes from HBM) is the whole cost. Instead of the
// reference's scalar DP4A + 64-partial LDS fold, one v_mfma_i32_16x16x64_i8
// consumes a 16-column x 64-byte slab of W per wave (A = 16 activation rows,
// B = 16 weight rows), so the K reduction happens inside the matrix core. M is
// padded to 16 (or 32: two A fragments) with zero activation rows.
//   - a workgroup (4 waves) stages the packed activation [M,K] in LDS once
//     (row stride K+16 bytes: 8 consecutive rows start in 8 different bank
//     groups) and then walks 16-column groups grid-stride, so the activation
//     is read from L2 once per workgroup, not once per column group;
//   - KSPLIT waves share one column group, each taking every KSPLIT-th
//     64-byte K chunk (KSPLIT=4 for narrow N so enough waves stream W; 1 for
//     the LM head); their 16x16 i32 partials are summed through LDS (exact);
//   - each wave issues all of its weight loads (dwordx4, 16 bytes per lane)
//     for a column group before its first MFMA; the first group's loads are
//     issued before the activation staging so the two overlap;
//   - fused epilogue: dequant, bias, bf16 RNE.
#include "bh_common.h"

namespace bh {

constexpr int GV_THREADS = 256;
constexpr int GV_WAVES = 4;
constexpr int GV_MAXC = 16;  // max 64-byte chunks a wave holds in registers per pass

struct GemvArgs {
    const uint32_t* xq;
    const uint32_t* wq;
    const float* sx;
    const float* sw;
    const float* bias;
    void* out;
    int m, kg, n;
};

template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED, int KSPLIT, bool XLDS>
__global__ __launch_bounds__(GV_THREADS) void gemv_i8_kernel(GemvArgs a) {
    constexpr int SLOTS = GV_WAVES / KSPLIT;  // column groups per workgroup pass
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // [MT*16][kbytes+16] when XLDS
    __shared__ int red[GV_WAVES][MT * 4][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int slot = wave / KSPLIT;   // which column group of this pass
    const int ks = wave % KSPLIT;     // which K slice
    const int m = a.m, n = a.n;
    const int kbytes = a.kg * 4;
    const int nchunks = (kbytes + 63) >> 6;
    const int ngroups = (n + 15) >> 4;
    const int xstride = kbytes + 16;
    const int ksub = (lane >> 4) * 16;  // this lane's 16-byte slice of a 64-byte chunk

    auto wrow_ptr = [&](int g) {
        int r = g * 16 + (lane & 15);
        r = r < n ? r : n - 1;  // clamped rows are loaded but never stored
        return reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)r * kbytes;
    };

    // First pass's weight loads, issued before the activation staging.
    int g = blockIdx.x * SLOTS + slot;
    v4i wf[GV_MAXC];
    const int my_chunks = (nchunks - ks + KSPLIT - 1) / KSPLIT;  // chunks c = ks + KSPLIT*j
    const bool single_pass = my_chunks <= GV_MAXC;
    if (single_pass && g < ngroups) {
        const uint8_t* wp = wrow_ptr(g);
#pragma unroll
        for (int j = 0; j < GV_MAXC; ++j)
            if (j < my_chunks) wf[j] = load_k16<ALIGNED>(wp, (ks + KSPLIT * j) * 64 + ksub, kbytes);
    }

    if constexpr (XLDS) {
        // Stage xq rows 0..MT*16-1 (zero past m) as 16-byte pieces.
        const int pieces = (kbytes >> 4);
        const int total = MT * 16 * pieces;
        for (int p = threadIdx.x; p < total; p += GV_THREADS) {
            const int r = p / pieces, c = p - r * pieces;
            v4i v = {0, 0, 0, 0};
            if (r < m) v = *reinterpret_cast<const v4i*>(reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)r * kbytes + c * 16);
            *reinterpret_cast<v4i*>(xs + r * xstride + c * 16) = v;
        }
        __syncthreads();
    }

    auto xfrag = [&](int t, int kb) -> v4i {
        const int r = (lane & 15) + 16 * t;
        if constexpr (XLDS) {
            if (kb >= kbytes) return v4i{0, 0, 0, 0};
            return *reinterpret_cast<const v4i*>(xs + r * xstride + kb);
        } else {
            if (r >= m) return v4i{0, 0, 0, 0};
            return load_k16<ALIGNED>(reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)r * kbytes, kb, kbytes);
        }
    };

    for (int gb = blockIdx.x; gb * SLOTS < ngroups; gb += gridDim.x) {
        g = gb * SLOTS + slot;
        v4i acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};
        if (g < ngroups) {
            const uint8_t* wp = wrow_ptr(g);
            if (single_pass) {
                if (gb != (int)blockIdx.x) {
#pragma unroll
                    for (int j = 0; j < GV_MAXC; ++j)
                        if (j < my_chunks) wf[j] = load_k16<ALIGNED>(wp, (ks + KSPLIT * j) * 64 + ksub, kbytes);
                }
#pragma unroll
                for (int j = 0; j < GV_MAXC; ++j) {
                    if (j < my_chunks) {
                        const int kb = (ks + KSPLIT * j) * 64 + ksub;
#pragma unroll
                        for (int t = 0; t < MT; ++t)
                            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xfrag(t, kb), wf[j], acc[t], 0, 0, 0);
                    }
                }
            } else {
                // Long K: passes of GV_MAXC chunks.
                for (int j0 = 0; j0 < my_chunks; j0 += GV_MAXC) {
#pragma unroll
                    for (int j = 0; j < GV_MAXC; ++j)
                        if (j0 + j < my_chunks)
                            wf[j] = load_k16<ALIGNED>(wp, (ks + KSPLIT * (j0 + j)) * 64 + ksub, kbytes);
#pragma unroll
                    for (int j = 0; j < GV_MAXC; ++j) {
                        if (j0 + j < my_chunks) {
                            const int kb = (ks + KSPLIT * (j0 + j)) * 64 + ksub;
#pragma unroll
                            for (int t = 0; t < MT; ++t)
                                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xfrag(t, kb), wf[j], acc[t], 0, 0, 0);
                        }
                    }
                }
            }
        }

        // Lane l, register i of a 16x16 i32 result holds row 4*(l/16)+i, column l%16.
        const int col = g * 16 + (lane & 15);
        if constexpr (KSPLIT == 1) {
            if (g < ngroups) {
#pragma unroll
                for (int ri = 0; ri < MT * 4; ++ri) {
                    const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
                    if (row < m && col < n) {
                        const int s = acc[ri >> 2][ri & 3];
                        const int64_t idx = (int64_t)row * n + col;
                        if constexpr (OUT == OUT_I32) {
                            reinterpret_cast<int*>(a.out)[idx] = s;
                        } else {
                            float v = dequant(s, a.sx[row], a.sw[col]);
                            if constexpr (HAS_BIAS) v = v + a.bias[col];
                            store_out<OUT>(a.out, idx, v);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][t * 4 + i][lane] = acc[t][i];
            __syncthreads();
            if (g < ngroups) {
                for (int ri = ks; ri < MT * 4; ri += KSPLIT) {
                    int s = 0;
#pragma unroll
                    for (int w = 0; w < KSPLIT; ++w) s += red[slot * KSPLIT + w][ri][lane];
                    const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
                    if (row < m && col < n) {
                        const int64_t idx = (int64_t)row * n + col;
                        if constexpr (OUT == OUT_I32) {
                            reinterpret_cast<int*>(a.out)[idx] = s;
                        } else {
                            float v = dequant(s, a.sx[row], a.sw[col]);
                            if constexpr (HAS_BIAS) v = v + a.bias[col];
                            store_out<OUT>(a.out, idx, v);
                        }
                    }
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------- host side
constexpr int GV_CUS = 256;
constexpr int GV_XLDS_MAX = 64 * 1024;

template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED, int KSPLIT>
static hipError_t gv_go(hipStream_t s, const GemvArgs& a) {
    constexpr int SLOTS = GV_WAVES / KSPLIT;
    const int ngroups = (a.n + 15) / 16;
    const int passes_needed = (ngroups + SLOTS - 1) / SLOTS;
    // One pass per workgroup: a workgroup's weight loads are all issued up
    // front and fresh workgroups keep the memory pipeline full, which beats a
    // persistent grid whose passes serialise load latency. (The grid-stride
    // loop only engages past the grid-size limit.)
    const int grid = passes_needed < 2147483647 ? passes_needed : 2147483647;
    const int kbytes = a.kg * 4;
    const size_t xlds = (size_t)MT * 16 * (kbytes + 16);
    if (ALIGNED && xlds <= (size_t)GV_XLDS_MAX) {
        gemv_i8_kernel<MT, OUT, HAS_BIAS, ALIGNED, KSPLIT, true><<<grid, GV_THREADS, xlds, s>>>(a);
    } else {
        gemv_i8_kernel<MT, OUT, HAS_BIAS, ALIGNED, KSPLIT, false><<<grid, GV_THREADS, 0, s>>>(a);
    }
    return hipGetLastError();
}

template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED>
static hipError_t gv_split(hipStream_t s, const GemvArgs& a) {
    const int ngroups = (a.n + 15) / 16;
    if (ngroups >= 4 * GV_CUS) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 1>(s, a);
    if (ngroups >= 2 * GV_CUS) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 2>(s, a);
    return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4>(s, a);
}

template <int MT, int OUT, bool HAS_BIAS>
static hipError_t gv_align(hipStream_t s, bool aligned, const GemvArgs& a) {
    if (aligned) return gv_split<MT, OUT, HAS_BIAS, true>(s, a);
    return gv_split<MT, OUT, HAS_BIAS, false>(s, a);
}

template <int MT>
static hipError_t gv_out(hipStream_t s, bool aligned, int out_dtype, const GemvArgs& a) {
    if (out_dtype == OUT_I32) return gv_align<MT, OUT_I32, false>(s, aligned, a);
    if (out_dtype == OUT_F32) {
        if (a.bias) return gv_align<MT, OUT_F32, true>(s, aligned, a);
        return gv_align<MT, OUT_F32, false>(s, aligned, a);
    }
    if (a.bias) return gv_align<MT, OUT_BF16, true>(s, aligned, a);
    return gv_align<MT, OUT_BF16, false>(s, aligned, a);
}

// Preconditions are checked by the C-ABI layer: 1 <= m <= 32, kg >= 0, n >= 1.
hipError_t launch_gemv_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n) {
    const bool aligned = ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
                         ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
    GemvArgs a{xq, wq, sx, sw, bias, out, m, kg, n};
    if (m <= 16) return gv_out<1>(s, aligned, out_dtype, a);
    return gv_out<2>(s, aligned, out_dtype, a);
}

}  // namespace bh
