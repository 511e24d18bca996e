// Prefill-regime W8A8 GEMM on gfx950 matrix cores.
//
// Computes crates/kernels/wgsl/matmul_i8_dyn.wgsl:50-280 (and the static-scale
// matmul_i8.wgsl:49-262):
//   acc[m,n] = sum_k xq[m,k]*wq[n,k]           (exact i32)
//   out[m,n] = (f32(acc)*sx[m])*sw[n] (+bias[n])  -> f32 | bf16 (RNE)
// Both operands are K-contiguous ([M,K] and [N,K] int8), i.e. an "NT" GEMM,
// which is exactly the operand layout v_mfma_i32_16x16x64_i8 wants: every lane
// feeds 16 consecutive K bytes of one row.
//
// Block tile BM x BN, K staged BK=128 bytes at a time through LDS, double
// buffered (one barrier per K step). LDS rows are 128 bytes; the 16-byte chunk
// c of row r is stored at chunk c ^ (r & 7), so the 16 lanes of a fragment
// read (16 rows, same logical chunk) and the 8 threads of a staging write
// (one row, 8 chunks) each touch distinct bank groups.
// The i32 accumulation is order-independent, so any tiling is bit-exact.
#include "bh_common.h"

namespace bh {

constexpr int GM_BK = 128;  // K bytes per LDS stage

template <int BM, int BN, int WM, int WN>
struct GemmCfg {
    static constexpr int NT = WM * WN * 64;
    static constexpr int WTM = BM / WM;  // wave tile rows
    static constexpr int WTN = BN / WN;  // wave tile cols
    static constexpr int FM = WTM / 16;
    static constexpr int FN = WTN / 16;
    static constexpr int A_CHUNKS = BM * GM_BK / 16 / NT;  // 16-byte chunks per thread
    static constexpr int B_CHUNKS = BN * GM_BK / 16 / NT;
    static constexpr int LDS_A = BM * GM_BK;
    static constexpr int LDS_B = BN * GM_BK;
    static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for block");
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * GM_BK + ((chunk ^ (row & 7)) << 4); }

// Logical tile index from the hardware workgroup id. Workgroups are dispatched
// round-robin over the 8 XCDs (each with its own L2); remap so that a run of
// consecutive logical tiles lands on one XCD, then walk tiles in GROUP_M-row
// groups so neighbouring workgroups share A rows and B columns in that L2.
__device__ __forceinline__ void tile_of(int tiles_m, int tiles_n, int& tm, int& tn) {
    int pid = blockIdx.x;
    const int total = gridDim.x;
    if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
    constexpr int GROUP_M = 8;
    const int in_group = GROUP_M * tiles_n;
    const int group = pid / in_group;
    const int first_m = group * GROUP_M;
    const int gsz = min(tiles_m - first_m, GROUP_M);
    const int r = pid % in_group;
    tm = first_m + (r % gsz);
    tn = r / gsz;
}

// STATIC: per-tensor scalar scales (matmul_i8.wgsl: out = f32(acc) * (sx*sw)).
template <int BM, int BN, int WM, int WN, int OUT, bool HAS_BIAS, bool ALIGNED, bool STATIC>
__global__ __launch_bounds__(WM* WN * 64) void gemm_i8_kernel(
    const uint32_t* __restrict__ xq, const uint32_t* __restrict__ wq, const float* __restrict__ sx,
    const float* __restrict__ sw, const float* __restrict__ bias, void* __restrict__ out, int m, int kg, int n,
    float ssx, float ssw) {
    using C = GemmCfg<BM, BN, WM, WN>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (C::LDS_A + C::LDS_B)];
    // Stage b: A tile at lds + b*STAGE, B tile right after it.
    constexpr int STAGE = C::LDS_A + C::LDS_B;

    const int tiles_m = (m + BM - 1) / BM;
    const int tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    tile_of(tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const int kbytes = kg * 4;
    const int nk = (kbytes + GM_BK - 1) / GM_BK;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // Staging assignment: chunk q = t + NT*i -> (row q/8, chunk q%8).
    const uint8_t* ag[C::A_CHUNKS];
    int a_lds[C::A_CHUNKS], a_cb[C::A_CHUNKS];
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; ++i) {
        const int q = t + C::NT * i;
        const int r = q >> 3, cb = q & 7;
        const int gr = min(row0 + r, m - 1);
        ag[i] = reinterpret_cast<const uint8_t*>(xq) + (int64_t)gr * kbytes;
        a_cb[i] = cb * 16;
        a_lds[i] = swz(r, cb);
    }
    const uint8_t* bg[C::B_CHUNKS];
    int b_lds[C::B_CHUNKS], b_cb[C::B_CHUNKS];
#pragma unroll
    for (int i = 0; i < C::B_CHUNKS; ++i) {
        const int q = t + C::NT * i;
        const int r = q >> 3, cb = q & 7;
        const int gr = min(col0 + r, n - 1);
        bg[i] = reinterpret_cast<const uint8_t*>(wq) + (int64_t)gr * kbytes;
        b_cb[i] = cb * 16;
        b_lds[i] = swz(r, cb);
    }

    v4i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    v4i ra[C::A_CHUNKS], rb[C::B_CHUNKS];
    auto gload = [&](int kt) {
        const int k0 = kt * GM_BK;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) ra[i] = load_k16<ALIGNED>(ag[i], k0 + a_cb[i], kbytes);
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) rb[i] = load_k16<ALIGNED>(bg[i], k0 + b_cb[i], kbytes);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) *reinterpret_cast<v4i*>(lds + buf * STAGE + a_lds[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; ++i) *reinterpret_cast<v4i*>(lds + buf * STAGE + C::LDS_A + b_lds[i]) = rb[i];
    };

    if (nk > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    const int frow = lane & 15;   // fragment row within a 16-row group
    const int fchk = lane >> 4;   // fragment chunk within a 64-byte k step
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < GM_BK / 64; ++ks) {
            v4i fa[C::FM], fb[C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int r = wm * C::WTM + i * 16 + frow;
                fa[i] = *reinterpret_cast<const v4i*>(lds + cur * STAGE + swz(r, ks * 4 + fchk));
            }
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const int r = wn * C::WTN + j * 16 + frow;
                fb[j] = *reinterpret_cast<const v4i*>(lds + cur * STAGE + C::LDS_A + swz(r, ks * 4 + fchk));
            }
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane l, register e of fragment (i,j) holds
    // row wm*WTM + 16i + 4(l/16) + e, column wn*WTN + 16j + l%16.
    float swv[C::FN], bv[C::FN];
    int cols[C::FN];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
        cols[j] = col0 + wn * C::WTN + j * 16 + (lane & 15);
        const bool ok = cols[j] < n;
        if constexpr (!STATIC && OUT != OUT_I32) swv[j] = ok ? sw[cols[j]] : 0.0f;
        if constexpr (HAS_BIAS) bv[j] = ok ? bias[cols[j]] : 0.0f;
    }
    const float sc = ssx * ssw;
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = row0 + wm * C::WTM + i * 16 + 4 * (lane >> 4) + e;
            if (row >= m) continue;
            float sxm = 0.0f;
            if constexpr (!STATIC && OUT != OUT_I32) sxm = sx[row];
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                if (cols[j] >= n) continue;
                if constexpr (OUT == OUT_I32) {
                    reinterpret_cast<int*>(out)[(int64_t)row * n + cols[j]] = acc[i][j][e];
                    continue;
                }
                float v;
                if constexpr (STATIC) v = (float)acc[i][j][e] * sc;
                else v = dequant(acc[i][j][e], sxm, swv[j]);
                if constexpr (HAS_BIAS) v = v + bv[j];
                store_out<OUT>(out, (int64_t)row * n + cols[j], v);
            }
        }
}

template <int OUT, bool HAS_BIAS, bool STATIC>
static hipError_t gemm_go(hipStream_t s, bool aligned, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int m, int kg, int n, float ssx,
                          float ssw) {
    constexpr int BM = 128, BN = 128, WM = 2, WN = 2;
    const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (aligned)
        gemm_i8_kernel<BM, BN, WM, WN, OUT, HAS_BIAS, true, STATIC>
            <<<tiles, WM * WN * 64, 0, s>>>(xq, wq, sx, sw, bias, out, m, kg, n, ssx, ssw);
    else
        gemm_i8_kernel<BM, BN, WM, WN, OUT, HAS_BIAS, false, STATIC>
            <<<tiles, WM * WN * 64, 0, s>>>(xq, wq, sx, sw, bias, out, m, kg, n, ssx, ssw);
    return hipGetLastError();
}

static inline bool gemm_aligned(const void* xq, const void* wq, int kg) {
    return ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
           ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
}

hipError_t launch_gemm_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n) {
    const bool al = gemm_aligned(xq, wq, kg);
    if (out_dtype == OUT_I32)
        return gemm_go<OUT_I32, false, false>(s, al, xq, wq, sx, sw, nullptr, out, m, kg, n, 0.f, 0.f);
    if (out_dtype == OUT_F32) {
        if (bias) return gemm_go<OUT_F32, true, false>(s, al, xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f);
        return gemm_go<OUT_F32, false, false>(s, al, xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f);
    }
    if (bias) return gemm_go<OUT_BF16, true, false>(s, al, xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f);
    return gemm_go<OUT_BF16, false, false>(s, al, xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f);
}

hipError_t launch_gemm_i8_static(hipStream_t s, const uint32_t* xq, const uint32_t* wq, float ssx, float ssw,
                                 float* out, int m, int kg, int n) {
    const bool al = gemm_aligned(xq, wq, kg);
    return gemm_go<OUT_F32, false, true>(s, al, xq, wq, nullptr, nullptr, nullptr, out, m, kg, n, ssx, ssw);
}

}  // namespace bh
