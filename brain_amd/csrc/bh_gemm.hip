// Prefill-regime W8A8 GEMM on gfx950 matrix cores.
//
// Computes crates/kernels/wgsl/matmul_i8_dyn.wgsl:50-280 (and the static-scale
// matmul_i8.wgsl:49-262):
//   acc[m,n] = sum_k xq[m,k]*wq[n,k]              (exact i32)
//   out[m,n] = (f32(acc)*sx[m])*sw[n] (+bias[n])  -> f32 | bf16 (RNE) | raw i32
// Both operands are K-contiguous ([M,K] and [N,K] int8), an "NT" GEMM, which is
// the operand layout v_mfma_i32_32x32x32_i8 wants: each lane feeds 16
// consecutive K bytes of one row. (On gfx950 the 32x32x32 i8 MFMA sustains
// about 1.5x the rate of the 16x16x64 one, so it is the only shape used here.)
//
// Block tile BM x BN, K staged BK=128 bytes at a time through LDS, double
// buffered with register prefetch (one barrier per stage). LDS rows are 128
// bytes; 16-byte chunk c of row r lives at chunk c ^ ((r >> 1) & 7), so the
// 16 lanes of an LDS phase (16 consecutive rows, one logical chunk) land in
// 16 distinct 16-byte slots of a 256-byte bank line. This register-staged
// kernel is the fallback for K % 128 != 0 or unaligned operands.
//
// Split-K (SPLITK), for shapes with too few output tiles to fill 256 CUs: S
// workgroups share one output tile, each summing a contiguous slice of K and
// storing its raw i32 partial tile into its own slab ws[split][m][n] (plain
// stores, no atomics, nothing to clear). A second kernel adds the S slabs in
// i32 (exact: integer addition in any order gives the same sum) and applies
// the epilogue, so the output is bit-identical to the unsplit kernel's.
#include <algorithm>
#include <cstdlib>

#include <mutex>

#include "bh_common.h"

namespace bh {

constexpr int GM_BK = 128;  // K bytes per LDS stage

template <int BM, int BN, int WM, int WN>
struct GemmCfg {
    static constexpr int NT = WM * WN * 64;
    static constexpr int WTM = BM / WM;  // wave tile rows
    static constexpr int WTN = BN / WN;  // wave tile cols
    static constexpr int FM = WTM / 32;  // 32x32 fragments per wave tile
    static constexpr int FN = WTN / 32;
    static constexpr int A_CHUNKS = BM * GM_BK / 16 / NT;  // 16-byte chunks per thread per stage
    static constexpr int B_CHUNKS = BN * GM_BK / 16 / NT;
    static constexpr int LDS_A = BM * GM_BK;
    static constexpr int LDS_B = BN * GM_BK;
    static constexpr int STAGE = LDS_A + LDS_B;
    static_assert(FM >= 1 && FN >= 1, "wave tile must hold whole 32x32 fragments");
    static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for block");
    static_assert(2 * STAGE <= 160 * 1024, "LDS budget");
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * GM_BK + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Logical tile from a linear tile id. Workgroups are dispatched round-robin
// over the 8 XCDs (each with its own L2): remap so a run of consecutive tile
// ids lands on one XCD, then walk tiles in GROUP_M-row groups so neighbouring
// workgroups share A rows and B columns in that L2.
__device__ __forceinline__ void tile_of(int pid, int total, int tiles_m, int tiles_n, int& tm, int& tn) {
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

struct GemmArgs {
    const uint32_t* xq;
    const uint32_t* wq;
    const float* sx;
    const float* sw;
    const float* bias;
    void* out;
    int m, kg, n;
    float ssx, ssw;   // STATIC scales
    int splits;       // S (1 = no split)
    int* ws;          // [S][m][n] i32 split-K partials
    // Row gate of moe_linear_gated_i8.wgsl (null: none): row r of the output
    // is +0 when gate[r * gate_stride + gate_col] <= 0.
    const float* gate;
    int gate_stride, gate_col;
    // Output row stride in elements (0: n). A launch over a column range of
    // a wider output (the column split of launch_gemm_i8) writes row r at
    // out + r * ldo; the split-K slabs stay compact ([S][m][n]).
    int ldo = 0;
    // Row compaction (moe_linear_gated_i8 at prefill sizes): the A rows are
    // the routed rows only, *m_dev of them (m is then an upper bound that
    // sizes the grid; tiles past *m_dev exit), and A row r is output row
    // row_map[r]. Null: m rows, row r is output row r. DMA kernel, f32/bf16
    // output, no split-K.
    const int* m_dev = nullptr;
    const int* row_map = nullptr;
};

__host__ __device__ __forceinline__ int64_t out_ld(const GemmArgs& a) { return a.ldo ? a.ldo : a.n; }

__device__ __forceinline__ bool gated_off(const GemmArgs& a, int row) {
    return a.gate && a.gate[(int64_t)row * a.gate_stride + a.gate_col] <= 0.0f;
}

// moe_linear_gated_i8's early exit for unrouted rows
// (crates/kernels/wgsl/moe_linear_gated_i8.wgsl:66-69), per output tile: when
// no row of [row0, row0+BM) is routed, the tile stores its +0 outputs and
// skips the K loop. (A tile with some routed rows multiplies them all; the
// epilogue zeroes the rest.) Split-K partial tiles never skip: the reduction
// reads every slab. Block-uniform result; all threads take part.
template <int BM, int BN, int NT, bool SPLITK>
__device__ __forceinline__ bool gated_tile_skipped(const GemmArgs& a, int row0, int col0) {
    if (SPLITK || !a.gate) return false;
    const int t = threadIdx.x;
    const bool live = t < BM && row0 + t < a.m && !gated_off(a, row0 + t);
    if (__syncthreads_or(live)) return false;
    float* out = reinterpret_cast<float*>(a.out);  // the gated linear's output is f32
    const int rows = min(BM, a.m - row0), cols = min(BN, a.n - col0);
    for (int i = t; i < rows * cols; i += NT) {
        const int r = i / cols, c = i - r * cols;
        out[(int64_t)(row0 + r) * out_ld(a) + col0 + c] = 0.0f;
    }
    return true;
}

// One output element through the epilogue.
template <int OUT, bool HAS_BIAS, bool STATIC>
__device__ __forceinline__ void emit(const GemmArgs& a, int row, int col, int acc, float sxm, float swn, float bn) {
    const int64_t idx = (int64_t)row * out_ld(a) + col;
    if constexpr (OUT == OUT_I32) {
        reinterpret_cast<int*>(a.out)[idx] = acc;
    } else {
        float v;
        if constexpr (STATIC) v = (float)acc * (a.ssx * a.ssw);
        else v = dequant(acc, sxm, swn);
        if constexpr (HAS_BIAS) v = v + bn;
        if (gated_off(a, row)) v = 0.0f;
        store_out<OUT>(a.out, idx, v);
    }
}

// Q4: the weight operand is int4 (W4A8, [N, K/8] u32, crates/model/src/int4.rs:46-67).
// Each thread loads half as many 16-byte pieces of B and unpacks every piece
// into the two int8 chunks the int8 layout holds at that K, so the LDS image,
// the MFMA loop and the epilogue are the int8 kernel's.
template <int BM, int BN, int WM, int WN, int OUT, bool HAS_BIAS, bool ALIGNED, bool STATIC, bool SPLITK, bool Q4 = false>
__global__ __launch_bounds__(WM* WN * 64) void gemm_i8_kernel(GemmArgs a) {
    using C = GemmCfg<BM, BN, WM, WN>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * C::STAGE];

    const int m = a.m, n = a.n;
    const int tiles_m = (m + BM - 1) / BM;
    const int tiles_n = (n + BN - 1) / BN;
    const int S = SPLITK ? a.splits : 1;
    const int tile_id = blockIdx.x / S;
    const int split = blockIdx.x - tile_id * S;
    int tm, tn;
    tile_of(tile_id, gridDim.x / S, tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    if (gated_tile_skipped<BM, BN, WM * WN * 64, SPLITK>(a, row0, col0)) return;
    const int kbytes = a.kg * 4;
    const int nk_all = (kbytes + GM_BK - 1) / GM_BK;
    const int kt0 = (int)(((int64_t)nk_all * split) / S);
    const int kt1 = (int)(((int64_t)nk_all * (split + 1)) / S);
    const int nk = kt1 - kt0;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // Staging assignment: chunk q = t + NT*i -> (row q/8, chunk q%8); 8
    // consecutive threads read one 128-byte row segment.
    const uint8_t* ag[C::A_CHUNKS];
    int a_lds[C::A_CHUNKS], a_cb[C::A_CHUNKS];
#pragma unroll
    for (int i = 0; i < C::A_CHUNKS; ++i) {
        const int q = t + C::NT * i;
        const int r = q >> 3, cb = q & 7;
        const int gr = min(row0 + r, m - 1);
        ag[i] = reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)gr * kbytes;
        a_cb[i] = cb * 16;
        a_lds[i] = swz(r, cb);
    }
    // int8 B: chunk q -> (row q/8, chunk q%8). int4 B: piece q -> (row q/4,
    // piece q%4) of the row's 64 int4 bytes per stage, landing in int8 chunks
    // 2*(q%4) and 2*(q%4)+1.
    constexpr int BL = Q4 ? C::B_CHUNKS / 2 : C::B_CHUNKS;  // global loads of B per thread
    const int bbytes = Q4 ? kbytes / 2 : kbytes;
    const uint8_t* bg[BL];
    int b_lds[BL], b_cb[BL];
#pragma unroll
    for (int i = 0; i < BL; ++i) {
        const int q = t + C::NT * i;
        const int r = Q4 ? q >> 2 : q >> 3, cb = Q4 ? q & 3 : q & 7;
        const int gr = min(col0 + r, n - 1);
        bg[i] = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)gr * bbytes;
        b_cb[i] = cb * 16;
        b_lds[i] = C::LDS_A + swz(r, Q4 ? 2 * cb : cb);
    }

    v16i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    v4i ra[C::A_CHUNKS], rb[BL];
    auto gload = [&](int kt) {
        const int k0 = kt * GM_BK;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) ra[i] = load_k16<ALIGNED>(ag[i], k0 + a_cb[i], kbytes);
#pragma unroll
        for (int i = 0; i < BL; ++i) rb[i] = load_k16<ALIGNED>(bg[i], (Q4 ? k0 / 2 : k0) + b_cb[i], bbytes);
    };
    auto sstore = [&](int buf) {
        uint8_t* base = lds + buf * C::STAGE;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) *reinterpret_cast<v4i*>(base + a_lds[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            if constexpr (Q4) {
                // chunk 2c and 2c+1 of a row are adjacent before the swizzle
                // (c ^ s and (c ^ s) ^ 1 for even c): recompute the second slot.
                const int q = t + C::NT * i;
                const int r = q >> 2, cb = q & 3;
                v4i lo, hi;
                unpack_q4x4(rb[i], lo, hi);
                *reinterpret_cast<v4i*>(base + b_lds[i]) = lo;
                *reinterpret_cast<v4i*>(base + C::LDS_A + swz(r, 2 * cb + 1)) = hi;
            } else {
                *reinterpret_cast<v4i*>(base + b_lds[i]) = rb[i];
            }
        }
    };

    if (nk > 0) {
        gload(kt0);
        sstore(0);
    }
    __syncthreads();

    const int frow = lane & 31;  // fragment row within a 32-row group
    const int fchk = lane >> 5;  // fragment chunk within a 32-byte k step
    for (int it = 0; it < nk; ++it) {
        const int cur = it & 1;
        if (it + 1 < nk) gload(kt0 + it + 1);
        const uint8_t* base = lds + cur * C::STAGE;
#pragma unroll
        for (int ks = 0; ks < GM_BK / 32; ++ks) {
            v4i fa[C::FM], fb[C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
                fa[i] = *reinterpret_cast<const v4i*>(base + swz(wm * C::WTM + i * 32 + frow, ks * 2 + fchk));
#pragma unroll
            for (int j = 0; j < C::FN; ++j)
                fb[j] = *reinterpret_cast<const v4i*>(base + C::LDS_A + swz(wn * C::WTN + j * 32 + frow, ks * 2 + fchk));
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (it + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // Lane l, register e of fragment (i,j) holds
    //   row wm*WTM + 32i + 8*(e/4) + 4*(l/32) + e%4,  column wn*WTN + 32j + l%32.
    const int rbase = row0 + wm * C::WTM + 4 * (lane >> 5);
    const int cbase = col0 + wn * C::WTN + (lane & 31);

    // Split-K: this workgroup's partial sums go raw to its own slab of the
    // workspace (the kernel is instantiated with OUT_I32 for it).
    if constexpr (SPLITK)
        if (S > 1) {
            a.out = a.ws + (int64_t)split * m * n;
            a.ldo = 0;
        }

    float swv[C::FN], bv[C::FN];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
        const int col = cbase + j * 32;
        const bool ok = col < n;
        swv[j] = 0.0f;
        bv[j] = 0.0f;
        if constexpr (!STATIC && OUT != OUT_I32) swv[j] = ok ? a.sw[col] : 0.0f;
        if constexpr (HAS_BIAS && OUT != OUT_I32) bv[j] = ok ? a.bias[col] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = rbase + i * 32 + 8 * (e >> 2) + (e & 3);
            if (row >= m) continue;
            float sxm = 0.0f;
            if constexpr (!STATIC && OUT != OUT_I32) sxm = a.sx[row];
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const int col = cbase + j * 32;
                if (col < n) emit<OUT, HAS_BIAS, STATIC>(a, row, col, acc[i][j][e], sxm, swv[j], bv[j]);
            }
        }
}

// ---------------------------------------------------------------- pipelined DMA kernel
// The main path for K % DK == 0 and 16-byte aligned operands. Global memory
// is copied straight into LDS with global_load_lds_dwordx4 (no staging
// registers), STAGES buffers of DK K-bytes deep, so the loads of the next
// STAGES-1 stages are in flight while one stage is multiplied. A DMA
// instruction writes 64 lanes x 16 bytes to consecutive LDS slots, so the
// bank swizzle is applied on the global side: LDS slot (row r, chunk p)
// receives logical K-chunk p ^ f(r).
//   DK=64  (4 chunks/row): f(r) = (r>>2) & 3
//   DK=128 (8 chunks/row): f(r) = (r>>1) & 7
// gfx950 LDS serves a ds_read_b128 16 lanes at a time from 64 four-byte banks
// (one 256-byte line); a fragment read has 16 lanes on 16 consecutive rows
// and one logical chunk, and f sends them to 16 distinct 16-byte slots of the
// line, so the read takes the minimum 4 cycles (measured with
// SQ_LDS_BANK_CONFLICT = 0; the ((r>>1)^(r>>3)) and r&7 variants cost +4).
//
// Within a stage the fragment reads for k-step ks+1 are issued before the
// MFMAs of k-step ks (sched_barrier keeps the compiler from sinking them), so
// LDS latency hides behind matrix-core work.
//
// The MFMA is fed B (weights) as its first operand, so each 32x32 result is
// the transposed tile: lane l, register e holds row m = l%32 and column
// n = 8*(e/4) + 4*(l/32) + e%4, i.e. four consecutive columns per lane, which
// the epilogue writes with one 8-byte (bf16) or 16-byte (f32) store.
template <int DK>
__device__ __forceinline__ int dswz(int r) {
    if constexpr (DK == 64) return (r >> 2) & 3;
    else if constexpr (DK == 128) return (r >> 1) & 7;
    else return r & 15;  // DK = 256: a row is one whole 256-byte bank line
}
template <int DK>
__device__ __forceinline__ int dslot(int r, int c) { return r * DK + ((c ^ dswz<DK>(r)) << 4); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

template <int BM, int BN, int WM, int WN, int STAGES, int DK>
struct DmaCfg {
    static constexpr int NT = WM * WN * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int CPR = DK / 16;  // 16-byte chunks per LDS row
    static constexpr int A_BYTES = BM * DK, B_BYTES = BN * DK;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int A_LOADS = A_BYTES / 16 / NT;  // DMA instructions per thread per stage
    static constexpr int B_LOADS = B_BYTES / 16 / NT;
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr int KSTEPS = DK / 32;
    static_assert(A_LOADS * 16 * NT == A_BYTES && B_LOADS * 16 * NT == B_BYTES, "whole DMA waves");
    static_assert(STAGES * STAGE <= 160 * 1024, "LDS budget");
    static_assert((STAGES - 2) * LOADS < 64, "vmcnt range");
    static_assert(STAGES >= 3, "the next stage's first k-step is read during this one");
};

// Wait until at most `ahead` stages (N loads each) remain in flight;
// MAXA is the largest `ahead` the caller passes.
template <int N, int MAXA>
__device__ __forceinline__ void wait_ahead(int ahead) {
    if constexpr (MAXA > 0) {
        if (ahead >= MAXA) {
            wait_vmcnt<MAXA * N>();
            return;
        }
        wait_ahead<N, MAXA - 1>(ahead);
    } else {
        wait_vmcnt<0>();
    }
}

template <int BM, int BN, int WM, int WN, int STAGES, int DK, int OUT, bool HAS_BIAS, bool STATIC, bool SPLITK,
          bool ILV_ENABLE = false, bool PP = false>
__global__ __launch_bounds__(WM* WN * 64) void gemm_i8_dma_kernel(GemmArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-DMA builtins exist only in the device pass
    using C = DmaCfg<BM, BN, WM, WN, STAGES, DK>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * C::STAGE];

    const int m = a.m, n = a.n;
    const int tiles_m = (m + BM - 1) / BM;
    const int tiles_n = (n + BN - 1) / BN;
    const int S = SPLITK ? a.splits : 1;
    const int tile_id = blockIdx.x / S;
    const int split = blockIdx.x - tile_id * S;
    int tm, tn;
    // Row compaction: the tiles that hold rows are the first ones, so they go
    // to the XCDs round-robin (no run-per-XCD remap, which would put them all
    // on one or two XCDs).
    tile_of(tile_id, a.m_dev ? 1 : gridDim.x / S, tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const int mrows = a.m_dev ? *a.m_dev : m;  // rows that exist (row compaction: the routed rows)
    if (row0 >= mrows) return;
    if (gated_tile_skipped<BM, BN, WM * WN * 64, SPLITK>(a, row0, col0)) return;
    const int kbytes = a.kg * 4;
    const int nk_all = kbytes / DK;
    const int kt0 = (int)(((int64_t)nk_all * split) / S);
    const int kt1 = (int)(((int64_t)nk_all * (split + 1)) / S);
    const int nk = kt1 - kt0;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // DMA source addresses: thread t's i-th load fills LDS slot q = t + NT*i
    // (16-byte slots, CPR per row) of the A (then B) tile.
    const uint8_t* asrc[C::A_LOADS];
    const uint8_t* bsrc[C::B_LOADS];
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) {
        const int q = t + C::NT * i, r = q / C::CPR, p = q % C::CPR;
        const int gr = min(row0 + r, mrows - 1);
        asrc[i] = reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)gr * kbytes + ((p ^ dswz<DK>(r)) << 4);
    }
#pragma unroll
    for (int i = 0; i < C::B_LOADS; ++i) {
        const int q = t + C::NT * i, r = q / C::CPR, p = q % C::CPR;
        const int gr = min(col0 + r, n - 1);
        bsrc[i] = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)gr * kbytes + ((p ^ dswz<DK>(r)) << 4);
    }
    // The wave-uniform LDS base of load i (the hardware adds lane*16). The
    // DMA is issued through inline asm so the compiler does not track it:
    // its completion is ordered only by the explicit vmcnt waits + barrier
    // below (hardware vmcnt covers the LDS write of an LDS-DMA load).
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds + wave * 64 * 16;
    auto dma = [&](const uint8_t* src, uint32_t ldsaddr) {
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :
                     : "v"(src), "s"(__builtin_amdgcn_readfirstlane(ldsaddr))
                     : "memory", "m0");
    };
    auto issue = [&](int kt, int buf) {
        const uint32_t base = lds_base + buf * C::STAGE;
        const int64_t koff = (int64_t)kt * DK;
#pragma unroll
        for (int i = 0; i < C::A_LOADS; ++i) dma(asrc[i] + koff, base + i * C::NT * 16);
#pragma unroll
        for (int i = 0; i < C::B_LOADS; ++i) dma(bsrc[i] + koff, base + C::A_BYTES + i * C::NT * 16);
    };

    // Epilogue operands of this tile (column scales and bias, row scales and
    // gate), one per thread, fetched before the first DMA so their latency
    // hides behind the K loop. They reach the epilogue through LDS: a global
    // load there would wait (vmcnt is in order) behind the output stores.
    constexpr bool EP_COLS = !STATIC && OUT != OUT_I32;
    constexpr bool EP_ROWS = OUT != OUT_I32;
    static_assert(BM <= C::NT && BN <= C::NT, "one epilogue operand per thread");
    __shared__ __attribute__((aligned(16))) float ep_sw[EP_COLS ? BN : 1];
    __shared__ __attribute__((aligned(16))) float ep_b[HAS_BIAS && EP_COLS ? BN : 1];
    __shared__ float ep_sx[EP_ROWS ? BM : 1];
    __shared__ int ep_off[EP_ROWS ? BM : 1];
    __shared__ int ep_map[EP_ROWS ? BM : 1];
    float r_sw = 0.0f, r_b = 0.0f, r_sx = 0.0f;
    bool r_off = false;
    int r_map = 0;
    if constexpr (EP_COLS) {
        if (t < BN && col0 + t < n) {
            r_sw = a.sw[col0 + t];
            if constexpr (HAS_BIAS) r_b = a.bias[col0 + t];
        }
    }
    if constexpr (EP_ROWS) {
        if (t < BM && row0 + t < mrows) {
            if constexpr (!STATIC) r_sx = a.sx[row0 + t];
            r_off = gated_off(a, row0 + t);
            r_map = a.row_map ? a.row_map[row0 + t] : row0 + t;
        }
    }

    v16i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(kt0 + s, s);

    const int frow = lane & 31, fchk = lane >> 5;
    auto read_frags = [&](const uint8_t* A, int ks, v4i* fa, v4i* fb) {
        const uint8_t* B = A + C::A_BYTES;
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
            fa[i] = *reinterpret_cast<const v4i*>(A + dslot<DK>(wm * C::WTM + i * 32 + frow, 2 * ks + fchk));
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
            fb[j] = *reinterpret_cast<const v4i*>(B + dslot<DK>(wn * C::WTN + j * 32 + frow, 2 * ks + fchk));
    };
    // One k-step of MFMAs with the next k-step's fragment reads interleaved:
    // MFMA, read, MFMA, read, ... then the remaining MFMAs.
    auto mfma_step = [&](const v4i* fa, const v4i* fb) {
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
    };
    auto interleave = [&]() {
#pragma unroll
        for (int q = 0; q < C::FM + C::FN; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, C::FM * C::FN - (C::FM + C::FN), 0);
    };

    // DMA interleave: LOADS/KSTEPS loads per k-step, one between every
    // ILV_MF of the MFMAs that follow the fragment-read ones.
    constexpr int ILV_PER_STEP = C::LOADS / C::KSTEPS;
    constexpr int ILV_TAIL = C::FM * C::FN - (C::FM + C::FN);
    constexpr int ILV_MF = ILV_PER_STEP > 0 ? ILV_TAIL / ILV_PER_STEP : 0;
    constexpr bool ILV = ILV_ENABLE && C::LOADS % C::KSTEPS == 0 && ILV_PER_STEP > 0 && ILV_MF > 0 &&
                         ILV_MF * ILV_PER_STEP == ILV_TAIL;
    auto dma_one = [&](int idx, uint32_t base, int64_t koff) {
        if (idx < C::A_LOADS) dma(asrc[idx] + koff, base + idx * C::NT * 16);
        else dma(bsrc[idx - C::A_LOADS] + koff, base + C::A_BYTES + (idx - C::A_LOADS) * C::NT * 16);
    };
    auto mfma_range = [&](const v4i* fa_, const v4i* fb_, int q0, int cnt) {
#pragma unroll
        for (int q = 0; q < C::FM * C::FN; ++q) {
            if (q < q0 || q >= q0 + cnt) continue;
            const int i = q / C::FN, j = q % C::FN;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb_[j], fa_[i], acc[i][j], 0, 0, 0);
        }
    };
    auto interleave_reads = [&]() {
#pragma unroll
        for (int q = 0; q < C::FM + C::FN; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
    };

    if constexpr (PP) {
        // Ping-pong: the 8 waves form two groups of 4 (one wave of each per
        // SIMD) that run one phase apart, so on every SIMD one wave multiplies
        // while the other reads LDS and issues DMA. Each stage takes two
        // phases per wave, L (wait for the stage, read all its fragments into
        // registers, issue the DMA of stage +3 into the buffer the stage
        // before freed) and C (the stage's MFMAs), each closed by a
        // workgroup barrier. Group 1 starts one barrier late and group 0 ends
        // one barrier later, so both pass the same number of barriers.
        //   Stage s is needed by group 0 at its L(s): its own DMA waits there;
        // group 1 waits for its share of stage s during L(s-1), which ends
        // before group 0's L(s); for stage 0 every wave waits before a common
        // first barrier.
        //   The DMA of L(s) overwrites stage s-1's buffer: group 0 read it in
        // L(s-1), two phases earlier, group 1 in the phase just before.
        static_assert(WM * WN == 8 && STAGES == 4, "ping-pong: 8 waves, 4 stages");
        // Wave-uniform in a scalar register, so the group branches are real
        // branches: a barrier under an exec mask would still execute.
        const int grp = __builtin_amdgcn_readfirstlane(wave) >> 2;
        v4i pa[C::KSTEPS][C::FM], pb[C::KSTEPS][C::FN];
        // Stage 0 complete (every wave's share) before group 0's first L.
        if (nk > 0) wait_ahead<C::LOADS, STAGES - 2>(min(nk - 1, STAGES - 2));
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 1) {
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int it = 0; it < nk; ++it) {
            if (grp == 0) wait_ahead<C::LOADS, STAGES - 2>(min(nk - 1 - it, STAGES - 2));
            else wait_ahead<C::LOADS, STAGES - 3>(min(nk - 2 - it, STAGES - 3));
            const uint8_t* A = lds + (it % STAGES) * C::STAGE;
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks) read_frags(A, ks, pa[ks], pb[ks]);
            if (it + STAGES - 1 < nk) issue(kt0 + it + STAGES - 1, (it + STAGES - 1) % STAGES);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the fragments are in registers
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks)
#pragma unroll
                for (int i = 0; i < C::FM; ++i)
#pragma unroll
                    for (int j = 0; j < C::FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pb[ks][j], pa[ks][i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
        if (grp == 0) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
    v4i fa[2][C::FM], fb[2][C::FN];
    if (nk > 0) {
        wait_ahead<C::LOADS, STAGES - 2>(min(nk - 1, STAGES - 2));
        __builtin_amdgcn_s_barrier();
        read_frags(lds + (0 % STAGES) * C::STAGE, 0, fa[0], fb[0]);
    }
    for (int it = 0; it < nk; ++it) {
        // Stages it and it+1 must have landed (the tail of this iteration
        // reads stage it+1's first k-step); later ones may still be in flight.
        wait_ahead<C::LOADS, STAGES - 3>(min(nk - 2 - it, STAGES - 3));
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        const bool do_issue = it + STAGES - 1 < nk;
        if constexpr (!ILV) {
            if (do_issue) issue(kt0 + it + STAGES - 1, (it + STAGES - 1) % STAGES);
        }
        const uint32_t ibase = lds_base + ((it + STAGES - 1) % STAGES) * C::STAGE;
        const int64_t ikoff = (int64_t)(kt0 + it + STAGES - 1) * DK;
        const uint8_t* A = lds + (it % STAGES) * C::STAGE;
        const uint8_t* An = lds + ((it + 1) % STAGES) * C::STAGE;
#pragma unroll
        for (int ks = 0; ks < C::KSTEPS; ++ks) {
            const int cur = ks & 1, nxt = cur ^ 1;
            __builtin_amdgcn_sched_barrier(0);
            // The last k-step reads the next stage's first fragments (on the
            // final iteration that buffer holds stale data that is never used).
            read_frags(ks + 1 < C::KSTEPS ? A : An, ks + 1 < C::KSTEPS ? ks + 1 : 0, fa[nxt], fb[nxt]);
            if constexpr (ILV) {
                // The first FM+FN MFMAs carry the fragment reads; each DMA of
                // the stage being refilled sits between two of the rest, so
                // the matrix pipe stays busy while it issues.
                mfma_range(fa[cur], fb[cur], 0, C::FM + C::FN);
                interleave_reads();
#pragma unroll
                for (int d = 0; d < ILV_PER_STEP; ++d) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (do_issue) dma_one(ks * ILV_PER_STEP + d, ibase, ikoff);
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_range(fa[cur], fb[cur], C::FM + C::FN + d * ILV_MF, ILV_MF);
                }
            } else {
                mfma_step(fa[cur], fb[cur]);
                interleave();
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (C::KSTEPS % 2 == 1) {
            // keep fa[0]/fb[0] as "current" for the next stage
#pragma unroll
            for (int i = 0; i < C::FM; ++i) fa[0][i] = fa[1][i];
#pragma unroll
            for (int j = 0; j < C::FN; ++j) fb[0][j] = fb[1][j];
        }
    }

    }

    // Lane l, register e of fragment (i,j): row rbase + 32i, columns
    // cbase + 32j + 8*(e/4) + (e%4).
    const int rbase = row0 + wm * C::WTM + (lane & 31);
    const int cbase = col0 + wn * C::WTN + 4 * (lane >> 5);

    if constexpr (SPLITK)
        if (S > 1) {
            a.out = a.ws + (int64_t)split * m * n;  // raw partials to this split's (compact) slab
            a.ldo = 0;
        }

    if constexpr (EP_COLS) {
        if (t < BN) {
            ep_sw[t] = r_sw;
            if constexpr (HAS_BIAS) ep_b[t] = r_b;
        }
    }
    if constexpr (EP_ROWS) {
        if (t < BM) {
            ep_sx[t] = r_sx;
            ep_off[t] = r_off;
            ep_map[t] = r_map;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every DMA and fragment read has landed
    __builtin_amdgcn_s_barrier();   // ... in every wave, before the stage buffers are reused

    // Staged epilogue. Written straight from the fragment layout, every store
    // instruction of a wave would touch 32 rows at 8-16 bytes each; instead
    // each wave converts one 32-row block of its tile at a time into its own
    // LDS region (row pitch = tile row + 16 bytes, an odd number of 16-byte
    // slots, so the 32 lanes of different rows hit distinct banks) and copies
    // it out as whole 16-byte chunks of consecutive columns, 256 or 512 bytes
    // of one row per 16/32 lanes. Needs n % 8 == 0 and a 16-byte aligned
    // output; anything else takes the direct path below.
    {
        constexpr int ESZ = (OUT == OUT_BF16) ? 2 : 4;
        constexpr int EP_PITCH = C::WTN * ESZ + 16;
        constexpr int EP_REGION = 32 * EP_PITCH;
        constexpr int EP_CPR = C::WTN * ESZ / 16;  // 16-byte chunks per tile row
        static_assert(WM * WN * EP_REGION <= STAGES * C::STAGE, "epilogue staging fits in the stage buffers");
        static_assert((32 * EP_CPR) % 64 == 0, "whole copy-out passes");
        const bool staged = (n % 8) == 0 && (out_ld(a) % 8) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15u) == 0;
        if (staged) {
            uint8_t* reg = lds + wave * EP_REGION;
            const int lrow = lane & 31;
            const int wrow0 = row0 + wm * C::WTM, wcol0 = col0 + wn * C::WTN;
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int lr = wm * C::WTM + i * 32 + lrow;  // row within the tile
                float sxm = 0.0f;
                bool off = false;
                if constexpr (EP_ROWS) {
                    sxm = ep_sx[lr];
                    off = ep_off[lr] != 0;
                }
#pragma unroll
                for (int j = 0; j < C::FN; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int lc = j * 32 + 8 * g + 4 * (lane >> 5);
                        const int tc = wn * C::WTN + lc;  // column within the tile
                        const int v0 = acc[i][j][4 * g + 0], v1 = acc[i][j][4 * g + 1];
                        const int v2 = acc[i][j][4 * g + 2], v3 = acc[i][j][4 * g + 3];
                        uint8_t* dst = reg + lrow * EP_PITCH + lc * ESZ;
                        if constexpr (OUT == OUT_I32) {
                            *reinterpret_cast<v4i*>(dst) = v4i{v0, v1, v2, v3};
                        } else {
                            float f0, f1, f2, f3;
                            if constexpr (STATIC) {
                                const float sc = a.ssx * a.ssw;
                                f0 = (float)v0 * sc; f1 = (float)v1 * sc; f2 = (float)v2 * sc; f3 = (float)v3 * sc;
                            } else {
                                const float4 swv = *reinterpret_cast<const float4*>(ep_sw + tc);
                                f0 = dequant(v0, sxm, swv.x); f1 = dequant(v1, sxm, swv.y);
                                f2 = dequant(v2, sxm, swv.z); f3 = dequant(v3, sxm, swv.w);
                            }
                            if constexpr (HAS_BIAS) {
                                const float4 bv = *reinterpret_cast<const float4*>(ep_b + tc);
                                f0 = f0 + bv.x; f1 = f1 + bv.y; f2 = f2 + bv.z; f3 = f3 + bv.w;
                            }
                            if (off) f0 = f1 = f2 = f3 = 0.0f;
                            if constexpr (OUT == OUT_F32) {
                                *reinterpret_cast<float4*>(dst) = make_float4(f0, f1, f2, f3);
                            } else {
                                const uint32_t lo = pack_bf16x2(f0, f1);
                                const uint32_t hi = pack_bf16x2(f2, f3);
                                *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
                            }
                        }
                    }
                // Only this wave reads its region: its LDS operations run in
                // order, so waiting for its own writes is enough.
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int q0 = 0; q0 < 32 * EP_CPR; q0 += 64) {
                    const int q = q0 + lane, r = q / EP_CPR, c = q % EP_CPR;
                    const v4i v = *reinterpret_cast<const v4i*>(reg + r * EP_PITCH + c * 16);
                    const int grow = wrow0 + i * 32 + r, gcol = wcol0 + c * (16 / ESZ);
                    if (grow < mrows && gcol < n) {
                        int orow = grow;
                        if constexpr (EP_ROWS) orow = ep_map[grow - row0];
                        *reinterpret_cast<v4i*>(reinterpret_cast<uint8_t*>(a.out) + ((int64_t)orow * out_ld(a) + gcol) * ESZ) = v;
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);
                __builtin_amdgcn_wave_barrier();
            }
            return;
        }
    }

    // Direct epilogue: four consecutive columns per (fragment, e/4) group,
    // stored as one vector when n % 4 == 0 and the output is aligned for it
    // (a step_sliced word offset may break that), else element by element.
    const bool vec_ok = (n % 4) == 0 && (out_ld(a) % 4) == 0 &&
                        (reinterpret_cast<uintptr_t>(a.out) & (OUT == OUT_BF16 ? 7u : 15u)) == 0;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int col = cbase + j * 32 + 8 * g;
            const int tc = col - col0;
            float4 swv = make_float4(0.f, 0.f, 0.f, 0.f), bv = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (EP_COLS) {
                swv = *reinterpret_cast<const float4*>(ep_sw + tc);
                if constexpr (HAS_BIAS) bv = *reinterpret_cast<const float4*>(ep_b + tc);
            }
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int row = rbase + i * 32;
                if (row >= mrows || col >= n) continue;
                float sxm = 0.0f;
                bool off = false;
                if constexpr (EP_ROWS) {
                    sxm = ep_sx[row - row0];
                    off = ep_off[row - row0] != 0;
                }
                const int v[4] = {acc[i][j][4 * g + 0], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                float f[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (OUT != OUT_I32) {
                    const float sv[4] = {swv.x, swv.y, swv.z, swv.w};
                    const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if constexpr (STATIC) f[q] = (float)v[q] * (a.ssx * a.ssw);
                        else f[q] = dequant(v[q], sxm, sv[q]);
                        if constexpr (HAS_BIAS) f[q] = f[q] + bb[q];
                        if (off) f[q] = 0.0f;
                    }
                }
                int orow = row;
                if constexpr (EP_ROWS) orow = ep_map[row - row0];
                const int64_t idx = (int64_t)orow * out_ld(a) + col;
                if (vec_ok && col + 3 < n) {
                    if constexpr (OUT == OUT_I32)
                        *reinterpret_cast<v4i*>(reinterpret_cast<int*>(a.out) + idx) = v4i{v[0], v[1], v[2], v[3]};
                    else if constexpr (OUT == OUT_F32)
                        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + idx) = make_float4(f[0], f[1], f[2], f[3]);
                    else
                        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + idx) =
                            make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (col + q >= n) continue;
                        if constexpr (OUT == OUT_I32) reinterpret_cast<int*>(a.out)[idx + q] = v[q];
                        else store_out<OUT>(a.out, idx + q, f[q]);
                    }
                }
            }
        }
#endif
}

// ---------------------------------------------------------------- split-K reduction
// out[r, c] = epilogue(sum_s ws[s][r][c]). VEC: four consecutive columns per
// thread (n % 4 == 0 and the output aligned for a 4-element store).
// SN > 0: the split count at compile time, so every slab load (and the
// row's scale, the columns' scales and bias) of a 4-column group issues before
// the first add; SN = 0 reads S from the arguments.
template <int OUT, bool HAS_BIAS, bool STATIC, bool VEC, int SN = 0>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs a) {
    const int n = a.n, S = SN > 0 ? SN : a.splits;
    const int64_t mn = (int64_t)a.m * n;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if constexpr (VEC) {
        const v4i* ws = reinterpret_cast<const v4i*>(a.ws);
        const int64_t q4 = mn >> 2;
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < q4; q += stride) {
            const int64_t idx = q << 2;
            const int row = (int)(idx / n), col = (int)(idx - (int64_t)row * n);
            v4i acc;
            float sxm = 0.0f;
            float4 swv = make_float4(0.f, 0.f, 0.f, 0.f), bv = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (SN > 0) {
                v4i v[SN];
#pragma unroll
                for (int sp = 0; sp < SN; ++sp) v[sp] = ws[(int64_t)sp * q4 + q];
                if constexpr (OUT != OUT_I32 && !STATIC) {
                    sxm = a.sx[row];
                    swv = make_float4(a.sw[col], a.sw[col + 1], a.sw[col + 2], a.sw[col + 3]);
                }
                if constexpr (OUT != OUT_I32 && HAS_BIAS)
                    bv = make_float4(a.bias[col], a.bias[col + 1], a.bias[col + 2], a.bias[col + 3]);
                acc = v[0];
#pragma unroll
                for (int sp = 1; sp < SN; ++sp) {
                    acc[0] += v[sp][0]; acc[1] += v[sp][1]; acc[2] += v[sp][2]; acc[3] += v[sp][3];
                }
            } else {
                acc = ws[q];
                for (int sp = 1; sp < S; ++sp) {
                    const v4i v = ws[(int64_t)sp * q4 + q];
                    acc[0] += v[0]; acc[1] += v[1]; acc[2] += v[2]; acc[3] += v[3];
                }
                if constexpr (OUT != OUT_I32 && !STATIC) {
                    sxm = a.sx[row];
                    swv = make_float4(a.sw[col], a.sw[col + 1], a.sw[col + 2], a.sw[col + 3]);
                }
                if constexpr (OUT != OUT_I32 && HAS_BIAS)
                    bv = make_float4(a.bias[col], a.bias[col + 1], a.bias[col + 2], a.bias[col + 3]);
            }
            const int64_t o4 = ((int64_t)row * out_ld(a) + col) >> 2;  // output index / 4 (ldo % 4 == 0)
            if constexpr (OUT == OUT_I32) {
                reinterpret_cast<v4i*>(a.out)[o4] = acc;
            } else {
                float f[4];
                const bool off = gated_off(a, row);
                const float sv[4] = {swv.x, swv.y, swv.z, swv.w};
                const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (STATIC) f[e] = (float)acc[e] * (a.ssx * a.ssw);
                    else f[e] = dequant(acc[e], sxm, sv[e]);
                    if constexpr (HAS_BIAS) f[e] = f[e] + bb[e];
                    if (off) f[e] = 0.0f;
                }
                if constexpr (OUT == OUT_F32)
                    reinterpret_cast<float4*>(a.out)[o4] = make_float4(f[0], f[1], f[2], f[3]);
                else
                    reinterpret_cast<uint2*>(a.out)[o4] = make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
            }
        }
    } else {
        for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < mn; idx += stride) {
            int acc = a.ws[idx];
            for (int sp = 1; sp < S; ++sp) acc += a.ws[(int64_t)sp * mn + idx];
            const int row = (int)(idx / n), col = (int)(idx - (int64_t)row * n);
            const float sxm = (STATIC || OUT == OUT_I32) ? 0.0f : a.sx[row];
            const float swn = (STATIC || OUT == OUT_I32) ? 0.0f : a.sw[col];
            const float bn = (HAS_BIAS && OUT != OUT_I32) ? a.bias[col] : 0.0f;
            emit<OUT, HAS_BIAS, STATIC>(a, row, col, acc, sxm, swn, bn);
        }
    }
}

// ---------------------------------------------------------------- host side
// Tile configurations of the DMA kernel (the register-staged fallback has
// only 256x256 and 128x128; every smaller choice maps to its 128x128).
enum TileCfg {
    TILE_256 = 0,     // 256x256, 8 waves of 128x64, 4 stages
    TILE_128 = 1,     // 128x128, 4 waves of 64x64, 4 stages
    TILE_64x128 = 2,  // 64x128, 4 waves of 32x64, 4 stages
    TILE_64 = 3,      // 64x64, 4 waves of 32x32, 4 stages
    TILE_64_DEEP = 4,  // 64x64 with 8 stages in flight (long K on a few tiles)
    TILE_256x128 = 5,  // 256x128, 8 waves of 64x64, 4 stages
    TILE_64_K128 = 6,     // 64x64, 8 stages of 128 K-bytes (what TILE_64_DEEP runs)
    TILE_64x128_K128 = 7,  // 64x128, 4 stages of 128 K-bytes (what TILE_64x128 runs)
    TILE_256x128_K128 = 8,  // 256x128, 3 stages of 128 K-bytes (what TILE_256x128 runs)
    TILE_32x64 = 9          // 32x64, 2 waves of 32x32, 4 stages of 256 K-bytes (8 of 128 if K % 256 != 0)
};

struct TileChoice {
    int cfg;     // TileCfg
    int splits;  // split-K factor S
};

// Measurement overrides, read once: BH_GEMM_TILE=c forces TileCfg c,
// BH_SPLITK=S forces the split factor (1 = never split).
static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}
static int tile_env() {
    static int v = env_int("BH_GEMM_TILE", -1);
    return v;
}
static int splitk_env() {
    static int v = env_int("BH_SPLITK", 0);
    return v;
}
// BH_GEMM_T32=0: no 32x64 tiles (for measurement).
static int t32x64_env() {
    static int v = env_int("BH_GEMM_T32", 1);
    return v;
}

constexpr size_t SPLITK_MAX_BYTES = size_t(64) << 20;  // workspace cap per call

// Split-K. Measured on MI355X, a tile alone on its CU costs a few us fixed
// (launch, first loads, epilogue) plus P us per 64-byte K stage (0.25 for
// 128x128, 0.18 for the 64-row tiles), so splitting K S ways shortens the
// chain by P * stages * (1 - 1/S) us. It pays for the i32 partial slabs
// (S*m*n*4 bytes written and read back, ~3 TB/s effective) and the reduction
// launch (~3 us). S is the largest value with tiles x S within two workgroups
// per CU and at least 8 stages per split, used only when the modelled gain
// exceeds 3 us (a margin for the model).
static int choose_splits(long tiles, double per_stage, int m, int kg, int n) {
    constexpr long CUS = 256;
    const long stages = (long)kg * 4 / 64;
    const double slab = (double)m * n * 4;
    const int forced = splitk_env();
    long S = forced > 0 ? forced : std::min<long>(8, (2 * CUS) / std::max<long>(tiles, 1));
    if (forced <= 0) {
        while (S > 1 && stages / S < 8) --S;
        if (S > 1) {
            const double gain = per_stage * stages * (1.0 - 1.0 / S) - 3.0 - S * slab / 3.0e6;
            if (gain < 3.0) S = 1;
        }
    }
    while (S > 1 && (stages / S < 1 || S * slab > (double)SPLITK_MAX_BYTES)) --S;
    return (int)std::max<long>(S, 1);
}

// Pick the tile that finishes first on 256 CUs.
//  - Enough 128x128 tiles to fill the chip: a launch runs in rounds of 256
//    workgroups, so its time is ~ rounds x (time of one tile). Per round, in
//    units of a 128x128 tile's time, measured on MI355X: 256x256 costs 4.0
//    (4x the work at ~1.25x the efficiency: half the LDS-staging bytes per
//    op), 256x128 on 8 waves 2.2, 128x128 1.4. The cheapest of
//    4.0 * ceil(t256/256), 2.2 * ceil(t256x128/256) and 1.4 * ceil(t128/256)
//    wins (e.g. 8192x1024x3072: 2 rounds of 256x256, one half empty, 8.0; 3
//    rounds of 256x128, 6.6; 6 rounds of 128x128, 8.4; 1152x3840x10240: one
//    round of 256x256, 4.0, measured 54 us, against 3 rounds of 128x128, 4.2,
//    measured 71 us).
//  - Fewer 128x128 tiles than CUs: smaller tiles put more CUs to work. A lone
//    tile's time is set by how fast one CU streams its operands, so halving a
//    tile side nearly halves its time. Measured on the prefill sweep shapes at
//    M=128..2048: 128-255 tiles of 128x128 run fastest as 64x128 tiles, fewer
//    as 64x64 tiles, and 64x64 tiles on at most one round of CUs with 32+
//    K stages run fastest with 8 stages in flight.
static TileChoice choose_tiles(int m, int kg, int n) {
    constexpr long CUS = 256;
    const long t256 = (long)((m + 255) / 256) * ((n + 255) / 256);
    const long t2x1 = (long)((m + 255) / 256) * ((n + 127) / 128);
    const long t128 = (long)((m + 127) / 128) * ((n + 127) / 128);
    const long t64 = (long)((m + 63) / 64) * ((n + 63) / 64);
    const long stages = (long)kg * 4 / 64;
    const double c256 = 4.0 * (double)((t256 + CUS - 1) / CUS);
    const double c2x1 = 2.2 * (double)((t2x1 + CUS - 1) / CUS);
    const double c128 = 1.4 * (double)((t128 + CUS - 1) / CUS);
    TileChoice tc{TILE_128, 1};
    if (c256 <= c2x1 && c256 <= c128) tc.cfg = TILE_256;
    else if (c2x1 < c128) tc.cfg = TILE_256x128;
    else if (t128 >= CUS) tc.cfg = TILE_128;
    else if (t128 >= CUS / 2) tc.cfg = TILE_64x128;
    else tc.cfg = (t64 <= CUS && stages >= 32) ? TILE_64_DEEP : TILE_64;
    // At most half the chip's worth of 64x64 tiles over a long K, where
    // 32x64 tiles fill more than half of it (e.g. 512x3072x1024: 128 tiles
    // of 64x64 on 48 K stages, 256 of 32x64), and no split-K.
    const long t32 = (long)((m + 31) / 32) * ((n + 63) / 64);
    if (tc.cfg == TILE_64_DEEP && t64 <= CUS / 2 && t32 > CUS / 2 && t32 <= CUS && t32x64_env())
        tc.cfg = TILE_32x64;
    if (tile_env() >= 0) tc.cfg = tile_env();
    switch (tc.cfg) {
        case TILE_128: tc.splits = choose_splits(t128, 0.25, m, kg, n); break;
        case TILE_64x128: tc.splits = choose_splits(t128 * 2, 0.2, m, kg, n); break;
        case TILE_64:
        case TILE_64_DEEP: tc.splits = choose_splits(t64, 0.18, m, kg, n); break;
        default: break;
    }
    // Big tiles on a grid that fills half the chip or less with a long K
    // (e.g. the DiT down projection, 1152x10240x3840: 150 tiles of 256x128
    // over 160 K stages): 256x256 tiles split S ways over K can fill it.
    // Measured per 64-byte stage: ~0.75 us for a 256x256 tile, ~0.6 us for
    // 256x128; a split adds the reduction (~3 us) and the slabs (S*m*n*4
    // bytes at ~3 TB/s). Taken when the model saves 15%; measured on the DiT
    // stack (30 such projections) the step drops from 7.97 to 7.80 ms.
    if ((tc.cfg == TILE_256 || tc.cfg == TILE_256x128) && tile_env() < 0 && splitk_env() <= 0 && t256 <= CUS / 2 &&
        stages >= 64) {
        const double slab = (double)m * n * 4;
        long S = std::min<long>(CUS / t256, stages / 32);
        while (S > 1 && S * slab > (double)SPLITK_MAX_BYTES) --S;
        if (S > 1) {
            const double cur = tc.cfg == TILE_256 ? 2.0 + 0.75 * stages : 2.0 + 0.6 * stages;
            const double split = 2.0 + 0.75 * (double)stages / S + 3.0 + S * slab / 3.0e6;
            if (split < 0.85 * cur) tc = TileChoice{TILE_256, (int)S};
        }
    }
    if (tc.cfg == TILE_256 && splitk_env() > 1) tc.splits = splitk_env();
    return tc;
}

template <int BM, int BN, int WM, int WN, int OUT, bool HAS_BIAS, bool STATIC, bool SPLITK, bool Q4 = false>
static hipError_t go(hipStream_t s, bool aligned, const GemmArgs& a) {
    const long tiles = (long)((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
    const unsigned grid = (unsigned)(tiles * (SPLITK ? a.splits : 1));
    constexpr int NT = WM * WN * 64;
    if (aligned)
        gemm_i8_kernel<BM, BN, WM, WN, OUT, HAS_BIAS, true, STATIC, SPLITK, Q4><<<grid, NT, 0, s>>>(a);
    else
        gemm_i8_kernel<BM, BN, WM, WN, OUT, HAS_BIAS, false, STATIC, SPLITK, Q4><<<grid, NT, 0, s>>>(a);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES, int DK, int OUT, bool HAS_BIAS, bool STATIC, bool SPLITK,
          bool ILV = false, bool PP = false>
static hipError_t go_dma(hipStream_t s, const GemmArgs& a) {
    const long tiles = (long)((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
    const unsigned grid = (unsigned)(tiles * (SPLITK ? a.splits : 1));
    gemm_i8_dma_kernel<BM, BN, WM, WN, STAGES, DK, OUT, HAS_BIAS, STATIC, SPLITK, ILV, PP><<<grid, WM * WN * 64, 0, s>>>(a);
    return hipGetLastError();
}

// Alternative large-tile DMA configurations for measurement (BH_GEMM_BIG):
// 0: 256x256, 8 waves (128x64 each: 2 waves per SIMD, ~200 VGPRs), DK=64,
//    4 stages, the two wave groups in ping-pong (default; 2-3% above 5 on the
//    large shapes)
// 1: 256x128, 4 waves (128x64 each), DK=128, 3 stages
// 2: 256x256, 8 waves, every wave reading and multiplying, no DMA interleave
// 3: 256x256, 4 waves (128x128 each), no interleave
// 4: 256x256, 4 waves (128x128 each), DMA interleave
// 5: 256x256, 8 waves, DMA issue interleaved between the MFMAs (5-10% above
//    the 4-wave forms)
static int big_cfg() {
    static int v = env_int("BH_GEMM_BIG", 0);
    return v;
}

// The DMA kernel for every tile but 256x256.
// The small tiles that run long K chains on few CUs, and the 8-wave 256x128
// tile, take 128-byte K stages: half the barriers and waits per K byte, which
// is what a lone small tile's stage time is made of (measured: 512x3072x1024
// 12.3 -> 10.7 us, 2048x3072x1024 15.0 -> 14.1 us, Qwen3 prefill 1-3%
// faster; more stages of 64 bytes instead, 16 in flight, measured slower;
// 256x128 in 3 stages of 128 bytes: 2048x4096x11008 118.8 -> 111.6 us,
// 8192x3072x1024 35.0 -> 31.0 us; 128x128 mixed, so it keeps 64-byte
// stages). BH_GEMM_DK128=0 keeps 64-byte stages, for measurements.
static int dk128_env() {
    static int v = env_int("BH_GEMM_DK128", 1);
    return v;
}

template <int OUT, bool HAS_BIAS, bool STATIC, bool SPLITK>
static hipError_t go_small(hipStream_t s, int cfg, const GemmArgs& a) {
    if (dk128_env()) {
        if (cfg == TILE_64_DEEP) cfg = TILE_64_K128;
        if (cfg == TILE_64x128) cfg = TILE_64x128_K128;
        if (cfg == TILE_256x128) cfg = TILE_256x128_K128;
    }
    switch (cfg) {
        case TILE_64x128: return go_dma<64, 128, 2, 2, 4, 64, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_64: return go_dma<64, 64, 2, 2, 4, 64, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_64_DEEP: return go_dma<64, 64, 2, 2, 8, 64, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_256x128: return go_dma<256, 128, 4, 2, 4, 64, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_64_K128: return go_dma<64, 64, 2, 2, 8, 128, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_64x128_K128: return go_dma<64, 128, 2, 2, 4, 128, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_256x128_K128: return go_dma<256, 128, 4, 2, 3, 128, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        case TILE_32x64:
            // 256-byte K stages (8 k-steps per barrier) where K allows.
            if ((a.kg * 4) % 256 == 0) return go_dma<32, 64, 1, 2, 4, 256, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
            return go_dma<32, 64, 1, 2, 8, 128, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
        default: return go_dma<128, 128, 2, 2, 4, 64, OUT, HAS_BIAS, STATIC, SPLITK>(s, a);
    }
}

// dma: K % 64 == 0 and both operands 16-byte aligned (the DMA path cannot
// zero-fill a K tail, so anything else takes the register-staged kernel).
template <int OUT, bool HAS_BIAS, bool STATIC>
static hipError_t go_cfg(hipStream_t s, bool aligned, bool dma, const TileChoice& tc, const GemmArgs& a) {
    if (dma) {
        if (tc.cfg == TILE_256) {
            switch (big_cfg()) {
                case 1: return go_dma<256, 128, 2, 2, 3, 128, OUT, HAS_BIAS, STATIC, false>(s, a);
                case 2: return go_dma<256, 256, 2, 4, 4, 64, OUT, HAS_BIAS, STATIC, false>(s, a);
                case 3: return go_dma<256, 256, 2, 2, 4, 64, OUT, HAS_BIAS, STATIC, false, false>(s, a);
                case 4: return go_dma<256, 256, 2, 2, 4, 64, OUT, HAS_BIAS, STATIC, false, true>(s, a);
                case 5: return go_dma<256, 256, 2, 4, 4, 64, OUT, HAS_BIAS, STATIC, false, true>(s, a);
                default: return go_dma<256, 256, 2, 4, 4, 64, OUT, HAS_BIAS, STATIC, false, false, true>(s, a);
            }
        }
        return go_small<OUT, HAS_BIAS, STATIC, false>(s, tc.cfg, a);
    }
    if (tc.cfg == TILE_256) return go<256, 256, 2, 2, OUT, HAS_BIAS, STATIC, false>(s, aligned, a);
    return go<128, 128, 2, 2, OUT, HAS_BIAS, STATIC, false>(s, aligned, a);
}

static inline bool gemm_aligned(const void* xq, const void* wq, int kg) {
    return ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
           ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
}

// Split-K workspace of the stream: at least `ints` i32 (grown outside graph
// capture only; hipErrorStreamCaptureUnsupported otherwise).
int* splitk_workspace(hipStream_t s, size_t ints, hipError_t* err, int slot = 0);

// Workspace elements the GEMM needs for this shape (0 = no split-K).
static int column_split(int m, int kg, int n, const TileChoice& tc, bool dma);

size_t gemm_workspace_ints(int m, int kg, int n) {
    const TileChoice tc = choose_tiles(m, kg, n);
    if (const int n_main = column_split(m, kg, n, tc, (kg * 4) % 128 == 0)) {
        const TileChoice tt = choose_tiles(m, kg, n - n_main);  // the column-split tail's own GEMM
        return tt.splits > 1 ? (size_t)tt.splits * m * (n - n_main) : 0;
    }
    return tc.splits > 1 ? (size_t)tc.splits * m * n : 0;
}

hipError_t gemm_reserve(hipStream_t s, int m, int kg, int n) {
    const size_t ints = gemm_workspace_ints(m, kg, n);
    if (!ints) return hipSuccess;
    hipError_t err = hipSuccess;
    return splitk_workspace(s, ints, &err) ? hipSuccess : err;
}

// Launches the chosen configuration: one kernel, or for S > 1 the split
// kernel (raw i32 partials) and the reduction that applies the epilogue.
// ws_fixed: caller-provided slab memory of at least splits*m*n i32 (the
// no-allocation entry point); null takes the stream's library workspace.
template <int OUT, bool HAS_BIAS, bool STATIC>
static hipError_t run_gemm(hipStream_t s, bool al, bool dma, const TileChoice& tc, GemmArgs a,
                           int* ws_fixed = nullptr) {
    if (tc.splits <= 1) return go_cfg<OUT, HAS_BIAS, STATIC>(s, al, dma, tc, a);
    hipError_t err = hipSuccess;
    a.ws = ws_fixed ? ws_fixed : splitk_workspace(s, (size_t)tc.splits * a.m * a.n, &err);
    if (!a.ws) return err == hipSuccess ? hipErrorOutOfMemory : err;
    a.splits = tc.splits;
    if (dma && tc.cfg == TILE_256)
        err = go_dma<256, 256, 2, 4, 4, 64, OUT_I32, false, false, true, false, true>(s, a);
    else if (dma)
        err = go_small<OUT_I32, false, false, true>(s, tc.cfg, a);
    else
        err = go<128, 128, 2, 2, OUT_I32, false, false, true>(s, al, a);
    if (err != hipSuccess) return err;
    const int64_t mn = (int64_t)a.m * a.n;
    const uintptr_t need = OUT == OUT_BF16 ? 7u : 15u;
    const bool vec = (a.n % 4) == 0 && (out_ld(a) % 4) == 0 && (reinterpret_cast<uintptr_t>(a.out) & need) == 0;
    const int64_t work = vec ? mn / 4 : mn;
    const unsigned grid = (unsigned)std::min<int64_t>((work + 255) / 256, 256 * 16);
    if (vec) {
        switch (a.splits) {
            case 2: splitk_reduce_kernel<OUT, HAS_BIAS, STATIC, true, 2><<<grid, 256, 0, s>>>(a); break;
            case 3: splitk_reduce_kernel<OUT, HAS_BIAS, STATIC, true, 3><<<grid, 256, 0, s>>>(a); break;
            case 4: splitk_reduce_kernel<OUT, HAS_BIAS, STATIC, true, 4><<<grid, 256, 0, s>>>(a); break;
            default: splitk_reduce_kernel<OUT, HAS_BIAS, STATIC, true><<<grid, 256, 0, s>>>(a); break;
        }
    } else {
        splitk_reduce_kernel<OUT, HAS_BIAS, STATIC, false><<<grid, 256, 0, s>>>(a);
    }
    return hipGetLastError();
}

// Column split of a 256x256 grid whose last round would run mostly empty
// (e.g. 8192x4096x11008: 1376 tiles, 5.4 rounds of 256 CUs): the first
// n_main columns as whole rounds of 256x256 tiles, the rest as its own GEMM
// with its own tile choice (there 768 columns, one round of 192 256x128
// tiles at about half a 256x256 round's cost), when the per-round cost model
// of choose_tiles says the pair finishes first. Returns n_main, or 0.
static int column_split(int m, int kg, int n, const TileChoice& tc, bool dma) {
    if (!dma || tc.cfg != TILE_256 || tc.splits != 1 || tile_env() >= 0 || splitk_env() > 0 || big_cfg() != 0)
        return 0;
    constexpr long CUS = 256;
    const long tm = (m + 255) / 256, tn = (n + 255) / 256;
    const long rounds = (tm * tn + CUS - 1) / CUS;
    if (rounds < 2 || (tm * tn) % CUS == 0) return 0;
    long g = CUS, t = tm;  // gcd(tm, CUS): tile columns per whole number of rounds = CUS / gcd
    while (t) {
        const long r = g % t;
        g = t;
        t = r;
    }
    const long step = CUS / g;
    const long c_main = (tn - 1) / step * step;  // whole rounds, at least one column left over
    if (c_main <= 0) return 0;
    const int n_main = (int)(c_main * 256), n_tail = n - n_main;
    const long t2x1 = tm * ((n_tail + 127) / 128), t128 = ((m + 127) / 128) * ((n_tail + 127) / 128);
    const double tail = std::min({4.0 * (double)((tm * ((n_tail + 255) / 256) + CUS - 1) / CUS),
                                  2.2 * (double)((t2x1 + CUS - 1) / CUS), 1.4 * (double)((t128 + CUS - 1) / CUS)});
    const double cost = 4.0 * (double)(tm * c_main / CUS) + tail + 0.25;  // 0.25: the second launch
    return cost < 4.0 * (double)rounds ? n_main : 0;
}

hipError_t launch_gemm_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n) {
    GemmArgs a{xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f, 1, nullptr};
    const bool al = gemm_aligned(xq, wq, kg);
    const bool dma = al && ((kg * 4) % 128 == 0);
    const TileChoice tc = choose_tiles(m, kg, n);
    if (const int n_main = column_split(m, kg, n, tc, dma)) {
        const size_t esz = out_dtype == OUT_BF16 ? 2 : 4;
        GemmArgs t = a;
        t.n = n - n_main;
        t.ldo = n;
        t.wq = wq + (size_t)n_main * kg;
        t.sw = sw + n_main;
        t.bias = bias ? bias + n_main : nullptr;
        t.out = static_cast<uint8_t*>(out) + (size_t)n_main * esz;
        const TileChoice tt = choose_tiles(m, kg, t.n);
        a.n = n_main;
        a.ldo = n;
        hipError_t e;
        if (out_dtype == OUT_I32) e = run_gemm<OUT_I32, false, false>(s, al, dma, tc, a);
        else if (out_dtype == OUT_F32) e = bias ? run_gemm<OUT_F32, true, false>(s, al, dma, tc, a)
                                                : run_gemm<OUT_F32, false, false>(s, al, dma, tc, a);
        else e = bias ? run_gemm<OUT_BF16, true, false>(s, al, dma, tc, a) : run_gemm<OUT_BF16, false, false>(s, al, dma, tc, a);
        if (e != hipSuccess) return e;
        const bool tal = gemm_aligned(xq, t.wq, kg);
        const bool tdma = tal && ((kg * 4) % 128 == 0);
        if (out_dtype == OUT_I32) return run_gemm<OUT_I32, false, false>(s, tal, tdma, tt, t);
        if (out_dtype == OUT_F32) return bias ? run_gemm<OUT_F32, true, false>(s, tal, tdma, tt, t)
                                              : run_gemm<OUT_F32, false, false>(s, tal, tdma, tt, t);
        return bias ? run_gemm<OUT_BF16, true, false>(s, tal, tdma, tt, t) : run_gemm<OUT_BF16, false, false>(s, tal, tdma, tt, t);
    }
    if (out_dtype == OUT_I32) return run_gemm<OUT_I32, false, false>(s, al, dma, tc, a);
    if (out_dtype == OUT_F32) {
        if (bias) return run_gemm<OUT_F32, true, false>(s, al, dma, tc, a);
        return run_gemm<OUT_F32, false, false>(s, al, dma, tc, a);
    }
    if (bias) return run_gemm<OUT_BF16, true, false>(s, al, dma, tc, a);
    return run_gemm<OUT_BF16, false, false>(s, al, dma, tc, a);
}

// ---------------------------------------------------------------- no allocation
// The split-K slabs of bh_matmul_i8_dyn_noalloc live in this fixed device
// array (one copy per GPU, held until the process ends) instead of the
// library's grown-on-demand per-stream workspace, so that call never
// allocates. In host code `scratch` only names the symbol: its device address
// comes from hipGetSymbolAddress, looked up once per device with that device
// current, and only that address is ever passed to a kernel.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) int scratch[NOALLOC_SCRATCH_BYTES / 4];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static int* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Overlap guard: the stream of the last call on each device that used the
// scratch, and an event recorded after that call's kernels. A call from
// another stream while that event is pending would race on the scratch, so
// it is refused (hipErrorNotReady) instead. Calls under graph capture are
// not tracked (their work runs when the graph is launched).
struct ScratchUse {
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
static ScratchUse g_scratch_use[NOALLOC_MAX_DEVICES];

// Device address of this device's `scratch` (current device, *dev), or
// null. Caller holds g_scratch_mu.
static int* scratch_ptr(hipError_t* err, int* dev_out) {
    int dev = 0;
    if ((*err = hipGetDevice(&dev)) != hipSuccess) return nullptr;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if ((*err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return nullptr;
        if ((*err = hipEventCreateWithFlags(&g_scratch_use[dev].ev, hipEventDisableTiming)) != hipSuccess)
            return nullptr;
        g_scratch_ptr[dev] = static_cast<int*>(p);
    }
    *dev_out = dev;
    return g_scratch_ptr[dev];
}

size_t noalloc_scratch_bytes() { return NOALLOC_SCRATCH_BYTES; }

// bh_matmul_i8_dyn without allocation: the same kernels and tile choice
// (one launch over all columns, without launch_gemm_i8's column split; the
// results are the same bits); the split-K slabs go to the fixed scratch. *need_bytes reports the slab
// bytes the shape needs (0 when it does not split K); hipErrorInvalidValue
// when that exceeds the scratch.
hipError_t launch_gemm_i8_noalloc(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                  const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n,
                                  size_t* need_bytes) {
    GemmArgs a{xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f, 1, nullptr};
    const bool al = gemm_aligned(xq, wq, kg);
    const bool dma = al && ((kg * 4) % 128 == 0);
    const TileChoice tc = choose_tiles(m, kg, n);
    *need_bytes = tc.splits > 1 ? (size_t)tc.splits * m * n * 4 : 0;
    if (*need_bytes > NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
    hipError_t err = hipSuccess;
    std::lock_guard<std::mutex> g(g_scratch_mu);  // check, launch and record as one step per host thread
    int dev = 0;
    int* ws = scratch_ptr(&err, &dev);  // the first call on a device looks the address up
    if (!ws) return err;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((err = hipStreamIsCapturing(s, &cs)) != hipSuccess) return err;
    ScratchUse& use = g_scratch_use[dev];
    const bool tracked = tc.splits > 1 && cs == hipStreamCaptureStatusNone;
    if (tracked && use.used && use.last != s) {
        const hipError_t q = hipEventQuery(use.ev);
        if (q == hipErrorNotReady) return hipErrorNotReady;
        if (q != hipSuccess) return q;
    }
    if (out_dtype == OUT_I32) err = run_gemm<OUT_I32, false, false>(s, al, dma, tc, a, ws);
    else if (out_dtype == OUT_F32) err = bias ? run_gemm<OUT_F32, true, false>(s, al, dma, tc, a, ws)
                                              : run_gemm<OUT_F32, false, false>(s, al, dma, tc, a, ws);
    else err = bias ? run_gemm<OUT_BF16, true, false>(s, al, dma, tc, a, ws)
                    : run_gemm<OUT_BF16, false, false>(s, al, dma, tc, a, ws);
    if (err != hipSuccess || !tracked) return err;
    if ((err = hipEventRecord(use.ev, s)) != hipSuccess) return err;
    use.last = s;
    use.used = true;
    return hipSuccess;
}

hipError_t launch_gemm_i8_static(hipStream_t s, const uint32_t* xq, const uint32_t* wq, float ssx, float ssw,
                                 float* out, int m, int kg, int n) {
    GemmArgs a{xq, wq, nullptr, nullptr, nullptr, out, m, kg, n, ssx, ssw, 1, nullptr};
    const bool al = gemm_aligned(xq, wq, kg);
    return run_gemm<OUT_F32, false, true>(s, al, al && ((kg * 4) % 128 == 0), choose_tiles(m, kg, n), a);
}

// W4A8 prefill GEMM (matmul_q4_dyn, crates/kernels/wgsl/matmul_q4_dyn.wgsl).
// k is the raw K (k % 8 == 0); the activation keeps its int8 [M, K/4] layout.
//  - M >= Q4_EXPAND_M and K % 32 == 0: the int4 weights are expanded once to
//    int8 ([N, K/4], the same values sign-extended) in a per-stream
//    workspace, and the int8 GEMM runs on them. The accumulators are the same
//    integers, so the output is bit-identical; the expansion moves 1.5*N*K
//    bytes, small beside the GEMM at these M.
//  - otherwise the register-staged kernel with int4 B unpacked on the way
//    into LDS.
constexpr int Q4_EXPAND_M = 256;

__global__ __launch_bounds__(256) void expand_q4_kernel(const v4i* w4, v4i* w8, int64_t pieces) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * 256) {
        v4i lo, hi;
        unpack_q4x4(w4[i], lo, hi);
        w8[2 * i] = lo;
        w8[2 * i + 1] = hi;
    }
}

size_t gemm_q4_workspace_ints(int m, int k, int n) {
    return (m >= Q4_EXPAND_M && k % 32 == 0) ? (size_t)n * (k / 4) : 0;
}

template <int OUT, bool HAS_BIAS>
static hipError_t go_q4(hipStream_t s, bool aligned, const GemmArgs& a) {
    TileChoice tc = choose_tiles(a.m, a.kg, a.n);
    if (tc.cfg == TILE_256) return go<256, 256, 2, 2, OUT, HAS_BIAS, false, false, true>(s, aligned, a);
    return go<128, 128, 2, 2, OUT, HAS_BIAS, false, false, true>(s, aligned, a);
}

hipError_t launch_gemm_q4(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int k, int n) {
    // Aligned 16-byte loads need 16-byte rows in both operands: K % 32 == 0.
    const bool al = (k % 32) == 0 && ((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15u) == 0;
    const size_t ints = gemm_q4_workspace_ints(m, k, n);
    if (al && ints) {
        hipError_t err = hipSuccess;
        int* w8 = splitk_workspace(s, ints, &err, 1);
        if (!w8) return err == hipSuccess ? hipErrorOutOfMemory : err;
        const int64_t pieces = (int64_t)n * k / 32;
        const unsigned grid = (unsigned)std::min<int64_t>((pieces + 255) / 256, 256 * 8);
        expand_q4_kernel<<<grid, 256, 0, s>>>(reinterpret_cast<const v4i*>(wq), reinterpret_cast<v4i*>(w8), pieces);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        return launch_gemm_i8(s, xq, reinterpret_cast<const uint32_t*>(w8), sx, sw, bias, out, out_dtype, m, k / 4, n);
    }
    GemmArgs a{xq, wq, sx, sw, bias, out, m, k / 4, n, 0.f, 0.f, 1, nullptr};
    switch (out_dtype) {
        case OUT_I32: return go_q4<OUT_I32, false>(s, al, a);
        case OUT_F32: return bias ? go_q4<OUT_F32, true>(s, al, a) : go_q4<OUT_F32, false>(s, al, a);
        default: return bias ? go_q4<OUT_BF16, true>(s, al, a) : go_q4<OUT_BF16, false>(s, al, a);
    }
}

// ---------------------------------------------------------------- GEMM + row quantization
// A bf16-output matmul_i8_dyn whose output is then quantized per row for the
// next linear (quant -> matmul_i8_dyn -> quant, as s3dit's block chains its
// int8 linears: crates/s3dit/src/block.rs:727-790). When the GEMM splits K
// over 256x256 tiles (a grid that would leave most CUs idle over a long K,
// e.g. the DiT down projection), one kernel per output row adds the S i32
// slabs, applies the epilogue, stores the bf16 row and quantizes it from the
// bf16 values exactly as quantize_rows_bf16_kernel does (same max, scale and
// rounding): the reduction pass and the quantization's read of the row
// become one pass. Otherwise the GEMM and quantize_rows_bf16 run one after
// the other. Splitting a GEMM only to fuse its quantization does not pay:
// the DiT out projection (1152x3840x3840) as 3-way split 256x256 tiles took
// 31 us + 12.7 us for the fused reduction, against 36.7 + 5.7 us for its
// unsplit 256x128 tiles and the quantization.

static int qfuse_env() {
    static int v = env_int("BH_GEMM_QUANT_FUSE", 1);
    return v;
}

// Splits of the fused form for this shape (0: not fused).
static int qfuse_splits(int m, int kg, int n, bool dma) {
    if (!dma || n % 8 != 0 || n / 4 > 256 * 8 || !qfuse_env()) return 0;
    const TileChoice tc = choose_tiles(m, kg, n);
    return tc.cfg == TILE_256 && tc.splits > 1 && tc.splits <= 4 && column_split(m, kg, n, tc, dma) == 0 ? tc.splits
                                                                                                        : 0;
}

size_t gemm_quant_workspace_ints(int m, int kg, int n) {
    const int S = qfuse_splits(m, kg, n, (kg * 4) % 128 == 0);
    return S ? (size_t)S * m * n : gemm_workspace_ints(m, kg, n);
}

// One block per row: 256 threads, NV groups of 4 columns each (n/4 <= 256*NV).
template <int SN, int NV, bool HAS_BIAS>
__global__ __launch_bounds__(256) void splitk_reduce_quant_kernel(GemmArgs a, float* sx_out, uint32_t* xq_out) {
    const int row = blockIdx.x, n = a.n, n4 = n >> 2;
    const v4i* ws = reinterpret_cast<const v4i*>(a.ws);
    const int64_t q4 = ((int64_t)a.m * n) >> 2;
    const int64_t rq = (int64_t)row * n4;
    v4i acc[NV];
    // Every slab load first, at clamped groups (n4 >= 1), then the scales.
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = min((int)threadIdx.x + 256 * i, n4 - 1);
        acc[i] = ws[rq + g];
    }
#pragma unroll
    for (int sp = 1; sp < SN; ++sp)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int g = min((int)threadIdx.x + 256 * i, n4 - 1);
            const v4i v = ws[(int64_t)sp * q4 + rq + g];
            acc[i][0] += v[0]; acc[i][1] += v[1]; acc[i][2] += v[2]; acc[i][3] += v[3];
        }
    const float sxm = a.sx[row];  // read before this block writes sx_out[row] (they may alias)
    uint2 hb[NV];
    float amax = 0.0f;
    uint2* orow = reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + (int64_t)row * out_ld(a));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + 256 * i;
        hb[i] = make_uint2(0u, 0u);
        if (g >= n4) continue;
        const int col = g * 4;
        const float4 swv = *reinterpret_cast<const float4*>(a.sw + col);
        float f[4] = {dequant(acc[i][0], sxm, swv.x), dequant(acc[i][1], sxm, swv.y), dequant(acc[i][2], sxm, swv.z),
                      dequant(acc[i][3], sxm, swv.w)};
        if constexpr (HAS_BIAS) {
            const float4 bv = *reinterpret_cast<const float4*>(a.bias + col);
            f[0] = f[0] + bv.x; f[1] = f[1] + bv.y; f[2] = f[2] + bv.z; f[3] = f[3] + bv.w;
        }
        hb[i] = make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
        orow[g] = hb[i];
        const uint32_t w[2] = {hb[i].x, hb[i].y};
#pragma unroll
        for (int j = 0; j < 2; ++j)
            amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(w[j] << 16)), fabsf(__uint_as_float(w[j] & 0xffff0000u))));
    }
    amax = xor_max<32>(amax);
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = fmaxf(mx, 1e-8f) / 127.0f;
    if (threadIdx.x == 0) sx_out[row] = sc;
    const float inv = 1.0f / sc;
    uint32_t* q = xq_out + (int64_t)row * n4;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int g = threadIdx.x + 256 * i;
        if (g >= n4) continue;
        q[g] = quant_word(make_float4(__uint_as_float(hb[i].x << 16), __uint_as_float(hb[i].x & 0xffff0000u),
                                      __uint_as_float(hb[i].y << 16), __uint_as_float(hb[i].y & 0xffff0000u)),
                          inv);
    }
}

template <int SN, bool HAS_BIAS>
static void launch_reduce_quant(hipStream_t s, const GemmArgs& a, float* sx_out, uint32_t* xq_out) {
    const int n4 = a.n / 4;
    if (n4 <= 256) splitk_reduce_quant_kernel<SN, 1, HAS_BIAS><<<a.m, 256, 0, s>>>(a, sx_out, xq_out);
    else if (n4 <= 512) splitk_reduce_quant_kernel<SN, 2, HAS_BIAS><<<a.m, 256, 0, s>>>(a, sx_out, xq_out);
    else if (n4 <= 1024) splitk_reduce_quant_kernel<SN, 4, HAS_BIAS><<<a.m, 256, 0, s>>>(a, sx_out, xq_out);
    else splitk_reduce_quant_kernel<SN, 8, HAS_BIAS><<<a.m, 256, 0, s>>>(a, sx_out, xq_out);
}

hipError_t launch_quantize_rows_bf16(hipStream_t s, const uint16_t* x, int m, int k, float* sx, uint32_t* xq);

hipError_t launch_gemm_i8_quant(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* bias, uint16_t* out, int m, int kg, int n, float* sx_out,
                                uint32_t* xq_out) {
    const bool al = gemm_aligned(xq, wq, kg);
    const bool dma = al && ((kg * 4) % 128 == 0);
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(sw) |
                          reinterpret_cast<uintptr_t>(bias)) & 15u) == 0;
    const int S = vec_ok ? qfuse_splits(m, kg, n, dma) : 0;
    if (S >= 2 && S <= 4) {
        hipError_t err = hipSuccess;
        GemmArgs a{xq, wq, sx, sw, bias, out, m, kg, n, 0.f, 0.f, S, nullptr};
        a.ws = splitk_workspace(s, (size_t)S * m * n, &err);
        if (a.ws) {
            err = go_dma<256, 256, 2, 4, 4, 64, OUT_I32, false, false, true, false, true>(s, a);
            if (err != hipSuccess) return err;
            switch (S * 2 + (bias ? 1 : 0)) {
                case 4: launch_reduce_quant<2, false>(s, a, sx_out, xq_out); break;
                case 5: launch_reduce_quant<2, true>(s, a, sx_out, xq_out); break;
                case 6: launch_reduce_quant<3, false>(s, a, sx_out, xq_out); break;
                case 7: launch_reduce_quant<3, true>(s, a, sx_out, xq_out); break;
                case 8: launch_reduce_quant<4, false>(s, a, sx_out, xq_out); break;
                default: launch_reduce_quant<4, true>(s, a, sx_out, xq_out); break;
            }
            return hipGetLastError();
        }
        if (err != hipErrorStreamCaptureUnsupported) return err == hipSuccess ? hipErrorOutOfMemory : err;
        (void)hipGetLastError();  // capturing without the workspace: the unfused pair below
    }
    hipError_t err = launch_gemm_i8(s, xq, wq, sx, sw, bias, out, OUT_BF16, m, kg, n);
    if (err != hipSuccess) return err;
    return launch_quantize_rows_bf16(s, out, m, n, sx_out, xq_out);
}

// ---------------------------------------------------------------- routed-row compaction
// moe_linear_gated_i8 multiplies only the rows routed to its expert
// (gate[r, e] <= 0 is false; moe_linear_gated_i8.wgsl:66-69). At prefill
// sizes the GEMM runs on those rows alone, packed in row order:
// moe_rank_kernel ranks each routed row within its 64-row block (one ballot)
// and counts the block; moe_gather_kernel, one block per row, adds the counts
// of the blocks before it to get the row's slot, copies its codes and scale
// there and records rowmap[slot] = r, or writes the +0 row of an unrouted
// row (row 0's block also stores the total). The GEMM reads the packed rows,
// skips tiles past the total and stores slot k's row to rowmap[k]. No
// counter to clear, no atomics.
constexpr int MOE_PACK_ROWS = 64;  // rows per rank block: one ballot

__global__ __launch_bounds__(64) void moe_rank_kernel(const float* gate, int stride, int col, int m, int* rowpos,
                                                      int* cnt) {
    const int r = blockIdx.x * MOE_PACK_ROWS + threadIdx.x;
    const bool routed = r < m && !(gate[(int64_t)r * stride + col] <= 0.0f);
    const unsigned long long bal = __ballot(routed);
    if (r < m) rowpos[r] = routed ? __popcll(bal & ((1ull << threadIdx.x) - 1ull)) : -1;
    if (threadIdx.x == 0) cnt[blockIdx.x] = __popcll(bal);
}

__global__ __launch_bounds__(256) void moe_gather_kernel(const uint32_t* xq, const float* sx, const int* rowpos,
                                                         const int* cnt, int m, int kg, int n, uint32_t* cxq,
                                                         float* csx, int* rowmap, int* count, float* out) {
    const int r = blockIdx.x;
    const int local = rowpos[r];  // block-uniform, as is r
    int base = 0;
    if (local >= 0 || r == 0) {
        // Row 0 sums every block's count (the total; its own base is 0),
        // a routed row those of the blocks before its own.
        const int lim = r == 0 ? (m + MOE_PACK_ROWS - 1) / MOE_PACK_ROWS : r / MOE_PACK_ROWS;
        int part = 0;
        for (int i = threadIdx.x; i < lim; i += 256) part += cnt[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
        __shared__ int red[4];
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
        __syncthreads();
        const int sum = red[0] + red[1] + red[2] + red[3];
        if (r == 0 && threadIdx.x == 0) *count = sum;
        base = r == 0 ? 0 : sum;
    }
    if (local >= 0) {
        const int k = base + local;
        const v4i* src = reinterpret_cast<const v4i*>(xq + (int64_t)r * kg);
        v4i* dst = reinterpret_cast<v4i*>(cxq + (int64_t)k * kg);
        for (int j = threadIdx.x; j < kg / 4; j += 256) dst[j] = src[j];
        if (threadIdx.x == 0) {
            csx[k] = sx[r];
            rowmap[k] = r;
        }
    } else {
        float* o = out + (int64_t)r * n;
        if ((n & 3) == 0) {
            float4* o4 = reinterpret_cast<float4*>(o);
            for (int j = threadIdx.x; j < n / 4; j += 256) o4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            for (int j = threadIdx.x; j < n; j += 256) o[j] = 0.0f;
        }
    }
}

// Rows from which the gated GEMM compacts; fewer take the per-tile skip.
// The compaction costs a gather of the routed rows and the +0 stores of the
// others (17-23 us at 16384 x 3072 f32) and pays off once the dense GEMM
// needs several waves of tiles. Measured, K=1024 N=3072, per-tile skip ->
// compacted: M=16384 78 -> 49 us at 1/8 routed, 78 -> 61 us at 1/4, 79 -> 96
// us with every row routed; M=8192 45 -> 32 / 46 -> 31 / 46 -> 61 us; M=4096
// and below slower at every fraction (25 -> 33 us at 1/8).
constexpr int MOE_COMPACT_MIN_ROWS = 8192;
static int moe_compact_env() {
    static int v = env_int("BH_MOE_COMPACT", 1);
    return v;
}

hipError_t launch_gemm_i8_gated(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* gate, int gate_stride, int gate_col, float* out, int m,
                                int kg, int n) {
    GemmArgs a{xq, wq, sx, sw, nullptr, out, m, kg, n, 0.f, 0.f, 1, nullptr, gate, gate_stride, gate_col};
    const bool al = gemm_aligned(xq, wq, kg);
    const bool dma = al && ((kg * 4) % 128 == 0);
    if (dma && m >= MOE_COMPACT_MIN_ROWS && moe_compact_env()) {
        // Workspace (its own slot of the stream's workspaces): packed codes
        // [m][kg], scales [m], rowmap [m], rowpos [m], block counts, total.
        // Under a capture that finds it too small, the uncompacted path below
        // runs instead.
        const size_t pad = ((size_t)m + 63) / 64 * 64;
        const size_t ints = (size_t)m * kg + 3 * pad + pad / MOE_PACK_ROWS + 64;
        hipError_t err = hipSuccess;
        int* ws = splitk_workspace(s, ints, &err, 3);
        if (ws) {
            uint32_t* cxq = reinterpret_cast<uint32_t*>(ws);
            float* csx = reinterpret_cast<float*>(ws + (size_t)m * kg);
            int* rowmap = ws + (size_t)m * kg + pad;
            int* rowpos = rowmap + pad;
            int* cnt = rowpos + pad;  // (m + 63) / 64 block counts
            int* count = cnt + pad / MOE_PACK_ROWS;
            moe_rank_kernel<<<(m + MOE_PACK_ROWS - 1) / MOE_PACK_ROWS, 64, 0, s>>>(gate, gate_stride, gate_col, m,
                                                                                 rowpos, cnt);
            if ((err = hipGetLastError()) != hipSuccess) return err;
            moe_gather_kernel<<<m, 256, 0, s>>>(xq, sx, rowpos, cnt, m, kg, n, cxq, csx, rowmap, count, out);
            if ((err = hipGetLastError()) != hipSuccess) return err;
            GemmArgs c{cxq, wq, csx, sw, nullptr, out, m, kg, n, 0.f, 0.f, 1, nullptr};
            c.m_dev = count;
            c.row_map = rowmap;
            TileChoice tc = choose_tiles(m, kg, n);
            tc.splits = 1;
            return go_cfg<OUT_F32, false, false>(s, true, true, tc, c);
        }
        (void)hipGetLastError();
    }
    return run_gemm<OUT_F32, false, false>(s, al, dma, choose_tiles(m, kg, n), a);
}

}  // namespace bh
