// C ABI of the gfx950 int8 backend: argument checking, the typed launchers,
// the backend_api::Backend mirror (buffers, recorded steps, ordered submit,
// per-kernel timing, stats), the I8 selector, the cost model and the host
// weight quantizer. See include/brain_hip.h for the contract of each call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <tuple>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/brain_hip.h"
#include "bh_common.h"
#include "bh_kv8.h"

namespace bh {
hipError_t launch_max_abs_rows(hipStream_t s, const float* x, int m, int k, float* sx);
hipError_t launch_quant_pack(hipStream_t s, const float* x, const float* sx, int m, int k, uint32_t* xq);
hipError_t launch_quantize_rows(hipStream_t s, const float* x, int m, int k, float* sx, uint32_t* xq);
hipError_t launch_quantize_rows_bf16(hipStream_t s, const uint16_t* x, int m, int k, float* sx, uint32_t* xq);
hipError_t launch_quantize_weight(hipStream_t s, const float* w, int n, int k, uint32_t* packed, float* sw);
hipError_t launch_gemv_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n,
                          bool keep_cached = false, float* am_v = nullptr, uint32_t* am_i = nullptr,
                          uint32_t* am_n = nullptr, int am_stride = 0);
hipError_t launch_gemm_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n);
hipError_t launch_gemm_i8_static(hipStream_t s, const uint32_t* xq, const uint32_t* wq, float ssx, float ssw,
                                 float* out, int m, int kg, int n);

size_t gemm_workspace_ints(int m, int kg, int n);
size_t gemm_quant_workspace_ints(int m, int kg, int n);
hipError_t launch_gemm_i8_quant(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* bias, uint16_t* out, int m, int kg, int n, float* sx_out,
                                uint32_t* xq_out);
hipError_t launch_gemm_i8_noalloc(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                  const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n,
                                  size_t* need_bytes);
size_t noalloc_scratch_bytes();
size_t gemm_q4_workspace_ints(int m, int k, int n);
hipError_t launch_gemv_i8_gated(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* gate, int gate_stride, int gate_col, float* out, int m,
                                int kg, int n);
hipError_t launch_gemm_i8_gated(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* gate, int gate_stride, int gate_col, float* out, int m,
                                int kg, int n);
hipError_t launch_linear_i8_fused(hipStream_t s, const float* x, const uint32_t* wq, const float* sw,
                                  const float* bias, float* sx_out, uint32_t* xq_out, void* out, int out_dtype, int m,
                                  int kg, int n);
hipError_t launch_gemv_q4(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                          const float* bias, void* out, int out_dtype, int m, int k, int n);
hipError_t launch_gemm_q4(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int k, int n);

// Split-K workspace, one per (device, stream): the S partial slabs of a
// split GEMM. Every split kernel overwrites the slabs it uses before the
// reduction reads them, so the buffer is never cleared. Calls on one stream
// are ordered, so they never share it concurrently; a graph captured on the
// stream replays in that stream's order too.
struct SplitWs {
    int device;
    hipStream_t stream;
    int slot;  // 0: split-K slabs, 1: W4A8 weights expanded to int8
    int* ws;
    size_t ints;
};
static std::mutex g_ws_mu;
static std::vector<SplitWs> g_ws;

int* splitk_workspace(hipStream_t st, size_t ints, hipError_t* err, int slot) {
    int dev = 0;
    *err = hipGetDevice(&dev);
    if (*err != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(g_ws_mu);
    SplitWs* w = nullptr;
    for (auto& x : g_ws)
        if (x.device == dev && x.stream == st && x.slot == slot) w = &x;
    if (!w) {
        g_ws.push_back(SplitWs{dev, st, slot, nullptr, 0});
        w = &g_ws.back();
    }
    if (w->ints < ints) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
            // No allocation inside a capture: the caller reserves beforehand.
            *err = hipErrorStreamCaptureUnsupported;
            return nullptr;
        }
        // Growing. The old buffer is kept, not freed, until the process ends:
        // a HIP graph captured earlier may still launch kernels that use it.
        // (Sizes only grow and each is capped, so this retains little.)
        int* nb = nullptr;
        if ((*err = hipMalloc(&nb, ints * 4)) != hipSuccess) return nullptr;
        w->ws = nb;
        w->ints = ints;
    }
    return w->ws;
}

// ---------------------------------------------------------------- small kernels
__global__ void f32_to_bf16_kernel(const float* x, uint16_t* out, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = f32_to_bf16_rne(x[i]);
}

__global__ void fill_zero_kernel(uint32_t* p, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// bias_add.wgsl: out[i] += bias[i % n]
__global__ void bias_add_kernel(float* out, const float* bias, uint64_t total, uint32_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = out[i] + bias[i % n];
}

// roof_dp4a.wgsl:28-63: eight independent dot4 chains, folded in the same
// order, out[idx] = inp[idx] + f32(s) (wrapping i32 arithmetic).
__global__ void roof_dp4a_kernel(const float* inp, float* out, uint32_t n, uint32_t iters, uint32_t a, uint32_t b) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    int c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = 0; i < iters; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_sdot4((int)a, (int)b, c[j], false);
    const int s = (int)(((uint32_t)c[0] + (uint32_t)c[1]) + ((uint32_t)c[2] + (uint32_t)c[3]) +
                        (((uint32_t)c[4] + (uint32_t)c[5]) + ((uint32_t)c[6] + (uint32_t)c[7])));
    out[idx] = inp[idx] + (float)s;
}

// Matrix-core roof: 4 independent v_mfma_i32_32x32x32_i8 chains per wave
// (65536 int ops each), the instruction the prefill GEMM is built on.
__global__ __launch_bounds__(256) void roof_mfma_i8_kernel(uint32_t iters, int32_t* out) {
    const int lane = threadIdx.x & 63;
    v4i a = {lane, lane * 3 + 1, lane ^ 5, 7};
    v4i b = {lane + 2, 11, lane * 5, lane ^ 9};
    v16i c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) c[j][e] = j + e;
    for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][5] + c[j][10] + c[j][15];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Bandwidth roof (the read side of crates/gpu-core/src/roof.rs:458-490's axpy
// probe): `words4` 16-byte words read with 16-byte non-temporal vector loads
// (the fastest plain streaming read measured: 6.3-6.6 TB/s against 5.6-5.8
// without the hint). Each workgroup
// reads contiguous runs of 256 x 8 words (8 loads in flight per thread, 4 KB
// apart), the runs spread over the grid; the words are XOR-folded so no load
// is dead, one word per thread written.
__device__ __forceinline__ uint4 nt_word4(const uint4* p) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(w[0], w[1], w[2], w[3]);
}
__global__ __launch_bounds__(256) void roof_hbm_read_kernel(const uint4* __restrict__ src, uint64_t words4,
                                                            uint32_t* out) {
    constexpr int U = 8;
    const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
    uint32_t acc = 0;
    uint64_t i = (uint64_t)blockIdx.x * 256 * U + threadIdx.x;
    for (; i + (U - 1) * 256 < words4; i += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = nt_word4(src + i + u * 256);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (int u = 0; u < U; ++u)
        if (i + u * 256 < words4) {
            const uint4 v = nt_word4(src + i + u * 256);
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    out[(uint64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// ---------------------------------------------------------------- errors
static thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

static int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return BH_OK;
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(BH_ERR_INVALID,
                    "%s: this shape needs the split-K workspace, which cannot be allocated while the stream is "
                    "capturing; call bh_reserve_workspace on this stream first",
                    what);
    return fail(BH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

static constexpr uint64_t I32MAX = 0x7fffffffull;

// ---------------------------------------------------------------- typed API checks
static int check_matmul(const void* xq, const void* wq, const void* sx, const void* sw, const void* out,
                        int out_dtype, uint32_t m, uint32_t kg, uint32_t n, const char* who) {
    if (out_dtype != OUT_F32 && out_dtype != OUT_BF16 && out_dtype != OUT_I32) return fail(BH_ERR_INVALID, "%s: out_dtype %d", who, out_dtype);
    if ((uint64_t)kg * 4 > I32MAX || m > I32MAX || n > I32MAX)
        return fail(BH_ERR_INVALID, "%s: shape m=%u kg=%u n=%u out of range", who, m, kg, n);
    if (m == 0 || n == 0) return BH_OK;
    if (!out || (out_dtype != OUT_I32 && (!sx || !sw)) || (kg > 0 && (!xq || !wq)))
        return fail(BH_ERR_INVALID, "%s: null buffer for m=%u kg=%u n=%u", who, m, kg, n);
    return BH_OK;
}

static const int GEMV_MAX_ROWS = 32;

// Measured GEMV-vs-tile choices, keyed by (row bucket, n, k): the bucket is m
// rounded up to a power of two (m <= 32), as Engine::mm8 keys its tuned map
// (crates/qwen3/src/serve.rs:1088-1097).
static std::mutex g_tune_mu;
static std::map<std::tuple<uint32_t, uint32_t, uint32_t>, int> g_tune;

static uint32_t row_bucket(uint32_t m) {
    uint32_t b = 1;
    while (b < m) b <<= 1;
    return std::min<uint32_t>(b, GEMV_MAX_ROWS);
}

// The tuned variant for this shape, or 0 when none was measured.
int tuned_variant(uint32_t m, uint32_t n, uint32_t k) {
    if (m == 0 || m > (uint32_t)GEMV_MAX_ROWS) return 0;
    std::lock_guard<std::mutex> g(g_tune_mu);
    auto it = g_tune.find({row_bucket(m), n, k});
    return it == g_tune.end() ? 0 : it->second;
}

}  // namespace bh

using namespace bh;

extern "C" {

const char* bh_last_error(void) { return g_err.c_str(); }
int bh_abi_version(void) { return BH_ABI_VERSION; }

int bh_max_abs_rows(void* stream, const float* x, uint32_t m, uint32_t k, float* sx) {
    if (m > I32MAX || k > I32MAX) return fail(BH_ERR_INVALID, "bh_max_abs_rows: m=%u k=%u", m, k);
    if (m == 0) return BH_OK;
    if (!sx || (k > 0 && !x)) return fail(BH_ERR_INVALID, "bh_max_abs_rows: null buffer");
    return hip_status(launch_max_abs_rows((hipStream_t)stream, x, (int)m, (int)k, sx), "max_abs_rows launch");
}

int bh_quant_pack(void* stream, const float* x, const float* sx, uint32_t m, uint32_t k, uint32_t* xq) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_quant_pack: k=%u is not a multiple of 4", k);
    if (m > I32MAX || k > I32MAX) return fail(BH_ERR_INVALID, "bh_quant_pack: m=%u k=%u", m, k);
    if (m == 0 || k == 0) return BH_OK;
    if (!x || !sx || !xq) return fail(BH_ERR_INVALID, "bh_quant_pack: null buffer");
    return hip_status(launch_quant_pack((hipStream_t)stream, x, sx, (int)m, (int)k, xq), "quant_pack launch");
}

int bh_quantize_rows(void* stream, const float* x, uint32_t m, uint32_t k, float* sx, uint32_t* xq) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_quantize_rows: k=%u is not a multiple of 4", k);
    if (m > I32MAX || k > I32MAX) return fail(BH_ERR_INVALID, "bh_quantize_rows: m=%u k=%u", m, k);
    if (m == 0) return BH_OK;
    if (!sx || (k > 0 && (!x || !xq))) return fail(BH_ERR_INVALID, "bh_quantize_rows: null buffer");
    return hip_status(launch_quantize_rows((hipStream_t)stream, x, (int)m, (int)k, sx, xq), "quantize_rows launch");
}

int bh_quantize_rows_bf16(void* stream, const uint16_t* x, uint32_t m, uint32_t k, float* sx, uint32_t* xq) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_quantize_rows_bf16: k=%u is not a multiple of 4", k);
    if (m > I32MAX || k > I32MAX) return fail(BH_ERR_INVALID, "bh_quantize_rows_bf16: m=%u k=%u", m, k);
    if (m == 0) return BH_OK;
    if (!sx || (k > 0 && (!x || !xq))) return fail(BH_ERR_INVALID, "bh_quantize_rows_bf16: null buffer");
    return hip_status(launch_quantize_rows_bf16((hipStream_t)stream, x, (int)m, (int)k, sx, xq), "quantize_rows_bf16 launch");
}

int bh_matmul_i8_gemv(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                      const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n) {
    int rc = check_matmul(xq, wq, sx, sw, out, out_dtype, m, kg, n, "bh_matmul_i8_gemv");
    if (rc) return rc;
    if (m > (uint32_t)GEMV_MAX_ROWS) return fail(BH_ERR_INVALID, "bh_matmul_i8_gemv: m=%u > %d", m, GEMV_MAX_ROWS);
    if (m == 0 || n == 0) return BH_OK;
    return hip_status(launch_gemv_i8((hipStream_t)stream, xq, wq, sx, sw, bias, out, out_dtype, (int)m, (int)kg,
                                     (int)n),
                      "gemv_i8 launch");
}

int bh_matmul_i8_dyn(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                     const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n) {
    int rc = check_matmul(xq, wq, sx, sw, out, out_dtype, m, kg, n, "bh_matmul_i8_dyn");
    if (rc) return rc;
    if (m == 0 || n == 0) return BH_OK;
    const uint64_t tiles = (((uint64_t)m + 127) / 128) * (((uint64_t)n + 127) / 128);
    if (tiles > I32MAX) return fail(BH_ERR_INVALID, "bh_matmul_i8_dyn: %llu tiles", (unsigned long long)tiles);
    hipError_t e = launch_gemm_i8((hipStream_t)stream, xq, wq, sx, sw, bias, out, out_dtype, (int)m, (int)kg, (int)n);
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(BH_ERR_INVALID,
                    "bh_matmul_i8_dyn: m=%u kg=%u n=%u needs the split-K workspace, which cannot be allocated while "
                    "the stream is capturing; call bh_reserve_workspace on this stream first",
                    m, kg, n);
    return hip_status(e, "gemm_i8 launch");
}

int bh_matmul_i8_dyn_quant(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                           const float* bias, uint16_t* out, uint32_t m, uint32_t kg, uint32_t n, float* sx_out,
                           uint32_t* xq_out) {
    int rc = check_matmul(xq, wq, sx, sw, out, OUT_BF16, m, kg, n, "bh_matmul_i8_dyn_quant");
    if (rc) return rc;
    if (n % 4 != 0) return fail(BH_ERR_INVALID, "bh_matmul_i8_dyn_quant: n=%u is not a multiple of 4", n);
    if (m == 0) return BH_OK;
    if (n == 0 || !sx_out || !xq_out) return fail(BH_ERR_INVALID, "bh_matmul_i8_dyn_quant: n=%u or null output", n);
    const uint64_t tiles = (((uint64_t)m + 127) / 128) * (((uint64_t)n + 127) / 128);
    if (tiles > I32MAX) return fail(BH_ERR_INVALID, "bh_matmul_i8_dyn_quant: %llu tiles", (unsigned long long)tiles);
    hipError_t e = launch_gemm_i8_quant((hipStream_t)stream, xq, wq, sx, sw, bias, out, (int)m, (int)kg, (int)n,
                                        sx_out, xq_out);
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(BH_ERR_INVALID,
                    "bh_matmul_i8_dyn_quant: m=%u kg=%u n=%u needs the split-K workspace, which cannot be allocated "
                    "while the stream is capturing; call bh_reserve_workspace on this stream first",
                    m, kg, n);
    return hip_status(e, "gemm_i8_quant launch");
}

int bh_matmul_i8_dyn_noalloc(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx,
                             const float* sw, const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg,
                             uint32_t n) {
    int rc = check_matmul(xq, wq, sx, sw, out, out_dtype, m, kg, n, "bh_matmul_i8_dyn_noalloc");
    if (rc) return rc;
    if (m == 0 || n == 0) return BH_OK;
    const uint64_t tiles = (((uint64_t)m + 127) / 128) * (((uint64_t)n + 127) / 128);
    if (tiles > I32MAX)
        return fail(BH_ERR_INVALID, "bh_matmul_i8_dyn_noalloc: %llu tiles", (unsigned long long)tiles);
    size_t need = 0;
    hipError_t e = launch_gemm_i8_noalloc((hipStream_t)stream, xq, wq, sx, sw, bias, out, out_dtype, (int)m, (int)kg,
                                          (int)n, &need);
    if (e == hipErrorNotReady)
        return fail(BH_ERR_INVALID,
                    "bh_matmul_i8_dyn_noalloc: a call on another stream of this GPU is still using the fixed "
                    "split-K scratch; order the calls (same stream, or wait for the other stream) and retry");
    if (e == hipErrorInvalidValue && need > noalloc_scratch_bytes())
        return fail(BH_ERR_INVALID,
                    "bh_matmul_i8_dyn_noalloc: m=%u kg=%u n=%u needs %zu bytes of split-K scratch, more than the "
                    "fixed %zu; use bh_matmul_i8_dyn",
                    m, kg, n, need, noalloc_scratch_bytes());
    return hip_status(e, "gemm_i8 launch (no allocation)");
}

int bh_reserve_workspace(void* stream, uint32_t m, uint32_t kg, uint32_t n) {
    if ((uint64_t)kg * 4 > I32MAX || m > I32MAX || n > I32MAX)
        return fail(BH_ERR_INVALID, "bh_reserve_workspace: m=%u kg=%u n=%u out of range", m, kg, n);
    // Both workspaces a GEMM of this shape may take: the split-K slabs of the
    // int8 GEMM (bh_matmul_i8_dyn or bh_matmul_i8_dyn_quant), and for W4A8
    // (K = 4*kg) the weights expanded to int8.
    const size_t need[2] = {std::max(gemm_workspace_ints((int)m, (int)kg, (int)n),
                                     gemm_quant_workspace_ints((int)m, (int)kg, (int)n)),
                            gemm_q4_workspace_ints((int)m, (int)kg * 4, (int)n)};
    for (int slot = 0; slot < 2; ++slot) {
        if (!need[slot]) continue;
        hipError_t err = hipSuccess;
        if (!splitk_workspace((hipStream_t)stream, need[slot], &err, slot)) {
            if (err == hipErrorStreamCaptureUnsupported)
                return fail(BH_ERR_INVALID, "bh_reserve_workspace: stream is capturing; reserve before capture");
            return fail(err == hipErrorOutOfMemory ? BH_ERR_NOMEM : BH_ERR_HIP, "bh_reserve_workspace: %s",
                        hipGetErrorString(err));
        }
    }
    return BH_OK;
}

// select::candidates, I8 arm (crates/backend-api/src/select.rs:197, 209,
// 323-331): above DECODE_REGIME_MAX_ROWS rows, or without workgroup
// reductions, the tile alone; up to I8_GEMV_MAX_ROWS the GEMV first; in
// between the tile first. This is the reference's order, unchanged; what
// runs on MI355X is bh_matmul_i8's launch policy below.
static const uint32_t DECODE_REGIME_MAX_ROWS = 32;
static const uint32_t I8_GEMV_MAX_ROWS = 8;

int bh_select_i8(uint32_t m, uint32_t n, uint32_t k, int int8_dot, int workgroup_reductions, int out[2]) {
    (void)n;
    (void)k;
    if (!out) return fail(BH_ERR_INVALID, "bh_select_i8: null out");
    if (!int8_dot) return 0;
    if (m > DECODE_REGIME_MAX_ROWS || !workgroup_reductions) {
        out[0] = BH_VARIANT_PACKED_INT8;
        return 1;
    }
    if (m <= I8_GEMV_MAX_ROWS) {
        out[0] = BH_VARIANT_WORKGROUP_PER_OUTPUT;
        out[1] = BH_VARIANT_PACKED_INT8;
    } else {
        out[0] = BH_VARIANT_PACKED_INT8;
        out[1] = BH_VARIANT_WORKGROUP_PER_OUTPUT;
    }
    return 2;
}

const char* bh_variant_kernel(int variant) {
    switch (variant) {
        case BH_VARIANT_PACKED_INT8: return "matmul_i8_dyn";
        case BH_VARIANT_WORKGROUP_PER_OUTPUT: return "matmul_i8_gemv";
        default: return nullptr;
    }
}

int bh_matmul_i8(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                 const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n) {
    // Launch policy: a measured choice for this shape (bh_tune_i8 /
    // bh_tune_set) wins; otherwise the MI355X crossover, which is not the
    // P40 one the reference's candidate order encodes (I8_GEMV_MAX_ROWS = 8):
    // the MFMA GEMV streams the weights once for up to 32 rows and beat the
    // tile at every measured m <= 32 of the configs[1] shapes, so every row
    // count in the decode regime takes the GEMV.
    int v = tuned_variant(m, n, kg * 4);
    if (!v) v = m <= DECODE_REGIME_MAX_ROWS ? BH_VARIANT_WORKGROUP_PER_OUTPUT : BH_VARIANT_PACKED_INT8;
    if (v == BH_VARIANT_WORKGROUP_PER_OUTPUT)
        return bh_matmul_i8_gemv(stream, xq, wq, sx, sw, bias, out, out_dtype, m, kg, n);
    return bh_matmul_i8_dyn(stream, xq, wq, sx, sw, bias, out, out_dtype, m, kg, n);
}

int bh_matmul_i8_static(void* stream, const uint32_t* xq, const uint32_t* wq, float sx, float sw, float* out,
                        uint32_t m, uint32_t kg, uint32_t n) {
    int rc = check_matmul(xq, wq, &sx, &sw, out, OUT_F32, m, kg, n, "bh_matmul_i8_static");
    if (rc) return rc;
    if (m == 0 || n == 0) return BH_OK;
    return hip_status(launch_gemm_i8_static((hipStream_t)stream, xq, wq, sx, sw, out, (int)m, (int)kg, (int)n),
                      "gemm_i8_static launch");
}

int bh_linear_i8(void* stream, const float* x, const uint32_t* wq, const float* sw, const float* bias,
                 float* sx_scratch, uint32_t* xq_scratch, void* out, int out_dtype, uint32_t m, uint32_t k,
                 uint32_t n) {
    // Decode rows on the GEMV: one launch that quantizes in its prologue
    // (bit-identical scratch contents and outputs), when its shape rules allow.
    if (m >= 1 && m <= 16 && k % 4 == 0 && k > 0 && n > 0 && x && wq && sw && out && sx_scratch && xq_scratch &&
        (out_dtype == OUT_F32 || out_dtype == OUT_BF16) && !tuned_variant(m, n, k) && m <= (uint32_t)GEMV_MAX_ROWS) {
        const hipError_t e = launch_linear_i8_fused((hipStream_t)stream, x, wq, sw, bias, sx_scratch, xq_scratch, out,
                                                    out_dtype, (int)m, (int)(k / 4), (int)n);
        if (e == hipSuccess) return BH_OK;
        if (e != hipErrorNotSupported) return hip_status(e, "linear_i8 fused launch");
    }
    int rc = bh_quantize_rows(stream, x, m, k, sx_scratch, xq_scratch);
    if (rc) return rc;
    return bh_matmul_i8(stream, xq_scratch, wq, sx_scratch, sw, bias, out, out_dtype, m, k / 4, n);
}

int bh_quantize_weight_device(void* stream, const float* w, uint32_t n, uint32_t k, uint32_t* packed, float* sw) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_quantize_weight_device: k=%u is not a multiple of 4", k);
    if (n > I32MAX || k > I32MAX) return fail(BH_ERR_INVALID, "bh_quantize_weight_device: n=%u k=%u", n, k);
    if (n == 0) return BH_OK;
    if (!sw || (k > 0 && (!w || !packed))) return fail(BH_ERR_INVALID, "bh_quantize_weight_device: null buffer");
    return hip_status(launch_quantize_weight((hipStream_t)stream, w, (int)n, (int)k, packed, sw),
                      "quantize_weight launch");
}

static int check_q4(const void* xq, const void* wq, const void* sx, const void* sw, const void* out, int out_dtype,
                    uint32_t m, uint32_t k, uint32_t n, const char* who) {
    if (k % 8) return fail(BH_ERR_INVALID, "%s: k=%u is not a multiple of 8", who, k);
    return check_matmul(xq, wq, sx, sw, out, out_dtype, m, k / 4, n, who);
}

int bh_matmul_q4_gemv(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                      const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n) {
    int rc = check_q4(xq, wq4, sx, sw, out, out_dtype, m, k, n, "bh_matmul_q4_gemv");
    if (rc) return rc;
    if (m > (uint32_t)GEMV_MAX_ROWS) return fail(BH_ERR_INVALID, "bh_matmul_q4_gemv: m=%u > %d", m, GEMV_MAX_ROWS);
    if (m == 0 || n == 0) return BH_OK;
    return hip_status(launch_gemv_q4((hipStream_t)stream, xq, wq4, sx, sw, bias, out, out_dtype, (int)m, (int)k, (int)n),
                      "gemv_q4 launch");
}

int bh_matmul_q4_dyn(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                     const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n) {
    int rc = check_q4(xq, wq4, sx, sw, out, out_dtype, m, k, n, "bh_matmul_q4_dyn");
    if (rc) return rc;
    if (m == 0 || n == 0) return BH_OK;
    return hip_status(launch_gemm_q4((hipStream_t)stream, xq, wq4, sx, sw, bias, out, out_dtype, (int)m, (int)k, (int)n),
                      "gemm_q4 launch");
}

int bh_matmul_q4(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                 const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n) {
    if (m <= (uint32_t)GEMV_MAX_ROWS) return bh_matmul_q4_gemv(stream, xq, wq4, sx, sw, bias, out, out_dtype, m, k, n);
    return bh_matmul_q4_dyn(stream, xq, wq4, sx, sw, bias, out, out_dtype, m, k, n);
}

int bh_moe_linear_gated_i8(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                           const float* gate, uint32_t n_experts, uint32_t e_idx, float* out, uint32_t m, uint32_t kg,
                           uint32_t n) {
    int rc = check_matmul(xq, wq, sx, sw, out, OUT_F32, m, kg, n, "bh_moe_linear_gated_i8");
    if (rc) return rc;
    if (m == 0 || n == 0) return BH_OK;
    if (!gate || e_idx >= n_experts || n_experts > I32MAX)
        return fail(BH_ERR_INVALID, "bh_moe_linear_gated_i8: gate null or e_idx %u >= n_experts %u", e_idx, n_experts);
    const hipError_t e = m <= (uint32_t)GEMV_MAX_ROWS
                             ? launch_gemv_i8_gated((hipStream_t)stream, xq, wq, sx, sw, gate, (int)n_experts, (int)e_idx,
                                                    out, (int)m, (int)kg, (int)n)
                             : launch_gemm_i8_gated((hipStream_t)stream, xq, wq, sx, sw, gate, (int)n_experts, (int)e_idx,
                                                    out, (int)m, (int)kg, (int)n);
    return hip_status(e, "moe_linear_gated_i8 launch");
}

// ---------------------------------------------------------------- int8 paged KV
static int check_kv_geom(const char* who, uint32_t kv_stride, uint32_t bs, uint32_t hd) {
    if (hd == 0 || hd % 4 || hd > 256 || kv_stride == 0 || kv_stride % hd || bs == 0)
        return fail(BH_ERR_INVALID, "%s: head_dim %u (a multiple of 4, <= 256), kv_stride %u (a multiple of "
                    "head_dim) and block_size %u (> 0) do not fit", who, hd, kv_stride, bs);
    return BH_OK;
}

int bh_paged_kv_append_i8(void* stream, const float* src, const uint32_t* blocks, const uint32_t* offsets,
                          const float* clip, uint32_t* pool, uint64_t pool_words, float* scales, uint64_t n_scales,
                          uint32_t batch, uint32_t kv_stride, uint32_t block_size, uint32_t head_dim) {
    int rc = check_kv_geom("bh_paged_kv_append_i8", kv_stride, block_size, head_dim);
    if (rc) return rc;
    if (batch == 0) return BH_OK;
    if (!src || !blocks || !offsets || !clip || !pool || !scales)
        return fail(BH_ERR_INVALID, "bh_paged_kv_append_i8: null buffer");
    if ((uint64_t)batch * (kv_stride / head_dim) > I32MAX)
        return fail(BH_ERR_INVALID, "bh_paged_kv_append_i8: batch %u x %u heads", batch, kv_stride / head_dim);
    return hip_status(launch_paged_kv_append_i8((hipStream_t)stream, src, blocks, offsets, clip, pool, pool_words,
                                                scales, n_scales, batch, kv_stride, block_size, head_dim),
                      "paged_kv_append_i8 launch");
}

static int paged_read(void* stream, bool apply, const char* who, const float* in, const uint32_t* pool,
                      uint64_t pool_words, const uint32_t* bt, const uint32_t* seq_lens, const float* scales,
                      uint64_t n_scales, float* out, uint32_t batch, uint32_t n_heads, uint32_t group, uint32_t hd,
                      uint32_t bs, uint32_t kv_stride, uint32_t cap, uint32_t max_bt, float scale) {
    int rc = check_kv_geom(who, kv_stride, bs, hd);
    if (rc) return rc;
    if (group == 0 || (n_heads && (n_heads - 1) / group >= kv_stride / hd))
        return fail(BH_ERR_INVALID, "%s: %u heads in groups of %u need more than the %u kv heads", who, n_heads,
                    group, kv_stride / hd);
    if (batch == 0 || n_heads == 0 || (!apply && cap == 0)) return BH_OK;
    if (!in || !pool || !bt || !seq_lens || !scales || !out) return fail(BH_ERR_INVALID, "%s: null buffer", who);
    if ((uint64_t)batch * n_heads * (((apply ? hd : cap) + 63) / 64) > I32MAX)
        return fail(BH_ERR_INVALID, "%s: grid too large", who);
    PagedReadArgs a{in, pool, pool_words, bt, seq_lens, scales, n_scales, out, n_heads, group, hd, bs, kv_stride,
                    cap, max_bt, scale};
    return hip_status(launch_paged_decode_i8((hipStream_t)stream, apply, a, batch), who);
}

int bh_paged_decode_scores_i8(void* stream, const float* q, const uint32_t* pool, uint64_t pool_words,
                              const uint32_t* block_tables, const uint32_t* seq_lens, const float* scales,
                              uint64_t n_scales, float* scores, uint32_t batch, uint32_t n_heads, uint32_t group,
                              uint32_t head_dim, uint32_t block_size, uint32_t kv_stride, uint32_t cap,
                              uint32_t max_bt, float scale) {
    return paged_read(stream, false, "bh_paged_decode_scores_i8", q, pool, pool_words, block_tables, seq_lens, scales,
                      n_scales, scores, batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt, scale);
}

int bh_paged_decode_apply_i8(void* stream, const float* probs, const uint32_t* pool, uint64_t pool_words,
                             const uint32_t* block_tables, const uint32_t* seq_lens, const float* scales,
                             uint64_t n_scales, float* ctx, uint32_t batch, uint32_t n_heads, uint32_t group,
                             uint32_t head_dim, uint32_t block_size, uint32_t kv_stride, uint32_t cap,
                             uint32_t max_bt) {
    return paged_read(stream, true, "bh_paged_decode_apply_i8", probs, pool, pool_words, block_tables, seq_lens,
                      scales, n_scales, ctx, batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt,
                      0.0f);
}

int bh_f32_to_bf16(void* stream, const float* x, uint16_t* out, uint64_t n) {
    if (n == 0) return BH_OK;
    if (!x || !out) return fail(BH_ERR_INVALID, "bh_f32_to_bf16: null buffer");
    const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
    f32_to_bf16_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(x, out, n);
    return hip_status(hipGetLastError(), "f32_to_bf16 launch");
}

int bh_roof_mfma_i8(void* stream, uint32_t blocks, uint32_t iters, int32_t* out) {
    if (blocks == 0 || blocks > I32MAX || !out) return fail(BH_ERR_INVALID, "bh_roof_mfma_i8: blocks=%u", blocks);
    roof_mfma_i8_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(iters, out);
    return hip_status(hipGetLastError(), "roof_mfma_i8 launch");
}

int bh_roof_hbm_read(void* stream, const void* src, uint64_t bytes, uint32_t blocks, uint32_t* out) {
    if (blocks == 0 || blocks > 65536 || !out || (bytes && !src) || bytes % 16 || ((uintptr_t)src & 15))
        return fail(BH_ERR_INVALID, "bh_roof_hbm_read: blocks=%u bytes=%llu (16-byte aligned multiple of 16)", blocks,
                    (unsigned long long)bytes);
    roof_hbm_read_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(static_cast<const uint4*>(src), bytes / 16, out);
    return hip_status(hipGetLastError(), "roof_hbm_read launch");
}

// ---------------------------------------------------------------- autotune
// Engine::measure_i8 (crates/qwen3/src/serve.rs:1133-1158): both candidates on
// the same buffers, `reps` dispatches back to back after one warm-up, mean ms
// per dispatch; the faster is recorded for the shape's row bucket.
int bh_tune_i8(void* stream, uint32_t m, uint32_t k, uint32_t n, uint32_t reps, int* variant, float ms[2]) {
    if (!variant || m == 0 || m > (uint32_t)GEMV_MAX_ROWS || n == 0 || k == 0 || k % 4 || reps == 0 ||
        (uint64_t)n * k > I32MAX)
        return fail(BH_ERR_INVALID, "bh_tune_i8: m=%u k=%u n=%u reps=%u (m must be 1..32)", m, k, n, reps);
    hipStream_t st = (hipStream_t)stream;
    void *xq = nullptr, *wq = nullptr, *sx = nullptr, *sw = nullptr, *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = BH_OK;
    float t[2] = {0.f, 0.f};
    auto cleanup = [&]() {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        for (void* p : {xq, wq, sx, sw, out})
            if (p) (void)hipFree(p);
    };
    if (hipMalloc(&xq, (size_t)m * k) != hipSuccess || hipMalloc(&wq, (size_t)n * k) != hipSuccess ||
        hipMalloc(&sx, (size_t)m * 4) != hipSuccess || hipMalloc(&sw, (size_t)n * 4) != hipSuccess ||
        hipMalloc(&out, (size_t)m * n * 4) != hipSuccess) {
        cleanup();
        return fail(BH_ERR_NOMEM, "bh_tune_i8: scratch allocation failed");
    }
    (void)hipMemsetAsync(xq, 1, (size_t)m * k, st);
    (void)hipMemsetAsync(wq, 1, (size_t)n * k, st);
    (void)hipMemsetAsync(sx, 0, (size_t)m * 4, st);
    (void)hipMemsetAsync(sw, 0, (size_t)n * 4, st);
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        cleanup();
        return fail(BH_ERR_HIP, "bh_tune_i8: event creation failed");
    }
    const int cand[2] = {BH_VARIANT_WORKGROUP_PER_OUTPUT, BH_VARIANT_PACKED_INT8};
    for (int c = 0; c < 2 && rc == BH_OK; ++c) {
        auto run = [&]() {
            return cand[c] == BH_VARIANT_WORKGROUP_PER_OUTPUT
                       ? bh_matmul_i8_gemv(stream, (const uint32_t*)xq, (const uint32_t*)wq, (const float*)sx,
                                           (const float*)sw, nullptr, out, OUT_F32, m, k / 4, n)
                       : bh_matmul_i8_dyn(stream, (const uint32_t*)xq, (const uint32_t*)wq, (const float*)sx,
                                          (const float*)sw, nullptr, out, OUT_F32, m, k / 4, n);
        };
        if ((rc = run()) != BH_OK) break;
        (void)hipEventRecord(e0, st);
        for (uint32_t i = 0; i < reps && rc == BH_OK; ++i) rc = run();
        (void)hipEventRecord(e1, st);
        if (rc == BH_OK && hipEventSynchronize(e1) == hipSuccess) {
            (void)hipEventElapsedTime(&t[c], e0, e1);
            t[c] /= (float)reps;
        }
    }
    cleanup();
    if (rc != BH_OK) return rc;
    const int best = t[0] <= t[1] ? cand[0] : cand[1];
    {
        std::lock_guard<std::mutex> g(g_tune_mu);
        g_tune[{row_bucket(m), n, k}] = best;
    }
    *variant = best;
    if (ms) {
        ms[0] = t[0];
        ms[1] = t[1];
    }
    return BH_OK;
}

int bh_tune_set(uint32_t m, uint32_t n, uint32_t k, int variant) {
    if (m == 0 || m > (uint32_t)GEMV_MAX_ROWS ||
        (variant != BH_VARIANT_WORKGROUP_PER_OUTPUT && variant != BH_VARIANT_PACKED_INT8 && variant != 0))
        return fail(BH_ERR_INVALID, "bh_tune_set: m=%u variant=%d", m, variant);
    std::lock_guard<std::mutex> g(g_tune_mu);
    if (variant == 0) g_tune.erase({row_bucket(m), n, k});
    else g_tune[{row_bucket(m), n, k}] = variant;
    return BH_OK;
}

void bh_tune_clear(void) {
    std::lock_guard<std::mutex> g(g_tune_mu);
    g_tune.clear();
}

int bh_tune_get(uint32_t m, uint32_t n, uint32_t k) { return tuned_variant(m, n, k); }

// Text store (gpu_core::tune::FileTuneStore's role,
// crates/qwen3/src/serve.rs:1118-1121): the header names the format, the ABI
// version, the device the table was measured on and a fingerprint of the
// GEMV/GEMM kernel sources and flags this library was built from (BH_KERNEL_FP,
// set by the build), then "m n k variant" lines. A table measured on another
// device or another kernel build is refused: its crossovers do not carry over.
#ifndef BH_KERNEL_FP
#error "BH_KERNEL_FP (the kernel-source fingerprint) must be defined by the build"
#endif
static const char* TUNE_HEADER = "brain-hip-tune 2";

// The current device as one token: "<gcnArchName>|<marketing name>" with
// blanks replaced, or "nodevice" when no GPU is visible.
static std::string tune_device_tag() {
    int dev = 0;
    hipDeviceProp_t prop{};
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        return "nodevice";
    }
    std::string tag = std::string(prop.gcnArchName) + "|" + prop.name;
    for (char& ch : tag)
        if (ch == ' ' || ch == '\t' || ch == '\n') ch = '_';
    return tag;
}

static std::string tune_header_line() {
    char buf[512];
    snprintf(buf, sizeof buf, "%s abi %d device %s kernels %016llx", TUNE_HEADER, BH_ABI_VERSION,
             tune_device_tag().c_str(), (unsigned long long)BH_KERNEL_FP);
    return buf;
}

int bh_tune_save(const char* path) {
    if (!path) return fail(BH_ERR_INVALID, "bh_tune_save: null path");
    const std::string hdr = tune_header_line();
    FILE* f = fopen(path, "w");
    if (!f) return fail(BH_ERR_INVALID, "bh_tune_save: cannot write %s", path);
    std::lock_guard<std::mutex> g(g_tune_mu);
    fprintf(f, "%s\n", hdr.c_str());
    for (const auto& kv : g_tune)
        fprintf(f, "%u %u %u %d\n", std::get<0>(kv.first), std::get<1>(kv.first), std::get<2>(kv.first), kv.second);
    fclose(f);
    return BH_OK;
}

int bh_tune_load(const char* path) {
    if (!path) return fail(BH_ERR_INVALID, "bh_tune_load: null path");
    FILE* f = fopen(path, "r");
    if (!f) return fail(BH_ERR_INVALID, "bh_tune_load: cannot read %s", path);
    char line[512];
    const std::string want = tune_header_line();
    if (!fgets(line, sizeof line, f)) {
        fclose(f);
        return fail(BH_ERR_INVALID, "bh_tune_load: %s is empty", path);
    }
    std::string got(line);
    while (!got.empty() && (got.back() == '\n' || got.back() == '\r')) got.pop_back();
    if (got != want) {
        fclose(f);
        return fail(BH_ERR_INVALID, "bh_tune_load: %s was measured on another device or kernel build (\"%s\", this "
                    "process: \"%s\")", path, got.c_str(), want.c_str());
    }
    std::map<std::tuple<uint32_t, uint32_t, uint32_t>, int> t;
    unsigned m, n, k;
    int v;
    while (fgets(line, sizeof line, f)) {
        if (sscanf(line, "%u %u %u %d", &m, &n, &k, &v) != 4 || m == 0 || m > (unsigned)GEMV_MAX_ROWS ||
            (v != BH_VARIANT_WORKGROUP_PER_OUTPUT && v != BH_VARIANT_PACKED_INT8)) {
            fclose(f);
            return fail(BH_ERR_INVALID, "bh_tune_load: bad line in %s: %s", path, line);
        }
        t[{row_bucket(m), n, k}] = v;
    }
    fclose(f);
    std::lock_guard<std::mutex> g(g_tune_mu);
    for (const auto& kv : t) g_tune[kv.first] = kv.second;
    return (int)t.size();
}

// ---------------------------------------------------------------- host quantizer
// Host threads for row-parallel work: OMP_NUM_THREADS when set (the CPU share
// a job is given), else the hardware's thread count.
static unsigned host_threads() {
    unsigned hw = std::thread::hardware_concurrency();
    if (const char* e = getenv("OMP_NUM_THREADS")) {
        const int v = atoi(e);
        if (v > 0) return hw ? std::min<unsigned>((unsigned)v, hw) : (unsigned)v;
    }
    return hw ? hw : 1;
}

static void parallel_rows(uint64_t n, const std::function<void(uint64_t, uint64_t)>& fn) {
    const unsigned hw = host_threads();
    uint64_t nt = std::min<uint64_t>(hw, std::max<uint64_t>(1, n / 16));
    if (nt <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    uint64_t per = (n + nt - 1) / nt;
    for (uint64_t t = 0; t < nt; ++t) {
        uint64_t a = t * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back(fn, a, b);
    }
    for (auto& x : th) x.join();
}

int bh_quantize_weight(const float* w, uint64_t n, uint64_t k, uint32_t* packed, float* sw) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_quantize_weight: k=%llu is not a multiple of 4", (unsigned long long)k);
    if (n == 0) return BH_OK;
    if (!sw || (k > 0 && (!w || !packed))) return fail(BH_ERR_INVALID, "bh_quantize_weight: null buffer");
    const uint64_t kg = k / 4;
    parallel_rows(n, [&](uint64_t r0, uint64_t r1) {
        for (uint64_t r = r0; r < r1; ++r) {
            const float* row = w + r * k;
            float a = 0.0f;
            for (uint64_t c = 0; c < k; ++c) a = std::fmax(a, std::fabs(row[c]));
            const float s = std::fmax(a, 1e-8f) / 127.0f;
            sw[r] = s;
            const float inv = 1.0f / s;
            for (uint64_t g = 0; g < kg; ++g) {
                uint32_t word = 0;
                for (int b = 0; b < 4; ++b) {
                    float v = std::round(row[g * 4 + b] * inv);  // ties away, like f32::round
                    int32_t q = 0;
                    if (!std::isnan(v)) q = (int32_t)std::fmin(std::fmax(v, -127.0f), 127.0f);
                    word |= (uint32_t)(uint8_t)q << (8 * b);
                }
                packed[r * kg + g] = word;
            }
        }
    });
    return BH_OK;
}

// crates/model/src/int4.rs:46-67: sw = max(max|w|, 1e-8)/7, q = clamp(round_half_away(w*(1/sw)), +-7),
// nibble b of word g = column 8g+b, two's complement.
int bh_quantize_weight_q4(const float* w, uint64_t n, uint64_t k, uint32_t* packed, float* sw) {
    if (k % 8) return fail(BH_ERR_INVALID, "bh_quantize_weight_q4: k=%llu is not a multiple of 8", (unsigned long long)k);
    if (n && k && (!w || !packed || !sw)) return fail(BH_ERR_INVALID, "bh_quantize_weight_q4: null buffer");
    const uint64_t kg = k / 8;
    parallel_rows(n, [&](uint64_t r0, uint64_t r1) {
        for (uint64_t r = r0; r < r1; ++r) {
            const float* row = w + r * k;
            float mx = 0.0f;
            for (uint64_t c = 0; c < k; ++c) mx = std::max(mx, std::fabs(row[c]));
            const float s = std::max(mx, 1e-8f) / 7.0f;
            sw[r] = s;
            const float inv = 1.0f / s;
            for (uint64_t g = 0; g < kg; ++g) {
                uint32_t word = 0;
                for (int b = 0; b < 8; ++b) {
                    float q = std::round(row[g * 8 + b] * inv);
                    q = std::min(std::max(q, -7.0f), 7.0f);
                    const int qi = std::isnan(q) ? 0 : (int)q;
                    word |= ((uint32_t)(uint8_t)qi & 0xFu) << (4 * b);
                }
                packed[r * kg + g] = word;
            }
        }
    });
    return BH_OK;
}

int bh_dequantize_weight(const uint32_t* packed, const float* sw, uint64_t n, uint64_t k, float* w) {
    if (k % 4 != 0) return fail(BH_ERR_INVALID, "bh_dequantize_weight: k=%llu is not a multiple of 4", (unsigned long long)k);
    if (n == 0 || k == 0) return BH_OK;
    if (!packed || !sw || !w) return fail(BH_ERR_INVALID, "bh_dequantize_weight: null buffer");
    const uint64_t kg = k / 4;
    for (uint64_t r = 0; r < n; ++r)
        for (uint64_t g = 0; g < kg; ++g) {
            const uint32_t word = packed[r * kg + g];
            for (int b = 0; b < 4; ++b) w[r * k + g * 4 + b] = (float)(int8_t)(uint8_t)(word >> (8 * b)) * sw[r];
        }
    return BH_OK;
}

// ---------------------------------------------------------------- cost model
int bh_cost(const char* name, const uint32_t* params, uint32_t nparams, bh_cost_t* out) {
    if (!name || !out) return fail(BH_ERR_INVALID, "bh_cost: null argument");
    auto p = [&](uint32_t i) -> uint64_t { return i < nparams && params ? params[i] : 0; };
    if (!strcmp(name, "matmul_i8") || !strcmp(name, "matmul_i8_dyn") || !strcmp(name, "matmul_i8_gemv")) {
        if (nparams < 3 || !params) return fail(BH_ERR_INVALID, "bh_cost(%s): needs [m, kg, n]", name);
        const uint64_t m = p(0), kg = p(1), n = p(2);
        out->flops = 2 * m * n;                               // dequant epilogue
        out->int_ops = 8 * m * kg * n;                        // 2*M*N*K
        out->bytes = 4 * (m * kg + n * kg + m * n + m + n);   // cost.rs:272-275
        return BH_OK;
    }
    return fail(BH_ERR_UNSUPPORTED, "bh_cost: no formula for '%s'", name);
}

}  // extern "C"

// ================================================================ Backend mirror
namespace bh {

enum KernelId : int {
    K_UNKNOWN = 0,
    K_MAX_ABS_ROW,
    K_MAX_ABS_ROWS,
    K_QUANT_PACK,
    K_MATMUL_I8_DYN,
    K_MATMUL_I8_GEMV,
    K_MATMUL_I8,
    K_BIAS_ADD,
    K_ROOF_DP4A,
    K_MATMUL_Q4_DYN,
    K_MATMUL_Q4_GEMV,
    K_MOE_LINEAR_GATED_I8,
    K_PAGED_KV_APPEND_I8,
    K_PAGED_DECODE_SCORES_I8,
    K_PAGED_DECODE_APPLY_I8,
};

struct KernelSpec {
    const char* name;
    KernelId id;
    uint32_t nbufs;
    uint32_t nparams;
};

static const KernelSpec kSpecs[] = {
    {"max_abs_row", K_MAX_ABS_ROW, 2, 2},      {"max_abs_rows", K_MAX_ABS_ROWS, 2, 2},
    {"quant_pack", K_QUANT_PACK, 3, 2},        {"matmul_i8_dyn", K_MATMUL_I8_DYN, 5, 3},
    {"matmul_i8_gemv", K_MATMUL_I8_GEMV, 5, 3}, {"matmul_i8", K_MATMUL_I8, 3, 5},
    {"bias_add", K_BIAS_ADD, 2, 2},            {"roof_dp4a", K_ROOF_DP4A, 2, 4},
    {"matmul_q4_dyn", K_MATMUL_Q4_DYN, 5, 3},   {"matmul_q4_gemv", K_MATMUL_Q4_GEMV, 5, 3},
    {"moe_linear_gated_i8", K_MOE_LINEAR_GATED_I8, 6, 5},
    // crates/qwen3/src/serve.rs:1267-1270: [src, blocks, offsets, clip, pool, scales] /
    // [b, kv_stride, block_size, head_dim]; [q|probs, pool, block_tables, seq_lens, scales,
    // scores|ctx] / [b, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt (, scale)].
    {"paged_kv_append_i8_clipped_batched", K_PAGED_KV_APPEND_I8, 6, 4},
    {"paged_decode_scores_i8_batched", K_PAGED_DECODE_SCORES_I8, 6, 9},
    {"paged_decode_apply_i8_batched", K_PAGED_DECODE_APPLY_I8, 6, 8},
};

static const KernelSpec* spec_of(const char* name) {
    for (const auto& s : kSpecs)
        if (!strcmp(s.name, name)) return &s;
    return nullptr;
}

}  // namespace bh

struct bh_buffer {
    std::atomic<int> rc{1};
    void* ptr = nullptr;
    uint64_t words = 0;
    int device = 0;
};

struct bh_dispatch {
    std::atomic<int> rc{1};
    uint32_t kind = 0;
    std::vector<bh_buffer*> bufs;
    std::vector<uint64_t> off;   // word offsets
    std::vector<uint64_t> span;  // words bound from off (the slice length, or to the end)
    std::vector<uint32_t> params;
};

struct PendingTime {
    uint32_t kind;
    hipEvent_t a, b;
};

struct bh_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<std::string> names;
    std::vector<bh::KernelId> ids;
    bh_caps_t caps{};
    std::atomic<uint64_t> submits{0}, dispatches{0}, readbacks{0}, bind_groups{0}, uniform_allocs{0};
    std::mutex mu;  // guards timing state
    bool timing = false;
    std::vector<double> ms;
    std::vector<uint64_t> calls;
    std::vector<PendingTime> pending;
};

namespace bh {

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

static void collect_times(bh_backend* be) {
    std::lock_guard<std::mutex> g(be->mu);
    for (auto& p : be->pending) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, p.a, p.b) == hipSuccess) {
            be->ms[p.kind] += t;
            be->calls[p.kind] += 1;
        }
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    be->pending.clear();
}

// Words each binding of a dispatch touches, derived from its params.
static int binding_needs(KernelId id, const std::vector<uint32_t>& p, std::vector<uint64_t>& need, const char* name) {
    const uint64_t a = p.size() > 0 ? p[0] : 0, b = p.size() > 1 ? p[1] : 0, c = p.size() > 2 ? p[2] : 0;
    switch (id) {
        case K_MAX_ABS_ROW:
        case K_MAX_ABS_ROWS: need = {a * b, a}; return BH_OK;
        case K_QUANT_PACK:
            if (b % 4) return fail(BH_ERR_INVALID, "%s: k=%llu is not a multiple of 4", name, (unsigned long long)b);
            need = {a * b, a, a * b / 4};
            return BH_OK;
        case K_MATMUL_I8_GEMV:
            if (a > (uint64_t)GEMV_MAX_ROWS)
                return fail(BH_ERR_INVALID, "%s: m=%llu > %d", name, (unsigned long long)a, GEMV_MAX_ROWS);
            [[fallthrough]];
        case K_MATMUL_I8_DYN: need = {a * b, c * b, a, c, a * c}; return BH_OK;
        case K_MATMUL_I8: need = {a * b, c * b, a * c}; return BH_OK;
        case K_MATMUL_Q4_GEMV:
            if (a > (uint64_t)GEMV_MAX_ROWS)
                return fail(BH_ERR_INVALID, "%s: m=%llu > %d", name, (unsigned long long)a, GEMV_MAX_ROWS);
            [[fallthrough]];
        case K_MATMUL_Q4_DYN:  // params [m, k, n] with the RAW k (crates/model/src/dispatch.rs:132-178)
            if (b % 8) return fail(BH_ERR_INVALID, "%s: k=%llu is not a multiple of 8", name, (unsigned long long)b);
            need = {a * b / 4, c * b / 8, a, c, a * c};
            return BH_OK;
        case K_MOE_LINEAR_GATED_I8: {  // params [m, kg, n, n_experts, e_idx]
            const uint64_t ne = p.size() > 3 ? p[3] : 0, ei = p.size() > 4 ? p[4] : 0;
            if (ei >= ne) return fail(BH_ERR_INVALID, "%s: e_idx %llu >= n_experts %llu", name, (unsigned long long)ei, (unsigned long long)ne);
            need = {a * b, c * b, a, c, a * ne, a * c};
            return BH_OK;
        }
        case K_PAGED_KV_APPEND_I8: {  // [b, kv_stride, block_size, head_dim]
            const uint64_t hd = p.size() > 3 ? p[3] : 0;
            if (hd == 0 || b % hd) return fail(BH_ERR_INVALID, "%s: kv_stride %llu is not a multiple of head_dim %llu",
                                               name, (unsigned long long)b, (unsigned long long)hd);
            // the pool and scale slots the tables name are checked on the device
            need = {a * b, a, a, b / hd, 0, 0};
            return BH_OK;
        }
        case K_PAGED_DECODE_SCORES_I8:
        case K_PAGED_DECODE_APPLY_I8: {  // [b, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt]
            const uint64_t hd = p.size() > 3 ? p[3] : 0, cap = p.size() > 6 ? p[6] : 0, mbt = p.size() > 7 ? p[7] : 0;
            const uint64_t qn = a * b * hd, pn = a * b * cap;
            need = {id == K_PAGED_DECODE_SCORES_I8 ? qn : pn, 0, a * mbt, a, 0, id == K_PAGED_DECODE_SCORES_I8 ? pn : qn};
            return BH_OK;
        }
        case K_BIAS_ADD: need = {a * b, b}; return BH_OK;
        case K_ROOF_DP4A: need = {a, a}; return BH_OK;
        default: return fail(BH_ERR_UNSUPPORTED, "kernel '%s' is not provided by the hip backend", name);
    }
}

// Bindings whose extent depends on device-side tables (the paged KV pool and
// scales): the kernel checks each access against the bound slice, and the
// alias check takes the whole slice.
static bool device_checked(KernelId id, uint32_t i) {
    switch (id) {
        case K_PAGED_KV_APPEND_I8: return i == 4 || i == 5;
        case K_PAGED_DECODE_SCORES_I8:
        case K_PAGED_DECODE_APPLY_I8: return i == 1 || i == 4;
        default: return false;
    }
}

// Which bindings a kernel writes (for the output-alias check).
static bool is_output(KernelId id, uint32_t i) {
    switch (id) {
        case K_MAX_ABS_ROW:
        case K_MAX_ABS_ROWS: return i == 1;
        case K_QUANT_PACK: return i == 2;
        case K_MATMUL_I8_DYN:
        case K_MATMUL_I8_GEMV:
        case K_MATMUL_Q4_DYN:
        case K_MATMUL_Q4_GEMV: return i == 4;
        case K_MOE_LINEAR_GATED_I8: return i == 5;
        case K_PAGED_KV_APPEND_I8: return i == 4 || i == 5;
        case K_PAGED_DECODE_SCORES_I8:
        case K_PAGED_DECODE_APPLY_I8: return i == 5;
        case K_MATMUL_I8: return i == 2;
        case K_BIAS_ADD: return i == 0;
        case K_ROOF_DP4A: return i == 1;
        default: return false;
    }
}

static int record(bh_backend* be, uint32_t kind, bh_buffer* const* bufs, const uint64_t* offsets, uint32_t nbufs,
                  const uint32_t* params, uint32_t nparams, bh_dispatch** out) {
    if (!be || !out) return fail(BH_ERR_INVALID, "step: null backend/out");
    if (kind >= be->ids.size()) return fail(BH_ERR_INVALID, "step: kernel index %u out of range", kind);
    const char* name = be->names[kind].c_str();
    const KernelSpec* sp = spec_of(name);
    if (!sp) return fail(BH_ERR_UNSUPPORTED, "kernel '%s' is not provided by the hip backend", name);
    if (nbufs != sp->nbufs) return fail(BH_ERR_INVALID, "%s: %u bindings, expected %u", name, nbufs, sp->nbufs);
    if (nparams < sp->nparams || (nparams && !params))
        return fail(BH_ERR_INVALID, "%s: %u params, expected %u", name, nparams, sp->nparams);
    std::vector<uint32_t> pv(params, params + nparams);
    std::vector<uint64_t> need;
    int rc = binding_needs(sp->id, pv, need, name);
    if (rc) return rc;
    std::vector<uint64_t> lo(nbufs), hi(nbufs), spans(nbufs);
    for (uint32_t i = 0; i < nbufs; ++i) {
        if (!bufs[i]) return fail(BH_ERR_INVALID, "%s: binding %u is null", name, i);
        const uint64_t off = offsets ? offsets[2 * i] : 0;
        const uint64_t len = offsets ? offsets[2 * i + 1] : 0;
        const uint64_t avail = bufs[i]->words;
        if (off > avail) return fail(BH_ERR_INVALID, "%s: binding %u offset %llu past %llu words", name, i,
                                     (unsigned long long)off, (unsigned long long)avail);
        const uint64_t span = len ? len : avail - off;
        if (len && off + len > avail)
            return fail(BH_ERR_INVALID, "%s: binding %u slice [%llu,+%llu) past %llu words", name, i,
                        (unsigned long long)off, (unsigned long long)len, (unsigned long long)avail);
        if (need[i] > span)
            return fail(BH_ERR_INVALID, "%s: binding %u needs %llu words, slice has %llu", name, i,
                        (unsigned long long)need[i], (unsigned long long)span);
        lo[i] = off;
        hi[i] = off + (device_checked(sp->id, i) ? span : need[i]);
        spans[i] = span;
    }
    // No output may alias another binding's range (crates/gpu-core/src/lib.rs:708).
    for (uint32_t i = 0; i < nbufs; ++i) {
        if (!is_output(sp->id, i) || hi[i] == lo[i]) continue;
        for (uint32_t j = 0; j < nbufs; ++j) {
            if (j == i || bufs[j] != bufs[i] || hi[j] == lo[j]) continue;
            if (lo[i] < hi[j] && lo[j] < hi[i])
                return fail(BH_ERR_INVALID, "%s: output binding %u overlaps binding %u", name, i, j);
        }
    }
    bh_dispatch* s = new bh_dispatch;
    s->kind = kind;
    s->params = pv;
    for (uint32_t i = 0; i < nbufs; ++i) {
        bh_buffer_retain(bufs[i]);
        s->bufs.push_back(bufs[i]);
        s->off.push_back(lo[i]);
        s->span.push_back(spans[i]);
    }
    be->uniform_allocs++;
    be->bind_groups++;
    *out = s;
    return BH_OK;
}

static inline void* wptr(const bh_dispatch* s, int i) {
    return static_cast<uint8_t*>(s->bufs[i]->ptr) + s->off[i] * 4;
}

static int launch_step(bh_backend* be, const bh_dispatch* s) {
    const KernelId id = be->ids[s->kind];
    const auto& p = s->params;
    hipStream_t st = be->stream;
    switch (id) {
        case K_MAX_ABS_ROW:
        case K_MAX_ABS_ROWS:
            return bh_max_abs_rows(st, (const float*)wptr(s, 0), p[0], p[1], (float*)wptr(s, 1));
        case K_QUANT_PACK:
            return bh_quant_pack(st, (const float*)wptr(s, 0), (const float*)wptr(s, 1), p[0], p[1],
                                 (uint32_t*)wptr(s, 2));
        case K_MATMUL_I8_DYN:
            return bh_matmul_i8_dyn(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                    (const float*)wptr(s, 2), (const float*)wptr(s, 3), nullptr, wptr(s, 4), OUT_F32,
                                    p[0], p[1], p[2]);
        case K_MATMUL_I8_GEMV:
            return bh_matmul_i8_gemv(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                     (const float*)wptr(s, 2), (const float*)wptr(s, 3), nullptr, wptr(s, 4), OUT_F32,
                                     p[0], p[1], p[2]);
        case K_MOE_LINEAR_GATED_I8:
            return bh_moe_linear_gated_i8(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                          (const float*)wptr(s, 2), (const float*)wptr(s, 3), (const float*)wptr(s, 4),
                                          p[3], p[4], (float*)wptr(s, 5), p[0], p[1], p[2]);
        case K_MATMUL_Q4_DYN:
            return bh_matmul_q4_dyn(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                    (const float*)wptr(s, 2), (const float*)wptr(s, 3), nullptr, wptr(s, 4), OUT_F32,
                                    p[0], p[1], p[2]);
        case K_MATMUL_Q4_GEMV:
            return bh_matmul_q4_gemv(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                     (const float*)wptr(s, 2), (const float*)wptr(s, 3), nullptr, wptr(s, 4), OUT_F32,
                                     p[0], p[1], p[2]);
        case K_MATMUL_I8: {
            float sx, sw;
            memcpy(&sx, &p[3], 4);
            memcpy(&sw, &p[4], 4);
            return bh_matmul_i8_static(st, (const uint32_t*)wptr(s, 0), (const uint32_t*)wptr(s, 1), sx, sw,
                                       (float*)wptr(s, 2), p[0], p[1], p[2]);
        }
        case K_PAGED_KV_APPEND_I8:
            return bh_paged_kv_append_i8(st, (const float*)wptr(s, 0), (const uint32_t*)wptr(s, 1),
                                         (const uint32_t*)wptr(s, 2), (const float*)wptr(s, 3), (uint32_t*)wptr(s, 4),
                                         s->span[4], (float*)wptr(s, 5), s->span[5], p[0], p[1], p[2], p[3]);
        case K_PAGED_DECODE_SCORES_I8: {
            float sc;
            memcpy(&sc, &p[8], 4);
            return bh_paged_decode_scores_i8(st, (const float*)wptr(s, 0), (const uint32_t*)wptr(s, 1), s->span[1],
                                             (const uint32_t*)wptr(s, 2), (const uint32_t*)wptr(s, 3),
                                             (const float*)wptr(s, 4), s->span[4], (float*)wptr(s, 5), p[0], p[1],
                                             p[2], p[3], p[4], p[5], p[6], p[7], sc);
        }
        case K_PAGED_DECODE_APPLY_I8:
            return bh_paged_decode_apply_i8(st, (const float*)wptr(s, 0), (const uint32_t*)wptr(s, 1), s->span[1],
                                            (const uint32_t*)wptr(s, 2), (const uint32_t*)wptr(s, 3),
                                            (const float*)wptr(s, 4), s->span[4], (float*)wptr(s, 5), p[0], p[1], p[2],
                                            p[3], p[4], p[5], p[6], p[7]);
        case K_BIAS_ADD: {
            const uint64_t total = (uint64_t)p[0] * p[1];
            if (total == 0) return BH_OK;
            const uint64_t blocks = std::min<uint64_t>((total + 255) / 256, 65536);
            bias_add_kernel<<<(unsigned)blocks, 256, 0, st>>>((float*)wptr(s, 0), (const float*)wptr(s, 1), total, p[1]);
            return hip_status(hipGetLastError(), "bias_add launch");
        }
        case K_ROOF_DP4A: {
            if (p[0] == 0) return BH_OK;
            roof_dp4a_kernel<<<(p[0] + 63) / 64, 64, 0, st>>>((const float*)wptr(s, 0), (float*)wptr(s, 1), p[0], p[1],
                                                          p[2], p[3]);
            return hip_status(hipGetLastError(), "roof_dp4a launch");
        }
        default: return fail(BH_ERR_UNSUPPORTED, "kernel '%s' is not provided by the hip backend", be->names[s->kind].c_str());
    }
}

}  // namespace bh

extern "C" {

int bh_backend_create(const char* const* names, const char* const* srcs, uint32_t n_kernels, int device,
                      uint32_t flags, bh_backend** out) {
    (void)srcs;
    if (!out) return fail(BH_ERR_INVALID, "bh_backend_create: null out");
    *out = nullptr;
    if (n_kernels && !names) return fail(BH_ERR_INVALID, "bh_backend_create: null names");
    std::vector<bh::KernelId> ids;
    for (uint32_t i = 0; i < n_kernels; ++i) {
        if (!names[i]) return fail(BH_ERR_INVALID, "bh_backend_create: kernel %u has no name", i);
        const bh::KernelSpec* sp = bh::spec_of(names[i]);
        if (!sp && !(flags & BH_CREATE_LENIENT))
            return fail(BH_ERR_UNSUPPORTED, "bh_backend_create: kernel '%s' is not provided by the hip backend", names[i]);
        ids.push_back(sp ? sp->id : bh::K_UNKNOWN);
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(BH_ERR_HIP, "bh_backend_create: no HIP device");
    if (device < 0 || device >= ndev) return fail(BH_ERR_INVALID, "bh_backend_create: device %d of %d", device, ndev);
    bh::DeviceGuard dg(device);
    hipDeviceProp_t prop;
    int rc = hip_status(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (rc) return rc;
    auto* be = new bh_backend;
    be->device = device;
    rc = hip_status(hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc) {
        delete be;
        return rc;
    }
    for (uint32_t i = 0; i < n_kernels; ++i) be->names.emplace_back(names[i]);
    be->ids = ids;
    be->ms.assign(n_kernels, 0.0);
    be->calls.assign(n_kernels, 0);
    bh_caps_t& c = be->caps;
    c.compute_units = (uint32_t)prop.multiProcessorCount;
    c.max_workgroup_size = (uint32_t)prop.maxThreadsPerBlock;
    c.workgroup_mem_bytes = (uint32_t)prop.sharedMemPerBlock;
    c.subgroup_size = (uint32_t)prop.warpSize;
    c.unified_memory = 0;
    c.workgroup_reductions = 1;
    c.numeric_f32 = 1;
    c.numeric_int8_dot = 1;
    c.numeric_f16 = 1;
    c.numeric_bf16 = 1;
    c.numeric_f16_storage = 1;
    c.numeric_bf16_storage = 1;
    c.numeric_coop_matrix = 1;
    c.max_buffer_bytes = (uint64_t)prop.totalGlobalMem;
    c.max_storage_binding_bytes = (uint64_t)prop.totalGlobalMem;
    snprintf(c.device_name, sizeof c.device_name, "%s", prop.gcnArchName);
    const char* prof = getenv("BRAIN_PROFILE");
    be->timing = prof && strcmp(prof, "0") != 0;
    *out = be;
    return BH_OK;
}

void bh_backend_destroy(bh_backend* be) {
    if (!be) return;
    bh::DeviceGuard dg(be->device);
    (void)hipStreamSynchronize(be->stream);
    bh::collect_times(be);
    (void)hipStreamDestroy(be->stream);
    delete be;
}

const char* bh_backend_kind(const bh_backend* be) { return be ? "hip" : nullptr; }

int bh_kernel_index(const bh_backend* be, const char* name) {
    if (!be || !name) return -1;
    for (size_t i = 0; i < be->names.size(); ++i)
        if (be->names[i] == name) return (int)i;
    return -1;
}

void* bh_backend_stream(const bh_backend* be) { return be ? (void*)be->stream : nullptr; }

int bh_caps(const bh_backend* be, bh_caps_t* caps) {
    if (!be || !caps) return fail(BH_ERR_INVALID, "bh_caps: null argument");
    *caps = be->caps;
    return BH_OK;
}

int bh_storage(bh_backend* be, uint64_t n_words, bh_buffer** out) {
    if (!be || !out) return fail(BH_ERR_INVALID, "bh_storage: null argument");
    *out = nullptr;
    bh::DeviceGuard dg(be->device);
    void* p = nullptr;
    const uint64_t bytes = std::max<uint64_t>(n_words, 1) * 4;
    if (hipMalloc(&p, bytes) != hipSuccess)
        return fail(BH_ERR_NOMEM, "bh_storage: hipMalloc(%llu) failed", (unsigned long long)bytes);
    // Zero-fill on the backend stream, then wait: the buffer is ready on return.
    const uint64_t blocks = std::min<uint64_t>((n_words + 255) / 256 + 1, 65536);
    bh::fill_zero_kernel<<<(unsigned)blocks, 256, 0, be->stream>>>((uint32_t*)p, std::max<uint64_t>(n_words, 1));
    int rc = hip_status(hipStreamSynchronize(be->stream), "bh_storage zero-fill");
    if (rc) {
        (void)hipFree(p);
        return rc;
    }
    auto* b = new bh_buffer;
    b->ptr = p;
    b->words = n_words;
    b->device = be->device;
    *out = b;
    return BH_OK;
}

int bh_storage_init(bh_backend* be, const char* label, const float* data, uint64_t n_words, bh_buffer** out) {
    (void)label;
    int rc = bh_storage(be, n_words, out);
    if (rc) return rc;
    if (n_words && data) {
        rc = bh_write(be, *out, reinterpret_cast<const uint32_t*>(data), n_words);
        if (rc) {
            bh_buffer_release(*out);
            *out = nullptr;
        }
    }
    return rc;
}

bh_buffer* bh_buffer_retain(bh_buffer* b) {
    if (b) b->rc.fetch_add(1, std::memory_order_relaxed);
    return b;
}

void bh_buffer_release(bh_buffer* b) {
    if (!b) return;
    if (b->rc.fetch_sub(1, std::memory_order_acq_rel) == 1) {
        bh::DeviceGuard dg(b->device);
        (void)hipFree(b->ptr);  // hipFree waits for outstanding work on the allocation
        delete b;
    }
}

uint64_t bh_buffer_words(const bh_buffer* b) { return b ? b->words : 0; }
void* bh_buffer_device_ptr(const bh_buffer* b) { return b ? b->ptr : nullptr; }

int bh_write_at(bh_backend* be, bh_buffer* buf, uint64_t offset_words, const uint32_t* data, uint64_t n_words) {
    if (!be || !buf || (n_words && !data)) return fail(BH_ERR_INVALID, "bh_write_at: null argument");
    if (offset_words > buf->words || n_words > buf->words - offset_words)
        return fail(BH_ERR_INVALID, "bh_write_at: [%llu,+%llu) past %llu words", (unsigned long long)offset_words,
                    (unsigned long long)n_words, (unsigned long long)buf->words);
    if (!n_words) return BH_OK;
    bh::DeviceGuard dg(be->device);
    int rc = hip_status(hipMemcpyAsync(static_cast<uint8_t*>(buf->ptr) + offset_words * 4, data, n_words * 4,
                                       hipMemcpyHostToDevice, be->stream),
                        "bh_write");
    if (rc) return rc;
    return hip_status(hipStreamSynchronize(be->stream), "bh_write sync");
}

int bh_write(bh_backend* be, bh_buffer* buf, const uint32_t* data, uint64_t n_words) {
    return bh_write_at(be, buf, 0, data, n_words);
}

int bh_read(bh_backend* be, const bh_buffer* buf, void* dst, uint64_t n_words) {
    if (!be || !buf || (n_words && !dst)) return fail(BH_ERR_INVALID, "bh_read: null argument");
    if (n_words > buf->words)
        return fail(BH_ERR_INVALID, "bh_read: %llu words of a %llu-word buffer", (unsigned long long)n_words,
                    (unsigned long long)buf->words);
    bh::DeviceGuard dg(be->device);
    be->readbacks++;
    if (n_words) {
        int rc = hip_status(hipMemcpyAsync(dst, buf->ptr, n_words * 4, hipMemcpyDeviceToHost, be->stream), "bh_read");
        if (rc) return rc;
    }
    int rc = hip_status(hipStreamSynchronize(be->stream), "bh_read sync");
    if (!rc) bh::collect_times(be);
    return rc;
}

int bh_step(bh_backend* be, uint32_t kind, bh_buffer* const* bufs, uint32_t nbufs, const uint32_t* params,
            uint32_t nparams, uint32_t threads, bh_dispatch** out) {
    (void)threads;
    return bh::record(be, kind, bufs, nullptr, nbufs, params, nparams, out);
}

int bh_step_sliced(bh_backend* be, uint32_t kind, bh_buffer* const* bufs, const uint64_t* offsets, uint32_t nbufs,
                   const uint32_t* params, uint32_t nparams, uint32_t threads, bh_dispatch** out) {
    (void)threads;
    return bh::record(be, kind, bufs, offsets, nbufs, params, nparams, out);
}

bh_dispatch* bh_step_retain(bh_dispatch* s) {
    if (s) s->rc.fetch_add(1, std::memory_order_relaxed);
    return s;
}

void bh_step_release(bh_dispatch* s) {
    if (!s) return;
    if (s->rc.fetch_sub(1, std::memory_order_acq_rel) == 1) {
        for (auto* b : s->bufs) bh_buffer_release(b);
        delete s;
    }
}

int bh_submit(bh_backend* be, bh_buffer* const* clears, uint32_t nclears, bh_dispatch* const* steps, uint32_t nsteps) {
    if (!be || (nclears && !clears) || (nsteps && !steps)) return fail(BH_ERR_INVALID, "bh_submit: null argument");
    bh::DeviceGuard dg(be->device);
    be->submits++;
    for (uint32_t i = 0; i < nclears; ++i) {
        bh_buffer* c = clears[i];
        if (!c) return fail(BH_ERR_INVALID, "bh_submit: clear %u is null", i);
        if (!c->words) continue;
        const uint64_t blocks = std::min<uint64_t>((c->words + 255) / 256, 65536);
        bh::fill_zero_kernel<<<(unsigned)blocks, 256, 0, be->stream>>>((uint32_t*)c->ptr, c->words);
        int rc = hip_status(hipGetLastError(), "bh_submit clear");
        if (rc) return rc;
    }
    for (uint32_t i = 0; i < nsteps; ++i) {
        if (!steps[i]) return fail(BH_ERR_INVALID, "bh_submit: step %u is null", i);
        bool timed;
        {
            std::lock_guard<std::mutex> g(be->mu);
            timed = be->timing;
        }
        PendingTime pt{steps[i]->kind, nullptr, nullptr};
        if (timed) {
            (void)hipEventCreate(&pt.a);
            (void)hipEventCreate(&pt.b);
            (void)hipEventRecord(pt.a, be->stream);
        }
        int rc = bh::launch_step(be, steps[i]);
        if (timed) {
            (void)hipEventRecord(pt.b, be->stream);
            std::lock_guard<std::mutex> g(be->mu);
            be->pending.push_back(pt);
        }
        if (rc) return rc;
        be->dispatches++;
    }
    return BH_OK;
}

int bh_flush(bh_backend* be) {
    if (!be) return fail(BH_ERR_INVALID, "bh_flush: null backend");
    return BH_OK;  // work is enqueued at submit; nothing is held back
}

int bh_poll_wait(bh_backend* be) {
    if (!be) return fail(BH_ERR_INVALID, "bh_poll_wait: null backend");
    bh::DeviceGuard dg(be->device);
    int rc = hip_status(hipStreamSynchronize(be->stream), "bh_poll_wait");
    if (!rc) bh::collect_times(be);
    return rc;
}

int bh_poll_wait_timeout(bh_backend* be, uint32_t timeout_ms) {
    if (!be) return fail(BH_ERR_INVALID, "bh_poll_wait_timeout: null backend");
    bh::DeviceGuard dg(be->device);
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        hipError_t e = hipStreamQuery(be->stream);
        if (e == hipSuccess) {
            bh::collect_times(be);
            return BH_OK;
        }
        if (e != hipErrorNotReady) return hip_status(e, "bh_poll_wait_timeout");
        if (std::chrono::steady_clock::now() - t0 >= std::chrono::milliseconds(timeout_ms))
            return fail(BH_ERR_TIMEOUT, "bh_poll_wait_timeout: not idle after %u ms", timeout_ms);
        std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
}

int bh_set_kernel_timing(bh_backend* be, int on) {
    if (!be) return 0;
    std::lock_guard<std::mutex> g(be->mu);
    be->timing = on != 0;
    return be->timing ? 1 : 0;
}

int bh_kernel_times(bh_backend* be, bh_kernel_time_t* out, uint32_t cap) {
    if (!be) return fail(BH_ERR_INVALID, "bh_kernel_times: null backend");
    std::lock_guard<std::mutex> g(be->mu);
    int cnt = 0;
    for (size_t i = 0; i < be->names.size(); ++i) {
        if (!be->calls[i]) continue;
        if (out && (uint32_t)cnt < cap) {
            snprintf(out[cnt].name, sizeof out[cnt].name, "%s", be->names[i].c_str());
            out[cnt].ms = be->ms[i];
            out[cnt].calls = be->calls[i];
        }
        ++cnt;
    }
    return cnt;
}

void bh_reset_kernel_times(bh_backend* be) {
    if (!be) return;
    std::lock_guard<std::mutex> g(be->mu);
    std::fill(be->ms.begin(), be->ms.end(), 0.0);
    std::fill(be->calls.begin(), be->calls.end(), 0);
}

int bh_stats(const bh_backend* be, bh_stats_t* st) {
    if (!be || !st) return fail(BH_ERR_INVALID, "bh_stats: null argument");
    st->submits = be->submits.load();
    st->dispatches = be->dispatches.load();
    st->readbacks = be->readbacks.load();
    st->bind_groups = be->bind_groups.load();
    st->uniform_allocs = be->uniform_allocs.load();
    return BH_OK;
}

int bh_quant_rows_steps(bh_backend* be, const uint32_t kernels[2], bh_buffer* x, bh_buffer* sx, bh_buffer* xq,
                        uint32_t r0, uint32_t r1, uint32_t k, bh_dispatch* out[2]) {
    if (!kernels || !out) return fail(BH_ERR_INVALID, "bh_quant_rows_steps: null argument");
    if (k % 4) return fail(BH_ERR_INVALID, "bh_quant_rows_steps: int8 K must be a multiple of 4 (got %u)", k);
    if (r0 % 64)
        return fail(BH_ERR_INVALID,
                    "bh_quant_rows_steps: row base %u breaks the 64-float alignment of the per-token scale buffer", r0);
    if (r1 < r0) return fail(BH_ERR_INVALID, "bh_quant_rows_steps: r1 %u < r0 %u", r1, r0);
    const uint32_t m = r1 - r0;
    const uint64_t xo[4] = {(uint64_t)r0 * k, (uint64_t)m * k, r0, m};
    const uint64_t qo[6] = {(uint64_t)r0 * k, (uint64_t)m * k, r0, m, (uint64_t)r0 * (k / 4), (uint64_t)m * (k / 4)};
    const uint32_t params[2] = {m, k};
    bh_buffer* b0[2] = {x, sx};
    bh_buffer* b1[3] = {x, sx, xq};
    int rc = bh_step_sliced(be, kernels[0], b0, xo, 2, params, 2, m, &out[0]);
    if (rc) return rc;
    rc = bh_step_sliced(be, kernels[1], b1, qo, 3, params, 2, m * (k / 4), &out[1]);
    if (rc) {
        bh_step_release(out[0]);
        out[0] = nullptr;
    }
    return rc;
}

int bh_mm8_rows_off(bh_backend* be, uint32_t kind, bh_buffer* xq, bh_buffer* wq, bh_buffer* sx, bh_buffer* sw,
                    bh_buffer* o, uint32_t xr0, uint64_t ooff, uint32_t m, uint32_t k, uint32_t n, bh_dispatch** out) {
    if (k % 4) return fail(BH_ERR_INVALID, "bh_mm8_rows_off: int8 K must be a multiple of 4 (got %u)", k);
    const uint64_t kg = k / 4;
    const uint64_t offs[10] = {(uint64_t)xr0 * kg, (uint64_t)m * kg, 0, 0, xr0, m, 0, 0, ooff, (uint64_t)m * n};
    bh_buffer* bufs[5] = {xq, wq, sx, sw, o};
    const uint32_t params[3] = {m, (uint32_t)kg, n};
    return bh_step_sliced(be, kind, bufs, offs, 5, params, 3, 0, out);
}

}  // extern "C"
