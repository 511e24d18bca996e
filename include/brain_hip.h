/* brain_hip.h — C ABI of the MI355X (gfx950) int8 W8A8 matmul backend.
 *
 * Drop-in boundary for the int8 linear path of swedishembedded/brain. The
 * reference's plugin seam is the generic kernel-dispatch trait
 * `backend_api::Backend` (crates/backend-api/src/lib.rs:696-908): kernels are
 * named, dispatched as `step(kind, bufs, params, threads)` and run in order by
 * `submit`. This header exports
 *   (1) that trait as plain C functions over opaque handles (section B), so a
 *       thin Rust `backend-hip` crate can `impl Backend` by forwarding, and
 *   (2) the same four kernels as typed, stream-ordered calls on caller-owned
 *       device pointers (section A) for callers that manage memory themselves.
 *   (3) the host-side int8 helpers the model layer calls (section C).
 *
 * Conventions
 *  - Every function returns an int status: BH_OK (0) or a negative BH_ERR_*;
 *    bh_last_error() gives a thread-local message. Nothing throws across the ABI.
 *  - Packed int8 tensors are `uint32_t` words holding 4 int8 values,
 *    little-endian along K (byte b of word g = element 4g+b). K must be a
 *    multiple of 4; `kg` = K/4 is the packed word count, as in the reference's
 *    `[m, kg, n]` matmul params.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream). Calls in
 *    section A only enqueue work; they never synchronise.
 *  - Arithmetic (bit-exact with the reference on the same inputs):
 *      sx[m]    = max(max_k |x[m,k]|, 1e-8) / 127
 *      xq[m,k]  = clamp(round_half_even(x[m,k] * (1/sx[m])), -127, 127)
 *      acc[m,n] = sum_k xq[m,k] * wq[n,k]                  (exact i32)
 *      out[m,n] = (f32(acc) * sx[m]) * sw[n] [+ bias[n]]   (no FMA; bf16 = RNE)
 */
#ifndef BRAIN_HIP_H
#define BRAIN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BH_ABI_VERSION 2

enum {
    BH_OK = 0,
    BH_ERR_INVALID = -1,     /* bad argument, shape or binding */
    BH_ERR_HIP = -2,         /* HIP runtime error */
    BH_ERR_UNSUPPORTED = -3, /* kernel name / feature not provided */
    BH_ERR_NOMEM = -4,       /* device allocation failed */
    BH_ERR_TIMEOUT = -5      /* bounded wait expired */
};

/* Output element type of the dequant epilogue. */
/* BH_OUT_I32 stores the raw i32 accumulators (sx, sw, bias unused) — the
 * hook for checking the integer sums bit for bit. */
enum { BH_OUT_F32 = 0, BH_OUT_BF16 = 1, BH_OUT_I32 = 2 };

/* Thread-local description of the last failing call on this thread. */
const char* bh_last_error(void);
int bh_abi_version(void);

/* ======================================================================
 * A. Typed, stream-ordered kernels on caller-owned device memory.
 * ====================================================================== */

/* Per-token scale. Replaces the `max_abs_row` / `max_abs_rows` dispatch,
 * bindings [x, sx], params [m, k] (crates/kernels/wgsl/max_abs_row.wgsl:27-34,
 * max_abs_rows.wgsl:60-84). x: [m,k] f32, sx: [m] f32. */
int bh_max_abs_rows(void* stream, const float* x, uint32_t m, uint32_t k, float* sx);

/* Quantize + pack. Replaces the `quant_pack` dispatch, bindings [x, sx, xq],
 * params [m, k] (crates/kernels/wgsl/quant_pack.wgsl:26-45). k % 4 == 0. */
int bh_quant_pack(void* stream, const float* x, const float* sx, uint32_t m, uint32_t k, uint32_t* xq);

/* max_abs_rows + quant_pack in one launch; bit-identical to the pair.
 * Replaces the two steps of `model::int8::quant_rows_steps`
 * (crates/model/src/int8.rs:221-235). */
int bh_quantize_rows(void* stream, const float* x, uint32_t m, uint32_t k, float* sx, uint32_t* xq);

/* bf16 activations (raw bf16 bits [m,k]): quantize_rows of the exactly
 * widened f32 values. The DiT-style stacks keep activations in bf16 between
 * linears; the reference's quant_pack reads f32 (quant_pack.wgsl:26-45), and
 * bf16 -> f32 is exact, so the bytes and scales equal bh_quantize_rows on
 * f32(x). */
int bh_quantize_rows_bf16(void* stream, const uint16_t* x, uint32_t m, uint32_t k, float* sx, uint32_t* xq);

/* W8A8 matmul: a tuned variant if bh_tune_i8 / bh_tune_set recorded one for
 * the shape, else the GEMV for m <= 32 (the MI355X crossover), the MFMA tile
 * otherwise. Replaces the `matmul_i8_dyn` / `matmul_i8_gemv` dispatches,
 * bindings [xq, wq, sx, sw, out], params [m, kg, n]
 * (crates/kernels/wgsl/matmul_i8_dyn.wgsl:50-280, matmul_i8_gemv.wgsl:39-76)
 * and the selection in crates/model/src/ops.rs:667-730.
 * xq [m,kg] u32, wq [n,kg] u32, sx [m] f32, sw [n] f32, bias [n] f32 or NULL
 * (the reference adds bias with a separate `bias_add` dispatch; fusing it is
 * bit-identical because the add happens after the same two products),
 * out [m,n] f32 (BH_OUT_F32) or bf16 bits (BH_OUT_BF16). */
int bh_matmul_i8(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                 const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n);

/* Forced decode variant (crates/kernels/wgsl/matmul_i8_gemv.wgsl:39-76); m <= 32. */
int bh_matmul_i8_gemv(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                      const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n);

/* Forced tiled variant (crates/kernels/wgsl/matmul_i8_dyn.wgsl:50-280); any m. */
int bh_matmul_i8_dyn(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                     const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg, uint32_t n);

/* bh_matmul_i8_dyn with bf16 output, then bh_quantize_rows_bf16 of that
 * output for the next linear (sx_out [m], xq_out [m, n/4]), in one call.
 * The reference runs the two as consecutive steps of a block's int8 linears
 * (crates/s3dit/src/block.rs:727-790: matmul_i8_dyn, then the next linear's
 * per-token activation quant); the results are the same bits as those two
 * calls. n % 4 == 0. When the GEMM's 256x256 grid leaves most of the GPU
 * idle, K is split and one pass over the partial sums applies the epilogue,
 * stores `out` and quantizes it. sx_out may be sx and xq_out may overlap xq
 * (they are written after the GEMM has read its inputs). Uses the stream's
 * split-K workspace like bh_matmul_i8_dyn (bh_reserve_workspace sizes it). */
int bh_matmul_i8_dyn_quant(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                           const float* bias, uint16_t* out, uint32_t m, uint32_t kg, uint32_t n, float* sx_out,
                           uint32_t* xq_out);

/* bh_matmul_i8_dyn that allocates nothing. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * kernels and results as bh_matmul_i8_dyn, in one launch without the column
 * split that bh_matmul_i8_dyn takes for some wide shapes; when the shape
 * splits K, the i32 partial slabs go to a fixed 32 MiB device array that the
 * library holds on each GPU until the process ends (instead of the per-stream
 * workspace bh_matmul_i8_dyn grows). A shape whose slabs exceed 32 MiB
 * returns BH_ERR_INVALID. Every call on one GPU shares that array: calls
 * that overlap on one GPU (two streams) would race, so a call whose shape
 * uses the array returns BH_ERR_INVALID while the last such call, made on
 * another stream, has not finished (an event recorded after it); calls on
 * one stream are ordered by the stream. Calls recorded into a HIP graph are
 * not checked: launching such graphs concurrently races. The slabs are
 * fully overwritten before they are read, so nothing needs clearing between
 * calls. */
int bh_matmul_i8_dyn_noalloc(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx,
                             const float* sw, const float* bias, void* out, int out_dtype, uint32_t m, uint32_t kg,
                             uint32_t n);

/* Pre-size the library-held split-K workspace of `stream` for a
 * bh_matmul_i8_dyn call of this shape (a no-op for shapes that do not split
 * K). The workspace is allocated per (device, stream) on first need and
 * grows on demand; a growth cannot happen while the stream is being captured
 * into a HIP graph, so callers that capture reserve for their largest shape
 * first. */
int bh_reserve_workspace(void* stream, uint32_t m, uint32_t kg, uint32_t n);

/* Static per-tensor scales: out = f32(acc) * (sx*sw). Replaces `matmul_i8`,
 * bindings [x, w, out], params [m, kg, n, sx_bits, sw_bits]
 * (crates/kernels/wgsl/matmul_i8.wgsl:49-262). */
int bh_matmul_i8_static(void* stream, const uint32_t* xq, const uint32_t* wq, float sx, float sw, float* out,
                        uint32_t m, uint32_t kg, uint32_t n);

/* One whole int8 linear: quantize x [m,k] f32 into the caller's scratch
 * (sx [m], xq [m,k/4]) and run bh_matmul_i8. The sequence
 * `Ops::act` + `Ops::matmul` (crates/model/src/ops.rs:574-580, 667-730). */
int bh_linear_i8(void* stream, const float* x, const uint32_t* wq, const float* sw, const float* bias,
                 float* sx_scratch, uint32_t* xq_scratch, void* out, int out_dtype, uint32_t m, uint32_t k,
                 uint32_t n);

/* Per-output-channel weight quantization on the device; bit-identical to
 * bh_quantize_weight (crates/model/src/int8.rs:33-59). w [n,k] f32 ->
 * packed [n,k/4] u32, sw [n] f32. */
int bh_quantize_weight_device(void* stream, const float* w, uint32_t n, uint32_t k, uint32_t* packed, float* sw);

/* W4A8 (crates/model/src/int4.rs, crates/kernels/wgsl/matmul_q4_{gemv,dyn}.wgsl):
 * int4 weights wq4 [n, k/8] u32 (8 nibbles per word, nibble b = K index 8g+b,
 * two's complement, per-row scale), the int8 activation xq [m, k/4] of the
 * int8 tier, the same (f32(acc)*sx)*sw epilogue. k is the RAW K, a multiple
 * of 8 (the q4 family's param contract, crates/model/src/dispatch.rs:132-178).
 * Step names "matmul_q4_gemv" / "matmul_q4_dyn" take params [m, k, n]. */
int bh_matmul_q4_gemv(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                      const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n);
int bh_matmul_q4_dyn(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                     const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n);
int bh_matmul_q4(void* stream, const uint32_t* xq, const uint32_t* wq4, const float* sx, const float* sw,
                 const float* bias, void* out, int out_dtype, uint32_t m, uint32_t k, uint32_t n);

/* Sparse-MoE expert linear, int8 (crates/kernels/wgsl/moe_linear_gated_i8.wgsl):
 * out [m,n] f32 = (f32(xq.wq^T) * sx) * sw for rows routed to expert e_idx,
 * +0 for rows with gate[row * n_experts + e_idx] <= 0 (moe_linear_gated_i8.wgsl:66-69).
 * The GEMV (m <= 32) or MFMA GEMM skips the weights of a launch (GEMV) or
 * output tile (GEMM) with no routed row, multiplies the rest and zeroes the
 * unrouted rows in the epilogue. From m = 8192 (K % 32 == 0, 16-byte
 * aligned xq/wq) the routed rows are first packed into the stream's
 * workspace and the GEMM runs over them alone.
 * Step name "moe_linear_gated_i8": bindings [xq, wq, sx, sw, gate, out],
 * params [m, kg, n, n_experts, e_idx]. */
int bh_moe_linear_gated_i8(void* stream, const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                           const float* gate, uint32_t n_experts, uint32_t e_idx, float* out, uint32_t m, uint32_t kg,
                           uint32_t n);

/* The int8 paged KV cache (brain's int8 serving attention, crates/qwen3/src/serve.rs:1262-1270).
 * pool: int8 codes, 4 per u32 word, kv_stride bytes per slot, slot = physical_block *
 * block_size + offset; scales: one f32 per (slot, kv head). pool_words / n_scales are
 * the lengths of those buffers: the slots the device-side tables name are checked
 * against them, and one outside is skipped (nothing stored or added) where the
 * reference would access out of bounds. head_dim % 4 == 0, head_dim <= 256,
 * kv_stride % head_dim == 0. Each f32 result keeps the reference's summation order.
 *
 * paged_kv_append_i8_clipped_batched (crates/kernels/wgsl/paged_kv_append_i8_clipped_batched.wgsl:46-77):
 * for each sequence b and kv head h of src [batch][kv_stride], scale = min(max|x|,
 * clip[h]) / 127 (1 when that is 0) into scales[slot*n_kv + h], codes clamp(round_even(x /
 * scale), +-127) into the pool, at slot blocks[b]*block_size + offsets[b]. Step bindings
 * [src, blocks, offsets, clip, pool, scales], params [batch, kv_stride, block_size, head_dim]. */
int bh_paged_kv_append_i8(void* stream, const float* src, const uint32_t* blocks, const uint32_t* offsets,
                          const float* clip, uint32_t* pool, uint64_t pool_words, float* scales, uint64_t n_scales,
                          uint32_t batch, uint32_t kv_stride, uint32_t block_size, uint32_t head_dim);
/* paged_decode_scores_i8_batched (crates/kernels/wgsl/paged_decode_scores_i8_batched.wgsl:28-54):
 * scores[b][h][j] = ((sum_d q[b][h][d] * code) * kscale) * scale for j < seq_lens[b]
 * (entries past it untouched), kv head h / group, position j at block_tables[b*max_bt +
 * j/block_size]. Step bindings [q, pool, block_tables, seq_lens, scales, scores], params
 * [batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt, scale_bits]. */
int bh_paged_decode_scores_i8(void* stream, const float* q, const uint32_t* pool, uint64_t pool_words,
                              const uint32_t* block_tables, const uint32_t* seq_lens, const float* scales,
                              uint64_t n_scales, float* scores, uint32_t batch, uint32_t n_heads, uint32_t group,
                              uint32_t head_dim, uint32_t block_size, uint32_t kv_stride, uint32_t cap,
                              uint32_t max_bt, float scale);
/* paged_decode_apply_i8_batched (crates/kernels/wgsl/paged_decode_apply_i8_batched.wgsl:28-53):
 * ctx[b][h*head_dim + d] = sum over j < min(seq_lens[b], cap) (in order) of
 * (probs[b][h][j] * code) * vscale. The reference loops to seq_lens[b]; past cap it would
 * read the next row's probabilities, so the sum stops at the row's end here. Step bindings [probs, pool, block_tables, seq_lens, scales, ctx], params
 * [batch, n_heads, group, head_dim, block_size, kv_stride, cap, max_bt]. */
int bh_paged_decode_apply_i8(void* stream, const float* probs, const uint32_t* pool, uint64_t pool_words,
                             const uint32_t* block_tables, const uint32_t* seq_lens, const float* scales,
                             uint64_t n_scales, float* ctx, uint32_t batch, uint32_t n_heads, uint32_t group,
                             uint32_t head_dim, uint32_t block_size, uint32_t kv_stride, uint32_t cap,
                             uint32_t max_bt);

/* f32 -> bf16 bits, round to nearest even, NaN -> (bits >> 16) | 0x0040: the
 * conversion every bf16 output of this library goes through
 * (crates/model/src/half.rs:49-58, f32_to_bf16). x [n] f32 -> out [n] u16. */
int bh_f32_to_bf16(void* stream, const float* x, uint16_t* out, uint64_t n);

/* Int8 matrix-core roof probe: `blocks` workgroups of 256 threads each run
 * `iters` rounds of 4 independent v_mfma_i32_32x32x32_i8 chains; out[blocks*256] i32
 * receives a data-dependent sum so nothing folds. Ops executed =
 * blocks*4*iters*4*65536. The MI355X counterpart of the `roof_dp4a` probe
 * (crates/kernels/wgsl/roof_dp4a.wgsl:28-63, crates/gpu-core/src/roof.rs:99-130). */
int bh_roof_mfma_i8(void* stream, uint32_t blocks, uint32_t iters, int32_t* out);
/* HBM read roof probe (the bandwidth half of crates/gpu-core/src/roof.rs:458-490):
 * `blocks` workgroups of 256 threads read `bytes` (a multiple of 16, 16-byte
 * aligned) from `src` with 16-byte non-temporal vector loads, 8 in flight per
 * thread, and write one folded word per thread to `out` (blocks*256 words).
 * Also a calibration kernel for the FETCH_SIZE counter. */
int bh_roof_hbm_read(void* stream, const void* src, uint64_t bytes, uint32_t blocks, uint32_t* out);

/* ======================================================================
 * B. backend_api::Backend as a C ABI (crates/backend-api/src/lib.rs:696-908).
 * ====================================================================== */

typedef struct bh_backend bh_backend; /* `Box<dyn Backend>` */
typedef struct bh_buffer bh_buffer;   /* `DeviceBuffer` (refcounted, clones alias) */
typedef struct bh_dispatch bh_dispatch; /* `Step` (refcounted recorded dispatch) */

/* Kernel names this backend executes (the reference's kernel catalogue names,
 * crates/kernels/src/lib.rs:555-713):
 *   "max_abs_row", "max_abs_rows"  bindings [x, sx]                    params [m, k]
 *   "quant_pack"                   bindings [x, sx, xq]                params [m, k]
 *   "matmul_i8_dyn", "matmul_i8_gemv"
 *                                  bindings [xq, wq, sx, sw, out]      params [m, kg, n]
 *   "matmul_i8"                    bindings [x, w, out]                params [m, kg, n, f32 sx, f32 sw]
 *   "bias_add"                     bindings [out, bias]                params [m, n]
 *   "roof_dp4a"                    bindings [inp, out]                 params [n, iters, a, b]
 * `threads` is accepted for signature parity and ignored: each kernel derives
 * its own grid from its params. */

/* Backend factory (`Factory`, crates/backend-api/src/lib.rs:992-1020).
 * names[i] (and optionally srcs[i], ignored except for being accepted) is the
 * kernel set; the returned backend's kernel index i is names[i]. With
 * flags & BH_CREATE_LENIENT, unknown names are accepted and fail with
 * BH_ERR_UNSUPPORTED only when dispatched; without it creation fails so the
 * caller can fall back to another backend. device = HIP device ordinal. */
#define BH_CREATE_LENIENT 1u
int bh_backend_create(const char* const* names, const char* const* srcs, uint32_t n_kernels, int device,
                      uint32_t flags, bh_backend** out);
void bh_backend_destroy(bh_backend* be);
/* `kind()`: "hip". */
const char* bh_backend_kind(const bh_backend* be);
/* Index of `name` in the creation list, or -1 (`Gpu::kernel_index`, crates/gpu-core/src/lib.rs:796). */
int bh_kernel_index(const bh_backend* be, const char* name);
/* The backend's HIP stream (hipStream_t) — steps run on it in submit order. */
void* bh_backend_stream(const bh_backend* be);

/* `DeviceCaps` + `NumericSupport` (crates/backend-api/src/lib.rs:177-213, 471-507). */
typedef struct {
    uint32_t compute_units;
    uint32_t max_workgroup_size;
    uint32_t workgroup_mem_bytes;
    uint32_t subgroup_size;
    uint32_t unified_memory;
    uint32_t workgroup_reductions; /* 1: cooperative (GEMV) variants are valid */
    float peak_bandwidth_gbs;      /* 0 = unmeasured */
    float peak_gflops;             /* 0 = unmeasured */
    uint32_t numeric_f32, numeric_int8_dot, numeric_f16, numeric_bf16;
    uint32_t numeric_f16_storage, numeric_bf16_storage, numeric_coop_matrix;
    uint64_t max_buffer_bytes;
    uint64_t max_storage_binding_bytes;
    char device_name[64];
} bh_caps_t;
int bh_caps(const bh_backend* be, bh_caps_t* caps);

/* `storage(n)`: n zeroed f32 words. */
int bh_storage(bh_backend* be, uint64_t n_words, bh_buffer** out);
/* `storage_init(name, data)`. */
int bh_storage_init(bh_backend* be, const char* label, const float* data, uint64_t n_words, bh_buffer** out);
bh_buffer* bh_buffer_retain(bh_buffer* b); /* DeviceBuffer::clone */
void bh_buffer_release(bh_buffer* b);      /* drop; memory freed on the last release */
uint64_t bh_buffer_words(const bh_buffer* b);
void* bh_buffer_device_ptr(const bh_buffer* b);
/* `write` / `write_at` (crates/backend-api/src/lib.rs:704-721): ordered after prior submits. */
int bh_write(bh_backend* be, bh_buffer* buf, const uint32_t* data, uint64_t n_words);
int bh_write_at(bh_backend* be, bh_buffer* buf, uint64_t offset_words, const uint32_t* data, uint64_t n_words);
/* `read(buf, n)`: blocks, copies the first n words back (as raw 32-bit words). */
int bh_read(bh_backend* be, const bh_buffer* buf, void* dst, uint64_t n_words);

/* `step(kind, bufs, params, threads)`. */
int bh_step(bh_backend* be, uint32_t kind, bh_buffer* const* bufs, uint32_t nbufs, const uint32_t* params,
            uint32_t nparams, uint32_t threads, bh_dispatch** out);
/* `step_sliced`: offsets holds nbufs (offset, len) pairs in 4-byte WORDS,
 * len 0 = to the end of the buffer (crates/backend-api/src/lib.rs:723-731;
 * the words-not-bytes convention of crates/model/src/int8.rs:208-220).
 * Every binding is bounds-checked against what the kernel will touch. */
int bh_step_sliced(bh_backend* be, uint32_t kind, bh_buffer* const* bufs, const uint64_t* offsets,
                   uint32_t nbufs, const uint32_t* params, uint32_t nparams, uint32_t threads, bh_dispatch** out);
bh_dispatch* bh_step_retain(bh_dispatch* s);
void bh_step_release(bh_dispatch* s);
/* `submit(clears, steps)`: zero `clears`, then enqueue every step in order. */
int bh_submit(bh_backend* be, bh_buffer* const* clears, uint32_t nclears, bh_dispatch* const* steps, uint32_t nsteps);
int bh_flush(bh_backend* be);
int bh_poll_wait(bh_backend* be);
/* `poll_wait_timeout`: BH_OK if idle within timeout_ms, BH_ERR_TIMEOUT otherwise. */
int bh_poll_wait_timeout(bh_backend* be, uint32_t timeout_ms);

/* Per-kernel device timing (`set_kernel_timing` / `kernel_times` /
 * `reset_kernel_times`, crates/backend-api/src/lib.rs:888-907; enabled at
 * creation when BRAIN_PROFILE is set and not "0", lib.rs:917-919). */
typedef struct {
    char name[48];
    double ms;
    uint64_t calls;
} bh_kernel_time_t;
int bh_set_kernel_timing(bh_backend* be, int on); /* returns 1 if timing is now on */
/* Writes up to cap entries; returns the number of kernels with calls > 0 (or <0 on error). */
int bh_kernel_times(bh_backend* be, bh_kernel_time_t* out, uint32_t cap);
void bh_reset_kernel_times(bh_backend* be);

/* `DeviceStats` (crates/backend-api/src/lib.rs:924-931). */
typedef struct {
    uint64_t submits, dispatches, readbacks, bind_groups, uniform_allocs;
} bh_stats_t;
int bh_stats(const bh_backend* be, bh_stats_t* st);

/* ======================================================================
 * C. Host-side int8 helpers of the model layer.
 * ====================================================================== */

/* crates/model/src/int8.rs:33-59 — row-parallel host quantizer (ties AWAY). */
int bh_quantize_weight(const float* w, uint64_t n, uint64_t k, uint32_t* packed, float* sw);
/* `model::int4::quantize_weight_q4` (crates/model/src/int4.rs:46-67): per-row
 * sw = max(max|w|,1e-8)/7, q = clamp(round_half_away(w*(1/sw)), +-7) packed
 * 8 per u32. k % 8 == 0. Host, row-parallel. */
int bh_quantize_weight_q4(const float* w, uint64_t n, uint64_t k, uint32_t* packed, float* sw);
/* crates/model/src/int8.rs:70-87 */
int bh_dequantize_weight(const uint32_t* packed, const float* sw, uint64_t n, uint64_t k, float* w);

/* `model::int8::quant_rows_steps` (crates/model/src/int8.rs:221-235): the
 * max_abs_row -> quant_pack steps for rows r0..r1 of x [.., k], with x/xq
 * offset in their own elements and sx in rows. r0 % 64 == 0 as in the
 * reference. kernels = {max_abs_row index, quant_pack index}. */
int bh_quant_rows_steps(bh_backend* be, const uint32_t kernels[2], bh_buffer* x, bh_buffer* sx, bh_buffer* xq,
                        uint32_t r0, uint32_t r1, uint32_t k, bh_dispatch* out[2]);

/* `model::dispatch::mm8_rows_off` (crates/model/src/dispatch.rs:119-130):
 * rows xr0..xr0+m of the packed activation -> m*n floats of o at ooff. */
int bh_mm8_rows_off(bh_backend* be, uint32_t kind, bh_buffer* xq, bh_buffer* wq, bh_buffer* sx, bh_buffer* sw,
                    bh_buffer* o, uint32_t xr0, uint64_t ooff, uint32_t m, uint32_t k, uint32_t n, bh_dispatch** out);

/* `backend_api::select::candidates` I8 arm (crates/backend-api/src/select.rs:197,209,323-331),
 * in the reference's order: m > 32 or no workgroup reductions -> tile only; m <= 8 -> GEMV
 * then tile; 8 < m <= 32 -> tile then GEMV. (bh_matmul_i8 does not follow this order: it
 * runs a tuned choice if one was measured, else the GEMV for every m <= 32, the MI355X
 * crossover.) Variant codes: */
enum { BH_VARIANT_PACKED_INT8 = 1, BH_VARIANT_WORKGROUP_PER_OUTPUT = 2 };
/* Fills out[0..ret) with candidate variants, best first; returns the count. */
int bh_select_i8(uint32_t m, uint32_t n, uint32_t k, int int8_dot, int workgroup_reductions, int out[2]);
/* The kernel name a variant binds to (`Ops::bind`, crates/model/src/ops.rs:603-625). */
const char* bh_variant_kernel(int variant);

/* GEMV-vs-tile autotune (`Engine::tune_i8` / `measure_i8`,
 * crates/qwen3/src/serve.rs:1117-1158; `AutoTuner`, crates/backend-api/src/select.rs:466-540).
 * bh_tune_i8 times both candidates for [m,k] x [n,k] (m <= 32) on scratch
 * buffers, `reps` dispatches each, records the faster for m's power-of-two
 * row bucket and returns it (ms[0] GEMV, ms[1] tile, mean per dispatch).
 * bh_matmul_i8 and the Qwen3 engine consult the recorded choices; without
 * one the static selector applies. The store is a text file: a header naming
 * the ABI version, the device and a fingerprint of the GEMV/GEMM kernel
 * sources and flags, then "m n k variant" lines; bh_tune_load refuses a file
 * whose header differs (a table from another device or kernel build). */
int bh_tune_i8(void* stream, uint32_t m, uint32_t k, uint32_t n, uint32_t reps, int* variant, float ms[2]);
int bh_tune_set(uint32_t m, uint32_t n, uint32_t k, int variant); /* variant 0 removes the entry */
int bh_tune_get(uint32_t m, uint32_t n, uint32_t k);               /* 0: none recorded */
void bh_tune_clear(void);
int bh_tune_save(const char* path);
int bh_tune_load(const char* path);                                /* returns the entries read */

/* `gpu_core::cost` (crates/gpu-core/src/cost.rs:267-275) for the int8 family:
 * flops, int_ops and bytes of one dispatch of `name` with `params`. */
typedef struct {
    uint64_t flops, int_ops, bytes;
} bh_cost_t;
int bh_cost(const char* name, const uint32_t* params, uint32_t nparams, bh_cost_t* out);

/* Inspect one tensor of a safetensors file (the int8 checkpoint container):
 * dtype (1 F32, 2 U32, 3 I8, 4 U8, 5 F16, 6 BF16, 7 I32, 0 other), rank and up
 * to max_rank dims. Host only. */
int bh_st_describe(const char* path, const char* name, int* dtype, uint64_t* shape, uint32_t max_rank,
                   uint32_t* rank);

/* ======================================================================
 * D. The int8 Qwen3 decoder (the caller of sections A-C the reference runs
 *    most): `qwen3::serve::Engine` with int8 weights
 *    (crates/qwen3/src/serve.rs:1194-1367 step tape, :1557-1620 prefill,
 *    :1332-1367 greedy head; config crates/qwen3/src/config.rs:100-118).
 *    Per layer: RMSNorm -> int8 q/k/v -> QK-norm -> RoPE -> KV append ->
 *    causal GQA attention -> int8 o -> residual -> RMSNorm -> int8 gate/up ->
 *    SwiGLU -> int8 down -> residual; then RMSNorm, the int8 head and a
 *    greedy argmax on the device. Activations f32; every linear quantizes its
 *    input per token (max_abs_row + quant_pack semantics) and runs
 *    bh_matmul_i8 with f32 output. The KV cache holds, per layer, K and V
 *    rows [slot][kv_dim] in one of two modes: f32 (kv_int8 = 0), or int8
 *    codes (kv_int8 = 1, 4 per u32 word) with one f32 scale per (slot, kv
 *    head) [slot][n_kv_heads], min(max|x|, clip)/127 (1 when that is 0),
 *    where the clip ceilings are per (layer, kv head) and default to FLT_MAX
 *    (no clipping; see bh_qwen3_set_kv_clip). Slots are either one
 *    contiguous slab of max_seq per sequence (kv_block_size = 0), or the
 *    reference's paged pool (crates/qwen3/src/serve.rs:349-356,
 *    paged_kv_append_i8_clipped_batched.wgsl:46-77): kv_num_blocks blocks of
 *    kv_block_size slots, position p of sequence b at slot
 *    table[b][p / kv_block_size] * kv_block_size + p % kv_block_size
 *    (bh_qwen3_set_block_table).
 * ====================================================================== */
typedef struct bh_qwen3 bh_qwen3;

/* `QwenConfig` fields the forward reads. head_dim % 64 == 0, head_dim <= 256,
 * n_heads % n_kv_heads == 0, d_model, q_dim, d_ff multiples of 4 and <= 8192. */
typedef struct {
    uint32_t vocab, n_layers, d_model, n_heads, n_kv_heads, head_dim, d_ff;
    float rope_theta, rms_eps;
    uint32_t tie_embeddings; /* 1: the head is tok.weight (quantized), else lm_head.weight */
    uint32_t qk_norm;        /* 1: per-head RMSNorm of q and k before RoPE */
    uint32_t kv_int8;        /* engine option: 1 = int8 KV cache with per-(token, kv head) scales
                                (paged_kv_append_i8_clipped_batched / paged_decode_{scores,apply}_i8_batched) */
    uint32_t kv_block_size;  /* engine option: 0 = one slab per sequence; else a paged pool of blocks of
                                this many positions (a multiple of 32) addressed through a block table */
    uint32_t kv_num_blocks;  /* paged: blocks in the pool (0: max_batch * ceil(max_seq / kv_block_size)) */
} bh_qwen3_config;

/* Engine for up to max_batch sequences of max_seq positions each; prefill
 * chunks hold at most max_rows token rows (batch * positions). Allocates every
 * device buffer once; weights start unset (zero). */
int bh_qwen3_create(const bh_qwen3_config* cfg, uint32_t max_batch, uint32_t max_seq, uint32_t max_rows,
                    int device, bh_qwen3** out);
void bh_qwen3_destroy(bh_qwen3* e);

/* Upload one f32 parameter by its reference name (`decoder_param_list`,
 * serve.rs:320-340: tok.weight, norm.weight, lm_head.weight,
 * blocks.{l}.{ln1,ln2}.weight, blocks.{l}.attn.{wq,wk,wv,wo,q_norm,k_norm}.weight,
 * blocks.{l}.mlp.{gate,up,down}.weight). Linear weights are quantized on the
 * device per output row (crates/model/src/int8.rs:33-59); with tied
 * embeddings tok.weight also becomes the int8 head. numel must match. */
int bh_qwen3_set_weight(bh_qwen3* e, const char* name, const float* host, uint64_t numel);
/* Upload an already-quantized linear (packed [n, k/4] u32 + scales [n], the
 * int8 on-disk layout of crates/model/src/int8.rs:112-187). */
int bh_qwen3_set_weight_i8(bh_qwen3* e, const char* name, const uint32_t* packed, const float* scale,
                           uint32_t n, uint32_t k);
/* Random init on the device with the reference's distributions
 * (crates/qwen3/src/init.rs:30-59): norm gains 1, wo/down N(0, 0.02/sqrt(2L)),
 * other linears and the embedding N(0, 0.02). Counter-based generator, so a
 * seed gives the same weights on every run (not the reference's stream). */
int bh_qwen3_init_random(bh_qwen3* e, uint64_t seed);

/* Start `batch` sequences from prompts tokens[batch][len] (row-major): runs
 * the prompt rows through every layer (chunked to max_rows), fills the KV
 * cache, and writes each sequence's greedy next token to next[batch]. */
int bh_qwen3_prefill(bh_qwen3* e, const uint32_t* tokens, uint32_t batch, uint32_t len, uint32_t* next);
/* `steps` greedy decode steps of every live sequence: each step feeds the
 * previous token back on the device (no host round trip) and appends the new
 * one. out[steps][batch] receives the generated tokens. The step is captured
 * once in a HIP graph and replayed (flags & BH_QWEN3_EAGER: launch eagerly).
 * flags & BH_QWEN3_UNFUSED: run every producer (norm, rotation + cache append,
 * attention merge, SwiGLU) as its own kernel instead of inside its consumer;
 * the results are the same bit for bit (a validation aid). */
#define BH_QWEN3_EAGER 1u
#define BH_QWEN3_UNFUSED 2u
int bh_qwen3_decode(bh_qwen3* e, uint32_t steps, uint32_t flags, uint32_t* out);
/* Logits [batch, vocab] f32 of the most recent head evaluation (prefill or
 * the last decode step). */
int bh_qwen3_logits(bh_qwen3* e, float* out, uint64_t n);
/* Positions filled so far (prompt + decoded) of each sequence: len[batch]. */
int bh_qwen3_lengths(bh_qwen3* e, uint32_t* len, uint32_t batch);
/* Copy the cache of one layer and sequence to the host (which: 0 = K, 1 = V):
 * positions pos0..pos0+npos, [npos][n_kv_heads*head_dim] f32, or int8 codes
 * with kv_int8, then (kv_int8, scales not NULL) their scales [npos][n_kv_heads].
 * A validation aid: the codes and scales are the engine's own. */
int bh_qwen3_kv_read(bh_qwen3* e, uint32_t layer, uint32_t seq, uint32_t which, uint32_t pos0, uint32_t npos,
                     void* data, float* scales);
/* Paged pool (kv_block_size > 0): the block table, table[rows][max_blocks_per_seq]
 * (max_blocks_per_seq = ceil(max_seq / kv_block_size)), entry i of row b the
 * physical block of positions [i * kv_block_size, (i + 1) * kv_block_size) of
 * sequence b, or BH_QWEN3_NO_BLOCK; rows past `rows` become unallocated. The
 * reference's BlockAllocator hands out such tables; bh_qwen3_prefill and
 * bh_qwen3_decode refuse to run a sequence whose positions reach a block that
 * is unallocated or also used by another sequence. Default when the pool
 * holds max_batch * max_blocks_per_seq blocks: row b owns blocks
 * b * max_blocks_per_seq + i; otherwise nothing is allocated. */
#define BH_QWEN3_NO_BLOCK 0xFFFFFFFFu
int bh_qwen3_set_block_table(bh_qwen3* e, const uint32_t* table, uint32_t rows, uint32_t max_blocks_per_seq);
/* The device memory of one layer's K (which 0) or V (1) cache: `pool` (f32
 * rows, or int8 codes 4 per u32 word, [slot][kv_dim], pool_words words) and,
 * with kv_int8, `scales` [slot][n_kv_heads] (n_scales floats; else NULL, 0).
 * With a paged pool these are the buffers the reference's paged kernels
 * (bh_paged_decode_scores_i8 / _apply_i8) read with the same block table.
 * Valid until bh_qwen3_destroy; writes race with the engine's own. */
int bh_qwen3_kv_pool(bh_qwen3* e, uint32_t layer, uint32_t which, void** pool, uint64_t* pool_words, float** scales,
                     uint64_t* n_scales);
/* int8 KV: per-kv-head ceilings of layer `layer` for K (which 0) or V (1);
 * the scale is min(max|x|, clip)/127. Default FLT_MAX (no clipping), the
 * reference's uncalibrated sentinel. */
int bh_qwen3_set_kv_clip(bh_qwen3* e, uint32_t layer, uint32_t which, const float* clip);
void* bh_qwen3_stream(bh_qwen3* e);
/* Measure the GEMV/tile choice for every distinct linear shape of the engine
 * at row buckets 1..max_batch (bh_tune_i8); BRAIN_NO_AUTOTUNE=1 skips it, as
 * in the reference. Returns the number of shapes measured. */
int bh_qwen3_autotune(bh_qwen3* e, uint32_t reps);

/* Load every parameter from an int8 checkpoint: a safetensors file in which a
 * quantized linear `name` is U32 [n, k/4] (the packed layout above) with an
 * F32 sibling `name.scale` [n], and any other tensor is F32
 * (crates/model/src/int8.rs:112-187, crates/qwen3omnimoe/src/import.rs:420-425).
 * An F32 linear is quantized on the device as bh_qwen3_set_weight does. The
 * file is memory-mapped and uploaded in row-aligned chunks, so host memory
 * stays bounded. Every parameter of the config must be present. */
int bh_qwen3_load(bh_qwen3* e, const char* path);

#ifdef __cplusplus
}
#endif
#endif /* BRAIN_HIP_H */
