/* CPU oracle for the brain int8 (W8A8) matmul path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's integer and f32 arithmetic, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. Nothing in brain_amd/ links, loads or calls this library; the
 * product path is the HIP library libbrain_hip.so.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the swedishembedded/brain source tree). Build with -ffp-contract=off so that
 * products such as (acc*sx)*sw are never fused into an FMA.
 *
 * Pinning (how each function is checked against something other than itself):
 *  - or_splitmix64_*       : SplitMix64 published constants; known first outputs
 *                            of the reference generator (tests/test_oracle.py).
 *  - or_quantize_weight    : the reference's serial oracle on its xorshift fixture
 *                            (5 shapes) plus round-trip |deq-w| <= sw/2 and the
 *                            sign-extension mutation test.
 *  - or_max_abs_row        : closed form (max is exact), all-zero row -> 1e-8/127.
 *  - or_quant_pack         : ties-to-even known answers [-2.5..3.5] -> [-2,-2,-0,0,2,2,4],
 *                            |x|=max -> +-127, x*(1/sx) vs x/sx discriminating case.
 *  - or_matmul_i8_acc      : the reference's dot4I8Packed known answer
 *                            (m=2,k=8,n=3 -> [[9660,17202,-10701],[14168,-7773,-10589]])
 *                            and numpy int64 brute force.
 *  - or_epilogue_*         : the same known answer's f32 outputs, and IEEE
 *                            left-to-right products evaluated independently in numpy.
 *  - or_f32_to_bf16        : RNE closed form against numpy/torch bf16 rounding,
 *                            ties, NaN quieting, Inf.
 */
#ifndef BRAIN_ORACLE_H
#define BRAIN_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* crates/data/src/rng.rs:13-73 (SplitMix64). */
typedef struct { uint64_t state; } or_rng;
void     or_rng_new(or_rng* r, uint64_t seed);
uint64_t or_rng_next_u64(or_rng* r);
double   or_rng_next_f64(or_rng* r);
float    or_rng_next_f32(or_rng* r);
int64_t  or_rng_gen_range_inclusive(or_rng* r, int64_t lo, int64_t hi);
double   or_rng_uniform(or_rng* r, double lo, double hi);
double   or_rng_next_gaussian(or_rng* r);

/* crates/model/src/int8.rs:33-59 — per-output-row weight quantization,
 * f32::round (ties AWAY from zero), packed 4 int8 per u32 little-endian. */
void or_quantize_weight(const float* w, int64_t n, int64_t k, uint32_t* packed, float* sw);
/* crates/model/src/int8.rs:70-87 */
void or_dequantize_weight(const uint32_t* packed, const float* sw, int64_t n, int64_t k, float* w);

/* crates/kernels/wgsl/max_abs_row.wgsl:27-34 (== max_abs_rows.wgsl:60-84). */
void or_max_abs_row(const float* x, int64_t m, int64_t k, float* sx);
/* crates/kernels/wgsl/quant_pack.wgsl:29-44 — round() is ties-to-even. */
void or_quant_pack(const float* x, const float* sx, int64_t m, int64_t k, uint32_t* xq);

/* Exact i32 accumulators of the packed int8 NT GEMM, acc[m*n_+n]
 * (crates/kernels/wgsl/matmul_i8_dyn.wgsl:129-156, matmul_i8_gemv.wgsl:57-66;
 * dot4I8Packed lowered as sign-extend multiply-add, crates/wgsl-cpu/src/lib.rs:1508-1524).
 * i32 arithmetic wraps like WGSL's. */
void or_matmul_i8_acc(const uint32_t* xq, const uint32_t* wq, int64_t m, int64_t kg, int64_t n, int32_t* acc);

/* Dequant epilogue (matmul_i8_dyn.wgsl:194, matmul_i8_gemv.wgsl:74):
 *   out = (f32(acc) * sx[m]) * sw[n]
 * then, if bias != NULL, out + bias[n] (bias_add.wgsl, a separate dispatch in
 * the reference), then for out_dtype==1 f32_to_bf16 RNE (crates/model/src/half.rs:49-58).
 * out_dtype 0: float* out; 1: uint16_t* out (bf16 bits). */
void or_epilogue(const int32_t* acc, const float* sx, const float* sw, const float* bias,
                 int64_t m, int64_t n, int out_dtype, void* out);
/* crates/kernels/wgsl/matmul_i8.wgsl:164-200 — static per-tensor scales:
 *   out = f32(acc) * (sx * sw) */
void or_epilogue_static(const int32_t* acc, float sx, float sw, int64_t m, int64_t n, float* out);

/* Whole W8A8 linear: or_matmul_i8_acc then or_epilogue. */
void or_matmul_i8(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                  const float* bias, int64_t m, int64_t kg, int64_t n, int out_dtype, void* out);

/* crates/model/src/half.rs:49-58 */
uint16_t or_f32_to_bf16(float f);
void or_f32_to_bf16_array(const float* x, uint16_t* out, size_t n);
/* W4A8: int4 weight quantizer (int4.rs:46-67), its inverse, exact accumulators. */
void or_quantize_weight_q4(const float* w, int64_t n, int64_t k, uint32_t* packed, float* sw);
void or_dequantize_weight_q4(const uint32_t* packed, const float* sw, int64_t n, int64_t k, float* w);
void or_matmul_q4_acc(const uint32_t* xq, const uint32_t* w4, int64_t m, int64_t k, int64_t n, int32_t* acc);

/* CPU baseline: backend-cpu's execution of max_abs_row -> quant_pack ->
 * matmul_i8_gemv, restated (one workgroup per output column, 64 invocations
 * run as a pre-barrier loop then the post-barrier fold; workgroups spread over
 * `threads` OpenMP threads like rayon over available_parallelism).
 * crates/backend-cpu/src/lib.rs:196-198,362-406; crates/wgsl-cpu/src/lib.rs:537-640;
 * crates/kernels/wgsl/matmul_i8_gemv.wgsl:39-76. m <= 32. */
void or_cpu_linear_gemv(const float* x, const uint32_t* wq, const float* sw,
                        int64_t m, int64_t k, int64_t n, int threads,
                        float* sx_scratch, uint32_t* xq_scratch, float* out);
/* Same restated GEMV applied to an already-quantized activation. */
void or_cpu_gemv_packed(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                        int64_t m, int64_t kg, int64_t n, int threads, float* out);
/* A stronger host reference for prefill, which backend-cpu has no int8 path
 * for (crates/gpu-core/tests/bench_matmul.rs:243-247): OpenMP over 4x4 output
 * tiles, each dot product an i32 sum over K (SIMD), then (f32(acc)*sx)*sw. */
void or_cpu_gemm_i8_tiled(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                          int64_t m, int64_t kg, int64_t n, int threads, float* out);

#ifdef __cplusplus
}
#endif
#endif
