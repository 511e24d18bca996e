/* CPU oracle for the brain int8 (W8A8) matmul path — TEST INFRASTRUCTURE ONLY.
 * See brain_oracle.h for the role of this file and how each function is pinned.
 * Compiled with -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile). */
#include "brain_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- crates/data/src/rng.rs:13-73 ------------------------------------- */
#define SM_GAMMA 0x9E3779B97F4A7C15ULL
void or_rng_new(or_rng* r, uint64_t seed) { r->state = seed + SM_GAMMA; } /* rng.rs:22-27 */
uint64_t or_rng_next_u64(or_rng* r) {                                        /* rng.rs:30-36 */
    r->state += SM_GAMMA;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
double or_rng_next_f64(or_rng* r) {                                          /* rng.rs:39-42 */
    return (double)(or_rng_next_u64(r) >> 11) / (double)(1ULL << 53);
}
float or_rng_next_f32(or_rng* r) { return (float)or_rng_next_f64(r); }       /* rng.rs:45-47 */
int64_t or_rng_gen_range_inclusive(or_rng* r, int64_t lo, int64_t hi) {      /* rng.rs:50-54 */
    uint64_t span = (uint64_t)(hi - lo + 1);
    return lo + (int64_t)(or_rng_next_u64(r) % span);
}
double or_rng_uniform(or_rng* r, double lo, double hi) {                      /* rng.rs:57-59 */
    return lo + (hi - lo) * or_rng_next_f64(r);
}
double or_rng_next_gaussian(or_rng* r) {                                     /* rng.rs:67-72 */
    double u1 = or_rng_next_f64(r);
    if (u1 < 1e-12) u1 = 1e-12;
    double u2 = or_rng_next_f64(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

/* Rust `f32::max` / WGSL `max`: the non-NaN operand wins (IEEE maxNum). */
static inline float mx(float a, float b) { return fmaxf(a, b); }

/* ---- crates/model/src/int8.rs:33-59 ------------------------------------ */
void or_quantize_weight(const float* w, int64_t n, int64_t k, uint32_t* packed, float* sw) {
    int64_t kg = k / 4;
    for (int64_t r = 0; r < n; ++r) {
        const float* row = w + r * k;
        float a = 0.0f;                                   /* fold(0f32, max(v.abs())) */
        for (int64_t c = 0; c < k; ++c) a = mx(a, fabsf(row[c]));
        float s = mx(a, 1e-8f) / 127.0f;
        sw[r] = s;
        float inv = 1.0f / s;
        for (int64_t g = 0; g < kg; ++g) {
            uint32_t word = 0;
            for (int b = 0; b < 4; ++b) {
                float v = roundf(row[g * 4 + b] * inv);   /* f32::round: ties away */
                /* f32::clamp then `as i32` (saturating, NaN -> 0) */
                int32_t q;
                if (isnan(v)) q = 0;
                else { if (v < -127.0f) v = -127.0f; if (v > 127.0f) v = 127.0f; q = (int32_t)v; }
                word |= ((uint32_t)(uint8_t)q) << (8 * b);
            }
            packed[r * kg + g] = word;
        }
    }
}

/* ---- crates/model/src/int8.rs:70-87 ------------------------------------ */
void or_dequantize_weight(const uint32_t* packed, const float* sw, int64_t n, int64_t k, float* w) {
    int64_t kg = k / 4;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t g = 0; g < kg; ++g) {
            uint32_t word = packed[r * kg + g];
            for (int b = 0; b < 4; ++b)
                w[r * k + g * 4 + b] = (float)(int8_t)(uint8_t)(word >> (8 * b)) * sw[r];
        }
}

/* ---- crates/kernels/wgsl/max_abs_row.wgsl:27-34 ------------------------ */
void or_max_abs_row(const float* x, int64_t m, int64_t k, float* sx) {
    for (int64_t r = 0; r < m; ++r) {
        float a = 0.0f;
        for (int64_t c = 0; c < k; ++c) a = mx(a, fabsf(x[r * k + c]));
        sx[r] = mx(a, 1e-8f) / 127.0f;
    }
}

/* ---- crates/kernels/wgsl/quant_pack.wgsl:29-44 ------------------------- */
static inline uint32_t qbyte(float v, float inv) {
    float q = rintf(v * inv);                  /* WGSL round: ties to even (FE_TONEAREST) */
    q = fminf(fmaxf(q, -127.0f), 127.0f);      /* clamp(e,lo,hi) = min(max(e,lo),hi) */
    return (uint32_t)((int32_t)q & 0xff);
}
void or_quant_pack(const float* x, const float* sx, int64_t m, int64_t k, uint32_t* xq) {
    int64_t kg = k / 4;
    for (int64_t r = 0; r < m; ++r) {
        float inv = 1.0f / sx[r];
        for (int64_t g = 0; g < kg; ++g) {
            const float* p = x + r * k + g * 4;
            uint32_t w = 0;
            for (int b = 0; b < 4; ++b) w |= qbyte(p[b], inv) << (8 * b);
            xq[r * kg + g] = w;
        }
    }
}

/* dot4I8Packed: sign-extend each byte, multiply, add (wgsl-cpu/src/lib.rs:1508-1524). */
static inline uint32_t dot4(uint32_t a, uint32_t b) {
    uint32_t s = 0;
    for (int i = 0; i < 4; ++i)
        s += (uint32_t)((int32_t)(int8_t)(uint8_t)(a >> (8 * i)) * (int32_t)(int8_t)(uint8_t)(b >> (8 * i)));
    return s;
}

void or_matmul_i8_acc(const uint32_t* xq, const uint32_t* wq, int64_t m, int64_t kg, int64_t n, int32_t* acc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            uint32_t s = 0;                              /* wrapping i32 */
            for (int64_t g = 0; g < kg; ++g) s += dot4(xq[i * kg + g], wq[j * kg + g]);
            acc[i * n + j] = (int32_t)s;
        }
}

/* ---- crates/model/src/half.rs:49-58 ------------------------------------ */
uint16_t or_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    if (isnan(f)) return (uint16_t)((bits >> 16) | 0x0040);
    uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

/* or_f32_to_bf16 over an array (the GPU conversion test's expected bits). */
void or_f32_to_bf16_array(const float* x, uint16_t* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) out[i] = or_f32_to_bf16(x[i]);
}

void or_epilogue(const int32_t* acc, const float* sx, const float* sw, const float* bias,
                 int64_t m, int64_t n, int out_dtype, void* out) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float v = (float)acc[i * n + j] * sx[i];   /* matmul_i8_dyn.wgsl:194 */
            v = v * sw[j];
            if (bias) v = v + bias[j];                 /* bias_add.wgsl */
            if (out_dtype == 1) ((uint16_t*)out)[i * n + j] = or_f32_to_bf16(v);
            else ((float*)out)[i * n + j] = v;
        }
}

void or_epilogue_static(const int32_t* acc, float sx, float sw, int64_t m, int64_t n, float* out) {
    float sc = sx * sw;                                /* matmul_i8.wgsl:164 */
    for (int64_t i = 0; i < m * n; ++i) out[i] = (float)acc[i] * sc;
}

void or_matmul_i8(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                  const float* bias, int64_t m, int64_t kg, int64_t n, int out_dtype, void* out) {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(m * n > 0 ? m * n : 1));
    or_matmul_i8_acc(xq, wq, m, kg, n, acc);
    or_epilogue(acc, sx, sw, bias, m, n, out_dtype, out);
    free(acc);
}

/* ---- CPU baseline: backend-cpu's execution of the decode path ----------
 * matmul_i8_gemv.wgsl:39-76 as the Cranelift JIT runs a single-barrier
 * workgroup kernel: the 64 invocations execute the pre-barrier segment in a
 * loop, then the post-barrier segment (wgsl-cpu/src/lib.rs:537-640);
 * workgroups (= output columns) are spread over the thread pool
 * (backend-cpu/src/lib.rs:196-198, 362-406). */
void or_cpu_gemv_packed(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                        int64_t m, int64_t kg, int64_t n, int threads, float* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
#endif
    for (int64_t col = 0; col < n; ++col) {
        int32_t partial[32 * 64];
        for (int t = 0; t < 64; ++t) {                  /* pre-barrier, per invocation */
            for (int64_t r = 0; r < m; ++r) partial[r * 64 + t] = 0;
            for (int64_t g = t; g < kg; g += 64) {
                uint32_t wv = wq[col * kg + g];
                for (int64_t r = 0; r < m; ++r)
                    partial[r * 64 + t] = (int32_t)((uint32_t)partial[r * 64 + t] + dot4(xq[r * kg + g], wv));
            }
        }
        for (int64_t t = 0; t < m; ++t) {               /* post-barrier fold, threads 0..m */
            uint32_t s = 0;
            for (int i = 0; i < 64; ++i) s += (uint32_t)partial[t * 64 + i];
            out[t * n + col] = (float)(int32_t)s * sx[t] * sw[col];
        }
    }
    (void)threads;
}

void or_cpu_gemm_i8_tiled(const uint32_t* xq, const uint32_t* wq, const float* sx, const float* sw,
                          int64_t m, int64_t kg, int64_t n, int threads, float* out) {
    const int64_t k = kg * 4;
    const int64_t TM = 4, TN = 4;
    const int64_t tiles_n = (n + TN - 1) / TN, tiles = ((m + TM - 1) / TM) * tiles_n;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads)
#endif
    for (int64_t t = 0; t < tiles; ++t) {
        const int64_t r0 = (t / tiles_n) * TM, c0 = (t % tiles_n) * TN;
        for (int64_t r = r0; r < r0 + TM && r < m; ++r) {
            const int8_t* xr = (const int8_t*)(xq + r * kg);
            for (int64_t c = c0; c < c0 + TN && c < n; ++c) {
                const int8_t* wr = (const int8_t*)(wq + c * kg);
                int32_t acc = 0;
#ifdef _OPENMP
#pragma omp simd reduction(+ : acc)
#endif
                for (int64_t i = 0; i < k; ++i) acc += (int32_t)xr[i] * (int32_t)wr[i];
                out[r * n + c] = (float)acc * sx[r] * sw[c];
            }
        }
    }
    (void)threads;
}

void or_cpu_linear_gemv(const float* x, const uint32_t* wq, const float* sw,
                        int64_t m, int64_t k, int64_t n, int threads,
                        float* sx, uint32_t* xq, float* out) {
    int64_t kg = k / 4;
    /* max_abs_row: one invocation per row */
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads)
#endif
    for (int64_t r = 0; r < m; ++r) {
        float a = 0.0f;
        for (int64_t c = 0; c < k; ++c) a = mx(a, fabsf(x[r * k + c]));
        sx[r] = mx(a, 1e-8f) / 127.0f;
    }
    /* quant_pack: one invocation per output word */
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads)
#endif
    for (int64_t idx = 0; idx < m * kg; ++idx) {
        int64_t r = idx / kg, g = idx % kg;
        float inv = 1.0f / sx[r];
        const float* p = x + r * k + g * 4;
        uint32_t w = 0;
        for (int b = 0; b < 4; ++b) w |= qbyte(p[b], inv) << (8 * b);
        xq[idx] = w;
    }
    or_cpu_gemv_packed(xq, wq, sx, sw, m, kg, n, threads, out);
}

/* ---- W4A8 (crates/model/src/int4.rs:46-67, crates/kernels/wgsl/matmul_q4_gemv.wgsl) ---- */

/* quantize_weight_q4: sw = max(max|w|,1e-8)/7; q = clamp(round_half_away(w*(1/sw)), -7, 7)
 * (Rust f32::round, `as i32` maps NaN to 0); nibble b of word g holds column 8g+b. */
void or_quantize_weight_q4(const float* w, int64_t n, int64_t k, uint32_t* packed, float* sw) {
    const int64_t kg = k / 8;
    for (int64_t r = 0; r < n; ++r) {
        float m = 0.0f;
        for (int64_t c = 0; c < k; ++c) m = mx(m, fabsf(w[r * k + c]));
        const float s = mx(m, 1e-8f) / 7.0f;
        sw[r] = s;
        const float inv = 1.0f / s;
        for (int64_t g = 0; g < kg; ++g) {
            uint32_t word = 0;
            for (int b = 0; b < 8; ++b) {
                float q = roundf(w[r * k + g * 8 + b] * inv);
                q = q < -7.0f ? -7.0f : (q > 7.0f ? 7.0f : q);
                const int32_t qi = (q != q) ? 0 : (int32_t)q;
                word |= ((uint32_t)(uint8_t)qi & 0xFu) << (4 * b);
            }
            packed[r * kg + g] = word;
        }
    }
}

/* The nibble of column c, sign-extended (int4.rs dequantize_weight_q4). */
static int32_t q4_at(const uint32_t* row, int64_t c) {
    const uint32_t raw = (row[c / 8] >> (4 * (c % 8))) & 0xFu;
    return raw < 8 ? (int32_t)raw : (int32_t)raw - 16;
}

void or_dequantize_weight_q4(const uint32_t* packed, const float* sw, int64_t n, int64_t k, float* w) {
    for (int64_t r = 0; r < n; ++r)
        for (int64_t c = 0; c < k; ++c) w[r * k + c] = (float)q4_at(packed + r * (k / 8), c) * sw[r];
}

/* Exact i32 accumulators of the W4A8 product: xq [m, k/4] int8, w4 [n, k/8]. */
void or_matmul_q4_acc(const uint32_t* xq, const uint32_t* w4, int64_t m, int64_t k, int64_t n, int32_t* acc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t s = 0;
            const int8_t* a = (const int8_t*)(xq + i * (k / 4));
            for (int64_t c = 0; c < k; ++c) s += (int64_t)a[c] * q4_at(w4 + j * (k / 8), c);
            acc[i * n + j] = (int32_t)s;
        }
}
