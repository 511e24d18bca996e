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
#include <cfloat>
#include <cstdlib>
#include <type_traits>

#include "bh_attn.h"
#include "bh_common.h"

// Phase timestamps for latency studies: a timing build defines BH_STAMP(i)
// to record s_memrealtime at the marked points; the library leaves it empty.
#ifndef BH_STAMP
#define BH_STAMP(i)
#endif

namespace bh {

constexpr int GV_WAVES = 4;

struct GemvArgs {
    const uint32_t* xq;
    const uint32_t* wq;
    const float* sx;
    const float* sw;
    const float* bias;
    void* out;
    int m, kg, n;
    const float* gate;  // moe_linear_gated_i8 row gate (null: none): row r is +0 when gate[r*stride+col] <= 0
    int gate_stride, gate_col;
    // XMODE 2 (quantization fused into the prologue): the f32 activation
    // [m, K] and the caller's scratch, which workgroup 0 fills with the same
    // sx [m] and xq [m, K/4] that bh_quantize_rows writes.
    const float* x;
    float* sx_out;
    uint32_t* xq_out;
    // XMODE 3 / 4 (the decoder's producers fused into the prologue):
    //   3: x = pre_emb[pre_tok[r]] or pre_a[r] (+ pre_b[r]); workgroup 0 stores
    //      x to res_out[r]; y = RMSNorm(x) * pre_w (eps); quantize y;
    //   4: y = silu(g) * u over pre_a = [m, 2K] (gate | up); quantize y.
    const uint32_t* pre_tok;
    const float* pre_emb;
    const float* pre_a;
    const float* pre_b;
    const float* pre_w;
    float* res_out;
    float eps;
    // XMODE 5 (the decoder's attention merge fused into the output
    // projection): the per-chunk partials and row positions of the split
    // attention; x = merge(part_o, part_ml) of row r over its chunks.
    const float* part_o = nullptr;
    const float* part_ml = nullptr;
    const uint32_t* pos = nullptr;
    int nh = 0, hd = 0, splits = 0;
    // The wide-N streaming kernel reads the weights with ordinary loads in
    // the MFMA's layout (for a caller that re-reads them every step and
    // wants them kept in the caches) instead of whole 128-byte lines with
    // the non-temporal hint.
    bool keep_cached = false;
    // Greedy-argmax partials of the wide-N streaming kernel (null: none):
    // wave w stores, for every row r < m, the first column of its largest
    // output (strictly above -FLT_MAX; NaN never wins) at am_v/am_i[r *
    // am_stride + w], (-FLT_MAX, 0xffffffff) when it has none, and wave 0
    // stores the number of waves to *am_n.
    float* am_v = nullptr;
    uint32_t* am_i = nullptr;
    uint32_t* am_n = nullptr;
    int am_stride = 0;
};

// XMODE: 0 = packed activation read from global memory, 1 = staged into
// LDS first, 2 = quantized from f32 into LDS by the workgroup itself (each
// wave quantizes whole rows: exact row max, sx = max(max,1e-8)/127, codes
// clamp(rne(x * (1/sx))) -- bit-identical to bh_quantize_rows).
// PRE (XMODE 3 / 4 with several rows): 8 * R + G fixes the prologue's rows
// per thread and float4 groups per row at compile time; 0 picks them at run
// time.
// NTW: the weights are read with the non-temporal hint. Measured on the
// Qwen3-0.6B decode step, whose per-layer GEMVs are the fused ones: batch 1
// 0.876 -> 0.860 ms per step, but batch 4 1.089 -> 1.100 and batch 8 1.208
// -> 1.231 (and no change on the configs[1] sweep), so only the fused
// one-row launches take it.
// LINES: the K chunks go to the waves in pairs (wave ks owns pairs ks,
// ks + KSPLIT, ...; slot u of a batch is chunk 2 * pair + u % 2), and each
// pair of a column group is two loads of whole 128-byte lines (rows 0-7,
// then rows 8-15), put into the MFMA's layout by a row_ror:8 exchange, as
// the streaming kernel does. Needs ALIGNED, K % 128 == 0 and an even U.
template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED, int KSPLIT, int XMODE, int U, int CG, int NW = GV_WAVES,
          int PRE = 0, bool NTW = false, bool LINES = false, int MF = 0, int KBT = 0>
__global__ __launch_bounds__(NW * 64) void gemv_i8_kernel(GemvArgs a) {
    static_assert(!LINES || (ALIGNED && U % 2 == 0 && XMODE != 4), "whole-line loads: aligned, pairs of chunks");
    constexpr bool XLDS = XMODE != 0;
    constexpr int SLOTS = NW / KSPLIT;  // wave slots per workgroup, each CG column groups
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // [MT*16][kbytes+16] when XLDS
    __shared__ int red[KSPLIT > 1 ? NW : 1][CG * MT * 4][64];

    BH_STAMP(0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int slot = wave / KSPLIT;   // which column group of this workgroup
    const int ks = wave % KSPLIT;     // which K slice
    // MF, KBT (the decoder's and the decode sweep's launches): MF rows and
    // K = KBT bytes fixed at compile time, so the row loops and the K
    // batches fold away and the launch runs (and fetches) only the code of
    // its own shape (0: read from the arguments).
    const int m = MF ? MF : a.m, n = a.n;
    const int kbytes = KBT ? KBT : a.kg * 4;
    const int nchunks = (kbytes + 63) >> 6;
    const int ngroups = (n + 15) >> 4;
    const int xstride = kbytes + 16;
    const int ksub = (lane >> 4) * 16;  // this lane's 16-byte slice of a 64-byte chunk
    const int g0 = (blockIdx.x * SLOTS + slot) * CG;  // first of this wave's CG column groups
    if constexpr (XMODE == 0) {
        // moe_linear_gated_i8's early exit (moe_linear_gated_i8.wgsl:66-69)
        // for the whole launch: with no routed row at all the workgroup
        // stores its +0 outputs and reads no weights. (Otherwise every row
        // is multiplied, since the weights are streamed once for all rows,
        // and the epilogue zeroes the unrouted ones.)
        if (a.gate) {
            const bool live = lane < m && !(a.gate[(int64_t)lane * a.gate_stride + a.gate_col] <= 0.0f);
            if (!__any(live)) {
                for (int i = threadIdx.x; i < m * SLOTS * CG * 16; i += NW * 64) {
                    const int r = i / (SLOTS * CG * 16), c = blockIdx.x * SLOTS * CG * 16 + i % (SLOTS * CG * 16);
                    if (c < n) reinterpret_cast<float*>(a.out)[(int64_t)r * n + c] = 0.0f;
                }
                return;
            }
        }
    }

    const uint8_t* wp[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) {
        int wr = (g0 + c) * 16 + (lane & 15);
        wr = wr < n ? wr : n - 1;  // clamped rows are loaded but never stored
        wp[c] = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)wr * kbytes;
    }
    v4i wf[U][CG];
    // Chunks of this wave: ks + KSPLIT*j, or with LINES the pairs ks + KSPLIT*v.
    const int my_chunks = g0 < ngroups ? (LINES ? 2 * ((nchunks / 2 - ks + KSPLIT - 1) / KSPLIT)
                                                : (nchunks - ks + KSPLIT - 1) / KSPLIT)
                                       : 0;
    auto chunk_of = [&](int j) { return LINES ? 2 * (ks + KSPLIT * (j >> 1)) + (j & 1) : ks + KSPLIT * j; };
    const uint8_t* wl[LINES ? CG : 1][2];  // LINES: the lane's rows c%8 and 8 + c%8 of each group
    const int lineoff = ((lane & 15) < 8 ? 0 : 64) + ksub;
    if constexpr (LINES) {
#pragma unroll
        for (int c = 0; c < CG; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int wr = min((g0 + c) * 16 + 8 * h + (lane & 7), n - 1);
                wl[c][h] = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)wr * kbytes + lineoff;
            }
    }
    // Slot u (even) and u + 1 of pair `pr`: two whole-line loads.
    auto load_pair = [&](int u, int pr) {
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            wf[u][c] = load_w16<NTW>(wl[c][0] + pr * 128);
            wf[u + 1][c] = load_w16<NTW>(wl[c][1] + pr * 128);
        }
    };

    // The first batch of weight loads. Most launches issue it here, ahead of
    // the activation or the prologue's inputs. The SwiGLU prologue (XMODE 4)
    // issues it right after its own input loads and before their first use,
    // so its long chain (its inputs come from L2, the weights from HBM) runs
    // while the weights are in flight: vmcnt completes in order, so waiting
    // for inputs issued after the weights waits for the weights too.
    // Measured per launch: SwiGLU + down 8.56 -> 7.39 us at 4 rows, 5.44 ->
    // 5.32 at 1 row. The one-row norm launch takes the same order (batch-1
    // step 0.684 -> 0.644 ms, once its row loads had no branch join in front
    // of them); the four-row norm launch measured slower with it (batch 4
    // 0.940 -> 0.946 ms) and the one-row merge unchanged (0.6426 ms), so
    // they keep the weights first.
    // INFIRST: the prologue's input loads go out first, then the weights.
    constexpr bool INFIRST = XMODE == 4 || (XMODE == 3 && MF == 1);
    auto issue_w = [&]() {
        if constexpr (!INFIRST && LINES) {
#pragma unroll
            for (int u = 0; u < U; u += 2)
                if (u < my_chunks) load_pair(u, ks + KSPLIT * (u >> 1));
        } else if constexpr (!INFIRST) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (u < my_chunks)
#pragma unroll
                    for (int c = 0; c < CG; ++c)
                        wf[u][c] = load_wk16<ALIGNED, NTW>(wp[c], (ks + KSPLIT * u) * 64 + ksub, kbytes);
        } else {
            // Unconditional, and with no masking (this mode needs K % 64 ==
            // 0): slots past this wave's chunks reload its last one (never
            // consumed). A load under a branch, or a select on its value,
            // would leave the compiler unable to count it, and it would wait
            // for all of them before the prologue's first use of its inputs.
            // The scheduling barriers keep them after the prologue's loads
            // and ahead of its arithmetic (the scheduler would otherwise
            // interleave the independent loads).
            // A wave that owns no chunk (ks >= nchunks when K has fewer
            // chunks than the waves splitting it) reloads the row's last
            // chunk, so no load leaves the row.
            const int last = my_chunks > 0 ? my_chunks - 1 : 0;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int c = 0; c < CG; ++c)
                    wf[u][c] = load_w16<NTW>(wp[c] + min(ks + KSPLIT * min(u, last), nchunks - 1) * 64 + ksub);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (!INFIRST) issue_w();

    float* sxs = reinterpret_cast<float*>(xs + MT * 16 * xstride);  // XMODE 2-4: row scales
    if constexpr (XMODE == 3 || XMODE == 4) {
      if (XMODE == 4 && m == 1) {
        // One row (batch-1 decode): the whole workgroup shares it, one float4
        // of the SwiGLU output per thread (K <= 4096 and NW >= 4 waves give at
        // most four), instead of one group of 256 threads taking them all.
        // Elementwise the same arithmetic, and the row max is exact in any
        // order, so the codes and the scale are the ones below.
        constexpr int NTH = NW * 64, GX = (1024 + NTH - 1) / NTH;
        __shared__ float pm[NW];
        const int d = kbytes, d4 = d >> 2;
        const float4* g4 = reinterpret_cast<const float4*>(a.pre_a);
        const float4* u4 = g4 + d4;
        float4 h[GX], gv[GX], uv[GX];
        float am = 0.0f;
        // Unconditional loads (groups past K read a clamped copy), then the
        // weights, then the arithmetic.
#pragma unroll
        for (int gi = 0; gi < GX; ++gi) {
            const int i = min((int)threadIdx.x + NTH * gi, d4 - 1);
            gv[gi] = g4[i];
            uv[gi] = u4[i];
        }
        issue_w();
#pragma unroll
        for (int gi = 0; gi < GX; ++gi) {
            const int i = threadIdx.x + NTH * gi;
            h[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < d4) {
                const float4 g = gv[gi], u = uv[gi];
                h[gi] = make_float4(g.x / (1.0f + expf(-g.x)) * u.x, g.y / (1.0f + expf(-g.y)) * u.y,
                                    g.z / (1.0f + expf(-g.z)) * u.z, g.w / (1.0f + expf(-g.w)) * u.w);
                am = fmaxf(am, fmaxf(fmaxf(fabsf(h[gi].x), fabsf(h[gi].y)), fmaxf(fabsf(h[gi].z), fabsf(h[gi].w))));
            }
        }
        am = xor_max<32>(am);
        if (lane == 0) pm[wave] = am;
        __syncthreads();
        float rm = pm[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) rm = fmaxf(rm, pm[w]);
        const float sxv = fmaxf(rm, 1e-8f) / 127.0f;
        const float invq = 1.0f / sxv;
#pragma unroll
        for (int gi = 0; gi < GX; ++gi) {
            const int i = threadIdx.x + NTH * gi;
            if (i < d4) *reinterpret_cast<uint32_t*>(xs + 4 * i) = quant_word(h[gi], invq);
        }
        if (threadIdx.x < 4) *reinterpret_cast<uint32_t*>(xs + d + 4 * threadIdx.x) = 0u;  // pad past K
        if (threadIdx.x == 0) sxs[0] = sxv;
        __syncthreads();
      } else {
        // Rows in groups of 256 threads, NW/4 groups; each thread holds R
        // rows (group grp takes rows grp, grp + NG, ...), so up to NG * R
        // rows share one burst of loads and two barriers. The loads
        // are unconditional (rows past m and float4 groups past K read
        // clamped addresses and are zeroed afterwards): a load under a branch
        // gets its own wait, one memory round trip per row. The sum of
        // squares of a row uses exactly the reduction of the decoder's
        // separate norm_quant kernel -- thread t accumulates float4 groups t,
        // t+256, ... in order, a wave xor-tree, then the 4 wave sums in
        // order -- so the quantized rows are bit-identical to that kernel's.
        //   R (1, 2 or 4) and G are picked at run time, each case its own
        // unrolled code: the kernel runs once per decoder linear, so its
        // executed code is fetched cold every launch and must stay short.
        static_assert(NW % 4 == 0, "row groups of 4 waves");
        constexpr int NG = NW / 4;  // row groups
        __shared__ float gred[4][NW];
        __shared__ float gmx[4][NW];
        const int grp = wave >> 2, gt = threadIdx.x & 255;
        const int d = kbytes, d4 = d >> 2;
        const bool first = blockIdx.x == 0;
        // G: float4 groups per thread and row (K <= 1024 G); K <= 4096.
        auto rows = [&](auto gtag, auto rtag) {
            constexpr int G = decltype(gtag)::value;
            constexpr int RMAX = decltype(rtag)::value;
            // The norm weights (the same for every row) go out with the
            // first loads, not behind the reduction and the residual stores.
            float4 wv[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                wv[g] = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (XMODE == 3) wv[g] = reinterpret_cast<const float4*>(a.pre_w)[min(gt + 256 * g, d4 - 1)];
            }
            for (int r0 = 0; r0 < m; r0 += NG * RMAX) {
                float4 v[RMAX][G];
                int rc[RMAX];
#pragma unroll
                for (int j = 0; j < RMAX; ++j) rc[j] = min(r0 + grp + NG * j, m - 1);
                if constexpr (XMODE == 3) {
                    // Row sources: the token's embedding row (the first
                    // layer; a dependent load), else pre_a; then pre_b (the
                    // residual's delta), or the first source again. Both
                    // loads are unconditional: with a load in each branch
                    // the compiler waited at the join for every load in
                    // flight, the weights from HBM included, before issuing
                    // the next ones (two memory round trips instead of one).
                    const float* sa[RMAX];
                    const float* sb[RMAX];
                    if (a.pre_tok) {
#pragma unroll
                        for (int j = 0; j < RMAX; ++j) {
                            sa[j] = a.pre_emb + (size_t)a.pre_tok[rc[j]] * d;
                            sb[j] = sa[j];
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < RMAX; ++j) {
                            sa[j] = a.pre_a + (size_t)rc[j] * d;
                            sb[j] = a.pre_b ? a.pre_b + (size_t)rc[j] * d : sa[j];
                        }
                    }
                    float4 bv[RMAX][G];
#pragma unroll
                    for (int j = 0; j < RMAX; ++j)
#pragma unroll
                        for (int g = 0; g < G; ++g) {
                            const int ic = min(gt + 256 * g, d4 - 1);
                            v[j][g] = reinterpret_cast<const float4*>(sa[j])[ic];
                            bv[j][g] = reinterpret_cast<const float4*>(sb[j])[ic];
                        }
                    if constexpr (INFIRST)
                        if (r0 == 0) issue_w();
                    if (a.pre_b && !a.pre_tok) {
#pragma unroll
                        for (int j = 0; j < RMAX; ++j)
#pragma unroll
                            for (int g = 0; g < G; ++g)
                                v[j][g] = make_float4(v[j][g].x + bv[j][g].x, v[j][g].y + bv[j][g].y,
                                                      v[j][g].z + bv[j][g].z, v[j][g].w + bv[j][g].w);
                    }
                } else {
                    float4 uv[RMAX][G];
#pragma unroll
                    for (int j = 0; j < RMAX; ++j)
#pragma unroll
                        for (int g = 0; g < G; ++g) {
                            const int ic = min(gt + 256 * g, d4 - 1);
                            v[j][g] = reinterpret_cast<const float4*>(a.pre_a + (size_t)rc[j] * 2 * d)[ic];
                            uv[j][g] = reinterpret_cast<const float4*>(a.pre_a + (size_t)rc[j] * 2 * d + d)[ic];
                        }
                    if (r0 == 0) issue_w();
#pragma unroll
                    for (int j = 0; j < RMAX; ++j)
#pragma unroll
                        for (int g = 0; g < G; ++g) {
                            const float4 gv = v[j][g], u = uv[j][g];
                            v[j][g] = make_float4(gv.x / (1.0f + expf(-gv.x)) * u.x, gv.y / (1.0f + expf(-gv.y)) * u.y,
                                                  gv.z / (1.0f + expf(-gv.z)) * u.z, gv.w / (1.0f + expf(-gv.w)) * u.w);
                        }
                }
                // Rows past m and groups past K hold clamped copies: zero them.
#pragma unroll
                for (int j = 0; j < RMAX; ++j)
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        if (r0 + grp + NG * j >= m || gt + 256 * g >= d4) v[j][g] = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (XMODE == 3) {
#pragma unroll
                    for (int j = 0; j < RMAX; ++j) {
                        const int r = r0 + grp + NG * j;
                        float ss = 0.0f;
#pragma unroll
                        for (int g = 0; g < G; ++g) {
                            const float4 x = v[j][g];
                            ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
                            if (first && r < m && gt + 256 * g < d4)
                                reinterpret_cast<float4*>(a.res_out + (size_t)r * d)[gt + 256 * g] = x;
                        }
                        ss = xor_sum<32>(ss);
                        if (lane == 0) gred[j][wave] = ss;
                    }
                    __syncthreads();
#pragma unroll
                    for (int j = 0; j < RMAX; ++j) {
                        float tot = gred[j][grp * 4];
#pragma unroll
                        for (int w = 1; w < 4; ++w) tot += gred[j][grp * 4 + w];
                        const float inv = 1.0f / sqrtf(tot / (float)d + a.eps);
                        const bool live = r0 + grp + NG * j < m;
#pragma unroll
                        for (int g = 0; g < G; ++g)
                            if (live && gt + 256 * g < d4)
                                v[j][g] = make_float4(v[j][g].x * inv * wv[g].x, v[j][g].y * inv * wv[g].y,
                                                      v[j][g].z * inv * wv[g].z, v[j][g].w * inv * wv[g].w);
                    }
                }
#pragma unroll
                for (int j = 0; j < RMAX; ++j) {
                    float am = 0.0f;
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        am = fmaxf(am, fmaxf(fmaxf(fabsf(v[j][g].x), fabsf(v[j][g].y)),
                                             fmaxf(fabsf(v[j][g].z), fabsf(v[j][g].w))));
                    am = xor_max<32>(am);
                    if (lane == 0) gmx[j][wave] = am;
                }
                __syncthreads();
#pragma unroll
                for (int j = 0; j < RMAX; ++j) {
                    const int r = r0 + grp + NG * j;
                    if (r >= m) continue;
                    float rm = gmx[j][grp * 4];
#pragma unroll
                    for (int w = 1; w < 4; ++w) rm = fmaxf(rm, gmx[j][grp * 4 + w]);
                    const float sxv = fmaxf(rm, 1e-8f) / 127.0f;
                    const float invq = 1.0f / sxv;
                    uint8_t* xr8 = xs + r * xstride;
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const int i = gt + 256 * g;
                        if (i < d4) *reinterpret_cast<uint32_t*>(xr8 + 4 * i) = quant_word(v[j][g], invq);
                    }
                    if (gt < 4) *reinterpret_cast<uint32_t*>(xr8 + d + 4 * gt) = 0u;  // pad past K
                    if (gt == 0) sxs[r] = sxv;
                }
                __syncthreads();  // the rows are in LDS for every wave; gred / gmx are reused by the next round
            }
        };
        auto by_k = [&](auto rtag) {
            if (d4 <= 256) rows(std::integral_constant<int, 1>{}, rtag);
            else if (d4 <= 512) rows(std::integral_constant<int, 2>{}, rtag);
            else if (d4 <= 768) rows(std::integral_constant<int, 3>{}, rtag);
            else rows(std::integral_constant<int, 4>{}, rtag);
        };
        if constexpr (PRE != 0) {
            rows(std::integral_constant<int, PRE % 8>{}, std::integral_constant<int, PRE / 8>{});
        } else {
            if (m <= NG) by_k(std::integral_constant<int, 1>{});
            else if (m <= 2 * NG) by_k(std::integral_constant<int, 2>{});
            else by_k(std::integral_constant<int, 4>{});
        }
      }
    } else if constexpr (XMODE == 2) {
        // Each row is split across wpr = NW/m waves (1 when m >= NW): partial
        // maxima meet in LDS, then every wave quantizes its share of the row.
        __shared__ float pmax[NW];
        const int k4 = kbytes >> 2;
        const int wpr = m < NW ? NW / m : 1;
        const int rows_per_round = NW / wpr;
        const bool first = blockIdx.x == 0;
        for (int r0 = 0; r0 < m; r0 += rows_per_round) {
            const int r = r0 + wave / wpr, part = wave % wpr;
            const float4* xr = reinterpret_cast<const float4*>(a.x + (int64_t)(r < m ? r : 0) * kbytes);
            float mx = 0.0f;
            if (r < m)
                for (int c = part * 64 + lane; c < k4; c += wpr * 64) {
                    const float4 v = xr[c];
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            mx = xor_max<32>(mx);
            if (lane == 0) pmax[wave] = mx;
            __syncthreads();
            if (r < m) {
                float rm = pmax[(wave / wpr) * wpr];
                for (int j = 1; j < wpr; ++j) rm = fmaxf(rm, pmax[(wave / wpr) * wpr + j]);
                const float sxv = fmaxf(rm, 1e-8f) / 127.0f;
                const float inv = 1.0f / sxv;
                uint8_t* xr8 = xs + r * xstride;
                for (int c = part * 64 + lane; c < k4; c += wpr * 64) {
                    const uint32_t w = quant_word(xr[c], inv);
                    *reinterpret_cast<uint32_t*>(xr8 + 4 * c) = w;
                    if (first) a.xq_out[(int64_t)r * k4 + c] = w;
                }
                if (part == 0 && lane < 4) *reinterpret_cast<uint32_t*>(xr8 + kbytes + 4 * lane) = 0u;  // pad past K
                if (part == 0 && lane == 0) {
                    sxs[r] = sxv;
                    if (first) a.sx_out[r] = sxv;
                }
            }
            __syncthreads();  // pmax is reused by the next round
        }
    } else if constexpr (XMODE == 5) {
        // Rows one at a time, the whole workgroup on each: every thread merges
        // one 4-element context group (the partial loads go out before the
        // row's position is read), then the row's int8 quantization. The same
        // operations as the separate merge kernel (attn_combine_first4, the
        // row max exact in any order), so the codes and scales are its own.
        // K <= 2048 (launch_gemv_i8_merge): one group per thread from 8 waves,
        // which keeps a thread's 16 preloaded chunk slots in registers.
        // PRE == 2 (HEAD32): head_dim 128, K = 2048 and at most ATTN_SB
        // chunks (512 positions), on 8 waves, so every
        // lane holds one context group and each head is one half-wave; the
        // chunk statistics are loaded and the chunk weights evaluated once
        // per chunk (attn_combine_head32) instead of on every lane of the
        // head (16 of the exponentials' ~14 instructions each per lane
        // before). The same results.
        constexpr int NTH = NW * 64, GX = (512 + NTH - 1) / NTH;
        constexpr bool HEAD32 = PRE == 2;
        static_assert(!HEAD32 || (NTH == 512 && GX == 1), "one context group per lane");
        __shared__ float pm[NW];
        const int q4 = kbytes >> 2;
        for (int r = 0; r < m; ++r) {
            AttnFirst4 fb[GX];
            size_t hs[GX];
            int dd[GX];
            bool live[GX];
#pragma unroll
            for (int gi = 0; gi < GX; ++gi) {
                const int i = threadIdx.x + NTH * gi;
                live[gi] = i < q4;
                const int e = (live[gi] ? i : 0) * 4, h = e / a.hd;
                dd[gi] = e - h * a.hd;
                hs[gi] = ((size_t)r * a.nh + h) * a.splits;
                // HEAD32: only the row's live chunks (its position is read
                // first; a uniform bound).
                if constexpr (HEAD32) attn_load_first4_o(a.part_o, hs[gi], min(((int)a.pos[r] + ATTN_KCH) / ATTN_KCH, a.splits), dd[gi], a.hd, fb[gi]);
                else attn_load_first4(a.part_o, a.part_ml, hs[gi], live[gi] ? a.splits : 0, dd[gi], a.hd, fb[gi]);
            }
            // HEAD32: lane q of each half-wave loads chunk q's (m, l).
            float2 mlq = make_float2(0.f, 0.f);
            if constexpr (HEAD32)
                mlq = reinterpret_cast<const float2*>(a.part_ml)[hs[0] + min((int)(lane & 31), a.splits - 1)];
            const int ns = ((int)a.pos[r] + ATTN_KCH) / ATTN_KCH;
            float4 y[GX];
            float am = 0.0f;
#pragma unroll
            for (int gi = 0; gi < GX; ++gi) {
                y[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (HEAD32) {
                    y[gi] = attn_combine_head32(mlq, ns, fb[gi]);  // splits <= ATTN_SB
                    am = fmaxf(am, fmaxf(fmaxf(fabsf(y[gi].x), fabsf(y[gi].y)), fmaxf(fabsf(y[gi].z), fabsf(y[gi].w))));
                } else if (live[gi]) {
                    y[gi] = attn_combine_first4(a.part_o, a.part_ml, hs[gi], ns, dd[gi], a.hd, fb[gi]);
                    am = fmaxf(am, fmaxf(fmaxf(fabsf(y[gi].x), fabsf(y[gi].y)), fmaxf(fabsf(y[gi].z), fabsf(y[gi].w))));
                }
            }
            am = xor_max<32>(am);
            if (lane == 0) pm[wave] = am;
            __syncthreads();
            float rm = pm[0];
#pragma unroll
            for (int w = 1; w < NW; ++w) rm = fmaxf(rm, pm[w]);
            const float sxv = fmaxf(rm, 1e-8f) / 127.0f;
            const float invq = 1.0f / sxv;
            uint8_t* xr8 = xs + r * xstride;
#pragma unroll
            for (int gi = 0; gi < GX; ++gi) {
                const int i = threadIdx.x + NTH * gi;
                if (live[gi]) *reinterpret_cast<uint32_t*>(xr8 + 4 * i) = quant_word(y[gi], invq);
            }
            if (threadIdx.x < 4) *reinterpret_cast<uint32_t*>(xr8 + kbytes + 4 * threadIdx.x) = 0u;  // pad past K
            if (threadIdx.x == 0) sxs[r] = sxv;
            __syncthreads();  // pm is reused by the next row; xs and sxs are complete
        }
    } else if constexpr (XLDS) {
        const int pieces = kbytes >> 4;
        const int total = MT * 16 * pieces;
        for (int p = threadIdx.x; p < total; p += NW * 64) {
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
            if (kb >= kbytes || (XMODE >= 2 && r >= m)) return v4i{0, 0, 0, 0};
            return *reinterpret_cast<const v4i*>(xs + r * xstride + kb);
        } else {
            if (r >= m) return v4i{0, 0, 0, 0};
            return load_k16<ALIGNED>(reinterpret_cast<const uint8_t*>(a.xq) + (int64_t)r * kbytes, kb, kbytes);
        }
    };

    // Epilogue operands fetched up front, off the critical path: the scale
    // of every row (MT*4 per lane) and of this lane's column in each group.
    float sxr[MT * 4], swc[CG];
#pragma unroll
    for (int ri = 0; ri < MT * 4; ++ri) {
        const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
        sxr[ri] = (OUT != OUT_I32 && row < m) ? (XMODE >= 2 ? sxs[row] : a.sx[row]) : 0.0f;
    }
#pragma unroll
    for (int c = 0; c < CG; ++c) {
        const int col = (g0 + c) * 16 + (lane & 15);
        swc[c] = (OUT != OUT_I32 && col < n) ? a.sw[col] : 0.0f;
    }

    v4i acc[CG][MT];
#pragma unroll
    for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[c][t] = v4i{0, 0, 0, 0};
    // One batch of U chunks: activation fragments, then the MFMAs. The first
    // batch is peeled out of the loop so that its activation loads issue
    // right behind the weight loads already in flight: inside the loop the
    // compiler waits for every outstanding load at the loop header, which
    // made the activation a second memory round trip.
    auto batch = [&](int j0) {
        v4i xf[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                xf[u][t] = (j0 + u < my_chunks) ? xfrag(t, chunk_of(j0 + u) * 64 + ksub) : v4i{0, 0, 0, 0};
        if constexpr (LINES) {
            // Lane (c, j) holds row c%8 (first load) or 8 + c%8 (second);
            // the MFMA wants row c, chunk j of the pair's first 64 bytes,
            // then of its second.
            const bool lo = (lane & 15) < 8;
#pragma unroll
            for (int u = 0; u < U; u += 2)
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    v4i r0, r1;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        r0[d] = __builtin_amdgcn_mov_dpp(wf[u][c][d], 0x128, 0xF, 0xF, false);
                        r1[d] = __builtin_amdgcn_mov_dpp(wf[u + 1][c][d], 0x128, 0xF, 0xF, false);
                    }
                    const v4i w0 = lo ? wf[u][c] : r1, w1 = lo ? r0 : wf[u + 1][c];
                    wf[u][c] = w0;
                    wf[u + 1][c] = w1;
                }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (j0 + u < my_chunks)
#pragma unroll
                for (int c = 0; c < CG; ++c)
#pragma unroll
                    for (int t = 0; t < MT; ++t)
                        acc[c][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xf[u][t], wf[u][c], acc[c][t], 0, 0, 0);
    };
    BH_STAMP(1);
    batch(0);
#pragma unroll 1
    for (int j0 = U; j0 < my_chunks; j0 += U) {
        if constexpr (LINES) {
#pragma unroll
            for (int u = 0; u < U; u += 2)
                if (j0 + u < my_chunks) load_pair(u, ks + KSPLIT * ((j0 + u) >> 1));
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (j0 + u < my_chunks)
#pragma unroll
                    for (int c = 0; c < CG; ++c)
                        wf[u][c] = load_wk16<ALIGNED, NTW>(wp[c], (ks + KSPLIT * (j0 + u)) * 64 + ksub, kbytes);
        }
        batch(j0);
    }
    BH_STAMP(2);

    // Lane l, register i of a 16x16 i32 result holds row 4*(l/16)+i, column l%16.
    auto emit = [&](int c, int ri, int s) {
        const int col = (g0 + c) * 16 + (lane & 15);
        const int row = 16 * (ri >> 2) + 4 * (lane >> 4) + (ri & 3);
        if (row < m && col < n) {
            const int64_t idx = (int64_t)row * n + col;
            if constexpr (OUT == OUT_I32) {
                reinterpret_cast<int*>(a.out)[idx] = s;
            } else {
                float v = dequant(s, sxr[ri], swc[c]);
                if constexpr (HAS_BIAS) v = v + a.bias[col];
                if (a.gate && a.gate[(int64_t)row * a.gate_stride + a.gate_col] <= 0.0f) v = 0.0f;
                store_out<OUT>(a.out, idx, v);
            }
        }
    };
    if constexpr (KSPLIT == 1) {
#pragma unroll
        for (int c = 0; c < CG; ++c)
            if (g0 + c < ngroups)
#pragma unroll
                for (int ri = 0; ri < MT * 4; ++ri) emit(c, ri, acc[c][ri >> 2][ri & 3]);
    } else {
#pragma unroll
        for (int c = 0; c < CG; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][(c * MT + t) * 4 + i][lane] = acc[c][t][i];
        __syncthreads();
        BH_STAMP(3);
        for (int q = ks; q < CG * MT * 4; q += KSPLIT) {
            const int c = q / (MT * 4), ri = q % (MT * 4);
            if (g0 + c >= ngroups) continue;
            int s = 0;
#pragma unroll
            for (int w = 0; w < KSPLIT; ++w) s += red[slot * KSPLIT + w][q][lane];
            emit(c, ri, s);
        }
    }
    BH_STAMP(4);
}

// Wide N (the LM head: thousands of 16-column groups), m <= 16: a resident
// grid streams W. Each wave owns every nwaves-th column group (an equal share)
// and covers the whole K of each, so there is no cross-wave sum and no
// barrier after the prologue. The packed activation is staged in LDS once
// per workgroup (its loads go out ahead of the first weights), so the
// L2 serves m*K bytes per workgroup instead of per column group. A wave keeps
// the weight loads of its next work item in flight while it multiplies the
// current one (two register sets, alternating), and the column scale of an
// item is loaded ahead of its weights, so no wait in the loop drains the
// memory pipe. Work items are (column group, batch of U = 16 64-byte K
// chunks); K (= KB bytes) is a compile-time multiple of 1024.
// Measured on MI355X (LM head, cold): two waves per SIMD (256 VGPRs, fewer
// parked results) was slower than this form (one wave per SIMD, 288 VGPRs
// with the accumulation registers).
// LINES: every weight load covers whole 128-byte lines (8 rows x 128 bytes)
// with the non-temporal hint, and a row_ror:8 lane exchange puts the values
// into the MFMA's layout (which alone would read 16 rows x 64 bytes per load,
// each line split over two loads). On the configs[1] sweep (cold weights):
// the LM head 29.3-29.5 -> 28.1-28.7 us and the 16-launch average 10.19-10.21
// -> 9.52 us; the non-temporal hint on the split-line layout was 2-3.5 us
// slower, whole lines without the hint slower too (30.6-31.0 us). The Qwen3
// engine's head, re-read every step, keeps the ordinary loads
// (GemvArgs::keep_cached).
// Q4: W4A8 weights (matmul_q4_gemv, crates/kernels/wgsl/matmul_q4_gemv.wgsl):
// rows of KB/2 bytes, 8 int4 per u32 word; per 128-K chunk each lane loads 16
// bytes of int4 (K 32q..32q+31 of its column, q = lane/16), unpacks them to
// two int8 fragments and feeds two MFMAs against the activation bytes of the
// same K (a permutation of K inside the chunk shared by both operands, so the
// sum is exact; the same pairing as gemv_q4_kernel).
__device__ __forceinline__ bool argmax_better(float v, uint32_t i, float bv, uint32_t bi) {
    if (i == 0xffffffffu) return false;
    if (bi == 0xffffffffu) return true;
    return v > bv || (v == bv && i < bi);
}

template <int OUT, bool HAS_BIAS, int KB, bool Q4 = false, bool LINES = false, bool AM = false>
__global__ __launch_bounds__(256) void gemv_i8_stream_kernel(GemvArgs a, int groups_per_wave) {
    static_assert(!AM || OUT == OUT_F32, "argmax over f32 outputs");
    constexpr int U = Q4 ? 8 : 16, kbytes = KB, nbatch = KB / 1024;
    constexpr int wbytes = Q4 ? KB / 2 : KB;  // weight bytes per row
    __shared__ __attribute__((aligned(16))) uint8_t xs[16 * (KB + 16)];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int m = a.m, n = a.n;
    const int ngroups = (n + 15) >> 4;
    constexpr int xstride = kbytes + 16;
    const int ksub = (lane >> 4) * 16;
    const int nwaves = gridDim.x * 4;
    const int gw = blockIdx.x * 4 + wave;
    // This wave's groups: gw + i * nwaves for i < ng.
    int ng = gw < ngroups ? (ngroups - 1 - gw) / nwaves + 1 : 0;
    ng = ng < groups_per_wave ? ng : groups_per_wave;
    const int items = ng * nbatch;

    struct Item {
        v4i w[U];
        float sw, bias;
    };
    auto load_item = [&](Item& it, int j) {
        const int i = j / nbatch, b = j - i * nbatch;
        const int g = gw + i * nwaves;
        int r = g * 16 + (lane & 15);
        r = r < n ? r : n - 1;  // clamped rows are loaded but never stored
        if (b == 0) {
            it.sw = OUT != OUT_I32 ? a.sw[r] : 0.0f;
            it.bias = HAS_BIAS ? a.bias[r] : 0.0f;
        }
        if constexpr (LINES) {
            // Whole 128-byte lines per load (Q4 too: its 64-byte blocks are
            // 128 K of int4): the pair (u, u+1) of k-blocks is
            // two loads, rows 0-7 then rows 8-15 of the group, lane (c, j)
            // (c = lane % 16, j = lane / 16) reading 16 bytes of row c % 8 at
            // chunk j (c < 8) or 4 + j (c >= 8) of the 128 bytes. consume()
            // moves them into the MFMA layout with a row_ror:8 exchange.
            const int c = lane & 15;
            const int off = b * U * 64 + (c < 8 ? ksub : 64 + ksub);
            const int r0 = min(g * 16 + (c & 7), n - 1), r1 = min(g * 16 + 8 + (c & 7), n - 1);
            const uint8_t* p0 = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)r0 * wbytes + off;
            const uint8_t* p1 = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)r1 * wbytes + off;
#pragma unroll
            for (int u = 0; u < U; u += 2) {
                it.w[u] = load_w16<true>(p0 + u * 64);
                it.w[u + 1] = load_w16<true>(p1 + u * 64);
            }
        } else {
            const uint8_t* rp = reinterpret_cast<const uint8_t*>(a.wq) + (int64_t)r * wbytes + b * U * 64 + ksub;
#pragma unroll
            for (int u = 0; u < U; ++u) it.w[u] = *reinterpret_cast<const v4i*>(rp + u * 64);
        }
    };

    // Activation image: 16 rows plus a 16-byte pad per row. Rows >= m repeat
    // row 0: they only feed accumulator rows that are never stored, and an
    // unconditional load keeps the compiler from turning it into a branch
    // (which would make it wait for the weights). Every thread loads its
    // kbytes/256 pieces first, then its first item's weights, and waits only
    // for the pieces before the LDS writes.
    constexpr int pieces = kbytes >> 4, nst = kbytes >> 8;
    v4i st[nst];
#pragma unroll
    for (int i = 0; i < nst; ++i) {
        const int p = threadIdx.x + 256 * i;
        const int r = p / pieces, c = p - r * pieces;
        st[i] = *reinterpret_cast<const v4i*>(reinterpret_cast<const uint8_t*>(a.xq) +
                                              (int64_t)(r < m ? r : 0) * kbytes + c * 16);
    }
    Item ia, ib;
    load_item(ia, 0);  // unconditional (rows clamped), so the waits below count only the pieces
#pragma unroll
    for (int i = 0; i < nst; ++i) {
        const int p = threadIdx.x + 256 * i;
        const int r = p / pieces, c = p - r * pieces;
        *reinterpret_cast<v4i*>(xs + r * xstride + c * 16) = st[i];
    }
    if (threadIdx.x < 16) *reinterpret_cast<v4i*>(xs + threadIdx.x * xstride + kbytes) = v4i{0, 0, 0, 0};
    float sxr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        sxr[i] = (OUT != OUT_I32 && row < m) ? a.sx[row] : 0.0f;
    }
    __syncthreads();
    // Argmax partials: this lane's best column for each of its 4 rows.
    float amv[4] = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
    uint32_t ami[4] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    auto am_store = [&]() {
        if constexpr (AM) {
            auto step = [&](int q, auto off) {
                const float ov = xor_lane<decltype(off)::value>(amv[q]);
                const uint32_t oi = xor_lane_u<decltype(off)::value>(ami[q]);
                if (argmax_better(ov, oi, amv[q], ami[q])) {
                    amv[q] = ov;
                    ami[q] = oi;
                }
            };
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                step(q, std::integral_constant<int, 8>{});
                step(q, std::integral_constant<int, 4>{});
                step(q, std::integral_constant<int, 2>{});
                step(q, std::integral_constant<int, 1>{});
            }
            if ((lane & 15) == 0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row = 4 * (lane >> 4) + q;
                    if (row < m) {
                        a.am_v[(int64_t)row * a.am_stride + gw] = amv[q];
                        a.am_i[(int64_t)row * a.am_stride + gw] = ami[q];
                    }
                }
            }
            if (gw == 0 && lane == 0) *a.am_n = (uint32_t)nwaves;
        }
    };
    if (items == 0) {
        am_store();
        return;
    }

    const uint8_t* xrow = xs + (lane & 15) * xstride + (Q4 ? 2 * ksub : ksub);
    v4i acc = {0, 0, 0, 0};
    // Results of the last npend groups (slot k = group i_last - k), not yet stored.
    constexpr int NPEND = 8;
    using PendT = typename std::conditional<OUT == OUT_I32, int, float>::type;
    PendT pend[NPEND][4];
#pragma unroll
    for (int k = 0; k < NPEND; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) pend[k][q] = 0;  // defined values: the shift below reads every slot
    int npend = 0;
    auto flush = [&](int i_last) {
#pragma unroll
        for (int k = 0; k < NPEND; ++k) {
            if (k < npend) {
                const int col = (gw + (i_last - k) * nwaves) * 16 + (lane & 15);
                if (col < n) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int row = 4 * (lane >> 4) + q;
                        if (row < m) {
                            const int64_t idx = (int64_t)row * n + col;
                            if constexpr (OUT == OUT_I32) reinterpret_cast<int*>(a.out)[idx] = pend[k][q];
                            else store_out<OUT>(a.out, idx, pend[k][q]);
                        }
                    }
                }
            }
        }
        npend = 0;
    };
    auto consume = [&](const Item& it, int j) {
        const int i = j / nbatch, b = j - i * nbatch;
        if constexpr (Q4) {
            const uint8_t* xp = xrow + b * U * 128;
            v4i wq4[U];
            if constexpr (LINES) {
                // The same exchange as below, then the int4 unpack.
                const bool lo = (lane & 15) < 8;
#pragma unroll
                for (int u = 0; u < U; u += 2) {
                    v4i r0, r1;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        r0[d] = __builtin_amdgcn_mov_dpp(it.w[u][d], 0x128, 0xF, 0xF, false);
                        r1[d] = __builtin_amdgcn_mov_dpp(it.w[u + 1][d], 0x128, 0xF, 0xF, false);
                    }
                    wq4[u] = lo ? it.w[u] : r1;
                    wq4[u + 1] = lo ? r0 : it.w[u + 1];
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) wq4[u] = it.w[u];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                v4i b0, b1;
                unpack_q4x4(wq4[u], b0, b1);
                const v4i x0 = *reinterpret_cast<const v4i*>(xp + u * 128);
                const v4i x1 = *reinterpret_cast<const v4i*>(xp + u * 128 + 16);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, b0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, b1, acc, 0, 0, 0);
            }
        } else if constexpr (LINES) {
            // Lane (c, j) holds row c%8 (first load) or 8 + c%8 (second) of
            // the group; the MFMA wants row c, chunk j for block u and chunk
            // 4 + j for block u+1. row_ror:8 swaps the two 8-lane halves of
            // each 16-lane row.
            const uint8_t* xp = xrow + b * U * 64;
            const bool lo = (lane & 15) < 8;
#pragma unroll
            for (int u = 0; u < U; u += 2) {
                v4i r0, r1;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    r0[d] = __builtin_amdgcn_mov_dpp(it.w[u][d], 0x128, 0xF, 0xF, false);
                    r1[d] = __builtin_amdgcn_mov_dpp(it.w[u + 1][d], 0x128, 0xF, 0xF, false);
                }
                const v4i w0 = lo ? it.w[u] : r1;
                const v4i w1 = lo ? r0 : it.w[u + 1];
                const v4i x0 = *reinterpret_cast<const v4i*>(xp + u * 64);
                const v4i x1 = *reinterpret_cast<const v4i*>(xp + (u + 1) * 64);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, w0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, w1, acc, 0, 0, 0);
            }
        } else {
            const uint8_t* xp = xrow + b * U * 64;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const v4i xf = *reinterpret_cast<const v4i*>(xp + u * 64);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xf, it.w[u], acc, 0, 0, 0);
            }
        }
        if (b != nbatch - 1) return;
        // Park the group's results; the stores go out in bursts of NPEND
        // groups (at the end of the wave for the LM head). A store in the loop
        // would sit in the in-order vmcnt queue ahead of the next item's
        // weights, so the next wait would also wait for its write ack.
#pragma unroll
        for (int k = NPEND - 1; k > 0; --k)
#pragma unroll
            for (int q = 0; q < 4; ++q) pend[k][q] = pend[k - 1][q];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (OUT == OUT_I32) {
                pend[0][q] = acc[q];
            } else {
                float v = dequant(acc[q], sxr[q], it.sw);
                if constexpr (HAS_BIAS) v = v + it.bias;
                pend[0][q] = v;
                if constexpr (AM) {
                    // Columns arrive in increasing order: a strictly larger
                    // value keeps the first index of the maximum.
                    const int col = (gw + i * nwaves) * 16 + (lane & 15);
                    if (col < n && v > amv[q]) {
                        amv[q] = v;
                        ami[q] = (uint32_t)col;
                    }
                }
            }
        }
        acc = v4i{0, 0, 0, 0};
        if (++npend == NPEND || i == ng - 1) flush(i);
    };
    // Two register sets: item j in ia (j even) or ib (j odd).
#pragma unroll 1
    for (int j = 0;; j += 2) {
        if (j + 1 >= items) {
            consume(ia, j);
            break;
        }
        load_item(ib, j + 1);
        consume(ia, j);
        if (j + 2 >= items) {
            consume(ib, j + 1);
            break;
        }
        load_item(ia, j + 2);
        consume(ib, j + 1);
    }
    am_store();
}

// ---------------------------------------------------------------- host side

static int gv_cfg() {
    static int v = [] {
        const char* e = getenv("BH_GEMV_CFG");
        return e ? atoi(e) : 0;
    }();
    return v;
}

template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED, int U, int CG, int KSPLIT = 4, int XMODE = 0, int PRE = 0,
          bool NTW = false, bool LINES = false, int MF = 0, int KBT = 0>
static hipError_t gv_go(hipStream_t s, const GemvArgs& a) {
    constexpr int NW = KSPLIT > GV_WAVES ? KSPLIT : GV_WAVES;  // waves per workgroup
    constexpr int per_wg = (NW / KSPLIT) * CG;
    const int ngroups = (a.n + 15) / 16;
    const int grid = (ngroups + per_wg - 1) / per_wg;
    const size_t lds = XMODE ? (size_t)MT * 16 * (a.kg * 4 + 16) + MT * 16 * 4 : 0;
    if ((MF && a.m != MF) || (KBT && a.kg * 4 != KBT)) return hipErrorInvalidValue;
    gemv_i8_kernel<MT, OUT, HAS_BIAS, ALIGNED, KSPLIT, XMODE, U, CG, NW, PRE, NTW, LINES, MF, KBT><<<grid, NW * 64, lds, s>>>(a);
    return hipGetLastError();
}

// The streaming wide-N kernel: as many waves as can be resident (so the
// whole grid is one round), each owning an equal share of the column groups.
template <int OUT, bool HAS_BIAS, int KB, bool Q4 = false, bool LINES = false, bool AM = false>
static hipError_t gv_stream_kb(hipStream_t s, const GemvArgs& a) {
    // Resident waves (the whole grid is one round).
    static const int slots = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_i8_stream_kernel<OUT, HAS_BIAS, KB, Q4, LINES, AM>, 256,
                                                         0) !=
                hipSuccess || per_cu < 1)
            per_cu = 1;
        return cus * per_cu * 4;
    }();
    const int ngroups = (a.n + 15) / 16;
    const int gpw = (ngroups + slots - 1) / slots;  // groups per wave
    const int waves = (ngroups + gpw - 1) / gpw;    // balanced: every wave gpw or gpw-1 groups
    if (AM && ((waves + 3) / 4) * 4 > a.am_stride) return hipErrorInvalidValue;
    gemv_i8_stream_kernel<OUT, HAS_BIAS, KB, Q4, LINES, AM><<<(waves + 3) / 4, 256, 0, s>>>(a, gpw);
    return hipGetLastError();
}

// The streaming wide-N kernel, instantiated for K = 1024 bytes (the LM head
// of the 1024-wide decoder), m <= 16.
template <int OUT, bool HAS_BIAS>
static hipError_t gv_stream(hipStream_t s, const GemvArgs& a) {
    if constexpr (OUT == OUT_F32 && !HAS_BIAS) {
        if (a.am_v) return gv_stream_kb<OUT, HAS_BIAS, 1024, false, false, true>(s, a);
    }
    if (a.am_v) return hipErrorNotSupported;
    if (a.keep_cached) return gv_stream_kb<OUT, HAS_BIAS, 1024>(s, a);
    return gv_stream_kb<OUT, HAS_BIAS, 1024, false, true>(s, a);
}

// Launch policy (measured on MI355X with rotating >256 MB weight pools):
//  - wide N (>= 1024 column groups, e.g. the LM head): each wave covers two
//    column groups (four above 8 rows), cutting activation (L2) traffic per
//    weight byte; batches
//    of 4 K-chunks keep VGPRs low (8 waves/SIMD) so ~16 KB per workgroup is
//    in flight across many resident workgroups;
//  - narrow N: one column group per wave; when a wave owns more than 4
//    K-chunks (few workgroups, long K) it issues up to 16 at once, so the
//    whole weight slice is a single memory round trip.
template <int MT, int OUT, bool HAS_BIAS, bool ALIGNED>
static hipError_t gv_split(hipStream_t s, const GemvArgs& a) {
    const int ngroups = (a.n + 15) / 16;
    const int wave_chunks = ((a.kg * 4 + 63) / 64 + 3) / 4;
    switch (gv_cfg()) {  // tuning override (BH_GEMV_CFG), 0 = policy
        case 1: return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1>(s, a);
        case 2: return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 2>(s, a);
        case 3: return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 16, 1>(s, a);
        case 4: return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1, 4>(s, a);
        default: break;
    }
    if (ngroups >= 1024 && MT == 1 && a.kg == 256 && !a.gate && gv_cfg() != 9) return gv_stream<OUT, HAS_BIAS>(s, a);
    // More than 8 rows: four column groups per wave (activation reads a
    // quarter of the weight reads; 4.5% faster on the LM head at m = 16,
    // 15% slower at m = 1).
    if (ngroups >= 1024) {
        if (a.m > 8) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 4>(s, a);
        return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 2>(s, a);
    }
    // Narrow N: split K 8 or 16 ways inside one workgroup (512 / 1024 threads)
    // so the grid holds ~1000+ waves instead of N/16 x 4. At exactly 16
    // K-chunks (K = 1024) 4 waves of 4 chunks measured 1-2% faster than 8 of 2
    // on every K = 1024 shape of the decode sweep.
    const int nchunks = (a.kg * 4 + 63) / 64;
    // K = 3072 and 2048: 8 waves of 6 / 4 chunks rather than 16 of 3 / 2
    // (batch-8 decode step 1.2137 -> 1.208 ms, batch 4 1.085 -> 1.082; the
    // configs[1] K = 3072 shapes 0.05-0.1 us faster each; 4 waves of 12 / 8
    // chunks measured 0.02-0.04 us slower than 8 waves on the same shapes).
    if (nchunks == 48) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 6, 1, 8>(s, a);
    if (nchunks == 32) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1, 8>(s, a);
    if (nchunks >= 32) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1, 16>(s, a);
    if (nchunks > 16) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1, 8>(s, a);
    if (wave_chunks > 4) return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 16, 1>(s, a);
    return gv_go<MT, OUT, HAS_BIAS, ALIGNED, 4, 1>(s, a);
}

// Quantization fused into the GEMV (XMODE 2), same launch policy as gv_split.
template <int MT, int OUT, bool HAS_BIAS>
static hipError_t gv_fused(hipStream_t s, const GemvArgs& a) {
    const int ngroups = (a.n + 15) / 16;
    const int nchunks = (a.kg * 4 + 63) / 64;
    (void)ngroups;
    if (nchunks >= 32) return gv_go<MT, OUT, HAS_BIAS, true, 4, 1, 16, 2>(s, a);
    if (nchunks >= 16) return gv_go<MT, OUT, HAS_BIAS, true, 4, 1, 8, 2>(s, a);
    return gv_go<MT, OUT, HAS_BIAS, true, 4, 1, 4, 2>(s, a);
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

// The W4A8 LM head on the streaming kernel: K = 1024, m <= 16, wide N (at
// least 1024 column groups), 16-byte aligned operands; hipErrorNotSupported
// otherwise (the caller keeps its own GEMV).
hipError_t launch_gemv_q4_stream(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                 const float* sw, const float* bias, void* out, int out_dtype, int m, int k, int n) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq);
    if (k != 1024 || m < 1 || m > 16 || (n + 15) / 16 < 1024 || (al & 15u) != 0 || gv_cfg() == 9)
        return hipErrorNotSupported;
    GemvArgs a{xq, wq, sx, sw, bias, out, m, k / 4, n, nullptr, 0, 0, nullptr, nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f};
    if (out_dtype == OUT_I32) return gv_stream_kb<OUT_I32, false, 1024, true, true>(s, a);
    if (out_dtype == OUT_F32)
        return bias ? gv_stream_kb<OUT_F32, true, 1024, true, true>(s, a) : gv_stream_kb<OUT_F32, false, 1024, true, true>(s, a);
    return bias ? gv_stream_kb<OUT_BF16, true, 1024, true, true>(s, a) : gv_stream_kb<OUT_BF16, false, 1024, true, true>(s, a);
}

// Preconditions are checked by the C-ABI layer: 1 <= m <= 32, kg >= 0, n >= 1.
hipError_t launch_gemv_i8(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                          const float* sw, const float* bias, void* out, int out_dtype, int m, int kg, int n,
                          bool keep_cached = false, float* am_v = nullptr, uint32_t* am_i = nullptr,
                          uint32_t* am_n = nullptr, int am_stride = 0) {
    const bool aligned = ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
                         ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
    GemvArgs a{xq, wq, sx, sw, bias, out, m, kg, n, nullptr, 0, 0, nullptr, nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f};
    a.keep_cached = keep_cached;
    if (am_v) {
        // The argmax partials come from the wide-N streaming kernel only.
        if (!aligned || m > 16 || kg != 256 || (n + 15) / 16 < 1024 || out_dtype != OUT_F32 || bias || gv_cfg() != 0)
            return hipErrorNotSupported;
        a.am_v = am_v;
        a.am_i = am_i;
        a.am_n = am_n;
        a.am_stride = am_stride;
    }
    if (m <= 16) return gv_out<1>(s, aligned, out_dtype, a);
    return gv_out<2>(s, aligned, out_dtype, a);
}

hipError_t launch_gemv_i8_gated(hipStream_t s, const uint32_t* xq, const uint32_t* wq, const float* sx,
                                const float* sw, const float* gate, int gate_stride, int gate_col, float* out, int m,
                                int kg, int n) {
    const bool aligned = ((kg * 4) % 16 == 0) && ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) &&
                         ((reinterpret_cast<uintptr_t>(wq) & 15u) == 0);
    GemvArgs a{xq, wq, sx, sw, nullptr, out, m, kg, n, gate, gate_stride, gate_col, nullptr, nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f};
    if (m <= 16) return gv_out<1>(s, aligned, OUT_F32, a);
    return gv_out<2>(s, aligned, OUT_F32, a);
}

// Quantize + GEMV in one launch for m <= 16 (bh_linear_i8's decode path).
// Needs K % 16 == 0, 16-byte aligned x / wq / scratch, and the LDS image of
// 16 rows (16 * (K + 16) bytes) within 64 KB; returns hipErrorNotSupported
// otherwise so the caller falls back to the two-launch path.
hipError_t launch_linear_i8_fused(hipStream_t s, const float* x, const uint32_t* wq, const float* sw,
                                  const float* bias, float* sx_out, uint32_t* xq_out, void* out, int out_dtype, int m,
                                  int kg, int n) {
    const int kbytes = kg * 4;
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wq) |
                         reinterpret_cast<uintptr_t>(xq_out);
    // Wide N (the LM head) keeps the separate quantization: thousands of
    // workgroups would each re-read the f32 activation. So do larger
    // activations (m*K > 12288): every workgroup re-quantizes all rows, which
    // measured slower than one quantize launch from m*K = 16384 up.
    if (m > 16 || kbytes % 16 != 0 || (al & 15u) != 0 || (size_t)16 * (kbytes + 16) + 64 > 64 * 1024 ||
        (n + 15) / 16 >= 1024 || (int64_t)m * kbytes > 12288)
        return hipErrorNotSupported;
    GemvArgs a{xq_out, wq, sx_out, sw, bias, out, m, kg, n, nullptr, 0, 0, x, sx_out, xq_out,
               nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f};
    if (out_dtype == OUT_I32) return gv_fused<1, OUT_I32, false>(s, a);
    if (out_dtype == OUT_F32) return bias ? gv_fused<1, OUT_F32, true>(s, a) : gv_fused<1, OUT_F32, false>(s, a);
    return bias ? gv_fused<1, OUT_BF16, true>(s, a) : gv_fused<1, OUT_BF16, false>(s, a);
}

// The decoder's fused producer + linear for m <= 16 rows, f32 out:
// mode 3 = [residual add |] RMSNorm + quantize + GEMV, mode 4 = SwiGLU +
// quantize + GEMV (K = the SwiGLU width, pre_a = [m, 2K]). K % 16 == 0 (64
// for mode 4), K <= 4096. Returns hipErrorNotSupported outside those limits.
hipError_t launch_gemv_i8_pre(hipStream_t s, int mode, const uint32_t* pre_tok, const float* pre_emb,
                              const float* pre_a, const float* pre_b, const float* pre_w, float* res_out, float eps,
                              const uint32_t* wq, const float* sw, float* out, int m, int kg, int n) {
    const int kbytes = kg * 4;
    if (m < 1 || m > 16 || kbytes % 16 != 0 || kbytes < 16 || kbytes > 4096 || (mode == 4 && kbytes % 64 != 0) ||
        (reinterpret_cast<uintptr_t>(wq) & 15u) != 0)
        return hipErrorNotSupported;
    GemvArgs a{nullptr, wq, nullptr, sw, nullptr, out, m, kg, n, nullptr, 0, 0, nullptr, nullptr, nullptr,
               pre_tok, pre_emb, pre_a, pre_b, pre_w, res_out, eps};
    const int nchunks = (kbytes + 63) / 64;
    // The decoder's own shapes (norm over K = 1024 on 8 waves, SwiGLU over
    // K = 3072 on 16) get prologues fixed at compile time.
    const int ng = nchunks >= 32 ? 4 : 2;  // row groups of the launch below
    const int rpt = m <= ng ? 1 : m <= 2 * ng ? 2 : 4;
    if (mode == 3 && kbytes == 1024) {
        // One row: K split 4 ways (4 waves of 4 chunks) rather than 8 (8 of 2):
        // batch-1 step 0.8495 -> 0.842 ms.
        if (m == 1) return gv_go<1, OUT_F32, false, true, 4, 1, 4, 3, 8 + 1, true, false, 1, 1024>(s, a);
        if (m == 4) return gv_go<1, OUT_F32, false, true, 4, 1, 8, 3, 16 + 1, false, false, 4, 1024>(s, a);
        if (rpt == 1) return gv_go<1, OUT_F32, false, true, 4, 1, 8, 3, 8 + 1>(s, a);
        if (rpt == 2) return gv_go<1, OUT_F32, false, true, 4, 1, 8, 3, 16 + 1>(s, a);
        return gv_go<1, OUT_F32, false, true, 4, 1, 8, 3, 32 + 1>(s, a);
    }
    if (mode == 4 && kbytes == 3072) {
        // 48 K-chunks over 16 waves: each wave's 3 chunks in one batch.
        // One row: 8 waves of 6 chunks rather than 16 of 3: batch-1 step
        // 0.8495 -> 0.831 ms, with the one-row norm change above 0.819 (same
        // box; 12 waves of 4 chunks 0.849, 4 of 12 0.858, two column groups
        // per wave 0.887).
        if (m == 1) return gv_go<1, OUT_F32, false, true, 6, 1, 8, 4, 8 + 3, true, false, 1, 3072>(s, a);
        if (m == 4) return gv_go<1, OUT_F32, false, true, 3, 1, 16, 4, 8 + 3, false, false, 4, 3072>(s, a);
        if (rpt == 1) return gv_go<1, OUT_F32, false, true, 3, 1, 16, 4, 8 + 3>(s, a);
        if (rpt == 2) return gv_go<1, OUT_F32, false, true, 3, 1, 16, 4, 16 + 3>(s, a);
        return gv_go<1, OUT_F32, false, true, 3, 1, 16, 4, 32 + 3>(s, a);
    }
    if (mode == 3) {
        if (nchunks >= 32) return gv_go<1, OUT_F32, false, true, 4, 1, 16, 3>(s, a);
        return gv_go<1, OUT_F32, false, true, 4, 1, 8, 3>(s, a);
    }
    if (nchunks >= 32) return gv_go<1, OUT_F32, false, true, 4, 1, 16, 4>(s, a);
    return gv_go<1, OUT_F32, false, true, 4, 1, 8, 4>(s, a);
}

// XMODE 5: out = (merge of the attention partials, quantized) . W^T, f32, for
// m <= 4 rows, K = nh * hd <= 2048, on 8 waves (512 threads, one 4-element
// context group each).
hipError_t launch_gemv_i8_merge(hipStream_t s, const float* part_o, const float* part_ml, const uint32_t* pos, int nh,
                                int hd, int splits, const uint32_t* wq, const float* sw, float* out, int m, int kg,
                                int n) {
    const int kbytes = kg * 4;
    if (m < 1 || m > 4 || kbytes % 16 != 0 || kbytes > 2048 || kbytes != nh * hd ||
        (reinterpret_cast<uintptr_t>(wq) & 15u) != 0)
        return hipErrorNotSupported;
    GemvArgs a{nullptr, wq, nullptr, sw, nullptr, out, m, kg, n, nullptr, 0, 0, nullptr, nullptr, nullptr,
               nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f};
    a.part_o = part_o;
    a.part_ml = part_ml;
    a.pos = pos;
    a.nh = nh;
    a.hd = hd;
    a.splits = splits;
    // One row: whole-line non-temporal weight loads. Batch-1 decode step
    // 0.859-0.861 -> 0.850-0.851 ms; the same loads in the one-row norm +
    // q|k|v and norm + gate|up launches made the step 0.859 ms (no gain),
    // and on the configs[1] sweep they took the narrow shapes' cold time
    // 3.65 -> 3.53 us on average without moving the 16-launch graph.
    // BH_MERGE_HEAD32 (any value) keeps the general merge, for measurement.
    static const bool head32_on = std::getenv("BH_MERGE_HEAD32") == nullptr;
    const bool head32 = hd == 128 && kbytes == 2048 && splits <= ATTN_SB && head32_on;
    if (m == 1 && head32) return gv_go<1, OUT_F32, false, true, 4, 1, 8, 5, 2, true, true, 1, 2048>(s, a);
    if (m == 1) return gv_go<1, OUT_F32, false, true, 4, 1, 8, 5, 0, true, true>(s, a);
    return gv_go<1, OUT_F32, false, true, 4, 1, 8, 5>(s, a);
}

}  // namespace bh
