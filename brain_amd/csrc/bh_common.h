// Internal helpers shared by the gfx950 int8 kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bh {

// Records the message returned by bh_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Cross-lane exchange on the VALU: the value of lane (lane ^ OFF) of a
// 64-lane wave, bit for bit what __shfl_xor(v, OFF, 64) returns. __shfl_xor
// is a ds_bpermute through the LDS unit, ~110 cycles per dependent step on
// MI355X (a 6-step wave reduction then costs ~0.3 us of a decode kernel's
// critical path); these are a few cycles each. OFF 1 and 2: DPP quad_perm;
// 4: DPP row_ror:4 (lane l - 4 within its row of 16) or row_ror:12 (l + 4),
// picked by bit 2 of the lane; 8: row_ror:8; 16 and 32: gfx950's
// v_permlane16_swap / v_permlane32_swap of the value with itself, whose two
// results hold the value unchanged in one and the partner's in the other,
// lane by lane (the one that differs from the value is the partner's; where
// neither differs they are equal). Call with the whole wave active.
template <int OFF>
__device__ __forceinline__ uint32_t xor_lane_u(uint32_t u) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane xor offset");
    const int x = (int)u;
    if constexpr (OFF == 32 || OFF == 16) {
        const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                                 : __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return r[0] != u ? (uint32_t)r[0] : (uint32_t)r[1];
    } else if constexpr (OFF == 8) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);
    } else if constexpr (OFF == 4) {
        const int dn = __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false);
        const int up = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, false);
        const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        return (uint32_t)((lane & 4u) ? dn : up);
    } else if constexpr (OFF == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);
    } else {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);
    }
}
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
    return __builtin_bit_cast(float, xor_lane_u<OFF>(__builtin_bit_cast(uint32_t, v)));
}
// The butterfly reductions `for (off = HI; off >= 1; off >>= 1) v = v (+|max) xor(v, off)`,
// step for step (the same additions in the same order, so the same sum).
template <int HI>
__device__ __forceinline__ float xor_sum(float v) {
    v += xor_lane<HI>(v);
    if constexpr (HI > 1) v = xor_sum<HI / 2>(v);
    return v;
}
template <int HI>
__device__ __forceinline__ float xor_max(float v) {
    v = fmaxf(v, xor_lane<HI>(v));
    if constexpr (HI > 1) v = xor_max<HI / 2>(v);
    return v;
}

// Output element types of the dequant epilogue.
// OUT_I32 stores the raw accumulator (scales and bias unused): the hook the
// parity tests use to check the integer sums themselves.
enum OutDtype : int { OUT_F32 = 0, OUT_BF16 = 1, OUT_I32 = 2 };

// f32 -> bf16, round to nearest even, NaN kept as a quiet NaN with the top
// payload bits ((bits >> 16) | 0x0040), as crates/model/src/half.rs:49-58.
// gfx950's v_cvt_pk_bf16_f32 produces exactly those bits for every one of the
// 2^32 inputs (checked exhaustively on MI355X; the GPU tests keep checking the
// special classes and a large random sample through bh_f32_to_bf16), so the
// conversion is one instruction per two values.
typedef __bf16 bh_bf16x2 __attribute__((ext_vector_type(2)));
typedef float bh_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bh_f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bh_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu); }

// One activation byte of quant_pack (crates/kernels/wgsl/quant_pack.wgsl:36-43):
// clamp(round_ties_even(v * inv), -127, 127) as two's-complement int8.
__device__ __forceinline__ uint32_t quant_byte(float v, float inv) {
    float q = rintf(v * inv);                 // ties to even
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return (uint32_t)((int)q & 0xff);
}
__device__ __forceinline__ uint32_t quant_word(float4 v, float inv) {
    return quant_byte(v.x, inv) | (quant_byte(v.y, inv) << 8) | (quant_byte(v.z, inv) << 16) |
           (quant_byte(v.w, inv) << 24);
}

// One int8 KV-cache code (paged_kv_append_i8_clipped_batched.wgsl:72):
// clamp(i32(round_ties_even(v / scale)), -127, 127), a true division; i32()
// saturates and maps NaN to 0 as the reference's CPU lowering does
// (crates/wgsl-cpu/src/lib.rs:1554, fcvt_to_sint_sat).
__device__ __forceinline__ uint8_t kv8_code(float v, float scale) {
    const float r = rintf(v / scale);
    const float q = r != r ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
    return (uint8_t)(int8_t)(int)q;
}

// W4A8: one u32 of 8 int4 nibbles (nibble b = K index 8g+b, two's complement,
// crates/model/src/int4.rs:46-67) -> 8 sign-extended int8 in K order, bytes
// 0..3 in lo and 4..7 in hi. The even and odd nibbles are masked into bytes;
// bit 3 is copied to bits 4..7 (x * 0x1E, no carry between bytes); then
// v_perm_b32 interleaves the two halves back into K order.
__device__ __forceinline__ void unpack_q4(uint32_t w, uint32_t& lo, uint32_t& hi) {
    uint32_t t0 = w & 0x0F0F0F0Fu;         // nibbles 0,2,4,6
    uint32_t t1 = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1,3,5,7
    t0 |= (t0 & 0x08080808u) * 0x1Eu;
    t1 |= (t1 & 0x08080808u) * 0x1Eu;
    lo = __builtin_amdgcn_perm(t1, t0, 0x05010400u);  // t0.b0 t1.b0 t0.b1 t1.b1
    hi = __builtin_amdgcn_perm(t1, t0, 0x07030602u);  // t0.b2 t1.b2 t0.b3 t1.b3
}
// 16 bytes of int4 (32 K values) -> two 16-byte int8 fragments (K 0..15, 16..31).
__device__ __forceinline__ void unpack_q4x4(v4i w, v4i& a, v4i& b) {
    uint32_t l0, h0, l1, h1, l2, h2, l3, h3;
    unpack_q4((uint32_t)w[0], l0, h0);
    unpack_q4((uint32_t)w[1], l1, h1);
    unpack_q4((uint32_t)w[2], l2, h2);
    unpack_q4((uint32_t)w[3], l3, h3);
    a = v4i{(int)l0, (int)h0, (int)l1, (int)h1};
    b = v4i{(int)l2, (int)h2, (int)l3, (int)h3};
}

// The dequant epilogue of matmul_i8_dyn / matmul_i8_gemv: (f32(acc)*sx)*sw,
// evaluated left to right with no fused multiply-add (the library is built
// with -ffp-contract=off), then the optional bias add.
__device__ __forceinline__ float dequant(int acc, float sxm, float swn) {
    float v = (float)acc * sxm;
    return v * swn;
}

template <int OUT>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
    if constexpr (OUT == OUT_F32) {
        reinterpret_cast<float*>(out)[idx] = v;
    } else {
        reinterpret_cast<uint16_t*>(out)[idx] = f32_to_bf16_rne(v);
    }
}

// 16 bytes (16 int8 along K) of row `row` starting at byte `kb`, zero beyond
// `kbytes`. ALIGNED: the row base and kb are 16-byte aligned and kbytes % 16
// == 0, so one dwordx4 load either lies fully inside the row or fully past it.
template <bool ALIGNED>
__device__ __forceinline__ v4i load_k16(const uint8_t* rowp, int kb, int kbytes) {
    v4i r = {0, 0, 0, 0};
    if constexpr (ALIGNED) {
        if (kb < kbytes) r = *reinterpret_cast<const v4i*>(rowp + kb);
    } else {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(rowp + kb);
#pragma unroll
        for (int d = 0; d < 4; ++d)
            if (kb + 4 * d < kbytes) r[d] = (int)p[d];
    }
    return r;
}

// Weight loads of gemv_i8_kernel, with or without the non-temporal hint
// (NT: global_load_dwordx4 ... nt). A plain streaming read of 256 MiB
// measured 6.3-6.6 TB/s with the hint against 5.6-5.8 without; which GEMV
// launches take it is set where they are launched, by measurement.
template <bool NT>
__device__ __forceinline__ v4i load_w16(const uint8_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    else return *reinterpret_cast<const v4i*>(p);
}
template <bool ALIGNED, bool NT>
__device__ __forceinline__ v4i load_wk16(const uint8_t* rowp, int kb, int kbytes) {
    if constexpr (!NT) {
        return load_k16<ALIGNED>(rowp, kb, kbytes);
    } else {
        v4i r = {0, 0, 0, 0};
        if constexpr (ALIGNED) {
            if (kb < kbytes) r = load_w16<true>(rowp + kb);
        } else {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(rowp + kb);
#pragma unroll
            for (int d = 0; d < 4; ++d)
                if (kb + 4 * d < kbytes) r[d] = (int)__builtin_nontemporal_load(p + d);
        }
        return r;
    }
}

}  // namespace bh
