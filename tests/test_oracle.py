"""Pins the CPU oracle (oracle/brain_oracle.c) against the reference's own
known-answer tests, published constants, closed forms and independent numpy /
torch evaluations. No GPU. Each test names what it pins and its source."""
import numpy as np
import pytest
import torch

from oracle import oracle as o


def _pack_bytes(v):
    """int8 values [r, k] -> u32 words, byte b of word g = element 4g+b."""
    v = np.ascontiguousarray(np.asarray(v, dtype=np.int8))
    return v.view(np.uint32).reshape(v.shape[0], v.shape[1] // 4)


# ---------------------------------------------------------------- SplitMix64
def test_splitmix64_published_sequence():
    # SplitMix64 (Steele et al.) from state 0 emits 0xe220a8397b1dcdaf,
    # 0x6e789e6aa1b965f4, 0x06c45d188009454f, ...; rng.rs:22-27 starts the state
    # at seed+GAMMA, so Rng::new(0) yields the 2nd and 3rd published values.
    r = o.Rng(0)
    assert r.next_u64() == 0x6E789E6AA1B965F4
    assert r.next_u64() == 0x06C45D188009454F
    assert [int(v) for v in o.splitmix_u64(0, 2)] == [0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_splitmix_vectorised_matches_scalar_stream():
    r = o.Rng(1234)
    want = [r.next_u64() for _ in range(50)]
    assert [int(v) for v in o.splitmix_u64(1234, 50)] == want


def test_rng_derived_draws():
    r = o.Rng(7)
    for _ in range(1000):
        v = r.gen_range_inclusive(-127, 127)
        assert -127 <= v <= 127
        f = r.next_f64()
        assert 0.0 <= f < 1.0
    # next_f64 is the top 53 bits over 2^53 (rng.rs:39-42).
    r1, r2 = o.Rng(9), o.Rng(9)
    assert r1.next_f64() == (r2.next_u64() >> 11) / float(1 << 53)


def test_synth_weights_follow_gen_range_and_uniform():
    wq, sw = o.synth_weights(3, 8, 11)
    r = o.Rng(11)
    q = [r.gen_range_inclusive(-127, 127) for _ in range(24)]
    s = [np.float32(r.uniform(0.002, 0.02)) for _ in range(3)]
    assert (o.unpack_i8(wq).reshape(-1) == np.array(q, np.int8)).all()
    assert (sw == np.array(s, np.float32)).all()


def test_synth_acts_follow_next_gaussian():
    x = o.synth_acts(2, 4, 5)
    r = o.Rng(5)
    g = np.array([r.next_gaussian() for _ in range(8)], np.float64).astype(np.float32)
    assert (x.reshape(-1) == g).all()


# ---------------------------------------------------------------- dot4 / acc KAT
def _kat_inputs():
    # crates/wgsl-cpu/src/lib.rs:1633-1679 (dot4i8packed_matches_host_reference)
    m, k, n = 2, 8, 3
    xi = np.array([((i * 37 + 11) % 255 - 127) for i in range(m * k)], np.int64).astype(np.int8).reshape(m, k)
    wi = np.array([((i * 53 + 5) % 255 - 127) for i in range(n * k)], np.int64).astype(np.int8).reshape(n, k)
    sx = np.array([0.5, 0.25], np.float32)
    sw = np.array([1.0, 2.0, 0.125], np.float32)
    return xi, wi, sx, sw


def test_dot4_known_answer():
    xi, wi, sx, sw = _kat_inputs()
    acc = o.matmul_i8_acc(_pack_bytes(xi), _pack_bytes(wi))
    assert acc.tolist() == [[9660, 17202, -10701], [14168, -7773, -10589]]
    out = o.epilogue(acc, sx, sw)
    assert out.tolist() == [[4830.0, 17202.0, -668.8125], [3542.0, -3886.5, -330.90625]]


def test_acc_against_int64_brute_force():
    rng = np.random.default_rng(0)
    for (m, k, n) in [(1, 4, 1), (5, 24, 7), (33, 132, 17), (3, 1024, 9)]:
        a = rng.integers(-128, 128, (m, k)).astype(np.int8)  # -128 included: sign extension
        b = rng.integers(-128, 128, (n, k)).astype(np.int8)
        want = a.astype(np.int64) @ b.astype(np.int64).T
        got = o.matmul_i8_acc(_pack_bytes(a), _pack_bytes(b))
        assert (got.astype(np.int64) == want).all(), (m, k, n)
        assert (o.acc_exact(_pack_bytes(a), _pack_bytes(b)).astype(np.int64) == want).all()


def test_acc_mutation_zero_extension_is_caught():
    # A zero-extending dot4 differs on negative bytes; the KAT above must see it.
    xi, wi, _, _ = _kat_inputs()
    wrong = xi.view(np.uint8).astype(np.int64) @ wi.view(np.uint8).astype(np.int64).T
    assert wrong.tolist() != [[9660, 17202, -10701], [14168, -7773, -10589]]


# ---------------------------------------------------------------- epilogue
def test_epilogue_matches_numpy_ieee_products():
    rng = np.random.default_rng(1)
    acc = rng.integers(-(2**27), 2**27, (17, 29)).astype(np.int32)
    sx = rng.uniform(1e-4, 1.0, 17).astype(np.float32)
    sw = rng.uniform(0.002, 0.02, 29).astype(np.float32)
    bias = rng.standard_normal(29).astype(np.float32)
    want = (acc.astype(np.float32) * sx[:, None]) * sw[None, :]   # numpy: one rounding per op
    assert (o.epilogue(acc, sx, sw) == want).all()
    assert (o.epilogue(acc, sx, sw, bias) == want + bias[None, :]).all()
    # Association matters: acc*(sx*sw) differs somewhere, so a swapped order is caught.
    alt = acc.astype(np.float32) * (sx[:, None] * sw[None, :])
    assert (alt != want).any()


def test_epilogue_static_association():
    acc = np.arange(-50, 50, dtype=np.int32).reshape(10, 10) * 977
    sx, sw = np.float32(0.0123), np.float32(0.0071)
    assert (o.epilogue_static(acc, sx, sw) == acc.astype(np.float32) * (sx * sw)).all()


def test_bf16_rne_matches_torch_and_specials():
    rng = np.random.default_rng(2)
    v = np.concatenate([
        rng.standard_normal(5000).astype(np.float32) * 1e3,
        np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-8 + 2**-20, -1.0 - 2**-8,  # ties / near ties
                  np.inf, -np.inf, 0.0, -0.0, 3.4e38, 1e-40], np.float32),
    ])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([o.f32_to_bf16(float(x)) for x in v], np.uint16)
    assert (got == want).all()
    # ties to even: 1+2^-8 -> 1.0 (0x3f80), 1+3*2^-8 -> 1+2^-6 (0x3f82)
    assert o.f32_to_bf16(1.0 + 2**-8) == 0x3F80 and o.f32_to_bf16(1.0 + 3 * 2**-8) == 0x3F82
    nan = o.f32_to_bf16(float("nan"))
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_epilogue_bf16_is_rne_of_f32():
    rng = np.random.default_rng(3)
    acc = rng.integers(-(2**20), 2**20, (8, 40)).astype(np.int32)
    sx = rng.uniform(0.01, 1, 8).astype(np.float32)
    sw = rng.uniform(0.002, 0.02, 40).astype(np.float32)
    f = o.epilogue(acc, sx, sw)
    b = o.epilogue(acc, sx, sw, out_dtype="bf16")
    assert (b == torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)).all()


# ---------------------------------------------------------------- activation quant
def test_max_abs_row_closed_form_and_zero_row():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((9, 37)).astype(np.float32)
    x[3] = 0.0
    sx = o.max_abs_row(x)
    want = np.maximum(np.abs(x).max(axis=1), np.float32(1e-8)) / np.float32(127.0)
    assert (sx == want.astype(np.float32)).all()
    assert sx[3] == np.float32(1e-8) / np.float32(127.0)


def test_quant_pack_ties_to_even():
    # crates/wgsl-cpu/tests/math_builtins.rs:84-91: round(ties) -> [-2,-2,-0,0,2,2,4]
    x = np.array([[-2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.5, 0.0]], np.float32)
    q = o.unpack_i8(o.quant_pack(x, np.array([1.0], np.float32)))
    assert q.tolist() == [[-2, -2, 0, 0, 2, 2, 4, 0]]


def test_quant_pack_extremes_and_clamp():
    x = np.array([[3.0, -3.0, 1.5, 0.0], [1e30, -1e30, 0.0, 5.0]], np.float32)
    sx = o.max_abs_row(x)
    q = o.unpack_i8(o.quant_pack(x, sx))
    assert q[0, 0] == 127 and q[0, 1] == -127       # |x| = max -> +-127 exactly
    assert q[1, 0] == 127 and q[1, 1] == -127
    # clamp: a scale below the true max saturates instead of wrapping
    q2 = o.unpack_i8(o.quant_pack(np.array([[500.0, -500.0, 1.0, -1.0]], np.float32), np.array([1.0], np.float32)))
    assert q2.tolist() == [[127, -127, 1, -1]]


def test_quant_pack_uses_reciprocal_multiply_not_divide():
    # quant_pack.wgsl:36-39 multiplies by inv=1/sx. Find inputs where that and
    # x/sx round differently, and check the oracle follows the multiply.
    # Candidates sit on half-integer quotients, where the two roundings can part.
    rng = np.random.default_rng(5)
    sx = rng.uniform(0.5, 2.0, 400000).astype(np.float32)
    x = ((rng.integers(-120, 120, 400000) + 0.5) * sx).astype(np.float32)
    inv = (np.float32(1.0) / sx).astype(np.float32)
    mul = np.rint(x * inv)
    div = np.rint(x / sx)
    idx = np.nonzero(mul != div)[0]
    assert len(idx) > 0
    i = idx[:4]
    xs = np.zeros((4, 4), np.float32)
    xs[:, 0] = x[i]
    got = o.unpack_i8(o.quant_pack(xs, sx[i]))[:, 0]
    assert (got == np.clip(mul[i], -127, 127).astype(np.int8)).all()
    assert (got != np.clip(div[i], -127, 127).astype(np.int8)).all()


def test_quant_pack_matches_numpy_rint():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((13, 64)) * 3).astype(np.float32)
    sx = o.max_abs_row(x)
    inv = (np.float32(1.0) / sx).astype(np.float32)
    want = np.clip(np.rint(x * inv[:, None]), -127, 127).astype(np.int8)
    assert (o.unpack_i8(o.quant_pack(x, sx)) == want).all()


# ---------------------------------------------------------------- weight quant
def _xorshift_fixture(n, k):
    # crates/model/tests/quantize_weight_is_schedule_invariant.rs:31-45
    s = 0x9E3779B97F4A7C15
    out = np.zeros(n * k, np.float32)
    m64 = (1 << 64) - 1
    for i in range(n * k):
        s ^= (s << 13) & m64
        s ^= s >> 7
        s ^= (s << 17) & m64
        u = np.float32(np.float32(s >> 32) / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
        out[i] = np.float32(u) * (np.float32(1.0) + np.float32(i // k) * np.float32(0.37))
    return out.reshape(n, k)


def _serial_quantize(w):
    # The reference test's serial oracle (:48-68), evaluated with numpy f32
    # scalars: ties-AWAY rounding (f32::round), x*(1/s), clamp, two's complement byte.
    n, k = w.shape
    packed = np.zeros((n, k // 4), np.uint32)
    sw = np.zeros(n, np.float32)
    for r in range(n):
        s = np.float32(max(np.float32(np.abs(w[r]).max()), np.float32(1e-8)) / np.float32(127.0))
        sw[r] = s
        inv = np.float32(1.0) / s
        v = (w[r] * inv).astype(np.float32)
        q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -127, 127).astype(np.int8)
        packed[r] = q.view(np.uint32)
    return packed, sw


@pytest.mark.parametrize("n,k", [(1, 64), (3, 8), (17, 24), (64, 4096), (129, 128)])
def test_quantize_weight_matches_reference_serial_oracle(n, k):
    w = _xorshift_fixture(n, k)
    packed, sw = o.quantize_weight(w)
    wp, wsw = _serial_quantize(w)
    assert (packed == wp).all() and (sw == wsw).all()
    assert n == 1 or (sw != sw[0]).any()      # per-row scales, not per-tensor


def test_quantize_weight_ties_away():
    # 0.5, 1.5, 2.5 units: f32::round goes away from zero (1, 2, 3), unlike rint.
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.0]], np.float32)
    packed, sw = o.quantize_weight(w)
    assert sw[0] == np.float32(1.0)
    assert o.unpack_i8(packed).tolist() == [[127, 1, 2, 3, -1, -2, -3, 0]]


def test_quantize_weight_round_trip_and_sign_handling():
    # crates/model/src/int8.rs:241-310
    n, k = 3, 8
    w = ((np.arange(n * k, dtype=np.float32) - 10.0) * np.float32(0.37)).reshape(n, k)
    packed, sw = o.quantize_weight(w)
    deq = o.dequantize_weight(packed, sw, k)
    assert (np.abs(deq - w) <= sw[:, None] * 0.5 + 1e-6).all()
    w2 = np.array([[-100.0, 50.0, -1.0, 90.0], [10.0, -80.0, 60.0, -40.0]], np.float32)
    p2, s2 = o.quantize_weight(w2)
    wrong = p2.view(np.uint8).reshape(2, 4).astype(np.float32) * s2[:, None]
    assert (np.abs(o.dequantize_weight(p2, s2, 4) - wrong) > 1e-3).any()


# ---------------------------------------------------------------- CPU baseline
def test_cpu_baseline_gemv_matches_oracle():
    x = o.synth_acts(16, 256, 1)
    wq, sw = o.synth_weights(96, 256, 2)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    want = o.matmul_i8(xq, wq, sx, sw)
    assert (o.cpu_linear_gemv(x, wq, sw, 4) == want).all()
    assert (o.cpu_gemv_packed(xq, wq, sx, sw, 2) == want).all()


def test_cpu_tiled_gemm_matches_oracle():
    """The prefill host reference equals the pinned matmul bit for bit, on
    ragged tiles and on arbitrary bytes (including -128, which quant_pack
    never emits) against the int64 brute force."""
    x = o.synth_acts(37, 520, 3)
    wq, sw = o.synth_weights(50, 520, 4)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    want = o.matmul_i8(xq, wq, sx, sw)
    assert (o.cpu_gemm_tiled(xq, wq, sx, sw, 3).view(np.uint32) == want.view(np.uint32)).all()
    rng = np.random.default_rng(9)
    xr = rng.integers(0, 2**32, (9, 64), dtype=np.uint64).astype(np.uint32)
    wr = rng.integers(0, 2**32, (7, 64), dtype=np.uint64).astype(np.uint32)
    sxr = rng.uniform(0.001, 0.1, 9).astype(np.float32)
    swr = rng.uniform(0.001, 0.1, 7).astype(np.float32)
    got = o.cpu_gemm_tiled(xr, wr, sxr, swr, 2)
    assert (got.view(np.uint32) == o.epilogue(o.acc_exact(xr, wr), sxr, swr).view(np.uint32)).all()
