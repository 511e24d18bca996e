"""Pins the W4A8 oracle (or_quantize_weight_q4 / or_matmul_q4_acc) and the
library's host int4 quantizer (crates/model/src/int4.rs)."""
import numpy as np
import pytest

from oracle import oracle as o


def test_sign_extension_every_nibble():
    """Reference test `sign_extend_nibble_trick_is_correct` (int4.rs): every one
    of the 16 nibble values, in every position of a word."""
    for raw in range(16):
        want = raw if raw < 8 else raw - 16
        word = np.array([[sum(raw << (4 * b) for b in range(8))]], np.uint32)
        deq = o.dequantize_weight_q4(word, np.array([1.0], np.float32), 8)
        assert (deq == want).all(), raw


def test_quantizer_known_answers():
    # max |w| = 7 -> sw = 1: 3.5 and -3.5 round AWAY from zero, 0.5 -> 1, 6.49 -> 6
    w = np.array([[7.0, -7.0, 3.5, -3.5, 0.5, -0.5, 6.49, 0.0]], np.float32)
    packed, sw = o.quantize_weight_q4(w)
    assert sw[0] == np.float32(1.0)
    assert o.unpack_q4(packed, 8).tolist() == [[7, -7, 4, -4, 1, -1, 6, 0]]
    # scale is max/7, not max/15; an all-zero row gets 1e-8/7 and zero codes
    z = np.zeros((1, 8), np.float32)
    p0, s0 = o.quantize_weight_q4(z)
    assert s0[0] == np.float32(np.float32(1e-8) / np.float32(7.0)) and p0[0, 0] == 0
    # NaN quantizes to 0 (Rust `as i32` of NaN)
    wn = np.array([[1.0, np.nan, -1.0, 0, 0, 0, 0, 0]], np.float32)
    assert o.unpack_q4(o.quantize_weight_q4(wn)[0], 8)[0, 1] == 0


def test_round_trip_half_step():
    w = np.random.default_rng(0).standard_normal((37, 96)).astype(np.float32)
    packed, sw = o.quantize_weight_q4(w)
    deq = o.dequantize_weight_q4(packed, sw, 96)
    assert (np.abs(deq - w) <= sw[:, None] * 0.5 + 1e-6).all()


def test_host_quantizer_matches_oracle():
    from brain_amd.int8_format import quantize_weight_host  # noqa: F401  (library loads)
    from brain_amd._lib import check, load
    w = (np.random.default_rng(1).standard_normal((129, 264)) * 3).astype(np.float32)
    w[5, 7] = np.nan
    packed = np.zeros((129, 33), np.uint32)
    sw = np.zeros(129, np.float32)
    check(load().bh_quantize_weight_q4(w.ctypes.data, 129, 264, packed.ctypes.data, sw.ctypes.data))
    p_ref, s_ref = o.quantize_weight_q4(w)
    assert np.array_equal(packed, p_ref) and np.array_equal(sw.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (3, 64, 5), (7, 264, 9)])
def test_accumulators_brute_force(m, k, n):
    rng = np.random.default_rng(m + k + n)
    x8 = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w4v = rng.integers(-8, 8, size=(n, k))          # includes -8 (not produced by the quantizer)
    packed = np.zeros((n, k // 8), np.uint32)
    for b in range(8):
        packed |= ((w4v[:, b::8] & 0xF).astype(np.uint32) << (4 * b))
    xq = x8.view(np.uint32).reshape(m, k // 4)
    want = (x8.astype(np.int64) @ w4v.T.astype(np.int64)).astype(np.int32)
    assert np.array_equal(o.matmul_q4_acc(xq, packed, k), want)
    assert np.array_equal(o.acc_exact_q4(xq, packed, k), want)
