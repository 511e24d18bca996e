"""Pins the int8 paged-KV oracle (oracle/kv8_oracle.c) to what the WGSL
kernels' arithmetic fixes independently of the oracle's own formula:
closed-form scales, code round trips, ties-to-even known answers, clip
saturation, slot arithmetic on hand-built block tables, and exact
integer-valued dot products (no rounding anywhere, so any order agrees)."""
import numpy as np
import pytest

from oracle import oracle as o

FMAX = np.finfo(np.float32).max


def unpack_codes(pool):
    return np.asarray(pool, np.uint32).view(np.int8)


def append(src, blocks, offsets, clip, n_blocks, bs, hd):
    batch, kv_stride = src.shape
    n_kv = kv_stride // hd
    pool = np.full(n_blocks * bs * kv_stride // 4, 0xDEADBEEF, np.uint32)
    scales = np.full(n_blocks * bs * n_kv, -1.0, np.float32)
    return o.paged_kv_append_i8(src, blocks, offsets, clip, pool, scales, bs, hd)


def test_kv8_code_known_answers():
    # scale 1: x/scale is exact, halfway cases round to even (WGSL round)
    assert [o.kv8_code(x, 1.0) for x in (-2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.5)] == [-2, -2, 0, 0, 2, 2, 4]
    # saturation at +-127, and i32() of NaN is 0 (fcvt_to_sint_sat)
    assert [o.kv8_code(x, 1.0) for x in (127.4, 127.6, 1e30, -1e30)] == [127, 127, 127, -127]
    assert o.kv8_code(float("nan"), 1.0) == 0
    # a true division, not a reciprocal multiply: x = 3 * 0.1f rounds to 3 only by division
    s = np.float32(0.1)
    x = np.float32(s * np.float32(3.5))
    assert o.kv8_code(float(x), float(s)) == int(np.rint(np.float32(x) / s))


def test_append_scale_and_roundtrip_without_clip():
    rng = np.random.default_rng(0)
    hd, n_kv, bs = 64, 4, 16
    src = (rng.standard_normal((3, n_kv * hd)) * rng.uniform(0.1, 30, (3, 1))).astype(np.float32)
    src[1, hd:2 * hd] = 0.0                                    # a zero head
    blocks, offsets = np.array([2, 0, 5]), np.array([3, 15, 0])
    pool, scales = append(src, blocks, offsets, np.full(n_kv, FMAX, np.float32), 6, bs, hd)
    codes = unpack_codes(pool).reshape(6 * bs, n_kv, hd)
    for b in range(3):
        slot = blocks[b] * bs + offsets[b]
        for h in range(n_kv):
            x = src[b, h * hd:(h + 1) * hd]
            mx = np.abs(x).max()
            want = np.float32(mx) / np.float32(127.0) if mx > 0 else np.float32(1.0)
            assert scales[slot * n_kv + h] == want
            c = codes[slot, h].astype(np.float32)
            assert (np.abs(c * want - x) <= want * 0.5 * (1 + 1e-6)).all()
            if mx > 0:
                assert np.abs(c).max() == 127 and c[np.argmax(np.abs(x))] == np.sign(x[np.argmax(np.abs(x))]) * 127
            else:
                assert (c == 0).all()
    # untouched slots keep their contents
    touched = {int(blocks[b] * bs + offsets[b]) for b in range(3)}
    for slot in range(6 * bs):
        if slot not in touched:
            assert (scales[slot * n_kv:(slot + 1) * n_kv] == -1.0).all()
            assert (pool.reshape(6 * bs, -1)[slot] == 0xDEADBEEF).all()


def test_append_clip_and_ties():
    hd = 8
    # row max 127 -> scale 1 exactly; halves round to even
    x = np.array([[127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -127.0]], np.float32)
    pool, scales = append(x, [0], [0], [FMAX], 1, 1, hd)
    assert scales[0] == 1.0
    assert list(unpack_codes(pool)) == [127, 2, -2, 4, 0, 0, 2, -127]
    # clip 63.5 < max 127: scale 0.5, codes of |x| > 63.5 saturate, 1.25/0.5 = 2.5 -> 2
    x2 = np.array([[127.0, 1.25, -1.75, 63.5, 100.0, -64.0, 0.0, 0.75]], np.float32)
    pool, scales = append(x2, [0], [0], [63.5], 1, 1, hd)
    assert scales[0] == np.float32(0.5)
    assert list(unpack_codes(pool)) == [127, 2, -4, 127, 127, -127, 0, 2]
    # clip 0 -> scale 0 -> replaced by 1
    pool, scales = append(x2, [0], [0], [0.0], 1, 1, hd)
    assert scales[0] == 1.0 and list(unpack_codes(pool)) == [127, 1, -2, 64, 100, -64, 0, 1]


def build_cache(rng, batch, n_kv, hd, bs, lens, n_blocks, max_bt, integer=False):
    """A pool filled through the oracle's own append, with permuted physical blocks."""
    kv_stride = n_kv * hd
    perm = rng.permutation(n_blocks)
    bt = np.zeros((batch, max_bt), np.uint32)
    for b in range(batch):
        bt[b] = perm[b * max_bt:(b + 1) * max_bt]
    pool = np.zeros(n_blocks * bs * kv_stride // 4, np.uint32)
    scales = np.zeros(n_blocks * bs * n_kv, np.float32)
    for j in range(max(lens)):
        live = [b for b in range(batch) if j < lens[b]]
        if integer:
            src = rng.integers(-127, 128, (len(live), kv_stride)).astype(np.float32)
            src[:, ::hd] = 127.0                      # scale exactly 1
        else:
            src = rng.standard_normal((len(live), kv_stride)).astype(np.float32)
        blocks = [bt[b, j // bs] for b in live]
        offs = [j % bs] * len(live)
        pool, scales = o.paged_kv_append_i8(src, blocks, offs, np.full(n_kv, FMAX, np.float32), pool, scales, bs,
                                            hd)
    return pool, scales, bt


def test_scores_and_apply_exact_integer_cases():
    rng = np.random.default_rng(1)
    batch, nh, n_kv, hd, bs, cap = 2, 4, 2, 16, 4, 12
    lens = [12, 7]
    max_bt = 3
    pool, scales, bt = build_cache(rng, batch, n_kv, hd, bs, lens, batch * max_bt, max_bt, integer=True)
    assert (scales[scales != 0] == 1.0).all()
    codes = unpack_codes(pool).reshape(-1, n_kv, hd).astype(np.int64)
    q = rng.integers(-8, 9, (batch, nh, hd)).astype(np.float32)
    sentinel = np.full((batch, nh, cap), 777.0, np.float32)
    got = o.paged_decode_scores_i8(q, pool, bt, lens, scales, sentinel, nh, nh // n_kv, hd, bs, n_kv * hd, cap, 0.25)
    probs = rng.integers(0, 5, (batch, nh, cap)).astype(np.float32) / 8.0
    ctx = o.paged_decode_apply_i8(probs, pool, bt, lens, scales, nh, nh // n_kv, hd, bs, n_kv * hd, cap)
    for b in range(batch):
        for h in range(nh):
            kvh = h // (nh // n_kv)
            rows = [codes[bt[b, j // bs] * bs + j % bs, kvh] for j in range(lens[b])]
            want = [float(np.dot(q[b, h].astype(np.int64), r)) * 0.25 for r in rows]
            assert list(got[b, h, :lens[b]]) == want
            assert (got[b, h, lens[b]:] == 777.0).all()          # left untouched
            wc = sum(probs[b, h, j] * rows[j] for j in range(lens[b]))
            assert (ctx[b, h * hd:(h + 1) * hd] == wc.astype(np.float32)).all()


def test_scores_and_apply_against_float64():
    rng = np.random.default_rng(2)
    batch, nh, n_kv, hd, bs, cap, max_bt = 3, 8, 2, 64, 8, 40, 5
    lens = [40, 1, 23]
    pool, scales, bt = build_cache(rng, batch, n_kv, hd, bs, lens, batch * max_bt, max_bt)
    codes = unpack_codes(pool).reshape(-1, n_kv, hd).astype(np.float64)
    q = rng.standard_normal((batch, nh, hd)).astype(np.float32)
    sc = 1.0 / np.sqrt(hd)
    got = o.paged_decode_scores_i8(q, pool, bt, lens, scales, np.zeros((batch, nh, cap), np.float32), nh,
                                   nh // n_kv, hd, bs, n_kv * hd, cap, sc)
    probs = rng.random((batch, nh, cap)).astype(np.float32)
    ctx = o.paged_decode_apply_i8(probs, pool, bt, lens, scales, nh, nh // n_kv, hd, bs, n_kv * hd, cap)
    for b in range(batch):
        for h in range(nh):
            kvh = h // (nh // n_kv)
            slots = [bt[b, j // bs] * bs + j % bs for j in range(lens[b])]
            k = np.stack([codes[s, kvh] * scales[s * n_kv + kvh] for s in slots])
            want = k @ q[b, h].astype(np.float64) * np.float32(sc)
            np.testing.assert_allclose(got[b, h, :lens[b]], want, rtol=2e-5, atol=2e-5 * np.abs(want).max())
            wc = probs[b, h, :lens[b]].astype(np.float64) @ k
            np.testing.assert_allclose(ctx[b, h * hd:(h + 1) * hd], wc, rtol=2e-5, atol=2e-5 * np.abs(wc).max())


def test_apply_stops_at_cap_when_seq_len_exceeds_it():
    """seq_lens[b] > cap: the sum ends at the row's cap probabilities (the WGSL
    loop would read the next row's); equal to seq_lens[b] == cap."""
    rng = np.random.default_rng(3)
    batch, nh, n_kv, hd, bs, cap, max_bt = 2, 4, 2, 16, 4, 8, 3
    pool, scales, bt = build_cache(rng, batch, n_kv, hd, bs, [12, 12], batch * max_bt, max_bt)
    probs = rng.random((batch, nh, cap)).astype(np.float32)
    over = o.paged_decode_apply_i8(probs, pool, bt, [12, 9], scales, nh, nh // n_kv, hd, bs, n_kv * hd, cap)
    at = o.paged_decode_apply_i8(probs, pool, bt, [cap, cap], scales, nh, nh // n_kv, hd, bs, n_kv * hd, cap)
    assert np.array_equal(over.view(np.uint32), at.view(np.uint32))


def test_append_non_finite_policy():
    """NaN and Inf in a head (the WGSL leaves max() with NaN implementation
    defined; this build fixes it): max|x| drops NaN (fmaxf), so the scale comes
    from the other elements and the NaN's code is 0 (i32(NaN) = 0); an Inf
    makes max|x| Inf, the clip (FLT_MAX when unclipped) bounds the scale, and
    Inf / scale saturates to +-127 while every finite element codes to 0."""
    hd = 8
    x = np.array([[np.nan, 2.0, -1.0, 0.5, 0.0, 1.0, -2.0, 0.25]], np.float32)
    pool, scales = append(x, [0], [0], [FMAX], 1, 1, hd)
    assert scales[0] == np.float32(2.0) / np.float32(127.0)
    assert list(unpack_codes(pool)) == [0, 127, -64, 32, 0, 64, -127, 16]
    y = np.array([[np.inf, 2.0, -1e37, 0.5, -np.inf, 1.0, -2.0, 0.25]], np.float32)
    pool, scales = append(y, [0], [0], [FMAX], 1, 1, hd)
    assert scales[0] == np.float32(FMAX) / np.float32(127.0)
    assert list(unpack_codes(pool)) == [127, 0, -4, 0, -127, 0, 0, 0]
    pool, scales = append(y, [0], [0], [12.7], 1, 1, hd)          # clipped: scale 0.1
    assert scales[0] == np.float32(12.7) / np.float32(127.0)
    assert list(unpack_codes(pool)) == [127, 20, -127, 5, -127, 10, -20, 2]
