"""The int8 paged KV kernels (paged_kv_append_i8_clipped_batched,
paged_decode_{scores,apply}_i8_batched) through the Backend mirror, and the
Qwen3 engine's int8 KV cache, against the oracle (oracle/kv8_oracle.c):
codes and scales byte for byte, scores and context bit for bit."""
import numpy as np
import pytest

from brain_amd.backend import HipBackend
from oracle import oracle as o

pytestmark = pytest.mark.gpu

FMAX = np.finfo(np.float32).max
NAMES = ["paged_kv_append_i8_clipped_batched", "paged_decode_scores_i8_batched", "paged_decode_apply_i8_batched"]


@pytest.fixture(scope="module")
def be(gpu):
    return HipBackend(NAMES)


def f32bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same(got, want, what):
    bad = np.argwhere(np.asarray(got).ravel() != np.asarray(want).ravel()).ravel()
    assert bad.size == 0, f"{what} differ at {bad.size} places, first {bad[:8].tolist()}: " \
                          f"{np.asarray(got).ravel()[bad[:4]].tolist()} vs {np.asarray(want).ravel()[bad[:4]].tolist()}"


def u32_as_f32(a):
    return np.ascontiguousarray(a, np.uint32).view(np.float32)


class Cache:
    """A paged pool on the device plus its oracle twin."""

    def __init__(self, be, n_blocks, bs, n_kv, hd, fill=0):
        self.be, self.bs, self.n_kv, self.hd = be, bs, n_kv, hd
        self.kv_stride = n_kv * hd
        self.pool_h = np.full(n_blocks * bs * self.kv_stride // 4, fill, np.uint32)
        self.sc_h = np.full(n_blocks * bs * n_kv, -1.0, np.float32)
        self.pool = be.storage_init("pool", u32_as_f32(self.pool_h))
        self.sc = be.storage_init("scales", self.sc_h)

    def append(self, src, blocks, offsets, clip):
        be = self.be
        b = src.shape[0]
        bufs = [be.storage_init("src", src), be.storage_init("blk", u32_as_f32(blocks)),
                be.storage_init("off", u32_as_f32(offsets)), be.storage_init("clip", clip), self.pool, self.sc]
        be.submit([], [be.step(be.kernel_index(NAMES[0]), bufs, [b, self.kv_stride, self.bs, self.hd], b * self.n_kv)])
        self.pool_h, self.sc_h = o.paged_kv_append_i8(src, blocks, offsets, clip, self.pool_h, self.sc_h, self.bs,
                                                      self.hd)

    def check(self):
        got_pool = self.be.read(self.pool, self.pool_h.size, np.uint32)
        got_sc = self.be.read(self.sc, self.sc_h.size, np.uint32)
        assert np.array_equal(got_pool, self.pool_h), "int8 codes differ"
        assert np.array_equal(got_sc, f32bits(self.sc_h)), "scales differ"


@pytest.mark.parametrize("n_kv,hd,bs", [(8, 128, 16), (2, 64, 4), (3, 36, 5), (1, 256, 32)])
def test_append_scores_apply_bit_exact(be, n_kv, hd, bs):
    rng = np.random.default_rng(n_kv * hd + bs)
    batch, group = 3, 2
    nh = n_kv * group
    max_bt = 4
    cap = max_bt * bs
    lens = [cap, 1, cap // 2 + 1]
    cache = Cache(be, batch * max_bt + 2, bs, n_kv, hd)
    perm = rng.permutation(batch * max_bt + 2)
    bt = perm[:batch * max_bt].reshape(batch, max_bt).astype(np.uint32)
    clip = np.where(rng.random(n_kv) < 0.5, FMAX, rng.uniform(0.5, 2.0, n_kv)).astype(np.float32)
    for j in range(max(lens)):
        live = [b for b in range(batch) if j < lens[b]]
        src = (rng.standard_normal((len(live), n_kv * hd)) * rng.uniform(0.2, 3, (len(live), 1))).astype(np.float32)
        if j == 0:
            src[0, :hd] = 0.0                                # zero head: scale 1
            src[-1, hd - 4:hd] = [127.0, 2.5, -2.5, 3.5]     # ties at a scale of 1 when not clipped
        cache.append(src, np.array([bt[b, j // bs] for b in live], np.uint32),
                     np.full(len(live), j % bs, np.uint32), clip)
    cache.check()

    q = rng.standard_normal((batch, nh, hd)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    pre = np.full((batch, nh, cap), 12345.0, np.float32)     # entries past seq_len stay untouched
    bufs = [be.storage_init("q", q), cache.pool, be.storage_init("bt", u32_as_f32(bt)),
            be.storage_init("len", u32_as_f32(np.array(lens, np.uint32))), cache.sc, be.storage_init("scores", pre)]
    params = [batch, nh, group, hd, bs, n_kv * hd, cap, max_bt, int(f32bits(scale)[0])]
    be.submit([], [be.step(be.kernel_index(NAMES[1]), bufs, params, batch * nh * cap)])
    got = be.read(bufs[5], pre.size, np.uint32)
    want = o.paged_decode_scores_i8(q, cache.pool_h, bt, lens, cache.sc_h, pre, nh, group, hd, bs, n_kv * hd, cap,
                                    float(scale))
    same(got, f32bits(want), "scores")

    probs = rng.random((batch, nh, cap)).astype(np.float32)
    ctx = be.storage(batch * nh * hd)
    bufs = [be.storage_init("probs", probs), cache.pool, bufs[2], bufs[3], cache.sc, ctx]
    be.submit([], [be.step(be.kernel_index(NAMES[2]), bufs, params[:8], batch * nh * hd)])
    got = be.read(ctx, batch * nh * hd, np.uint32)
    want = o.paged_decode_apply_i8(probs, cache.pool_h, bt, lens, cache.sc_h, nh, group, hd, bs, n_kv * hd, cap)
    same(got, f32bits(want), "context")


def test_append_clip_ties_and_layout(be):
    hd, bs = 8, 2
    cache = Cache(be, 3, bs, 2, hd, fill=0xA5A5A5A5)
    src = np.array([[127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -127.0,          # head 0: scale 1, ties to even
                     127.0, 1.25, -1.75, 63.5, 100.0, -64.0, 0.0, 0.75]],    # head 1: clipped at 63.5
                   np.float32)
    cache.append(src, np.array([2], np.uint32), np.array([1], np.uint32), np.array([FMAX, 63.5], np.float32))
    cache.check()
    codes = cache.pool_h.view(np.int8).reshape(3 * bs, 2, hd)
    assert list(codes[5, 0]) == [127, 2, -2, 4, 0, 0, 2, -127]
    assert list(codes[5, 1]) == [127, 2, -4, 127, 127, -127, 0, 2]
    assert (cache.pool_h.reshape(3 * bs, -1)[:5] == 0xA5A5A5A5).all()    # only slot 2*2+1 written


def test_rejects_bad_geometry(be):
    from brain_amd import BrainHipError
    src = be.storage(64)
    small = be.storage(8)
    with pytest.raises(BrainHipError, match="multiple of head_dim"):
        be.step(be.kernel_index(NAMES[0]), [src, small, small, small, src, small], [1, 60, 4, 16])
    with pytest.raises(BrainHipError, match="overlaps"):   # the pool may not alias the source
        be.step(be.kernel_index(NAMES[0]), [src, small, small, small, src, be.storage(8)], [1, 32, 4, 16])


def test_engine_kv_int8_codes_and_scales_byte_exact(gpu):
    """The Qwen3 engine's int8 cache is the oracle's append of the f32 values:
    layer 0's keys and values do not depend on the cache mode, so an f32-KV
    engine gives the inputs and the int8 engine's codes and scales must be
    exactly or_paged_kv_append_i8 of them, with a clip table that clips some
    heads and not others."""
    from brain_amd.qwen3 import Qwen3Engine
    from test_qwen3_gpu import SMALL, scaled_weights
    cfg = dict(SMALL)
    w = scaled_weights(cfg, seed=41)
    prompts = np.random.default_rng(3).integers(0, cfg["vocab"], size=(2, 19))
    nkv, hd = cfg["n_kv_heads"], cfg["head_dim"]
    f = Qwen3Engine(dict(cfg, kv_int8=0), 2, 32)
    f.load_weights(w)
    f.prefill(prompts)
    i8 = Qwen3Engine(dict(cfg, kv_int8=1), 2, 32)
    i8.load_weights(w)
    kclip = np.array([FMAX, 0.7], np.float32)[:nkv]
    vclip = np.array([0.05, FMAX], np.float32)[:nkv]
    i8.set_kv_clip(0, 0, kclip)
    i8.set_kv_clip(0, 1, vclip)
    i8.prefill(prompts)
    n = prompts.shape[1]
    for seq in range(2):
        for which, clip in ((0, kclip), (1, vclip)):
            x = f.kv(0, seq, which, n)                              # [n, kv_dim] f32
            codes, scales = i8.kv(0, seq, which, n)
            pool, sc = o.paged_kv_append_i8(x, np.arange(n, dtype=np.uint32), np.zeros(n, np.uint32), clip,
                                            np.zeros(n * nkv * hd // 4, np.uint32), np.zeros(n * nkv, np.float32),
                                            1, hd)
            assert np.array_equal(codes.view(np.uint8).ravel(), pool.view(np.uint8)), (seq, which)
            assert np.array_equal(f32bits(scales).ravel(), f32bits(sc)), (seq, which)
            assert (np.abs(codes) == 127).any()
    f.close()
    i8.close()


def test_engine_clip_matches_oracle(gpu):
    """A clip table that binds on some heads: the engine's int8-KV decoder
    against the oracle's with the same table, under the decoder's noise bars."""
    from test_qwen3_gpu import SMALL, compare_clip, scaled_weights
    cfg = dict(SMALL, kv_int8=1)
    w = scaled_weights(cfg, seed=43)
    rng = np.random.default_rng(4)
    shape = (cfg["n_layers"], cfg["n_kv_heads"])
    kclip = np.where(rng.random(shape) < 0.5, FMAX, rng.uniform(0.3, 1.0, shape)).astype(np.float32)
    vclip = np.where(rng.random(shape) < 0.5, FMAX, rng.uniform(0.02, 0.2, shape)).astype(np.float32)
    prompts = rng.integers(0, cfg["vocab"], size=(2, 9))
    compare_clip(cfg, w, prompts, 6, kclip, vclip)


def test_append_non_finite_matches_oracle(be):
    """NaN / Inf heads: the kernel's policy (NaN dropped from max|x| and coded
    0; Inf bounded by the clip and saturated to +-127) equals the oracle's."""
    hd, bs = 8, 1
    cache = Cache(be, 3, bs, 2, hd)
    src = np.array([[np.nan, 2.0, -1.0, 0.5, 0.0, 1.0, -2.0, 0.25, np.inf, 2.0, -1e37, 0.5, -np.inf, 1.0, -2.0, 0.25],
                    [np.inf, 2.0, -1e37, 0.5, -np.inf, 1.0, -2.0, 0.25, np.nan, np.nan, 3.0, 0, 0, 0, 0, 0]],
                   np.float32)
    cache.append(src, np.array([0, 2], np.uint32), np.array([0, 0], np.uint32), np.array([FMAX, 12.7], np.float32))
    cache.check()


def test_apply_stops_at_cap(be):
    """seq_lens > cap: the context sums the row's cap probabilities only."""
    rng = np.random.default_rng(11)
    n_kv, hd, bs, group, max_bt = 2, 64, 4, 2, 3
    nh, cap, batch = n_kv * group, 8, 2
    cache = Cache(be, batch * max_bt, bs, n_kv, hd)
    bt = np.arange(batch * max_bt, dtype=np.uint32).reshape(batch, max_bt)
    for j in range(max_bt * bs):
        src = rng.standard_normal((batch, n_kv * hd)).astype(np.float32)
        cache.append(src, bt[:, j // bs].copy(), np.full(batch, j % bs, np.uint32), np.full(n_kv, FMAX, np.float32))
    lens = np.array([12, 9], np.uint32)
    probs = rng.random((batch, nh, cap)).astype(np.float32)
    ctx = be.storage(batch * nh * hd)
    bufs = [be.storage_init("probs", probs), cache.pool, be.storage_init("bt", u32_as_f32(bt)),
            be.storage_init("len", u32_as_f32(lens)), cache.sc, ctx]
    be.submit([], [be.step(be.kernel_index(NAMES[2]), bufs, [batch, nh, group, hd, bs, n_kv * hd, cap, max_bt],
                           batch * nh * hd)])
    got = be.read(ctx, batch * nh * hd, np.uint32)
    want = o.paged_decode_apply_i8(probs, cache.pool_h, bt, [cap, cap], cache.sc_h, nh, group, hd, bs, n_kv * hd, cap)
    same(got, f32bits(want), "context")
