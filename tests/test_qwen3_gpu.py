"""The int8 Qwen3 decoder engine (bh_qwen3_*) against the C oracle.

The engine's int8 linears are bit-exact with the oracle's. Its RMSNorm sums,
attention reductions and libm calls (exp, pow, sin, cos) differ from the
oracle's in order and rounding. A one-ulp difference occasionally moves an
activation across an int8 rounding boundary, and that flip then propagates.
Measured on MI355X, a sequence without a flip matches the oracle to about
1e-7 rel-L2; one with a flip can drift to a few 1e-3. The checks are:
  - exactness: at every step, the best-matching sequence agrees to 1e-4. A
    systematic error (RoPE, eps, scale, indexing) hits every sequence and
    fails this;
  - noise bound: every sequence agrees to 2e-2 rel-L2 with the int8 oracle,
    and to the reference's own 0.10 against the fp32 model
    (crates/qwen3/src/model.rs:2638-2661);
  - greedy tokens are equal wherever the oracle's top-2 margin clears the
    noise. After the first mismatch at a near-tie the sequences are
    different inputs and the comparison stops.

Within the engine the results are deterministic, so these must be
bit-identical:
  - graph decode and eager decode;
  - a prefill chunked to a few rows (every linear on the GEMV) and one done
    whole (every linear on the MFMA GEMM).
"""
import numpy as np
import pytest

from brain_amd.qwen3 import QWEN3_0_6B, Qwen3Engine
from oracle import oracle as o

pytestmark = pytest.mark.gpu

SMALL = dict(vocab=1000, n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
             rope_theta=1.0e6, rms_eps=1e-6, tie_embeddings=1, qk_norm=1)


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def scaled_weights(cfg, seed):
    w = o.qwen3_init(cfg, seed=seed, gain_noise=0.2)
    for n in w:
        # Larger logit margins than the 0.02 init, and attention away from uniform
        # (kept mild: very sharp softmax turns one int8 rounding flip into a
        # visible logit change).
        if n == "tok.weight" or n == "lm_head.weight":
            w[n] = (w[n] * 10.0).astype(np.float32)
        elif "attn.w" in n:
            w[n] = (w[n] * 3.0).astype(np.float32)
    return w


def engine_for(cfg, w, max_batch, max_seq, max_rows=None):
    e = Qwen3Engine(cfg, max_batch, max_seq, max_rows)
    e.load_weights(w)
    return e


def compare(cfg, w, prompts, steps, max_rows=None):
    compare_clip(cfg, w, prompts, steps, None, None, max_rows)


def compare_clip(cfg, w, prompts, steps, kclip, vclip, max_rows=None):
    """The engine against the oracle; kclip/vclip [n_layers, n_kv_heads] are
    int8 KV clip tables given to both (None: no clipping)."""
    toks_o, logits_o = o.qwen3_generate(cfg, w, prompts, steps, int8=True, kclip=kclip, vclip=vclip)
    _, logits_f = o.qwen3_generate(cfg, w, prompts, 0, int8=False)
    e = engine_for(cfg, w, prompts.shape[0], prompts.shape[1] + steps + 1, max_rows)
    for l in range(cfg["n_layers"]):
        if kclip is not None:
            e.set_kv_clip(l, 0, kclip[l])
        if vclip is not None:
            e.set_kv_clip(l, 1, vclip[l])
    first = e.prefill(prompts)
    got_logits = [e.logits()]
    got_toks = [first]
    for _ in range(steps):
        got_toks.append(e.decode(1)[0])
        got_logits.append(e.logits())
    if kclip is None and vclip is None:  # the reference's int8-vs-fp32 bound holds without clipping
        assert rel_l2(got_logits[0], logits_f[0]) < 0.10
    checked = 0
    for s in range(steps + 1):
        per_seq = [rel_l2(got_logits[s][b], logits_o[s][b]) for b in range(prompts.shape[0])]
        assert min(per_seq) < 1e-4, (s, per_seq)
        assert max(per_seq) < 2e-2, (s, per_seq)
        top2 = np.sort(logits_o[s], axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2e-2 * np.abs(logits_o[s]).max()
        assert (got_toks[s][clear] == toks_o[s][clear]).all(), (s, got_toks[s], toks_o[s])
        checked += int(clear.sum())
        if not (got_toks[s] == toks_o[s]).all():
            break
    assert checked >= prompts.shape[0]
    e.close()


@pytest.mark.parametrize("batch,plen", [(1, 1), (1, 3), (2, 2), (4, 1)])
def test_engine_short_prompt_matches_oracle(gpu, batch, plen):
    """Prompts of at most 4 rows in all: the prefill itself takes the fused
    producers (RMSNorm and SwiGLU inside the GEMV prologues; for one row also
    the attention merge), which the decode-only comparisons do not reach."""
    w = scaled_weights(SMALL, seed=41 + plen)
    prompts = np.random.default_rng(plen + 10 * batch).integers(0, SMALL["vocab"], size=(batch, plen))
    steps = 5
    toks_o, logits_o = o.qwen3_generate(SMALL, w, prompts, steps, int8=True)
    e = engine_for(SMALL, w, batch, plen + steps + 1)
    got = [(e.prefill(prompts), e.logits())]
    for _ in range(steps):
        got.append((e.decode(1)[0], e.logits()))
    e.close()
    # One sequence can meet an int8 rounding flip (~5e-3 rel-L2, as with
    # longer prompts); most steps must still be exact.
    exact = 0
    for s_, (tk, lg) in enumerate(got):
        worst = max(rel_l2(lg[b], logits_o[s_][b]) for b in range(batch))
        assert worst < 2e-2, (s_, worst)
        exact += worst < 1e-4
        top2 = np.sort(logits_o[s_], axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2e-2 * np.abs(logits_o[s_]).max()
        assert (tk[clear] == toks_o[s_][clear]).all(), (s_, tk, toks_o[s_])
        if not (tk == toks_o[s_]).all():
            break
    assert exact >= 3, exact


@pytest.mark.parametrize("cfg_over", [{}, dict(tie_embeddings=0), dict(qk_norm=0, n_kv_heads=4), dict(kv_int8=1),
                                      dict(kv_int8=1, n_kv_heads=1, tie_embeddings=0)],
                         ids=["tied", "untied", "mha_no_qknorm", "kv_int8", "kv_int8_mqa"])
def test_engine_matches_oracle(gpu, cfg_over):
    cfg = dict(SMALL, **cfg_over)
    w = scaled_weights(cfg, seed=7)
    prompts = np.random.default_rng(3).integers(0, cfg["vocab"], size=(3, 9))
    compare(cfg, w, prompts, steps=6)


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_engine_long_context_matches_oracle(gpu, kv_int8):
    """Positions past 512: the merge of more than 16 key chunks takes its
    batched two-pass form (same operations in the same order as the one-batch
    form), and the prompt runs as two prefill chunks. Over 530 positions
    every sequence meets int8 rounding flips (measured ~5e-3 rel-L2, the same
    as a flipped sequence at 100 positions), so this checks the noise bound
    and the clear-margin tokens only."""
    cfg = dict(SMALL, kv_int8=kv_int8)
    w = scaled_weights(cfg, seed=17)
    prompts = np.random.default_rng(6).integers(0, cfg["vocab"], size=(3, 530))
    steps = 3
    toks_o, logits_o = o.qwen3_generate(cfg, w, prompts, steps, int8=True)
    e = engine_for(cfg, w, 3, 530 + steps + 1, 640)
    got = [(e.prefill(prompts), e.logits())]
    for _ in range(steps):
        got.append((e.decode(1)[0], e.logits()))
    for s_, (tk, lg) in enumerate(got):
        per_seq = [rel_l2(lg[b], logits_o[s_][b]) for b in range(3)]
        assert max(per_seq) < 2e-2, (s_, per_seq)
        top2 = np.sort(logits_o[s_], axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2e-2 * np.abs(logits_o[s_]).max()
        assert (tk[clear] == toks_o[s_][clear]).all(), (s_, tk, toks_o[s_])
        if not (tk == toks_o[s_]).all():
            break
    e.close()


def test_engine_chunked_prefill_matches_oracle(gpu):
    """max_rows = 8 with batch 2 splits the prompt into 4-position chunks."""
    cfg = SMALL
    w = scaled_weights(cfg, seed=9)
    prompts = np.random.default_rng(4).integers(0, cfg["vocab"], size=(2, 11))
    compare(cfg, w, prompts, steps=3, max_rows=8)


def test_chunking_and_graph_are_bit_identical(gpu):
    cfg = SMALL
    w = scaled_weights(cfg, seed=12)
    prompts = np.random.default_rng(5).integers(0, cfg["vocab"], size=(2, 40))
    a = engine_for(cfg, w, 2, 64)               # whole prompt: 80 rows -> MFMA GEMM
    b = engine_for(cfg, w, 2, 64, max_rows=4)   # 2-position chunks -> GEMV
    ta, tb = a.prefill(prompts), b.prefill(prompts)
    assert (ta == tb).all()
    assert np.array_equal(a.logits(), b.logits())
    ga = a.decode(10)                 # graph replays
    gb = b.decode(10, eager=True)     # eager launches
    assert (ga == gb).all()
    assert np.array_equal(a.logits(), b.logits())
    a.close()
    b.close()


def test_engine_argument_errors(gpu):
    from brain_amd._lib import BrainHipError
    e = Qwen3Engine(SMALL, 2, 16)
    with pytest.raises(BrainHipError):
        e.decode(1)                                   # no prefill yet
    with pytest.raises(BrainHipError):
        e.prefill(np.array([[SMALL["vocab"]]]))       # token outside the vocabulary
    with pytest.raises(BrainHipError):
        e.prefill(np.zeros((3, 4)))                   # batch above max_batch
    with pytest.raises(BrainHipError):
        e.set_weight("blocks.9.ln1.weight", np.ones(256))
    with pytest.raises(BrainHipError):
        e.set_weight("blocks.0.ln1.weight", np.ones(255))
    e.prefill(np.zeros((1, 10)))
    with pytest.raises(BrainHipError):
        e.decode(7)                                   # 10 + 7 > max_seq 16
    e.close()


def test_qwen3_0_6b_shape_runs(gpu):
    """The config-3 architecture with device random init: batch 8, a 128-token
    prompt, greedy steps through the graph; graph and eager agree exactly."""
    e = Qwen3Engine(QWEN3_0_6B, 8, 160, max_rows=1024)
    e.init_random(7)
    prompts = np.random.default_rng(0).integers(0, QWEN3_0_6B["vocab"], size=(8, 128))
    first = e.prefill(prompts)
    assert first.shape == (8,) and (first < QWEN3_0_6B["vocab"]).all()
    lg = e.logits()
    assert np.isfinite(lg).all() and lg.std() > 0
    g = e.decode(8)
    assert (g < QWEN3_0_6B["vocab"]).all()
    e2 = Qwen3Engine(QWEN3_0_6B, 8, 160, max_rows=1024)
    e2.init_random(7)
    assert (e2.prefill(prompts) == first).all()
    assert (e2.decode(8, eager=True) == g).all()
    e.close()
    e2.close()


def test_int8_checkpoint_load_matches_f32_upload(gpu, tmp_path):
    """bh_qwen3_load of the int8 safetensors format (packed linears + scales,
    one linear left F32 to exercise the device-quantize branch) gives exactly
    the engine that set_weight builds from the f32 weights."""
    from brain_amd import int8_format as fmt
    cfg = dict(SMALL, tie_embeddings=0)
    w = scaled_weights(cfg, seed=21)
    path = str(tmp_path / "q.safetensors")
    fmt.write_int8_checkpoint(path, w, never=("tok.weight",), keep_f32=("blocks.1.mlp.up.weight",))
    prompts = np.random.default_rng(8).integers(0, cfg["vocab"], size=(2, 7))
    a = engine_for(cfg, w, 2, 16)
    b = Qwen3Engine(cfg, 2, 16)
    b.load(path)
    assert (a.generate(prompts, 5) == b.generate(prompts, 5)).all()
    assert np.array_equal(a.logits(), b.logits())
    a.close()
    b.close()


@pytest.mark.parametrize("tied", [1, 0])
def test_int8_checkpoint_with_quantized_embedding(gpu, tmp_path, tied):
    """The reference's importer also packs the embedding (import.rs:349-351,
    622-623). Loading such a file gives the engine whose gather table is the
    dequantized embedding (int8.rs:70-87) and whose head is the file's packed
    head: the same model as an untied engine built from those f32 tables."""
    from brain_amd import int8_format as fmt
    cfg = dict(SMALL, tie_embeddings=tied)
    w = scaled_weights(cfg, seed=23)
    path = str(tmp_path / "qe.safetensors")
    fmt.write_int8_checkpoint(path, w)
    assert fmt.describe(path, "tok.weight") == ("U32", (cfg["vocab"], cfg["d_model"] // 4))
    packed, sw = o.quantize_weight(w["tok.weight"])
    ref_w = dict(w)
    ref_w["tok.weight"] = o.dequantize_weight(packed, sw, cfg["d_model"])
    if tied:
        ref_w["lm_head.weight"] = w["tok.weight"]  # the packed head is quantize(tok) either way
    ref_cfg = dict(cfg, tie_embeddings=0)
    prompts = np.random.default_rng(10).integers(0, cfg["vocab"], size=(2, 5))
    a = engine_for(ref_cfg, ref_w, 2, 16)
    b = Qwen3Engine(cfg, 2, 16)
    b.load(path)
    assert (a.generate(prompts, 4) == b.generate(prompts, 4)).all()
    assert np.array_equal(a.logits(), b.logits())
    a.close()
    b.close()


def test_autotune_changes_no_result(gpu):
    """Both candidates are bit-exact, so the measured choice changes speed only."""
    from brain_amd._lib import load as L
    cfg = SMALL
    w = scaled_weights(cfg, seed=22)
    prompts = np.random.default_rng(9).integers(0, cfg["vocab"], size=(4, 6))
    a = engine_for(cfg, w, 4, 16)
    ref = a.generate(prompts, 6)
    ref_logits = a.logits()
    assert a.autotune(reps=2) > 0
    assert L().bh_tune_get(4, cfg["vocab"], cfg["d_model"]) in (1, 2)
    for v in (1, 2):   # force every decode-regime linear onto one candidate
        for m in (1, 2, 4):
            for n, k in ((512, 256), (256, 256), (1024, 256), (256, 512), (1000, 256)):
                L().bh_tune_set(m, n, k, v)
        b = engine_for(cfg, w, 4, 16)
        assert (b.generate(prompts, 6) == ref).all()
        assert np.array_equal(b.logits(), ref_logits)
        b.close()
    L().bh_tune_clear()
    a.close()


def test_kv_int8_chunking_graph_and_clip(gpu):
    """int8 KV: chunked prefill and graph decode stay bit-identical; an explicit
    FLT_MAX clip equals the default; a tight clip changes the result."""
    cfg = dict(SMALL, kv_int8=1)
    w = scaled_weights(cfg, seed=31)
    prompts = np.random.default_rng(6).integers(0, cfg["vocab"], size=(2, 30))
    a = engine_for(cfg, w, 2, 48)
    b = engine_for(cfg, w, 2, 48, max_rows=6)
    big = np.full(cfg["n_kv_heads"], np.finfo(np.float32).max, np.float32)
    for l in range(cfg["n_layers"]):
        b.set_kv_clip(l, 0, big)
        b.set_kv_clip(l, 1, big)
    assert (a.generate(prompts, 8) == b.generate(prompts, 8, eager=True)).all()
    assert np.array_equal(a.logits(), b.logits())
    c = engine_for(cfg, w, 2, 48)
    for l in range(cfg["n_layers"]):
        c.set_kv_clip(l, 0, np.full(cfg["n_kv_heads"], 0.05, np.float32))
    c.generate(prompts, 8)
    assert not np.array_equal(a.logits(), c.logits())
    for e in (a, b, c):
        e.close()


@pytest.mark.parametrize("batch,kv_int8", [(1, 0), (3, 0), (6, 0), (2, 1), (6, 1)])
def test_fused_decode_is_bit_identical_to_unfused(gpu, batch, kv_int8):
    """Decode with the producers inside their consumers (rotation + cache
    append inside attention; RMSNorm and SwiGLU inside the following GEMV's
    prologue, up to 4 rows; one row also takes the SwiGLU path that spreads
    the row over the whole workgroup and the attention merge inside the output
    projection) against every producer as its own kernel:
    tokens, logits and the KV cache contents they leave must agree exactly.
    Batch 6 keeps the separate GEMV producers but still fuses the rotation."""
    cfg = dict(SMALL, kv_int8=kv_int8)
    w = scaled_weights(cfg, seed=31 + batch)
    prompts = np.random.default_rng(batch).integers(0, cfg["vocab"], size=(batch, 37))
    a = engine_for(cfg, w, batch, 96)
    b = engine_for(cfg, w, batch, 96)
    ta = a.generate(prompts, 40)
    tb = b.generate(prompts, 40, eager=True, unfused=True)
    assert (ta == tb).all()
    assert np.array_equal(a.logits(), b.logits())
    # Both continue from caches the two modes wrote: still identical.
    assert (a.decode(5, eager=True, unfused=True) == b.decode(5)).all()
    assert np.array_equal(a.logits(), b.logits())
    a.close()
    b.close()


@pytest.mark.parametrize("batch,kv_int8", [(1, 0), (2, 0), (4, 0), (8, 0), (8, 1)])
def test_qwen3_0_6b_fused_decode_matches_unfused(gpu, batch, kv_int8):
    """The fused decode kernels at the config-3 shapes (head_dim 128, a
    2048-wide merge on 512 threads, 16 waves per GEMV workgroup; batch 1 takes
    the one-row prologues and batch 4 the four-row ones, both compiled for
    their row count and K; batch 8 the separate producers on 1024-thread
    SwiGLU rows; at 8 rows the attention reads the position before the
    cache, with the f32 and the int8 cache) against the separate ones."""
    prompts = np.random.default_rng(5).integers(0, QWEN3_0_6B["vocab"], size=(batch, 40))
    out = []
    for unfused in (False, True):
        e = Qwen3Engine(dict(QWEN3_0_6B, kv_int8=kv_int8), batch, 64, max_rows=8 * 64)
        e.init_random(11)
        out.append((e.generate(prompts, 6, eager=unfused, unfused=unfused), e.logits()))
        e.close()
    assert (out[0][0] == out[1][0]).all()
    assert np.array_equal(out[0][1], out[1][1])
