"""Pins the C oracle of the int8 Qwen3 decoder (oracle/qwen3_oracle.c).

- Its f32 model must equal an independent numpy float64 forward written in
  matrix form over whole sequences with a causal mask. The oracle instead
  feeds tokens one at a time through a KV cache, so agreement also pins
  causal prefill == incremental decode (crates/qwen3/src/model.rs:2604-2635).
  The check covers the logits of the prompt and of every greedy step.
- Its int8 model must track its f32 model within the reference's own bound:
  rel-L2 < 0.10 (crates/qwen3/src/model.rs:2638-2661).
- The greedy argmax must follow argmax_row.wgsl: first index of the maximum,
  NaN never wins, and nothing above -FLT_MAX gives 0.
"""
import numpy as np
import pytest

from oracle import oracle as o

TINY = dict(vocab=97, n_layers=2, d_model=32, n_heads=4, n_kv_heads=2, head_dim=8, d_ff=64,
            rope_theta=1.0e4, rms_eps=1e-6, tie_embeddings=1, qk_norm=1)


def np_forward(cfg, w, tokens):
    """Logits [T, vocab] at every position of `tokens`, float64, matrix form."""
    f = lambda a: np.asarray(a, np.float64)
    d, hd, nh, nkv = cfg["d_model"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    G, eps, T = nh // nkv, cfg["rms_eps"], len(tokens)

    def rms(x, g):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * f(g)

    half = hd // 2
    ang = np.arange(T)[:, None] * cfg["rope_theta"] ** (-2.0 * np.arange(half) / hd)
    cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

    def rope(h):  # [T, heads, hd]
        a, b = h[..., :half], h[..., half:]
        return np.concatenate([a * cos - b * sin, b * cos + a * sin], -1)

    x = f(w["tok.weight"])[np.asarray(tokens)]
    mask = np.triu(np.full((T, T), -np.inf), 1)
    for l in range(cfg["n_layers"]):
        p = lambda s: f(w[f"blocks.{l}.{s}"])
        xn = rms(x, p("ln1.weight"))
        q = (xn @ p("attn.wq.weight").T).reshape(T, nh, hd)
        k = (xn @ p("attn.wk.weight").T).reshape(T, nkv, hd)
        v = (xn @ p("attn.wv.weight").T).reshape(T, nkv, hd)
        if cfg["qk_norm"]:
            q, k = rms(q, p("attn.q_norm.weight")), rms(k, p("attn.k_norm.weight"))
        q, k = rope(q), rope(k)
        ctx = np.zeros((T, nh, hd))
        for h in range(nh):
            s = q[:, h] @ k[:, h // G].T / np.sqrt(hd) + mask
            s = np.exp(s - s.max(-1, keepdims=True))
            ctx[:, h] = (s / s.sum(-1, keepdims=True)) @ v[:, h // G]
        x = x + ctx.reshape(T, -1) @ p("attn.wo.weight").T
        xn = rms(x, p("ln2.weight"))
        g, u = xn @ p("mlp.gate.weight").T, xn @ p("mlp.up.weight").T
        x = x + (g / (1 + np.exp(-g)) * u) @ p("mlp.down.weight").T
    head = w["tok.weight"] if cfg["tie_embeddings"] else w["lm_head.weight"]
    return rms(x, w["norm.weight"]) @ f(head).T


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


CFGS = [TINY, dict(TINY, tie_embeddings=0), dict(TINY, qk_norm=0, n_kv_heads=4), dict(TINY, n_kv_heads=1)]


@pytest.mark.parametrize("cfg", CFGS, ids=["tied", "untied", "no_qknorm_mha", "mqa"])
def test_oracle_f32_matches_numpy_forward(cfg):
    w = o.qwen3_init(cfg, seed=3, gain_noise=0.2)
    # Larger weights than the reference init so attention is far from uniform.
    for n in w:
        if "attn.w" in n:
            w[n] = w[n] * 20.0
    prompts = np.random.default_rng(1).integers(0, cfg["vocab"], size=(2, 7))
    steps = 5
    toks, logits = o.qwen3_generate(cfg, w, prompts, steps, int8=False)
    for b in range(prompts.shape[0]):
        seq = list(prompts[b]) + list(toks[:steps, b])
        ref = np_forward(cfg, w, seq)[prompts.shape[1] - 1:]
        assert rel_l2(logits[:, b], ref) < 1e-5
        assert (toks[:, b] == ref.argmax(-1)).all()


def test_oracle_int8_tracks_f32():
    cfg = dict(TINY, d_model=64, d_ff=128)
    w = o.qwen3_init(cfg, seed=11)
    prompts = np.random.default_rng(2).integers(0, cfg["vocab"], size=(2, 6))
    _, lf = o.qwen3_generate(cfg, w, prompts, 0, int8=False)
    _, lq = o.qwen3_generate(cfg, w, prompts, 0, int8=True)
    r = rel_l2(lq, lf)
    assert 0 < r < 0.10, r


def test_oracle_int8_linears_are_the_pinned_path():
    """With every layer's contribution zeroed (wo = down = 0) the logits are the
    int8 head applied to rmsnorm(emb[tok]); that head is or_matmul_i8 on
    or_quantize_weight / or_max_abs_row / or_quant_pack, all pinned on their own."""
    cfg = TINY
    w = o.qwen3_init(cfg, seed=5, gain_noise=0.3)
    for n in w:
        if n.endswith(("attn.wo.weight", "mlp.down.weight")):
            w[n][:] = 0
    prompts = np.array([[4, 9, 1]])
    _, logits = o.qwen3_generate(cfg, w, prompts, 0, int8=True)
    x = w["tok.weight"][1].astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(np.float32((x * x).sum(dtype=np.float32)) / np.float32(32) + np.float32(1e-6))
    xn = (x * inv * w["norm.weight"]).astype(np.float32)[None]
    wq, sw = o.quantize_weight(w["tok.weight"])
    sx = o.max_abs_row(xn)
    want = o.matmul_i8(o.quant_pack(xn, sx), wq, sx, sw)
    np.testing.assert_allclose(logits[0, 0], want[0], rtol=1e-5, atol=1e-6)


def test_argmax_rule():
    nan, inf = np.nan, np.inf
    assert o.argmax_row([1.0, 3.0, 3.0, 2.0]) == 1           # first maximum
    assert o.argmax_row([nan, 1.0, nan, 2.0]) == 3           # NaN never wins
    assert o.argmax_row([nan, nan]) == 0                     # nothing valid -> 0
    assert o.argmax_row([-inf, -inf]) == 0
    assert o.argmax_row([-3.4028235e38, -inf]) == 0          # must be strictly above -FLT_MAX
    assert o.argmax_row([-inf, -1e30, 5.0, inf]) == 3


def test_oracle_int8_kv_tracks_fp32_kv():
    """crates/qwen3/src/model.rs:2638-2661 (int8_kv_decode_tracks_fp32): the
    int8 KV cache stays within rel-L2 0.10 of the f32 cache."""
    cfg = dict(TINY, d_model=64, d_ff=128)
    w = o.qwen3_init(cfg, seed=13, gain_noise=0.1)
    prompts = np.random.default_rng(4).integers(0, cfg["vocab"], size=(2, 6))
    _, l32 = o.qwen3_generate(cfg, w, prompts, 3, int8=True)
    _, l8 = o.qwen3_generate(dict(cfg, kv_int8=1), w, prompts, 3, int8=True)
    r = rel_l2(l8[0], l32[0])
    assert 0 < r < 0.10, r
