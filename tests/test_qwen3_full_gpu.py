"""Config 3 at full size (Qwen3-0.6B: 28 layers, d 1024, 16q/8kv heads of
128, ff 3072, vocab 151936, RoPE theta 1e6, tied embeddings, QK-norm)
against the C oracle, with positions past 512 so the rotation tables,
the 151936-wide two-stage argmax and the K = 3072 linears are exercised at
their real sizes.

The engine's int8 linears are bit-exact with the oracle's, but its f32
reductions (RMSNorm sums, the chunked attention merge) round differently, so
an activation now and then lands on the other side of an int8 rounding
boundary, and in these random models one such flip moves the logits by about
1% rel-L2: the oracle itself moves by 0.8-2% when only its norm gains are
perturbed by one ulp (its f32 model by 3e-7), at 2 layers and 64 positions
as at 8-12 layers. Through 8 layers with 4 positions, or 2 layers with 32
(one attention chunk), the engine matches the oracle to 1e-7 or exactly. So:
  - the full 28-layer model meets the reference's own int8-vs-fp32 bound,
    rel-L2 < 0.10 (crates/qwen3/src/model.rs:2638-2661), and stays within
    NOISE = 2e-2 of the int8 oracle at every step of a 520-token prompt,
    greedy tokens equal where the oracle's top-2 margin clears that noise;
  - what that bar could hide is pinned directly: layer 0's rotated keys at
    all 600 positions against a float64 restatement (a wrong rotation
    table past 512 moves a row by O(1)), and the device argmax against
    the first maximum of the 151936 logits it returns.
"""
import numpy as np
import pytest

from brain_amd.qwen3 import QWEN3_0_6B, Qwen3Engine
from oracle import oracle as o

pytestmark = pytest.mark.gpu

NOISE = 2e-2


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def full_weights(seed):
    """The reference's init distributions (crates/qwen3/src/init.rs:30-59)
    with the test decoder's scalings (embedding x10 for clear logit margins,
    attention x3 so that attention is far from uniform), drawn in f32."""
    cfg = QWEN3_0_6B
    rng = np.random.default_rng(seed)
    proj = 0.02 / np.sqrt(2.0 * cfg["n_layers"])
    w = {}
    for name, shape in o.qwen3_param_list(cfg):
        if len(shape) == 1:
            w[name] = (1.0 + 0.2 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
            continue
        std = proj if name.endswith(("attn.wo.weight", "mlp.down.weight")) else 0.02
        if name == "tok.weight":
            std *= 10.0
        elif "attn.w" in name:
            std *= 3.0
        w[name] = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
    return w


@pytest.fixture(scope="module")
def weights():
    return full_weights(5)


def test_full_size_short_prompt_within_reference_bound(gpu, weights):
    cfg = QWEN3_0_6B
    prompts = np.random.default_rng(1).integers(0, cfg["vocab"], size=(2, 4))
    _, logits_f = o.qwen3_generate(cfg, weights, prompts, 0, int8=False)
    _, logits_o = o.qwen3_generate(cfg, weights, prompts, 0, int8=True)
    e = Qwen3Engine(cfg, 2, 8)
    e.load_weights(weights)
    e.prefill(prompts)
    got = e.logits()
    e.close()
    for b in range(2):
        assert rel_l2(got[b], logits_f[0][b]) < 0.10
        assert rel_l2(got[b], logits_o[0][b]) < NOISE


def test_full_size_past_position_512_matches_oracle(gpu, weights):
    cfg = QWEN3_0_6B
    plen, steps = 520, 3
    prompts = np.random.default_rng(2).integers(0, cfg["vocab"], size=(1, plen))
    toks_o, logits_o = o.qwen3_generate(cfg, weights, prompts, steps, int8=True)
    e = Qwen3Engine(cfg, 1, plen + steps + 1, max_rows=256)  # chunked prefill: GEMM and GEMV linears
    e.load_weights(weights)
    got_toks = [e.prefill(prompts)]
    got_logits = [e.logits()]
    for _ in range(steps):
        got_toks.append(e.decode(1)[0])
        got_logits.append(e.logits())
    e.close()
    errs = [rel_l2(got_logits[s][0], logits_o[s][0]) for s in range(steps + 1)]
    print("full-size rel-L2 per step vs the int8 oracle:", errs)
    checked = 0
    for s in range(steps + 1):
        assert errs[s] < NOISE, (s, errs)
        top2 = np.sort(logits_o[s][0])[-2:]
        if top2[1] - top2[0] > NOISE * np.abs(logits_o[s][0]).max():
            assert got_toks[s][0] == toks_o[s][0], (s, got_toks[s], toks_o[s])
            checked += 1
        if got_toks[s][0] != toks_o[s][0]:
            break
    assert checked >= 1


def test_rotated_keys_past_position_512(gpu, weights):
    """Layer 0's cached keys over 600 positions against a float64 restatement
    (int8 k projection of the RMSNorm'd embedding, per-head QK-norm, the
    rotate-half RoPE of rope_paged.wgsl:27-38 with theta 1e6). The keys do
    not depend on attention, so an f32 engine reproduces them up to f32
    rounding and the rare int8 flip; a wrong rotation table at any position
    (past 512 in particular) moves that row by O(1)."""
    cfg = dict(QWEN3_0_6B, n_layers=1)
    w = {n: weights[n] for n, _ in o.qwen3_param_list(cfg)}
    plen, d, hd, nkv = 600, cfg["d_model"], cfg["head_dim"], cfg["n_kv_heads"]
    prompts = np.random.default_rng(4).integers(0, cfg["vocab"], size=(1, plen))
    e = Qwen3Engine(cfg, 1, plen + 1, max_rows=256)
    e.load_weights(w)
    e.prefill(prompts)
    k_eng = e.kv(0, 0, 0, plen).astype(np.float64).reshape(plen, nkv, hd)
    e.close()
    x = w["tok.weight"][prompts[0]]
    inv = 1.0 / np.sqrt((x.astype(np.float32) ** 2).sum(1, dtype=np.float32) / np.float32(d) + np.float32(1e-6))
    xn = (x * inv[:, None].astype(np.float32) * w["blocks.0.ln1.weight"]).astype(np.float32)
    sx = o.max_abs_row(xn)
    wk, swk = o.quantize_weight(w["blocks.0.attn.wk.weight"])
    k = o.matmul_i8(o.quant_pack(xn, sx), wk, sx, swk).astype(np.float64).reshape(plen, nkv, hd)
    k = k / np.sqrt((k ** 2).mean(-1, keepdims=True) + 1e-6) * w["blocks.0.attn.k_norm.weight"]
    half = hd // 2
    ang = np.arange(plen)[:, None] * cfg["rope_theta"] ** (-2.0 * np.arange(half)[None, :] / hd)
    c, s_ = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    ref = np.concatenate([k[..., :half] * c - k[..., half:] * s_, k[..., half:] * c + k[..., :half] * s_], -1)
    err = np.abs(k_eng - ref).max(axis=(1, 2)) / np.abs(ref).max(axis=(1, 2))
    print("rotated-key row error: median %.2e, max %.2e" % (np.median(err), err.max()))
    assert np.median(err) < 1e-5
    assert (err < 1e-3).mean() > 0.98 and (err[512:] < 1e-3).mean() > 0.95
    assert err.max() < 5e-2


def test_greedy_token_is_the_argmax_of_the_full_vocab(gpu, weights):
    """The engine's two-stage device argmax over 151936 logits picks the
    first largest entry of the logits it returns (argmax_row.wgsl)."""
    cfg = dict(QWEN3_0_6B, n_layers=1)
    w = {n: weights[n] for n, _ in o.qwen3_param_list(cfg)}
    prompts = np.random.default_rng(5).integers(0, cfg["vocab"], size=(4, 6))
    e = Qwen3Engine(cfg, 4, 16)
    e.load_weights(w)
    toks = [e.prefill(prompts)]
    lg = [e.logits()]
    for _ in range(3):
        toks.append(e.decode(1)[0])
        lg.append(e.logits())
    e.close()
    for t, l in zip(toks, lg):
        assert [o.argmax_row(r) for r in l] == list(t)
        assert list(np.argmax(l, axis=1)) == list(t)


def test_full_size_batch8_128_token_prompt_matches_oracle(gpu, weights):
    """configs[3] at the bench's own shape: batch 8, a 128-token prompt
    (prefilled as one 1024-row chunk, max_rows = 8 x 128 as in the bench),
    then 3 greedy steps through the batch-8 decode graph (separate norm and
    SwiGLU kernels above 4 rows, 8 live rows in every launch), every
    sequence against the int8 oracle under the same bar as the batch-1
    test: within NOISE at every step, tokens equal where the oracle's top-2
    margin clears the noise (the reference's own bound is
    crates/qwen3/src/model.rs:2638-2661)."""
    cfg = QWEN3_0_6B
    batch, plen, steps = 8, 128, 3
    prompts = np.random.default_rng(8).integers(0, cfg["vocab"], size=(batch, plen))
    toks_o, logits_o = o.qwen3_generate(cfg, weights, prompts, steps, int8=True)
    e = Qwen3Engine(cfg, batch, plen + steps + 1, max_rows=batch * plen)
    e.load_weights(weights)
    got_toks = [e.prefill(prompts)]
    got_logits = [e.logits()]
    for _ in range(steps):
        got_toks.append(e.decode(1)[0])
        got_logits.append(e.logits())
    e.close()
    checked = 0
    for b in range(batch):
        errs = [rel_l2(got_logits[s][b], logits_o[s][b]) for s in range(steps + 1)]
        print(f"sequence {b}: rel-L2 per step vs the int8 oracle {errs}")
        for s in range(steps + 1):
            assert errs[s] < NOISE, (b, s, errs)
            top2 = np.sort(logits_o[s][b])[-2:]
            if top2[1] - top2[0] > NOISE * np.abs(logits_o[s][b]).max():
                assert got_toks[s][b] == toks_o[s][b], (b, s, got_toks[s], toks_o[s])
                checked += 1
            if got_toks[s][b] != toks_o[s][b]:
                break
    assert checked >= batch
