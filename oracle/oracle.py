"""numpy/ctypes front end of the C oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker. Each wrapper names the C function (and through it the
reference file:line) it calls. `acc_exact` additionally offers an exact i32
accumulator through float64 BLAS for shapes where the scalar C loop is too
slow: every product is an integer of magnitude <= 127*127 and every partial
sum is an integer below 127*127*K < 2**53 for K < 5.5e8, so float64
arithmetic is exact and any summation order gives the same integer.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        vp, i64, i32, u64, u32 = C.c_void_p, C.c_int64, C.c_int, C.c_uint64, C.c_uint32
        sig = {
            "or_rng_new": (None, [vp, u64]),
            "or_rng_next_u64": (u64, [vp]),
            "or_rng_next_f64": (C.c_double, [vp]),
            "or_rng_next_f32": (C.c_float, [vp]),
            "or_rng_gen_range_inclusive": (i64, [vp, i64, i64]),
            "or_rng_uniform": (C.c_double, [vp, C.c_double, C.c_double]),
            "or_rng_next_gaussian": (C.c_double, [vp]),
            "or_quantize_weight": (None, [vp, i64, i64, vp, vp]),
            "or_dequantize_weight": (None, [vp, vp, i64, i64, vp]),
            "or_max_abs_row": (None, [vp, i64, i64, vp]),
            "or_quant_pack": (None, [vp, vp, i64, i64, vp]),
            "or_matmul_i8_acc": (None, [vp, vp, i64, i64, i64, vp]),
            "or_epilogue": (None, [vp, vp, vp, vp, i64, i64, i32, vp]),
            "or_epilogue_static": (None, [vp, C.c_float, C.c_float, i64, i64, vp]),
            "or_matmul_i8": (None, [vp, vp, vp, vp, vp, i64, i64, i64, i32, vp]),
            "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "or_f32_to_bf16_array": (None, [C.c_void_p, C.c_void_p, C.c_size_t]),
            "or_cpu_linear_gemv": (None, [vp, vp, vp, i64, i64, i64, i32, vp, vp, vp]),
            "or_cpu_gemv_packed": (None, [vp, vp, vp, vp, i64, i64, i64, i32, vp]),
            "or_cpu_gemm_i8_tiled": (None, [vp, vp, vp, vp, i64, i64, i64, i32, vp]),
            "or_argmax_row": (u32, [vp, u32]),
            "or_quantize_weight_q4": (None, [vp, i64, i64, vp, vp]),
            "or_dequantize_weight_q4": (None, [vp, vp, i64, i64, vp]),
            "or_matmul_q4_acc": (None, [vp, vp, i64, i64, i64, vp]),
            "or_qwen3_param_count": (u64, [vp]),
            "or_qwen3_generate": (i32, [vp, vp, i32, vp, u32, u32, u32, vp, vp]),
            "or_qwen3_cpu_decode": (C.c_double, [vp, u64, i32, u32, u32]),
            "or_qwen3_generate_clip": (i32, [vp, vp, i32, vp, u32, u32, u32, vp, vp, vp, vp]),
            "or_kv8_code": (C.c_int8, [C.c_float, C.c_float]),
            "or_paged_kv_append_i8_clipped": (None, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32]),
            "or_paged_decode_scores_i8": (None, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32,
                                                 C.c_float]),
            "or_paged_decode_apply_i8": (None, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class Rng:
    """crates/data/src/rng.rs SplitMix64 via or_rng_*."""

    class _S(C.Structure):
        _fields_ = [("state", C.c_uint64)]

    def __init__(self, seed):
        self.s = Rng._S()
        lib().or_rng_new(C.byref(self.s), seed)

    def next_u64(self):
        return lib().or_rng_next_u64(C.byref(self.s))

    def next_f64(self):
        return lib().or_rng_next_f64(C.byref(self.s))

    def next_f32(self):
        return lib().or_rng_next_f32(C.byref(self.s))

    def gen_range_inclusive(self, lo, hi):
        return lib().or_rng_gen_range_inclusive(C.byref(self.s), lo, hi)

    def uniform(self, lo, hi):
        return lib().or_rng_uniform(C.byref(self.s), lo, hi)

    def next_gaussian(self):
        return lib().or_rng_next_gaussian(C.byref(self.s))


def quantize_weight(w):
    """or_quantize_weight (crates/model/src/int8.rs:33-59) -> (packed u32 [n,k/4], sw f32 [n])."""
    w = _c(w, np.float32)
    n, k = w.shape
    packed = np.zeros((n, k // 4), np.uint32)
    sw = np.zeros(n, np.float32)
    lib().or_quantize_weight(_p(w), n, k, _p(packed), _p(sw))
    return packed, sw


def dequantize_weight(packed, sw, k):
    packed = _c(packed, np.uint32)
    sw = _c(sw, np.float32)
    n = packed.shape[0]
    w = np.zeros((n, k), np.float32)
    lib().or_dequantize_weight(_p(packed), _p(sw), n, k, _p(w))
    return w


def max_abs_row(x):
    """or_max_abs_row (max_abs_row.wgsl:27-34)."""
    x = _c(x, np.float32)
    m, k = x.shape
    sx = np.zeros(m, np.float32)
    lib().or_max_abs_row(_p(x), m, k, _p(sx))
    return sx


def quant_pack(x, sx):
    """or_quant_pack (quant_pack.wgsl:29-44)."""
    x = _c(x, np.float32)
    sx = _c(sx, np.float32)
    m, k = x.shape
    xq = np.zeros((m, k // 4), np.uint32)
    lib().or_quant_pack(_p(x), _p(sx), m, k, _p(xq))
    return xq


def matmul_i8_acc(xq, wq):
    """or_matmul_i8_acc — exact wrapping-i32 sums, scalar C loop."""
    xq = _c(xq, np.uint32)
    wq = _c(wq, np.uint32)
    m, kg = xq.shape
    n = wq.shape[0]
    acc = np.zeros((m, n), np.int32)
    lib().or_matmul_i8_acc(_p(xq), _p(wq), m, kg, n, _p(acc))
    return acc


def unpack_i8(packed):
    """[r, kg] u32 words -> [r, 4*kg] int8 (byte b of word g is element 4g+b)."""
    p = _c(packed, np.uint32)
    return p.view(np.int8).reshape(p.shape[0], p.shape[1] * 4)


def acc_exact(xq, wq, rows=None, cols=None):
    """Exact i32 accumulators through float64 BLAS (see module doc); optional
    row/col index arrays restrict the result to that sub-grid."""
    a = unpack_i8(xq if rows is None else np.asarray(xq)[rows]).astype(np.float64)
    b = unpack_i8(wq if cols is None else np.asarray(wq)[cols]).astype(np.float64)
    assert a.shape[1] * 127 * 127 < 2**53
    return (a @ b.T).astype(np.int64).astype(np.int32)


def epilogue(acc, sx, sw, bias=None, out_dtype="f32"):
    """or_epilogue: (f32(acc)*sx)*sw (+bias), f32 or bf16 bits (uint16)."""
    acc = _c(acc, np.int32)
    m, n = acc.shape
    sx = _c(sx, np.float32)
    sw = _c(sw, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    code = {"f32": 0, "bf16": 1}[out_dtype]
    out = np.zeros((m, n), np.float32 if code == 0 else np.uint16)
    lib().or_epilogue(_p(acc), _p(sx), _p(sw), _p(b), m, n, code, _p(out))
    return out


def epilogue_static(acc, sx, sw):
    acc = _c(acc, np.int32)
    m, n = acc.shape
    out = np.zeros((m, n), np.float32)
    lib().or_epilogue_static(_p(acc), float(sx), float(sw), m, n, _p(out))
    return out


def matmul_i8(xq, wq, sx, sw, bias=None, out_dtype="f32"):
    """or_matmul_i8: exact accumulators + epilogue."""
    return epilogue(matmul_i8_acc(xq, wq), sx, sw, bias, out_dtype)


def f32_to_bf16(f):
    return lib().or_f32_to_bf16(float(f))


def f32_to_bf16_array(x):
    """or_f32_to_bf16 applied to every element of f32 array x -> uint16 bits."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def cpu_linear_gemv(x, wq, sw, threads):
    """The restated backend-cpu decode path: max_abs_row -> quant_pack -> matmul_i8_gemv."""
    x = _c(x, np.float32)
    wq = _c(wq, np.uint32)
    sw = _c(sw, np.float32)
    m, k = x.shape
    n = wq.shape[0]
    sx = np.zeros(m, np.float32)
    xq = np.zeros((m, k // 4), np.uint32)
    out = np.zeros((m, n), np.float32)
    lib().or_cpu_linear_gemv(_p(x), _p(wq), _p(sw), m, k, n, threads, _p(sx), _p(xq), _p(out))
    return out


def cpu_gemv_packed(xq, wq, sx, sw, threads):
    xq = _c(xq, np.uint32)
    wq = _c(wq, np.uint32)
    sx = _c(sx, np.float32)
    sw = _c(sw, np.float32)
    m, kg = xq.shape
    n = wq.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().or_cpu_gemv_packed(_p(xq), _p(wq), _p(sx), _p(sw), m, kg, n, threads, _p(out))
    return out


def cpu_gemm_tiled(xq, wq, sx, sw, threads):
    """OpenMP tiled i32 GEMM on the host (prefill CPU reference)."""
    xq = _c(xq, np.uint32)
    wq = _c(wq, np.uint32)
    sx = _c(sx, np.float32)
    sw = _c(sw, np.float32)
    m, kg = xq.shape
    n = wq.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().or_cpu_gemm_i8_tiled(_p(xq), _p(wq), _p(sx), _p(sw), m, kg, n, threads, _p(out))
    return out


# ---- synthetic inputs of the BASELINE configs (seeded SplitMix64) -----------

def synth_weights(n, k, seed):
    """int8 uniform in [-127,127] (gen_range_inclusive), sw ~ U(0.002, 0.02).
    Vectorised SplitMix64: identical stream to Rng(seed)."""
    u = splitmix_u64(seed, n * k + n)
    q = (u[: n * k] % np.uint64(255)).astype(np.int64) - 127
    wq = q.astype(np.int8).reshape(n, k).view(np.uint32).reshape(n, k // 4)
    f = (u[n * k:] >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    sw = (0.002 + (0.02 - 0.002) * f).astype(np.float32)
    return np.ascontiguousarray(wq), sw


def synth_acts(m, k, seed):
    """x ~ N(0,1) by Box-Muller on the SplitMix64 stream (rng.rs next_gaussian)."""
    u = splitmix_u64(seed, 2 * m * k)
    f = (u >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    u1 = np.maximum(f[0::2], 1e-12)
    u2 = f[1::2]
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2 * np.pi * u2)
    return g.astype(np.float32).reshape(m, k)


_GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix_u64(seed, count):
    """The first `count` outputs of Rng::new(seed).next_u64(), vectorised."""
    with np.errstate(over="ignore"):
        st = np.uint64(seed) + _GAMMA + _GAMMA * np.arange(1, count + 1, dtype=np.uint64)
        z = st
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


# ---------------------------------------------------------------- Qwen3 decoder
class Qwen3Config(C.Structure):
    """or_qwen3_config (qwen3_oracle.h), the QwenConfig fields the forward reads."""
    _fields_ = [(n, C.c_uint32) for n in ("vocab", "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "d_ff")] + \
               [("rope_theta", C.c_float), ("rms_eps", C.c_float), ("tie_embeddings", C.c_uint32), ("qk_norm", C.c_uint32),
                ("kv_int8", C.c_uint32)]


def qwen3_param_list(cfg):
    """(name, shape) in decoder_param_list order (crates/qwen3/src/serve.rs:320-340)."""
    d, ff, hd = cfg["d_model"], cfg["d_ff"], cfg["head_dim"]
    hq, hkv = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    out = []
    for l in range(cfg["n_layers"]):
        p = f"blocks.{l}."
        out += [(p + "ln1.weight", (d,)), (p + "attn.wq.weight", (hq, d)), (p + "attn.wk.weight", (hkv, d)),
                (p + "attn.wv.weight", (hkv, d)), (p + "attn.q_norm.weight", (hd,)), (p + "attn.k_norm.weight", (hd,)),
                (p + "attn.wo.weight", (d, hq)), (p + "ln2.weight", (d,)), (p + "mlp.gate.weight", (ff, d)),
                (p + "mlp.up.weight", (ff, d)), (p + "mlp.down.weight", (d, ff))]
    out += [("norm.weight", (d,)), ("tok.weight", (cfg["vocab"], d))]
    if not cfg.get("tie_embeddings", 1):
        out.append(("lm_head.weight", (cfg["vocab"], d)))
    return out


def qwen3_init(cfg, seed, gain_noise=0.0):
    """Seeded weights with the reference's distributions (crates/qwen3/src/init.rs:30-59):
    gains 1 (plus optional noise so they matter in a test), wo/down N(0, 0.02/sqrt(2L)),
    everything else N(0, 0.02). numpy's generator, not the reference's stream."""
    rng = np.random.default_rng(seed)
    proj = 0.02 / np.sqrt(2.0 * cfg["n_layers"])
    w = {}
    for name, shape in qwen3_param_list(cfg):
        if name.endswith(("ln1.weight", "ln2.weight", "norm.weight")):
            v = 1.0 + gain_noise * rng.standard_normal(shape)
        elif name.endswith(("attn.wo.weight", "mlp.down.weight")):
            v = proj * rng.standard_normal(shape)
        else:
            v = 0.02 * rng.standard_normal(shape)
        w[name] = v.astype(np.float32)
    return w


def _qcfg(cfg):
    c = Qwen3Config()
    for k in ("vocab", "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "d_ff"):
        setattr(c, k, cfg[k])
    c.rope_theta, c.rms_eps = cfg.get("rope_theta", 1e6), cfg.get("rms_eps", 1e-6)
    c.tie_embeddings, c.qk_norm = cfg.get("tie_embeddings", 1), cfg.get("qk_norm", 1)
    c.kv_int8 = cfg.get("kv_int8", 0)
    return c


def qwen3_generate(cfg, weights, prompts, steps, int8=True, kclip=None, vclip=None):
    """or_qwen3_generate_clip: greedy tokens [(steps+1), batch] and logits
    [(steps+1), batch, vocab]; kclip/vclip [n_layers, n_kv_heads] are the int8
    KV clip ceilings (None: FLT_MAX)."""
    c = _qcfg(cfg)
    blob = np.concatenate([weights[n].ravel() for n, _ in qwen3_param_list(cfg)]).astype(np.float32)
    assert blob.size == lib().or_qwen3_param_count(C.byref(c))
    prompts = _c(prompts, np.uint32)
    batch, ln = prompts.shape
    toks = np.zeros((steps + 1, batch), np.uint32)
    logits = np.zeros((steps + 1, batch, cfg["vocab"]), np.float32)
    kc = None if kclip is None else _c(kclip, np.float32)
    vc = None if vclip is None else _c(vclip, np.float32)
    for t in (kc, vc):
        assert t is None or t.size == cfg["n_layers"] * cfg["n_kv_heads"]
    rc = lib().or_qwen3_generate_clip(C.byref(c), _p(blob), 1 if int8 else 0, _p(prompts), batch, ln, steps,
                                      _p(toks), _p(logits), _p(kc), _p(vc))
    assert rc == 0
    return toks, logits


def argmax_row(x):
    x = _c(x, np.float32)
    return lib().or_argmax_row(_p(x), x.size)


def qwen3_cpu_decode_seconds(cfg, threads, ctx, steps, seed=1):
    """or_qwen3_cpu_decode: seconds for `steps` batch-1 int8 decode steps on the CPU."""
    c = _qcfg(cfg)
    return lib().or_qwen3_cpu_decode(C.byref(c), seed, threads, ctx, steps)


# ---------------------------------------------------------------- W4A8
def quantize_weight_q4(w):
    """or_quantize_weight_q4 (crates/model/src/int4.rs:46-67) -> (packed u32 [n,k/8], sw f32 [n])."""
    w = _c(w, np.float32)
    n, k = w.shape
    packed = np.zeros((n, k // 8), np.uint32)
    sw = np.zeros(n, np.float32)
    lib().or_quantize_weight_q4(_p(w), n, k, _p(packed), _p(sw))
    return packed, sw


def dequantize_weight_q4(packed, sw, k):
    packed = _c(packed, np.uint32)
    sw = _c(sw, np.float32)
    out = np.zeros((packed.shape[0], k), np.float32)
    lib().or_dequantize_weight_q4(_p(packed), _p(sw), packed.shape[0], k, _p(out))
    return out


def matmul_q4_acc(xq, w4, k):
    """or_matmul_q4_acc: exact i32 [m, n] (scalar C; small shapes)."""
    xq = _c(xq, np.uint32)
    w4 = _c(w4, np.uint32)
    m, n = xq.shape[0], w4.shape[0]
    acc = np.zeros((m, n), np.int32)
    lib().or_matmul_q4_acc(_p(xq), _p(w4), m, k, n, _p(acc))
    return acc


def unpack_q4(w4, k):
    """Signed int4 values [n, k] of packed [n, k/8] (numpy, for float64-BLAS exact sums)."""
    w4 = _c(w4, np.uint32)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    nib = ((w4[:, :, None] >> shifts[None, None, :]) & 0xF).astype(np.int16)
    nib = np.where(nib >= 8, nib - 16, nib)
    return nib.reshape(w4.shape[0], -1)[:, :k].astype(np.int8)


def acc_exact_q4(xq, w4, k, rows=None, cols=None):
    """Exact i32 accumulators through float64 BLAS (|acc| < 127*7*k < 2**53)."""
    a = unpack_i8(xq if rows is None else np.asarray(xq)[rows]).astype(np.float64)[:, :k]
    b = unpack_q4(w4 if cols is None else np.asarray(w4)[cols], k).astype(np.float64)
    return (a @ b.T).astype(np.int64).astype(np.int32)


# ---------------------------------------------------------------- int8 paged KV
def kv8_code(x, scale):
    """or_kv8_code: clamp(i32(round_even(x / scale)), -127, 127)."""
    return int(lib().or_kv8_code(float(x), float(scale)))


def paged_kv_append_i8(src, blocks, offsets, clip, pool, scales, block_size, head_dim):
    """or_paged_kv_append_i8_clipped on (copies of) pool [u32 words] and scales; returns both."""
    src = _c(src, np.float32)
    batch, kv_stride = src.shape
    blocks, offsets, clip = _c(blocks, np.uint32), _c(offsets, np.uint32), _c(clip, np.float32)
    pool = _c(pool, np.uint32).copy()
    scales = _c(scales, np.float32).copy()
    lib().or_paged_kv_append_i8_clipped(_p(src), _p(blocks), _p(offsets), _p(clip), _p(pool), _p(scales), batch,
                                        kv_stride, block_size, head_dim)
    return pool, scales


def paged_decode_scores_i8(q, pool, block_tables, seq_lens, scales, scores, n_heads, group, head_dim, block_size,
                           kv_stride, cap, scale):
    """or_paged_decode_scores_i8; `scores` [batch, n_heads, cap] is copied and
    returned with the entries below each seq_len overwritten."""
    block_tables = _c(block_tables, np.uint32)
    batch, max_bt = block_tables.shape
    q, pool, seq_lens, scales = _c(q, np.float32), _c(pool, np.uint32), _c(seq_lens, np.uint32), _c(scales, np.float32)
    out = _c(scores, np.float32).copy()
    lib().or_paged_decode_scores_i8(_p(q), _p(pool), _p(block_tables), _p(seq_lens), _p(scales), _p(out), batch,
                                    n_heads, group, head_dim, block_size, kv_stride, cap, max_bt, scale)
    return out


def paged_decode_apply_i8(probs, pool, block_tables, seq_lens, scales, n_heads, group, head_dim, block_size,
                          kv_stride, cap):
    """or_paged_decode_apply_i8: ctx [batch, n_heads*head_dim]."""
    block_tables = _c(block_tables, np.uint32)
    batch, max_bt = block_tables.shape
    probs, pool = _c(probs, np.float32), _c(pool, np.uint32)
    seq_lens, scales = _c(seq_lens, np.uint32), _c(scales, np.float32)
    ctx = np.zeros((batch, n_heads * head_dim), np.float32)
    lib().or_paged_decode_apply_i8(_p(probs), _p(pool), _p(block_tables), _p(seq_lens), _p(scales), _p(ctx), batch,
                                   n_heads, group, head_dim, block_size, kv_stride, cap, max_bt)
    return ctx
