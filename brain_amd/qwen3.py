"""The int8 Qwen3 decoder engine (section D of include/brain_hip.h).

Mirrors the serving surface of qwen3::serve::Engine with int8 weights
(crates/qwen3/src/serve.rs): weights by their reference names
(`decoder_param_list`, serve.rs:320-340), prompt prefill (serve.rs:1557-1620)
and greedy decode with the head and argmax on the device (serve.rs:1332-1367,
1846 `generate_greedy`). All compute runs in libbrain_hip.so; this class only
marshals host arrays.
"""
import ctypes as C

import numpy as np

from ._lib import Qwen3ConfigT, check, load

QWEN3_0_6B = dict(vocab=151936, n_layers=28, d_model=1024, n_heads=16, n_kv_heads=8, head_dim=128,
                  d_ff=3072, rope_theta=1.0e6, rms_eps=1e-6, tie_embeddings=1, qk_norm=1, kv_int8=0,
                  kv_block_size=0, kv_num_blocks=0)
"""QwenConfig::qwen3_0_6b (crates/qwen3/src/config.rs:100-118)."""

EAGER = 1
UNFUSED = 2
NO_BLOCK = 0xFFFFFFFF


class Qwen3Engine:
    def __init__(self, cfg, max_batch, max_seq, max_rows=None, device=0):
        self.cfg = dict(QWEN3_0_6B, **cfg) if cfg is not QWEN3_0_6B else dict(cfg)
        c = Qwen3ConfigT()
        for k in ("vocab", "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "d_ff", "tie_embeddings", "qk_norm",
                  "kv_int8", "kv_block_size", "kv_num_blocks"):
            setattr(c, k, int(self.cfg[k]))
        c.rope_theta, c.rms_eps = float(self.cfg["rope_theta"]), float(self.cfg["rms_eps"])
        self._h = C.c_void_p()
        self.max_batch = max_batch
        check(load().bh_qwen3_create(C.byref(c), max_batch, max_seq, max_rows or max_batch * max_seq, device,
                                     C.byref(self._h)))
        self.batch = 0

    def close(self):
        if self._h:
            load().bh_qwen3_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return load().bh_qwen3_stream(self._h)

    def set_weight(self, name, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        check(load().bh_qwen3_set_weight(self._h, name.encode(), w.ctypes.data, w.size))

    def set_weight_i8(self, name, packed, scale):
        packed = np.ascontiguousarray(packed, dtype=np.uint32)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        n, kw = packed.shape
        check(load().bh_qwen3_set_weight_i8(self._h, name.encode(), packed.ctypes.data, scale.ctypes.data, n, kw * 4))

    def load_weights(self, weights):
        for name, w in weights.items():
            self.set_weight(name, w)

    def load(self, path):
        """Every parameter from an int8 safetensors checkpoint (brain_amd.int8_format)."""
        check(load().bh_qwen3_load(self._h, path.encode()))

    def set_kv_clip(self, layer, which, clip):
        """int8 KV ceilings per kv head for layer `layer`, K (which=0) or V (1)."""
        clip = np.ascontiguousarray(clip, dtype=np.float32)
        check(load().bh_qwen3_set_kv_clip(self._h, layer, which, clip.ctypes.data))

    def set_block_table(self, table):
        """Paged pool (kv_block_size > 0): table [rows, max_blocks_per_seq] of
        physical blocks (NO_BLOCK = unallocated), as the reference's
        BlockAllocator hands them out."""
        t = np.ascontiguousarray(table, dtype=np.uint32)
        check(load().bh_qwen3_set_block_table(self._h, t.ctypes.data, t.shape[0], t.shape[1]))

    def kv_pool(self, layer, which):
        """Device pointers of one layer's K/V pool: (pool, pool_words, scales, n_scales)."""
        pool, words, sc, ns = C.c_void_p(), C.c_uint64(), C.c_void_p(), C.c_uint64()
        check(load().bh_qwen3_kv_pool(self._h, layer, which, C.byref(pool), C.byref(words), C.byref(sc),
                                      C.byref(ns)))
        return pool.value, words.value, sc.value, ns.value

    def autotune(self, reps=8):
        """Measure GEMV vs tile for every linear shape at row buckets up to max_batch."""
        return check(load().bh_qwen3_autotune(self._h, reps))

    def init_random(self, seed):
        check(load().bh_qwen3_init_random(self._h, seed))

    def prefill(self, prompts):
        """prompts [batch, len] -> next token per sequence [batch]."""
        prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
        batch, ln = prompts.shape
        nxt = np.zeros(batch, np.uint32)
        check(load().bh_qwen3_prefill(self._h, prompts.ctypes.data, batch, ln, nxt.ctypes.data))
        self.batch = batch
        return nxt

    def decode(self, steps, eager=False, unfused=False):
        """`steps` greedy steps -> tokens [steps, batch]. `unfused`: every
        producer as its own kernel (bit-identical results; validation aid)."""
        out = np.zeros((steps, self.batch), np.uint32)
        flags = (EAGER if eager else 0) | (UNFUSED if unfused else 0)
        check(load().bh_qwen3_decode(self._h, steps, flags, out.ctypes.data))
        return out

    def kv(self, layer, seq, which, npos, pos0=0):
        """The engine's cache for (layer, seq): K (which=0) or V (1) over
        positions pos0..pos0+npos. f32 [npos, kv_dim], or with kv_int8
        (int8 codes [npos, kv_dim], scales [npos, n_kv_heads])."""
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        int8 = bool(self.cfg.get("kv_int8", 0))
        data = np.zeros((npos, kvd), np.int8 if int8 else np.float32)
        sc = np.zeros((npos, self.cfg["n_kv_heads"]), np.float32)
        check(load().bh_qwen3_kv_read(self._h, layer, seq, which, pos0, npos, data.ctypes.data,
                                      sc.ctypes.data if int8 else None))
        return (data, sc) if int8 else data

    def logits(self):
        out = np.zeros((self.batch, self.cfg["vocab"]), np.float32)
        check(load().bh_qwen3_logits(self._h, out.ctypes.data, out.size))
        return out

    def generate(self, prompts, steps, eager=False, unfused=False):
        """Greedy tokens [(steps+1), batch]: row 0 from the prefill, then `steps` decode steps."""
        first = self.prefill(prompts)
        rest = self.decode(steps, eager, unfused) if steps else np.zeros((0, len(first)), np.uint32)
        return np.vstack([first[None, :], rest])
