"""The Qwen3 engine on the reference's paged KV pool (kv_block_size > 0):
block tables as crates/qwen3/src/serve.rs hands them out, the pool laid out
as paged_kv_append_i8_clipped_batched.wgsl:46-77 writes it (slot = block *
block_size + offset, int8 codes 4 per word, one scale per (slot, kv head)).

  - Addressing only changes where a key lives, not any arithmetic, so a paged
    engine with a shuffled table gives the slab engine's logits and tokens
    bit for bit (f32 and int8 KV, graph decode, fused and unfused).
  - The int8 pool's codes and scales are the oracle's paged append of the
    same f32 keys/values with the same table, byte for byte, and the
    reference's own paged decode kernel (bh_paged_decode_scores_i8, itself
    bit-exact against the oracle) reads the engine's pool through that table
    to the oracle's scores bit for bit.
  - Tables that leave a used position without a block, or give one block to
    two sequences, are refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from brain_amd import BrainHipError
from brain_amd._lib import check, load
from brain_amd.qwen3 import NO_BLOCK, Qwen3Engine
from oracle import oracle as o
from test_qwen3_gpu import SMALL, scaled_weights

pytestmark = pytest.mark.gpu

FMAX = np.finfo(np.float32).max
BS = 32


def shuffled_table(rng, batch, max_bt, used_blocks, nblk):
    """Distinct random physical blocks for the first `used_blocks` of each
    row, the rest unallocated."""
    phys = rng.permutation(nblk)[:batch * used_blocks].reshape(batch, used_blocks)
    t = np.full((batch, max_bt), NO_BLOCK, np.uint32)
    t[:, :used_blocks] = phys
    return t


def run(cfg, w, prompts, steps, table=None, nblk=0, unfused=False):
    batch, plen = prompts.shape
    max_seq = 96
    paged = table is not None
    e = Qwen3Engine(dict(cfg, kv_block_size=BS if paged else 0, kv_num_blocks=nblk if paged else 0), batch, max_seq)
    e.load_weights(w)
    if paged:
        e.set_block_table(table)
    toks = [e.prefill(prompts)]
    logits = [e.logits()]
    for _ in range(steps):
        toks.append(e.decode(1, unfused=unfused)[0])
        logits.append(e.logits())
    return e, np.array(toks), np.array(logits)


@pytest.mark.parametrize("kv_int8", [0, 1])
@pytest.mark.parametrize("unfused", [False, True])
def test_paged_engine_equals_slab_engine(gpu, kv_int8, unfused):
    cfg = dict(SMALL, kv_int8=kv_int8)
    w = scaled_weights(cfg, seed=51)
    rng = np.random.default_rng(5)
    prompts = rng.integers(0, cfg["vocab"], size=(3, 37))
    steps = 8                                       # positions up to 45: blocks 0 and 1 of each row
    e0, t0, l0 = run(cfg, w, prompts, steps)
    e1, t1, l1 = run(cfg, w, prompts, steps, shuffled_table(rng, 3, 3, 2, 11), nblk=11, unfused=unfused)
    e0.close()
    e1.close()
    assert np.array_equal(t0, t1)
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))


def test_default_table_is_the_slab_layout(gpu):
    cfg = dict(SMALL, kv_int8=1)
    w = scaled_weights(cfg, seed=52)
    prompts = np.random.default_rng(6).integers(0, cfg["vocab"], size=(2, 40))
    e0, t0, l0 = run(cfg, w, prompts, 4)
    e1 = Qwen3Engine(dict(cfg, kv_block_size=BS), 2, 96)      # default: row b owns blocks 3b..3b+2
    e1.load_weights(w)
    t1 = [e1.prefill(prompts)] + [e1.decode(1)[0] for _ in range(4)]
    assert np.array_equal(t0, np.array(t1)) and np.array_equal(l0[-1].view(np.uint32), e1.logits().view(np.uint32))
    for seq in range(2):
        assert np.array_equal(e0.kv(1, seq, 1, 44)[0], e1.kv(1, seq, 1, 44)[0])
    e0.close()
    e1.close()


def test_paged_int8_pool_is_the_reference_layout(gpu):
    cfg = dict(SMALL)
    nkv, hd, nh = cfg["n_kv_heads"], cfg["head_dim"], cfg["n_heads"]
    w = scaled_weights(cfg, seed=53)
    rng = np.random.default_rng(7)
    batch, plen, nblk, max_bt = 3, 45, 10, 3
    prompts = rng.integers(0, cfg["vocab"], size=(batch, plen))
    table = shuffled_table(rng, batch, max_bt, 2, nblk)
    f = Qwen3Engine(dict(cfg, kv_int8=0), batch, 96)            # the f32 keys/values of layer 0
    f.load_weights(w)
    f.prefill(prompts)
    e = Qwen3Engine(dict(cfg, kv_int8=1, kv_block_size=BS, kv_num_blocks=nblk), batch, 96)
    e.load_weights(w)
    e.set_block_table(table)
    kclip = np.array([FMAX, 0.7], np.float32)[:nkv]
    e.set_kv_clip(0, 0, kclip)
    e.prefill(prompts)
    lib = load()
    for which, clip in ((0, kclip), (1, np.full(nkv, FMAX, np.float32))):
        # The oracle's paged append of every (sequence, position), same table.
        pool = np.zeros(nblk * BS * nkv * hd // 4, np.uint32)
        sc = np.zeros(nblk * BS * nkv, np.float32)
        for b in range(batch):
            x = f.kv(0, b, which, plen)
            pos = np.arange(plen)
            pool, sc = o.paged_kv_append_i8(x, table[b, pos // BS], (pos % BS).astype(np.uint32), clip, pool, sc,
                                            BS, hd)
        for b in range(batch):
            codes, scales = e.kv(0, b, which, plen)
            slots = table[b, np.arange(plen) // BS].astype(np.int64) * BS + np.arange(plen) % BS
            want = pool.view(np.uint8).reshape(nblk * BS, nkv * hd)[slots]
            assert np.array_equal(codes.view(np.uint8), want), (which, b)
            assert np.array_equal(scales.view(np.uint32), sc.reshape(-1, nkv)[slots].view(np.uint32)), (which, b)
        if which == 1:
            continue
        # The reference's paged scores kernel on the engine's own pool.
        p_ptr, p_words, s_ptr, n_sc = e.kv_pool(0, which)
        assert p_words == nblk * BS * nkv * hd // 4 and n_sc == nblk * BS * nkv
        cap = max_bt * BS
        lens = np.array([plen, 33, 1], np.uint32)
        q = torch.randn(batch, nh, hd, device=gpu)
        bt = torch.from_numpy(table.view(np.int32)).to(gpu)
        ln = torch.from_numpy(lens.view(np.int32)).to(gpu)
        scores = torch.full((batch, nh, cap), 7.0, device=gpu)
        scale = 1.0 / np.sqrt(hd)
        check(lib.bh_paged_decode_scores_i8(torch.cuda.current_stream().cuda_stream, q.data_ptr(), p_ptr, p_words,
                                            bt.data_ptr(), ln.data_ptr(), s_ptr, n_sc, scores.data_ptr(), batch,
                                            nh, nh // nkv, hd, BS, nkv * hd, cap, max_bt, C.c_float(scale)))
        torch.cuda.synchronize()
        want = o.paged_decode_scores_i8(q.cpu().numpy(), pool, table, lens, sc, np.full((batch, nh, cap), 7.0,
                                        np.float32), nh, nh // nkv, hd, BS, nkv * hd, cap, float(np.float32(scale)))
        assert np.array_equal(scores.cpu().numpy().view(np.uint32), want.view(np.uint32))
    f.close()
    e.close()


def test_bad_tables_are_refused(gpu):
    cfg = dict(SMALL)
    w = scaled_weights(cfg, seed=54)
    prompts = np.random.default_rng(8).integers(0, cfg["vocab"], size=(2, 40))
    e = Qwen3Engine(dict(cfg, kv_block_size=BS, kv_num_blocks=5), 2, 96)
    e.load_weights(w)
    with pytest.raises(BrainHipError, match="has no block"):           # small pool: nothing allocated by default
        e.prefill(prompts)
    with pytest.raises(BrainHipError, match="two sequences"):
        e.set_block_table(np.array([[0, 1, NO_BLOCK], [2, 1, NO_BLOCK]]))
        e.prefill(prompts)
    with pytest.raises(BrainHipError, match="outside the pool"):
        e.set_block_table(np.array([[0, 5, NO_BLOCK], [2, 3, NO_BLOCK]]))
    e.set_block_table(np.array([[4, 0, NO_BLOCK], [2, 3, NO_BLOCK]]))
    e.prefill(prompts)
    e.decode(20)                                                         # positions up to 59: blocks 0 and 1
    with pytest.raises(BrainHipError, match="has no block"):
        e.decode(10)                                                     # position 64+ needs a third block
    with pytest.raises(BrainHipError, match="multiple of 32"):
        Qwen3Engine(dict(cfg, kv_block_size=16), 2, 96)
    e.close()


def test_paged_engine_equals_slab_engine_qwen3_0_6b(gpu):
    """The bench's paged configuration at full size: Qwen3-0.6B shapes, batch 8,
    128-token prompt, int8 KV in blocks of 32 scattered over a pool with
    spare blocks, 4 graph decode steps: bit-identical to the slab engine."""
    from brain_amd.qwen3 import QWEN3_0_6B
    cfg = dict(QWEN3_0_6B, kv_int8=1)
    batch, plen, max_seq = 8, 128, 140
    prompts = np.random.default_rng(12).integers(0, cfg["vocab"], size=(batch, plen))
    max_bt = -(-max_seq // BS)
    nblk = batch * max_bt + 16
    table = np.random.default_rng(13).permutation(nblk)[:batch * max_bt].reshape(batch, max_bt)
    out = []
    for paged in (False, True):
        c = dict(cfg, kv_block_size=BS if paged else 0, kv_num_blocks=nblk if paged else 0)
        e = Qwen3Engine(c, batch, max_seq, max_rows=batch * plen)
        if paged:
            e.set_block_table(table)
        e.init_random(5)
        toks = [e.prefill(prompts)] + [e.decode(1)[0] for _ in range(4)]
        out.append((np.array(toks), e.logits()))
        e.close()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
