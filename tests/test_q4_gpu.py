"""W4A8 (matmul_q4_gemv / matmul_q4_dyn) on MI355X against the oracle.

Bar: the int8 family's. i32 accumulators are exact (BH_OUT_I32). f32 and bf16
outputs are the oracle epilogue of those accumulators, bit for bit. Weights
come from the oracle's int4 quantizer (int4.rs:46-67); activations from its
per-token int8 quantizer.
"""
import numpy as np
import pytest
import torch

from brain_amd import ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def dev_u32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def make(m, k, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    w4, sw = o.quantize_weight_q4(w)
    bias = rng.standard_normal(n).astype(np.float32)
    return xq, w4, sx, sw, bias


def check(gpu, m, k, n, variant, seed, sample=None):
    xq, w4, sx, sw, bias = make(m, k, n, seed)
    d = dict(xq=dev_u32(xq, gpu), wq4=dev_u32(w4, gpu), sx=torch.from_numpy(sx).to(gpu),
             sw=torch.from_numpy(sw).to(gpu))
    acc_d = ops.matmul_q4(d["xq"], d["wq4"], d["sx"], d["sw"], None, torch.int32, variant).cpu().numpy()
    f32_d = ops.matmul_q4(d["xq"], d["wq4"], d["sx"], d["sw"], None, torch.float32, variant).cpu().numpy()
    bf_d = ops.matmul_q4(d["xq"], d["wq4"], d["sx"], d["sw"], torch.from_numpy(bias).to(gpu), torch.bfloat16,
                         variant).cpu().view(torch.int16).numpy().view(np.uint16)
    if sample is None:
        rows, cols = np.arange(m), np.arange(n)
    else:
        rng = np.random.default_rng(seed)
        rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, sample)]))
        cols = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, sample)]))
    acc = o.acc_exact_q4(xq, w4, k, rows, cols)
    assert np.array_equal(acc_d[np.ix_(rows, cols)], acc)
    want = o.epilogue(acc, sx[rows], sw[cols])
    assert np.array_equal(f32_d[np.ix_(rows, cols)].view(np.uint32), want.view(np.uint32))
    wantb = o.epilogue(acc, sx[rows], sw[cols], bias[cols], "bf16")
    assert np.array_equal(bf_d[np.ix_(rows, cols)], wantb)


DECODE_KN = [(1024, 3072), (3072, 1024), (1024, 2048), (1024, 151936)]


@pytest.mark.parametrize("m", [1, 4, 8, 16, 17, 32])
@pytest.mark.parametrize("k,n", DECODE_KN)
def test_q4_gemv_decode_shapes(gpu, m, k, n):
    check(gpu, m, k, n, "gemv", seed=m * 7 + k + n, sample=400 if n > 20000 else None)


@pytest.mark.parametrize("m,n", [(1, 16384), (5, 16390), (16, 40001), (3, 151936)])
def test_q4_gemv_wide_n_streaming(gpu, m, n):
    # Wide N at K = 1024 takes the streaming kernel (the activation staged
    # once per workgroup, each wave streaming many column groups): ragged N,
    # row counts that leave the 16-row tile partly empty.
    check(gpu, m, 1024, n, "gemv", seed=m + n, sample=300 if n > 20000 else None)


@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (3, 24, 17), (5, 136, 33), (2, 1000, 40), (32, 4104, 64)])
def test_q4_gemv_edges(gpu, m, k, n):
    check(gpu, m, k, n, "gemv", seed=m + k + n)


@pytest.mark.parametrize("m,k,n", [(512, 1024, 3072), (512, 3072, 1024), (2048, 4096, 4096), (1152, 3840, 11520)])
def test_q4_dyn_prefill_shapes(gpu, m, k, n):
    check(gpu, m, k, n, "dyn", seed=m + k + n, sample=None if m * n <= 512 * 3072 else 300)


# From M=256 with K % 32 == 0 the int4 weights are expanded to int8 and the
# int8 GEMM runs (here also splitting K: 256x4096x130); below, or with K % 32
# != 0, the register-staged int4 kernel.
@pytest.mark.parametrize("m,k,n", [(33, 8, 1), (40, 24, 130), (129, 200, 257), (1, 4096, 5), (300, 200, 64),
                                   (256, 4096, 130), (255, 1024, 96)])
def test_q4_dyn_edges(gpu, m, k, n):
    check(gpu, m, k, n, "dyn", seed=m + k + n)


def test_q4_expanded_gemm_in_a_graph(gpu):
    """The expansion + int8 GEMM recorded in a HIP graph (its workspaces sized
    first with bh_reserve_workspace, kg = K/4) replays to the eager bits."""
    m, k, n = 512, 2048, 384
    xq, w4, sx, sw, _ = make(m, k, n, 8)
    d = [dev_u32(xq, gpu), dev_u32(w4, gpu), torch.from_numpy(sx).to(gpu), torch.from_numpy(sw).to(gpu)]
    out = torch.empty(m, n, device=gpu)
    eager = ops.matmul_q4(*d, None, torch.float32, "dyn").clone()
    cap = torch.cuda.Stream()
    ops.reserve_workspace(m, k, n, cap)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        ops.matmul_q4(*d, None, torch.float32, "dyn", out=out)
    for _ in range(3):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_q4_steps_through_the_backend(gpu):
    """Step names matmul_q4_gemv / matmul_q4_dyn with the raw-k params [m, k, n]."""
    from brain_amd.backend import HipBackend
    m, k, n = 8, 256, 48
    xq, w4, sx, sw, _ = make(m, k, n, 3)
    be = HipBackend(["matmul_q4_gemv", "matmul_q4_dyn"])
    bx, bw = be.storage_init("xq", xq.view(np.float32).ravel()), be.storage_init("w4", w4.view(np.float32).ravel())
    bsx, bsw = be.storage_init("sx", sx), be.storage_init("sw", sw)
    want = o.epilogue(o.acc_exact_q4(xq, w4, k), sx, sw)
    for name in ("matmul_q4_gemv", "matmul_q4_dyn"):
        out = be.storage(m * n)
        be.submit([], [be.step(be.kernel_index(name), [bx, bw, bsx, bsw, out], [m, k, n], n * 64)])
        got = be.read(out, m * n).reshape(m, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
