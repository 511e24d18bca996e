"""moe_linear_gated_i8 (sparse-MoE expert linear, int8) against the oracle.

Routed rows (gate[row, e_idx] > 0, and NaN, which the reference's `<= 0`
test lets through) are the matmul_i8_dyn result bit for bit; other rows are
exactly +0.0.
"""
import numpy as np
import pytest
import torch

from brain_amd import ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def dev_u32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


@pytest.mark.parametrize("m,k,n", [(1, 1024, 768), (8, 1024, 768), (32, 2048, 512), (33, 512, 300), (512, 1024, 1536),
                                   (200, 4096, 300)])
def test_moe_linear_gated_i8(gpu, m, k, n):
    rng = np.random.default_rng(m + k + n)
    n_experts, e_idx = 8, 3
    x = rng.standard_normal((m, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.quantize_weight(rng.standard_normal((n, k)).astype(np.float32))
    gate = rng.standard_normal((m, n_experts)).astype(np.float32)
    gate[::5, e_idx] = 0.0                   # exactly 0: not routed
    if m > 2:
        gate[2, e_idx] = np.nan              # NaN: `<= 0` is false, so computed
    got = ops.moe_linear_gated_i8(dev_u32(xq, gpu), dev_u32(wq, gpu), torch.from_numpy(sx).to(gpu),
                                  torch.from_numpy(sw).to(gpu), torch.from_numpy(gate).to(gpu), e_idx).cpu().numpy()
    want = o.epilogue(o.acc_exact(xq, wq), sx, sw)
    off = gate[:, e_idx] <= 0
    want[off] = 0.0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert (got[off].view(np.uint32) == 0).all()      # +0, not -0


def test_moe_step_through_the_backend(gpu):
    from brain_amd.backend import HipBackend
    m, k, n, ne, ei = 4, 256, 64, 4, 1
    rng = np.random.default_rng(9)
    x = rng.standard_normal((m, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.quantize_weight(rng.standard_normal((n, k)).astype(np.float32))
    gate = np.array([[0, 1, 0, 0], [0, -1, 0, 0], [0, 0.5, 0, 0], [0, 0, 0, 0]], np.float32)
    be = HipBackend(["moe_linear_gated_i8"])
    bufs = [be.storage_init("xq", xq.view(np.float32).ravel()), be.storage_init("wq", wq.view(np.float32).ravel()),
            be.storage_init("sx", sx), be.storage_init("sw", sw), be.storage_init("gate", gate.ravel())]
    out = be.storage(m * n)
    be.submit([], [be.step(be.kernel_index("moe_linear_gated_i8"), bufs + [out], [m, k // 4, n, ne, ei], m * n)])
    got = be.read(out, m * n).reshape(m, n)
    want = o.epilogue(o.acc_exact(xq, wq), sx, sw)
    want[[1, 3]] = 0.0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,k,n,pattern", [
    (8, 1024, 768, "none"),          # GEMV: no routed row -> the launch reads no weights
    (4, 1024, 16390, "some"),        # wide N, K=1024: the gated GEMV keeps the gate
    (512, 1024, 1536, "blocks"),     # GEMM: whole tiles of unrouted rows skip their K loop
    (300, 2048, 700, "none"),        # GEMM, nothing routed
    (200, 4096, 300, "blocks"),      # split-K shape: partial tiles never skip
])
def test_moe_unrouted_tiles_skip(gpu, m, k, n, pattern):
    rng = np.random.default_rng(m * 3 + n)
    n_experts, e_idx = 4, 2
    x = rng.standard_normal((m, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.quantize_weight(rng.standard_normal((n, k)).astype(np.float32))
    gate = np.abs(rng.standard_normal((m, n_experts))).astype(np.float32) + 0.1
    if pattern == "none":
        gate[:, e_idx] = 0.0
    elif pattern == "some":
        gate[1::2, e_idx] = -1.0
    else:
        gate[128:384, e_idx] = 0.0
        gate[7, e_idx] = -0.0
    out = torch.full((m, n), float("nan"), device=gpu)   # every output must be written
    got = ops.moe_linear_gated_i8(dev_u32(xq, gpu), dev_u32(wq, gpu), torch.from_numpy(sx).to(gpu),
                                  torch.from_numpy(sw).to(gpu), torch.from_numpy(gate).to(gpu), e_idx,
                                  out=out).cpu().numpy()
    off = gate[:, e_idx] <= 0
    want = np.zeros((m, n), np.float32)
    on = np.nonzero(~off)[0]
    if len(on):
        want[on] = o.epilogue(o.acc_exact(xq[on], wq), sx[on], sw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,k,n,frac", [(8192, 1024, 768, 0.25), (8200, 2048, 1000, 0.125), (8192, 1024, 512, 0.0),
                                        (8256, 1024, 256, 1.0), (12000, 1024, 256, 0.5)])
def test_moe_compacted_rows(gpu, m, k, n, frac):
    """Long prefills (>= 8192 rows): the routed rows are compacted, multiplied
    as a dense GEMM and scattered back; every routed row equals the dense
    result bit for bit and every other row is +0 -- with no routed row at
    all, every row routed, a width that is not a multiple of 8 (the direct
    epilogue) and a row count that is not a multiple of 64 (a partial last
    slot-assignment block)."""
    rng = np.random.default_rng(m + n)
    n_experts, e_idx = 4, 2
    x = rng.standard_normal((m, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, m + 1)
    gate = rng.standard_normal((m, n_experts)).astype(np.float32)
    routed = rng.random(m) < frac
    gate[:, e_idx] = np.where(routed, np.abs(gate[:, e_idx]) + 0.1, -np.abs(gate[:, e_idx]))
    if frac > 0 and m > 7:
        gate[7, e_idx] = np.nan              # routed (`<= 0` is false)
        routed[7] = True
    got = ops.moe_linear_gated_i8(dev_u32(xq, gpu), dev_u32(wq, gpu), torch.from_numpy(sx).to(gpu),
                                  torch.from_numpy(sw).to(gpu), torch.from_numpy(gate).to(gpu), e_idx).cpu().numpy()
    rows = np.nonzero(routed)[0]
    if rows.size:
        want = o.epilogue(o.acc_exact(xq, wq, rows, np.arange(n)), sx[rows], sw)
        assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))
    assert (got[~routed].view(np.uint32) == 0).all()


@pytest.mark.parametrize("m,k,n,frac", [(16384, 1024, 3072, 0.125), (8192, 1024, 3072, 0.25)])
def test_moe_compacted_rows_big_tiles(gpu, m, k, n, frac):
    """The compaction on the big-tile GEMMs (256x256 ping-pong tiles at
    16384 x 3072, 256x128 at 8192 x 3072), whose epilogues also store packed
    row k to its row of the output: a sample of the routed rows (the first,
    the last, the NaN-gated one and 256 more) against the oracle bit for bit,
    every unrouted row +0."""
    rng = np.random.default_rng(m + n + 1)
    n_experts, e_idx = 8, 5
    x = rng.standard_normal((m, k)).astype(np.float32)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, m + 3)
    gate = rng.standard_normal((m, n_experts)).astype(np.float32)
    routed = rng.random(m) < frac
    gate[:, e_idx] = np.where(routed, np.abs(gate[:, e_idx]) + 0.1, -np.abs(gate[:, e_idx]))
    gate[11, e_idx] = np.nan
    routed[11] = True
    got = ops.moe_linear_gated_i8(dev_u32(xq, gpu), dev_u32(wq, gpu), torch.from_numpy(sx).to(gpu),
                                  torch.from_numpy(sw).to(gpu), torch.from_numpy(gate).to(gpu), e_idx).cpu().numpy()
    rows = np.nonzero(routed)[0]
    pick = np.unique(np.concatenate([rows[:1], rows[-1:], [11], rng.choice(rows, 256, replace=False)]))
    want = o.epilogue(o.acc_exact(xq, wq, pick, np.arange(n)), sx[pick], sw)
    assert np.array_equal(got[pick].view(np.uint32), want.view(np.uint32))
    assert (got[~routed].view(np.uint32) == 0).all()


def test_moe_compacted_rows_graph_replays(gpu):
    """The compaction under a HIP graph: captured once (after a warm call on
    the capture stream, which sizes its workspace), replayed with a different
    routing written into the gate between replays (eager work and
    synchronizations in between); every replay equals the eager call on the
    same gate, bit for bit."""
    m, k, n, n_experts, e_idx = 8192, 1024, 512, 4, 1
    g = torch.Generator(device=gpu).manual_seed(11)
    xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=gpu, generator=g).view(torch.int32)
    wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=gpu, generator=g).view(torch.int32)
    sx = torch.rand(m, device=gpu, generator=g) * 0.02 + 0.001
    sw = torch.rand(n, device=gpu, generator=g) * 0.02 + 0.002
    gate = torch.empty(m, n_experts, device=gpu)
    out = torch.empty(m, n, device=gpu)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ops.moe_linear_gated_i8(xq, wq, sx, sw, gate.fill_(1.0), e_idx, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        ops.moe_linear_gated_i8(xq, wq, sx, sw, gate, e_idx, out=out)
    for frac in (0.125, 1.0, 0.0, 0.4):
        gate.copy_(torch.where(torch.rand(m, n_experts, device=gpu, generator=g) < frac, 1.0, -1.0))
        want = ops.moe_linear_gated_i8(xq, wq, sx, sw, gate, e_idx)
        torch.cuda.synchronize()
        out.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), frac
