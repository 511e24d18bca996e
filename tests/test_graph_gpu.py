"""The int8 linear captured in a HIP graph: every replay (with eager work and
synchronisations between replays) must equal the eager result bit for bit."""
import numpy as np
import pytest
import torch

from brain_amd import ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu):
    shapes = [(1, 1024, 3072), (16, 3072, 1024), (64, 1024, 640), (512, 1024, 1024)]
    data = []
    for i, (m, k, n) in enumerate(shapes):
        x = torch.from_numpy(o.synth_acts(m, k, 10 + i)).to(gpu)
        wq, sw = o.synth_weights(n, k, 20 + i)
        data.append(dict(x=x, wq=torch.from_numpy(wq.view(np.int32)).to(gpu), sw=torch.from_numpy(sw).to(gpu),
                         bias=torch.randn(n, device=gpu), sx=torch.empty(m, device=gpu),
                         xq=torch.empty(m, k // 4, dtype=torch.int32, device=gpu),
                         out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu)))

    def run():
        for d in data:
            ops.linear_i8(d["x"], d["wq"], d["sw"], d["bias"], torch.bfloat16, sx=d["sx"], xq=d["xq"], out=d["out"])

    run()
    torch.cuda.synchronize()
    eager = [d["out"].clone() for d in data]
    cap = torch.cuda.Stream()
    for (m, k, n) in shapes:
        ops.reserve_workspace(m, k, n, cap)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        run()
    for rep in range(4):
        for d in data:
            d["out"].fill_(0)
        _ = torch.randn(1000, device=gpu).sum()  # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for d, e in zip(data, eager):
            assert torch.equal(d["out"].view(torch.int16), e.view(torch.int16)), f"replay {rep} differs"



def test_graph_survives_workspace_growth(gpu):
    """A graph that captured a split-K GEMM keeps working after a larger
    split-K GEMM on the same stream grew the workspace (the old buffer the
    graph uses must stay valid)."""
    def case(m, k, n, seed):
        x = torch.from_numpy(o.synth_acts(m, k, seed)).to(gpu)
        wq, sw = o.synth_weights(n, k, seed + 1)
        return dict(x=x, wq=torch.from_numpy(wq.view(np.int32)).to(gpu), sw=torch.from_numpy(sw).to(gpu),
                    sx=torch.empty(m, device=gpu), xq=torch.empty(m, k // 4, dtype=torch.int32, device=gpu),
                    out=torch.empty(m, n, dtype=torch.float32, device=gpu))

    small, big = case(128, 3072, 1024, 40), case(300, 4096, 520, 50)   # both take the split-K path

    def run(d):
        ops.linear_i8(d["x"], d["wq"], d["sw"], None, torch.float32, sx=d["sx"], xq=d["xq"], out=d["out"])

    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        run(small)
    torch.cuda.synchronize()
    eager = small["out"].clone()
    ops.reserve_workspace(128, 3072, 1024, cap)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        run(small)
    with torch.cuda.stream(cap):
        run(big)                      # grows the workspace of `cap`
    torch.cuda.synchronize()
    for _ in range(3):
        small["out"].fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(small["out"], eager)
