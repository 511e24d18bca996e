"""The DiT int8 linear stack (config 4) against the C oracle.

Bar, as for every linear here:
  - the bf16-input quantizer gives the oracle's bytes and scales for f32(x);
  - each GEMM at the DiT shapes gives exact i32 accumulators;
  - the bf16 outputs are exactly the oracle's epilogue rounded by its
    f32_to_bf16.
One whole layer is chained on the GPU and replayed on the CPU oracle. Each
stage feeds the next, so the final activation must match bit for bit.
"""
import numpy as np
import pytest
import torch

from brain_amd import dit, ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def host_bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("m,k", [(1152, 3840), (1152, 10240), (3, 8), (5, 36), (7, 3844), (2, 20480)])
def test_quantize_rows_bf16_bit_exact(gpu, m, k):
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + k)).to(torch.bfloat16)
    if m > 1:
        x[1] = 0
    sx, xq = ops.quantize_rows_bf16(x.to(gpu))
    xf = bf16_to_f32(host_bits(x))
    sx_ref = o.max_abs_row(xf)
    assert (sx.cpu().numpy().view(np.uint32) == sx_ref.view(np.uint32)).all()
    assert (xq.cpu().numpy().view(np.uint32) == o.quant_pack(xf, sx_ref)).all()


def test_dit_layer_chain_bit_exact(gpu):
    st = dit.DitInt8Stack(layers=1, device=gpu, seed=3)
    x0 = bf16_to_f32(host_bits(st.x))
    lw = {n: (v[0].cpu().numpy().view(np.uint32), v[1].cpu().numpy()) for n, v in st.w[0].items()}
    st.step()
    torch.cuda.synchronize()

    def mm8(x, name):
        sx = o.max_abs_row(x)
        xq = o.quant_pack(x, sx)
        wq, sw = lw[name]
        return bf16_to_f32(o.epilogue(o.acc_exact(xq, wq), sx, sw, None, "bf16"))

    qkv = mm8(x0, "qkv")
    assert np.array_equal(bf16_to_f32(host_bits(st.qkv)), qkv)
    out = mm8(x0, "o")
    assert np.array_equal(bf16_to_f32(host_bits(st.o)), out)
    h = mm8(out, "w1")
    assert np.array_equal(bf16_to_f32(host_bits(st.h)), h)
    x1 = mm8(h, "w2")
    assert np.array_equal(bf16_to_f32(host_bits(st.x)), x1)
    assert 0.3 < np.std(x1) < 3.0   # the scale choice keeps activations O(1)


def test_dit_stack_graph_replays_match_eager(gpu):
    st = dit.DitInt8Stack(layers=3, device=gpu, seed=4)
    st.x.copy_(st.x0)
    st.step()
    torch.cuda.synchronize()
    eager = st.x.clone()
    st.x.copy_(st.x0)
    st.capture()            # capture() runs one warm step, then records one
    for _ in range(3):
        st.x.copy_(st.x0)
        torch.cuda.synchronize()
        st.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.x, eager)
    assert torch.isfinite(st.x.float()).all()
