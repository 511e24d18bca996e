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


@pytest.mark.parametrize("m,k,n,bias", [(1152, 10240, 3840, False), (1152, 16384, 6144, True), (1152, 3840, 3840, False),
                                        (300, 1024, 2048, True), (200, 2048, 1004, False), (7, 1024, 768, False)])
def test_matmul_i8_quant_equals_matmul_then_quantize(gpu, m, k, n, bias):
    """bh_matmul_i8_dyn_quant gives the bits of bh_matmul_i8_dyn (bf16) then
    bh_quantize_rows_bf16: the fused split-K form (the DiT down projection,
    3-way; a 2-way split with 1536 column groups per row and a bias) and the
    unfused pair (unsplit GEMMs, n % 8 != 0)."""
    g = torch.Generator(device=gpu).manual_seed(m + k + n)
    xq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=gpu, generator=g).view(torch.int32)
    wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=gpu, generator=g).view(torch.int32)
    sx = torch.rand(m, device=gpu, generator=g) * 0.02 + 0.001
    sw = (torch.rand(n, device=gpu, generator=g) + 0.5) / (73.3 * k ** 0.5)
    b = torch.randn(n, device=gpu, generator=g) if bias else None
    want = ops.matmul_i8(xq, wq, sx, sw, b, torch.bfloat16, "dyn")
    want_sx, want_xq = ops.quantize_rows_bf16(want)
    got, got_sx, got_xq = ops.matmul_i8_quant(xq, wq, sx, sw, b)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got_sx.view(torch.int32), want_sx.view(torch.int32))
    assert torch.equal(got_xq, want_xq)
    # In place, as the DiT stack calls it: sx_out is sx and xq_out is the
    # head of xq's buffer.
    if n <= k:
        xq2, sx2 = xq.clone(), sx.clone()
        ops.matmul_i8_quant(xq2, wq, sx2, sw, b, sx_out=sx2, xq_out=xq2.view(-1)[: m * n // 4].view(m, n // 4))
        torch.cuda.synchronize()
        assert torch.equal(sx2.view(torch.int32), want_sx.view(torch.int32))
        assert torch.equal(xq2.view(-1)[: m * n // 4], want_xq.view(-1))


def test_dit_stack_fused_equals_unfused(gpu):
    fused = dit.DitInt8Stack(layers=3, device=gpu, seed=5)
    plain = dit.DitInt8Stack(layers=3, device=gpu, seed=5, fuse=False)
    fused.step()
    plain.step()
    torch.cuda.synchronize()
    for name in ("x", "qkv", "o", "h", "sx", "xq"):
        assert torch.equal(getattr(fused, name).view(torch.int16), getattr(plain, name).view(torch.int16)), name
