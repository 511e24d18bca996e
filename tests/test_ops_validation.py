"""brain_amd.ops rejects wrong dtypes and short operands before any launch
(the C ABI takes bare pointers, so a short or mistyped buffer would become an
out-of-bounds device access). CPU only: the checks run before the library is
called, and the tensors carry is_cuda=True through a stand-in."""
import pytest
import torch

from brain_amd import ops


class FakeCuda:
    """Wraps a CPU tensor and reports is_cuda=True, so ops' host-side checks
    run without a GPU; any attempt to launch would fail on data_ptr use."""

    def __init__(self, t):
        self.t = t

    def __getattr__(self, name):
        return getattr(self.t, name)

    @property
    def is_cuda(self):
        return True

    @property
    def shape(self):
        return self.t.shape

    @property
    def dtype(self):
        return self.t.dtype

    def data_ptr(self):
        raise AssertionError("reached a launch")


def f(*shape, dtype=torch.float32):
    return FakeCuda(torch.zeros(*shape, dtype=dtype))


M, K, N = 4, 64, 8


def test_linear_i8_checks():
    good = dict(x=f(M, K), wq=f(N, K // 4, dtype=torch.int32), sw=f(N))
    with pytest.raises(ValueError, match="x: dtype"):
        ops.linear_i8(f(M, K, dtype=torch.bfloat16), good["wq"], good["sw"])
    with pytest.raises(ValueError, match="wq"):
        ops.linear_i8(good["x"], f(N, K // 4 - 1, dtype=torch.int32), good["sw"])
    with pytest.raises(ValueError, match="sw"):
        ops.linear_i8(good["x"], good["wq"], f(N - 1))
    with pytest.raises(ValueError, match="bias"):
        ops.linear_i8(good["x"], good["wq"], good["sw"], bias=f(N, dtype=torch.float64))
    with pytest.raises(ValueError, match="sx"):
        ops.linear_i8(good["x"], good["wq"], good["sw"], sx=f(M - 1))
    with pytest.raises(ValueError, match="xq"):
        ops.linear_i8(good["x"], good["wq"], good["sw"], xq=f(M, K // 4))
    with pytest.raises(ValueError, match="out"):
        ops.linear_i8(good["x"], good["wq"], good["sw"], out=f(M, N, dtype=torch.bfloat16))


def test_matmul_static_q4_moe_checks():
    xq, wq = f(M, K // 4, dtype=torch.int32), f(N, K // 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="xq"):
        ops.matmul_i8_static(f(M, K // 4), wq, 1.0, 1.0)
    with pytest.raises(ValueError, match="out"):
        ops.matmul_i8_static(xq, wq, 1.0, 1.0, out=f(M, N - 1))
    wq4 = f(N, K // 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="sx"):
        ops.matmul_q4(xq, wq4, f(M - 1), f(N))
    with pytest.raises(ValueError, match="sw"):
        ops.matmul_q4(xq, wq4, f(M), f(N, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bias"):
        ops.matmul_q4(xq, wq4, f(M), f(N), bias=f(N - 1))
    gate = f(M, 2)
    with pytest.raises(ValueError, match="wq"):
        ops.moe_linear_gated_i8(xq, f(N, K // 4), f(M), f(N), gate, 0)
    with pytest.raises(ValueError, match="sx"):
        ops.moe_linear_gated_i8(xq, wq, f(M - 1), f(N), gate, 0)
    with pytest.raises(ValueError, match="out"):
        ops.moe_linear_gated_i8(xq, wq, f(M), f(N), gate, 0, out=f(M, N, dtype=torch.bfloat16))
