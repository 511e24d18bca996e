"""The C-ABI library without a GPU: it loads, exports every symbol the header
declares, and its host-only entry points (cost model, selector, host weight
quantizer) agree with the reference's tests and the oracle."""
import ctypes as C
import os
import re

import numpy as np

import brain_amd
from brain_amd import _lib
from oracle import oracle as o

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "brain_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(bh_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = brain_amd.load()
    names = _declared()
    assert len(names) >= 40
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.bh_abi_version() == 2


def test_cost_matches_reference_formula():
    # crates/gpu-core/src/cost.rs:1233-1241: [m=2, kg=8, n=3] -> 384 int ops, 12 flops
    lib = brain_amd.load()
    c = _lib.CostT()
    p = (C.c_uint32 * 3)(2, 8, 3)
    for name in (b"matmul_i8_dyn", b"matmul_i8_gemv", b"matmul_i8"):
        assert lib.bh_cost(name, p, 3, C.byref(c)) == 0
        assert (c.int_ops, c.flops) == (384, 12)
        assert c.bytes == 4 * (2 * 8 + 3 * 8 + 2 * 3 + 2 + 3)
    assert lib.bh_cost(b"matmul", p, 3, C.byref(c)) == _lib.BH_ERR_UNSUPPORTED


def test_selector_i8_arm():
    lib = brain_amd.load()
    out = (C.c_int * 2)()
    # no int8_dot -> no int8 candidate (the model falls back to fp32)
    assert lib.bh_select_i8(1, 1024, 1024, 0, 1, out) == 0
    # the reference's order (select.rs:323-331): GEMV first up to I8_GEMV_MAX_ROWS = 8 ...
    for m in (1, 4, 8):
        assert lib.bh_select_i8(m, 3072, 1024, 1, 1, out) == 2
        assert list(out) == [_lib.BH_VARIANT_WORKGROUP_PER_OUTPUT, _lib.BH_VARIANT_PACKED_INT8]
    # ... the tile first above it, through DECODE_REGIME_MAX_ROWS = 32
    for m in (9, 16, 32):
        assert lib.bh_select_i8(m, 3072, 1024, 1, 1, out) == 2
        assert list(out) == [_lib.BH_VARIANT_PACKED_INT8, _lib.BH_VARIANT_WORKGROUP_PER_OUTPUT]
    # no workgroup reductions -> tile only (select.rs:324)
    assert lib.bh_select_i8(4, 3072, 1024, 1, 0, out) == 1 and out[0] == _lib.BH_VARIANT_PACKED_INT8
    # prefill
    assert lib.bh_select_i8(33, 3072, 1024, 1, 1, out) == 1 and out[0] == _lib.BH_VARIANT_PACKED_INT8
    assert lib.bh_variant_kernel(_lib.BH_VARIANT_PACKED_INT8) == b"matmul_i8_dyn"
    assert lib.bh_variant_kernel(_lib.BH_VARIANT_WORKGROUP_PER_OUTPUT) == b"matmul_i8_gemv"


def test_host_quantize_weight_matches_oracle():
    lib = brain_amd.load()
    rng = np.random.default_rng(0)
    for n, k in [(1, 4), (7, 24), (129, 128), (300, 1024)]:
        w = (rng.standard_normal((n, k)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
        w[0, :4] = [0.5, -0.5, 1.5, 2.5]  # ties at unit scale only if max is 127; harmless otherwise
        packed = np.zeros((n, k // 4), np.uint32)
        sw = np.zeros(n, np.float32)
        assert lib.bh_quantize_weight(w.ctypes.data, n, k, packed.ctypes.data, sw.ctypes.data) == 0
        wp, wsw = o.quantize_weight(w)
        assert (packed == wp).all() and (sw == wsw).all()
        deq = np.zeros((n, k), np.float32)
        assert lib.bh_dequantize_weight(packed.ctypes.data, sw.ctypes.data, n, k, deq.ctypes.data) == 0
        assert (deq == o.dequantize_weight(wp, wsw, k)).all()


def test_host_quantize_weight_rejects_bad_k():
    lib = brain_amd.load()
    w = np.zeros((2, 6), np.float32)
    rc = lib.bh_quantize_weight(w.ctypes.data, 2, 6, None, None)
    assert rc == _lib.BH_ERR_INVALID
    assert b"multiple of 4" in lib.bh_last_error()


def test_step_api_rejects_null_backend():
    lib = brain_amd.load()
    out = C.c_void_p()
    assert lib.bh_step(None, 0, None, 0, None, 0, 0, C.byref(out)) == _lib.BH_ERR_INVALID


def test_matmul_quant_rejects_bad_arguments():
    # Checked before anything reaches the GPU: n not a multiple of 4, a null
    # output buffer, and a missing quantized output.
    lib = brain_amd.load()
    p = C.c_void_p(16)  # never dereferenced: the checks fail first
    assert lib.bh_matmul_i8_dyn_quant(None, p, p, p, p, None, p, 8, 4, 6, p, p) == _lib.BH_ERR_INVALID
    assert b"multiple of 4" in lib.bh_last_error()
    assert lib.bh_matmul_i8_dyn_quant(None, p, p, p, p, None, None, 8, 4, 8, p, p) == _lib.BH_ERR_INVALID
    assert lib.bh_matmul_i8_dyn_quant(None, p, p, p, p, None, p, 8, 4, 8, p, None) == _lib.BH_ERR_INVALID
    assert lib.bh_matmul_i8_dyn_quant(None, p, p, p, p, None, p, 0, 4, 8, None, None) == _lib.BH_OK  # m = 0: nothing to do
