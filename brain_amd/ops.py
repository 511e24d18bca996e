"""torch-tensor wrappers of the typed, stream-ordered calls in libbrain_hip.so.

torch only supplies device memory and the current HIP stream; all arithmetic
runs in the library's gfx950 kernels. Packed int8 tensors are torch.int32
tensors holding the u32 words (4 int8 per word, little-endian along K).
"""
import torch

from ._lib import BH_OUT_BF16, BH_OUT_F32, BH_OUT_I32, check, load

_CODES = {torch.float32: BH_OUT_F32, torch.bfloat16: BH_OUT_BF16, torch.int32: BH_OUT_I32}


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _dev(*ts):
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("brain_amd.ops: tensors must live on the GPU")
        if not t.is_contiguous():
            raise ValueError("brain_amd.ops: tensors must be contiguous")


def _need(t, dtype, numel, name):
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, needs {numel}")


def max_abs_rows(x, sx=None):
    """sx[m] = max(max|x[m,:]|, 1e-8)/127 (max_abs_row.wgsl)."""
    m, k = x.shape
    _dev(x)
    _need(x, torch.float32, m * k, "x")
    sx = torch.empty(m, device=x.device, dtype=torch.float32) if sx is None else sx
    check(load().bh_max_abs_rows(_stream(), _ptr(x), m, k, _ptr(sx)))
    return sx


def quant_pack(x, sx, xq=None):
    """xq [m, k/4] int32 words: clamp(rne(x/sx), +-127) packed (quant_pack.wgsl)."""
    m, k = x.shape
    _dev(x, sx)
    _need(x, torch.float32, m * k, "x")
    _need(sx, torch.float32, m, "sx")
    xq = torch.empty(m, k // 4, device=x.device, dtype=torch.int32) if xq is None else xq
    check(load().bh_quant_pack(_stream(), _ptr(x), _ptr(sx), m, k, _ptr(xq)))
    return xq


def quantize_rows(x, sx=None, xq=None):
    """Fused max_abs_rows + quant_pack; returns (sx, xq)."""
    m, k = x.shape
    _dev(x)
    _need(x, torch.float32, m * k, "x")
    sx = torch.empty(m, device=x.device, dtype=torch.float32) if sx is None else sx
    xq = torch.empty(m, k // 4, device=x.device, dtype=torch.int32) if xq is None else xq
    check(load().bh_quantize_rows(_stream(), _ptr(x), m, k, _ptr(sx), _ptr(xq)))
    return sx, xq


def quantize_rows_bf16(x, sx=None, xq=None):
    """Per-token quantization of bf16 activations (exactly quantize_rows of x.float())."""
    m, k = x.shape
    _dev(x)
    _need(x, torch.bfloat16, m * k, "x")
    sx = torch.empty(m, device=x.device, dtype=torch.float32) if sx is None else sx
    xq = torch.empty(m, k // 4, device=x.device, dtype=torch.int32) if xq is None else xq
    check(load().bh_quantize_rows_bf16(_stream(), _ptr(x), m, k, _ptr(sx), _ptr(xq)))
    return sx, xq


_VARIANTS = {"auto": "bh_matmul_i8", "gemv": "bh_matmul_i8_gemv", "dyn": "bh_matmul_i8_dyn"}


def matmul_i8(xq, wq, sx, sw, bias=None, out_dtype=torch.float32, variant="auto", out=None):
    """out[m,n] = (f32(xq.wq^T) * sx[m]) * sw[n] (+ bias[n]), f32 or bf16;
    out_dtype=torch.int32 returns the raw i32 accumulators."""
    m, kg = xq.shape
    n = wq.shape[0]
    _dev(xq, wq, sx, sw, bias, out)
    _need(xq, torch.int32, m * kg, "xq")
    _need(wq, torch.int32, n * kg, "wq")
    _need(sx, torch.float32, m, "sx")
    _need(sw, torch.float32, n, "sw")
    if bias is not None:
        _need(bias, torch.float32, n, "bias")
    code = _CODES[out_dtype]
    out = torch.empty(m, n, device=xq.device, dtype=out_dtype) if out is None else out
    _need(out, out_dtype, m * n, "out")
    fn = getattr(load(), _VARIANTS[variant])
    check(fn(_stream(), _ptr(xq), _ptr(wq), _ptr(sx), _ptr(sw), _ptr(bias), _ptr(out), code, m, kg, n))
    return out


def matmul_i8_quant(xq, wq, sx, sw, bias=None, out=None, sx_out=None, xq_out=None):
    """bf16 out[m,n] = matmul_i8_dyn(xq, wq, sx, sw, bias), then the per-row
    quantization of out (quantize_rows_bf16) into sx_out [m], xq_out [m, n/4]
    for the next linear, in one call (split-K GEMMs reduce and quantize in one
    pass). sx_out may be sx and xq_out may overlap xq."""
    m, kg = xq.shape
    n = wq.shape[0]
    if n % 4:
        raise ValueError(f"matmul_i8_quant: n={n} is not a multiple of 4")
    _dev(xq, wq, sx, sw, bias, out, sx_out, xq_out)
    _need(xq, torch.int32, m * kg, "xq")
    _need(wq, torch.int32, n * kg, "wq")
    _need(sx, torch.float32, m, "sx")
    _need(sw, torch.float32, n, "sw")
    if bias is not None:
        _need(bias, torch.float32, n, "bias")
    out = torch.empty(m, n, device=xq.device, dtype=torch.bfloat16) if out is None else out
    sx_out = torch.empty(m, device=xq.device, dtype=torch.float32) if sx_out is None else sx_out
    xq_out = torch.empty(m, n // 4, device=xq.device, dtype=torch.int32) if xq_out is None else xq_out
    _need(out, torch.bfloat16, m * n, "out")
    _need(sx_out, torch.float32, m, "sx_out")
    _need(xq_out, torch.int32, m * n // 4, "xq_out")
    check(load().bh_matmul_i8_dyn_quant(_stream(), _ptr(xq), _ptr(wq), _ptr(sx), _ptr(sw), _ptr(bias), _ptr(out),
                                        m, kg, n, _ptr(sx_out), _ptr(xq_out)))
    return out, sx_out, xq_out


def matmul_i8_static(xq, wq, sx, sw, out=None):
    """matmul_i8.wgsl: out = f32(acc) * (sx*sw) with scalar per-tensor scales."""
    m, kg = xq.shape
    n = wq.shape[0]
    _dev(xq, wq, out)
    _need(xq, torch.int32, m * kg, "xq")
    _need(wq, torch.int32, n * kg, "wq")
    out = torch.empty(m, n, device=xq.device, dtype=torch.float32) if out is None else out
    _need(out, torch.float32, m * n, "out")
    check(load().bh_matmul_i8_static(_stream(), _ptr(xq), _ptr(wq), float(sx), float(sw), _ptr(out), m, kg, n))
    return out


def linear_i8(x, wq, sw, bias=None, out_dtype=torch.float32, sx=None, xq=None, out=None):
    """Quantize x per token, then the W8A8 matmul (Ops::act + Ops::matmul)."""
    m, k = x.shape
    n = wq.shape[0]
    if k % 4:
        raise ValueError(f"linear_i8: k={k} is not a multiple of 4")
    _dev(x, wq, sw, bias, sx, xq, out)
    _need(x, torch.float32, m * k, "x")
    _need(wq, torch.int32, n * (k // 4), "wq")
    _need(sw, torch.float32, n, "sw")
    if bias is not None:
        _need(bias, torch.float32, n, "bias")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"linear_i8: out_dtype {out_dtype}, expected float32 or bfloat16")
    sx = torch.empty(m, device=x.device, dtype=torch.float32) if sx is None else sx
    xq = torch.empty(m, k // 4, device=x.device, dtype=torch.int32) if xq is None else xq
    _need(sx, torch.float32, m, "sx")
    _need(xq, torch.int32, m * (k // 4), "xq")
    code = {torch.float32: BH_OUT_F32, torch.bfloat16: BH_OUT_BF16}[out_dtype]
    out = torch.empty(m, n, device=x.device, dtype=out_dtype) if out is None else out
    _need(out, out_dtype, m * n, "out")
    check(load().bh_linear_i8(_stream(), _ptr(x), _ptr(wq), _ptr(sw), _ptr(bias), _ptr(sx), _ptr(xq),
                              _ptr(out), code, m, k, n))
    return out


def quantize_weight_device(w):
    """Per-output-channel weight quantization on the GPU (int8.rs quantize_weight)."""
    n, k = w.shape
    _dev(w)
    packed = torch.empty(n, k // 4, device=w.device, dtype=torch.int32)
    sw = torch.empty(n, device=w.device, dtype=torch.float32)
    check(load().bh_quantize_weight_device(_stream(), _ptr(w), n, k, _ptr(packed), _ptr(sw)))
    return packed, sw


def f32_to_bf16(x):
    """bf16 bit patterns (int16 tensor) of f32 `x`, the library's output rounding (half.rs f32_to_bf16)."""
    _dev(x)
    out = torch.empty(x.shape, device=x.device, dtype=torch.int16)
    check(load().bh_f32_to_bf16(_stream(), _ptr(x), _ptr(out), x.numel()))
    return out


def reserve_workspace(m, k, n, stream=None):
    """Pre-size the workspaces of `stream` (default: current) that an
    [m,k] x [n,k] GEMM may take (split-K slabs; for W4A8 the int4 weights
    expanded to int8); required before capturing such a GEMM in a graph."""
    sp = (stream or torch.cuda.current_stream()).cuda_stream
    check(load().bh_reserve_workspace(sp, m, k // 4, n))


_Q4_VARIANTS = {"auto": "bh_matmul_q4", "gemv": "bh_matmul_q4_gemv", "dyn": "bh_matmul_q4_dyn"}


def matmul_q4(xq, wq4, sx, sw, bias=None, out_dtype=torch.float32, variant="auto", out=None):
    """W4A8: xq [m, k/4] int8 activation words, wq4 [n, k/8] int4 weight words
    (crates/model/src/int4.rs), (f32(acc)*sx)*sw (+bias) -> out [m, n]."""
    m, kg = xq.shape
    n, kw = wq4.shape
    k = kg * 4
    if kw * 8 != k:
        raise ValueError(f"matmul_q4: xq has K={k}, wq4 has K={kw * 8}")
    _dev(xq, wq4, sx, sw, bias, out)
    _need(xq, torch.int32, m * kg, "xq")
    _need(wq4, torch.int32, n * kw, "wq4")
    _need(sx, torch.float32, m, "sx")
    _need(sw, torch.float32, n, "sw")
    if bias is not None:
        _need(bias, torch.float32, n, "bias")
    code = _CODES[out_dtype]
    out = torch.empty(m, n, device=xq.device, dtype=out_dtype) if out is None else out
    _need(out, out_dtype, m * n, "out")
    check(getattr(load(), _Q4_VARIANTS[variant])(
        _stream(), _ptr(xq), _ptr(wq4), _ptr(sx), _ptr(sw), _ptr(bias), _ptr(out), code, m, k, n))
    return out


def moe_linear_gated_i8(xq, wq, sx, sw, gate, e_idx, out=None):
    """moe_linear_gated_i8.wgsl: f32 out [m, n], rows with gate[row, e_idx] <= 0 are +0."""
    m, kg = xq.shape
    n = wq.shape[0]
    n_experts = gate.shape[1]
    _dev(xq, wq, sx, sw, gate, out)
    _need(xq, torch.int32, m * kg, "xq")
    _need(wq, torch.int32, n * kg, "wq")
    _need(sx, torch.float32, m, "sx")
    _need(sw, torch.float32, n, "sw")
    _need(gate, torch.float32, m * n_experts, "gate")
    out = torch.empty(m, n, device=xq.device, dtype=torch.float32) if out is None else out
    _need(out, torch.float32, m * n, "out")
    check(load().bh_moe_linear_gated_i8(_stream(), _ptr(xq), _ptr(wq), _ptr(sx), _ptr(sw), _ptr(gate), n_experts,
                                        e_idx, _ptr(out), m, kg, n))
    return out
