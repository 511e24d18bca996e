"""HIP kernels vs the CPU oracle on the same seeded inputs (MI355X only).

Bar: bit-exact. Scales and packed activations byte-for-byte; i32 accumulators
exactly (BH_OUT_I32); f32 outputs bit-for-bit; bf16 outputs equal to the RNE
of the oracle's f32. Full BASELINE shapes are checked in full where the oracle
is fast (float64-BLAS exact accumulators) and on a seeded sample of output
entries otherwise.
"""
import numpy as np
import pytest
import torch

from brain_amd import ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def dev_u32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def host_u32(t):
    return t.cpu().numpy().view(np.uint32)


def dev_f32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def bf16_bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def special_acts(m, k, seed):
    x = o.synth_acts(m, k, seed)
    if m > 1:
        x[1] = 0.0                               # all-zero row -> sx = 1e-8/127, q = 0
    if m > 2:
        x[2, 0] = 1e30                           # one huge outlier
    if m > 3 and k >= 8:
        x[3, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]  # exact ties at sx = 1
    return x


# ---------------------------------------------------------------- bf16 rounding
def test_f32_to_bf16_matches_reference_rule(gpu):
    """Every bf16 output goes through one hardware conversion; it must give the
    reference's bits (half.rs f32_to_bf16) on every class of input: all 65536
    upper halves with the rounding-critical lower halves (exact, below, at and
    above the tie, all ones: zeros, subnormals, ties, overflow to inf, NaN
    payloads), plus a large random sample of bit patterns."""
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    classes = (hi[:, None] | lows[None, :]).ravel()
    rand = np.random.default_rng(5).integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    bits = np.concatenate([classes, rand])
    x = bits.view(np.float32)
    got = ops.f32_to_bf16(dev_f32(x, gpu)).cpu().numpy().view(np.uint16)
    want = o.f32_to_bf16_array(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first input 0x{int(bits[bad[0]]):08x}"


# ---------------------------------------------------------------- quantization
QUANT_SHAPES = [(1, 4), (1, 1024), (3, 8), (4, 36), (16, 1024), (7, 3072), (64, 4096), (513, 1024), (5, 10240),
                (1027, 1024), (2048, 504), (1024, 4)]


@pytest.mark.parametrize("m,k", QUANT_SHAPES)
def test_quant_kernels_bit_exact(gpu, m, k):
    x = special_acts(m, k, 100 + m + k)
    sx_ref = o.max_abs_row(x)
    xq_ref = o.quant_pack(x, sx_ref)
    xd = dev_f32(x, gpu)
    sx = ops.max_abs_rows(xd)
    assert (sx.cpu().numpy().view(np.uint32) == sx_ref.view(np.uint32)).all()
    xq = ops.quant_pack(xd, sx)
    assert (host_u32(xq) == xq_ref).all()
    sx2, xq2 = ops.quantize_rows(xd)
    assert (sx2.cpu().numpy().view(np.uint32) == sx_ref.view(np.uint32)).all()
    assert (host_u32(xq2) == xq_ref).all()


def test_quant_ties_at_unit_scale(gpu):
    x = np.array([[-2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.5, 0.0]], np.float32)
    xq = ops.quant_pack(dev_f32(x, gpu), dev_f32([1.0], gpu))
    assert o.unpack_i8(host_u32(xq)).tolist() == [[-2, -2, 0, 0, 2, 2, 4, 0]]


def test_quant_unaligned_rows_and_odd_k_scale(gpu):
    # x starting one float into an allocation: the scalar (non-float4) paths.
    m, k = 6, 132
    x = special_acts(m, k, 7)
    base = torch.zeros(m * k + 1, device=gpu)
    base[1:] = dev_f32(x.reshape(-1), gpu)
    xv = base[1:].view(m, k)
    sx_ref = o.max_abs_row(x)
    sx, xq = ops.quantize_rows(xv)
    assert (sx.cpu().numpy() == sx_ref).all()
    assert (host_u32(xq) == o.quant_pack(x, sx_ref)).all()
    assert (host_u32(ops.quant_pack(xv, sx)) == o.quant_pack(x, sx_ref)).all()
    # max_abs_row alone accepts any k (no packing)
    x5 = o.synth_acts(3, 5, 9)
    assert (ops.max_abs_rows(dev_f32(x5, gpu)).cpu().numpy() == o.max_abs_row(x5)).all()


# ---------------------------------------------------------------- matmul helpers
def run_and_check(gpu, m, k, n, variant, seed, bias=False, sample=None, must_rows=(), must_cols=()):
    x = special_acts(m, k, seed)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, seed + 1)
    b = o.synth_acts(1, n, seed + 2)[0] if bias else None
    dx, dw, dsx, dsw = dev_u32(xq, gpu), dev_u32(wq, gpu), dev_f32(sx, gpu), dev_f32(sw, gpu)
    db = None if b is None else dev_f32(b, gpu)
    acc_d = ops.matmul_i8(dx, dw, dsx, dsw, None, torch.int32, variant).cpu().numpy()
    f32_d = ops.matmul_i8(dx, dw, dsx, dsw, db, torch.float32, variant).cpu().numpy()
    bf_d = bf16_bits(ops.matmul_i8(dx, dw, dsx, dsw, db, torch.bfloat16, variant))
    if sample is None:
        rows, cols = np.arange(m), np.arange(n)
    else:
        rng = np.random.default_rng(seed)
        rows = np.unique(np.concatenate([[0, m - 1], list(must_rows), rng.integers(0, m, sample)])).astype(np.int64)
        cols = np.unique(np.concatenate([[0, n - 1], list(must_cols), rng.integers(0, n, sample)])).astype(np.int64)
    acc = o.acc_exact(xq, wq, rows, cols)
    bsub = None if b is None else b[cols]
    assert (acc_d[np.ix_(rows, cols)] == acc).all(), "i32 accumulators differ"
    want = o.epilogue(acc, sx[rows], sw[cols], bsub)
    got = f32_d[np.ix_(rows, cols)]
    assert (got.view(np.uint32) == want.view(np.uint32)).all(), "f32 outputs differ"
    wantb = o.epilogue(acc, sx[rows], sw[cols], bsub, "bf16")
    assert (bf_d[np.ix_(rows, cols)] == wantb).all(), "bf16 outputs differ"


# Config 1 (decode GEMV sweep), full size.
DECODE_KN = [(1024, 3072), (3072, 1024), (1024, 2048), (1024, 151936)]


@pytest.mark.parametrize("k,n", DECODE_KN)
@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_gemv_decode_sweep_full(gpu, m, k, n):
    run_and_check(gpu, m, k, n, "gemv", seed=m * 7 + k + n, bias=(m == 4))


@pytest.mark.parametrize("m,k,n", [(17, 1024, 300), (32, 512, 257), (2, 8, 3), (6, 24, 13), (5, 36, 33),
                                   (1, 4, 1), (31, 132, 70), (3, 2048 + 64, 100),
                                   (20, 1032, 16390), (9, 64, 16401), (32, 200, 16384),
                                   # the streaming wide-N kernel (K = 1024, >= 1024 column groups)
                                   (16, 1024, 16390), (3, 1024, 40001), (1, 1024, 16384), (13, 1024, 151936)])
def test_gemv_edges(gpu, m, k, n):
    run_and_check(gpu, m, k, n, "gemv", seed=m + k + n, bias=True)


# Config 2 (prefill sweep): full check at M=512, sampled at larger M.
PREFILL_KN = [(1024, 3072), (3072, 1024), (4096, 11008), (4096, 4096)]


@pytest.mark.parametrize("k,n", PREFILL_KN)
def test_gemm_prefill_m512_full(gpu, k, n):
    run_and_check(gpu, 512, k, n, "dyn", seed=k + n, bias=True)


@pytest.mark.parametrize("k,n", PREFILL_KN)
@pytest.mark.parametrize("m", [2048, 8192])
def test_gemm_prefill_sampled(gpu, m, k, n):
    run_and_check(gpu, m, k, n, "dyn", seed=m + k + n, bias=True, sample=300)


@pytest.mark.parametrize("m,k,n", [(37, 24, 41), (33, 132, 17), (1, 4, 1), (130, 64, 257), (128, 1024, 128),
                                   (255, 520, 129), (64, 8, 300), (1152, 3840, 384)])
def test_gemm_edges(gpu, m, k, n):
    run_and_check(gpu, m, k, n, "dyn", seed=m * 3 + k + n, bias=True)


# Few output tiles and long K: the GEMM splits K over workgroups and adds the
# i32 partials in a second kernel. Covered: the LDS-DMA and register-staged
# (K % 128 != 0, K % 64 != 0) split kernels, the 4-column and per-element
# (N % 4 != 0) reductions, and the largest split factor (8).
@pytest.mark.parametrize("m,k,n", [(300, 4096, 520), (256, 4104, 130), (40, 8192, 64), (129, 5000, 255),
                                   (128, 3072, 1024), (64, 16384, 128)])
def test_gemm_split_k(gpu, m, k, n):
    run_and_check(gpu, m, k, n, "dyn", seed=m + 5 * k + n, bias=True)


@pytest.mark.parametrize("m,k,n", [(1152, 10240, 3840), (2048, 16384, 3072)])
def test_gemm_split_k_big_tiles(gpu, m, k, n):
    # 256x256 tiles split over K: the DiT down projection (150 tiles of
    # 256x128 over 160 K stages, split 3 ways) and 192 tiles of 256x128 over
    # 256 K stages (split 2 ways).
    run_and_check(gpu, m, k, n, "dyn", seed=77 + m, bias=True, sample=300)


@pytest.mark.parametrize("m,k,n", [(2048, 1024, 2048), (2048, 9216, 2048), (1024, 8192, 2048), (1280, 2048, 1536)])
def test_gemm_mid_tiles(gpu, m, k, n):
    # Tile configurations the other shapes do not reach: exactly 256 tiles of
    # 128x128 (the 128x128 DMA tile), the same split 2 ways over a long K,
    # 128 tiles of 128x128 as 64x128 tiles split 2 ways, and 480 tiles of
    # 64x64 (the 4-stage 64-byte form).
    run_and_check(gpu, m, k, n, "dyn", seed=m + 3 * k + n, bias=True, sample=300)


@pytest.mark.parametrize("n", [11008, 10995])
def test_gemm_column_split(gpu, n):
    # 32 x 43 tiles of 256x256 would be 5.4 rounds of 256 CUs: the first
    # 10240 columns run as 5 whole rounds, the rest as a second GEMM writing
    # into the same rows (output row stride n, its own tile choice). An odd
    # width takes the per-element stores. The seam between the two GEMMs
    # (columns 10240 +- 64, each side's last and first tile columns), the
    # last column and the tile-row boundaries are always in the sample.
    seam = list(range(10240 - 64, 10240 + 64)) + [n - 2, n - 1]
    run_and_check(gpu, 8192, 1024, n, "dyn", seed=n, bias=True, sample=300, must_cols=seam,
                  must_rows=[1, 255, 256, 257, 4095, 4096, 8190])


@pytest.mark.parametrize("k,n", [(3840, 3840), (3840, 10240), (3840, 11520)])
def test_gemm_dit_shapes(gpu, k, n):
    # Config 4's other linears at M = 1152 (4.5 rows of 256-row tiles): the
    # out projection on 256x128 tiles, FFN up and QKV on 256x256.
    run_and_check(gpu, 1152, k, n, "dyn", seed=k + n, bias=True, sample=300)


def test_static_scale_matmul_split_k(gpu):
    m, k, n = 64, 4096, 256
    xq = o.quant_pack(o.synth_acts(m, k, 3), np.full(m, 0.02, np.float32))
    wq, _ = o.synth_weights(n, k, 4)
    sx, sw = np.float32(0.0031), np.float32(0.0007)
    got = ops.matmul_i8_static(dev_u32(xq, gpu), dev_u32(wq, gpu), sx, sw).cpu().numpy()
    want = o.epilogue_static(o.acc_exact(xq, wq), sx, sw)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_auto_variant_and_gemv_equals_gemm(gpu):
    for m in (1, 16, 32, 33, 64):
        run_and_check(gpu, m, 1024, 640, "auto", seed=m)
    x = special_acts(24, 512, 5)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(200, 512, 6)
    args = [dev_u32(xq, gpu), dev_u32(wq, gpu), dev_f32(sx, gpu), dev_f32(sw, gpu)]
    a = ops.matmul_i8(*args, variant="gemv").cpu().numpy()
    b = ops.matmul_i8(*args, variant="dyn").cpu().numpy()
    assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_matmul_unaligned_operands(gpu):
    # Packed operands starting one word into their allocations (step_sliced
    # word offsets make this legal) take the dword-load path.
    m, k, n = 40, 256, 96
    x = special_acts(m, k, 3)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, 4)
    xb = torch.zeros(m * k // 4 + 1, dtype=torch.int32, device=gpu)
    wb = torch.zeros(n * k // 4 + 1, dtype=torch.int32, device=gpu)
    xb[1:] = dev_u32(xq.reshape(-1), gpu)
    wb[1:] = dev_u32(wq.reshape(-1), gpu)
    want = o.epilogue(o.acc_exact(xq, wq), sx, sw)
    for variant, mm in (("gemv", 32), ("dyn", m)):
        got = ops.matmul_i8(xb[1:].view(m, k // 4)[:mm], wb[1:].view(n, k // 4), dev_f32(sx[:mm], gpu),
                            dev_f32(sw, gpu), variant=variant).cpu().numpy()
        assert (got.view(np.uint32) == want[:mm].view(np.uint32)).all(), variant


def test_matmul_k_zero_and_empty(gpu):
    sx = dev_f32([0.5, 0.25], gpu)
    sw = dev_f32([1.0, 2.0, 3.0], gpu)
    bias = dev_f32([1.0, -2.0, 0.5], gpu)
    xq = torch.zeros(2, 0, dtype=torch.int32, device=gpu)
    wq = torch.zeros(3, 0, dtype=torch.int32, device=gpu)
    for variant in ("gemv", "dyn"):
        out = ops.matmul_i8(xq, wq, sx, sw, bias, variant=variant).cpu().numpy()
        assert out.tolist() == [[1.0, -2.0, 0.5]] * 2
    empty = ops.matmul_i8(torch.zeros(0, 4, dtype=torch.int32, device=gpu), torch.zeros(3, 4, dtype=torch.int32,
                          device=gpu), torch.zeros(0, device=gpu), sw)
    assert empty.shape == (0, 3)


def test_gemv_rejects_more_than_32_rows(gpu):
    from brain_amd import BrainHipError
    xq = torch.zeros(33, 4, dtype=torch.int32, device=gpu)
    with pytest.raises(BrainHipError, match="m=33"):
        ops.matmul_i8(xq, xq[:5], torch.ones(33, device=gpu), torch.ones(5, device=gpu), variant="gemv")


@pytest.mark.parametrize("m,k,n", [(70, 264, 150), (512, 1024, 3072), (2048, 1024, 4096), (4096, 1024, 8192)])
def test_static_scale_matmul(gpu, m, k, n):
    # The register-staged kernel (K % 128 != 0), then the LDS-DMA kernel on
    # 64x64, 256x128 and 256x256 tiles.
    xq = o.quant_pack(o.synth_acts(m, k, 1), np.full(m, 0.02, np.float32))
    wq, _ = o.synth_weights(n, k, 2)
    sx, sw = np.float32(0.0123), np.float32(0.0071)
    got = ops.matmul_i8_static(dev_u32(xq, gpu), dev_u32(wq, gpu), sx, sw).cpu().numpy()
    rng = np.random.default_rng(m + n)
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 200)])) if m > 512 else np.arange(m)
    cols = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 200)])) if m > 512 else np.arange(n)
    want = o.epilogue_static(o.acc_exact(xq, wq, rows, cols), sx, sw)
    assert (got[np.ix_(rows, cols)].view(np.uint32) == want.view(np.uint32)).all()


def test_linear_config0(gpu):
    # Config 0: M=16, K=1024, N=3072, f32 activations quantized in-path, f32 out.
    m, k, n = 16, 1024, 3072
    x = o.synth_acts(m, k, 0)
    wq, sw = o.synth_weights(n, k, 1)
    got = ops.linear_i8(dev_f32(x, gpu), dev_u32(wq, gpu), dev_f32(sw, gpu)).cpu().numpy()
    sx = o.max_abs_row(x)
    want = o.matmul_i8(o.quant_pack(x, sx), wq, sx, sw)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    assert (o.cpu_linear_gemv(x, wq, sw, 4).view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("m", [1, 4, 8, 16])
@pytest.mark.parametrize("k,n", [(1024, 3072), (3072, 1024), (1024, 2048), (1024, 151936), (1024, 40001), (32, 7),
                                 (2032, 40)])
def test_linear_fused_quant(gpu, m, k, n):
    """bh_linear_i8 on the decode path quantizes inside the GEMV: outputs (f32
    and bf16 with bias) and the sx / xq scratch it leaves must be exactly the
    two-launch results."""
    x = special_acts(m, k, m + k)
    wq, sw = o.synth_weights(n, k, 3)
    bias = np.random.default_rng(k).standard_normal(n).astype(np.float32)
    sx_ref = o.max_abs_row(x)
    xq_ref = o.quant_pack(x, sx_ref)
    rows = np.arange(m)
    cols = np.arange(n) if n < 20000 else np.unique(np.r_[0, n - 1, np.random.default_rng(1).integers(0, n, 500)])
    acc = o.acc_exact(xq_ref, wq, rows, cols)
    sx_s = torch.empty(m, device=gpu)
    xq_s = torch.empty(m, k // 4, device=gpu, dtype=torch.int32)
    xd, wd, swd = dev_f32(x, gpu), dev_u32(wq, gpu), dev_f32(sw, gpu)
    got = ops.linear_i8(xd, wd, swd, sx=sx_s, xq=xq_s).cpu().numpy()
    assert (sx_s.cpu().numpy().view(np.uint32) == sx_ref.view(np.uint32)).all()
    assert (host_u32(xq_s) == xq_ref).all()
    want = o.epilogue(acc, sx_ref, sw[cols])
    assert (got[:, cols].view(np.uint32) == want.view(np.uint32)).all()
    gotb = bf16_bits(ops.linear_i8(xd, wd, swd, dev_f32(bias, gpu), torch.bfloat16))
    wantb = o.epilogue(acc, sx_ref, sw[cols], bias[cols], "bf16")
    assert (gotb[:, cols] == wantb).all()


@pytest.mark.parametrize("n,k", [(1, 64), (3, 8), (17, 24), (64, 4096), (129, 128), (300, 1000), (5, 2052),
                                 (6, 1500), (33, 4100)])
def test_device_weight_quantizer(gpu, n, k):
    rng = np.random.default_rng(n + k)
    w = (rng.standard_normal((n, k)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w[0, :4] = [0.5, -0.5, 1.5, -2.5]
    w[-1, :4] = [127.0, 0.5, 1.5, 2.5] if n > 1 else w[-1, :4]
    packed, sw = ops.quantize_weight_device(dev_f32(w, gpu))
    wp, wsw = o.quantize_weight(w)
    assert (host_u32(packed) == wp).all()
    assert (sw.cpu().numpy() == wsw).all()


@pytest.mark.parametrize("variant,m", [("dyn", 300), ("dyn", 1024), ("gemv", 7)])
def test_matmul_unaligned_scales_bias_and_output(gpu, variant, m):
    # sw, bias and out one word into their allocations (legal with step_sliced
    # word offsets): the vector epilogue must fall back to scalar accesses.
    k, n = 1024, 516
    x = special_acts(m, k, 8)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, 9)
    bias = o.synth_acts(1, n, 10)[0]
    swb = torch.zeros(n + 1, device=gpu)
    swb[1:] = dev_f32(sw, gpu)
    bb = torch.zeros(n + 1, device=gpu)
    bb[1:] = dev_f32(bias, gpu)
    acc = o.acc_exact(xq, wq)
    for dt, want in ((torch.float32, o.epilogue(acc, sx, sw, bias).view(np.uint32)),
                     (torch.bfloat16, o.epilogue(acc, sx, sw, bias, "bf16"))):
        ob = torch.zeros(m * n + 1, dtype=dt, device=gpu)
        ops.matmul_i8(dev_u32(xq, gpu), dev_u32(wq, gpu), dev_f32(sx, gpu), swb[1:], bb[1:], dt, variant,
                      out=ob[1:].view(m, n))
        got = ob[1:].view(m, n).cpu()
        got = got.numpy().view(np.uint32) if dt == torch.float32 else bf16_bits(got)
        assert (got == want).all(), dt
