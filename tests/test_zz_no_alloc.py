"""bh_matmul_i8_dyn_noalloc: the prefill GEMM with its split-K slabs in the
library's fixed device scratch instead of an allocated workspace. It must
give exactly bh_matmul_i8_dyn's results, call after call (the scratch keeps
the previous call's contents), and refuse shapes whose slabs exceed the
scratch."""
import ctypes as C

import numpy as np
import pytest
import torch

from brain_amd import _lib
from oracle import oracle as o

pytestmark = pytest.mark.gpu

OUTS = ((_lib.BH_OUT_I32, torch.int32), (_lib.BH_OUT_F32, torch.float32), (_lib.BH_OUT_BF16, torch.bfloat16))


def operands(m, k, n, seed, gpu):
    x = o.synth_acts(m, k, seed)
    sx = o.max_abs_row(x)
    xq = o.quant_pack(x, sx)
    wq, sw = o.synth_weights(n, k, seed + 1)
    bias = o.synth_acts(1, n, seed + 2)[0]
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(gpu)
    return t(xq, np.int32), t(wq, np.int32), t(sx, np.float32), t(sw, np.float32), t(bias, np.float32)


def call(fn, ops, m, k, n, code, dt, gpu):
    xq, wq, sx, sw, bias = ops
    out = torch.full((m, n), 7, dtype=dt, device=gpu)
    b = None if code == _lib.BH_OUT_I32 else bias.data_ptr()
    rc = fn(torch.cuda.current_stream().cuda_stream, xq.data_ptr(), wq.data_ptr(), sx.data_ptr(), sw.data_ptr(), b,
            out.data_ptr(), code, m, k // 4, n)
    return rc, out


def test_noalloc_matches_dyn_two_calls(gpu):
    lib = _lib.load()
    # 128x3072x1024 splits K 6 ways (3 MB of slabs); 64x4096x512 splits 8 ways
    # (1 MB): the second, smaller call reuses the scratch the first filled.
    for m, k, n in ((128, 3072, 1024), (64, 4096, 512)):
        ops = operands(m, k, n, m + k + n, gpu)
        for code, dt in OUTS:
            print(f"noalloc m={m} k={k} n={n} out={code}", flush=True)
            rc0, want = call(lib.bh_matmul_i8_dyn, ops, m, k, n, code, dt, gpu)
            rc1, got = call(lib.bh_matmul_i8_dyn_noalloc, ops, m, k, n, code, dt, gpu)
            torch.cuda.synchronize()
            assert rc0 == 0 and rc1 == 0, _lib.load().bh_last_error().decode()
            assert torch.equal(got.view(torch.int32 if dt != torch.bfloat16 else torch.int16),
                               want.view(torch.int32 if dt != torch.bfloat16 else torch.int16)), (m, k, n, code)
    # The i32 accumulators are the exact integer sums.
    m, k, n = 64, 4096, 512
    ops = operands(m, k, n, m + k + n, gpu)
    rc, acc = call(lib.bh_matmul_i8_dyn_noalloc, ops, m, k, n, _lib.BH_OUT_I32, torch.int32, gpu)
    xq = ops[0].cpu().numpy().view(np.uint32)
    wq = ops[1].cpu().numpy().view(np.uint32)
    assert rc == 0 and (acc.cpu().numpy() == o.acc_exact(xq, wq, np.arange(m), np.arange(n))).all()


def test_noalloc_takes_no_device_memory(gpu):
    lib = _lib.load()
    m, k, n = 128, 4096, 768  # splits K; a shape no other test runs, so no workspace of that size exists
    ops = operands(m, k, n, 5, gpu)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc, _ = call(lib.bh_matmul_i8_dyn_noalloc, ops, m, k, n, _lib.BH_OUT_F32, torch.float32, gpu)
    torch.cuda.synchronize()
    assert rc == 0, _lib.load().bh_last_error().decode()
    # (the output tensor comes from torch's cache, allocated above by `call`
    # before the library runs; compare against a second identical call)
    free1 = torch.cuda.mem_get_info()[0]
    rc, _ = call(lib.bh_matmul_i8_dyn_noalloc, ops, m, k, n, _lib.BH_OUT_F32, torch.float32, gpu)
    torch.cuda.synchronize()
    assert rc == 0 and torch.cuda.mem_get_info()[0] == free1
    assert free0 - free1 <= 4 << 20  # at most torch's own block for `out`, never the 6+ MB of slabs


def test_noalloc_rejects_slabs_beyond_scratch(gpu):
    lib = _lib.load()
    # The DiT down projection splits its 256x256 tiles 3 ways: 3*1152*3840*4
    # bytes = 53 MB of slabs, beyond the 32 MiB scratch.
    m, k, n = 1152, 10240, 3840
    xq = torch.zeros(m, k // 4, dtype=torch.int32, device=gpu)
    wq = torch.zeros(n, k // 4, dtype=torch.int32, device=gpu)
    sx = torch.ones(m, device=gpu)
    sw = torch.ones(n, device=gpu)
    out = torch.zeros(m, n, device=gpu)
    rc = lib.bh_matmul_i8_dyn_noalloc(torch.cuda.current_stream().cuda_stream, xq.data_ptr(), wq.data_ptr(),
                                      sx.data_ptr(), sw.data_ptr(), None, out.data_ptr(), _lib.BH_OUT_F32, m, k // 4, n)
    assert rc == _lib.BH_ERR_INVALID
    assert "scratch" in _lib.load().bh_last_error().decode()
    torch.cuda.synchronize()
    assert int(out.abs().sum().item()) == 0  # nothing launched


def test_noalloc_refuses_an_overlapping_call_from_another_stream(gpu):
    """The scratch is one array per GPU: while a call that uses it is still
    queued on one stream (held behind a short spin kernel), a call on another
    stream is refused; once the first stream is idle the same call runs and
    matches bh_matmul_i8_dyn."""
    lib = _lib.load()
    m, k, n = 128, 3072, 1024  # splits K: uses the scratch
    ops = operands(m, k, n, 5, gpu)
    xq, wq, sx, sw, bias = ops
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    out_a = torch.empty(m, n, dtype=torch.float32, device=gpu)
    out_b = torch.empty(m, n, dtype=torch.float32, device=gpu)
    args = lambda st, out: (st.cuda_stream, xq.data_ptr(), wq.data_ptr(), sx.data_ptr(), sw.data_ptr(),
                            bias.data_ptr(), out.data_ptr(), _lib.BH_OUT_F32, m, k // 4, n)
    assert a.cuda_stream != b.cuda_stream
    with torch.cuda.stream(a):
        torch.cuda._sleep(200_000_000)          # tens of ms or more of spinning ahead of the call on stream a
    assert lib.bh_matmul_i8_dyn_noalloc(*args(a, out_a)) == 0
    rc = lib.bh_matmul_i8_dyn_noalloc(*args(b, out_b))
    busy = not a.query()                        # still busy now => was busy when the call checked
    assert busy, "the spin on stream a ended before the second call; lengthen it"
    assert rc != 0 and "another stream" in lib.bh_last_error().decode()
    a.synchronize()
    assert lib.bh_matmul_i8_dyn_noalloc(*args(b, out_b)) == 0
    b.synchronize()
    _, want = call(lib.bh_matmul_i8_dyn, ops, m, k, n, _lib.BH_OUT_F32, torch.float32, gpu)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int32), want.view(torch.int32))
    assert torch.equal(out_b.view(torch.int32), want.view(torch.int32))
