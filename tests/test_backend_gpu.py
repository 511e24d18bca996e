"""The backend_api::Backend mirror on the GPU: name-keyed steps, word offsets,
ordered submit, bounds/alias rejection, clears, timing and stats — exercised
the way brain's model layer drives a backend (crates/model/src/int8.rs,
dispatch.rs, ops.rs)."""
import numpy as np
import pytest

from brain_amd import BrainHipError
from brain_amd import _lib
from brain_amd.backend import HipBackend
from oracle import oracle as o

pytestmark = pytest.mark.gpu

NAMES = ["max_abs_row", "max_abs_rows", "quant_pack", "matmul_i8_dyn", "matmul_i8_gemv", "matmul_i8",
         "bias_add", "roof_dp4a"]


@pytest.fixture(scope="module")
def be(gpu):
    return HipBackend(NAMES)


def K(be, name):
    return be.kernel_index(name)


def test_caps_and_identity(be):
    c = be.caps()
    assert be.kind() == "hip"
    assert c.numeric_int8_dot == 1 and c.workgroup_reductions == 1
    assert c.subgroup_size == 64 and c.compute_units >= 1
    assert be.kernel_index("matmul_i8_dyn") == 3 and be.kernel_index("nope") is None


def test_unknown_kernel_strict_and_lenient(gpu):
    with pytest.raises(BrainHipError, match="rmsnorm"):
        HipBackend(["matmul_i8_dyn", "rmsnorm"])
    b = HipBackend(["matmul_i8_dyn", "rmsnorm"], lenient=True)
    buf = b.storage(4)
    with pytest.raises(BrainHipError, match="not provided"):
        b.step(1, [buf, buf], [1, 4])


def test_gemv_known_answer_through_step(be):
    # crates/wgsl-cpu/src/lib.rs:1633-1679, dispatched like the reference test.
    m, k, n = 2, 8, 3
    xi = np.array([((i * 37 + 11) % 255 - 127) for i in range(m * k)], np.int64).astype(np.int8)
    wi = np.array([((i * 53 + 5) % 255 - 127) for i in range(n * k)], np.int64).astype(np.int8)
    xq = be.storage(m * k // 4)
    be.write(xq, xi.view(np.uint32))
    wq = be.storage(n * k // 4)
    be.write(wq, wi.view(np.uint32))
    sx = be.storage_init("sx", [0.5, 0.25])
    sw = be.storage_init("sw", [1.0, 2.0, 0.125])
    for name in ("matmul_i8_gemv", "matmul_i8_dyn"):
        out = be.storage(m * n)
        be.submit([], [be.step(K(be, name), [xq, wq, sx, sw, out], [m, k // 4, n], n * 64)])
        assert be.read(out, m * n).reshape(m, n).tolist() == [[4830.0, 17202.0, -668.8125],
                                                              [3542.0, -3886.5, -330.90625]]


def test_quant_rows_steps_and_mm8_row_offset(be):
    # ops_facade_parity.rs:320-340: rows xr0=64.. of a batch equal the same rows
    # quantized and multiplied on their own.
    rows, k, n = 128, 256, 96
    x = o.synth_acts(rows, k, 21)
    wqh, swh = o.synth_weights(n, k, 22)
    xb = be.storage_init("x", x.reshape(-1))
    sxb = be.storage(rows)
    xqb = be.storage(rows * k // 4)
    wqb = be.storage(n * k // 4)
    be.write(wqb, wqh)
    swb = be.storage_init("sw", swh)
    ob = be.storage(rows * n)
    kq = [K(be, "max_abs_row"), K(be, "quant_pack")]
    steps = be.quant_rows_steps(kq, xb, sxb, xqb, 64, 128, k)
    steps += [be.mm8_rows_off(K(be, "matmul_i8_dyn"), xqb, wqb, sxb, swb, ob, 64, 64 * n, 64, k, n)]
    be.submit([ob], steps)
    got = be.read(ob, rows * n).reshape(rows, n)
    sub = x[64:]
    sx = o.max_abs_row(sub)
    want = o.matmul_i8(o.quant_pack(sub, sx), wqh, sx, swh)
    assert (got[64:].view(np.uint32) == want.view(np.uint32)).all()
    assert (got[:64] == 0).all()   # cleared, never written
    with pytest.raises(BrainHipError, match="64-float alignment"):
        be.quant_rows_steps(kq, xb, sxb, xqb, 32, 64, k)


def test_sliced_gemv_with_row_offset_matches_unsliced(be):
    m, k, n = 8, 1024, 320
    x = o.synth_acts(m + 5, k, 31)
    sxh = o.max_abs_row(x)
    xqh = o.quant_pack(x, sxh)
    wqh, swh = o.synth_weights(n, k, 32)
    xq = be.storage(xqh.size)
    be.write(xq, xqh)
    wq = be.storage(wqh.size)
    be.write(wq, wqh)
    sx = be.storage_init("sx", sxh)
    sw = be.storage_init("sw", swh)
    out = be.storage(m * n + 7)
    kg = k // 4
    st = be.step_sliced(K(be, "matmul_i8_gemv"), [xq, wq, sx, sw, out],
                        [(5 * kg, m * kg), (0, 0), (5, m), (0, 0), (7, m * n)], [m, kg, n])
    be.submit([out], [st])
    got = be.read(out, m * n + 7)[7:].reshape(m, n)
    want = o.matmul_i8(xqh[5:], wqh, sxh[5:], swh)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_bindings_are_bounds_checked(be):
    xq = be.storage(16)
    wq = be.storage(16)
    sx = be.storage(4)
    sw = be.storage(4)
    out = be.storage(15)
    with pytest.raises(BrainHipError, match="binding 4 needs 16"):
        be.step(K(be, "matmul_i8_dyn"), [xq, wq, sx, sw, out], [4, 4, 4])
    with pytest.raises(BrainHipError, match="4 bindings, expected 5"):
        be.step(K(be, "matmul_i8_dyn"), [xq, wq, sx, sw], [4, 4, 4])
    with pytest.raises(BrainHipError, match="past"):
        be.step_sliced(K(be, "matmul_i8_dyn"), [xq, wq, sx, sw, out],
                       [(0, 0), (0, 0), (0, 0), (0, 0), (10, 10)], [1, 1, 1])
    with pytest.raises(BrainHipError, match="m=33"):
        big = be.storage(33 * 4)
        be.step(K(be, "matmul_i8_gemv"), [big, wq, big, sw, big], [33, 1, 1])
    with pytest.raises(BrainHipError, match="overlaps"):
        be.step(K(be, "matmul_i8_dyn"), [xq, wq, sx, sw, xq], [2, 2, 2])


def test_static_bias_add_and_roof_steps(be):
    m, k, n = 20, 64, 40
    xqh = o.quant_pack(o.synth_acts(m, k, 41), np.full(m, 0.02, np.float32))
    wqh, _ = o.synth_weights(n, k, 42)
    xq = be.storage(xqh.size)
    be.write(xq, xqh)
    wq = be.storage(wqh.size)
    be.write(wq, wqh)
    out = be.storage(m * n)
    bias = o.synth_acts(1, n, 43)[0]
    bb = be.storage_init("b", bias)
    sxs, sws = np.float32(0.013), np.float32(0.007)
    p = [m, k // 4, n, int(np.array(sxs).view(np.uint32)), int(np.array(sws).view(np.uint32))]
    be.submit([], [be.step(K(be, "matmul_i8"), [xq, wq, out], p), be.step(K(be, "bias_add"), [out, bb], [m, n])])
    want = o.epilogue_static(o.matmul_i8_acc(xqh, wqh), sxs, sws) + bias[None, :]
    assert (be.read(out, m * n).reshape(m, n).view(np.uint32) == want.view(np.uint32)).all()
    # roof_dp4a: out = inp + f32(8*iters*dot4(a,b)) with wrapping i32
    nn, iters, a, b = 100, 1000, 0x7F80FF01, 0x01FF7F80
    inp = np.arange(nn, dtype=np.float32)
    ib = be.storage_init("inp", inp)
    ob = be.storage(nn)
    be.submit([], [be.step(K(be, "roof_dp4a"), [ib, ob], [nn, iters, a, b])])
    ai = np.array([a], np.uint32).view(np.int8).astype(np.int64)
    bi = np.array([b], np.uint32).view(np.int8).astype(np.int64)
    s = np.int64(8 * iters * int((ai * bi).sum()))
    s32 = np.array([s & 0xFFFFFFFF], np.uint32).view(np.int32)[0]
    assert (be.read(ob, nn) == inp + np.float32(s32)).all()


def test_timing_stats_and_waits(be):
    m, k, n = 4, 256, 64
    xq = be.storage(m * k // 4)
    wq = be.storage(n * k // 4)
    sx = be.storage_init("sx", np.ones(m, np.float32))
    sw = be.storage_init("sw", np.ones(n, np.float32))
    out = be.storage(m * n)
    before = be.stats()
    assert be.set_kernel_timing(True)
    be.reset_kernel_times()
    st = be.step(K(be, "matmul_i8_gemv"), [xq, wq, sx, sw, out], [m, k // 4, n])
    be.submit([], [st, st, st])
    assert be.poll_wait_timeout(10000)
    be.poll_wait()
    times = dict((name, (ms, calls)) for name, ms, calls in be.kernel_times())
    assert times["matmul_i8_gemv"][1] == 3 and times["matmul_i8_gemv"][0] > 0
    be.set_kernel_timing(False)
    after = be.stats()
    assert after["submits"] == before["submits"] + 1
    assert after["dispatches"] == before["dispatches"] + 3
    assert after["bind_groups"] == before["bind_groups"] + 1


def test_buffers_refcount_and_write_at(be):
    b = be.storage(10)
    c = b.clone()
    del b
    be.write_at(c, 3, np.array([1.5, 2.5], np.float32))
    assert be.read(c, 10).tolist() == [0, 0, 0, 1.5, 2.5, 0, 0, 0, 0, 0]
    with pytest.raises(BrainHipError, match="past"):
        be.write_at(c, 9, np.array([1.0, 2.0], np.float32))
    assert c.words == 10 and c.ptr
    assert _lib.BH_ERR_TIMEOUT == -5
