"""Object wrapper of the C-ABI `backend_api::Backend` mirror in libbrain_hip.so.

Mirrors how a Rust `backend-hip` crate forwards `impl Backend` to the C ABI:
buffers and recorded steps are refcounted handles; `step_sliced` offsets are in
4-byte words; `submit` zeroes `clears` and runs steps in order.
"""
import ctypes as C

import numpy as np

from ._lib import CapsT, KernelTimeT, StatsT, check, load


class Buffer:
    def __init__(self, be, handle):
        self.be, self.h = be, handle

    @property
    def words(self):
        return load().bh_buffer_words(self.h)

    @property
    def ptr(self):
        return load().bh_buffer_device_ptr(self.h)

    def clone(self):
        return Buffer(self.be, load().bh_buffer_retain(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            load().bh_buffer_release(self.h)
            self.h = None


class Step:
    def __init__(self, handle):
        self.h = handle

    def __del__(self):
        if getattr(self, "h", None):
            load().bh_step_release(self.h)
            self.h = None


class HipBackend:
    """`Box<dyn Backend>` built by the "hip" factory for a kernel-name list."""

    def __init__(self, names, device=0, lenient=False):
        lib = load()
        arr = (C.c_char_p * len(names))(*[n.encode() for n in names])
        h = C.c_void_p()
        check(lib.bh_backend_create(arr, None, len(names), device, 1 if lenient else 0, C.byref(h)))
        self.h = h.value
        self.names = list(names)

    def __del__(self):
        if getattr(self, "h", None):
            load().bh_backend_destroy(self.h)
            self.h = None

    def kind(self):
        return load().bh_backend_kind(self.h).decode()

    def kernel_index(self, name):
        i = load().bh_kernel_index(self.h, name.encode())
        return None if i < 0 else i

    def caps(self):
        c = CapsT()
        check(load().bh_caps(self.h, C.byref(c)))
        return c

    def storage(self, n_words):
        h = C.c_void_p()
        check(load().bh_storage(self.h, n_words, C.byref(h)))
        return Buffer(self, h.value)

    def storage_init(self, name, data):
        a = np.ascontiguousarray(data, dtype=np.float32)
        h = C.c_void_p()
        check(load().bh_storage_init(self.h, name.encode(), a.ctypes.data, a.size, C.byref(h)))
        return Buffer(self, h.value)

    def write(self, buf, data):
        a = np.ascontiguousarray(data).view(np.uint32).reshape(-1)
        check(load().bh_write(self.h, buf.h, a.ctypes.data, a.size))

    def write_at(self, buf, offset_words, data):
        a = np.ascontiguousarray(data).view(np.uint32).reshape(-1)
        check(load().bh_write_at(self.h, buf.h, offset_words, a.ctypes.data, a.size))

    def read(self, buf, n, dtype=np.float32):
        out = np.zeros(n, np.uint32)
        check(load().bh_read(self.h, buf.h, out.ctypes.data, n))
        return out.view(dtype)

    def _bufs(self, bufs):
        return (C.c_void_p * len(bufs))(*[b.h for b in bufs])

    def step(self, kind, bufs, params, threads=0):
        p = (C.c_uint32 * len(params))(*[int(v) & 0xFFFFFFFF for v in params])
        h = C.c_void_p()
        check(load().bh_step(self.h, kind, self._bufs(bufs), len(bufs), p, len(params), threads, C.byref(h)))
        return Step(h.value)

    def step_sliced(self, kind, bufs, offsets, params, threads=0):
        p = (C.c_uint32 * len(params))(*[int(v) & 0xFFFFFFFF for v in params])
        off = (C.c_uint64 * (2 * len(bufs)))(*[int(v) for pair in offsets for v in pair])
        h = C.c_void_p()
        check(load().bh_step_sliced(self.h, kind, self._bufs(bufs), off, len(bufs), p, len(params), threads,
                                    C.byref(h)))
        return Step(h.value)

    def submit(self, clears, steps):
        cl = (C.c_void_p * max(1, len(clears)))(*[b.h for b in clears])
        st = (C.c_void_p * max(1, len(steps)))(*[s.h for s in steps])
        check(load().bh_submit(self.h, cl, len(clears), st, len(steps)))

    def poll_wait(self):
        check(load().bh_poll_wait(self.h))

    def poll_wait_timeout(self, ms):
        return load().bh_poll_wait_timeout(self.h, ms) == 0

    def set_kernel_timing(self, on):
        return bool(load().bh_set_kernel_timing(self.h, 1 if on else 0))

    def kernel_times(self):
        arr = (KernelTimeT * 64)()
        n = check(load().bh_kernel_times(self.h, arr, 64))
        return [(arr[i].name.decode(), arr[i].ms, arr[i].calls) for i in range(min(n, 64))]

    def reset_kernel_times(self):
        load().bh_reset_kernel_times(self.h)

    def stats(self):
        s = StatsT()
        check(load().bh_stats(self.h, C.byref(s)))
        return {f: getattr(s, f) for f, _ in StatsT._fields_}

    # --- model-layer helpers (crates/model/src/int8.rs, dispatch.rs) ---
    def quant_rows_steps(self, kernels, x, sx, xq, r0, r1, k):
        ks = (C.c_uint32 * 2)(*kernels)
        out = (C.c_void_p * 2)()
        check(load().bh_quant_rows_steps(self.h, ks, x.h, sx.h, xq.h, r0, r1, k, out))
        return [Step(out[0]), Step(out[1])]

    def mm8_rows_off(self, kind, xq, wq, sx, sw, o, xr0, ooff, m, k, n):
        h = C.c_void_p()
        check(load().bh_mm8_rows_off(self.h, kind, xq.h, wq.h, sx.h, sw.h, o.h, xr0, ooff, m, k, n, C.byref(h)))
        return Step(h.value)
