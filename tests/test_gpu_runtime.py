"""The runtime surface on the GPU: streams, events, asynchronous copies
through pinned host memory, and a code object's kernels launched by name
(tatara_stream_* / tatara_event_* / tatara_memcpy_*_async /
tatara_host_*_pinned / tatara_module_*; crates/gpu-runtime/src/lib.rs:186-390,
native_backend.rs:17-300).

The kernels are those of tests/kernels/runtime_selftest.hip, compiled to a
gfx950 code object by build().  Their outputs are integer or single
rounding-step float work, so every check is bit-exact against numpy.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from tatara_amd import runtime as rt
from tatara_amd._lib import TataraError, check, load

pytestmark = pytest.mark.gpu

IMAGE = Path(__file__).resolve().parent / "kernels" / "runtime_selftest.hsaco"


class Dev:
    """A device buffer of n elements of a numpy dtype."""

    def __init__(self, n, dtype):
        self.n, self.dtype = n, np.dtype(dtype)
        self.nbytes = n * self.dtype.itemsize
        p = C.c_void_p()
        check(load().tatara_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            check(load().tatara_free(self.ptr))
            self.ptr = None


class Pinned:
    """Pinned host memory seen as a numpy array."""

    def __init__(self, n, dtype):
        self.dtype = np.dtype(dtype)
        self.nbytes = n * self.dtype.itemsize
        self.ptr = rt.alloc_pinned_host(self.nbytes)
        self.a = np.frombuffer((C.c_char * self.nbytes).from_address(self.ptr), dtype=self.dtype)

    def free(self):
        if self.ptr:
            self.a = None
            rt.free_pinned_host(self.ptr)
            self.ptr = None


@pytest.fixture(scope="module")
def module(gpu):
    assert IMAGE.exists(), f"{IMAGE} is missing: run __graft_entry__.build()"
    m = rt.Module.from_file(IMAGE)
    yield m
    m.close()


def test_device_attributes(gpu):
    cus, threads = rt.device_occupancy_attributes(0)
    assert cus == 256 and threads >= 2048, (cus, threads)
    assert rt.compute_capability(0) == (9, 5)


def test_axpy_through_pinned_async_copies_on_one_stream(module):
    n = 100_003
    rng = np.random.default_rng(1)
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    a = np.float32(-1.75)
    hx, hy, out = Pinned(n, np.float32), Pinned(n, np.float32), Pinned(n, np.float32)
    dx, dy = Dev(n, np.float32), Dev(n, np.float32)
    hx.a[:] = x
    hy.a[:] = y
    with rt.Stream() as s:
        rt.memcpy_htod_async(dx.ptr, hx.ptr, dx.nbytes, s)
        rt.memcpy_htod_async(dy.ptr, hy.ptr, dy.nbytes, s)
        args = rt.KernelArgs().push_slice(dy.ptr, n).push_slice(dx.ptr, n).push_scalar(a, C.c_float)
        module.launch("selftest_axpy", s, rt.LaunchConfig.for_num_elems(n), args)
        rt.memcpy_dtoh_async(out.ptr, dy.ptr, dy.nbytes, s)
        s.synchronize()
    exp = a * x + y  # one rounding for the product, one for the sum (no contraction)
    assert np.array_equal(out.a, exp)
    for b in (hx, hy, out, dx, dy):
        b.free()


def test_two_dimensional_launch(module):
    w, h, base = 1000, 37, 12345
    d = Dev(w * h, np.uint32)
    out = np.zeros(w * h, np.uint32)
    with rt.Stream() as s:
        rt.memset_d8_async(d.ptr, 0xFF, d.nbytes, s)
        args = (rt.KernelArgs().push_slice(d.ptr, w * h).push_scalar(w, C.c_uint32).push_scalar(h, C.c_uint32)
                .push_scalar(base, C.c_uint32))
        cfg = rt.LaunchConfig((-(-w // 16), -(-h // 16), 1), (16, 16, 1), 0)
        module.launch("selftest_iota2d", s, cfg, args)
        s.synchronize()
    check(load().tatara_memcpy_dtoh(out.ctypes.data, d.ptr, d.nbytes))
    assert np.array_equal(out, base + np.arange(w * h, dtype=np.uint32))
    d.free()


def test_dynamic_shared_memory(module):
    bs, nblk = 256, 40
    n = bs * nblk
    src = np.arange(n, dtype=np.uint32) * 7 + 3
    din, dout = Dev(n, np.uint32), Dev(n, np.uint32)
    check(load().tatara_memcpy_htod(din.ptr, src.ctypes.data, din.nbytes))
    args = rt.KernelArgs().push_slice(dout.ptr, n).push_slice(din.ptr, n)
    module.launch("selftest_reverse_segments", None, rt.LaunchConfig((nblk, 1, 1), (bs, 1, 1), bs * 4), args)
    check(load().tatara_synchronize())
    out = np.zeros(n, np.uint32)
    check(load().tatara_memcpy_dtoh(out.ctypes.data, dout.ptr, dout.nbytes))
    assert np.array_equal(out, src.reshape(nblk, bs)[:, ::-1].reshape(-1))
    din.free()
    dout.free()


def test_cross_stream_order_through_an_event(module):
    """Upload and compute on one stream, download on another that waits on an
    event recorded after the kernel (the upload ring's h2d_done pattern,
    trainer_common.rs:1229)."""
    n = 1 << 20
    rng = np.random.default_rng(2)
    x = rng.standard_normal(n).astype(np.float32)
    hx, out = Pinned(n, np.float32), Pinned(n, np.float32)
    hx.a[:] = x
    out.a[:] = np.nan
    dx, dy = Dev(n, np.float32), Dev(n, np.float32)
    a, b = rt.Stream(), rt.Stream()
    t0, t1, done = rt.Event(), rt.Event(), rt.Event(flags=rt.EVENT_DISABLE_TIMING)
    t0.record(a)
    rt.memset_d8_async(dy.ptr, 0, dy.nbytes, a)
    rt.memcpy_htod_async(dx.ptr, hx.ptr, dx.nbytes, a)
    args = rt.KernelArgs().push_slice(dy.ptr, n).push_slice(dx.ptr, n).push_scalar(3.0, C.c_float)
    module.launch("selftest_axpy", a, rt.LaunchConfig.for_num_elems(n), args)
    t1.record(a)
    done.record(a)
    b.wait(done)
    rt.memcpy_dtoh_async(out.ptr, dy.ptr, dy.nbytes, b)
    b.synchronize()
    assert np.array_equal(out.a, np.float32(3.0) * x)
    t1.synchronize()
    assert t1.query() and done.query()
    assert t0.elapsed_ms(t1) >= 0.0
    with pytest.raises(TataraError):  # timing disabled on `done`
        t0.elapsed_ms(done)
    for e in (t0, t1, done):
        e.close()
    a.close()
    b.close()
    for buf in (hx, out, dx, dy):
        buf.free()


def test_unknown_kernel_name_fails_before_launch(module):
    with pytest.raises(TataraError, match="no_such_kernel"):
        module.launch("no_such_kernel", None, rt.LaunchConfig((1, 1, 1), (64, 1, 1)), rt.KernelArgs())
    # the reported error does not linger: the library's next launch check
    # (here tatara_op_copy's) sees only its own launch
    src, dst = Dev(1024, np.float32), Dev(1024, np.float32)
    vals = np.arange(1024, dtype=np.float32)
    check(load().tatara_memcpy_htod(src.ptr, vals.ctypes.data, src.nbytes))
    check(load().tatara_op_copy(dst.ptr, src.ptr, src.nbytes))
    got = np.zeros(1024, np.float32)
    check(load().tatara_memcpy_dtoh(got.ctypes.data, dst.ptr, dst.nbytes))
    assert np.array_equal(got, vals)
    src.free()
    dst.free()
    # the module still launches its own kernels afterwards
    d = Dev(64, np.uint32)
    args = (rt.KernelArgs().push_slice(d.ptr, 64).push_scalar(64, C.c_uint32).push_scalar(1, C.c_uint32)
            .push_scalar(0, C.c_uint32))
    module.launch("selftest_iota2d", None, rt.LaunchConfig((1, 1, 1), (64, 1, 1)), args)
    check(load().tatara_synchronize())
    out = np.zeros(64, np.uint32)
    check(load().tatara_memcpy_dtoh(out.ctypes.data, d.ptr, d.nbytes))
    assert np.array_equal(out, np.arange(64, dtype=np.uint32))
    d.free()
