"""Host-side mirror of the reference's device runtime surface.

Streams, events, asynchronous copies, pinned host memory and code objects
launched by kernel name, over the C ABI (tatara_stream_*, tatara_event_*,
tatara_memcpy_*_async, tatara_host_*_pinned, tatara_module_*).  The names and
argument meanings follow crates/gpu-runtime: CudaStream / CudaEvent /
CudaModule / KernelArgs / LaunchConfig (native_backend.rs:17-281),
alloc_pinned_host / free_pinned_host / memset_d8_async / memcpy_*_async /
device_occupancy_attributes (lib.rs:232-390) and grid_dim_1d
(kernel_loader.rs:16-19).  Errors raise TataraError (OutOfMemory for an
allocation failure), as the reference's Result does.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from pathlib import Path

from . import _lib
from ._lib import check

EVENT_BLOCKING_SYNC = 1
EVENT_DISABLE_TIMING = 2
BLOCK_DIM = 256  # kernel_loader.rs:13


def grid_dim_1d(n: int, block: int = BLOCK_DIM) -> tuple[int, int, int]:
    """ceil(n / block) blocks, one block for n = 0 (kernel_loader.rs:16-19)."""
    return (-(-max(n, 1) // block), 1, 1)


@dataclass
class LaunchConfig:
    grid_dim: tuple[int, int, int]
    block_dim: tuple[int, int, int]
    shared_mem_bytes: int = 0

    @classmethod
    def for_num_elems(cls, n: int) -> "LaunchConfig":
        """256-thread blocks over n elements (native_backend.rs:23-31)."""
        return cls((-(-n // 256), 1, 1), (256, 1, 1), 0)


def device_occupancy_attributes(device: int = 0) -> tuple[int, int]:
    """(compute units, max threads per compute unit)."""
    cu, th = C.c_int32(), C.c_int32()
    check(_lib.load().tatara_device_occupancy_attributes(device, C.byref(cu), C.byref(th)))
    return cu.value, th.value


def compute_capability(device: int = 0) -> tuple[int, int]:
    ma, mi = C.c_int32(), C.c_int32()
    check(_lib.load().tatara_device_compute_capability(device, C.byref(ma), C.byref(mi)))
    return ma.value, mi.value


class Stream:
    """A non-blocking stream at the default priority (CudaContext::new_stream)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(_lib.load().tatara_stream_create(device, C.byref(h)))
        self.handle = h.value
        self.device = device

    def synchronize(self) -> None:
        check(_lib.load().tatara_stream_synchronize(self.handle))

    def wait(self, event: "Event") -> None:
        """Work queued on this stream after the call waits for `event`."""
        check(_lib.load().tatara_stream_wait_event(self.handle, event.handle))

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            check(_lib.load().tatara_stream_destroy(h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    """CudaContext::new_event; flags: EVENT_BLOCKING_SYNC | EVENT_DISABLE_TIMING."""

    def __init__(self, device: int = 0, flags: int = 0):
        h = C.c_void_p()
        check(_lib.load().tatara_event_create(device, flags, C.byref(h)))
        self.handle = h.value
        self.device = device

    def record(self, stream: Stream | None) -> None:
        check(_lib.load().tatara_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self) -> None:
        check(_lib.load().tatara_event_synchronize(self.handle))

    def query(self) -> bool:
        done = C.c_int32()
        check(_lib.load().tatara_event_query(self.handle, C.byref(done)))
        return bool(done.value)

    def elapsed_ms(self, end: "Event") -> float:
        """Milliseconds from this event to `end`, both completed."""
        ms = C.c_float()
        check(_lib.load().tatara_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            check(_lib.load().tatara_event_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sh(stream: Stream | None):
    return stream.handle if stream else None


def memset_d8_async(dst: int, value: int, nbytes: int, stream: Stream | None) -> None:
    check(_lib.load().tatara_memset_d8_async(dst, value, nbytes, _sh(stream)))


def memcpy_htod_async(dst: int, src: int, nbytes: int, stream: Stream | None) -> None:
    """The host buffer at `src` must stay alive until the stream has passed the copy."""
    check(_lib.load().tatara_memcpy_htod_async(dst, src, nbytes, _sh(stream)))


def memcpy_dtoh_async(dst: int, src: int, nbytes: int, stream: Stream | None) -> None:
    """The host buffer at `dst` must not be read until the stream has passed the copy."""
    check(_lib.load().tatara_memcpy_dtoh_async(dst, src, nbytes, _sh(stream)))


def alloc_pinned_host(nbytes: int) -> int:
    p = C.c_void_p()
    check(_lib.load().tatara_host_alloc_pinned(nbytes, C.byref(p)))
    return p.value


def free_pinned_host(ptr: int) -> None:
    check(_lib.load().tatara_host_free_pinned(ptr))


class KernelArgs:
    """Kernel arguments in launch order; each value is kept alive here and
    passed by address (native_backend.rs:256-281)."""

    def __init__(self):
        self._values: list = []

    def push_scalar(self, value, ctype) -> "KernelArgs":
        self._values.append(ctype(value))
        return self

    def push_slice(self, ptr: int, length: int) -> "KernelArgs":
        """A device buffer: its pointer and its element count as u64."""
        self._values.append(C.c_void_p(ptr))
        self._values.append(C.c_uint64(length))
        return self

    def pointers(self):
        arr = (C.c_void_p * max(len(self._values), 1))()
        for i, v in enumerate(self._values):
            arr[i] = C.cast(C.byref(v), C.c_void_p)
        return arr


class Module:
    """A gfx950 code object (hipcc --genco) whose kernels launch by name
    (CudaContext::load_module_from_image, CudaModule::launch)."""

    def __init__(self, image: bytes, device: int = 0):
        h = C.c_void_p()
        buf = C.create_string_buffer(bytes(image), len(image))
        check(_lib.load().tatara_module_load_image(device, buf, len(image), C.byref(h)))
        self.handle = h.value
        self.device = device

    @classmethod
    def from_file(cls, path: str | Path, device: int = 0) -> "Module":
        return cls(Path(path).read_bytes(), device)

    def launch(self, kernel: str, stream: Stream | None, config: LaunchConfig, args: KernelArgs) -> None:
        grid = (C.c_uint32 * 3)(*config.grid_dim)
        block = (C.c_uint32 * 3)(*config.block_dim)
        ptrs = args.pointers()
        check(_lib.load().tatara_module_launch(self.handle, kernel.encode(), _sh(stream), grid, block,
                                               config.shared_mem_bytes, ptrs))

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            check(_lib.load().tatara_module_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
