"""Device runtime objects: HIP context, device buffers, the buffer pool and the
command stream, over the C ABI of ``libwxx_hip.so``.

Mirrors the interface of the reference's WebGPU runtime
(reference src/wxx/backend/device.py:9-273: ``WebGPUContext``,
``GPUBufferPool``, ``GPUCommandBuffer`` and the ``get_*`` singletons) so the
Tensor/functional layers keep their shape, but the mechanics are HIP's:

* device memory comes from the library's caching allocator (exact-size
  buckets, no 4 MiB cap) and returns to it when a :class:`DeviceBuffer` is
  garbage collected;
* all work is enqueued on the library's single in-order stream, so there is
  no command encoder to flush: ``flush(wait=True)`` synchronises the stream
  and ``defer_destroy`` may release at once (stream order protects the
  pending kernels);
* the device is opened lazily on first use, so importing the package works
  on a machine without a GPU (host-only logic and tests).
"""

import ctypes as C
import os
import sys
import weakref

import numpy as np

from . import lib as _lib

_state = {"init": False}


def ensure_device():
    """Initialise the HIP runtime on ``$WXX_DEVICE`` (default 0) once."""
    if not _state["init"]:
        dev = int(os.environ.get("WXX_DEVICE", "0"))
        _lib.call("wxx_init", dev)
        _state["init"] = True
    return _lib.load()


def device_available():
    """True when the library loads and at least one HIP device is visible."""
    try:
        lib = _lib.load()
    except (OSError, RuntimeError):
        return False
    n = C.c_int(0)
    return lib.wxx_device_count(C.byref(n)) == 0 and n.value > 0


class DeviceBuffer:
    """An allocation in device memory.  ``size`` is in bytes."""

    __slots__ = ("ptr", "size", "label", "__weakref__")

    def __init__(self, ptr, size, label=None):
        self.ptr = ptr
        self.size = size
        self.label = label

    def destroy(self):
        ptr, self.ptr = self.ptr, None
        if ptr:
            try:
                _lib.load().wxx_free(ptr)
            except Exception:  # interpreter shutdown
                pass

    def __del__(self):
        self.destroy()

    def __repr__(self):
        return f"DeviceBuffer(ptr=0x{self.ptr or 0:x}, size={self.size}, label={self.label!r})"


class HIPContext:
    """The opened device (counterpart of the reference's ``WebGPUContext``)."""

    def __init__(self):
        self._info = None

    @property
    def info(self):
        if self._info is None:
            lib = ensure_device()
            cus = C.c_int(0)
            name = C.create_string_buffer(256)
            mem = C.c_size_t(0)
            _lib.call("wxx_device_info", C.byref(cus), name, 256, C.byref(mem))
            self._info = {
                "compute_units": cus.value,
                "name": name.value.decode(errors="replace"),
                "total_memory": mem.value,
            }
            del lib
        return self._info


class DeviceBufferPool:
    """Allocation front end (counterpart of the reference's ``GPUBufferPool``)."""

    def __init__(self):
        self._active = {}

    def create_buffer(self, size, usage=None, label=None):
        lib = ensure_device()
        size = max(4, (int(size) + 3) & ~3)
        ptr = lib.wxx_alloc(size)
        if not ptr:
            raise MemoryError(f"device allocation of {size} bytes failed: {_lib.last_error()}")
        if label is None:
            label = sys._getframe(1).f_code.co_name
        buf = DeviceBuffer(ptr, size, label)
        self._active[id(buf)] = (weakref.ref(buf), size, label)
        return buf

    def create_buffer_with_data(self, data, usage=None, label=None):
        if isinstance(data, np.ndarray):
            arr = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
        else:
            arr = np.frombuffer(memoryview(data).tobytes() if not isinstance(data, bytes) else data,
                                dtype=np.uint8)
        nbytes = int(arr.nbytes)
        if nbytes % 4:
            raise ValueError("device buffer data size must be a multiple of 4 bytes")
        caller = sys._getframe(1).f_code.co_name
        label = caller if label is None else f"{caller}: {label}"
        buf = self.create_buffer(nbytes, usage, label=label)
        if nbytes:
            _lib.call("wxx_h2d", C.c_void_p(buf.ptr), arr.ctypes.data_as(C.c_void_p), nbytes)
        return buf

    def release(self, buffer):
        self._active.pop(id(buffer), None)
        buffer.destroy()

    def get_memory_snapshot(self):
        active = []
        for key, (ref, size, label) in list(self._active.items()):
            if ref() is None or ref().ptr is None:
                del self._active[key]
            else:
                active.append({"label": label, "size": size})
        live = C.c_size_t(0)
        cached = C.c_size_t(0)
        peak = C.c_size_t(0)
        nmal = C.c_size_t(0)
        if _state["init"]:
            _lib.load().wxx_mem_stats(C.byref(live), C.byref(cached), C.byref(peak), C.byref(nmal))
        return {
            "active": active,
            "cached": [],
            "active_bytes": sum(a["size"] for a in active),
            "cached_bytes": cached.value,
            "device_live_bytes": live.value,
            "device_peak_bytes": peak.value,
            "device_mallocs": nmal.value,
        }

    def clear_cache(self):
        if _state["init"]:
            _lib.call("wxx_empty_cache")


class CommandStream:
    """Counterpart of the reference's ``GPUCommandBuffer`` over one HIP stream."""

    def flush(self, wait=False):
        if wait and _state["init"]:
            _lib.call("wxx_sync")

    def keep_alive(self, buf):
        """No-op: kernel arguments are passed by value, nothing must outlive a launch."""

    def defer_destroy(self, buf):
        buf.destroy()

    def complete_pending(self):
        """No-op: frees are stream ordered."""

    def sync(self):
        if _state["init"]:
            _lib.call("wxx_sync")


gpu_ctx = HIPContext()
buffer_pool = DeviceBufferPool()
cmd_buf = CommandStream()


def get_device():
    return gpu_ctx


def get_ctx():
    return gpu_ctx


def get_cmd_buffer():
    return cmd_buf


def get_buffer_pool():
    return buffer_pool


def synchronize():
    cmd_buf.sync()


__all__ = [
    "DeviceBuffer",
    "HIPContext",
    "DeviceBufferPool",
    "CommandStream",
    "ensure_device",
    "device_available",
    "get_device",
    "get_ctx",
    "get_cmd_buffer",
    "get_buffer_pool",
    "synchronize",
]
