"""Contexts and device arrays over the C ABI (no torch: one HIP runtime only).

A ``Context`` owns a HIP stream on one gfx950 device; ``DeviceArray`` is a
typed, shaped device allocation made through the library's own allocator,
with synchronous host<->device copies for tests and set-up code.
"""

from __future__ import annotations

import ctypes as C
import json
import threading

import numpy as np

from . import _abi


def device_count() -> int:
    n = C.c_int32(0)
    _abi.call("focr_hip_device_count", C.byref(n))
    return int(n.value)


class Context:
    """A focr_hip_ctx: one device, one default-priority stream, scratch."""

    def __init__(self, device: int = 0):
        self._h = C.c_void_p()
        _abi.call("focr_hip_ctx_create", int(device), C.byref(self._h))
        self.device = device

    @property
    def handle(self) -> C.c_void_p:
        if not self._h:
            raise _abi.FocrHipError(_abi.E_BAD_HANDLE, "context destroyed")
        return self._h

    def close(self) -> None:
        if self._h:
            _abi.lib().focr_hip_ctx_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self) -> None:
        _abi.call("focr_hip_ctx_synchronize", self.handle)

    def device_synchronize(self) -> None:
        _abi.call("focr_hip_device_synchronize", self.handle)

    def stream(self) -> int:
        s = C.c_void_p()
        _abi.call("focr_hip_ctx_stream", self.handle, C.byref(s))
        return int(s.value or 0)

    def scratch_bytes(self) -> int:
        """Bytes the context's grow-only scratch slots hold (a diagnostic)."""
        n = C.c_size_t()
        _abi.call("focr_hip_ctx_scratch_bytes", self.handle, C.byref(n))
        return int(n.value)

    def set_route_wait(self, ticks: int) -> None:
        """Bound of the MoE route's cross-block wait (10 ns ticks; a test hook:
        0 makes every token's lead block compute all of its logits)."""
        _abi.call("focr_hip_ctx_set_route_wait", self.handle, int(ticks))

    def info(self) -> dict:
        arch = C.create_string_buffer(64)
        cus = C.c_int32(0)
        _abi.call("focr_hip_ctx_device_info", self.handle, arch, 64, C.byref(cus))
        return {"arch": arch.value.decode(), "cu_count": int(cus.value)}

    # -- profiling (GPU-timed per-kernel totals) --
    def prof_enable(self, on: bool = True) -> None:
        _abi.call("focr_hip_prof_enable", self.handle, 1 if on else 0)

    def prof_reset(self) -> None:
        _abi.call("focr_hip_prof_reset", self.handle)

    def prof_read(self) -> dict:
        buf = C.create_string_buffer(1 << 16)
        _abi.call("focr_hip_prof_read", self.handle, buf, len(buf))
        return json.loads(buf.value.decode())

    def mark(self) -> None:
        """Record a step mark (an event) on the context's stream."""
        _abi.call("focr_hip_mark", self.handle)

    def marks_read(self, cap: int = 1 << 16) -> list[float]:
        """Synchronise and return the ms between consecutive marks (and drop them)."""
        out = np.zeros(cap, np.float32)
        n = C.c_size_t()
        _abi.call("focr_hip_marks_read", self.handle, out.ctypes.data_as(C.c_void_p), cap, C.byref(n))
        return [float(v) for v in out[: n.value]]

    # -- allocation --
    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def to_device(self, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = DeviceArray(self, arr.shape, arr.dtype)
        d.copy_from(arr)
        return d


_default: dict[int, Context] = {}
_default_lock = threading.Lock()


def default_context(device: int = 0) -> Context:
    """A process-wide context per device (created on first use)."""
    with _default_lock:
        ctx = _default.get(device)
        if ctx is None:
            ctx = Context(device)
            _default[device] = ctx
        return ctx


class DeviceArray:
    """A contiguous device allocation with a numpy dtype and shape."""

    def __init__(self, ctx: Context, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._p = C.c_void_p()
        _abi.call("focr_hip_dmalloc", ctx.handle, max(self.nbytes, 16), C.byref(self._p))

    @classmethod
    def adopt(cls, ctx: Context, ptr: C.c_void_p, shape, dtype) -> "DeviceArray":
        """Take ownership of a device allocation made by the library (freed
        with focr_hip_dfree like any other DeviceArray)."""
        a = cls.__new__(cls)
        a.ctx = ctx
        a.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        a.dtype = np.dtype(dtype)
        a.nbytes = int(np.prod(a.shape, dtype=np.int64)) * a.dtype.itemsize
        a._p = ptr
        return a

    @property
    def ptr(self) -> int:
        return int(self._p.value or 0)

    @property
    def c_ptr(self) -> C.c_void_p:
        return self._p

    def __del__(self):  # pragma: no cover
        try:
            if self._p and self.ctx._h:
                self.free()
        except Exception:
            pass

    def copy_from(self, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: host {arr.nbytes} B vs device {self.nbytes} B")
        _abi.call("focr_hip_h2d", self.ctx.handle, self._p, arr.ctypes.data_as(C.c_void_p), self.nbytes)
        return self

    def copy_from_device(self, other: "DeviceArray") -> "DeviceArray":
        if other.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        _abi.call("focr_hip_d2d", self.ctx.handle, self._p, other._p, self.nbytes)
        return self

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _abi.call("focr_hip_d2h", self.ctx.handle, out.ctypes.data_as(C.c_void_p), self._p, self.nbytes)
        return out

    def view_rows(self, r0: int, r1: int) -> "DeviceArray":
        """Rows [r0, r1) of a 2-D array as a DeviceArray that borrows this
        allocation (it frees nothing; keep the parent alive while using it)."""
        if len(self.shape) != 2 or not 0 <= r0 <= r1 <= self.shape[0]:
            raise ValueError("row view out of range")
        row = self.shape[1] * self.dtype.itemsize
        v = DeviceArray.__new__(DeviceArray)
        v.ctx, v.shape, v.dtype = self.ctx, (r1 - r0, self.shape[1]), self.dtype
        v.nbytes = (r1 - r0) * row
        v._p = C.c_void_p(self.ptr + r0 * row)
        v._borrowed = self
        return v

    def free(self) -> None:
        if self._p and not getattr(self, "_borrowed", None):
            _abi.lib().focr_hip_dfree(self.ctx.handle, self._p)
        self._p = C.c_void_p()

    def offset(self, nbytes: int) -> C.c_void_p:
        """A raw pointer nbytes into this allocation (for sub-views)."""
        if nbytes < 0 or nbytes > self.nbytes:
            raise ValueError("offset out of range")
        return C.c_void_p(self.ptr + nbytes)
