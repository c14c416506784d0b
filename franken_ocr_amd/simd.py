"""The reference's ``simd`` kernel-tier surface, served by the gfx950 tier.

Mirrors ``src/simd/mod.rs:70-73`` (``igemm_s8s8``, ``igemm_u8s8``,
``caps``/``detected_tier``/``available_tiers``/``tier_string``/``selftest``)
and ``src/simd/int4.rs`` (``igemm_s4s8``, ``igemm_s4s8_packed``,
``unpack_to_i8``) with the same argument meaning: flat host arrays plus
``m, k, n``; ``out`` accumulated (``+=``) for int8, overwritten for int4.
A contract violation raises ``ContractViolation`` carrying the exact text
the reference panics with (``checked_len``/``assert_eq!`` messages).

Every call runs on the GPU through libfocr_hip.so; nothing here computes on
the CPU.
"""

from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass

import numpy as np

from . import _abi
from .device import Context, default_context


def _ptr(a: np.ndarray | None) -> C.c_void_p:
    # Empty slices carry no data; the ABI accepts NULL with a zero length.
    if a is None or a.size == 0:
        return C.c_void_p()
    return a.ctypes.data_as(C.c_void_p)


def _as(a, dtype) -> np.ndarray:
    arr = np.asarray(a)
    if arr.dtype != np.dtype(dtype):
        raise TypeError(f"expected {np.dtype(dtype)} array, got {arr.dtype}")
    if not arr.flags.c_contiguous:
        raise ValueError("arrays must be C-contiguous")
    return arr.reshape(-1)


def _out(a, dtype) -> np.ndarray:
    arr = _as(a, dtype)
    if not arr.flags.writeable:
        raise ValueError("out must be writeable")
    return arr


def igemm_s8s8(a, b, m: int, k: int, n: int, out, ctx: Context | None = None) -> None:
    """``C[M,N] += A[M,K] (i8) . B[N,K]^T (i8, output-channel-major)`` in i32
    (scalar.rs:78-116)."""
    ctx = ctx or default_context()
    a8, b8, o = _as(a, np.int8), _as(b, np.int8), _out(out, np.int32)
    _abi.call("focr_hip_igemm_s8s8", ctx.handle, _ptr(a8), a8.size, _ptr(b8), b8.size, m, k, n, _ptr(o), o.size)


def igemm_u8s8(a, b, m: int, k: int, n: int, out, ctx: Context | None = None) -> None:
    """``C[M,N] += A[M,K] (u8) . B[N,K]^T (i8)`` in i32 (scalar.rs:129-166)."""
    ctx = ctx or default_context()
    a8, b8, o = _as(a, np.uint8), _as(b, np.int8), _out(out, np.int32)
    _abi.call("focr_hip_igemm_u8s8", ctx.handle, _ptr(a8), a8.size, _ptr(b8), b8.size, m, k, n, _ptr(o), o.size)


def _s4(name, a, b_packed, scales, group, m, k, n, out, ctx):
    ctx = ctx or default_context()
    a8, b8 = _as(a, np.int8), _as(b_packed, np.uint8)
    s32, o = _as(scales, np.float32), _out(out, np.float32)
    _abi.call(name, ctx.handle, _ptr(a8), a8.size, _ptr(b8), b8.size, _ptr(s32), s32.size, group, m, k, n, _ptr(o), o.size)


def igemm_s4s8_packed(a, b_packed, scales, group: int, m: int, k: int, n: int, out, ctx: Context | None = None) -> None:
    """Native packed int4 x int8 GEMM (int4.rs:437-461): per-group i32 dots,
    f32 sum over groups in increasing order, ``out`` overwritten."""
    _s4("focr_hip_igemm_s4s8_packed", a, b_packed, scales, group, m, k, n, out, ctx)


def igemm_s4s8(a, b_packed, scales, group: int, m: int, k: int, n: int, out, ctx: Context | None = None) -> None:
    """int4.rs:170-229 entry (same result as the packed kernel)."""
    _s4("focr_hip_igemm_s4s8", a, b_packed, scales, group, m, k, n, out, ctx)


def unpack_to_i8(b_packed, n: int, k: int, ctx: Context | None = None) -> np.ndarray:
    """int4.rs:125-142: ``[n, k/2]`` packed -> ``[n, k]`` i8 in [-8, 7]."""
    ctx = ctx or default_context()
    b8 = _as(b_packed, np.uint8)
    # Only allocate for a shape the contract can accept; otherwise let the
    # library report the reference's panic text (odd k, n*k/2 overflow, ...).
    ok = k % 2 == 0 and n * (k // 2) == b8.size and n * k < 2**48
    out = np.zeros(n * k if ok else 0, dtype=np.int8)
    _abi.call("focr_hip_unpack_to_i8", ctx.handle, _ptr(b8), b8.size, n, k, _ptr(out), n * k if ok else 0)
    return out


def s4s8_group_i32(a, b_packed, group: int, m: int, k: int, n: int, ctx: Context | None = None) -> np.ndarray:
    """Per-group i32 partial sums ``[m][n][k/group]`` of the packed kernel."""
    ctx = ctx or default_context()
    a8, b8 = _as(a, np.int8), _as(b_packed, np.uint8)
    groups = k // group if group in (16, 32) and group else 0
    out = np.zeros(m * n * groups, dtype=np.int32)
    _abi.call("focr_hip_debug_s4s8_group_i32", ctx.handle, _ptr(a8), a8.size, _ptr(b8), b8.size, group, m, k, n,
              _ptr(out), out.size)
    return out


# ---- tier reflection (dispatch.rs:48-138) -------------------------------------

@dataclass(frozen=True)
class IsaTier:
    tag: str
    feature: str

    def feature_string(self) -> str:
        return self.feature


def _tier() -> IsaTier:
    t, f = C.create_string_buffer(64), C.create_string_buffer(64)
    _abi.call("focr_hip_tier", t, 64, f, 64)
    return IsaTier(t.value.decode(), f.value.decode())


GFX950 = None  # resolved lazily from the library


@dataclass
class Caps:
    selected: IsaTier
    available: list


def caps() -> Caps:
    t = _tier()
    return Caps(selected=t, available=[t])


def detected_tier() -> IsaTier:
    return caps().selected


def available_tiers() -> list:
    return caps().available


def tier_string() -> str:
    return detected_tier().feature_string()


@dataclass
class SelftestCase:
    kind: str
    label: str
    m: int
    k: int
    n: int
    ok: bool
    mismatches: int
    first_bad: tuple | None


@dataclass
class SelftestReport:
    selected: str
    available: list
    cases: list
    all_ok: bool
    raw: dict


def selftest(ctx: Context | None = None) -> SelftestReport:
    """dispatch.rs:376-429: the 24-case battery through the gfx950 tier."""
    ctx = ctx or default_context()
    buf = C.create_string_buffer(1 << 16)
    ok = C.c_int32(0)
    _abi.call("focr_hip_selftest", ctx.handle, buf, len(buf), C.byref(ok))
    raw = json.loads(buf.value.decode())
    cases = [
        SelftestCase(c["kind"], c["label"], c["m"], c["k"], c["n"], c["ok"], c["mismatches"],
                     tuple(c["first_bad"]) if "first_bad" in c else None)
        for c in raw["cases"]
    ]
    return SelftestReport(raw["selected"], raw["available"], cases, bool(ok.value), raw)
