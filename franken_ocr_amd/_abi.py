"""ctypes binding of include/focr_hip.h (libfocr_hip.so, built in-tree).

The library is loaded lazily on first use. There is no CPU fallback: if the
shared library is missing or fails to load, every entry point raises
ExtensionMissing — build it with ``python -m franken_ocr_amd.build``.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import os

# FOCR_HIP_LIB selects another build of the same library (the host-sanitized
# copy that franken_ocr_amd/sanitize.py runs the CPU checks against).
LIB_PATH = Path(os.environ.get("FOCR_HIP_LIB") or Path(__file__).resolve().parent / "libfocr_hip.so")

OK = 0
E_SHAPE = -1
E_HIP = -2
E_OOM = -3
E_NO_DEVICE = -4
E_BAD_HANDLE = -5
E_ARG = -6
E_ROUTE = -7
E_STATE = -8
E_FORMAT = -9
E_NOT_FOUND = -10
E_NOT_IMPLEMENTED = -11

DT_F32, DT_F16, DT_BF16, DT_QINT8_PER_CHAN, DT_QINT4_PER_GROUP = range(5)

_P = C.c_void_p
_SZ = C.c_size_t
_I32 = C.c_int32
_F32 = C.c_float

# name -> argtypes (all return int32 status unless listed in _RESTYPE)
_SIGS: dict[str, list] = {
    "focr_hip_last_error": [],
    "focr_hip_version": [],
    "focr_hip_device_count": [_P],
    "focr_hip_ctx_create": [_I32, _P],
    "focr_hip_ctx_destroy": [_P],
    "focr_hip_ctx_synchronize": [_P],
    "focr_hip_device_synchronize": [_P],
    "focr_hip_ctx_stream": [_P, _P],
    "focr_hip_ctx_device_info": [_P, C.c_char_p, _SZ, _P],
    "focr_hip_tier": [C.c_char_p, _SZ, C.c_char_p, _SZ],
    "focr_hip_dmalloc": [_P, _SZ, _P],
    "focr_hip_dfree": [_P, _P],
    "focr_hip_h2d": [_P, _P, _P, _SZ],
    "focr_hip_d2h": [_P, _P, _P, _SZ],
    "focr_hip_d2d": [_P, _P, _P, _SZ],
    "focr_hip_igemm_s8s8": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_igemm_u8s8": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_igemm_s4s8_packed": [_P, _P, _SZ, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_igemm_s4s8": [_P, _P, _SZ, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_unpack_to_i8": [_P, _P, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_debug_s4s8_group_i32": [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _SZ],
    "focr_hip_selftest": [_P, C.c_char_p, _SZ, _P],
    "focr_hip_igemm_s8s8_dev": [_P, _P, _P, _SZ, _SZ, _SZ, _P],
    "focr_hip_igemm_s8s8_batched_dev": [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P],
    "focr_hip_igemm_u8s8_dev": [_P, _P, _P, _SZ, _SZ, _SZ, _P],
    "focr_hip_igemm_s4s8_packed_dev": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P],
    "focr_hip_qint8_upload": [_P, _P, _P, _SZ, _SZ, _P],
    "focr_hip_qint8_from_device": [_P, _P, _P, _SZ, _SZ, _P],
    "focr_hip_qint8_free": [_P],
    "focr_hip_quantize_rows_i8": [_P, _P, _SZ, _SZ, _P, _P, _I32],
    "focr_hip_gemv_i8": [_P, _P, _P, _SZ, _P],
    "focr_hip_gemv_i8_prequant": [_P, _P, _P, _P, _SZ, _P, _P],
    "focr_hip_lm_head_i8": [_P, _P, _P, _SZ, _P, _P],
    "focr_hip_argmax_rows": [_P, _P, _SZ, _SZ, _P],
    "focr_hip_lm_head_sample_i8": [_P, _P, _P, _SZ, _P, _SZ, _P, _SZ, _SZ, _P, _SZ, _F32, C.c_uint32, _I32, _P,
                                   _P, _P, _I32],
    "focr_hip_sample_rows": [_P, _P, _SZ, _SZ, _P, _SZ, _P, _SZ, _SZ, _P, _SZ, _F32, C.c_uint32, _I32, _P, _P,
                             _I32],
    "focr_hip_moe_layer_create": [_P, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _I32, _P],
    "focr_hip_moe_layer_set_shared": [_P, _SZ, _P, _P, _P, _P, _P, _P, _I32],
    "focr_hip_moe_layer_free": [_P],
    "focr_hip_moe_decode": [_P, _P, _P, _SZ, _I32, _F32, _I32, _P, _P, _P, _I32],
    "focr_hip_moe_decode_noalloc": [_P, _P, _P, _SZ, _I32, _F32, _I32, _P, _P, _P, _I32],
    "focr_hip_static_scratch_bytes": [],
    "focr_hip_chunk_prefill_attention": [_P, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _P],
    "focr_hip_prefill_attention": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _P],
    "focr_hip_rswa_prefill_chunk": [_P, _P, _SZ, _P, _P, _P, _SZ, _SZ, _P],
    "focr_hip_moe_route": [_P, _P, _P, _SZ, _I32, _F32, _P, _P, _P],
    "focr_hip_moe_layer_i4_create": [_P, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _I32, _P],
    "focr_hip_moe_layer_i4_free": [_P],
    "focr_hip_moe_prefill_i4": [_P, _P, _P, _SZ, _SZ, _P, _P, _P, _I32],
    "focr_hip_linear_i8_dynamic": [_P, _P, _P, _SZ, _P, _P],
    "focr_hip_moe_prefill_i8": [_P, _P, _P, _SZ, _P, _P, _I32, _P, _I32],
    "focr_hip_rms_norm": [_P, _P, _SZ, _SZ, _P, _F32, _P],
    "focr_hip_decoder_layer_create": [_P, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _F32, _P],
    "focr_hip_decoder_layer_free": [_P],
    "focr_hip_decoder_layer_prefill": [_P, _P, _P, _SZ, _P, _SZ, _SZ, _P, _I32],
    "focr_hip_decoder_layer_step": [_P, _P, _P, _P, _P, _P, _I32],
    "focr_hip_decoder_create": [_P, _SZ, _P, _P, _F32, _P, _P],
    "focr_hip_decoder_free": [_P],
    "focr_hip_decoder_step": [_P, _P, _P, _P, _P, _P, _P, _P, _I32],
    "focr_hip_decoder_step_sample": [_P, _P, _P, _P, _P, _P, _SZ, _P, _SZ, _SZ, _P, _SZ, _F32, C.c_uint32, _I32,
                                     _P, _P, _P, _P, _I32],
    "focr_hip_decoder_prefill": [_P, _P, _P, _SZ, _P, _SZ, _SZ, _P, _P, _P, _I32],
    "focr_hip_rswa_create": [_P, _SZ, _SZ, _P],
    "focr_hip_rswa_free": [_P],
    "focr_hip_rswa_record_prefill": [_P, _P, _SZ, _P, _P, _SZ],
    "focr_hip_rswa_write_decode_step": [_P, _P, _P, _P, _P],
    "focr_hip_rswa_decode_attention": [_P, _P, _P, _P],
    "focr_hip_rswa_step": [_P, _P, _P, _P, _P, _P],
    "focr_hip_rswa_get_state": [_P, _SZ, _P, _P, _P],
    "focr_hip_rswa_set_state": [_P, _SZ, C.c_uint32, C.c_uint32],
    "focr_hip_rswa_regions": [_P, _SZ, _P, _P, _P, _P],
    "focr_hip_focrq_open": [C.c_char_p, _P],
    "focr_hip_focrq_from_bytes": [_P, _SZ, _P],
    "focr_hip_focrq_close": [_P],
    "focr_hip_focrq_info": [_P, _P, _P, _P, C.c_char_p, _SZ, C.c_char_p, _SZ, C.c_char_p, _SZ],
    "focr_hip_focrq_name": [_P, _SZ, C.c_char_p, _SZ],
    "focr_hip_focrq_record": [_P, C.c_char_p, _P, _P, _SZ, _P, _P, _P, _P, _P, _P, _P],
    "focr_hip_focrq_census": [_P, _P, _SZ],
    "focr_hip_focrq_read_f32": [_P, C.c_char_p, _P, _SZ, _P, _P],
    "focr_hip_focrq_read_qint8": [_P, C.c_char_p, _P, _SZ, _P, _SZ, _P, _P],
    "focr_hip_focrq_read_qint4": [_P, C.c_char_p, _P, _SZ, _P, _SZ, _P, _P, _P, _P],
    "focr_hip_focrq_upload_qint8": [_P, _P, C.c_char_p, C.c_uint64, _P],
    "focr_hip_focrq_upload_f32": [_P, _P, C.c_char_p, _P, _P, _P],
    "focr_hip_focrq_moe_layer": [_P, _P, _SZ, _SZ, _SZ, _I32, _P],
    "focr_hip_focrq_moe_layer_i4": [_P, _P, _SZ, _SZ, _P],
    "focr_hip_quantize_weight_i8": [_P, _P, _I32, _SZ, _SZ, _P, _P],
    "focr_hip_pack_weight_i4": [_P, _P, _I32, _SZ, _SZ, _SZ, _P, _P],
    "focr_hip_focrq_writer_new": [_P],
    "focr_hip_focrq_writer_free": [_P],
    "focr_hip_focrq_writer_set_meta": [_P, C.c_uint8, _P, C.c_char_p, C.c_char_p, _I32],
    "focr_hip_focrq_writer_set_json": [_P, C.c_char_p, C.c_char_p],
    "focr_hip_focrq_writer_add_tensor": [_P, C.c_char_p, _I32, _P, _SZ, _P, _SZ],
    "focr_hip_focrq_writer_add_quantized": [_P, C.c_char_p, _I32, _P, _SZ, _P, _SZ, _P, _SZ, C.c_uint64,
                                            C.c_uint8],
    "focr_hip_focrq_writer_build": [_P, _P, _SZ, _P],
    "focr_hip_focrq_writer_write": [_P, C.c_char_p],
    "focr_hip_ctx_scratch_bytes": [_P, _P],
    "focr_hip_ctx_set_route_wait": [_P, C.c_uint32],
    "focr_hip_prof_enable": [_P, _I32],
    "focr_hip_prof_reset": [_P],
    "focr_hip_prof_read": [_P, C.c_char_p, _SZ],
    "focr_hip_mark": [_P],
    "focr_hip_marks_read": [_P, _P, _SZ, _P],
}

_RESTYPE = {"focr_hip_last_error": C.c_char_p, "focr_hip_version": C.c_char_p,
            "focr_hip_static_scratch_bytes": C.c_size_t}


class ExtensionMissing(RuntimeError):
    """libfocr_hip.so is not built or cannot be loaded (no CPU fallback exists)."""


class FocrHipError(RuntimeError):
    """A non-OK status from the C ABI; ``.status`` holds the code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class ContractViolation(FocrHipError, ValueError):
    """FOCR_HIP_E_SHAPE: the reference would have panicked with this message."""


class RouteError(FocrHipError):
    """FOCR_HIP_E_ROUTE: moe.rs "no finite router score"."""


class StateError(FocrHipError):
    """FOCR_HIP_E_STATE: ring-cache state errors (rswa.rs)."""


class NoDevice(FocrHipError):
    """FOCR_HIP_E_NO_DEVICE: no gfx950 device visible."""


class FormatMismatch(FocrHipError, ValueError):
    """FOCR_HIP_E_FORMAT: FocrError::FormatMismatch of the weight container."""


class ModelNotFound(FocrHipError):
    """FOCR_HIP_E_NOT_FOUND: FocrError::ModelNotFound (weights file unreadable)."""


class NotImplementedPath(FocrHipError, NotImplementedError):
    """FOCR_HIP_E_NOT_IMPLEMENTED: FocrError::NotImplemented (temperature > 0 sampling)."""


_lock = threading.Lock()
_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load libfocr_hip.so (once) and bind the declared signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ExtensionMissing(
                f"{LIB_PATH} is not built; run `python -m franken_ocr_amd.build` (hipcc, gfx950)"
            )
        try:
            h = C.CDLL(str(LIB_PATH))
        except OSError as e:  # pragma: no cover - depends on the host runtime
            raise ExtensionMissing(f"cannot load {LIB_PATH}: {e}") from e
        for name, args in _SIGS.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, C.c_int32)
        _lib = h
        return h


def exported_symbols() -> list[str]:
    return list(_SIGS)


def last_error() -> str:
    msg = lib().focr_hip_last_error()
    return msg.decode() if msg else ""


_ERR = {E_SHAPE: ContractViolation, E_ROUTE: RouteError, E_STATE: StateError, E_NO_DEVICE: NoDevice,
        E_FORMAT: FormatMismatch, E_NOT_FOUND: ModelNotFound, E_NOT_IMPLEMENTED: NotImplementedPath}


def check(status: int) -> None:
    """Raise the typed error for a non-OK status (message = the library's)."""
    if status != OK:
        cls = _ERR.get(status, FocrHipError)
        raise cls(status, last_error() or f"focr_hip status {status}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
