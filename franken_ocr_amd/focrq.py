"""The weight container (.focrq / safetensors) through the C ABI.

``Weights`` mirrors src/native_engine/weights.rs ``Weights`` (load /
from_bytes, names, record, census, mat / vec, qint8 / qint4 and the
provenance getters) and adds the upload-once path into HBM
(``DecoderWeightCacheI8::build``, decoder.rs:2018-2116): ``upload_qint8``
(quant_oc_loaded, decoder.rs:1777-1786), ``upload_f32``, ``moe_layer`` and
``moe_layer_i4``. ``FocrqBuilder`` mirrors src/quant/focrq.rs
``FocrqBuilder``. Errors are ``_abi.FormatMismatch`` / ``_abi.ModelNotFound``
carrying the reference's messages.

``quantize_weight_i8`` / ``pack_weight_i4`` are the converter-side weight
quantizers (quant/int8.rs:145-163, quant/int4.rs:142-205) run on the device.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _abi
from .device import Context, DeviceArray, default_context

F32, F16, BF16, QINT8_PER_CHAN, QINT4_PER_GROUP = "F32", "F16", "BF16", "QInt8PerChan", "QInt4PerGroup"
DTYPES = (F32, F16, BF16, QINT8_PER_CHAN, QINT4_PER_GROUP)
_CODE = {name: i for i, name in enumerate(DTYPES)}
DEFAULT_LICENSE_NOTICE = "Baidu Unlimited-OCR - Copyright (c) 2026 Baidu, MIT License"


@dataclass(frozen=True)
class TensorRecord:
    """weights.rs:196-230 TensorRecord."""

    dtype: str
    shape: tuple
    byte_offset: int
    byte_len: int
    scales_offset: int
    scales_len: int
    group_size: int
    tier: int


@dataclass
class QInt8Host:
    """tensor.rs:149-179 QInt8 on the host."""

    w: np.ndarray
    scales: np.ndarray
    n: int
    k: int


@dataclass
class QInt4Host:
    """tensor.rs:190-204 QInt4 on the host."""

    packed: np.ndarray
    scales: np.ndarray
    n: int
    k: int
    group_size: int
    tier: int


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


class Weights:
    """A parsed weight container (the C++ reader; a path is memory-mapped)."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle

    @classmethod
    def load(cls, path) -> "Weights":
        h = C.c_void_p()
        _abi.call("focr_hip_focrq_open", str(path).encode(), C.byref(h))
        return cls(h)

    @classmethod
    def from_bytes(cls, blob: bytes) -> "Weights":
        buf = np.frombuffer(bytes(blob), dtype=np.uint8)
        h = C.c_void_p()
        _abi.call("focr_hip_focrq_from_bytes", _ptr(buf) if buf.size else C.c_void_p(), buf.size, C.byref(h))
        return cls(h)

    @classmethod
    def load_with_census(cls, path, expected_names) -> "Weights":
        w = cls.load(path)
        w.census(expected_names)
        return w

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            _abi.lib().focr_hip_focrq_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- provenance (weights.rs:687-717) ----
    def _info(self) -> dict:
        is_fq, arch, n = C.c_int32(), C.c_uint8(), C.c_size_t()
        sha, mid = C.create_string_buffer(128), C.create_string_buffer(64)
        lic = C.create_string_buffer(4096)
        _abi.call("focr_hip_focrq_info", self._h, C.byref(is_fq), C.byref(arch), C.byref(n), sha, len(sha), mid,
                  len(mid), lic, len(lic))
        return {"is_focrq": bool(is_fq.value), "arch_target": arch.value, "len": n.value,
                "source_sha256": sha.value.decode(), "model_id": mid.value.decode(),
                "license_notice": lic.value.decode()}

    def is_focrq(self) -> bool:
        return self._info()["is_focrq"]

    def arch_target(self) -> int:
        return self._info()["arch_target"]

    def source_sha256(self) -> str:
        return self._info()["source_sha256"]

    def license_notice(self) -> str:
        return self._info()["license_notice"]

    def model_id(self) -> str:
        return self._info()["model_id"]

    def __len__(self) -> int:
        return self._info()["len"]

    def is_empty(self) -> bool:
        return len(self) == 0

    def names(self) -> list[str]:
        out = []
        buf = C.create_string_buffer(4096)
        for i in range(len(self)):
            _abi.call("focr_hip_focrq_name", self._h, i, buf, len(buf))
            out.append(buf.value.decode())
        return out

    def contains(self, name: str) -> bool:
        return self.record(name) is not None

    def record(self, name: str) -> TensorRecord | None:
        dt, rank = C.c_int32(), C.c_size_t()
        shape = (C.c_uint64 * 16)()
        vals = [C.c_uint64() for _ in range(5)]
        tier = C.c_uint8()
        st = _abi.lib().focr_hip_focrq_record(self._h, name.encode(), C.byref(dt), shape, 16, C.byref(rank),
                                              *[C.byref(v) for v in vals], C.byref(tier))
        if st == _abi.E_FORMAT:
            return None
        _abi.check(st)
        return TensorRecord(DTYPES[dt.value], tuple(shape[i] for i in range(rank.value)), vals[0].value,
                            vals[1].value, vals[2].value, vals[3].value, vals[4].value, tier.value)

    def census(self, expected_names) -> None:
        names = [n.encode() for n in expected_names]
        arr = (C.c_char_p * max(len(names), 1))(*names)
        _abi.call("focr_hip_focrq_census", self._h, arr, len(names))

    # ---- host accessors (weights.rs:776-923) ----
    def mat(self, name: str) -> np.ndarray:
        rows, cols = C.c_uint64(), C.c_uint64()
        _abi.call("focr_hip_focrq_read_f32", self._h, name.encode(), None, 0, C.byref(rows), C.byref(cols))
        out = np.empty((rows.value, cols.value), dtype=np.float32)
        _abi.call("focr_hip_focrq_read_f32", self._h, name.encode(), _ptr(out), out.size, None, None)
        return out

    def vec(self, name: str) -> np.ndarray:
        return self.mat(name).reshape(-1)

    def qint8(self, name: str) -> QInt8Host:
        n, k = C.c_uint64(), C.c_uint64()
        _abi.call("focr_hip_focrq_read_qint8", self._h, name.encode(), None, 0, None, 0, C.byref(n), C.byref(k))
        w = np.empty((n.value, k.value), dtype=np.int8)
        s = np.empty(n.value, dtype=np.float32)
        _abi.call("focr_hip_focrq_read_qint8", self._h, name.encode(), _ptr(w), w.size, _ptr(s), s.size, None, None)
        return QInt8Host(w, s, n.value, k.value)

    def qint4(self, name: str) -> QInt4Host:
        n, k, g, tier = C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint8()
        _abi.call("focr_hip_focrq_read_qint4", self._h, name.encode(), None, 0, None, 0, C.byref(n), C.byref(k),
                  C.byref(g), C.byref(tier))
        packed = np.empty((n.value, k.value // 2), dtype=np.uint8)
        s = np.empty((n.value, k.value // g.value), dtype=np.float32)
        _abi.call("focr_hip_focrq_read_qint4", self._h, name.encode(), _ptr(packed), packed.size, _ptr(s), s.size,
                  None, None, None, None)
        return QInt4Host(packed, s, n.value, k.value, g.value, tier.value)

    # ---- upload once into HBM ----
    def upload_qint8(self, name: str, out_channels: int = 0, ctx: Context | None = None):
        """quant_oc_loaded (decoder.rs:1777-1786) into an engine QInt8."""
        from .engine import QInt8

        ctx = ctx or default_context()
        h = C.c_void_p()
        _abi.call("focr_hip_focrq_upload_qint8", ctx.handle, self._h, name.encode(), int(out_channels), C.byref(h))
        q = QInt8.__new__(QInt8)
        q.ctx = ctx
        q._h = h
        rec = self.record(name)
        if rec.dtype == QINT8_PER_CHAN:
            q.n, q.k = rec.shape
        else:
            numel = int(np.prod(rec.shape, dtype=np.int64))
            q.n = int(out_channels) if out_channels else (rec.shape[0] if len(rec.shape) == 2 else 1)
            q.k = numel // q.n
        return q

    def upload_f32(self, name: str, ctx: Context | None = None) -> DeviceArray:
        """mat() widened on the device: a DeviceArray [rows, cols] f32."""
        ctx = ctx or default_context()
        p = C.c_void_p()
        rows, cols = C.c_uint64(), C.c_uint64()
        _abi.call("focr_hip_focrq_upload_f32", ctx.handle, self._h, name.encode(), C.byref(p), C.byref(rows),
                  C.byref(cols))
        return DeviceArray.adopt(ctx, p, (rows.value, cols.value), np.float32)

    def moe_layer(self, layer: int, n_experts: int, top_k: int, with_shared: bool = False,
                  ctx: Context | None = None):
        """The MoE MLP of model.layers.{layer} as an engine MoeLayer."""
        from .engine import MoeLayer

        ctx = ctx or default_context()
        h = C.c_void_p()
        _abi.call("focr_hip_focrq_moe_layer", ctx.handle, self._h, int(layer), int(n_experts), int(top_k),
                  1 if with_shared else 0, C.byref(h))
        router = self.record(f"model.layers.{layer}.mlp.gate.weight")
        gate0 = self.record(f"model.layers.{layer}.mlp.experts.0.gate_proj.weight")
        hidden = router.shape[-1]
        inter = gate0.shape[0] if len(gate0.shape) == 2 else int(np.prod(gate0.shape)) // hidden
        return MoeLayer.adopt(ctx, h, hidden, inter, n_experts, top_k)

    def moe_layer_i4(self, layer: int, n_experts: int, ctx: Context | None = None):
        """The QInt4PerGroup experts of model.layers.{layer} as an engine MoeLayerI4."""
        from .engine import MoeLayerI4

        ctx = ctx or default_context()
        h = C.c_void_p()
        _abi.call("focr_hip_focrq_moe_layer_i4", ctx.handle, self._h, int(layer), int(n_experts), C.byref(h))
        gate0 = self.record(f"model.layers.{layer}.mlp.experts.0.gate_proj.weight")
        inter, hidden = gate0.shape
        return MoeLayerI4.adopt(ctx, h, hidden, inter, n_experts, gate0.group_size)


class FocrqBuilder:
    """src/quant/focrq.rs FocrqBuilder (the C++ writer)."""

    def __init__(self):
        self._h = C.c_void_p()
        _abi.call("focr_hip_focrq_writer_new", C.byref(self._h))
        self._arch, self._sha, self._notice, self._model_id, self._align = 0, bytes(32), None, None, False

    def _meta(self) -> "FocrqBuilder":
        sha = (C.c_uint8 * 32).from_buffer_copy(self._sha)
        _abi.call("focr_hip_focrq_writer_set_meta", self._h, self._arch, sha,
                  None if self._notice is None else self._notice.encode(),
                  None if self._model_id is None else self._model_id.encode(), 1 if self._align else 0)
        return self

    def with_arch_target(self, arch: int) -> "FocrqBuilder":
        self._arch = int(arch)
        return self._meta()

    def with_source_sha256(self, sha: bytes) -> "FocrqBuilder":
        if len(sha) != 32:
            raise ValueError("source_sha256 must be 32 bytes")
        self._sha = bytes(sha)
        return self._meta()

    def with_license_notice(self, notice: str) -> "FocrqBuilder":
        self._notice = notice
        return self._meta()

    def with_model_id(self, model_id: str) -> "FocrqBuilder":
        self._model_id = model_id
        return self._meta()

    def with_alignment(self, on: bool) -> "FocrqBuilder":
        self._align = bool(on)
        return self._meta()

    def with_provenance_json(self, text: str) -> "FocrqBuilder":
        _abi.call("focr_hip_focrq_writer_set_json", self._h, b"provenance", text.encode())
        return self

    def with_model_config_json(self, text: str) -> "FocrqBuilder":
        _abi.call("focr_hip_focrq_writer_set_json", self._h, b"model_config", text.encode())
        return self

    def with_packing_manifest_json(self, text: str) -> "FocrqBuilder":
        _abi.call("focr_hip_focrq_writer_set_json", self._h, b"packing_manifest", text.encode())
        return self

    def add_tensor(self, name: str, dtype: str, shape, data: bytes) -> None:
        sh = np.asarray(shape, dtype=np.uint64).reshape(-1)
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        _abi.call("focr_hip_focrq_writer_add_tensor", self._h, name.encode(), _CODE[dtype],
                  _ptr(sh) if sh.size else None, sh.size, _ptr(buf) if buf.size else None, buf.size)

    def add_quantized(self, name: str, dtype: str, shape, data: bytes, scales, group_size: int = 0,
                      tier: int = 0) -> None:
        sh = np.asarray(shape, dtype=np.uint64).reshape(-1)
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        sc = np.ascontiguousarray(np.asarray(scales, dtype=np.float32).reshape(-1))
        _abi.call("focr_hip_focrq_writer_add_quantized", self._h, name.encode(), _CODE[dtype],
                  _ptr(sh) if sh.size else None, sh.size, _ptr(buf) if buf.size else None, buf.size,
                  _ptr(sc) if sc.size else None, sc.size, int(group_size), int(tier))

    def build(self) -> bytes:
        n = C.c_size_t()
        _abi.call("focr_hip_focrq_writer_build", self._h, None, 0, C.byref(n))
        out = np.empty(n.value, dtype=np.uint8)
        _abi.call("focr_hip_focrq_writer_build", self._h, _ptr(out), out.size, C.byref(n))
        return out.tobytes()

    def write(self, path) -> None:
        _abi.call("focr_hip_focrq_writer_write", self._h, str(path).encode())

    def close(self) -> None:
        if self._h:
            _abi.lib().focr_hip_focrq_writer_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


def _src_code(src: DeviceArray, src_dtype: str | None) -> int:
    if src_dtype is None:
        if src.dtype == np.float32:
            return _abi.DT_F32
        if src.dtype == np.float16:
            return _abi.DT_F16
        raise ValueError("pass src_dtype='BF16' for a bfloat16 payload held as uint16")
    return _CODE[src_dtype]


def quantize_weight_i8(src: DeviceArray, n: int, k: int, src_dtype: str | None = None):
    """quant/int8.rs:145-163 on the device: (q [n,k] i8, scales [n] f32) DeviceArrays."""
    ctx = src.ctx
    q = DeviceArray(ctx, (n, k), np.int8)
    s = DeviceArray(ctx, (n,), np.float32)
    _abi.call("focr_hip_quantize_weight_i8", ctx.handle, src.c_ptr, _src_code(src, src_dtype), int(n), int(k),
              q.c_ptr, s.c_ptr)
    return q, s


def pack_weight_i4(src: DeviceArray, n: int, k: int, group: int = 32, src_dtype: str | None = None):
    """quant/int4.rs:142-205 on the device: (packed [n,k/2] u8, scales [n,k/group] f32)."""
    ctx = src.ctx
    p = DeviceArray(ctx, (n, k // 2), np.uint8)
    s = DeviceArray(ctx, (n, max(k // max(group, 1), 1)), np.float32)
    _abi.call("focr_hip_pack_weight_i4", ctx.handle, src.c_ptr, _src_code(src, src_dtype), int(n), int(k),
              int(group), p.c_ptr, s.c_ptr)
    return p, s
