"""Test oracle: a pure-Python restatement of the reference's weight container.

TEST INFRASTRUCTURE ONLY. Imported by tests/ as the checker for the C++
reader/writer in libfocr_hip.so; never by the product.

Reader: src/native_engine/weights.rs:443-540 (from_bytes, from_focrq_bytes),
:546-620 (from_safetensors_bytes), :634-676 (census, preview :1069-1076),
:744-923 (tensor / mat / qint8 / qint4), :949-990 (validate_directory),
:55-136 (checked_shape_len, resolve_model_id, validate_license_notice,
validate_source_sha256_hex), :232-277 (TensorRecord::expected_byte_len).
Writer: src/quant/focrq.rs:351-463 (insert_checked, validate_scales),
:479-533 (build), :544-551 (alignment), :559-692 (canonical header JSON).

Pinned by: the reference's own reader/writer tests restated in
tests/test_focrq.py (weights.rs:1229-1846, focrq.rs:743-1020), the layout
table of docs/focrq-format.md (51-byte prefix, canonical JSON, 64-byte
alignment), and a byte-level re-derivation of the prefix in the tests.

Errors are raised as FormatMismatch(message) with the reference's texts; a
JSON syntax error carries only the ".focrq header JSON invalid" prefix (the
text after it is serde_json's and is not restated).
"""

from __future__ import annotations

import json
import struct

MAGIC = b"FOCRQ\0"
FORMAT_VERSION = 1
DEFAULT_NOTICE = "Baidu Unlimited-OCR - Copyright (c) 2026 Baidu, MIT License"
# model_arch.rs:186-196, :313-401, :417-425
REGISTRY = {
    "unlimited-ocr": DEFAULT_NOTICE,
    "got-ocr2": "GOT-OCR2.0 (StepFun) - Apache-2.0",
    "smolvlm2": "SmolVLM2 (HuggingFaceTB) - Apache-2.0",
    "onechart": "OneChart - Apache-2.0",
    "tromr": "Polyphonic-TrOMR (NetEase) - Apache-2.0",
    "trocr": "TrOCR (Microsoft) - MIT",
    "pix2tex": "pix2tex / LaTeX-OCR - MIT",
}
DTYPES = ("F32", "F16", "BF16", "QInt8PerChan", "QInt4PerGroup")
U64_MAX = 2**64 - 1


class FormatMismatch(Exception):
    pass


def dbg(s: str) -> str:
    """Rust's {:?} of a str (the escapes the tests exercise)."""
    out = ['"']
    for ch in s:
        o = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif ch == "\0":
            out.append("\\0")
        elif o < 0x20 or o == 0x7F:
            out.append("\\u{%x}" % o)
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def dbg_shape(shape) -> str:
    return "[" + ", ".join(str(d) for d in shape) + "]"


class Record:
    __slots__ = ("dtype", "shape", "byte_offset", "byte_len", "scales_offset", "scales_len", "group_size", "tier")

    def __init__(self, dtype, shape, byte_offset, byte_len, scales_offset=0, scales_len=0, group_size=0, tier=0):
        self.dtype, self.shape = dtype, list(shape)
        self.byte_offset, self.byte_len = byte_offset, byte_len
        self.scales_offset, self.scales_len = scales_offset, scales_len
        self.group_size, self.tier = group_size, tier

    def as_tuple(self):
        return (self.dtype, tuple(self.shape), self.byte_offset, self.byte_len, self.scales_offset,
                self.scales_len, self.group_size, self.tier)


def _mul(a: int, b: int):
    p = a * b
    return p if p <= U64_MAX else None


def expected_byte_len(name: str, r: Record) -> int:
    numel = 1
    for d in r.shape:
        numel = _mul(numel, d)
        if numel is None:
            raise FormatMismatch(f"tensor {dbg(name)}: shape {dbg_shape(r.shape)} element count overflows usize")
    if r.dtype == "QInt4PerGroup":
        if numel % 2:
            raise FormatMismatch(
                f"tensor {dbg(name)}: QInt4 shape {dbg_shape(r.shape)} has odd element count {numel}")
        return numel // 2
    eb = {"F32": 4, "F16": 2, "BF16": 2, "QInt8PerChan": 1}[r.dtype]
    out = _mul(numel, eb)
    if out is None:
        raise FormatMismatch(
            f"tensor {dbg(name)}: byte length for {r.dtype}, shape {dbg_shape(r.shape)} overflows usize")
    return out


def validate_directory(directory: dict, payload_len: int) -> None:
    for name in sorted(directory, key=lambda s: s.encode()):
        r = directory[name]
        end = r.byte_offset + r.byte_len
        if end > U64_MAX:
            raise FormatMismatch(f"tensor {dbg(name)} byte range overflows")
        if end > payload_len:
            raise FormatMismatch(f"tensor {dbg(name)} ends at {end} but payload is {payload_len} bytes")
        exp = expected_byte_len(name, r)
        if r.byte_len != exp:
            raise FormatMismatch(f"tensor {dbg(name)}: byte_len {r.byte_len} != shape×dtype {exp} "
                                 f"({r.dtype}, shape {dbg_shape(r.shape)})")
        send = r.scales_offset + r.scales_len
        if send > U64_MAX:
            raise FormatMismatch(f"tensor {dbg(name)} scales range overflows")
        if send > payload_len:
            raise FormatMismatch(f"tensor {dbg(name)} scales end at {send} but payload is {payload_len} bytes")


def _reject_constant(c):
    raise ValueError(f"invalid number {c}")


class _Obj(list):
    """A JSON object as its (key, value) pairs: duplicates and order kept, the
    typed decoders resolve them; JSON arrays stay plain lists."""


def _pairs(pairs):
    return _Obj(pairs)


def _json(text: bytes, prefix: str):
    try:
        s = text.decode("utf-8")
        return json.loads(s, object_pairs_hook=_pairs, parse_constant=_reject_constant)
    except (UnicodeDecodeError, ValueError, RecursionError) as e:
        raise FormatMismatch(f"{prefix} JSON invalid: {e}") from None


def _is_uint(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and 0 <= v <= U64_MAX


def _u64(v, field, prefix):
    if not _is_uint(v):
        raise FormatMismatch(f"{prefix} JSON invalid: invalid type for field `{field}`")
    return v


def _u8(v, field, prefix):
    v = _u64(v, field, prefix)
    if v > 255:
        raise FormatMismatch(f"{prefix} JSON invalid: invalid value for field `{field}`")
    return v


def _str(v, field, prefix):
    if not isinstance(v, str):
        raise FormatMismatch(f"{prefix} JSON invalid: invalid type for field `{field}`")
    return v


def _shape(v, field, prefix):
    if type(v) is not list:
        raise FormatMismatch(f"{prefix} JSON invalid: invalid type for field `{field}`")
    return [_u64(d, field, prefix) for d in v]


def _record(pairs, prefix) -> Record:
    if not isinstance(pairs, _Obj):
        raise FormatMismatch(f"{prefix} JSON invalid: expected struct TensorRecord")
    known = ("dtype", "shape", "byte_offset", "byte_len", "scales_offset", "scales_len", "group_size", "tier")
    got = {}
    for k, v in pairs:
        if k in known:
            if k in got:
                raise FormatMismatch(f"{prefix} JSON invalid: duplicate field `{k}`")
            if k == "dtype":
                if not isinstance(v, str) or v not in DTYPES:
                    raise FormatMismatch(f"{prefix} JSON invalid: unknown variant")
                got[k] = v
            elif k == "shape":
                got[k] = _shape(v, k, prefix)
            elif k == "tier":
                got[k] = _u8(v, k, prefix)
            else:
                got[k] = _u64(v, k, prefix)
    for k in ("dtype", "shape", "byte_offset", "byte_len"):
        if k not in got:
            raise FormatMismatch(f"{prefix} JSON invalid: missing field `{k}`")
    return Record(got["dtype"], got["shape"], got["byte_offset"], got["byte_len"], got.get("scales_offset", 0),
                  got.get("scales_len", 0), got.get("group_size", 0), got.get("tier", 0))


class Weights:
    """The parsed container (weights.rs Weights)."""

    def __init__(self):
        self.bytes = b""
        self.payload_base = 0
        self.directory: dict[str, Record] = {}
        self.arch_target = 0
        self.source_sha256 = ""
        self.license_notice = ""
        self.model_id = "unlimited-ocr"
        self.is_focrq = False

    # weights.rs:447-453
    @classmethod
    def from_bytes(cls, blob: bytes) -> "Weights":
        w = cls()
        w.bytes = bytes(blob)
        if len(blob) >= 6 and blob[:6] == MAGIC:
            w._focrq()
        else:
            w._safetensors()
        return w

    def _focrq(self) -> None:
        b = self.bytes
        if len(b) < 51:
            raise FormatMismatch(f".focrq truncated: {len(b)} bytes < 51-byte preamble")
        (version,) = struct.unpack_from("<I", b, 6)
        if version > FORMAT_VERSION:
            raise FormatMismatch(f".focrq format_version {version} is newer than this binary supports "
                                 f"(max {FORMAT_VERSION})")
        preamble_arch = b[10]
        preamble_sha = b[11:43].hex()
        (header_len,) = struct.unpack_from("<Q", b, 43)
        header_end = 51 + header_len
        if header_end > U64_MAX:
            raise FormatMismatch(".focrq header_len overflows")
        if header_end > len(b):
            raise FormatMismatch(f".focrq header ({header_len} bytes) overruns file ({len(b)} bytes)")
        h = _json(b[51:header_end], ".focrq header")
        if not isinstance(h, _Obj):
            raise FormatMismatch(".focrq header JSON invalid: expected struct FocrqHeader")
        fields = {}
        directory = {}
        for k, v in h:  # fields decode in document order
            if k in ("tensors", "arch_target", "source_sha256", "license_notice", "model_id"):
                if k in fields:
                    raise FormatMismatch(f".focrq header JSON invalid: duplicate field `{k}`")
                if k == "arch_target":
                    v = _u8(v, k, ".focrq header")
                elif k == "tensors":
                    if not isinstance(v, _Obj):
                        raise FormatMismatch(".focrq header JSON invalid: expected a map for field `tensors`")
                    for name, rec in v:
                        directory[name] = _record(rec, ".focrq header")
                else:
                    v = _str(v, k, ".focrq header")
                fields[k] = v
        if "tensors" not in fields:
            raise FormatMismatch(".focrq header JSON invalid: missing field `tensors`")
        model_id = fields.get("model_id", "")
        if model_id == "":
            model_id = "unlimited-ocr"
        elif model_id not in REGISTRY:
            raise FormatMismatch(f".focrq declares unknown model_id {dbg(model_id)} (not in the model registry; "
                                 f"this binary cannot load it)")
        notice = fields.get("license_notice", "")
        if model_id == "unlimited-ocr":
            if not (notice == DEFAULT_NOTICE or ("Copyright (c) 2026 Baidu" in notice and "MIT License" in notice)):
                raise FormatMismatch(".focrq license_notice must include Copyright (c) 2026 Baidu and MIT License")
        elif notice != REGISTRY[model_id]:
            raise FormatMismatch(f".focrq license_notice does not match the registered {model_id} notice "
                                 f"(expected {dbg(REGISTRY[model_id])})")
        sha = fields.get("source_sha256", "")
        if sha and not (len(sha) == 64 and all(c in "0123456789abcdef" for c in sha)):
            raise FormatMismatch(".focrq source_sha256 must be 64 lowercase hex chars when present")
        self.payload_base = header_end
        validate_directory(directory, len(b) - header_end)
        self.directory = directory
        arch = fields.get("arch_target", 0)
        self.arch_target = arch if arch != 0 else preamble_arch
        self.source_sha256 = sha if sha else preamble_sha
        self.license_notice = notice
        self.model_id = model_id
        self.is_focrq = True

    def _safetensors(self) -> None:
        b = self.bytes
        if len(b) < 8:
            raise FormatMismatch(f"safetensors truncated: {len(b)} bytes < 8-byte header length prefix")
        (header_len,) = struct.unpack_from("<Q", b, 0)
        header_end = 8 + header_len
        if header_end > U64_MAX:
            raise FormatMismatch("safetensors header_len overflows")
        if header_end > len(b):
            raise FormatMismatch(f"safetensors header ({header_len} bytes) overruns file ({len(b)} bytes)")
        h = _json(b[8:header_end], "safetensors header")
        if not isinstance(h, _Obj):
            raise FormatMismatch("safetensors header JSON invalid: expected a map")
        directory = {}
        for name, v in h:
            if name == "__metadata__":
                continue
            pre = f"safetensors entry {dbg(name)} invalid:"
            if not isinstance(v, _Obj):
                raise FormatMismatch(f"{pre} expected struct StEntry")
            got = {}
            for k, x in v:
                if k == "dtype":
                    if not isinstance(x, str):
                        raise FormatMismatch(f"{pre} invalid type")
                    got[k] = x
                elif k in ("shape", "data_offsets"):
                    if type(x) is not list or not all(_is_uint(d) for d in x):
                        raise FormatMismatch(f"{pre} invalid type")
                    if k == "data_offsets" and len(x) != 2:
                        raise FormatMismatch(f"{pre} invalid length")
                    got[k] = x
            for k in ("dtype", "shape", "data_offsets"):
                if k not in got:
                    raise FormatMismatch(f"{pre} missing field `{k}`")
            beg, end = got["data_offsets"]
            if end < beg:
                raise FormatMismatch(f"safetensors entry {dbg(name)} has end {end} < beg {beg}")
            if got["dtype"] not in ("F32", "F16", "BF16"):
                raise FormatMismatch(f"unsupported safetensors dtype {dbg(got['dtype'])} "
                                     f"(expected F32/F16/BF16; the upstream Unlimited-OCR shard is BF16)")
            directory[name] = Record(got["dtype"], got["shape"], beg, end - beg)
        self.payload_base = header_end
        validate_directory(directory, len(b) - header_end)
        self.directory = directory
        self.is_focrq = False

    # ---- accessors ----
    def names(self) -> list[str]:
        return sorted(self.directory, key=lambda s: s.encode())

    def _slice(self, name, off, ln) -> bytes:
        start, end = self.payload_base + off, self.payload_base + off + ln
        if end > len(self.bytes):
            raise FormatMismatch(f"tensor {dbg(name)} range [{off}, {off + ln}) overruns payload")
        return self.bytes[start:end]

    def tensor(self, name):
        if name not in self.directory:
            raise FormatMismatch(f"tensor {dbg(name)} not found in weights directory")
        r = self.directory[name]
        data = self._slice(name, r.byte_offset, r.byte_len)
        scales = self._slice(name, r.scales_offset, r.scales_len) if r.scales_len else b""
        return r, data, scales

    def mat(self, name):
        """Widened f32 values (list of floats as numpy-free Python floats) and (rows, cols)."""
        r, data, _ = self.tensor(name)
        if len(r.shape) == 1:
            rows, cols = 1, r.shape[0]
        elif len(r.shape) == 2:
            rows, cols = r.shape
        else:
            raise FormatMismatch(f"tensor {dbg(name)} has rank {len(r.shape)}; mat() needs a 1-D or 2-D tensor")
        if r.dtype in ("QInt8PerChan", "QInt4PerGroup"):
            raise FormatMismatch(f"tensor {dbg(name)}: decode_f32: {r.dtype} is quantized; use qint8()/qint4()")
        eb = 4 if r.dtype == "F32" else 2
        if len(data) % eb:
            raise FormatMismatch(f"tensor {dbg(name)}: {r.dtype} byte len {len(data)} is not a multiple of {eb}")
        if r.dtype == "F32":
            vals = list(struct.unpack(f"<{len(data) // 4}f", data))
        elif r.dtype == "BF16":
            vals = [struct.unpack("<f", struct.pack("<I", h << 16))[0]
                    for h in struct.unpack(f"<{len(data) // 2}H", data)]
        else:
            vals = list(struct.unpack(f"<{len(data) // 2}e", data))
        exp = _mul(rows, cols)
        if exp is None:
            raise FormatMismatch(f"tensor {dbg(name)}: rows*cols overflows usize ({rows} * {cols})")
        if len(vals) != exp:
            raise FormatMismatch(f"tensor {dbg(name)} element count {len(vals)} != rows*cols {exp}")
        return vals, (rows, cols)

    def census(self, expected) -> None:
        exp = set(expected)
        missing = sorted((n for n in exp if n not in self.directory), key=lambda s: s.encode())
        unexpected = [n for n in self.names() if n not in exp]
        if not missing and not unexpected:
            return

        def preview(v):
            return "[" + ", ".join(v) + "]" if len(v) <= 6 else "[" + ", ".join(v[:6]) + ", …]"

        raise FormatMismatch(f"weights census failed: expected {len(exp)} tensors, found {len(self.directory)} "
                             f"(missing {len(missing)}: {preview(missing)}; "
                             f"unexpected {len(unexpected)}: {preview(unexpected)})")


# ---- writer (quant/focrq.rs) -------------------------------------------------

def _json_str(v: str) -> str:
    out = ['"']
    for ch in v:
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif ord(ch) < 0x20:
            out.append("\\u%04x" % ord(ch))
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def build(tensors: dict, arch_target: int = 0, source_sha256: bytes = bytes(32), license_notice: str = DEFAULT_NOTICE,
          model_id: str | None = None, align: bool = False, model_config: str | None = None,
          packing_manifest: str | None = None, provenance: str | None = None) -> bytes:
    """focrq.rs:479-533. tensors: name -> (dtype, shape, data bytes, scales bytes, group_size, tier)."""
    payload = bytearray()

    def pad():
        if align and len(payload) % 64:
            payload.extend(bytes(64 - len(payload) % 64))

    recs = []
    for name in sorted(tensors, key=lambda s: s.encode()):
        dt, shape, data, scales, group, tier = tensors[name]
        pad()
        off = len(payload)
        payload.extend(data)
        q = dt in ("QInt8PerChan", "QInt4PerGroup")
        soff = slen = 0
        if q:
            pad()
            soff = len(payload)
            payload.extend(scales)
            slen = len(scales)
        r = f'{{"byte_len":{len(data)},"byte_offset":{off},"dtype":{_json_str(dt)}'
        if q:
            r += f',"group_size":{group},"scales_len":{slen},"scales_offset":{soff}'
        r += ',"shape":[' + ",".join(str(d) for d in shape) + "]"
        if q:
            r += f',"tier":{tier}'
        recs.append(_json_str(name) + ":" + r + "}")
    h = f'{{"arch_target":{arch_target},"format_version":1,"license_notice":{_json_str(license_notice)},'
    if model_config:
        h += f'"model_config":{model_config},'
    if model_id and model_id != "unlimited-ocr":
        h += f'"model_id":{_json_str(model_id)},'
    if packing_manifest:
        h += f'"packing_manifest":{packing_manifest},'
    if provenance:
        h += f'"provenance":{provenance},'
    h += f'"source_sha256":{_json_str(bytes(source_sha256).hex())},"tensors":{{' + ",".join(recs) + "}}"
    hb = h.encode("utf-8")
    return MAGIC + struct.pack("<IB", FORMAT_VERSION, arch_target) + bytes(source_sha256) + \
        struct.pack("<Q", len(hb)) + hb + bytes(payload)
