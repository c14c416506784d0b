"""Weight container (.focrq / safetensors) reader and writer — CPU tests.

The C++ reader/writer in libfocr_hip.so (host code; no GPU call is made) is
checked three ways:

* the reference's own reader/writer tests, restated case by case
  (src/native_engine/weights.rs:1229-1846, src/quant/focrq.rs:743-1020),
  each run against the library AND the Python oracle (oracle/focrq_ref.py);
* the layout rules of docs/focrq-format.md re-derived byte by byte (51-byte
  prefix, canonical sorted-key JSON, payload-relative 64-byte-aligned
  ranges with zero padding);
* a seeded differential fuzz: mutated blobs must be accepted or refused the
  same way, with the same message, by the library and the oracle.
"""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from franken_ocr_amd import _abi
from franken_ocr_amd.focrq import FocrqBuilder, Weights
from oracle import focrq_ref as R

NOTICE = R.DEFAULT_NOTICE
GOT = R.REGISTRY["got-ocr2"]
U64_MAX = 2**64 - 1


def bf16_le(vals) -> bytes:
    return (np.asarray(vals, np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()


def f32_le(vals) -> bytes:
    return np.asarray(vals, np.float32).tobytes()


def _esc(s: str) -> str:
    return s.replace("\\", "\\\\").replace('"', '\\"')


# weights.rs:1085-1151 build_focrq / _with_license / _and_header_source_sha
def build_focrq(version, arch, sha, directory_json, payload, license_notice=NOTICE, header_sha=""):
    header = (f'{{"tensors":{directory_json},"arch_target":{arch},"source_sha256":"{_esc(header_sha)}",'
              f'"license_notice":"{_esc(license_notice)}"}}').encode()
    return (b"FOCRQ\0" + struct.pack("<IB", version, arch) + bytes(sha) + struct.pack("<Q", len(header)) + header
            + bytes(payload))


# weights.rs:1153-1178 build_focrq_with_model_id
def build_focrq_with_model_id(directory_json, payload, license_notice, model_id):
    header = (f'{{"tensors":{directory_json},"arch_target":0,"source_sha256":"",'
              f'"license_notice":"{_esc(license_notice)}","model_id":"{_esc(model_id)}"}}').encode()
    return (b"FOCRQ\0" + struct.pack("<IB", 1, 0) + bytes(32) + struct.pack("<Q", len(header)) + header
            + bytes(payload))


# weights.rs:1180-1200 build_safetensors
def build_safetensors(tensors):
    entries, payload = [], b""
    for name, dtype, shape, data in tensors:
        beg = len(payload)
        payload += data
        entries.append(f'"{name}":{{"dtype":"{dtype}","shape":{json.dumps(list(shape)).replace(" ", "")},'
                       f'"data_offsets":[{beg},{len(payload)}]}}')
    header = ("{" + ",".join(entries) + "}").encode()
    return struct.pack("<Q", len(header)) + header + payload


def load_both(blob):
    """(library Weights, oracle Weights) or the pair of FormatMismatch messages."""
    try:
        lw = Weights.from_bytes(blob)
        lerr = None
    except _abi.FormatMismatch as e:
        lw, lerr = None, str(e)
    try:
        ow = R.Weights.from_bytes(blob)
        oerr = None
    except R.FormatMismatch as e:
        ow, oerr = None, str(e)
    return lw, lerr, ow, oerr


def _norm(msg):
    # JSON decode errors: only the reference's prefix is restated.
    for cut in ("JSON invalid:", " invalid: "):
        if cut in msg:
            return msg[: msg.index(cut) + len(cut)]
    return msg


def ok_both(blob):
    lw, lerr, ow, oerr = load_both(blob)
    assert lerr is None and oerr is None, (lerr, oerr)
    assert lw.names() == ow.names()
    return lw, ow


def err_both(blob):
    lw, lerr, ow, oerr = load_both(blob)
    assert lerr is not None and oerr is not None, (lerr, oerr)
    assert _norm(lerr) == _norm(oerr)
    return lerr


# ---- weights.rs tests --------------------------------------------------------

def test_focrq_roundtrips_bf16_tensor_bit_exactly():
    vals = [1.0, -2.0, 0.5, 3.0, 0.0, -0.25]
    payload = bf16_le(vals)
    d = f'{{"w":{{"dtype":"BF16","shape":[2,3],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    w, o = ok_both(build_focrq(1, 2, [7] * 32, d, payload))
    assert w.is_focrq() and len(w) == 1 and w.arch_target() == 2
    assert w.source_sha256() == "07" * 32 == o.source_sha256
    assert w.license_notice() == NOTICE
    assert w.record("w").dtype == "BF16" and w.record("w").shape == (2, 3)
    m = w.mat("w")
    assert m.shape == (2, 3) and m.reshape(-1).tolist() == vals == o.mat("w")[0]


def test_rejects_focrq_without_baidu_mit_license_notice():
    msg = err_both(build_focrq(1, 0, [0] * 32, "{}", b"", license_notice="Copyright (c) 2026 Baidu"))
    assert "license_notice" in msg and "MIT License" in msg


def test_focrq_absent_and_empty_model_id_resolve_to_unlimited_ocr():
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, "{}", b""))
    assert w.model_id() == "unlimited-ocr"
    w, _ = ok_both(build_focrq_with_model_id("{}", b"", NOTICE, ""))
    assert w.model_id() == "unlimited-ocr"


def test_focrq_declares_got_ocr2_with_apache_notice_loads():
    w, o = ok_both(build_focrq_with_model_id("{}", b"", GOT, "got-ocr2"))
    assert w.model_id() == "got-ocr2" == o.model_id


def test_focrq_unknown_model_id_is_refused():
    assert "unknown model_id" in err_both(build_focrq_with_model_id("{}", b"", NOTICE, "totally-bogus-model"))


def test_focrq_got_ocr2_with_wrong_notice_is_refused():
    msg = err_both(build_focrq_with_model_id("{}", b"", NOTICE, "got-ocr2"))
    assert "does not match the registered got-ocr2 notice" in msg


@pytest.mark.parametrize("arch", list(R.REGISTRY))
def test_every_registered_arch_accepts_only_its_notice(arch):
    w, _ = ok_both(build_focrq_with_model_id("{}", b"", R.REGISTRY[arch], arch))
    assert w.model_id() == arch
    if arch != "unlimited-ocr":
        err_both(build_focrq_with_model_id("{}", b"", R.REGISTRY[arch] + " ", arch))


def test_safetensors_reports_default_model_id():
    w, _ = ok_both(build_safetensors([("w", "BF16", [1], bf16_le([1.0]))]))
    assert w.model_id() == "unlimited-ocr" and not w.is_focrq()


def test_focrq_header_source_sha256_overrides_prefix_when_valid():
    payload = bf16_le([1.0])
    d = f'{{"w":{{"dtype":"BF16","shape":[1],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    w, _ = ok_both(build_focrq(1, 0, [7] * 32, d, payload, header_sha="ab" * 32))
    assert w.source_sha256() == "ab" * 32


def test_rejects_malformed_focrq_header_source_sha256_override():
    payload = bf16_le([1.0])
    d = f'{{"w":{{"dtype":"BF16","shape":[1],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    msg = err_both(build_focrq(1, 0, [7] * 32, d, payload, header_sha="AB-not-lowercase-or-64-hex"))
    assert "source_sha256" in msg and "64 lowercase hex" in msg


def test_focrq_roundtrips_f32_tensor_bit_exactly():
    vals = [1.5, -0.125, 1024.0, -3.0]
    payload = f32_le(vals)
    d = f'{{"b":{{"dtype":"F32","shape":[4],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, payload))
    m = w.mat("b")
    assert m.shape == (1, 4) and m.reshape(-1).tolist() == vals


def test_focrq_two_tensors_index_by_byte_range():
    a, b = bf16_le([1.0, 2.0]), f32_le([9.0, 8.0, 7.0])
    d = (f'{{"a":{{"dtype":"BF16","shape":[2],"byte_offset":0,"byte_len":{len(a)}}},'
         f'"b":{{"dtype":"F32","shape":[3],"byte_offset":{len(a)},"byte_len":{len(b)}}}}}')
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, a + b))
    assert w.vec("a").tolist() == [1.0, 2.0] and w.vec("b").tolist() == [9.0, 8.0, 7.0]


def test_focrq_qint8_roundtrips():
    wb = np.array([1, -2, 3, 4, -5, 6], np.int8).tobytes()
    d = ('{"q":{"dtype":"QInt8PerChan","shape":[2,3],"byte_offset":0,"byte_len":6,"scales_offset":6,'
         '"scales_len":8}}')
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, wb + f32_le([0.1, 0.2])))
    q = w.qint8("q")
    assert (q.n, q.k) == (2, 3)
    assert q.w.reshape(-1).tolist() == [1, -2, 3, 4, -5, 6]
    assert q.scales.tolist() == np.array([0.1, 0.2], np.float32).tolist()


def test_focrq_qint4_roundtrips():
    packed = bytes(range(16))
    d = ('{"e":{"dtype":"QInt4PerGroup","shape":[2,16],"byte_offset":0,"byte_len":16,"scales_offset":16,'
         '"scales_len":8,"group_size":16,"tier":3}}')
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, packed + f32_le([0.1, 0.2])))
    q = w.qint4("e")
    assert (q.n, q.k, q.group_size, q.tier) == (2, 16, 16, 3)
    assert q.packed.tobytes() == packed
    assert q.scales.reshape(-1).tolist() == np.array([0.1, 0.2], np.float32).tolist()


def test_focrq_load_from_temp_file_roundtrips(tmp_path):
    vals = [1.0, -2.0, 4.0, 8.0]
    payload = bf16_le(vals)
    d = f'{{"t":{{"dtype":"BF16","shape":[2,2],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    p = tmp_path / "t.focrq"
    p.write_bytes(build_focrq(1, 1, [3] * 32, d, payload))
    with Weights.load(p) as w:
        m = w.mat("t")
        assert m.shape == (2, 2) and m.reshape(-1).tolist() == vals


def test_census_accepts_exact_set_and_rejects_missing_and_unexpected(tmp_path):
    payload = bf16_le([1.0, 2.0])
    d = f'{{"x":{{"dtype":"BF16","shape":[2],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    blob = build_focrq(1, 0, [0] * 32, d, payload)
    w, o = ok_both(blob)
    w.census(["x"])
    with pytest.raises(_abi.FormatMismatch) as e:
        w.census(["x", "y"])
    assert "missing" in str(e.value)
    with pytest.raises(R.FormatMismatch) as eo:
        o.census(["x", "y"])
    assert str(e.value) == str(eo.value)
    a, b = bf16_le([1.0]), bf16_le([2.0])
    d2 = (f'{{"x":{{"dtype":"BF16","shape":[1],"byte_offset":0,"byte_len":{len(a)}}},'
          f'"stale":{{"dtype":"BF16","shape":[1],"byte_offset":{len(a)},"byte_len":{len(b)}}}}}')
    w2, o2 = ok_both(build_focrq(1, 0, [0] * 32, d2, a + b))
    with pytest.raises(_abi.FormatMismatch) as e:
        w2.census(["x"])
    assert "unexpected" in str(e.value)
    # more than six names: the preview is cut at six with ", …"
    many = [f"n{i}" for i in range(9)]
    with pytest.raises(_abi.FormatMismatch) as e:
        w2.census(many)
    with pytest.raises(R.FormatMismatch) as eo:
        o2.census(many)
    assert str(e.value) == str(eo.value) and "…" in str(e.value)
    p = tmp_path / "c.focrq"
    p.write_bytes(blob)
    Weights.load_with_census(p, ["x"]).close()
    with pytest.raises(_abi.FormatMismatch):
        Weights.load_with_census(p, ["x", "missing"])


def test_safetensors_header_parses_widens_and_skips_metadata():
    vals = [1.0, -2.0, 0.5, 3.0]
    w, _ = ok_both(build_safetensors([("model.norm.weight", "BF16", [4], bf16_le(vals))]))
    assert not w.is_focrq() and len(w) == 1 and w.contains("model.norm.weight")
    assert w.mat("model.norm.weight").shape == (1, 4) and w.vec("model.norm.weight").tolist() == vals
    payload = f32_le([1.0, 2.0])
    header = (f'{{"__metadata__":{{"format":"pt"}},"w":{{"dtype":"F32","shape":[2],'
              f'"data_offsets":[0,{len(payload)}]}}}}').encode()
    w, _ = ok_both(struct.pack("<Q", len(header)) + header + payload)
    assert len(w) == 1 and w.vec("w").tolist() == [1.0, 2.0]
    w, _ = ok_both(build_safetensors([("a", "F32", [2], f32_le([1.0, 2.0])),
                                      ("b", "BF16", [3], bf16_le([4.0, 5.0, 6.0]))]))
    assert w.vec("a").tolist() == [1.0, 2.0] and w.vec("b").tolist() == [4.0, 5.0, 6.0]
    with pytest.raises(_abi.FormatMismatch):
        w.vec("missing")


def test_safetensors_rejections():
    assert "unsupported safetensors dtype" in err_both(build_safetensors([("w", "I8", [1], b"\0")]))
    header = b'{"w":{"dtype":"F32","shape":[1],"data_offsets":[8,4]}}'
    assert "has end 4 < beg 8" in err_both(struct.pack("<Q", len(header)) + header + bytes(8))
    assert "safetensors truncated" in err_both(b"\1\2\3")


def test_bf16_and_f16_widening_of_known_values():
    vals = [0.0, 1.0, -1.0, 2.0, 0.5, -0.5, 256.0, -3.0]
    w, _ = ok_both(build_safetensors([("b", "BF16", [8], bf16_le(vals))]))
    assert w.vec("b").tolist() == vals
    # bf16(1.1) keeps the top 16 bits: 1.1015625 (weights.rs:1635-1642)
    w, _ = ok_both(build_safetensors([("b", "BF16", [1], struct.pack("<H", 0x3F8D))]))
    assert abs(w.vec("b")[0] - 1.1015625) < 1e-7
    f16 = [0.0, 1.0, -2.0, 0.25, 65504.0, 2.0**-24, -(2.0**-14)]
    w, o = ok_both(build_safetensors([("h", "F16", [len(f16)], np.asarray(f16, np.float16).tobytes())]))
    assert w.vec("h").tolist() == f16 == o.mat("h")[0]


def test_rejects_unknown_magic():
    err_both(struct.pack("<Q", 9999) + b"junk")


def test_rejects_future_focrq_version():
    payload = bf16_le([1.0])
    d = f'{{"x":{{"dtype":"BF16","shape":[1],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    assert "newer than this binary" in err_both(build_focrq(2, 0, [0] * 32, d, payload))


def test_rejects_directory_overrunning_payload_and_bad_byte_len():
    payload = bf16_le([1.0, 2.0])
    err_both(build_focrq(1, 0, [0] * 32, '{"x":{"dtype":"BF16","shape":[2],"byte_offset":0,"byte_len":100}}',
                         payload))
    msg = err_both(build_focrq(1, 0, [0] * 32, '{"x":{"dtype":"BF16","shape":[2,3],"byte_offset":0,"byte_len":4}}',
                               payload))
    assert "shape×dtype" in msg or "overruns" in msg


def test_rejects_shape_numel_overflow_without_panicking():
    d = f'{{"x":{{"dtype":"BF16","shape":[{U64_MAX},2],"byte_offset":0,"byte_len":0}}}}'
    assert "element count overflows" in err_both(build_focrq(1, 0, [0] * 32, d, b""))


def test_qint4_accessor_rejects_noncanonical_group_size_even_when_it_divides_k():
    d = ('{"q":{"dtype":"QInt4PerGroup","shape":[1,32],"byte_offset":0,"byte_len":16,"scales_offset":16,'
         '"scales_len":16,"group_size":8,"tier":1}}')
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, bytes(16) + f32_le([1.0] * 4)))
    with pytest.raises(_abi.FormatMismatch) as e:
        w.qint4("q")
    assert "must be 16 or 32" in str(e.value)


def test_rejects_qint4_odd_numel_at_load_time():
    d = ('{"odd":{"dtype":"QInt4PerGroup","shape":[1,3],"byte_offset":0,"byte_len":1,"scales_offset":1,'
         '"scales_len":0,"group_size":1}}')
    assert "odd element count" in err_both(build_focrq(1, 0, [0] * 32, d, b"\0"))


def test_tensor_not_found_and_mat_rejects_quantized():
    payload = bf16_le([1.0])
    d = f'{{"x":{{"dtype":"BF16","shape":[1],"byte_offset":0,"byte_len":{len(payload)}}}}}'
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, payload))
    for fn in (w.mat, w.qint8, w.qint4):
        with pytest.raises(_abi.FormatMismatch) as e:
            fn("nope")
        assert 'tensor "nope" not found in weights directory' == str(e.value)
    assert w.record("nope") is None
    d = ('{"q":{"dtype":"QInt8PerChan","shape":[2,2],"byte_offset":0,"byte_len":4,"scales_offset":4,'
         '"scales_len":8}}')
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, d, np.array([1, 2, 3, 4], np.int8).tobytes() + f32_le([0.1, 0.2])))
    with pytest.raises(_abi.FormatMismatch):
        w.mat("q")
    w.qint8("q")
    with pytest.raises(_abi.FormatMismatch) as e:
        w.qint4("q")
    assert str(e.value) == 'tensor "q" is QInt8PerChan, not QInt4PerGroup'


def test_load_missing_file_is_model_not_found(tmp_path):
    with pytest.raises(_abi.ModelNotFound) as e:
        Weights.load("/definitely/not/a/real/weights.focrq")
    assert e.value.status == _abi.E_NOT_FOUND
    with pytest.raises(_abi.ModelNotFound):
        Weights.load(tmp_path)  # a directory


def test_names_are_sorted_and_complete():
    w, _ = ok_both(build_safetensors([("zeta", "F32", [1], f32_le([1.0])), ("alpha", "F32", [1], f32_le([2.0])),
                                      ("mid", "F32", [1], f32_le([3.0]))]))
    assert w.names() == ["alpha", "mid", "zeta"]


def test_empty_blob_and_empty_container():
    err_both(b"")
    w, _ = ok_both(build_focrq(1, 0, [0] * 32, "{}", b""))
    assert w.is_empty()
    w.census([])


# ---- quant/focrq.rs writer tests ---------------------------------------------

def test_writer_roundtrips_every_dtype_through_reader():
    vals = [1.0, -2.0, 0.5, 3.0, 0.0, -0.25]
    b = FocrqBuilder().with_arch_target(2).with_source_sha256(bytes([7] * 32))
    b.add_tensor("w", "BF16", [2, 3], bf16_le(vals))
    b.add_tensor("bias", "F32", [4], f32_le([1.5, -0.125, 1024.0, -3.0]))
    b.add_quantized("q", "QInt8PerChan", [2, 3], np.array([1, -2, 3, 4, -5, 6], np.int8).tobytes(), [0.1, 0.2])
    b.add_quantized("e", "QInt4PerGroup", [2, 16], bytes(range(16)), [0.1, 0.2], 16, 3)
    w, _ = ok_both(b.build())
    assert w.arch_target() == 2 and w.source_sha256() == "07" * 32 and w.license_notice() == NOTICE
    assert w.mat("w").reshape(-1).tolist() == vals
    assert w.mat("bias").shape == (1, 4)
    assert w.qint8("q").w.reshape(-1).tolist() == [1, -2, 3, 4, -5, 6]
    q4 = w.qint4("e")
    assert (q4.group_size, q4.tier) == (16, 3) and q4.packed.tobytes() == bytes(range(16))


def test_writer_forward_compat_fields_are_ignored_by_reader():
    b = (FocrqBuilder().with_provenance_json('{"hf_commit":"abc","source_sha256_hex":"00"}')
         .with_model_config_json('{"hidden_size":1280,"use_mla":false}')
         .with_packing_manifest_json('{"quant_recipe":"decoder-ffn-int8-v1"}'))
    b.add_tensor("x", "BF16", [2], bf16_le([1.0, 2.0]))
    blob = b.build()
    w, _ = ok_both(blob)
    assert w.vec("x").tolist() == [1.0, 2.0]
    assert blob == R.build({"x": ("BF16", [2], bf16_le([1.0, 2.0]), b"", 0, 0)},
                           model_config='{"hidden_size":1280,"use_mla":false}',
                           packing_manifest='{"quant_recipe":"decoder-ffn-int8-v1"}',
                           provenance='{"hf_commit":"abc","source_sha256_hex":"00"}')
    with pytest.raises(_abi.FocrHipError):
        FocrqBuilder().with_provenance_json("{not json")


def test_writer_census_determinism_and_sorted_emission():
    def make():
        b = FocrqBuilder().with_arch_target(1).with_source_sha256(bytes([5] * 32))
        b.add_tensor("zeta", "BF16", [2], bf16_le([3.0, 4.0]))
        b.add_tensor("alpha", "F32", [2], f32_le([1.0, 2.0]))
        b.add_tensor("mid", "F32", [1], f32_le([3.0]))
        return b.build()

    assert make() == make()
    w, _ = ok_both(make())
    assert w.names() == ["alpha", "mid", "zeta"]
    w.census(["alpha", "mid", "zeta"])
    with pytest.raises(_abi.FormatMismatch):
        w.census(["alpha"])


def test_writer_model_id_rules():
    b = FocrqBuilder().with_model_id("got-ocr2").with_license_notice(GOT)
    b.add_tensor("w", "BF16", [2], bf16_le([1.0, 2.0]))
    blob = b.build()
    assert b'"model_id":"got-ocr2"' in blob
    w, _ = ok_both(blob)
    assert w.model_id() == "got-ocr2"

    def make(set_default):
        b = FocrqBuilder().with_arch_target(1).with_source_sha256(bytes([9] * 32))
        if set_default:
            b.with_model_id("unlimited-ocr")
        b.add_tensor("t", "BF16", [2], bf16_le([3.0, 4.0]))
        return b.build()

    assert make(False) == make(True) and b"model_id" not in make(False)
    b = FocrqBuilder().with_model_id("")
    b.add_tensor("t", "F32", [1], f32_le([1.0]))
    assert b"model_id" not in b.build()


def test_writer_rejections_carry_reference_texts():
    b = FocrqBuilder()
    b.add_tensor("x", "F32", [1], f32_le([1.0]))
    cases = [
        (lambda: b.add_tensor("x", "F32", [1], f32_le([1.0])), 'add tensor: duplicate name "x"'),
        (lambda: b.add_tensor("q", "QInt8PerChan", [1], b"\0"),
         'add_tensor: "q" is a quantized dtype QInt8PerChan; use add_quantized'),
        (lambda: b.add_quantized("h", "BF16", [1], b"\0\0", []),
         'add_quantized: "h" dtype Bf16 is not quantized; use add_tensor'),
        (lambda: b.add_tensor("y", "F32", [2], f32_le([1.0])),
         'tensor "y": data len 4 != shape×dtype 8 (F32, shape [2])'),
        (lambda: b.add_quantized("z", "QInt8PerChan", [4], b"\0" * 4, [1.0] * 4),
         'tensor "z": QInt8 shape must be rank-2 [n,k], got [4]'),
        (lambda: b.add_quantized("z", "QInt8PerChan", [1, 4], b"\0" * 4, [1.0], 16, 0),
         'tensor "z": QInt8 group_size and tier must be zero'),
        (lambda: b.add_quantized("z", "QInt8PerChan", [2, 2], b"\0" * 4, [1.0]),
         'tensor "z": scale bytes 4 != qint8 n*f32 8'),
        (lambda: b.add_quantized("z", "QInt4PerGroup", [1, 32], b"\0" * 16, [1.0] * 4, 8, 0),
         'tensor "z": QInt4 group_size 8 must be 16 or 32'),
        (lambda: b.add_quantized("z", "QInt4PerGroup", [1, 48], b"\0" * 24, [1.0] * 2, 32, 0),
         'tensor "z": QInt4 k 48 must be divisible by group_size 32'),
        (lambda: b.add_quantized("z", "QInt4PerGroup", [1, 3], b"\0", [1.0], 16, 0),
         'tensor "z": QInt4 shape [1, 3] has odd element count 3'),
        (lambda: b.add_quantized("z", "QInt4PerGroup", [1, 32], b"\0" * 16, [1.0], 16, 0),
         'tensor "z": scale bytes 4 != qint4 n*(k/group_size)*f32 8'),
    ]
    for fn, text in cases:
        with pytest.raises(_abi.FormatMismatch) as e:
            fn()
        assert str(e.value) == text


# ---- docs/focrq-format.md layout, re-derived byte by byte ----------------------

def _parse_prefix(blob):
    magic, version, arch = blob[:6], *struct.unpack_from("<IB", blob, 6)
    sha = blob[11:43]
    (hlen,) = struct.unpack_from("<Q", blob, 43)
    header = blob[51:51 + hlen]
    return magic, version, arch, sha, header, blob[51 + hlen:]


@pytest.mark.parametrize("align", [False, True])
def test_layout_prefix_canonical_json_and_alignment(align):
    rng = np.random.default_rng(7)
    b = FocrqBuilder().with_arch_target(3).with_source_sha256(bytes(range(32))).with_alignment(align)
    tensors = {}
    for i, (dt, shape) in enumerate([("BF16", [3, 5]), ("QInt8PerChan", [7, 9]), ("QInt4PerGroup", [5, 64]),
                                     ("F32", [11]), ("QInt4PerGroup", [3, 32])]):
        name = f"model.layers.{i}.w"
        n = int(np.prod(shape))
        if dt == "BF16":
            data = rng.integers(0, 2**16, n, dtype=np.uint16).tobytes()
            b.add_tensor(name, dt, shape, data)
            tensors[name] = (dt, shape, data, b"")
        elif dt == "F32":
            data = rng.standard_normal(n).astype(np.float32).tobytes()
            b.add_tensor(name, dt, shape, data)
            tensors[name] = (dt, shape, data, b"")
        elif dt == "QInt8PerChan":
            data = rng.integers(-127, 128, n, dtype=np.int8).tobytes()
            sc = rng.random(shape[0]).astype(np.float32)
            b.add_quantized(name, dt, shape, data, sc)
            tensors[name] = (dt, shape, data, sc.tobytes())
        else:
            group = 32 if shape[1] % 64 == 0 else 16
            data = rng.integers(0, 256, n // 2, dtype=np.uint8).tobytes()
            sc = rng.random(shape[0] * shape[1] // group).astype(np.float32)
            b.add_quantized(name, dt, shape, data, sc, group, 2)
            tensors[name] = (dt, shape, data, sc.tobytes())
    blob = b.build()
    magic, version, arch, sha, header, payload = _parse_prefix(blob)
    assert magic == b"FOCRQ\0" and version == 1 and arch == 3 and sha == bytes(range(32))
    h = json.loads(header)
    # canonical: sorted keys, no insignificant whitespace
    assert header.decode() == json.dumps(h, sort_keys=True, separators=(",", ":"), ensure_ascii=False)
    assert h["format_version"] == 1 and h["arch_target"] == 3 and h["source_sha256"] == bytes(range(32)).hex()
    assert h["license_notice"] == NOTICE and "model_id" not in h
    used = np.zeros(len(payload), bool)
    for name, (dt, shape, data, sc) in tensors.items():
        r = h["tensors"][name]
        assert r["dtype"] == dt and r["shape"] == shape and r["byte_len"] == len(data)
        assert payload[r["byte_offset"]:r["byte_offset"] + r["byte_len"]] == data
        assert not used[r["byte_offset"]:r["byte_offset"] + r["byte_len"]].any()
        used[r["byte_offset"]:r["byte_offset"] + r["byte_len"]] = True
        if align:
            assert r["byte_offset"] % 64 == 0
        if dt.startswith("QInt"):
            assert payload[r["scales_offset"]:r["scales_offset"] + r["scales_len"]] == sc
            assert not used[r["scales_offset"]:r["scales_offset"] + r["scales_len"]].any()
            used[r["scales_offset"]:r["scales_offset"] + r["scales_len"]] = True
            assert ("tier" in r) and ("group_size" in r)
            if align:
                assert r["scales_offset"] % 64 == 0
        else:
            assert "tier" not in r and "scales_len" not in r
    # everything not covered by a range is zero padding (none without alignment)
    assert not np.frombuffer(payload, np.uint8)[~used].any()
    if not align:
        assert used.all()
    # the library writer and the oracle writer agree byte for byte
    assert blob == R.build({k: (v[0], v[1], v[2], v[3], h["tensors"][k].get("group_size", 0),
                                h["tensors"][k].get("tier", 0)) for k, v in tensors.items()},
                           arch_target=3, source_sha256=bytes(range(32)), align=align)
    w, _ = ok_both(blob)
    for name, (dt, shape, data, sc) in tensors.items():
        rec = w.record(name)
        assert rec.shape == tuple(shape) and rec.dtype == dt


# ---- differential fuzz: library vs oracle on mutated blobs ----------------------

def _seed_blobs():
    out = []
    for align in (False, True):
        b = FocrqBuilder().with_arch_target(1).with_source_sha256(bytes([0xA5] * 32)).with_alignment(align)
        b.add_tensor("a.w", "BF16", [2, 3], bf16_le([1, 2, 3, 4, 5, 6]))
        b.add_tensor("b", "F32", [3], f32_le([1, 2, 3]))
        b.add_quantized("c", "QInt8PerChan", [2, 4], bytes(8), [0.5, 0.25])
        b.add_quantized("d", "QInt4PerGroup", [2, 32], bytes(32), [1.0] * 4, 16, 1)
        out.append(b.build())
    out.append(build_safetensors([("x", "F32", [2], f32_le([1, 2])), ("y", "F16", [1, 2], bytes(4))]))
    out.append(build_focrq_with_model_id('{"t":{"dtype":"F16","shape":[1],"byte_offset":0,"byte_len":2}}', b"\0<",
                                         GOT, "got-ocr2"))
    return out


_TOKENS = [b"0", b"1", b"9", b"-1", b"-0", b"1.0", b"1e3", b"18446744073709551615", b"18446744073709551616",
           b'"x"', b"null", b"true", b"[]", b"{}", b",", b"}", b"]", b'"', b"\\", b" ", b"F32", b"BF16",
           b"QInt8PerChan", b"QInt4PerGroup", b"F64", b"shape", b"tier", b"256", b"group_size", b"model_id",
           b"\xff", b"\xc3\xa9"]


def _mutate(blob: bytes, rng) -> bytes:
    b = bytearray(blob)
    is_fq = blob[:6] == b"FOCRQ\0"
    hstart = 51 if is_fq else 8
    if len(blob) < hstart:  # already cut inside the prefix: flip or cut further
        if b and rng.random() < 0.5:
            b[int(rng.integers(0, len(b)))] ^= 0x5A
            return bytes(b)
        return bytes(b[: int(rng.integers(0, len(b) + 1))])
    (hlen,) = struct.unpack_from("<Q", blob, hstart - 8)
    hlen = min(hlen, len(blob) - hstart)
    kind = rng.integers(0, 7)
    if kind == 0 and len(b) > 1:  # flip a byte anywhere
        i = int(rng.integers(0, len(b)))
        b[i] ^= int(rng.integers(1, 256))
    elif kind == 1:  # truncate
        b = b[: int(rng.integers(0, len(b) + 1))]
    elif kind == 2:  # change header_len
        struct.pack_into("<Q", b, hstart - 8, max(0, hlen + int(rng.integers(-3, 4))))
    elif kind in (3, 4):  # replace a header token by another token
        hdr = bytes(b[hstart:hstart + hlen])
        pos = int(rng.integers(0, max(hlen, 1)))
        ln = int(rng.integers(1, 6))
        tok = _TOKENS[int(rng.integers(0, len(_TOKENS)))]
        hdr = hdr[:pos] + tok + hdr[pos + ln:]
        b = b[: hstart - 8] + struct.pack("<Q", len(hdr)) + hdr + b[hstart + hlen:]
    elif kind == 5 and is_fq:  # version / arch bytes
        b[6 + int(rng.integers(0, 5))] = int(rng.integers(0, 256))
    else:  # duplicate a header slice
        hdr = bytes(b[hstart:hstart + hlen])
        i, j = sorted(rng.integers(0, max(hlen, 1), 2))
        hdr = hdr[:j] + hdr[i:j] + hdr[j:]
        b = b[: hstart - 8] + struct.pack("<Q", len(hdr)) + hdr + b[hstart + hlen:]
    return bytes(b)


def test_differential_fuzz_library_matches_oracle():
    rng = np.random.default_rng(20261201)
    seeds = _seed_blobs()
    accepted = refused = 0
    for it in range(3000):
        blob = _mutate(seeds[it % len(seeds)], rng)
        if rng.random() < 0.3:
            blob = _mutate(blob, rng)
        lw, lerr, ow, oerr = load_both(blob)
        assert (lerr is None) == (oerr is None), (it, blob[:200], lerr, oerr)
        if lerr is not None:
            assert _norm(lerr) == _norm(oerr), (it, lerr, oerr)
            refused += 1
            continue
        accepted += 1
        assert lw.names() == ow.names()
        assert lw.arch_target() == ow.arch_target and lw.source_sha256() == ow.source_sha256
        assert lw.model_id() == ow.model_id and lw.license_notice() == ow.license_notice
        for n in ow.names():
            r = lw.record(n)
            assert (r.dtype, r.shape, r.byte_offset, r.byte_len, r.scales_offset, r.scales_len, r.group_size,
                    r.tier) == ow.directory[n].as_tuple()
            try:
                want = ow.mat(n)
            except R.FormatMismatch as e:
                with pytest.raises(_abi.FormatMismatch) as le:
                    lw.mat(n)
                assert str(le.value) == str(e)
                continue
            got = lw.mat(n)
            assert got.shape == want[1]
            np.testing.assert_array_equal(got.reshape(-1), np.asarray(want[0], np.float32))
    assert accepted > 100 and refused > 1000, (accepted, refused)
