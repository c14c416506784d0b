"""GPU parity for the upload-once weight path (.focrq -> HBM).

* the device weight quantizers (quant/int8.rs:104-163, quant/int4.rs:142-205)
  bit-exact against the oracle for F32 / BF16 / F16 payloads, including zero
  rows, NaN, +-Inf and exact .5 ties;
* quant_oc_loaded (decoder.rs:1777-1786): a BF16 record quantized on upload
  and a QInt8PerChan record copied verbatim both give GEMV outputs bit-equal
  to the oracle's gemv on the oracle-quantized weight;
* a whole MoE layer (decoder.rs:2069-2098) and an int4 prefill layer read
  from a .focrq give outputs bit-identical to the same layers built from the
  arrays directly (whose parity with the oracle the MoE tests establish),
  and the decode output stays within rel 1e-3 of the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-focrq] {msg}", flush=True)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (the stored payload)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, np.float32))
    r[nan] = 0x7FC0
    return r.astype(np.uint16)


def widen_bf16(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _stored(x: np.ndarray, dtype: str):
    """(payload array to upload, exact f32 widening of it)."""
    if dtype == "F32":
        return x.astype(np.float32), x.astype(np.float32)
    if dtype == "F16":
        h = x.astype(np.float16)
        return h, h.astype(np.float32)
    b = to_bf16_bits(x)
    return b, widen_bf16(b)


def _special_rows(n, k, seed):
    x = synth.f32_normal(synth.seed_of(seed), n * k).reshape(n, k) * 3.0
    x[0] = 0.0  # all-zero row: scale 1.0, codes 0
    x[1, ::7] = np.nan  # NaN skipped by the max, coded 0
    x[2, 3] = np.inf  # scale inf: finite -> 0, inf/inf -> NaN -> 0
    x[3, :8] = [127.0, 63.5, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]  # scale 1.0, exact ties
    x[3, 8:] = np.clip(x[3, 8:], -100, 100)
    x[4] = -0.0
    return x


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
@pytest.mark.parametrize("n,k", [(37, 160), (896, 1280), (1, 16)])
def test_quantize_weight_i8_bit_exact(ctx, dtype, n, k):
    from franken_ocr_amd.focrq import quantize_weight_i8

    _say(f"quantize_weight_i8 {dtype} n={n} k={k}")
    x = _special_rows(n, k, 40) if n >= 5 else synth.f32_normal(synth.seed_of(41), n * k).reshape(n, k)
    payload, wide = _stored(x, dtype)
    src = ctx.to_device(payload)
    q, s = quantize_weight_i8(src, n, k, src_dtype=dtype)
    st, wq, ws = O.quantize_int8_f32(wide, n, k)
    assert st == 0
    assert np.array_equal(q.numpy().reshape(-1), wq)
    assert np.array_equal(s.numpy().view(np.uint32), ws.view(np.uint32))
    if n >= 5:
        assert s.numpy()[0] == 1.0 and not q.numpy()[0].any()
        assert q.numpy()[3, :8].tolist() == [127, 64, 0, 2, 2, 0, -2, -2]


@pytest.mark.parametrize("dtype", ["F32", "BF16"])
@pytest.mark.parametrize("group", [16, 32])
def test_pack_weight_i4_bit_exact(ctx, dtype, group):
    from franken_ocr_amd.focrq import pack_weight_i4

    n, k = 129, 256
    _say(f"pack_weight_i4 {dtype} group={group}")
    x = _special_rows(n, k, 50)
    payload, wide = _stored(x, dtype)
    p, s = pack_weight_i4(ctx.to_device(payload), n, k, group, src_dtype=dtype)
    st, wp, ws = O.pack_int4_f32(wide, n, k, group)
    assert st == 0
    assert np.array_equal(p.numpy().reshape(-1), wp)
    assert np.array_equal(s.numpy().reshape(-1).view(np.uint32), ws.view(np.uint32))


def test_upload_qint8_bf16_and_qint8_records(ctx):
    from franken_ocr_amd.engine import gemv_i8
    from franken_ocr_amd.focrq import FocrqBuilder, Weights

    n, k, m = 300, 1280, 8
    _say(f"upload_qint8 n={n} k={k}")
    x32 = synth.f32_normal(synth.seed_of(60), n * k).reshape(n, k) * 0.02
    bits = to_bf16_bits(x32)
    wide = widen_bf16(bits)
    st, wq, ws = O.quantize_int8_f32(wide, n, k)
    assert st == 0
    b = FocrqBuilder().with_alignment(True)
    b.add_tensor("proj.bf16", "BF16", [n, k], bits.tobytes())
    b.add_quantized("proj.q8", "QInt8PerChan", [n, k], wq.tobytes(), ws)
    b.add_tensor("norm", "BF16", [k], to_bf16_bits(np.linspace(-1, 1, k, dtype=np.float32)).tobytes())
    w = Weights.from_bytes(b.build())
    xa = synth.f32_normal(synth.seed_of(61), m * k).reshape(m, k)
    want, _, _, _ = O.gemv_i8_batched(xa, wq, ws, n, k)
    for name in ("proj.bf16", "proj.q8"):
        q = w.upload_qint8(name, ctx=ctx)
        assert (q.n, q.k) == (n, k)
        dy = ctx.empty((m, n), np.float32)
        gemv_i8(q, ctx.to_device(xa), dy)
        assert np.array_equal(dy.numpy(), want), name
        q.free()
    # out_channels reshapes a flat record the way quant_oc(data, out) does
    q = w.upload_qint8("proj.bf16", out_channels=n * 2, ctx=ctx)
    assert (q.n, q.k) == (2 * n, k // 2)
    q.free()
    d = w.upload_f32("norm", ctx=ctx)
    assert d.shape == (1, k) and np.array_equal(d.numpy(), w.mat("norm"))


def _moe_arrays(seed, h, inter, e, si):
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((e, h)) * 0.02).astype(np.float32)
    f32 = {}
    for i in range(e):
        f32[f"experts.{i}.gate_proj"] = (rng.standard_normal((inter, h)) * 0.05).astype(np.float32)
        f32[f"experts.{i}.up_proj"] = (rng.standard_normal((inter, h)) * 0.05).astype(np.float32)
        f32[f"experts.{i}.down_proj"] = (rng.standard_normal((h, inter)) * 0.05).astype(np.float32)
    for pname, shape in (("gate_proj", (si, h)), ("up_proj", (si, h)), ("down_proj", (h, si))):
        f32[f"shared_experts.{pname}"] = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    return router, f32


def test_moe_layer_from_focrq_matches_direct_and_oracle(ctx):
    from franken_ocr_amd.engine import MoeLayer
    from franken_ocr_amd.focrq import FocrqBuilder, Weights

    h, inter, e, k, si, layer = 256, 128, 8, 2, 128, 3
    _say(f"moe_layer from .focrq h={h} inter={inter} e={e}")
    router, f32 = _moe_arrays(70, h, inter, e, si)
    b = FocrqBuilder().with_alignment(True)
    pre = f"model.layers.{layer}.mlp."
    b.add_tensor(pre + "gate.weight", "BF16", [e, h], to_bf16_bits(router).tobytes())
    quant = {}
    for j, (name, w) in enumerate(sorted(f32.items())):
        bits = to_bf16_bits(w)
        st, q, s = O.quantize_int8_f32(widen_bf16(bits), w.shape[0], w.shape[1])
        assert st == 0
        quant[name] = (q.reshape(w.shape), s)
        if j % 2:  # half the experts stored pre-quantized, half as BF16
            b.add_quantized(pre + name + ".weight", "QInt8PerChan", list(w.shape), q.tobytes(), s)
        else:
            b.add_tensor(pre + name + ".weight", "BF16", list(w.shape), bits.tobytes())
    wts = Weights.from_bytes(b.build())
    L = wts.moe_layer(layer, e, k, with_shared=True, ctx=ctx)

    def stack(p):
        return np.stack([quant[f"experts.{i}.{p}"][0] for i in range(e)]), \
            np.stack([quant[f"experts.{i}.{p}"][1] for i in range(e)])

    wg, sg = stack("gate_proj")
    wu, su = stack("up_proj")
    wd, sd = stack("down_proj")
    r32 = widen_bf16(to_bf16_bits(router))
    D = MoeLayer(h, inter, e, k, r32, wg, sg, wu, su, wd, sd, ctx=ctx)
    sh = [quant[f"shared_experts.{p}"] for p in ("gate_proj", "up_proj", "down_proj")]
    D.set_shared(si, sh[0][0], sh[0][1], sh[1][0], sh[1][1], sh[2][0], sh[2][1])
    t = 8
    x = synth.f32_normal(synth.seed_of(71), t * h).reshape(t, h)
    dx = ctx.to_device(x)
    outs = []
    for lay in (L, D):
        out, idx = ctx.empty((t, h), np.float32), ctx.empty((t, k), np.uint32)
        lay.decode(dx, out, idx, norm_topk=True, with_shared=True)
        outs.append((out.numpy(), idx.numpy()))
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][0], outs[1][0])
    st, want, widx, _ = O.moe_decode(x, r32, wg, sg, wu, su, wd, sd, e, k, inter, norm_topk=True,
                                     shared=(si, sh[0][0], sh[0][1], sh[1][0], sh[1][1], sh[2][0], sh[2][1]))
    assert st == 0 and np.array_equal(outs[0][1], widx)
    rel = np.abs(outs[0][0].astype(np.float64) - want) / np.maximum(np.abs(want), np.abs(want).max() * 1e-2)
    assert rel.max() <= 1e-3
    L.free()
    D.free()


def test_moe_layer_i4_from_focrq_matches_direct(ctx):
    from franken_ocr_amd.engine import MoeLayerI4
    from franken_ocr_amd.focrq import FocrqBuilder, Weights

    h, inter, e, group, layer = 256, 128, 8, 32, 1
    _say(f"moe_layer_i4 from .focrq h={h} inter={inter} e={e} group={group}")
    rng = np.random.default_rng(80)
    b = FocrqBuilder().with_alignment(True)
    packs = {}
    for i in range(e):
        for pname, (n, kk) in (("gate_proj", (inter, h)), ("up_proj", (inter, h)), ("down_proj", (h, inter))):
            w = (rng.standard_normal((n, kk)) * 0.05).astype(np.float32)
            st, pk, sc = O.pack_int4_f32(w, n, kk, group)
            assert st == 0
            packs[(i, pname)] = (pk.reshape(n, kk // 2), sc.reshape(n, kk // group))
            b.add_quantized(f"model.layers.{layer}.mlp.experts.{i}.{pname}.weight", "QInt4PerGroup", [n, kk],
                            pk.tobytes(), sc, group, 2)
    wts = Weights.from_bytes(b.build())
    L = wts.moe_layer_i4(layer, e, ctx=ctx)
    assert (L.hidden, L.inter, L.group) == (h, inter, group)

    def stack(p):
        return (np.stack([packs[(i, p)][0] for i in range(e)]), np.stack([packs[(i, p)][1] for i in range(e)]))

    (wg, sg), (wu, su), (wd, sd) = stack("gate_proj"), stack("up_proj"), stack("down_proj")
    D = MoeLayerI4(h, inter, e, group, wg, sg, wu, su, wd, sd, ctx=ctx)
    t, top_k = 96, 2
    x = synth.f32_normal(synth.seed_of(81), t * h).reshape(t, h)
    idx = np.stack([rng.choice(e, top_k, replace=False) for _ in range(t)]).astype(np.uint32)
    gates = rng.random((t, top_k)).astype(np.float32)
    outs = []
    for lay in (L, D):
        out = ctx.empty((t, h), np.float32)
        lay.prefill(ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates), out)
        outs.append(out.numpy())
    assert np.array_equal(outs[0], outs[1])
    st, want, _, _ = O.moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, e, inter)
    assert st == 0
    rel = np.abs(outs[0].astype(np.float64) - want) / np.maximum(np.abs(want), np.abs(want).max() * 1e-2)
    assert rel.max() <= 1e-3
    L.free()
    D.free()


def test_focrq_upload_errors_are_format_mismatch(ctx):
    from franken_ocr_amd import _abi
    from franken_ocr_amd.focrq import FocrqBuilder, Weights

    b = FocrqBuilder()
    b.add_tensor("model.layers.0.mlp.gate.weight", "F32", [4, 32], np.zeros(128, np.float32).tobytes())
    w = Weights.from_bytes(b.build())
    with pytest.raises(_abi.FormatMismatch) as e:
        w.moe_layer(0, 4, 2, ctx=ctx)
    assert "experts.0.gate_proj.weight" in str(e.value) and "not found" in str(e.value)
    with pytest.raises(_abi.FormatMismatch):
        w.moe_layer(0, 5, 2, ctx=ctx)  # router rows != n_experts
    with pytest.raises(_abi.FormatMismatch):
        w.moe_layer_i4(0, 4, ctx=ctx)
