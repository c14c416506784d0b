"""Committed golden fixtures (tests/golden/): the CPU oracle must reproduce
them exactly (CPU), and the GPU path must match them (gpu-marked tests)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import pyoracle as O

G = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(G / name, allow_pickle=False))


# ---- CPU: oracle vs fixtures -------------------------------------------------------

def test_known_answers_json_against_oracle():
    ka = json.loads((G / "known_answers.json").read_text())
    for c in ka["igemm_s8s8"]:
        out = np.array(c["out0"], np.int32)
        O.igemm_s8s8(c["a"], c["b"], c["m"], c["k"], c["n"], out)
        assert out.tolist() == c["want"], c["src"]
    for c in ka["igemm_u8s8"]:
        out = np.array(c["out0"], np.int32)
        O.igemm_u8s8(c["a"], c["b"], c["m"], c["k"], c["n"], out)
        assert out.tolist() == c["want"], c["src"]
    for c in ka["k6848_extremes"]:
        a = np.full(6848, c["a"], np.uint8 if c["unsigned"] else np.int8)
        f = O.igemm_u8s8 if c["unsigned"] else O.igemm_s8s8
        assert int(f(a, np.full(6848, c["b"], np.int8), 1, 6848, 1)[0]) == c["want"], c["src"]
    L = O.lib()
    assert [L.oracle_sign_extend_nibble(n) for n in range(16)] == ka["int4_sign_extend"]["want"]
    for c in ka["int4_unpack"]:
        assert O.unpack_to_i8(c["packed"], c["n"], c["k"])[1].tolist() == c["want"], c["src"]
    c = ka["int4_adversarial_cell"]
    st, out = O.igemm_s4s8_packed(np.full(c["m"] * c["k"], c["a"], np.int8),
                                  np.full(c["n"] * c["k"] // 2, c["weights_byte"], np.uint8),
                                  np.ones(c["n"] * c["k"] // c["group"], np.float32), c["group"], c["m"], c["k"], c["n"])
    assert np.all(out == c["want"])
    for c in ka["quantize_int8_f32"]:
        st, q, s = O.quantize_int8_f32(c["w"], c["n"], c["k"])
        assert q.tolist() == c["q"] and s.tolist() == c["scales"], c["src"]
    for c in ka["argmax_row"]:
        vals = [float(v) for v in c["logits"]]
        assert O.argmax_row(vals) == (0, c["want"]), c["src"]
    hid = np.zeros((1, 1280), np.float32)
    hid[0, 0] = 1.0
    gate = np.zeros((64, 1280), np.float32)
    for e, v in ka["route_top6"]["boost"].items():
        gate[int(e), 0] = v
    assert O.route(hid, gate, 64, 6)[1][0].tolist() == ka["route_top6"]["want"]


def test_selftest_vectors_reproduce():
    want = load("selftest_i32.npz")
    assert len(want) == 24
    for i in range(12):
        for unsigned in (False, True):
            label, m, k, n, seed, a, b = O.selftest_case(i, unsigned)
            f = O.igemm_u8s8 if unsigned else O.igemm_s8s8
            key = f"{'u8s8' if unsigned else 's8s8'}|{label}"
            assert np.array_equal(f(a, b, m, k, n), want[key]), key


def test_cfg1_fixture():
    d = load("cfg1_igemm_small.npz")
    M, N, K = int(d["M"]), int(d["N"]), int(d["K"])
    acc = O.igemm_s8s8(d["a"], d["w"], M, K, N)
    assert np.array_equal(acc, d["acc"])
    assert np.array_equal(acc.astype(np.int64), (d["a"].reshape(M, K).astype(np.int64) @
                                                 d["w"].reshape(N, K).astype(np.int64).T).reshape(-1))


def test_cfg2_fixture():
    d = load("cfg2_lmhead_small.npz")
    logits, am = O.lm_head_i8(d["x"], d["w"], d["s"], int(d["N"]), int(d["K"]))
    assert np.array_equal(logits, d["logits"]) and np.array_equal(am, d["argmax"])


def test_cfg3_fixture():
    d = load("cfg3_moe_small.npz")
    st, out, idx, gates = O.moe_decode(d["x"], d["router"], d["wg"], d["sg"], d["wu"], d["su"], d["wd"], d["sd"],
                                       int(d["E"]), int(d["K"]), int(d["I"]), norm_topk=True)
    assert st == 0 and np.array_equal(idx, d["idx"]) and np.array_equal(gates, d["gates"])
    assert np.array_equal(out, d["out"])


def test_cfg4_fixture():
    d = load("cfg4_int4_small.npz")
    m, k, n, g = (int(d[x]) for x in ("m", "k", "n", "group"))
    assert np.array_equal(O.igemm_s4s8_packed(d["a"], d["b"], d["s"], g, m, k, n)[1], d["out"])
    assert np.array_equal(O.s4s8_group_i32(d["a"], d["b"], g, m, k, n)[1], d["parts"])


def test_cfg5_fixture():
    d = load("cfg5_rswa_small.npz")
    Gr = int(d["G"])
    r = O.Ring(Gr)
    r.record_prefill(d["k"], d["v"], Gr)
    from franken_ocr_amd import synth

    slots = []
    for step in range(int(d["steps"])):
        slots.append(r.write(synth.f32_normal(synth.seed_of(9100 + step), 1280),
                             synth.f32_normal(synth.seed_of(9300 + step), 1280)))
    assert slots == d["slots"].tolist()
    st, out = r.attend(d["q"])
    assert np.array_equal(out, d["out"])


# ---- GPU: device path vs fixtures ---------------------------------------------------

def _rel_floored(got, want):
    """max |got - want| / max(|want|, 1% of the row's largest |want|): the GPU
    tests' relative-error rule (a pure relative error is meaningless for
    elements that a sum with cancellation leaves near zero)."""
    want = np.asarray(want, np.float64)
    floor = np.max(np.abs(want), axis=-1, keepdims=True) * 1e-2
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), floor)))


@pytest.mark.gpu
def test_gpu_matches_golden(ctx):
    from franken_ocr_amd import simd, synth
    from franken_ocr_amd.engine import MoeLayer, QInt8, RingCache, lm_head_i8

    print("[gpu-golden] selftest vectors", flush=True)
    want = load("selftest_i32.npz")
    for i in range(12):
        for unsigned in (False, True):
            label, m, k, n, seed, a, b = O.selftest_case(i, unsigned)
            got = np.zeros(m * n, np.int32)
            (simd.igemm_u8s8 if unsigned else simd.igemm_s8s8)(a, b, m, k, n, got, ctx)
            assert np.array_equal(got, want[f"{'u8s8' if unsigned else 's8s8'}|{label}"])

    print("[gpu-golden] cfg1", flush=True)
    d = load("cfg1_igemm_small.npz")
    M, N, K = int(d["M"]), int(d["N"]), int(d["K"])
    acc = np.zeros(M * N, np.int32)
    simd.igemm_s8s8(d["a"], d["w"], M, K, N, acc, ctx)
    assert np.array_equal(acc, d["acc"])

    print("[gpu-golden] cfg2", flush=True)
    d = load("cfg2_lmhead_small.npz")
    M, N, K = int(d["M"]), int(d["N"]), int(d["K"])
    q = QInt8(d["w"], d["s"], N, K, ctx)
    dl, da = ctx.empty((M, N), np.float32), ctx.empty((M,), np.uint32)
    lm_head_i8(q, ctx.to_device(d["x"]), da, dl)
    assert np.array_equal(dl.numpy(), d["logits"]) and np.array_equal(da.numpy(), d["argmax"])

    print("[gpu-golden] cfg3", flush=True)
    d = load("cfg3_moe_small.npz")
    T, H, I, E, Kk = (int(d[x]) for x in ("T", "H", "I", "E", "K"))
    L = MoeLayer(H, I, E, Kk, d["router"], d["wg"], d["sg"], d["wu"], d["su"], d["wd"], d["sd"], ctx=ctx)
    dout, didx, dg = ctx.empty((T, H), np.float32), ctx.empty((T, Kk), np.uint32), ctx.empty((T, Kk), np.float32)
    L.decode(ctx.to_device(d["x"]), dout, didx, dg, norm_topk=True)
    assert np.array_equal(didx.numpy(), d["idx"])
    np.testing.assert_allclose(dg.numpy(), d["gates"], rtol=1e-6)
    assert _rel_floored(dout.numpy(), d["out"]) <= 1e-3

    print("[gpu-golden] cfg4", flush=True)
    d = load("cfg4_int4_small.npz")
    m, k, n, g = (int(d[x]) for x in ("m", "k", "n", "group"))
    out = np.zeros(m * n, np.float32)
    simd.igemm_s4s8_packed(d["a"], d["b"], d["s"], g, m, k, n, out, ctx)
    assert np.array_equal(out, d["out"])
    assert np.array_equal(simd.s4s8_group_i32(d["a"], d["b"], g, m, k, n, ctx), d["parts"])

    print("[gpu-golden] cfg5", flush=True)
    d = load("cfg5_rswa_small.npz")
    Gr = int(d["G"])
    cache = RingCache(1, Gr, ctx)
    cache.record_prefill(0, ctx.to_device(d["k"]), ctx.to_device(d["v"]), Gr)
    slots = []
    for step in range(int(d["steps"])):
        ks = ctx.to_device(synth.f32_normal(synth.seed_of(9100 + step), 1280))
        vs = ctx.to_device(synth.f32_normal(synth.seed_of(9300 + step), 1280))
        slots += cache.write_decode_step(ks, vs)
    assert slots == d["slots"].tolist()
    assert cache.state(0) == (Gr, int(d["ring_len"]), int(d["ring_pos"]))
    dout = ctx.empty((1, 1280), np.float32)
    cache.decode_attention(ctx.to_device(d["q"]), dout)
    assert _rel_floored(dout.numpy(), d["out"].reshape(1, -1)) <= 1e-4
