"""The timed CPU baseline computes the reference's function (CPU only).

`oracle/cpu_tier.c` restates the reference's x86 int8 tiers (src/simd/x86.rs:
AVX2 :327-385, AVX-VNNI :549-616, AVX-512-VNNI :709-768, with the +128 S8S8
correction of `vpdpbusd`, :744-757) for the `cpu_baseline` bench leg. Every tier
this host can run is checked here against the scalar oracle
(`oracle_igemm_s8s8`, scalar.rs:78-116) on the self-test battery
(dispatch.rs:340-429) and the K = 6848 extremes, and the baseline's GEMV,
LM-head and MoE-decode compositions against the oracle's, so the number the
bench reports is the time of the same computation.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pyoracle as O

TIERS = [0, 1, 2, 3]  # scalar, avx2, avxvnni, avx512vnni (cpu_tier.h)


def _available():
    L = O.lib()
    return [t for t in TIERS if L.cpu_tier_available(t)]


def _tier_params():
    return [pytest.param(t, id=O.lib().cpu_tier_tag(t).decode()) for t in TIERS]


def _need(tier):
    if not O.lib().cpu_tier_available(tier):
        pytest.skip(f"host lacks {O.lib().cpu_tier_tag(tier).decode()}")


def _cpu_igemm(tier, a, b, m, k, n, out=None):
    out = np.zeros(m * n, np.int32) if out is None else out
    O.lib().cpu_igemm_s8s8(tier, O.p(np.ascontiguousarray(a, np.int8)), O.p(np.ascontiguousarray(b, np.int8)),
                           m, k, n, O.p(out))
    return out


def test_detected_tier_is_the_best_available():
    # dispatch.rs:179-200: avx512vnni > avxvnni > avx2 > scalar
    L = O.lib()
    assert L.cpu_detect_tier() == max(_available())
    assert L.cpu_tier_available(0) == 1


@pytest.mark.parametrize("tier", _tier_params())
def test_igemm_tier_selftest_battery(tier):
    _need(tier)
    for i in range(O.lib().oracle_selftest_n_shapes()):
        label, m, k, n, _, a, b = O.selftest_case(i)
        want = O.igemm_s8s8(a, b, m, k, n)
        got = _cpu_igemm(tier, a, b, m, k, n)
        assert np.array_equal(got, want), f"tier {tier} case {label}"


@pytest.mark.parametrize("tier", _tier_params())
@pytest.mark.parametrize("av,bv,want", [(127, 127, 110_451_392), (-128, -128, 112_197_632),
                                        (-128, 127, -111_321_088), (127, -128, -111_321_088)])
def test_igemm_tier_k6848_extremes(tier, av, bv, want):
    # scalar.rs:227-249 bounds; the +128 correction must not overflow at either sign
    _need(tier)
    K = 6848
    a = np.full(2 * K, av, np.int8)
    b = np.full(3 * K, bv, np.int8)
    got = _cpu_igemm(tier, a, b, 2, K, 3)
    assert (got == want).all()


@pytest.mark.parametrize("tier", _tier_params())
def test_igemm_tier_accumulates_and_tails(tier, rng):
    # out += A.B^T (scalar.rs:186-195); K tails below each tier's step (64/32/16)
    _need(tier)
    for m, k, n in [(1, 1, 1), (3, 17, 5), (2, 63, 3), (5, 129, 7), (4, 1280, 9), (1, 896, 6)]:
        a = rng.integers(-128, 128, m * k).astype(np.int8)
        b = rng.integers(-128, 128, n * k).astype(np.int8)
        seed = rng.integers(-1000, 1000, m * n).astype(np.int32)
        want = seed.astype(np.int64) + (a.reshape(m, k).astype(np.int64) @ b.reshape(n, k).astype(np.int64).T).ravel()
        got = _cpu_igemm(tier, a, b, m, k, n, seed.copy())
        assert np.array_equal(got.astype(np.int64), want), (m, k, n)


@pytest.mark.parametrize("tier", _tier_params())
def test_gemv_and_lm_head_tier_match_oracle(tier, rng):
    _need(tier)
    L = O.lib()
    n, k = 4096 + 37, 1280
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    for m in (1, 3):
        x = rng.standard_normal((m, k)).astype(np.float32)
        logits = np.zeros(m * n, np.float32)
        am = np.zeros(m, np.uint32)
        L.cpu_lm_head_i8(tier, O.p(x), m, O.p(w), O.p(s), n, k, O.p(logits), O.p(am))
        want_l, want_a = O.lm_head_i8(x, w, s, n, k)
        assert np.array_equal(logits.reshape(m, n), want_l) and np.array_equal(am, want_a)
        y = np.zeros(m * n, np.float32)
        L.cpu_gemv_i8(tier, O.p(x), m, O.p(w), O.p(s), n, k, O.p(y))
        assert np.array_equal(y.reshape(m, n), want_l)


@pytest.mark.parametrize("tier", _tier_params())
@pytest.mark.parametrize("h,inter,E,t", [(1280, 896, 16, 4), (200, 72, 8, 3)])
def test_moe_decode_tier_matches_oracle(tier, h, inter, E, t, rng):
    # the baseline's expert GEMVs run on the tier; the result must be the
    # oracle's decode_mlp_i8 (decoder.rs:2199-2268) bit for bit: same integer
    # sums, same f32 epilogue and slot-order combine
    _need(tier)
    K = 6
    router = (rng.standard_normal((E, h)) * 0.02).astype(np.float32)
    wg = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wu = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wd = rng.integers(-127, 128, E * h * inter).astype(np.int8)
    sg = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    su = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    sd = rng.uniform(1e-3, 2e-2, E * h).astype(np.float32)
    x = rng.standard_normal((t, h)).astype(np.float32)
    st, want, want_idx, want_g = O.moe_decode(x, router, wg, sg, wu, su, wd, sd, E, K, inter, norm_topk=True)
    assert st == 0
    out = np.zeros(t * h, np.float32)
    idx = np.zeros(t * K, np.uint32)
    gates = np.zeros(t * K, np.float32)
    st = O.lib().cpu_moe_decode(tier, O.p(x), t, h, inter, E, K, O.p(router), O.p(wg), O.p(sg), O.p(wu), O.p(su),
                                O.p(wd), O.p(sd), 1, 1.0, O.p(out), O.p(idx), O.p(gates))
    assert st == 0
    assert np.array_equal(idx.reshape(t, K), want_idx.reshape(t, K))
    assert np.array_equal(gates.reshape(t, K), want_g.reshape(t, K))
    assert np.array_equal(out.reshape(t, h), want.reshape(t, h))


@pytest.mark.parametrize("tier", _tier_params())
def test_igemm_batched_tier_matches_oracle(tier, rng):
    # cfg1 batched baseline: instance i is igemm_s8s8 on its own slices, out +=
    _need(tier)
    B, m, k, n = 5, 3, 1280, 70
    a = rng.integers(-127, 128, B * m * k).astype(np.int8)
    b = rng.integers(-127, 128, B * n * k).astype(np.int8)
    seed = rng.integers(-1000, 1000, B * m * n).astype(np.int32)
    got = seed.copy()
    O.lib().cpu_igemm_s8s8_batched(tier, O.p(a), O.p(b), B, m, k, n, O.p(got))
    for i in range(B):
        want = O.igemm_s8s8(a[i * m * k:(i + 1) * m * k], b[i * n * k:(i + 1) * n * k], m, k, n,
                            seed[i * m * n:(i + 1) * m * n].copy())
        assert np.array_equal(got[i * m * n:(i + 1) * m * n], want), i


@pytest.mark.parametrize("tier", _tier_params())
def test_linear_i8_dynamic_tier_matches_oracle(tier, rng):
    # the dynamic activation rule, the i32 products on the tier, the dequant order
    _need(tier)
    m, k, n = 37, 1280, 200
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3] = 0.0  # an all-zero row: scale 1.0
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    ws = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    y = np.zeros(m * n, np.float32)
    O.lib().cpu_linear_i8_dynamic(tier, O.p(x), m, k, O.p(w), O.p(ws), n, O.p(y))
    st, want, _, _ = O.linear_i8_dynamic(x, w, ws, n)
    assert st == 0 and np.array_equal(y.reshape(m, n), want)


def _moe_weights(rng, E, h, inter, si):
    wg, wu = (rng.integers(-127, 128, E * inter * h).astype(np.int8) for _ in range(2))
    wd = rng.integers(-127, 128, E * h * inter).astype(np.int8)
    sg, su = (rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32) for _ in range(2))
    sd = rng.uniform(1e-3, 2e-2, E * h).astype(np.float32)
    shared = (si, rng.integers(-127, 128, si * h).astype(np.int8), rng.uniform(1e-3, 2e-2, si).astype(np.float32),
              rng.integers(-127, 128, si * h).astype(np.int8), rng.uniform(1e-3, 2e-2, si).astype(np.float32),
              rng.integers(-127, 128, h * si).astype(np.int8), rng.uniform(1e-3, 2e-2, h).astype(np.float32))
    return wg, sg, wu, su, wd, sd, shared


@pytest.mark.parametrize("tier", _tier_params())
def test_moe_decode_shared_tier_matches_oracle(tier, rng):
    # decode_mlp_i8 with the shared expert: routed slots in slot order, shared last
    _need(tier)
    E, h, inter, si, K, t = 16, 1280, 896, 1792, 6, 3
    router = (rng.standard_normal((E, h)) * 0.02).astype(np.float32)
    wg, sg, wu, su, wd, sd, shared = _moe_weights(rng, E, h, inter, si)
    x = rng.standard_normal((t, h)).astype(np.float32)
    st, want, want_idx, _ = O.moe_decode(x, router, wg, sg, wu, su, wd, sd, E, K, inter, shared=shared)
    assert st == 0
    out = np.zeros(t * h, np.float32)
    idx = np.zeros(t * K, np.uint32)
    gates = np.zeros(t * K, np.float32)
    sh = [O.p(a) for a in shared[1:]]
    st = O.lib().cpu_moe_decode_shared(tier, O.p(x), t, h, inter, E, K, O.p(router), O.p(wg), O.p(sg), O.p(wu),
                                       O.p(su), O.p(wd), O.p(sd), 0, 1.0, *sh, si, O.p(out), O.p(idx), O.p(gates))
    assert st == 0
    assert np.array_equal(idx.reshape(t, K), want_idx)
    assert np.array_equal(out.reshape(t, h), want)


def test_decoder_layer_step_baseline_matches_oracle_composition(rng):
    # the decode-layer CPU baseline (C, on the best tier) is the oracle's
    # batched_decode_step_i8_streams layer (pyoracle.decoder_layer_step)
    L = O.lib()
    tier = L.cpu_detect_tier()
    B, G, h, E, K, inter, si = 3, 40, 1280, 8, 6, 896, 1792
    D = 1280
    router = (rng.standard_normal((E, h)) * 0.02).astype(np.float32)
    wg, sg, wu, su, wd, sd, shared = _moe_weights(rng, E, h, inter, si)
    wqkv = rng.integers(-127, 128, 3 * D * h).astype(np.int8)
    sqkv = rng.uniform(1e-3, 2e-2, 3 * D).astype(np.float32)
    wo = rng.integers(-127, 128, h * D).astype(np.int8)
    so = rng.uniform(1e-3, 2e-2, h).astype(np.float32)
    ln1, ln2 = (rng.uniform(0.5, 1.5, h).astype(np.float32) for _ in range(2))
    x = rng.standard_normal((B, h)).astype(np.float32)
    pos = np.array([G, G + 3, G + 7], np.uint32)
    rings = [O.Ring(G) for _ in range(B)]
    for s, r in enumerate(rings):
        r.record_prefill(rng.standard_normal(10 * G * 128).astype(np.float32),
                         rng.standard_normal(10 * G * 128).astype(np.float32), G)
        for _ in range(s * 5):  # rings at different fills
            r.write(rng.standard_normal(1280).astype(np.float32), rng.standard_normal(1280).astype(np.float32))
    # the C baseline works on copies of the same ring state
    import copy
    import ctypes as C

    crings = [copy.deepcopy(r) for r in rings]
    lw = {"input_ln": ln1, "post_ln": ln2, "qkv": (wqkv, sqkv), "o": (wo, so),
          "moe": {"router": router, "wg": wg, "sg": sg, "wu": wu, "su": su, "wd": wd, "sd": sd, "n_experts": E,
                  "top_k": K, "inter": inter, "shared": shared}}
    want = O.decoder_layer_step(x, pos, rings, lw)

    def arr(name):
        return (C.c_void_p * B)(*[getattr(r, name).ctypes.data for r in crings])

    got = x.copy()
    plen = np.array([r.prefill_len for r in crings], np.uint32)
    rlen = np.array([r.ring_len.value for r in crings], np.uint32)
    rpos = np.array([r.ring_pos.value for r in crings], np.uint32)
    st = L.cpu_decoder_layer_step(tier, O.p(got), B, O.p(pos), arr("ref_k"), arr("ref_v"), G, O.p(plen),
                                  arr("ring_k"), arr("ring_v"), O.p(rlen), O.p(rpos), O.p(ln1), O.p(ln2), 1e-6,
                                  10000.0, O.p(wqkv), O.p(sqkv), O.p(wo), O.p(so), O.p(router), E, K, inter, O.p(wg),
                                  O.p(sg), O.p(wu), O.p(su), O.p(wd), O.p(sd), *[O.p(a) for a in shared[1:]], si)
    assert st == 0
    assert np.array_equal(got, want)
    assert [int(v) for v in rlen] == [r.ring_len.value for r in rings]


@pytest.mark.parametrize("kind", [0, 1], ids=["packed_scalar", "unpack_then_int8"])
def test_int4_paths_match_oracle(kind, rng):
    # both x86 int4 paths of the reference (int4.rs:245-343) give the oracle's
    # f32 output bit for bit, at both group sizes and K tails of the AVX2 unpack
    L = O.lib()
    for group, m, k, n in [(32, 3, 1280, 17), (16, 2, 896, 9), (32, 1, 64 + 32, 5), (16, 4, 16, 3)]:
        a = rng.integers(-127, 128, m * k).astype(np.int8)
        bp = rng.integers(0, 256, n * k // 2).astype(np.uint8)
        s = rng.uniform(1e-3, 2e-2, n * (k // group)).astype(np.float32)
        got = np.zeros(m * n, np.float32)
        L.cpu_igemm_s4s8(kind, O.p(a), O.p(bp), O.p(s), group, m, k, n, O.p(got))
        st, want = O.igemm_s4s8_packed(a, bp, s, group, m, k, n)
        assert st == 0 and np.array_equal(got, want), (group, m, k, n)


@pytest.mark.parametrize("kind", [0, 1], ids=["packed_scalar", "unpack_then_int8"])
def test_int4_moe_prefill_baseline_matches_oracle(kind, rng):
    # the expert-gathered int4 MoE block equals the oracle's per-token one
    from franken_ocr_amd import synth

    L = O.lib()
    E, h, inter, K, t, group = 8, 1280, 896, 6, 12, 32
    wg, wu = (rng.integers(0, 256, E * inter * h // 2).astype(np.uint8) for _ in range(2))
    wd = rng.integers(0, 256, E * h * inter // 2).astype(np.uint8)
    sg, su = (rng.uniform(1e-3, 2e-2, E * inter * (h // group)).astype(np.float32) for _ in range(2))
    sd = rng.uniform(1e-3, 2e-2, E * h * (inter // group)).astype(np.float32)
    x = rng.standard_normal((t, h)).astype(np.float32)
    idx, gates = synth.zipf_routing(synth.seed_of(5), t, E, K)
    st, want, _, _ = O.moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter)
    assert st == 0
    out = np.zeros(t * h, np.float32)
    st = L.cpu_moe_prefill_i4(kind, O.p(x), t, h, inter, E, K, O.p(np.ascontiguousarray(idx)),
                              O.p(np.ascontiguousarray(gates)), group, O.p(wg), O.p(sg), O.p(wu), O.p(su), O.p(wd),
                              O.p(sd), O.p(out))
    assert st == 0 and np.array_equal(out.reshape(t, h), want)
