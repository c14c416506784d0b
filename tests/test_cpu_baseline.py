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
