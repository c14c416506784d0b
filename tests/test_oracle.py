"""Pin the CPU oracle before trusting it (CPU only).

Each test checks an oracle function against something other than its own
formula: the reference's known answers (file:line cited), integer brute
force in numpy int64, independent numpy restatements written from the spec
(as the reference's own int4 parity test does), closed forms, and float64
recomputations — chosen so a plausible mistake (wrong rounding mode, a
transposed operand, a dropped term, a wrong slot order) fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import pyoracle as O


# ---- igemm (src/simd/scalar.rs) -------------------------------------------------

def test_igemm_s8s8_hand_values():
    # scalar.rs:176-183 and simd/mod.rs:84-94
    out = O.igemm_s8s8([1, 2, 3, 4, 5, 6], [1, 0, 1, 0, 1, 0], 2, 3, 2)
    assert out.tolist() == [4, 2, 10, 5]


def test_igemm_accumulates():
    # scalar.rs:186-195: out is +=
    out = np.array([100], np.int32)
    O.igemm_s8s8([1, 2, 3], [1, 1, 1], 1, 3, 1, out)
    assert out.tolist() == [106]
    O.igemm_s8s8([1, 2, 3], [1, 1, 1], 1, 3, 1, out)
    assert out.tolist() == [112]


def test_igemm_u8s8_and_negatives():
    # scalar.rs:200-220
    assert O.igemm_u8s8([10, 20, 30], [2, -1, 1], 1, 3, 1).tolist() == [30]
    assert O.igemm_s8s8([-2, 3], [-1, -1, 4, -2], 1, 2, 2).tolist() == [-1, -14]


@pytest.mark.parametrize(
    "av,bv,unsigned,want",
    [
        (127, 127, False, 110_451_392),  # scalar.rs:227-236
        (-128, -128, False, 112_197_632),  # scalar.rs:240-249
        (255, 127, True, 221_772_480),  # scalar.rs:253-262
        (255, -128, True, -223_518_720),  # dispatch.rs:604-618 self-test extreme
    ],
)
def test_igemm_k6848_extremes(av, bv, unsigned, want):
    K = 6848
    a = np.full(K, av, np.uint8 if unsigned else np.int8)
    b = np.full(K, bv, np.int8)
    out = (O.igemm_u8s8 if unsigned else O.igemm_s8s8)(a, b, 1, K, 1)
    assert int(out[0]) == want


@pytest.mark.parametrize("m,k,n", [(3, 17, 5), (4, 13, 6), (5, 64, 7), (2, 1280, 9)])
def test_igemm_matches_i64_brute_force(m, k, n, rng):
    # scalar.rs:268-302 pattern: an independent i64 oracle
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, n * k).astype(np.int8)
    want = a.reshape(m, k).astype(np.int64) @ b.reshape(n, k).astype(np.int64).T
    assert np.array_equal(O.igemm_s8s8(a, b, m, k, n).reshape(m, n).astype(np.int64), want)
    au = rng.integers(0, 256, m * k).astype(np.uint8)
    want_u = au.reshape(m, k).astype(np.int64) @ b.reshape(n, k).astype(np.int64).T
    assert np.array_equal(O.igemm_u8s8(au, b, m, k, n).reshape(m, n).astype(np.int64), want_u)


# ---- self-test battery (src/simd/dispatch.rs:340-429) ----------------------------

def _xs32_stream(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint32)
    s = seed
    for i in range(count):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s
    return out


def test_selftest_shapes_and_fills_regenerate_independently():
    L = O.lib()
    assert L.oracle_selftest_n_shapes() == 12  # dispatch.rs:352-368 (24 cases with both domains)
    labels = []
    for i in range(12):
        label, m, k, n, seed, a, b = O.selftest_case(i)
        labels.append(label)
        _, _, _, _, _, au, bu = O.selftest_case(i, unsigned=True)
        if seed == 0:
            assert (a == 127).all() and (b == -128).all() and (au == 255).all() and (bu == -128).all()
            continue
        if m * k + n * k <= 200_000:
            st = _xs32_stream(seed | 1, m * k + n * k)
            assert np.array_equal(a.view(np.uint8), (st[: m * k] & 0xFF).astype(np.uint8))
            assert np.array_equal(b.view(np.uint8), (st[m * k :] & 0xFF).astype(np.uint8))
            rot = ((seed << 7) | (seed >> 25)) & 0xFFFFFFFF
            su = _xs32_stream(rot | 1, m * k + n * k)
            assert np.array_equal(au, (su[: m * k] & 0xFF).astype(np.uint8))
    assert labels[0] == "edge:1x1x1" and labels[-1] == "overflow:max_mag_k6848"


# ---- quantizers (decoder.rs:1588-1597 / :1647-1656) ---------------------------------

def _np_quant(x: np.ndarray, ties_even: bool):
    x = np.asarray(x, np.float32)
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
    scale = np.float32(amax / np.float32(127)) if amax > 0 else np.float32(1)
    inv = np.float32(np.float32(1) / scale)
    v = (x * inv).astype(np.float64)
    r = np.rint(v) if ties_even else np.sign(v) * np.floor(np.abs(v) + 0.5)
    return np.clip(r, -127, 127).astype(np.int8), scale


def test_quantize_row_rounding_modes_split():
    # scale forced to 1 by the 127; the .5 ties separate the two rules
    row = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    q, s = O.quantize_row_i8(row)
    assert s == 1.0 and q.tolist() == [127, 1, 2, 3, -1, -2, -3]  # f32::round: half away
    q, s = O.quantize_row_i8(row, ties_even=True)
    assert q.tolist() == [127, 0, 2, 2, 0, -2, -2]  # round_ties_even (nn.rs:600-628 style)


def test_quantize_row_zero_and_scale():
    q, s = O.quantize_row_i8([0.0, -0.0, 0.0])
    assert s == 1.0 and q.tolist() == [0, 0, 0]  # amax == 0 -> scale 1.0 (decoder.rs:1590)
    q, s = O.quantize_row_i8([254.0, -2.0, 100.0])
    assert s == 2.0 and q.tolist() == [127, -1, 50]


@pytest.mark.parametrize("ties_even", [False, True])
def test_quantize_row_matches_numpy_restatement(ties_even, rng):
    for k in (1, 7, 896, 1280):
        x = (rng.standard_normal(k) * rng.uniform(0.01, 10)).astype(np.float32)
        q, s = O.quantize_row_i8(x, ties_even)
        wq, ws = _np_quant(x, ties_even)
        assert s == ws and np.array_equal(q, wq)


def test_gemv_dequant_order(rng):
    # y = ((f32)acc * a_scale) * w_scale, left to right (decoder.rs:1636)
    n, k = 37, 64
    x = rng.standard_normal((3, k)).astype(np.float32)
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    sc = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    y, acc, xq, a_s = O.gemv_i8_batched(x, w, sc, n, k)
    want_acc = xq.astype(np.int64) @ w.reshape(n, k).astype(np.int64).T
    assert np.array_equal(acc.astype(np.int64), want_acc)
    want = (acc.astype(np.float32) * a_s[:, None]).astype(np.float32) * sc[None, :]
    assert np.array_equal(y, want.astype(np.float32))
    # the other association order differs somewhere (so the test has teeth)
    other = acc.astype(np.float32) * (a_s[:, None] * sc[None, :])
    assert not np.array_equal(y, other)


# ---- argmax (sampler.rs:168-186) ------------------------------------------------------

def test_argmax_known_answers():
    assert O.argmax_row([0.1, -2.0, 3.5, 3.4, 0.0]) == (0, 2)  # sampler.rs:618-621
    assert O.argmax_row([0.0, 5.0, 1.0, 5.0]) == (0, 1)  # ties -> lowest index, :624-634
    assert O.argmax_row([np.nan, -np.inf, 2.0, 1.0]) == (0, 2)  # NaN skipped, :637-645
    assert O.argmax_row([np.nan, np.nan]) == (0, 0)  # all NaN -> 0 (sampler.rs:184)
    assert O.argmax_row([-np.inf, -np.inf]) == (0, 0)
    assert O.argmax_row([-0.0, 0.0]) == (0, 0)  # -0 == +0: first wins
    assert O.argmax_row([])[0] != 0  # empty row is an error


def test_argmax_random_vs_numpy(rng):
    for _ in range(20):
        v = rng.standard_normal(1000).astype(np.float32)
        v[rng.integers(0, 1000, 5)] = np.nan
        v[rng.integers(0, 1000, 3)] = np.nanmax(v)
        assert O.argmax_row(v) == (0, int(np.nanargmax(v)))


# ---- router (moe.rs:181-266) ------------------------------------------------------------

def _route_gate_with_col0(logits_by_expert: dict, h: int = 1280, E: int = 64):
    hid = np.zeros((1, h), np.float32)
    hid[0, 0] = 1.0
    gate = np.zeros((E, h), np.float32)
    for e, v in logits_by_expert.items():
        gate[e, 0] = v
    return hid, gate


def test_route_known_answer_greedy_top6():
    # moe.rs:777-820: experts 10..15 with logits 10..5 -> indices [10..15]
    hid, gate = _route_gate_with_col0({10: 10.0, 11: 9.0, 12: 8.0, 13: 7.0, 14: 6.0, 15: 5.0})
    st, idx, w, probs = O.route(hid, gate, 64, 6)
    assert st == 0 and idx[0].tolist() == [10, 11, 12, 13, 14, 15]
    ex = np.exp(np.array([10, 9, 8, 7, 6, 5], np.float64) - 10.0)
    den = ex.sum() + 58 * math.exp(-10.0)
    np.testing.assert_allclose(w[0], ex / den, rtol=1e-6)
    assert float(w[0].sum()) < 1.0  # raw softmax probs (norm_topk_prob = false)
    assert np.all(np.diff(w[0]) < 0)


def test_route_renorm_and_scaling():
    hid, gate = _route_gate_with_col0({10: 10.0, 11: 9.0, 12: 8.0, 13: 7.0, 14: 6.0, 15: 5.0})
    _, _, w, _ = O.route(hid, gate, 64, 6, norm_topk=True)
    assert abs(float(w[0].astype(np.float64).sum()) - 1.0) < 1e-5 and np.all(np.diff(w[0]) < 0)
    _, _, w1, _ = O.route(hid, gate, 64, 6)
    _, _, w25, _ = O.route(hid, gate, 64, 6, routed_scale=2.5)
    np.testing.assert_allclose(w25, w1 * np.float32(2.5), rtol=1e-6)


def test_route_uniform_ties_pick_lowest_indices():
    # all-zero gate -> uniform softmax -> experts 0..5 at 1/64 each (moe.rs:938-980)
    hid = np.ones((1, 8), np.float32)
    gate = np.zeros((64, 8), np.float32)
    st, idx, w, _ = O.route(hid, gate, 64, 6)
    assert st == 0 and idx[0].tolist() == [0, 1, 2, 3, 4, 5]
    assert np.all(w == np.float32(1 / 64))


def test_route_nan_is_an_error():
    # moe.rs:261-265 "no finite router score"
    hid = np.full((1, 8), np.nan, np.float32)
    gate = np.ones((64, 8), np.float32)
    st, *_ = O.route(hid, gate, 64, 6)
    assert st == -7


def test_route_matches_float64_restatement(rng):
    t, h, E = 16, 1280, 64
    hid = rng.standard_normal((t, h)).astype(np.float32)
    gate = (rng.standard_normal((E, h)) * 0.02).astype(np.float32)
    st, idx, w, probs = O.route(hid, gate, E, 6, norm_topk=True)
    assert st == 0
    logits = (hid.astype(np.float64) @ gate.astype(np.float64).T).astype(np.float32)
    z = logits.astype(np.float64)
    ex = np.exp(z - z.max(axis=1, keepdims=True))
    p = (ex / ex.sum(axis=1, keepdims=True)).astype(np.float32)
    np.testing.assert_allclose(probs, p, rtol=1e-6, atol=0)
    for r in range(t):
        order = sorted(range(E), key=lambda e: (-float(p[r, e]), e))[:6]
        assert idx[r].tolist() == order


# ---- SwiGLU expert / MoE decode (decoder.rs:1744-1755, :2199-2268) -------------------

def test_silu_values():
    L = O.lib()
    assert abs(L.oracle_silu(2.0) - 2.0 / (1.0 + math.exp(-2.0))) < 1e-6
    assert L.oracle_silu(0.0) == 0.0


def test_moe_identity_experts_known_answer():
    # moe.rs:938-980: identity SwiGLU experts, uniform gate -> 6/64 * silu(1).
    # The int8 weights of I (2x2) quantize to 127 on the diagonal, scale 1/127.
    h, inter, E = 2, 2, 64
    eye = np.array([127, 0, 0, 127], np.int8)
    wg = np.tile(eye, E)
    s = np.full(E * 2, np.float32(1.0) / np.float32(127.0), np.float32)
    hid = np.ones((1, h), np.float32)
    router = np.zeros((E, h), np.float32)
    st, out, idx, gates = O.moe_decode(hid, router, wg, s, wg, s, wg, s, E, 6, inter)
    assert st == 0 and idx[0].tolist() == [0, 1, 2, 3, 4, 5]
    silu1 = 1.0 / (1.0 + math.exp(-1.0))
    np.testing.assert_allclose(out[0], 6.0 / 64 * silu1, rtol=1e-5)


def test_expert_i32_accumulators_and_float64_check(rng):
    h, inter = 64, 48
    x = rng.standard_normal(h).astype(np.float32)
    wg = rng.integers(-127, 128, inter * h).astype(np.int8)
    wu = rng.integers(-127, 128, inter * h).astype(np.int8)
    wd = rng.integers(-127, 128, h * inter).astype(np.int8)
    sg = rng.uniform(1e-3, 2e-2, inter).astype(np.float32)
    su = rng.uniform(1e-3, 2e-2, inter).astype(np.float32)
    sd = rng.uniform(1e-3, 2e-2, h).astype(np.float32)
    y, act, aq, as2 = O.expert_i8(x, h, inter, wg, sg, wu, su, wd, sd)
    xq, xs = _np_quant(x, False)
    g = xq.astype(np.int64) @ wg.reshape(inter, h).astype(np.int64).T
    u = xq.astype(np.int64) @ wu.reshape(inter, h).astype(np.int64).T
    g64 = g * float(xs) * sg.astype(np.float64)
    u64 = u * float(xs) * su.astype(np.float64)
    act64 = g64 / (1 + np.exp(-g64)) * u64
    np.testing.assert_allclose(act, act64, rtol=1e-5, atol=1e-7)
    wq, ws = _np_quant(act, False)
    assert np.array_equal(aq, wq) and as2 == ws
    d = aq.astype(np.int64) @ wd.reshape(h, inter).astype(np.int64).T
    np.testing.assert_allclose(y, d * float(as2) * sd.astype(np.float64), rtol=1e-6)


def test_moe_decode_combine_slot_order(rng):
    # out = ((0 + y0*w0) + y1*w1) ... in slot order; check vs float64 sum and
    # that every token's output is the gate-weighted sum of its experts.
    h, inter, E, t = 32, 32, 8, 3
    router = (rng.standard_normal((E, h)) * 0.5).astype(np.float32)
    wg = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wu = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wd = rng.integers(-127, 128, E * h * inter).astype(np.int8)
    sg = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    su = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    sd = rng.uniform(1e-3, 2e-2, E * h).astype(np.float32)
    hid = rng.standard_normal((t, h)).astype(np.float32)
    st, out, idx, gates = O.moe_decode(hid, router, wg, sg, wu, su, wd, sd, E, 4, inter, norm_topk=True)
    assert st == 0
    for r in range(t):
        acc32 = np.zeros(h, np.float32)
        acc64 = np.zeros(h, np.float64)
        for j in range(4):
            e = int(idx[r, j])
            y, *_ = O.expert_i8(hid[r], h, inter, wg[e * inter * h:(e + 1) * inter * h], sg[e * inter:(e + 1) * inter],
                                wu[e * inter * h:(e + 1) * inter * h], su[e * inter:(e + 1) * inter],
                                wd[e * h * inter:(e + 1) * h * inter], sd[e * h:(e + 1) * h])
            acc32 = (acc32 + (y * gates[r, j]).astype(np.float32)).astype(np.float32)
            acc64 += y.astype(np.float64) * float(gates[r, j])
        assert np.array_equal(out[r], acc32)
        np.testing.assert_allclose(out[r], acc64, rtol=1e-5, atol=1e-7)


# ---- int4 (src/simd/int4.rs) -------------------------------------------------------------

def test_int4_sign_extension_table():
    # int4.rs:660-670
    L = O.lib()
    want = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]
    assert [L.oracle_sign_extend_nibble(n) for n in range(16)] == want


def test_int4_unpack_fixtures():
    # int4.rs:676-696
    for byte, lo_hi in [(0x21, [1, 2]), (0x43, [3, 4]), (0x87, [7, -8]), (0xF0, [0, -1]), (0x00, [0, 0]),
                        (0x88, [-8, -8])]:
        assert O.unpack_to_i8([byte], 1, 2)[1].tolist() == lo_hi
    assert O.unpack_to_i8([0x21, 0x43, 0x65, 0x87], 2, 4)[1].tolist() == [1, 2, 3, 4, 5, 6, 7, -8]
    assert O.unpack_to_i8([0x21], 1, 3)[0] != 0  # odd k rejected


def _spec_s4s8(a, packed, scales, group, m, k, n):
    """Independent restatement from the packing spec (int4.rs:775-810 pattern)."""
    b = np.zeros((n, k), np.int64)
    pk = packed.reshape(n, k // 2).astype(np.int64)
    lo = pk & 0xF
    hi = pk >> 4
    b[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    b[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    A = a.reshape(m, k).astype(np.int64)
    G = k // group
    parts = np.einsum("mgk,ngk->mng", A.reshape(m, G, group), b.reshape(n, G, group))
    out = np.zeros((m, n), np.float32)
    sc = scales.reshape(n, G)
    for g in range(G):
        out = (out + (sc[None, :, g] * parts[:, :, g].astype(np.float32)).astype(np.float32)).astype(np.float32)
    return out.reshape(-1), parts.reshape(-1)


@pytest.mark.parametrize("m,k,n,group", [(1, 16, 1, 16), (2, 32, 3, 16), (4, 64, 5, 32), (3, 96, 2, 16),
                                         (2, 128, 7, 32), (5, 1280, 9, 32)])
def test_int4_matches_spec_oracle(m, k, n, group, rng):
    a = rng.integers(-127, 128, m * k).astype(np.int8)
    packed = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    scales = rng.uniform(-1, 1, n * (k // group)).astype(np.float32)
    st, out = O.igemm_s4s8_packed(a, packed, scales, group, m, k, n)
    want, parts = _spec_s4s8(a, packed, scales, group, m, k, n)
    assert st == 0 and np.array_equal(out, want)
    st, got_parts = O.s4s8_group_i32(a, packed, group, m, k, n)
    assert st == 0 and np.array_equal(got_parts.astype(np.int64), parts)


def test_int4_adversarial_known_answers():
    # int4.rs:853-892: all -8 weights; +/-127 alternating -> 0.0; all -127 -> 32,512 per cell
    m, k, n, g = 2, 32, 3, 16
    packed = np.full(n * k // 2, 0x88, np.uint8)
    scales = np.ones(n * (k // g), np.float32)
    alt = np.array([127 if i % 2 == 0 else -127 for i in range(m * k)], np.int8)
    assert np.all(O.igemm_s4s8_packed(alt, packed, scales, g, m, k, n)[1] == 0.0)
    assert np.all(O.igemm_s4s8_packed(np.full(m * k, -127, np.int8), packed, scales, g, m, k, n)[1] == 32512.0)


def test_int4_single_group_equals_int8_per_channel(rng):
    # int4.rs:901-925: group == k == 16 collapses to per-channel int8
    m, k, n = 3, 16, 4
    a = rng.integers(-127, 128, m * k).astype(np.int8)
    packed = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    scales = np.array([0.0625 + i * 0.03125 for i in range(n)], np.float32)
    _, out = O.igemm_s4s8_packed(a, packed, scales, 16, m, k, n)
    _, b = O.unpack_to_i8(packed, n, k)
    acc = O.igemm_s8s8(a, b, m, k, n).reshape(m, n)
    assert np.array_equal(out.reshape(m, n), (scales[None, :] * acc.astype(np.float32)).astype(np.float32))


def test_int4_shape_rejections():
    a = np.ones(32, np.int8)
    assert O.igemm_s4s8_packed(a, np.zeros(16, np.uint8), np.ones(4, np.float32), 8, 1, 32, 1)[0] != 0  # int4.rs:928
    assert O.igemm_s4s8_packed(np.ones(24, np.int8), np.zeros(12, np.uint8), np.ones(2, np.float32), 16, 1, 24, 1)[0] != 0


# ---- weight quantizers (src/quant) ---------------------------------------------------------

def test_quantize_int8_known_answers():
    # quant/int8.rs:300-366
    assert O.quantize_int8_f32([127.0, -127.0, 0.0, 64.0], 1, 4)[1:] and True
    st, q, s = O.quantize_int8_f32([127.0, -127.0, 0.0, 64.0], 1, 4)
    assert s.tolist() == [1.0] and q.tolist() == [127, -127, 0, 64]
    st, q, s = O.quantize_int8_f32([254.0, -2.0, 100.0], 1, 3)
    assert s.tolist() == [2.0] and q.tolist() == [127, -1, 50]
    st, q, s = O.quantize_int8_f32([127.0, 0.0, -64.0, 254.0, -254.0, 0.0], 2, 3)
    assert s.tolist() == [1.0, 2.0] and q.tolist() == [127, 0, -64, 127, -127, 0]
    st, q, s = O.quantize_int8_f32([0.0, 0.0, -0.0, 0.0], 1, 4)
    assert s.tolist() == [1.0] and q.tolist() == [0, 0, 0, 0]
    st, q, s = O.quantize_int8_f32([127.0, 0.5, 1.5, 2.5], 1, 4)
    assert q.tolist() == [127, 0, 2, 2]
    st, q, s = O.quantize_int8_f32([-127.0, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 127.0], 1, 8)
    assert q.tolist() == [-127, -2, -2, 0, 0, 2, 2, 127]
    st, q, s = O.quantize_int8_f32([-1000.0, 1000.0], 1, 2)
    assert q.tolist() == [-127, 127]


def _pack_codes(w, n, k, g):
    st, packed, s = O.pack_int4_f32(np.asarray(w, np.float32), n, k, g)
    assert st == 0
    return packed, s, O.unpack_to_i8(packed, n, k)[1]


def test_pack_int4_known_answers():
    # quant/int4.rs:344-360 exact_int4_values_roundtrip_with_unit_scale
    vals = [7.0, -7.0, 0.0, 1.0, -1.0, 3.0, -3.0, 6.0, -6.0, 2.0, -2.0, 4.0, -4.0, 5.0, -5.0, 7.0]
    packed, s, codes = _pack_codes(vals, 1, 16, 16)
    assert s.tolist() == [1.0] and codes.tolist() == [int(v) for v in vals]
    # :362-373 packed_and_scale_counts_match_layout
    packed, s, _ = _pack_codes(np.ones(64), 2, 32, 16)
    assert packed.size == 32 and s.size == 4
    assert _pack_codes(np.ones(64), 2, 32, 32)[1].size == 2
    # :375-390 per_group_scales_are_independent: -7/2 = -3.5 -> ties-even -> -4
    w = np.zeros(32, np.float32)
    w[0], w[16], w[17] = 7.0, 14.0, -7.0
    _, s, codes = _pack_codes(w, 1, 32, 16)
    assert s.tolist() == [1.0, 2.0] and (codes[0], codes[16], codes[17]) == (7, 7, -4)
    # :392-399 all_zero_group_unit_scale_no_nan
    _, s, codes = _pack_codes(np.zeros(16), 1, 16, 16)
    assert s.tolist() == [1.0] and not codes.any()
    # :401-414 clamps: 16/(16/7) -> 7, -16/(16/7) -> -7
    w = np.zeros(16, np.float32)
    w[0], w[1] = 16.0, -16.0
    _, s, codes = _pack_codes(w, 1, 16, 16)
    assert (codes[0], codes[1]) == (7, -7) and codes.min() >= -8 and codes.max() <= 7
    # :425-439 unpack_is_exact_inverse_of_pack_nibbles: low nibble = even column
    vals = [-8.0, 7.0, -1.0, 1.0, -8.0, -8.0, 7.0, 7.0, 0.0, 0.0, -4.0, 4.0, -2.0, 2.0, -6.0, 6.0]
    packed, _, codes = _pack_codes(vals, 1, 16, 16)
    for j in range(8):
        assert packed[j] == ((int(codes[2 * j]) & 0xF) | ((int(codes[2 * j + 1]) & 0xF) << 4))
    # :441-455 multi_row_packing_indexes_rows_correctly: -8/(8/7) = -7
    w = np.concatenate([np.full(16, 7.0), np.full(16, -8.0)])
    _, s, codes = _pack_codes(w, 2, 16, 16)
    assert (codes[:16] == 7).all() and (codes[16:] == -7).all()
    assert s[0] == 1.0 and s[1] == np.float32(8.0) / np.float32(7.0)
    # ties at unit scale split the rounding rules: 2.5 -> 2 and 0.5 -> 0 (ties-even),
    # where half-away-from-zero would give 3 and 1
    w = np.zeros(16, np.float32)
    w[:6] = [7.0, 2.5, 0.5, -0.5, -2.5, 1.5]
    _, _, codes = _pack_codes(w, 1, 16, 16)
    assert codes[:6].tolist() == [7, 2, 0, 0, -2, 2]
    assert O.pack_int4_f32(np.zeros(16, np.float32), 1, 16, 8)[0] != 0  # :459 "must be 16 or 32"
    assert O.pack_int4_f32(np.zeros(24, np.float32), 1, 24, 16)[0] != 0  # :465 "must divide k"


def _np_pack_int4(w, n, k, g):
    """pack_int4_f32 restated from its documented contract (int4.rs:130-205):
    scale = max|group| / 7 (1.0 for an all-zero group), q = clamp(RNE(w / scale)
    with true f32 division, -8, 7), low nibble = even column."""
    w = np.asarray(w, np.float32).reshape(n, k // g, g)
    mx = np.abs(w).max(axis=2)
    s = np.where(mx == 0, np.float32(1), (mx / np.float32(7)).astype(np.float32)).astype(np.float32)
    q = np.clip(np.rint((w / s[:, :, None]).astype(np.float32)), -8, 7).astype(np.int64).reshape(n, k)
    nib = q & 0xF
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8).reshape(-1), s.reshape(-1)


def _planted_division_ties(rng, count):
    """Groups whose values sit exactly on a .5 code boundary under true division
    but not under a reciprocal multiply (w * (1/s)): a reciprocal-multiply
    packer gives a different code for at least one of them."""
    found = []
    while len(found) < count:
        mx = np.float32(rng.uniform(0.5, 40.0))
        s = np.float32(mx / np.float32(7))
        inv = np.float32(np.float32(1) / s)
        for c in range(-7, 7):
            x = np.float32((c + 0.5) * s)
            if np.float32(x / s) == np.float32(c + 0.5) and np.rint(np.float32(x * inv)) != np.rint(np.float32(x / s)):
                found.append((mx, x))
                break
    return found


@pytest.mark.parametrize("n,k,g", [(3, 64, 32), (5, 96, 16), (7, 1280, 32), (4, 896, 32)])
def test_pack_int4_matches_numpy_restatement(n, k, g, rng):
    w = (rng.standard_normal(n * k) * rng.uniform(0.01, 3.0)).astype(np.float32)
    # plant exact .5 ties at unit scale (group max 7) and division-only ties in
    # further groups, plus one all-zero group
    w[:g] = 0.0
    w[0], w[1], w[2] = 7.0, 2.5, -0.5
    for i, (mx, x) in enumerate(_planted_division_ties(rng, 2)):
        base = (i + 1) * g
        w[base:base + g] = 0.0
        w[base], w[base + 1] = mx, x
    if n * k // g > 3:
        w[3 * g:4 * g] = 0.0
    st, packed, s = O.pack_int4_f32(w, n, k, g)
    want_p, want_s = _np_pack_int4(w, n, k, g)
    assert st == 0 and np.array_equal(s, want_s) and np.array_equal(packed, want_p)
    # the planted cases discriminate: half-away or reciprocal rounding packs differently
    grp = w.reshape(-1, g)
    sc = want_s.reshape(-1)
    half_away = np.clip(np.sign(grp / sc[:, None]) * np.floor(np.abs(grp / sc[:, None]) + 0.5), -8, 7)
    recip = np.clip(np.rint(grp * (np.float32(1) / sc)[:, None].astype(np.float32)), -8, 7)
    codes = O.unpack_to_i8(packed, n, k)[1].reshape(-1, g)
    assert not np.array_equal(codes, half_away) and not np.array_equal(codes, recip)
    # and the dequantized codes stay within half a step of the input
    deq = codes.astype(np.float32) * sc[:, None]
    assert np.all(np.abs(deq - grp) <= sc[:, None] * (0.5 + 1e-6))


# ---- R-SWA ring + attention (src/native_engine/rswa.rs) ------------------------------------

H, D, W = 10, 128, 128


def test_attention_single_key_returns_value():
    # rswa.rs:1475-1488
    r = O.Ring(8)
    k = np.zeros((H, 1, D), np.float32)
    k[:, :, 0] = 1.0
    r.record_prefill(k, np.full((H, 1, D), 7.0, np.float32), 1)
    q = np.zeros((H, D), np.float32)
    q[:, 0] = 5.0
    st, out = r.attend(q)
    assert st == 0 and np.allclose(out, 7.0, atol=1e-5)


def test_attention_equal_scores_average():
    # rswa.rs:1493-1507
    r = O.Ring(8)
    k = np.zeros((H, 2, D), np.float32)
    k[:, :, 0] = 1.0
    v = np.zeros((H, 2, D), np.float32)
    v[:, 0] = 2.0
    v[:, 1] = 4.0
    r.record_prefill(k, v, 2)
    q = np.zeros((H, D), np.float32)
    q[:, 0] = 3.0
    st, out = r.attend(q)
    assert np.allclose(out, 3.0, atol=1e-5)


def test_attention_online_matches_float64_softmax(rng):
    # rswa.rs:1511-1553 (online == naive) at a ring-wrapped random state
    cap, seq = 64, 50
    r = O.Ring(cap)
    k = rng.standard_normal((H, seq, D)).astype(np.float32)
    v = rng.standard_normal((H, seq, D)).astype(np.float32)
    r.record_prefill(k, v, seq)
    steps = 150  # wraps past W = 128
    for _ in range(steps):
        r.write(rng.standard_normal(H * D).astype(np.float32), rng.standard_normal(H * D).astype(np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    st, out = r.attend(q)
    assert st == 0
    keys = np.concatenate([r.ref_k[:, :seq], r.ring_k[:, : r.ring_len.value]], axis=1).astype(np.float64)
    vals = np.concatenate([r.ref_v[:, :seq], r.ring_v[:, : r.ring_len.value]], axis=1).astype(np.float64)
    sc = np.einsum("hd,hkd->hk", q.astype(np.float64), keys) / math.sqrt(128.0)
    p = np.exp(sc - sc.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    want = np.einsum("hk,hkd->hd", p, vals).reshape(-1)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)


def test_ring_write_regimes():
    # rswa.rs:1557-1613: warm-up appends in order, ring_pos tracks ring_len and
    # wraps to 0 when full; steady state overwrites slots 0, 1, ... modulo W
    r = O.Ring(4)
    r.record_prefill(np.zeros((H, 2, D), np.float32), np.zeros((H, 2, D), np.float32), 2)
    z = np.zeros(H * D, np.float32)
    for step in range(W):
        assert r.write(z, z) == step
        assert r.ring_len.value == step + 1
    assert r.ring_pos.value == 0
    kt = np.full(H * D, 99.0, np.float32)
    assert r.write(kt, kt) == 0 and r.ring_pos.value == 1
    assert r.write(kt, kt) == 1 and r.ring_pos.value == 2
    assert r.ring_len.value == W and r.ring_k[0, 0, 0] == 99.0
    for expected in range(2, W + 3):
        assert r.write(z, z) == expected % W


def test_attention_empty_key_set_is_error():
    r = O.Ring(4)
    r.record_prefill(np.zeros((H, 0, D), np.float32), np.zeros((H, 0, D), np.float32), 0)
    st, _ = r.attend(np.zeros(H * D, np.float32))
    assert st != 0


# ---- prefill int8 linear (nn::linear_int8_dynamic) and moe_block_i8 --------------------

def test_linear_i8_dynamic_known_answers():
    # nn.rs:549-556: x=[[1,2,3]], W=[[1,0,1],[0,1,0]] quantized per channel -> y ~ [4, 2]
    st, wq, ws = 0, np.zeros(6, np.int8), np.zeros(2, np.float32)
    assert O.lib().oracle_quantize_int8_f32(O.p(np.array([1, 0, 1, 0, 1, 0], np.float32)), 2, 3, O.p(wq),
                                            O.p(ws)) == 0
    st, y, _, _ = O.linear_i8_dynamic(np.array([[1, 2, 3]], np.float32), wq, ws, 2)
    assert st == 0 and abs(y[0, 0] - 4.0) < 0.1 and abs(y[0, 1] - 2.0) < 0.1
    # nn.rs:601-628: ties round to even (a half-away quantizer gives [1, 3])
    x = np.array([[-127, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 127], [0] * 8], np.float32)
    w = np.array([[0, 0, 0, 0, 1, 0, 0, 0], [0, 0, 0, 0, 0, 0, 1, 0]], np.int8)
    st, y, xq, xs = O.linear_i8_dynamic(x, w, np.ones(2, np.float32), 2)
    assert st == 0 and y.ravel().tolist() == [0.0, 2.0, 0.0, 0.0]
    assert xq[0].tolist() == [-127, -2, -2, 0, 0, 2, 2, 127] and xs.tolist() == [1.0, 1.0]  # all-zero row: 1.0
    st, y2, _, _ = O.linear_i8_dynamic(x, w, np.ones(2, np.float32), 2)
    assert np.array_equal(y, y2)


def test_quantize_row_dynamic_is_true_division(rng):
    # docs/focrq-format.md:296-320: q = round_ties_even(clamp(x / scale)), true
    # division. Find rows where x * (1/scale) rounds differently from x / scale
    # and check the oracle takes the division.
    hits = 0
    for _ in range(400):
        x = rng.standard_normal(256).astype(np.float32)
        s = np.float32(np.abs(x).max()) / np.float32(127.0)
        # plant exact ties x = (k + 0.5) * s (rounded to f32) so the two rules can split
        k = rng.integers(-120, 120, 32)
        x[:32] = ((k + 0.5).astype(np.float32) * s).astype(np.float32)
        x[32] = np.float32(127.0) * s  # keep amax (and so s) fixed
        s = np.float32(np.abs(x).max()) / np.float32(127.0)
        div = np.rint(np.clip(x / s, -127, 127)).astype(np.int8)
        rec = np.rint(np.clip(x * (np.float32(1.0) / s), -127, 127)).astype(np.int8)
        q, qs = O.quantize_row_dynamic(x)
        assert qs == s and np.array_equal(q, div)
        hits += int((div != rec).any())
    assert hits > 0, "no row separated true division from a reciprocal multiply"


@pytest.mark.parametrize("m,k,n", [(1, 16, 8), (7, 64, 33), (64, 1280, 96)])
def test_linear_i8_dynamic_vs_int64_and_float64(m, k, n, rng):
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    x[0, :5] = 0.0
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    ws = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    st, y, xq, xs = O.linear_i8_dynamic(x, w, ws, n, bias=b)
    assert st == 0
    for r in range(m):
        q, s = O.quantize_row_dynamic(x[r])
        assert np.array_equal(xq[r], q) and xs[r] == s
    acc = xq.astype(np.int64) @ w.reshape(n, k).astype(np.int64).T  # |acc| < 2^31 here
    want = acc * xs.astype(np.float64)[:, None] * ws.astype(np.float64)[None, :] + b.astype(np.float64)[None, :]
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def _np_expert_mlp_i8(x, wg, sg, wu, su, wd, sd, inter):
    """expert_mlp_i8 (decoder.rs:2120-2135) composed from three oracle
    linear_int8_dynamic calls (each pinned above) and the f32 SiLU."""
    h = x.shape[1]
    _, g, _, _ = O.linear_i8_dynamic(x, wg, sg, inter)
    _, u, _, _ = O.linear_i8_dynamic(x, wu, su, inter)
    silu = np.vectorize(lambda v: O.lib().oracle_silu(float(v)), otypes=[np.float32])
    act = (silu(g) * u).astype(np.float32)  # f32 silu(g) * u, as decoder.rs:2125-2131
    _, y, _, _ = O.linear_i8_dynamic(act, wd, sd, h)
    return y


def test_moe_prefill_i8_ascending_expert_scatter_and_shared(rng):
    h, inter, E, K, t = 48, 32, 8, 3, 10
    wg = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wu = rng.integers(-127, 128, E * inter * h).astype(np.int8)
    wd = rng.integers(-127, 128, E * h * inter).astype(np.int8)
    sg = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    su = rng.uniform(1e-3, 2e-2, E * inter).astype(np.float32)
    sd = rng.uniform(1e-3, 2e-2, E * h).astype(np.float32)
    x = rng.standard_normal((t, h)).astype(np.float32)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(t)]).astype(np.uint32)
    idx[3] = [5, 5, 1]  # a token routed twice to one expert: both slots are members
    gates = rng.uniform(0.05, 1.0, (t, K)).astype(np.float32)
    st, out = O.moe_prefill_i8(x, idx, gates, wg, sg, wu, su, wd, sd, E, inter)
    assert st == 0
    want32 = np.zeros((t, h), np.float32)
    want64 = np.zeros((t, h), np.float64)
    for e in range(E):  # ascending expert order, (token, slot) order inside
        sl = slice(e * inter * h, (e + 1) * inter * h)
        for r in range(t):
            for j in range(K):
                if idx[r, j] != e:
                    continue
                y = _np_expert_mlp_i8(x[r:r + 1], wg[sl], sg[e * inter:(e + 1) * inter], wu[sl],
                                      su[e * inter:(e + 1) * inter], wd[e * h * inter:(e + 1) * h * inter],
                                      sd[e * h:(e + 1) * h], inter)[0]
                want32[r] = (want32[r] + (np.float32(gates[r, j]) * y).astype(np.float32)).astype(np.float32)
                want64[r] += float(gates[r, j]) * y.astype(np.float64)
    assert np.array_equal(out, want32)
    np.testing.assert_allclose(out, want64, rtol=1e-5, atol=1e-6)
    # the shared expert is added last at weight 1.0
    si = 40
    sw = [rng.integers(-127, 128, si * h).astype(np.int8), rng.uniform(1e-3, 2e-2, si).astype(np.float32),
          rng.integers(-127, 128, si * h).astype(np.int8), rng.uniform(1e-3, 2e-2, si).astype(np.float32),
          rng.integers(-127, 128, h * si).astype(np.int8), rng.uniform(1e-3, 2e-2, h).astype(np.float32)]
    st, out_s = O.moe_prefill_i8(x, idx, gates, wg, sg, wu, su, wd, sd, E, inter, shared=(si, *sw))
    assert st == 0
    ys = _np_expert_mlp_i8(x, sw[0], sw[1], sw[2], sw[3], sw[4], sw[5], si)
    assert np.array_equal(out_s, (out + ys).astype(np.float32))
    bad = idx.copy()
    bad[0, 0] = E
    assert O.moe_prefill_i8(x, bad, gates, wg, sg, wu, su, wd, sd, E, inter)[0] != 0


def _np_moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter):
    """moe_block_i8's grouped structure (decoder.rs:2142-2181) over int4 experts,
    restated in numpy from the pinned pieces' specs: ties-even reciprocal
    quantize of x (decoder.rs:1647-1656), the packed int4 GEMM spec (int4.rs:
    304-343, `_spec_s4s8`), f32 SiLU·up, act re-quantized ties-even, the down
    product scaled by the act scale, and the scatter `out[t] += w·y` in
    ascending expert order with a token's slots in slot order."""
    t, h = x.shape
    silu = np.vectorize(lambda v: O.lib().oracle_silu(float(v)), otypes=[np.float32])
    xq = [_np_quant(x[r], ties_even=True) for r in range(t)]
    gi, gh = inter // group, h // group
    out = np.zeros((t, h), np.float32)
    for e in range(E):
        wg_e, wu_e = wg[e * inter * h // 2:(e + 1) * inter * h // 2], wu[e * inter * h // 2:(e + 1) * inter * h // 2]
        wd_e = wd[e * h * inter // 2:(e + 1) * h * inter // 2]
        for r in range(t):
            slots = [j for j in range(idx.shape[1]) if idx[r, j] == e]
            if not slots:
                continue
            q, xs = xq[r]
            g = _spec_s4s8(q, wg_e, sg[e * inter * gh:(e + 1) * inter * gh], group, 1, h, inter)[0]
            u = _spec_s4s8(q, wu_e, su[e * inter * gh:(e + 1) * inter * gh], group, 1, h, inter)[0]
            act = (silu((g * xs).astype(np.float32)) * (u * xs).astype(np.float32)).astype(np.float32)
            aq, as2 = _np_quant(act, ties_even=True)
            y = _spec_s4s8(aq, wd_e, sd[e * h * gi:(e + 1) * h * gi], group, 1, inter, h)[0]
            yv = (y * as2).astype(np.float32)
            for j in slots:
                out[r] = (out[r] + (np.float32(gates[r, j]) * yv).astype(np.float32)).astype(np.float32)
    return out


def _f64_moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter):
    """The same layer in float64 from the integer codes (int64 dot products,
    float64 group scaling, SwiGLU, down projection and gate-weighted sum):
    catches a dropped scale or a transposed operand, independent of f32 order."""
    t, h = x.shape

    def codes(packed, n, k):
        pk = packed.reshape(n, k // 2).astype(np.int64)
        b = np.zeros((n, k), np.int64)
        b[:, 0::2] = np.where((pk & 0xF) >= 8, (pk & 0xF) - 16, pk & 0xF)
        b[:, 1::2] = np.where((pk >> 4) >= 8, (pk >> 4) - 16, pk >> 4)
        return b

    def gemv(a, packed, scales, k, n):
        b = codes(packed, n, k).reshape(n, k // group, group)
        parts = (b * a.astype(np.int64).reshape(1, k // group, group)).sum(axis=2)
        return (parts * scales.reshape(n, k // group).astype(np.float64)).sum(axis=1)

    def quant(v):
        amax = np.abs(v).max()
        s = amax / 127.0 if amax > 0 else 1.0
        return np.clip(np.rint(v / s), -127, 127), s

    out = np.zeros((t, h))
    gi, gh = inter // group, h // group
    for r in range(t):
        q, xs = quant(x[r].astype(np.float64))
        for j in range(idx.shape[1]):
            e = int(idx[r, j])
            g = gemv(q, wg[e * inter * h // 2:(e + 1) * inter * h // 2], sg[e * inter * gh:(e + 1) * inter * gh],
                     h, inter) * xs
            u = gemv(q, wu[e * inter * h // 2:(e + 1) * inter * h // 2], su[e * inter * gh:(e + 1) * inter * gh],
                     h, inter) * xs
            act = g / (1.0 + np.exp(-g)) * u
            aq, as2 = quant(act)
            y = gemv(aq, wd[e * h * inter // 2:(e + 1) * h * inter // 2], sd[e * h * gi:(e + 1) * h * gi], inter,
                     h) * as2
            out[r] += float(gates[r, j]) * y
    return out


@pytest.mark.parametrize("group", [16, 32])
def test_moe_prefill_i4_matches_restatements(group, rng):
    h, inter, E, K, t = 64, 32, 8, 3, 10
    wg = rng.integers(0, 256, E * inter * h // 2).astype(np.uint8)
    wu = rng.integers(0, 256, E * inter * h // 2).astype(np.uint8)
    wd = rng.integers(0, 256, E * h * inter // 2).astype(np.uint8)
    sg = rng.uniform(1e-3, 2e-2, E * inter * (h // group)).astype(np.float32)
    su = rng.uniform(1e-3, 2e-2, E * inter * (h // group)).astype(np.float32)
    sd = rng.uniform(1e-3, 2e-2, E * h * (inter // group)).astype(np.float32)
    x = rng.standard_normal((t, h)).astype(np.float32)
    # row 2 has scale 1 (max 127) and exact .5 ties: ties-even codes 2, 0, -2, where
    # half-away-from-zero gives 3, 1, -3
    x[2, :5] = [127.0, 2.5, 0.5, -2.5, 1.5]
    idx = np.stack([rng.permutation(E)[:K] for _ in range(t)]).astype(np.uint32)
    idx[4] = [6, 6, 1]  # a token routed twice to one expert: both slots are members
    gates = rng.uniform(0.05, 1.0, (t, K)).astype(np.float32)
    st, out, xq, xs = O.moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter)
    assert st == 0
    assert xq[2, :5].tolist() == [127, 2, 0, -2, 2] and xs[2] == 1.0
    assert not np.array_equal(xq[2], _np_quant(x[2], ties_even=False)[0])
    want = _np_moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter)
    assert np.array_equal(out, want)
    # the scatter order is observable: summing a token's experts in slot order
    # instead of ascending expert order changes the f32 result somewhere
    swapped = idx.copy()
    order = np.argsort(-idx.astype(np.int64), axis=1, kind="stable")
    swapped = np.take_along_axis(idx, order, axis=1)
    swapped_g = np.take_along_axis(gates, order, axis=1)
    by_slot = np.zeros_like(out)
    for r in range(t):
        one = [_np_moe_prefill_i4(x[r:r + 1], swapped[r:r + 1, j:j + 1], swapped_g[r:r + 1, j:j + 1], group, wg, sg,
                                  wu, su, wd, sd, E, inter)[0] for j in range(K)]
        for y in one:
            by_slot[r] = (by_slot[r] + y).astype(np.float32)
    assert not np.array_equal(by_slot, out)
    want64 = _f64_moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, E, inter)
    scale = np.abs(want64).max(axis=1, keepdims=True)
    # f32 rounding plus an occasional one-code flip of a re-quantized act value
    assert np.max(np.abs(out - want64) / scale) < 2e-2
    bad = idx.copy()
    bad[0, 0] = E
    assert O.moe_prefill_i4(x, bad, gates, group, wg, sg, wu, su, wd, sd, E, inter)[0] != 0


def test_moe_prefill_i4_hand_case():
    # 1 token, 2 experts of width 16 (group 16), every weight nibble 1, unit
    # group scales. x = [127, 0, ...] -> xq = x, scale 1: gate = up = 127 for
    # every row; act = silu(127)*127 on every row -> aq = 127, as2 = act/127;
    # down = 16 * 127 per output; y = 16 * act. Gates 0.25 and 0.5 on experts 1, 0
    # -> out = 0.75 * 16 * act per column.
    h = inter = 16
    ones = np.full(inter * h // 2, 0x11, np.uint8)
    wg = np.concatenate([ones, ones])
    x = np.zeros((1, h), np.float32)
    x[0, 0] = 127.0
    s = np.ones(2 * inter, np.float32)
    idx = np.array([[1, 0]], np.uint32)
    gates = np.array([[0.25, 0.5]], np.float32)
    st, out, xq, xs = O.moe_prefill_i4(x, idx, gates, 16, wg, s, wg, s, wg, s, 2, inter)
    assert st == 0 and xs[0] == 1.0 and xq[0, 0] == 127
    act = 127.0 / (1.0 + math.exp(-127.0)) * 127.0
    np.testing.assert_allclose(out[0], np.full(h, 0.75 * 16 * act), rtol=1e-6)


def test_moe_prefill_i4_act_requant_is_ties_even(rng):
    # Exact .5 ties in the SiLU·up row, so the act re-quantization's rounding
    # rule is observable. x = [127, 1, 0...] -> xq = x, scale 1; gate/up row i
    # reads nibbles (n0, n1) of columns 0, 1, so acc = 127·n0 + n1 and, with
    # power-of-two scales, g and u are exact. silu(g) == g in f32 for g >= 32.
    # act = [127, 2.5, 0.5, -2.5, 1.5, 0...] -> scale 1, codes [127, 2, 0, -2, 2]
    # (half-away-from-zero would give [127, 3, 1, -3, 2]).
    h, inter, group = 32, 16, 16
    gi, gh = inter // group, h // group
    wg = np.zeros((inter, h // 2), np.uint8)
    wu = np.zeros((inter, h // 2), np.uint8)
    sg = np.ones((inter, gh), np.float32)
    su = np.ones((inter, gh), np.float32)
    wg[0, 0], wu[0, 0] = 0x01, 0x10  # g = 127, u = 1 -> act 127
    for i, n1 in zip(range(1, 5), (5, 1, -5, 3)):
        wg[i, 0] = 0x11  # acc 128, scale 1/4 -> g = 32
        sg[i, 0] = 0.25
        wu[i, 0] = (n1 & 0xF) << 4  # acc n1, scale 1/64
        su[i, 0] = 1.0 / 64.0
    wd = rng.integers(0, 256, h * inter // 2).astype(np.uint8)
    sd = rng.uniform(1e-3, 2e-2, h * gi).astype(np.float32)
    x = np.zeros((1, h), np.float32)
    x[0, :2] = [127.0, 1.0]
    idx = np.array([[0]], np.uint32)
    gates = np.array([[0.5]], np.float32)
    st, out, _, _ = O.moe_prefill_i4(x, idx, gates, group, wg.reshape(-1), sg.reshape(-1), wu.reshape(-1),
                                     su.reshape(-1), wd, sd, 1, inter)
    assert st == 0

    def down(codes):
        aq = np.zeros(inter, np.int8)
        aq[:5] = codes
        y = _spec_s4s8(aq, wd, sd, group, 1, inter, h)[0]
        return (np.float32(0.5) * y).astype(np.float32)

    assert np.array_equal(out[0], down([127, 2, 0, -2, 2]))
    assert not np.array_equal(out[0], down([127, 3, 1, -3, 2]))


# ---- decode-layer ops: RMSNorm, RoPE, the layer step ------------------------------------

def test_rms_norm_hand_values():
    # nn.rs:438-458: [3, 4], eps 0 -> rstd = 1/sqrt(12.5); weight [2, 0.5]
    rstd = 1.0 / math.sqrt(12.5)
    y = O.rms_norm(np.array([[3.0, 4.0]], np.float32), eps=0.0)
    np.testing.assert_allclose(y[0], [3 * rstd, 4 * rstd], atol=1e-6)
    y = O.rms_norm(np.array([[3.0, 4.0]], np.float32), np.array([2.0, 0.5], np.float32), eps=0.0)
    np.testing.assert_allclose(y[0], [3 * rstd * 2, 4 * rstd * 0.5], atol=1e-6)


def test_rms_norm_vs_float64(rng):
    x = (rng.standard_normal((5, 1280)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1280).astype(np.float32)
    y = O.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y, want, rtol=2e-7, atol=1e-7)


def test_rope_known_answers():
    # decoder.rs:3711-3720 position 0 is the identity
    np.testing.assert_array_equal(O.rope(np.array([1, 2, 3, 4], np.float32), 0, 1, 4), [1, 2, 3, 4])
    # :3723-3739 head_dim 2, pos 1: [a c - b s, b c + a s]
    s, c = math.sin(1.0), math.cos(1.0)
    np.testing.assert_allclose(O.rope(np.array([3, 5], np.float32), 1, 1, 2), [3 * c - 5 * s, 5 * c + 3 * s],
                               atol=1e-5)
    # :3766-3780 two heads share the phase
    s, c = math.sin(2.0), math.cos(2.0)
    np.testing.assert_allclose(O.rope(np.array([1, 0, 0, 1], np.float32), 2, 2, 2), [c, s, -s, c], atol=1e-5)


def test_rope_rotation_vs_float64(rng):
    # the NEOX rotate_half over each head's halves, angle pos * theta^(-2i/d)
    x = rng.standard_normal(10 * 128).astype(np.float32)
    for pos in (0, 7, 1023, 4000):
        y = O.rope(x, pos)
        inv = (1.0 / 10000.0 ** (np.arange(64) * 2 / 128)).astype(np.float32).astype(np.float64)
        ang = pos * inv
        xh = x.astype(np.float64).reshape(10, 2, 64)
        want = np.stack([xh[:, 0] * np.cos(ang) - xh[:, 1] * np.sin(ang),
                         xh[:, 1] * np.cos(ang) + xh[:, 0] * np.sin(ang)], axis=1).reshape(-1)
        np.testing.assert_allclose(y, want, rtol=0, atol=2e-5 * max(1.0, pos / 100))
        # per-head norms preserved (decoder.rs:3742-3763)
        np.testing.assert_allclose((y.reshape(10, 128) ** 2).sum(1), (x.reshape(10, 128) ** 2).sum(1), rtol=1e-5)


def _small_layer(rng, moe=True):
    H, D = 1280, 1280
    lw = {"input_ln": rng.uniform(0.5, 1.5, H).astype(np.float32),
          "post_ln": rng.uniform(0.5, 1.5, H).astype(np.float32),
          "qkv": (rng.integers(-127, 128, 3 * D * H).astype(np.int8), rng.uniform(1e-3, 2e-2, 3 * D).astype(np.float32)),
          "o": (rng.integers(-127, 128, H * D).astype(np.int8), rng.uniform(1e-3, 2e-2, H).astype(np.float32))}
    E, I = 8, 64
    if moe:
        lw["moe"] = {"router": (rng.standard_normal((E, H)) * 0.02).astype(np.float32),
                     "wg": rng.integers(-127, 128, E * I * H).astype(np.int8), "sg": rng.uniform(1e-3, 2e-2, E * I).astype(np.float32),
                     "wu": rng.integers(-127, 128, E * I * H).astype(np.int8), "su": rng.uniform(1e-3, 2e-2, E * I).astype(np.float32),
                     "wd": rng.integers(-127, 128, E * H * I).astype(np.int8), "sd": rng.uniform(1e-3, 2e-2, E * H).astype(np.float32),
                     "n_experts": E, "top_k": 2, "inter": I}
    else:
        lw["dense"] = {"wg": rng.integers(-127, 128, I * H).astype(np.int8), "sg": rng.uniform(1e-3, 2e-2, I).astype(np.float32),
                       "wu": rng.integers(-127, 128, I * H).astype(np.int8), "su": rng.uniform(1e-3, 2e-2, I).astype(np.float32),
                       "wd": rng.integers(-127, 128, H * I).astype(np.int8), "sd": rng.uniform(1e-3, 2e-2, H).astype(np.float32),
                       "inter": I}
    return lw


@pytest.mark.parametrize("moe", [True, False])
def test_decoder_layer_step_batched_equals_per_stream(rng, moe):
    # batched_decode_step_i8_streams == decode_step_with_cache_i8 per stream
    # (the reference's tests/batched_attention_parity.rs / batched_moe_parity.rs invariant)
    lw = _small_layer(rng, moe)
    B, G = 3, 16
    x = rng.standard_normal((B, 1280)).astype(np.float32)
    pos = [G, G + 5, G + 9]

    def rings():
        rs = []
        for s in range(B):
            r = O.Ring(64)
            kv = np.random.default_rng(s).standard_normal((2, 10 * G * 128)).astype(np.float32)
            r.record_prefill(kv[0], kv[1], G)
            rs.append(r)
        return rs

    rb = rings()
    got = O.decoder_layer_step(x, pos, rb, lw)
    got2 = O.decoder_layer_step(got, [p + 1 for p in pos], rb, lw)  # a second step reads the first's ring slot
    rs = rings()
    for s in range(B):
        one = O.decoder_layer_step(x[s:s + 1], [pos[s]], [rs[s]], lw)
        assert np.array_equal(one[0], got[s])
        two = O.decoder_layer_step(one, [pos[s] + 1], [rs[s]], lw)
        assert np.array_equal(two[0], got2[s])
    assert all(r.ring_len.value == 2 for r in rb)


def test_decoder_layer_step_zero_projections_is_identity(rng):
    # o_proj and the MLP's down weights zero: both residual branches add 0
    lw = _small_layer(rng, True)
    lw["o"] = (np.zeros_like(lw["o"][0]), lw["o"][1])
    lw["moe"]["wd"] = np.zeros_like(lw["moe"]["wd"])
    r = O.Ring(16)
    r.record_prefill(np.ones(10 * 4 * 128, np.float32), np.ones(10 * 4 * 128, np.float32), 4)
    x = rng.standard_normal((1, 1280)).astype(np.float32)
    assert np.array_equal(O.decoder_layer_step(x, [4], [r], lw), x)


# ---- prefill attention (decoder.rs:568-640) and chunked prefill attention (:1282-1340) ----

def _sin_fill(seq, dim, salt):
    # decoder.rs:3508-3513: ((i + salt) * 0.37).sin() * 1.7 - 0.2, in f32
    i = np.arange(seq * dim, dtype=np.float32)
    x = ((i + np.float32(salt)) * np.float32(0.37)).astype(np.float32)
    return (np.sin(x).astype(np.float32) * np.float32(1.7) - np.float32(0.2)).astype(np.float32).reshape(seq, dim)


def _f64_attention(q, k, v, num_heads, head_dim, c0=0):
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    out = np.zeros(q.shape)
    for i in range(q.shape[0]):
        t = c0 + i
        for h in range(num_heads):
            sl = slice(h * head_dim, (h + 1) * head_dim)
            s = k[: t + 1, sl] @ q[i, sl] / math.sqrt(head_dim)
            p = np.exp(s - s.max())
            out[i, sl] = (p / p.sum()) @ v[: t + 1, sl]
    return out


def test_prefill_attention_known_answers():
    # decoder.rs:4104-4126: row 0 attends only to itself -> v[0]; row 1 is a
    # convex blend strictly between v[0] and v[1]
    q = np.array([[1, 0], [0, 1]], np.float32)
    v = np.array([[5, 6], [7, 8]], np.float32)
    st, out = O.prefill_attention(q, q.copy(), v, 1, 2)
    assert st == 0 and out[0].tolist() == [5.0, 6.0]
    assert 5.0 < out[1, 0] < 7.0 and 6.0 < out[1, 1] < 8.0
    # one key -> its value; equal scores -> the mean (rswa.rs:1475-1510 pattern)
    k = np.zeros((3, 4), np.float32)
    vv = np.array([[1, 2, 3, 4], [3, 4, 5, 6], [8, 0, 1, 2]], np.float32)
    st, out = O.prefill_attention(np.ones((3, 4), np.float32), k, vv, 1, 4)
    assert out[0].tolist() == vv[0].tolist()
    np.testing.assert_allclose(out[2], vv.mean(axis=0), rtol=1e-6)


def test_chunked_attention_is_byte_identical_to_monolithic():
    # decoder.rs:3503-3535: 3 heads x 4 dims, seq 11, chunks 1, 2, 3 and the full length
    nh, hd, seq = 3, 4, 11
    dim = nh * hd
    q, k, v = _sin_fill(seq, dim, 0.0), _sin_fill(seq, dim, 11.0), _sin_fill(seq, dim, 23.0)
    st, mono = O.prefill_attention(q, k, v, nh, hd)
    assert st == 0
    for chunk in (1, 2, 3, seq):
        got = np.zeros_like(mono)
        for c0 in range(0, seq, chunk):
            c1 = min(c0 + chunk, seq)
            st, ctx = O.chunk_prefill_attention(q[c0:c1], k[:c1], v[:c1], nh, hd, c0)
            assert st == 0
            got[c0:c1] = ctx
        assert np.array_equal(got.view(np.uint32), mono.view(np.uint32)), chunk


@pytest.mark.parametrize("seq,nh,hd", [(17, 2, 8), (40, 10, 128)])
def test_prefill_attention_vs_float64_and_causal_mask(seq, nh, hd, rng):
    q, k, v = (rng.standard_normal((seq, nh * hd)).astype(np.float32) for _ in range(3))
    st, out = O.prefill_attention(q, k, v, nh, hd)
    assert st == 0
    want = _f64_attention(q, k, v, nh, hd)
    # evaluated in float64 and rounded once: within f32 rounding of the numpy restatement
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-7)
    # the f32 restatement of the reference's order: same math to f32 rounding
    st, o32 = O.prefill_attention_f32(q, k, v, nh, hd)
    assert st == 0
    np.testing.assert_allclose(o32, want, rtol=1e-3, atol=2e-5)
    assert not np.array_equal(o32, out)
    # the mask: changing keys / values at positions > r leaves rows <= r unchanged
    r = seq // 2
    k2, v2 = k.copy(), v.copy()
    k2[r + 1:] += 3.0
    v2[r + 1:] -= 5.0
    st, out2 = O.prefill_attention(q, k2, v2, nh, hd)
    assert np.array_equal(out2[: r + 1], out[: r + 1]) and not np.array_equal(out2[r + 1:], out[r + 1:])
    # heads are independent: a change confined to head 0's columns leaves head 1 unchanged
    k3 = k.copy()
    k3[:, :hd] *= -1.0
    st, out3 = O.prefill_attention(q, k3, v, nh, hd)
    assert np.array_equal(out3[:, hd:], out[:, hd:]) and not np.array_equal(out3[:, :hd], out[:, :hd])


def test_prefill_attention_f32_variant_known_answers():
    # the f32 restatement obeys the same known answers (decoder.rs:4104-4126)
    q = np.array([[1, 0], [0, 1]], np.float32)
    v = np.array([[5, 6], [7, 8]], np.float32)
    st, out = O.prefill_attention_f32(q, q.copy(), v, 1, 2)
    assert st == 0 and out[0].tolist() == [5.0, 6.0] and 5.0 < out[1, 0] < 7.0 and 6.0 < out[1, 1] < 8.0


def test_chunk_prefill_attention_rejects_bad_chunks():
    # decoder.rs:1320-1325: c0 > c1 or c0 + cs != c1
    z = np.zeros((4, 8), np.float32)
    assert O.chunk_prefill_attention(z[:2], z, z, 2, 4, 1)[0] != 0
    assert O.chunk_prefill_attention(z[:2], z, z, 2, 4, 2)[0] == 0
