"""GPU parity for the decode GEMV and the LM head + argmax on uploaded int8
weights (decoder.rs:1607-1640, :2703-2747, :2275-2296; sampler.rs:168-186).
The f32 logits are expected bit-exact (same IEEE ops in the same order);
The configs' floor is rel 1e-4. Argmax ids are bit-exact."""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-gemv] {msg}", flush=True)


def _weights(n, k, seed):
    w = synth.int8_uniform(synth.seed_of(seed), n * k)
    s = synth.f32_uniform(synth.seed_of(seed + 1), n, 1e-3, 2e-2)
    return w, s


@pytest.mark.parametrize("m,n,k", [(1, 896, 1280), (16, 896, 1280), (2, 1280, 896), (5, 3840, 1280),
                                   (32, 100, 1280), (8, 17, 16), (8, 1280, 6848), (20, 1280, 1792),
                                   (3, 131, 3200), (1, 64, 8192)])
def test_gemv_i8_bit_exact(ctx, m, n, k):
    from franken_ocr_amd.engine import QInt8, gemv_i8, gemv_i8_prequant, quantize_rows_i8

    _say(f"gemv m={m} n={n} k={k}")
    w, s = _weights(n, k, 10)
    x = synth.f32_normal(synth.seed_of(12), m * k).reshape(m, k)
    q = QInt8(w, s, n, k, ctx)
    dx = ctx.to_device(x)
    dy = ctx.empty((m, n), np.float32)
    gemv_i8(q, dx, dy)
    y = dy.numpy()
    want, acc, xq, a_s = O.gemv_i8_batched(x, w, s, n, k)
    assert np.array_equal(y, want)
    # prequant path with the raw i32 accumulators (cfg1: bit-exact i32)
    dxq, das = ctx.empty((m, k), np.int8), ctx.empty((m,), np.float32)
    quantize_rows_i8(dx, dxq, das)
    assert np.array_equal(dxq.numpy(), xq) and np.array_equal(das.numpy(), a_s)
    dacc = ctx.empty((m, n), np.int32)
    gemv_i8_prequant(q, dxq, das, dy, dacc)
    assert np.array_equal(dacc.numpy(), acc) and np.array_equal(dy.numpy(), want)


def test_quantize_ties_even_rows(ctx):
    from franken_ocr_amd.engine import quantize_rows_i8

    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5] + [0.0] * 9], np.float32)
    dx = ctx.to_device(x)
    dq, ds = ctx.empty((1, 16), np.int8), ctx.empty((1,), np.float32)
    quantize_rows_i8(dx, dq, ds, ties_even=False)
    assert dq.numpy()[0, :7].tolist() == [127, 1, 2, 3, -1, -2, -3]
    quantize_rows_i8(dx, dq, ds, ties_even=True)
    assert dq.numpy()[0, :7].tolist() == [127, 0, 2, 2, 0, -2, -2]


@pytest.mark.parametrize("m,n", [(1, 4099), (8, 20000), (1, 129280), (8, 129280)])
def test_lm_head_logits_and_argmax(ctx, m, n):
    from franken_ocr_amd.engine import QInt8, lm_head_i8

    k = 1280
    _say(f"lm_head m={m} n={n}")
    w, s = _weights(n, k, 20)
    x = synth.f32_normal(synth.seed_of(22), m * k).reshape(m, k)
    q = QInt8(w, s, n, k, ctx)
    dx = ctx.to_device(x)
    dl = ctx.empty((m, n), np.float32)
    da = ctx.empty((m,), np.uint32)
    lm_head_i8(q, dx, da, dl)
    want_l, want_a = O.lm_head_i8(x, w, s, n, k)
    got_l = dl.numpy()
    assert np.array_equal(got_l, want_l)  # bit-exact (floor: rel 1e-4)
    assert np.array_equal(da.numpy(), want_a)
    # logits = nullptr path (argmax only)
    da2 = ctx.empty((m,), np.uint32)
    lm_head_i8(q, dx, da2, None)
    assert np.array_equal(da2.numpy(), want_a)


def test_lm_head_argmax_ties_pick_lowest(ctx):
    """Duplicate the winning row so two vocab ids tie: the lower id wins."""
    from franken_ocr_amd.engine import QInt8, lm_head_i8

    n, k = 5000, 1280
    w, s = _weights(n, k, 30)
    x = synth.f32_normal(synth.seed_of(31), k).reshape(1, k)
    _, a = O.lm_head_i8(x, w, s, n, k)
    win = int(a[0])
    w2, s2 = w.copy().reshape(n, k), s.copy()
    lo = 7 if win > 7 else n - 3
    first, second = min(lo, win), max(lo, win)
    w2[first] = w2[win]
    w2[second] = w2[win]
    s2[first] = s2[win]
    s2[second] = s2[win]
    q = QInt8(w2.reshape(-1), s2, n, k, ctx)
    da = ctx.empty((1,), np.uint32)
    lm_head_i8(q, ctx.to_device(x), da)
    _, want = O.lm_head_i8(x, w2.reshape(-1), s2, n, k)
    assert int(da.numpy()[0]) == int(want[0]) == first


def test_argmax_rows_edge_cases(ctx):
    from franken_ocr_amd.engine import argmax_rows

    n = 129280
    rows = np.random.default_rng(1).standard_normal((6, n)).astype(np.float32)
    rows[0, 100] = rows[0, 90000] = 50.0  # tie -> 100
    rows[1, :] = np.nan  # all NaN -> 0
    rows[2, :] = np.nan
    rows[2, 77777] = -np.inf  # only -inf finite-ish candidate
    rows[3, ::3] = np.nan
    rows[4, :] = -0.0
    rows[4, 5] = 0.0  # -0 == +0 -> index 0
    rows[5, n - 1] = 1e30  # last element
    d = ctx.to_device(rows)
    da = ctx.empty((6,), np.uint32)
    argmax_rows(d, da)
    want = [O.argmax_row(r)[1] for r in rows]
    assert da.numpy().tolist() == want == [100, 0, 77777, want[3], 0, n - 1]
