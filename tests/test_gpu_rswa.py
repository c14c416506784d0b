"""GPU parity for R-SWA: ring write regimes bit-exact (slots, cursors, the
written rows), decode attention within rel 1e-4 (config 5's tolerance) of the CPU
online-softmax path (rswa.rs:894-939), B = 8 streams, G = 1024 reference
rows, ring at random fill level and wrap offset."""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

NH, D, W = 10, 128, 128


def _say(msg):
    print(f"[gpu-rswa] {msg}", flush=True)


def assert_rel(got, want, rtol):
    scale = np.maximum(np.abs(want), np.max(np.abs(want)) * 1e-2)
    rel = np.abs(got.astype(np.float64) - want) / scale
    assert rel.max() <= rtol, f"max rel err {rel.max():.3e} > {rtol}"


def _h2d(ctx, ptr, arr):
    import ctypes as C

    from franken_ocr_amd import _abi

    arr = np.ascontiguousarray(arr)
    _abi.call("focr_hip_h2d", ctx.handle, C.c_void_p(ptr), arr.ctypes.data_as(C.c_void_p), arr.nbytes)


def _d2h(ctx, ptr, shape):
    import ctypes as C

    from franken_ocr_amd import _abi

    out = np.empty(shape, np.float32)
    _abi.call("focr_hip_d2h", ctx.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), out.nbytes)
    return out


def _fill(cache, rings, ctx, b, G, seed):
    for s in range(b):
        k = synth.f32_normal(synth.seed_of(seed + 10 * s), NH * G * D)
        v = synth.f32_normal(synth.seed_of(seed + 10 * s + 1), NH * G * D)
        cache.record_prefill(s, ctx.to_device(k), ctx.to_device(v), G)
        rings[s].record_prefill(k, v, G)


def _random_rings(cache, rings, ctx, b, rng, seed):
    """Random fill level per stream and, when full, a random wrap offset."""
    for s in range(b):
        rl = int(rng.integers(0, W + 1))
        rp = rl % W if rl < W else int(rng.integers(0, W))
        rk = synth.f32_normal(synth.seed_of(seed + 2 * s), NH * W * D).reshape(NH, W, D)
        rv = synth.f32_normal(synth.seed_of(seed + 2 * s + 1), NH * W * D).reshape(NH, W, D)
        reg = cache.regions(s)
        _h2d(ctx, reg["ring_k"], rk)
        _h2d(ctx, reg["ring_v"], rv)
        cache.set_state(s, rl, rp)
        rings[s].ring_k[:] = rk
        rings[s].ring_v[:] = rv
        rings[s].ring_len.value = rl
        rings[s].ring_pos.value = rp


@pytest.mark.parametrize("G", [1024, 37, 0])
def test_rswa_decode_matches_oracle(ctx, G):
    """cfg5: write this step's K/V into each stream's ring (warm-up append or
    steady-state overwrite, per stream), then attend; slots, ring rows and
    contexts are compared with the oracle."""
    from franken_ocr_amd.engine import RingCache

    B = 8
    cap = max(G, 1)
    rng = np.random.default_rng(G + 5)
    cache = RingCache(B, cap, ctx)
    rings = [O.Ring(cap) for _ in range(B)]
    _fill(cache, rings, ctx, B, G, 700)
    _random_rings(cache, rings, ctx, B, rng, 750)
    _say(f"rswa G={G} states={[cache.state(s) for s in range(B)]}")
    ks = synth.f32_normal(synth.seed_of(800), B * NH * D).reshape(B, NH * D)
    vs = synth.f32_normal(synth.seed_of(801), B * NH * D).reshape(B, NH * D)
    slots = cache.write_decode_step(ctx.to_device(ks), ctx.to_device(vs))
    assert slots == [rings[s].write(ks[s], vs[s]) for s in range(B)]
    for s in range(B):
        assert cache.state(s) == (G, rings[s].ring_len.value, rings[s].ring_pos.value)
        got = _d2h(ctx, cache.regions(s)["ring_k"], (NH, W, D))
        assert np.array_equal(got, rings[s].ring_k)
    q = synth.f32_normal(synth.seed_of(999), B * NH * D).reshape(B, NH * D)
    dout = ctx.empty((B, NH * D), np.float32)
    cache.decode_attention(ctx.to_device(q), dout)
    got = dout.numpy()
    for s in range(B):
        st, want = rings[s].attend(q[s])
        assert st == 0
        assert_rel(got[s], want.astype(np.float64), 1e-4)


def test_rswa_batched_write_sequence(ctx):
    """300 batched steps: slots follow warm-up append then modular overwrite."""
    from franken_ocr_amd.engine import RingCache

    B = 3
    cache = RingCache(B, 4, ctx)
    rings = [O.Ring(4) for _ in range(B)]
    _fill(cache, rings, ctx, B, 4, 1000)
    z = ctx.to_device(np.zeros((B, NH * D), np.float32))
    zh = np.zeros(NH * D, np.float32)
    for step in range(300):
        slots = cache.write_decode_step(z, z)
        want = [rings[s].write(zh, zh) for s in range(B)]
        assert slots == want == [step if step < W else (step - W) % W] * B


def test_rswa_step_write_then_attend(ctx):
    """rswa.rs:1184-1200: the step's own K/V is attended."""
    from franken_ocr_amd.engine import RingCache

    B, G = 8, 1024
    cache = RingCache(B, G, ctx)
    rings = [O.Ring(G) for _ in range(B)]
    _fill(cache, rings, ctx, B, G, 1100)
    for s in range(B):
        cache.set_state(s, 128, int(s * 13 % 128))
        rings[s].ring_len.value = 128
        rings[s].ring_pos.value = int(s * 13 % 128)
    for step in range(3):
        q = synth.f32_normal(synth.seed_of(1200 + step), B * NH * D).reshape(B, NH * D)
        ks = synth.f32_normal(synth.seed_of(1300 + step), B * NH * D).reshape(B, NH * D)
        vs = synth.f32_normal(synth.seed_of(1400 + step), B * NH * D).reshape(B, NH * D)
        dout = ctx.empty((B, NH * D), np.float32)
        cache.step(ctx.to_device(q), ctx.to_device(ks), ctx.to_device(vs), dout)
        got = dout.numpy()
        for s in range(B):
            rings[s].write(ks[s], vs[s])
            st, want = rings[s].attend(q[s])
            assert_rel(got[s], want.astype(np.float64), 1e-4)


def test_rswa_known_answers(ctx):
    """rswa.rs:1475-1507: single key returns V; equal scores average."""
    from franken_ocr_amd.engine import RingCache

    cache = RingCache(1, 8, ctx)
    k = np.zeros((NH, 2, D), np.float32)
    k[:, :, 0] = 1.0
    v = np.zeros((NH, 2, D), np.float32)
    v[:, 0], v[:, 1] = 2.0, 4.0
    cache.record_prefill(0, ctx.to_device(k), ctx.to_device(v), 2)
    q = np.zeros((1, NH * D), np.float32)
    q[0, ::D] = 3.0
    dout = ctx.empty((1, NH * D), np.float32)
    cache.decode_attention(ctx.to_device(q), dout)
    assert np.allclose(dout.numpy(), 3.0, atol=1e-5)
    v1 = np.full((NH, 1, D), 7.0, np.float32)
    cache.record_prefill(0, ctx.to_device(k[:, :1].copy()), ctx.to_device(v1), 1)
    cache.decode_attention(ctx.to_device(q), dout)
    assert np.allclose(dout.numpy(), 7.0, atol=1e-5)


def test_rswa_state_errors(ctx):
    from franken_ocr_amd._abi import StateError
    from franken_ocr_amd.engine import RingCache

    cache = RingCache(2, 16, ctx)
    q = ctx.empty((2, NH * D), np.float32)
    with pytest.raises(StateError, match="before record_prefill"):
        cache.decode_attention(q, q)
    z = ctx.to_device(np.zeros(NH * 4 * D, np.float32))
    cache.record_prefill(0, z, z, 0)
    cache.record_prefill(1, z, z, 4)
    with pytest.raises(StateError, match="empty attention key set"):
        cache.decode_attention(q, ctx.empty((2, NH * D), np.float32))
    with pytest.raises(StateError, match="exceeds ref_capacity"):
        big = ctx.to_device(np.zeros(NH * 17 * D, np.float32))
        cache.record_prefill(0, big, big, 17)


def test_rswa_attention_across_cache_shapes(ctx):
    """Caches of different stream counts and capacities share the context's
    split-K partials buffer: attended in turn and twice around, including 70
    streams (two launches of at most 64), each stream within 1e-4 of the
    oracle and the same answer each time."""
    from franken_ocr_amd.engine import RingCache

    shapes = [(3, 200), (70, 64), (8, 1024)]
    setups = []
    for n, (b, cap) in enumerate(shapes):
        rng = np.random.default_rng(40 + n)
        cache = RingCache(b, cap, ctx)
        rings = [O.Ring(cap) for _ in range(b)]
        _fill(cache, rings, ctx, b, cap - 5 * n, 900 + 100 * n)
        _random_rings(cache, rings, ctx, b, rng, 950 + 100 * n)
        q = synth.f32_normal(synth.seed_of(990 + n), b * NH * D).reshape(b, NH * D)
        setups.append((cache, rings, q, ctx.to_device(q), ctx.empty((b, NH * D), np.float32)))
    first = {}
    for rnd in range(2):
        for n, (cache, rings, q, dq, dout) in enumerate(setups):
            _say(f"round {rnd}: {shapes[n][0]} streams, capacity {shapes[n][1]}")
            cache.decode_attention(dq, dout)
            got = dout.numpy()
            if rnd == 0:
                for s in range(len(rings)):
                    st, want = rings[s].attend(q[s])
                    assert st == 0
                    assert_rel(got[s], want.astype(np.float64), 1e-4)
                first[n] = got
            else:
                assert np.array_equal(got, first[n]), shapes[n]
    for cache, *_ in setups:
        cache.free()
