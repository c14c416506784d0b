"""GPU parity for one decoder layer's decode step (decoder.rs:2542-2627 per
stream, :2812-2933 batched) against the oracle's composition of the pinned
pieces (RMSNorm, int8 GEMV, RoPE, ring write, R-SWA attention, MoE decode or
the dense SwiGLU MLP, residuals).

Tolerance: the layer output x within rel 1e-3 after each of three steps.
RoPE's sin/cos (device libm vs glibc, ~1 ulp), the RMSNorm's f64 sum order
and SiLU's expf move values by ulps, which can flip a re-quantized int8 code
(one term of a 1280-wide dot) — everything else is the same arithmetic. The
batched step equals the same streams stepped one at a time, bit for bit
(every row's work is independent; the GEMV's i32 sums are exact)."""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

H, D, E, K, I = 1280, 1280, 64, 6, 896
G = 64  # prefilled reference-block tokens per stream


def _say(msg):
    print(f"[gpu-layer] {msg}", flush=True)


def assert_rel(got, want, rtol):
    want = np.asarray(want, np.float64)
    scale = np.maximum(np.abs(want), np.abs(want).max() * 1e-2)
    rel = np.abs(np.asarray(got, np.float64) - want) / scale
    assert rel.max() <= rtol, f"max rel err {rel.max():.3e} > {rtol}"


def _weights(seed, dense_inter=None):
    lw = {"input_ln": synth.f32_uniform(synth.seed_of(seed), H, 0.5, 1.5),
          "post_ln": synth.f32_uniform(synth.seed_of(seed + 1), H, 0.5, 1.5),
          "qkv": (synth.int8_uniform(synth.seed_of(seed + 2), 3 * D * H),
                  synth.f32_uniform(synth.seed_of(seed + 3), 3 * D, 1e-3, 2e-2)),
          "o": (synth.int8_uniform(synth.seed_of(seed + 4), H * D),
                synth.f32_uniform(synth.seed_of(seed + 5), H, 1e-3, 2e-2))}
    if dense_inter is None:
        from test_gpu_moe import make_layer

        router, wg, sg, wu, su, wd, sd = make_layer(seed + 10)
        si = 1792
        shared = (si, synth.int8_uniform(synth.seed_of(seed + 20), si * H),
                  synth.f32_uniform(synth.seed_of(seed + 21), si, 1e-3, 2e-2),
                  synth.int8_uniform(synth.seed_of(seed + 22), si * H),
                  synth.f32_uniform(synth.seed_of(seed + 23), si, 1e-3, 2e-2),
                  synth.int8_uniform(synth.seed_of(seed + 24), H * si),
                  synth.f32_uniform(synth.seed_of(seed + 25), H, 1e-3, 2e-2))
        lw["moe"] = {"router": router, "wg": wg, "sg": sg, "wu": wu, "su": su, "wd": wd, "sd": sd,
                     "n_experts": E, "top_k": K, "inter": I, "shared": shared}
    else:
        n = dense_inter
        lw["dense"] = {"wg": synth.int8_uniform(synth.seed_of(seed + 30), n * H),
                       "sg": synth.f32_uniform(synth.seed_of(seed + 31), n, 1e-3, 2e-2),
                       "wu": synth.int8_uniform(synth.seed_of(seed + 32), n * H),
                       "su": synth.f32_uniform(synth.seed_of(seed + 33), n, 1e-3, 2e-2),
                       "wd": synth.int8_uniform(synth.seed_of(seed + 34), H * n),
                       "sd": synth.f32_uniform(synth.seed_of(seed + 35), H, 1e-3, 2e-2), "inter": n}
    return lw


def _gpu_layer(ctx, lw):
    from franken_ocr_amd.engine import DecoderLayer, MoeLayer, QInt8

    qkv = QInt8(lw["qkv"][0], lw["qkv"][1], 3 * D, H, ctx)
    o = QInt8(lw["o"][0], lw["o"][1], H, D, ctx)
    if "moe" in lw:
        m = lw["moe"]
        moe = MoeLayer(H, I, E, K, m["router"], m["wg"], m["sg"], m["wu"], m["su"], m["wd"], m["sd"], ctx=ctx)
        moe.set_shared(*m["shared"])
        return DecoderLayer(H, lw["input_ln"], lw["post_ln"], qkv, o, moe=moe, ctx=ctx)
    d = lw["dense"]
    n = d["inter"]
    dense = (QInt8(d["wg"], d["sg"], n, H, ctx), QInt8(d["wu"], d["su"], n, H, ctx), QInt8(d["wd"], d["sd"], H, n, ctx))
    return DecoderLayer(H, lw["input_ln"], lw["post_ln"], qkv, o, dense=dense, ctx=ctx)


def _prefill(ctx, B, seed):
    """Per stream: G reference-block K/V rows, head-major [10][G][128]."""
    from franken_ocr_amd.engine import RingCache

    kv = [(synth.f32_normal(synth.seed_of(seed + 2 * s), 10 * G * 128),
           synth.f32_normal(synth.seed_of(seed + 2 * s + 1), 10 * G * 128)) for s in range(B)]
    cache = RingCache(B, G, ctx=ctx)
    rings = []
    for s in range(B):
        cache.record_prefill(s, ctx.to_device(kv[s][0]), ctx.to_device(kv[s][1]), G)
        r = O.Ring(G)
        r.record_prefill(kv[s][0], kv[s][1], G)
        rings.append(r)
    return cache, rings, kv


# moe 20: a second 16-row qkv pass; dense 2 / 8 (its stream limit): the
# three-launch dense MLP; dense 1: the separate kernels it replaces
@pytest.mark.parametrize("kind,B", [("moe", 4), ("dense", 2), ("moe", 20), ("dense", 8), ("dense", 1)])
def test_decoder_layer_steps_match_oracle(ctx, kind, B):
    _say(f"{kind} layer, {B} streams, 3 steps")
    lw = _weights(12000 if kind == "moe" else 12500, None if kind == "moe" else 6848)
    layer = _gpu_layer(ctx, lw)
    cache, rings, _ = _prefill(ctx, B, 13000)
    x = synth.f32_normal(synth.seed_of(13100), B * H).reshape(B, H)
    dx = ctx.to_device(x)
    pos = np.array([G + 3 * s for s in range(B)], np.uint32)
    want = x
    for step in range(3):
        layer.step(cache, pos + step, dx)
        want = O.decoder_layer_step(want, (pos + step).tolist(), rings, lw)
        got = dx.numpy()
        assert np.isfinite(got).all()
        assert_rel(got, want, 1e-3)
        _say(f"step {step}: max |got - want| {np.abs(got - want).max():.3e}")
        want = got  # continue from the device's state (both rings hold the same steps)


@pytest.mark.parametrize("kind,B", [("moe", 40), ("dense", 12)])
def test_decoder_layer_more_streams_than_one_pass(ctx, kind, B):
    """More streams than one pass takes (32; 8 with the 6848-wide dense MLP)
    run in groups through views of the cache: each stream equals the same
    stream stepped alone, bit for bit, over two steps, and the cursors
    advance for every stream."""
    from franken_ocr_amd.engine import RingCache

    _say(f"{kind} layer, {B} streams, 2 steps (groups)")
    lw = _weights(14000 if kind == "moe" else 14500, None if kind == "moe" else 6848)
    layer = _gpu_layer(ctx, lw)
    cache, _, kv = _prefill(ctx, B, 14600)
    x = synth.f32_normal(synth.seed_of(14700), B * H).reshape(B, H)
    pos = np.array([G + (5 * s) % 17 for s in range(B)], np.uint32)
    dx = ctx.to_device(x)
    for step in range(2):
        layer.step(cache, pos + step, dx, check_route=False)
    assert [cache.state(s) for s in range(B)] == [(G, 2, 2)] * B
    got = dx.numpy()
    for s in sorted({0, 7, 8, 31, 32, B - 1} & set(range(B))):
        one = RingCache(1, G, ctx=ctx)
        one.record_prefill(0, ctx.to_device(kv[s][0]), ctx.to_device(kv[s][1]), G)
        d1 = ctx.to_device(np.ascontiguousarray(x[s:s + 1]))
        for step in range(2):
            layer.step(one, pos[s:s + 1] + step, d1, check_route=False)
        assert np.array_equal(d1.numpy()[0], got[s]), f"stream {s}"
        one.free()
    cache.free()


def test_decoder_layer_batched_equals_per_stream(ctx):
    from franken_ocr_amd.engine import RingCache

    lw = _weights(12000)
    layer = _gpu_layer(ctx, lw)
    B = 3
    cache, _, kv = _prefill(ctx, B, 13500)
    x = synth.f32_normal(synth.seed_of(13600), B * H).reshape(B, H)
    pos = np.array([G, G + 7, G + 11], np.uint32)
    dx = ctx.to_device(x)
    for step in range(2):
        layer.step(cache, pos + step, dx)
    for s in range(B):
        one = RingCache(1, G, ctx=ctx)
        one.record_prefill(0, ctx.to_device(kv[s][0]), ctx.to_device(kv[s][1]), G)
        d1 = ctx.to_device(np.ascontiguousarray(x[s:s + 1]))
        for step in range(2):
            layer.step(one, pos[s:s + 1] + step, d1)
        assert np.array_equal(d1.numpy()[0], dx.numpy()[s]), f"stream {s}"
