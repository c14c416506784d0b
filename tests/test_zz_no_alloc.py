"""The allocation-free MoE decode entry point (focr_hip_moe_decode_noalloc)
against focr_hip_moe_decode, through the C ABI.

Both run the same kernels in the same order, so the layer output, routing
indices and gates must be identical bit for bit. Two calls in a row: the
first at T = 48 with the shared expert (the grouped down path and the largest
carve of the static scratch), the second at T = 5 without it, so the second
call reads what the first left in the shared array. On a fresh context the
call leaves the context's scratch slots as they were (nothing allocated).
Calls from two contexts on one GPU, issued back to back without a host
synchronisation, give the results each gives alone (the library orders the
calls that share the device's array). Then a layer whose intermediates
exceed the static array is rejected before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import _abi, synth

pytestmark = pytest.mark.gpu

H, I, E, K, SI = 1280, 896, 64, 6, 1792


def _say(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)


def _weights(seed, e, inter, h):
    return [synth.f32_normal(synth.seed_of(seed), e * h, 0.0, 0.02).reshape(e, h),
            synth.int8_uniform(synth.seed_of(seed + 1), e * inter * h),
            synth.f32_uniform(synth.seed_of(seed + 2), e * inter, 1e-3, 2e-2),
            synth.int8_uniform(synth.seed_of(seed + 3), e * inter * h),
            synth.f32_uniform(synth.seed_of(seed + 4), e * inter, 1e-3, 2e-2),
            synth.int8_uniform(synth.seed_of(seed + 5), e * h * inter),
            synth.f32_uniform(synth.seed_of(seed + 6), e * h, 1e-3, 2e-2)]


def test_noalloc_matches_moe_decode_twice(ctx):
    from franken_ocr_amd.engine import MoeLayer

    assert _abi.lib().focr_hip_static_scratch_bytes() == 8 << 20
    layer = MoeLayer(H, I, E, K, *_weights(900, E, I, H), ctx=ctx)
    sh = _weights(950, 1, SI, H)[1:]
    layer.set_shared(SI, *sh)
    for t, shared, norm in ((48, True, True), (5, False, False)):
        _say(f"t={t} shared={shared} norm_topk={norm}")
        x = synth.f32_normal(synth.seed_of(960 + t), t * H).reshape(t, H)
        dx = ctx.to_device(x)
        outs = []
        for fn in (layer.decode, layer.decode_noalloc):
            dout = ctx.empty((t, H), np.float32)
            didx, dg = ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32)
            fn(dx, dout, didx, dg, norm_topk=norm, with_shared=shared, check_route=True)
            outs.append((dout.numpy(), didx.numpy(), dg.numpy()))
        (o0, i0, g0), (o1, i1, g1) = outs
        assert np.array_equal(i0, i1) and np.array_equal(g0.view(np.uint32), g1.view(np.uint32))
        assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
        assert np.isfinite(o1).all() and np.abs(o1).max() > 0


def test_noalloc_leaves_a_fresh_context_unallocated():
    # on a fresh context the call must not carve the context's grow-only
    # scratch slots (the ordinary entry point does, which the check confirms)
    from franken_ocr_amd.device import Context
    from franken_ocr_amd.engine import MoeLayer

    c = Context(0)
    layer = MoeLayer(H, I, E, K, *_weights(900, E, I, H), ctx=c)
    layer.set_shared(SI, *_weights(950, 1, SI, H)[1:])
    t = 48
    dx = c.to_device(synth.f32_normal(synth.seed_of(1008), t * H).reshape(t, H))
    dout = c.empty((t, H), np.float32)
    c.synchronize()
    before = c.scratch_bytes()
    _say(f"fresh context: slots hold {before} B")
    layer.decode_noalloc(dx, dout, with_shared=True, check_route=True)
    layer.decode_noalloc(dx.view_rows(0, 8), dout.view_rows(0, 8), check_route=True)
    c.synchronize()
    assert c.scratch_bytes() == before
    layer.decode(dx, dout, with_shared=True)
    c.synchronize()
    assert c.scratch_bytes() > before
    layer.free()
    c.close()


def test_noalloc_calls_from_two_contexts_are_ordered(ctx):
    # two contexts (two streams) on one GPU share its static array: calls
    # issued back to back, with no host synchronisation between them, must
    # give the results each gives alone
    from franken_ocr_amd.device import Context
    from franken_ocr_amd.engine import MoeLayer

    ca, cb = Context(0), Context(0)
    layer = MoeLayer(H, I, E, K, *_weights(900, E, I, H), ctx=ca)
    layer.set_shared(SI, *_weights(950, 1, SI, H)[1:])
    cases = [(ca, 48, True), (cb, 8, False), (ca, 5, True), (cb, 32, True)]
    inputs = []
    for c, t, shared in cases:
        x = synth.f32_normal(synth.seed_of(1100 + t), t * H).reshape(t, H)
        inputs.append((c, c.to_device(x), c.empty((t, H), np.float32), c.empty((t, K), np.uint32), shared))
    alone = []
    for c, dx, dout, didx, shared in inputs:
        layer.decode_noalloc(dx, dout, didx, with_shared=shared, check_route=True, ctx=c)
        c.synchronize()
        alone.append((dout.numpy(), didx.numpy()))
    for rep in range(2):
        _say(f"two contexts back to back, pass {rep}")
        for c, dx, dout, didx, shared in inputs:
            layer.decode_noalloc(dx, dout, didx, with_shared=shared, check_route=False, ctx=c)
        ca.synchronize()
        cb.synchronize()
        for (c, dx, dout, didx, shared), (o, i) in zip(inputs, alone):
            assert np.array_equal(didx.numpy(), i)
            assert np.array_equal(dout.numpy().view(np.uint32), o.view(np.uint32))
    layer.free()
    ca.close()
    cb.close()


def test_noalloc_rejects_scratch_beyond_the_static_array(ctx):
    from franken_ocr_amd.engine import MoeLayer

    # 8 experts, top-8, hidden = inter = 2048: at t = 64 the act rows and the
    # grouped path's expert outputs are 4 MiB each, past the 8 MiB array
    h = inter = 2048
    e = k = 8
    w = [np.zeros((e, h), np.float32), np.zeros(e * inter * h, np.int8), np.ones(e * inter, np.float32),
         np.zeros(e * inter * h, np.int8), np.ones(e * inter, np.float32), np.zeros(e * h * inter, np.int8),
         np.ones(e * h, np.float32)]
    layer = MoeLayer(h, inter, e, k, *w, ctx=ctx)
    t = 64
    dx = ctx.to_device(np.zeros((t, h), np.float32))
    dout = ctx.empty((t, h), np.float32)
    with pytest.raises(_abi.ContractViolation, match="moe_decode_noalloc: t 64 needs .* bytes of scratch"):
        layer.decode_noalloc(dx, dout)
    _say("oversized request rejected")
