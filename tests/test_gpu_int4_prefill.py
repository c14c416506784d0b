"""GPU parity for the int4 chunked-prefill MoE (cfg4) — the grouped
structure of decoder.rs:2142-2181 over int4 experts on the gfx950 matrix
cores — against the CPU oracle (oracle_moe_prefill_i4), through the C ABI.

Tolerance: layer output within rel 1e-3 (config 4's f32 bar; relative
to each element, floored at 1% of its row's largest magnitude). The int4 GEMMs themselves are bit-exact (the drop-in entry runs the
same MFMA kernel and is compared exactly in test_gpu_tier.py); the slack is
for SiLU's expf, whose last-ulp differences from the host libm can move a
requantized act code by one."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-i4] {msg}", flush=True)


def assert_rel(got, want, rtol):
    """Per element |got - want| / max(|want|, 1% of the row's max |want|)."""
    want = want.astype(np.float64)
    scale = np.maximum(np.abs(want), np.max(np.abs(want), axis=-1, keepdims=True) * 1e-2)
    rel = np.abs(got.astype(np.float64) - want) / scale
    assert rel.max() <= rtol, f"max rel err {rel.max():.3e} > {rtol}"


def make_layer(seed, h, inter, e, group):
    from franken_ocr_amd import synth

    wg = synth.bytes_uniform(synth.seed_of(seed), e * inter * h // 2)
    wu = synth.bytes_uniform(synth.seed_of(seed + 1), e * inter * h // 2)
    wd = synth.bytes_uniform(synth.seed_of(seed + 2), e * h * inter // 2)
    sg = synth.f32_uniform(synth.seed_of(seed + 3), e * inter * (h // group), 1e-3, 2e-2)
    su = synth.f32_uniform(synth.seed_of(seed + 4), e * inter * (h // group), 1e-3, 2e-2)
    sd = synth.f32_uniform(synth.seed_of(seed + 5), e * h * (inter // group), 1e-3, 2e-2)
    return wg, sg, wu, su, wd, sd


def random_routing(rng, t, e, k):
    idx = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.uint32)
    g = rng.uniform(0.1, 1.0, (t, k)).astype(np.float32)
    return idx, (g / g.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)


def run_gpu(ctx, layer_arrays, h, inter, e, group, x, idx, gates):
    from franken_ocr_amd.engine import MoeLayerI4

    L = MoeLayerI4(h, inter, e, group, *layer_arrays, ctx=ctx)
    dx, di, dg = ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates)
    dout = ctx.empty(x.shape, np.float32)
    L.prefill(dx, di, dg, dout)
    out = dout.numpy()
    L.free()
    return out


@pytest.mark.parametrize("group", [32, 16])
def test_prefill_small_matches_oracle(ctx, rng, group):
    from franken_ocr_amd import synth

    t, h, inter, e, k = 40, 256, 128, 8, 3
    _say(f"small t={t} h={h} i={inter} e={e} k={k} g={group}")
    layer = make_layer(7000, h, inter, e, group)
    x = synth.f32_normal(synth.seed_of(7100), t * h).reshape(t, h)
    idx, gates = random_routing(rng, t, e, k)
    got = run_gpu(ctx, layer, h, inter, e, group, x, idx, gates)
    st, want, _, _ = O.moe_prefill_i4(x, idx, gates, group, *layer, e, inter)
    assert st == 0
    assert_rel(got, want, 1e-3)


def test_prefill_cfg4_shapes_zipf_matches_oracle(ctx):
    """Full cfg4 shapes (hidden 1280, inter 896, 64 experts, top-6, group 32)
    with Zipf routing, on 64 tokens (the oracle's scalar GEMMs bound the size)."""
    from franken_ocr_amd import synth

    t, h, inter, e, k, group = 64, 1280, 896, 64, 6, 32
    _say(f"cfg4 shapes t={t}")
    layer = make_layer(7200, h, inter, e, group)
    x = synth.f32_normal(synth.seed_of(7300), t * h).reshape(t, h)
    idx, gates = synth.zipf_routing(synth.seed_of(7400), t, e, k)
    got = run_gpu(ctx, layer, h, inter, e, group, x, idx, gates)
    st, want, _, _ = O.moe_prefill_i4(x, idx, gates, group, *layer, e, inter)
    assert st == 0
    assert_rel(got, want, 1e-3)


def test_prefill_duplicate_expert_slots(ctx, rng):
    """moe_block_i8 pushes one member per slot (decoder.rs:2156-2160): a token
    that names an expert twice gets both contributions, in slot order."""
    from franken_ocr_amd import synth

    t, h, inter, e, k, group = 6, 128, 64, 4, 3, 32
    layer = make_layer(7500, h, inter, e, group)
    x = synth.f32_normal(synth.seed_of(7600), t * h).reshape(t, h)
    idx = np.array([[1, 1, 2], [0, 3, 0], [2, 2, 2], [3, 0, 1], [1, 2, 3], [0, 0, 1]], np.uint32)
    gates = rng.uniform(0.1, 1.0, (t, k)).astype(np.float32)
    got = run_gpu(ctx, layer, h, inter, e, group, x, idx, gates)
    st, want, _, _ = O.moe_prefill_i4(x, idx, gates, group, *layer, e, inter)
    assert st == 0
    assert_rel(got, want, 1e-3)


def test_prefill_bad_expert_index_is_shape_error(ctx, rng):
    from franken_ocr_amd import synth
    from franken_ocr_amd._abi import ContractViolation
    from franken_ocr_amd.engine import MoeLayerI4

    t, h, inter, e, k, group = 4, 64, 32, 4, 2, 32
    L = MoeLayerI4(h, inter, e, group, *make_layer(7700, h, inter, e, group), ctx=ctx)
    x = ctx.to_device(synth.f32_normal(synth.seed_of(7800), t * h).reshape(t, h))
    idx = ctx.to_device(np.array([[0, 1], [2, 3], [1, 4], [0, 2]], np.uint32))
    gates = ctx.to_device(np.full((t, k), 0.5, np.float32))
    out = ctx.empty((t, h), np.float32)
    with pytest.raises(ContractViolation, match="expert index out of range"):
        L.prefill(x, idx, gates, out)
    L.free()


def test_prefill_full_size_properties(ctx):
    """cfg4 at its full size (512 tokens, Zipf routing): deterministic run to
    run, and exactly linear in the gates (doubling every gate doubles every
    output bit for bit: each contribution is gate * y, and scaling by 2 is
    exact in f32)."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import MoeLayerI4

    t, h, inter, e, k, group = 512, 1280, 896, 64, 6, 32
    _say("cfg4 full size properties")
    L = MoeLayerI4(h, inter, e, group, *make_layer(7900, h, inter, e, group), ctx=ctx)
    x = ctx.to_device(synth.f32_normal(synth.seed_of(8000), t * h).reshape(t, h))
    idx, gates = synth.zipf_routing(synth.seed_of(8100), t, e, k)
    di = ctx.to_device(idx)
    outs = []
    for gv in (gates, gates, gates * np.float32(2.0)):
        out = ctx.empty((t, h), np.float32)
        L.prefill(x, di, ctx.to_device(gv.astype(np.float32)), out)
        outs.append(out.numpy())
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[2], np.float32(2.0) * outs[0])
    assert np.isfinite(outs[0]).all() and np.abs(outs[0]).max() > 0
    L.free()
