"""GPU parity for the MoE decode layer (moe.rs:181-266 route;
decoder.rs:2199-2268 decode_mlp_i8 per token): routing indices bit-exact,
gates within rel 1e-6, layer output within rel 1e-3 (config 3's tolerance) — the
only f32 differences come from expf in SiLU (~1 ulp) propagating through
the act re-quantization."""

from __future__ import annotations

import math

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

H, I, E, K = 1280, 896, 64, 6


def _say(msg):
    print(f"[gpu-moe] {msg}", flush=True)


def make_layer(seed: int, h=H, inter=I, e=E):
    router = synth.f32_normal(synth.seed_of(seed), e * h, 0.0, 0.02).reshape(e, h)
    wg = synth.int8_uniform(synth.seed_of(seed + 1), e * inter * h)
    wu = synth.int8_uniform(synth.seed_of(seed + 2), e * inter * h)
    wd = synth.int8_uniform(synth.seed_of(seed + 3), e * h * inter)
    sg = synth.f32_uniform(synth.seed_of(seed + 4), e * inter, 1e-3, 2e-2)
    su = synth.f32_uniform(synth.seed_of(seed + 5), e * inter, 1e-3, 2e-2)
    sd = synth.f32_uniform(synth.seed_of(seed + 6), e * h, 1e-3, 2e-2)
    return router, wg, sg, wu, su, wd, sd


def assert_rel(got, want, rtol):
    scale = np.maximum(np.abs(want), np.max(np.abs(want), axis=-1, keepdims=True) * 1e-2)
    rel = np.abs(got.astype(np.float64) - want) / scale
    assert rel.max() <= rtol, f"max rel err {rel.max():.3e} > {rtol}"


@pytest.fixture(scope="module")
def layer_w():
    return make_layer(100)


@pytest.fixture(scope="module")
def gpu_layer(ctx, layer_w):
    from franken_ocr_amd.engine import MoeLayer

    return MoeLayer(H, I, E, K, *layer_w, ctx=ctx)


@pytest.mark.parametrize("t", [1, 8, 32, 64, 65, 300, 1024])
@pytest.mark.parametrize("norm_topk", [True, False])
def test_route_bit_exact(ctx, gpu_layer, layer_w, t, norm_topk):
    _say(f"route t={t} norm={norm_topk}")
    x = synth.f32_normal(synth.seed_of(200 + t), t * H).reshape(t, H)
    dx = ctx.to_device(x)
    didx, dg, dp = ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32), ctx.empty((t, E), np.float32)
    gpu_layer.route(dx, didx, dg, dp, norm_topk=norm_topk)
    st, idx, w, probs = O.route(x, layer_w[0], E, K, norm_topk=norm_topk)
    assert st == 0
    assert np.array_equal(didx.numpy(), idx)
    np.testing.assert_allclose(dg.numpy(), w, rtol=1e-6, atol=0)
    np.testing.assert_allclose(dp.numpy(), probs, rtol=1e-6, atol=1e-12)


@pytest.mark.parametrize("tied", [False, True])
def test_route_many_rows_equals_the_split_route(ctx, layer_w, tied):
    """Above 64 rows the route runs as a logits kernel (the router read once
    per 8 tokens) and a rank kernel; at most 64 it is the split route. The
    same f64 dots in the same lane order and the same softmax / top-k: a
    200-row call gives the bits of the 64-row call on its first 64 rows
    (indices, gates, probabilities), also with tied router rows."""
    from franken_ocr_amd.engine import MoeLayer

    router = layer_w[0].copy()
    if tied:
        router[[2, 11, 19, 33, 47, 52, 60], :] = np.abs(synth.f32_normal(synth.seed_of(711), H, 0.0, 0.02)) * 5.0
    L = MoeLayer(H, I, E, K, router, *layer_w[1:], ctx=ctx)
    t = 200
    x = synth.f32_normal(synth.seed_of(712), t * H).reshape(t, H)
    if tied:
        x = np.abs(x)
    outs = []
    for n in (64, t):
        didx, dg, dp = ctx.empty((n, K), np.uint32), ctx.empty((n, K), np.float32), ctx.empty((n, E), np.float32)
        L.route(ctx.to_device(np.ascontiguousarray(x[:n])), didx, dg, dp, norm_topk=True)
        outs.append((didx.numpy(), dg.numpy(), dp.numpy()))
    (i64, g64, p64), (ia, ga, pa) = outs
    assert np.array_equal(ia[:64], i64)
    assert np.array_equal(ga[:64].view(np.uint32), g64.view(np.uint32))
    assert np.array_equal(pa[:64].view(np.uint32), p64.view(np.uint32))
    st, idx, w, probs = O.route(x, router, E, K, norm_topk=True)
    assert st == 0 and np.array_equal(ia, idx)
    np.testing.assert_allclose(ga, w, rtol=1e-6, atol=0)


@pytest.mark.parametrize("e,k,h", [(37, 5, 1280), (9, 2, 640), (64, 8, 1024)])
def test_route_many_rows_other_shapes(ctx, e, k, h):
    """The many-row route at expert counts that leave a part of the last
    eight-expert block empty, other top-k and narrower rows: the bits of the
    split route on the first 64 rows, the oracle's indices on all 100."""
    from franken_ocr_amd.engine import MoeLayer

    inter = 64
    w = make_layer(720 + e, h=h, inter=inter, e=e)
    L = MoeLayer(h, inter, e, k, *w, ctx=ctx)
    t = 100
    x = synth.f32_normal(synth.seed_of(721 + e), t * h).reshape(t, h)
    outs = []
    for n in (64, t):
        didx, dg, dp = ctx.empty((n, k), np.uint32), ctx.empty((n, k), np.float32), ctx.empty((n, e), np.float32)
        L.route(ctx.to_device(np.ascontiguousarray(x[:n])), didx, dg, dp, norm_topk=True)
        outs.append((didx.numpy(), dg.numpy(), dp.numpy()))
    (i64, g64, p64), (ia, ga, pa) = outs
    assert np.array_equal(ia[:64], i64)
    assert np.array_equal(ga[:64].view(np.uint32), g64.view(np.uint32))
    assert np.array_equal(pa[:64].view(np.uint32), p64.view(np.uint32))
    st, idx, gw, probs = O.route(x, w[0], e, k, norm_topk=True)
    assert st == 0 and np.array_equal(ia, idx)
    np.testing.assert_allclose(ga, gw, rtol=1e-6, atol=0)
    np.testing.assert_allclose(pa, probs, rtol=1e-6, atol=1e-12)


def test_route_ties_at_the_cutoff_pick_lower_indices(ctx):
    """Seven identical router rows that dominate every token: their logits and
    probabilities are bit-identical, so the greedy top-6 (moe.rs:215-240: rank
    by probability, then index) must take the six lowest of them, in index
    order, with equal gates."""
    from franken_ocr_amd.engine import MoeLayer

    router, wg, sg, wu, su, wd, sd = make_layer(700)
    tied = [2, 11, 19, 33, 47, 52, 60]
    router[tied, :] = np.abs(synth.f32_normal(synth.seed_of(701), H, 0.0, 0.02)) * 5.0
    t = 8
    x = np.abs(synth.f32_normal(synth.seed_of(702), t * H)).reshape(t, H)
    L = MoeLayer(H, I, E, K, router, wg, sg, wu, su, wd, sd, ctx=ctx)
    didx, dg, dp = ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32), ctx.empty((t, E), np.float32)
    L.route(ctx.to_device(x), didx, dg, dp, norm_topk=True)
    st, idx, w, probs = O.route(x, router, E, K, norm_topk=True)
    assert st == 0
    assert idx.tolist() == [tied[:6]] * t  # the oracle itself resolves the tie this way
    assert np.array_equal(didx.numpy(), idx)
    np.testing.assert_allclose(dg.numpy(), w, rtol=1e-6, atol=0)
    assert (dg.numpy() == dg.numpy()[:, :1]).all()  # tied probabilities: equal gates


@pytest.mark.parametrize("t", [1, 8, 32])
def test_moe_decode_matches_oracle(ctx, gpu_layer, layer_w, t):
    _say(f"moe_decode t={t}")
    x = synth.f32_normal(synth.seed_of(300 + t), t * H).reshape(t, H)
    dx = ctx.to_device(x)
    dout = ctx.empty((t, H), np.float32)
    didx, dg = ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32)
    gpu_layer.decode(dx, dout, didx, dg, norm_topk=True)
    st, out, idx, gates = O.moe_decode(x, *layer_w, E, K, I, norm_topk=True)
    assert st == 0
    assert np.array_equal(didx.numpy(), idx)
    np.testing.assert_allclose(dg.numpy(), gates, rtol=1e-6, atol=0)
    assert_rel(dout.numpy(), out.astype(np.float64), 1e-3)
    # deterministic: a second run is bitwise identical
    dout2 = ctx.empty((t, H), np.float32)
    gpu_layer.decode(dx, dout2, norm_topk=True)
    assert np.array_equal(dout.numpy(), dout2.numpy())


def test_moe_decode_reference_default_config(ctx, gpu_layer, layer_w):
    """norm_topk_prob = false, routed_scaling_factor = 1.0 (moe.rs:70-73)."""
    t = 8
    x = synth.f32_normal(synth.seed_of(400), t * H).reshape(t, H)
    dout = ctx.empty((t, H), np.float32)
    gpu_layer.decode(ctx.to_device(x), dout, norm_topk=False, routed_scale=1.0)
    st, out, _, _ = O.moe_decode(x, *layer_w, E, K, I, norm_topk=False)
    assert_rel(dout.numpy(), out.astype(np.float64), 1e-3)


def test_moe_decode_all_tokens_one_expert(ctx):
    """Every token routes to the same 6 experts (P = T pairs per expert)."""
    from franken_ocr_amd.engine import MoeLayer

    router, wg, sg, wu, su, wd, sd = make_layer(500)
    router = np.zeros_like(router)
    router[[3, 9, 17, 30, 41, 63], :] = 0.05  # same top-6 for every positive-sum row
    t = 40
    x = np.abs(synth.f32_normal(synth.seed_of(501), t * H)).reshape(t, H)
    L = MoeLayer(H, I, E, K, router, wg, sg, wu, su, wd, sd, ctx=ctx)
    dout, didx = ctx.empty((t, H), np.float32), ctx.empty((t, K), np.uint32)
    L.decode(ctx.to_device(x), dout, didx, norm_topk=True)
    st, out, idx, _ = O.moe_decode(x, router, wg, sg, wu, su, wd, sd, E, K, I, norm_topk=True)
    assert np.array_equal(didx.numpy(), idx) and sorted(idx[0].tolist()) == [3, 9, 17, 30, 41, 63]
    assert_rel(dout.numpy(), out.astype(np.float64), 1e-3)


def test_moe_identity_experts_known_answer(ctx):
    """moe.rs:938-980 with int8 identity experts: 6/64 * silu(1)."""
    from franken_ocr_amd.engine import MoeLayer

    h = inter = 16
    eye = (np.eye(16, dtype=np.int8) * 127).reshape(-1)
    w = np.tile(eye, E)
    s = np.full(E * 16, np.float32(1.0) / np.float32(127.0), np.float32)
    L = MoeLayer(h, inter, E, K, np.zeros((E, h), np.float32), w, s, w, s, w, s, ctx=ctx)
    dout = ctx.empty((1, h), np.float32)
    didx = ctx.empty((1, K), np.uint32)
    L.decode(ctx.to_device(np.ones((1, h), np.float32)), dout, didx)
    assert didx.numpy()[0].tolist() == [0, 1, 2, 3, 4, 5]
    np.testing.assert_allclose(dout.numpy()[0], 6.0 / 64 * (1.0 / (1.0 + math.exp(-1.0))), rtol=1e-5)


def test_moe_shared_expert(ctx, layer_w):
    from franken_ocr_amd.engine import MoeLayer

    si = 1792
    swg = synth.int8_uniform(synth.seed_of(600), si * H)
    swu = synth.int8_uniform(synth.seed_of(601), si * H)
    swd = synth.int8_uniform(synth.seed_of(602), H * si)
    ssg = synth.f32_uniform(synth.seed_of(603), si, 1e-3, 2e-2)
    ssu = synth.f32_uniform(synth.seed_of(604), si, 1e-3, 2e-2)
    ssd = synth.f32_uniform(synth.seed_of(605), H, 1e-3, 2e-2)
    L = MoeLayer(H, I, E, K, *layer_w, ctx=ctx)
    L.set_shared(si, swg, ssg, swu, ssu, swd, ssd)
    t = 4
    x = synth.f32_normal(synth.seed_of(606), t * H).reshape(t, H)
    dout = ctx.empty((t, H), np.float32)
    L.decode(ctx.to_device(x), dout, with_shared=True)
    st, out, _, _ = O.moe_decode(x, *layer_w, E, K, I, shared=(si, swg, ssg, swu, ssu, swd, ssd))
    assert st == 0
    assert_rel(dout.numpy(), out.astype(np.float64), 1e-3)


@pytest.mark.parametrize("t", [40, 48, 64])
def test_moe_grouped_down_matches_per_token_down(ctx, gpu_layer, t):
    """From T = 40 the layer runs the expert-grouped down kernel + slot-order
    combine; below it, down + combine per token. Both compute every pair's
    y = ((f32)acc * as) * sd * gate and sum a token's slots in the same
    order, so a T-token step equals its 8-token chunks bit for bit — the
    reference's batched == per-stream invariant (tests/batched_moe_parity.rs).
    Row 5 has no finite router score: both paths write zeros for it."""
    _say(f"moe grouped vs per-token t={t}")
    x = synth.f32_normal(synth.seed_of(700 + t), t * H).reshape(t, H)
    x[5] = np.nan
    full = ctx.empty((t, H), np.float32)
    gpu_layer.decode(ctx.to_device(x), full, norm_topk=True, check_route=False)
    parts = []
    for lo in range(0, t, 8):
        n = min(8, t - lo)
        d = ctx.empty((n, H), np.float32)
        gpu_layer.decode(ctx.to_device(np.ascontiguousarray(x[lo:lo + n])), d, norm_topk=True, check_route=False)
        parts.append(d.numpy())
    got = full.numpy()
    assert np.array_equal(got, np.concatenate(parts))
    assert not got[5].any() and np.isfinite(got).all()


def test_moe_shared_expert_grouped_path(ctx, layer_w):
    from franken_ocr_amd.engine import MoeLayer

    si = 1792
    swg = synth.int8_uniform(synth.seed_of(610), si * H)
    swu = synth.int8_uniform(synth.seed_of(611), si * H)
    swd = synth.int8_uniform(synth.seed_of(612), H * si)
    ssg = synth.f32_uniform(synth.seed_of(613), si, 1e-3, 2e-2)
    ssu = synth.f32_uniform(synth.seed_of(614), si, 1e-3, 2e-2)
    ssd = synth.f32_uniform(synth.seed_of(615), H, 1e-3, 2e-2)
    L = MoeLayer(H, I, E, K, *layer_w, ctx=ctx)
    L.set_shared(si, swg, ssg, swu, ssu, swd, ssd)
    t = 44
    x = synth.f32_normal(synth.seed_of(616), t * H).reshape(t, H)
    dout = ctx.empty((t, H), np.float32)
    L.decode(ctx.to_device(x), dout, with_shared=True)
    st, out, _, _ = O.moe_decode(x, *layer_w, E, K, I, shared=(si, swg, ssg, swu, ssu, swd, ssd))
    assert st == 0
    assert_rel(dout.numpy(), out.astype(np.float64), 1e-3)


@pytest.mark.parametrize("t", [2, 200])
def test_route_nan_reports_error(ctx, gpu_layer, t):
    """A row without a finite router score is reported (moe.rs:261-265),
    also past 64 rows (the prefill-sized route), naming the first such row."""
    from franken_ocr_amd._abi import RouteError

    x = synth.f32_normal(synth.seed_of(290), t * H).reshape(t, H)
    x[t - 1] = np.nan
    didx, dg = ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32)
    with pytest.raises(RouteError, match=f"no finite router score for token {t - 1}"):
        gpu_layer.route(ctx.to_device(x), didx, dg)


def test_moe_shape_errors(ctx, gpu_layer):
    from franken_ocr_amd._abi import ContractViolation

    with pytest.raises(ContractViolation, match=r"t 16385 outside 1..=16384"):
        gpu_layer.decode(ctx.empty((16385, H), np.float32), ctx.empty((16385, H), np.float32))


def test_moe_decode_past_64_rows_runs_in_chunks(ctx, gpu_layer, layer_w):
    """A call of more than 64 rows runs as chunks of 64: its rows are the
    bits of the same rows decoded in separate calls, and match the oracle; a
    row without a finite score is reported by its index in the whole call."""
    from franken_ocr_amd._abi import RouteError

    t = 150
    _say(f"moe_decode t={t} (chunks of 64)")
    x = synth.f32_normal(synth.seed_of(380), t * H).reshape(t, H)
    dout, didx, dg = ctx.empty((t, H), np.float32), ctx.empty((t, K), np.uint32), ctx.empty((t, K), np.float32)
    gpu_layer.decode(ctx.to_device(x), dout, didx, dg, norm_topk=True)
    got, gi = dout.numpy(), didx.numpy()
    for r0, r1 in ((0, 50), (50, 64), (64, 150)):
        o = ctx.empty((r1 - r0, H), np.float32)
        gpu_layer.decode(ctx.to_device(np.ascontiguousarray(x[r0:r1])), o, norm_topk=True)
        assert np.array_equal(o.numpy(), got[r0:r1]), (r0, r1)
    st, out, idx, gates = O.moe_decode(x, *layer_w, E, K, I, norm_topk=True)
    assert st == 0
    assert np.array_equal(gi, idx)
    np.testing.assert_allclose(dg.numpy(), gates, rtol=1e-6, atol=0)
    assert_rel(got, out.astype(np.float64), 1e-3)
    x[70] = np.nan
    with pytest.raises(RouteError, match="no finite router score for token 70"):
        gpu_layer.decode(ctx.to_device(x), dout)


@pytest.mark.parametrize("t", [1, 8, 40])
def test_route_fallback_when_the_other_blocks_are_not_waited_for(layer_w, t):
    # The route splits each token's router rows over several blocks that
    # exchange logits through the L2, and a block that waited too long
    # computes the missing logits itself. A wait bound of 0 forces that path
    # for every part of every token: routing, probabilities and the layer
    # output must be the same bits as with the exchange (and the oracle's).
    from franken_ocr_amd.device import Context
    from franken_ocr_amd.engine import MoeLayer

    c = Context(0)
    layer = MoeLayer(H, I, E, K, *layer_w, ctx=c)
    x = synth.f32_normal(synth.seed_of(1300 + t), t * H).reshape(t, H)
    dx = c.to_device(x)
    res = []
    for ticks in (1000, 0, 1000):
        _say(f"route wait {ticks} ticks, t={t}")
        c.set_route_wait(ticks)
        di, dg, dp = c.empty((t, K), np.uint32), c.empty((t, K), np.float32), c.empty((t, E), np.float32)
        layer.route(dx, di, dg, dp, norm_topk=True)
        dout = c.empty((t, H), np.float32)
        layer.decode(dx, dout, norm_topk=True)
        res.append((di.numpy(), dg.numpy(), dp.numpy(), dout.numpy()))
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for a, b in zip(res[0], res[2]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    st, want_i, want_g, want_p = O.route(x, layer_w[0], E, K, norm_topk=True)
    assert st == 0 and np.array_equal(res[1][0], want_i)
    layer.free()
    c.close()
