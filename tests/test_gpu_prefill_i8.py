"""GPU parity for the prefill path on int8 weights (int8 matrix cores, i32
accumulation): nn::linear_int8_dynamic (nn.rs:151-173) and moe_block_i8
(decoder.rs:2142-2181) against the CPU oracle.

The linear's outputs are bit-exact: the activation bytes follow the same
rule (true division, ties to even), the i32 sums are exact, and the dequant
is the same two rounded multiplies (+ bias). The MoE block is compared within
rel 1e-3 (the MoE configs' layer-output tolerance): SiLU goes
through expf, which may differ from glibc's by an ulp and flip an act code
in the re-quantization, everything else is the same arithmetic."""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

H, I, E, K = 1280, 896, 64, 6


def _say(msg):
    print(f"[gpu-prefill-i8] {msg}", flush=True)


def assert_rel(got, want, rtol):
    want = np.asarray(want, np.float64)
    scale = np.maximum(np.abs(want), np.abs(want).max() * 1e-2)
    rel = np.abs(np.asarray(got, np.float64) - want) / scale
    assert rel.max() <= rtol, f"max rel err {rel.max():.3e} > {rtol}"


@pytest.mark.parametrize("m,k,n,bias", [(1, 64, 8, False), (5, 128, 33, True), (64, 1280, 256, False),
                                        (100, 1280, 3840, True), (513, 896, 1280, False), (7, 6848, 64, True),
                                        (130, 1792, 300, False), (256, 1280, 256, True), (700, 960, 1000, True),
                                        (300, 6848, 96, False), (512, 1280, 6848, True), (257, 192, 33, True),
                                        (256, 8256, 40, True), (256, 1280, 1280, False), (17, 1280, 3840, False),
                                        (200, 6848, 1280, False), (256, 1792, 1280, False)])
def test_linear_i8_dynamic_bit_exact(ctx, m, k, n, bias):
    from franken_ocr_amd.engine import QInt8, linear_i8_dynamic

    _say(f"linear m={m} k={k} n={n} bias={bias}")
    seed = 9000 + m + k + n
    x = (synth.f32_normal(synth.seed_of(seed), m * k) * 3).reshape(m, k)
    x[0, :7] = 0.0
    w = synth.int8_uniform(synth.seed_of(seed + 1), n * k)
    ws = synth.f32_uniform(synth.seed_of(seed + 2), n, 1e-3, 2e-2)
    b = synth.f32_normal(synth.seed_of(seed + 3), n) if bias else None
    q = QInt8(w, ws, n, k, ctx)
    dy = ctx.empty((m, n), np.float32)
    linear_i8_dynamic(q, ctx.to_device(x), dy, None if b is None else ctx.to_device(b))
    st, want, _, _ = O.linear_i8_dynamic(x, w, ws, n, bias=b)
    assert st == 0
    got = dy.numpy()
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} differ"


def test_linear_i8_dynamic_ties_even_known_answer(ctx):
    """nn.rs:601-628, zero-padded to k = 64 (zeros change neither the
    activation scale nor any sum): [0, 2, 0, 0], byte-identical on repeat."""
    from franken_ocr_amd.engine import QInt8, linear_i8_dynamic

    x = np.zeros((2, 64), np.float32)
    x[0, :8] = [-127.0, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 127.0]
    w = np.zeros((2, 64), np.int8)
    w[0, 4] = 1
    w[1, 6] = 1
    q = QInt8(w.reshape(-1), np.ones(2, np.float32), 2, 64, ctx)
    dx = ctx.to_device(x)
    y1, y2 = ctx.empty((2, 2), np.float32), ctx.empty((2, 2), np.float32)
    linear_i8_dynamic(q, dx, y1)
    linear_i8_dynamic(q, dx, y2)
    assert y1.numpy().ravel().tolist() == [0.0, 2.0, 0.0, 0.0]
    assert np.array_equal(y1.numpy(), y2.numpy())


def test_quantize_rows_dynamic_rule_bit_exact(ctx):
    from franken_ocr_amd.engine import QUANT_DYNAMIC, quantize_rows_i8

    m, k = 37, 1280
    x = (synth.f32_normal(synth.seed_of(9100), m * k) * 5).reshape(m, k)
    x[3] = 0.0
    s = np.float32(np.abs(x[5]).max()) / np.float32(127.0)
    x[5, :64] = ((np.arange(64) - 32 + 0.5).astype(np.float32) * s).astype(np.float32)  # planted ties
    xq, xs = ctx.empty((m, k), np.int8), ctx.empty((m,), np.float32)
    quantize_rows_i8(ctx.to_device(x), xq, xs, rule=QUANT_DYNAMIC)
    for r in range(m):
        q, sc = O.quantize_row_dynamic(x[r])
        assert np.array_equal(xq.numpy()[r], q) and xs.numpy()[r] == sc, f"row {r}"


def test_linear_i8_dynamic_rejects_k_not_multiple_of_64(ctx):
    from franken_ocr_amd._abi import ContractViolation
    from franken_ocr_amd.engine import QInt8, linear_i8_dynamic

    q = QInt8(np.zeros(4 * 80, np.int8), np.ones(4, np.float32), 4, 80, ctx)
    with pytest.raises(ContractViolation, match="multiple of 64"):
        linear_i8_dynamic(q, ctx.to_device(np.zeros((2, 80), np.float32)), ctx.empty((2, 4), np.float32))


@pytest.fixture(scope="module")
def layer_w():
    from test_gpu_moe import make_layer

    return make_layer(9200)


@pytest.fixture(scope="module")
def gpu_layer(ctx, layer_w):
    from franken_ocr_amd.engine import MoeLayer

    return MoeLayer(H, I, E, K, *layer_w, ctx=ctx)


@pytest.mark.parametrize("t", [1, 24, 130])
def test_moe_prefill_i8_matches_oracle(ctx, gpu_layer, layer_w, t):
    _say(f"moe prefill i8 t={t}")
    x = synth.f32_normal(synth.seed_of(9300 + t), t * H).reshape(t, H)
    idx, gates = synth.zipf_routing(synth.seed_of(9400 + t), t, E, K)
    dout = ctx.empty((t, H), np.float32)
    dx, di, dg = ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates)
    gpu_layer.prefill(dx, di, dg, dout)
    st, want = O.moe_prefill_i8(x, idx, gates, *layer_w[1:], E, I)
    assert st == 0
    assert_rel(dout.numpy(), want, 1e-3)
    again = ctx.empty((t, H), np.float32)
    gpu_layer.prefill(dx, di, dg, again)
    assert np.array_equal(dout.numpy(), again.numpy())


@pytest.mark.parametrize("t", [130, 300])
def test_moe_prefill_i8_hot_expert_and_shared(ctx, layer_w, t):
    """Every token routed to the same six experts (t rows each: 64-row tiles
    per expert, the last one ragged) plus the shared expert, whose gate/up
    runs as extra units of the routed launch (3 and 5 row tiles)."""
    from franken_ocr_amd.engine import MoeLayer

    si = 1792
    _say(f"moe prefill i8 shared t={t}")
    x = synth.f32_normal(synth.seed_of(9500), t * H).reshape(t, H)
    idx = np.tile(np.array([[40, 3, 17, 63, 0, 9]], np.uint32), (t, 1))
    gates = synth.f32_uniform(synth.seed_of(9501), t * K, 0.05, 1.0).reshape(t, K)
    sw = [synth.int8_uniform(synth.seed_of(9502), si * H), synth.f32_uniform(synth.seed_of(9503), si, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(9504), si * H), synth.f32_uniform(synth.seed_of(9505), si, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(9506), H * si), synth.f32_uniform(synth.seed_of(9507), H, 1e-3, 2e-2)]
    L = MoeLayer(H, I, E, K, *layer_w, ctx=ctx)
    L.set_shared(si, *sw)
    dout = ctx.empty((t, H), np.float32)
    L.prefill(ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates), dout, with_shared=True)
    st, want = O.moe_prefill_i8(x, idx, gates, *layer_w[1:], E, I, shared=(si, *sw))
    assert st == 0
    assert_rel(dout.numpy(), want, 1e-3)


def test_moe_prefill_i8_plan_forms_agree(ctx, gpu_layer):
    """1400 tokens (8400 pairs) take the plan's round-by-round scatter, 700
    its barrier-free form for up to 8192 pairs; a token's output does not
    depend on the other tokens of the call (exact i32 sums per row, its own
    epilogue, its own ascending-expert combine), so one call over 1400 rows
    equals two calls over 700 bit for bit."""
    t = 1400
    _say(f"moe prefill i8 plan forms t={t}")
    x = synth.f32_normal(synth.seed_of(9600), t * H).reshape(t, H)
    idx, gates = synth.zipf_routing(synth.seed_of(9601), t, E, K)
    whole = ctx.empty((t, H), np.float32)
    gpu_layer.prefill(ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates), whole)
    halves = []
    for a, b in ((0, t // 2), (t // 2, t)):
        out = ctx.empty((b - a, H), np.float32)
        gpu_layer.prefill(ctx.to_device(x[a:b]), ctx.to_device(idx[a:b]), ctx.to_device(gates[a:b]), out)
        halves.append(out.numpy())
    assert np.array_equal(whole.numpy(), np.concatenate(halves))


def test_moe_prefill_i8_bad_expert_index(ctx, gpu_layer):
    from franken_ocr_amd._abi import ContractViolation

    t = 4
    idx = np.zeros((t, K), np.uint32)
    idx[2, 3] = E
    dout = ctx.empty((t, H), np.float32)
    with pytest.raises(ContractViolation, match="expert index out of range"):
        gpu_layer.prefill(ctx.to_device(np.ones((t, H), np.float32)), ctx.to_device(idx),
                          ctx.to_device(np.ones((t, K), np.float32)), dout)
