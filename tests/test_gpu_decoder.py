"""GPU tests of the whole batched decode step as one call
(focr_hip_decoder_step / focr_hip_decoder_step_sample: decoder.rs:2812-2933
batched_decode_step_i8 through every layer, :2943-2965 batched_lm_head_i8,
sampler.rs:168-186 argmax_row or :426-460 / :491-545 the n-gram-banned
greedy step).

* The one call equals the same work issued call by call (each layer's
  focr_hip_decoder_layer_step, the final RMSNorm, the LM head / sampler) bit
  for bit over two steps: hidden rows, logits, tokens, every MoE layer's
  expert ids and the caches' ring state. The per-layer calls are pinned to
  the oracle by tests/test_gpu_decoder_layer.py, the LM head and sampler by
  tests/test_gpu_tier.py and tests/test_gpu_sampler.py.
* A small decoder (the dense layer 0, two MoE layers with the shared expert,
  a 4096-row LM head) against the oracle's composition (decoder_layer_step
  per layer, rms_norm, lm_head_i8): logits rows within 1e-3 of their row max
  (the layers' tolerance; an int8 code can flip on a rounding boundary, see
  tests/test_gpu_layer_prefill.py), and, on those rows, every token the
  oracle's argmax where its top two logits are further apart than that.
* Argument errors: a cache list of the wrong length, caches with different
  stream counts, temperature > 0 (refused before any layer runs).
"""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import _abi, synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

H, D, K, V = 1280, 1280, 6, 4096
G = 24  # reference-block tokens per stream


def _say(msg):
    print(f"[gpu-decoder] {msg}", flush=True)


def _tame(lw):
    """Scales times 0.03: the layers' gain near 1, so three of them in a row
    keep activations O(1)."""
    lw = dict(lw)
    for key in ("qkv", "o"):
        lw[key] = (lw[key][0], (lw[key][1] * 0.03).astype(np.float32))
    if "moe" in lw:
        m = dict(lw["moe"])
        for key in ("sg", "su", "sd"):
            m[key] = (m[key] * 0.03).astype(np.float32)
        si, wg, sg, wu, su, wd, sd = m["shared"]
        m["shared"] = (si, wg, (sg * 0.03).astype(np.float32), wu, (su * 0.03).astype(np.float32), wd,
                       (sd * 0.03).astype(np.float32))
        lw["moe"] = m
    if "dense" in lw:
        d = dict(lw["dense"])
        for key in ("sg", "su", "sd"):
            d[key] = (d[key] * 0.03).astype(np.float32)
        lw["dense"] = d
    return lw


@pytest.fixture(scope="module")
def model():
    from test_gpu_decoder_layer import _weights

    lws = [_tame(_weights(21000, 6848)), _tame(_weights(21100)), _tame(_weights(21200))]
    final = synth.f32_uniform(synth.seed_of(21300), H, 0.5, 1.5)
    lm_w = synth.int8_uniform(synth.seed_of(21301), V * H)
    lm_s = synth.f32_uniform(synth.seed_of(21302), V, 1e-3, 2e-2)
    return lws, final, lm_w, lm_s


def _device(ctx, model):
    from test_gpu_decoder_layer import _gpu_layer

    from franken_ocr_amd.engine import Decoder, QInt8

    lws, final, lm_w, lm_s = model
    layers = [_gpu_layer(ctx, lw) for lw in lws]
    lm = QInt8(lm_w, lm_s, V, H, ctx)
    return layers, lm, Decoder(layers, final, lm, ctx=ctx)


def _caches(ctx, B, seed):
    from franken_ocr_amd.engine import RingCache

    out, rings = [], []
    for layer in range(3):
        kv = [(synth.f32_normal(synth.seed_of(seed + 100 * layer + 2 * s), 10 * G * 128),
               synth.f32_normal(synth.seed_of(seed + 100 * layer + 2 * s + 1), 10 * G * 128)) for s in range(B)]
        cache = RingCache(B, G, ctx=ctx)
        rs = []
        for s in range(B):
            cache.record_prefill(s, ctx.to_device(kv[s][0]), ctx.to_device(kv[s][1]), G)
            r = O.Ring(G)
            r.record_prefill(kv[s][0], kv[s][1], G)
            rs.append(r)
        out.append(cache)
        rings.append(rs)
    return out, rings


@pytest.mark.parametrize("B", [1, 5, 40])
def test_decoder_step_equals_the_calls_one_by_one(ctx, model, B):
    from franken_ocr_amd.engine import lm_head_i8, rms_norm

    _say(f"{B} streams, 2 steps: one call vs the calls one by one")
    layers, lm, dec = _device(ctx, model)
    final_dev = ctx.to_device(model[1])
    ca, _ = _caches(ctx, B, 22000)
    cb, _ = _caches(ctx, B, 22000)
    x0 = synth.f32_normal(synth.seed_of(22500), B * H).reshape(B, H)
    xa, xb = ctx.to_device(x0), ctx.to_device(x0)
    xn = ctx.empty((B, H), np.float32)
    pos = np.array([G + 2 * s for s in range(B)], np.uint32)
    for step in range(2):
        ta, tb = ctx.empty((B, 1), np.uint32), ctx.empty((B,), np.uint32)
        la, lb = ctx.empty((B, V), np.float32), ctx.empty((B, V), np.float32)
        ia = [ctx.empty((B, K), np.uint32) for _ in range(3)]
        ib = ctx.empty((3, B, K), np.uint32)
        for li, layer in enumerate(layers):
            layer.step(ca[li], pos + step, xa, ia[li] if li else None, check_route=False)
        rms_norm(xa, xn, final_dev)
        for r0 in range(0, B, 32):  # the LM head takes up to 32 rows per call
            r1 = min(B, r0 + 32)
            lm_head_i8(lm, xn.view_rows(r0, r1), ta.view_rows(r0, r1), la.view_rows(r0, r1))
        dec.step(cb, pos + step, xb, tb, lb, ib)
        assert np.array_equal(xa.numpy(), xb.numpy()), step
        assert np.array_equal(la.numpy(), lb.numpy()), step
        assert np.array_equal(ta.numpy().ravel(), tb.numpy()), step
        for li in (1, 2):
            assert np.array_equal(ia[li].numpy(), ib.numpy()[li]), (step, li)
        for li in range(3):
            assert [ca[li].state(s) for s in range(B)] == [cb[li].state(s) for s in range(B)]
    for c in ca + cb:
        c.free()
    dec.free()


def test_decoder_step_sample_equals_the_calls_one_by_one(ctx, model):
    from franken_ocr_amd.engine import lm_head_sample_i8, rms_norm

    B, cap = 3, 64
    _say(f"{B} streams, 3 steps with the n-gram sampler (appending)")
    layers, lm, dec = _device(ctx, model)
    final_dev = ctx.to_device(model[1])
    ca, _ = _caches(ctx, B, 23000)
    cb, _ = _caches(ctx, B, 23000)
    x0 = synth.f32_normal(synth.seed_of(23500), B * H).reshape(B, H)
    xa, xb = ctx.to_device(x0), ctx.to_device(x0)
    xn = ctx.empty((B, H), np.float32)
    hist0 = np.zeros((B, cap), np.uint32)
    hist0[:, :6] = synth.bytes_uniform(synth.seed_of(23600), B * 6).reshape(B, 6) % 64
    hlen0 = np.full(B, 6, np.uint32)
    ha, hb = ctx.to_device(hist0), ctx.to_device(hist0)
    na, nb = ctx.to_device(hlen0), ctx.to_device(hlen0)
    pos = np.array([G, G + 5, G + 9], np.uint32)
    for step in range(3):
        ta, tb = ctx.empty((B,), np.uint32), ctx.empty((B,), np.uint32)
        ea, eb = ctx.empty((B,), np.uint8), ctx.empty((B,), np.uint8)
        for li, layer in enumerate(layers):
            layer.step(ca[li], pos + step, xa, check_route=False)
        rms_norm(xa, xn, final_dev)
        lm_head_sample_i8(lm, xn, ta, ha, na, ngram_size=3, window=16, append=True, is_eos=ea, check=True)
        dec.step_sample(cb, pos + step, xb, tb, hb, nb, ngram_size=3, window=16, append=True, is_eos=eb)
        assert np.array_equal(xa.numpy(), xb.numpy()), step
        assert np.array_equal(ta.numpy(), tb.numpy()), step
        assert np.array_equal(ea.numpy(), eb.numpy()), step
        assert np.array_equal(ha.numpy(), hb.numpy()), step
        assert np.array_equal(na.numpy(), nb.numpy()), step
    assert (nb.numpy() == 9).all()
    for c in ca + cb:
        c.free()
    dec.free()


def test_decoder_step_matches_oracle(ctx, model):
    lws, final, lm_w, lm_s = model
    B = 4
    _say(f"{B} streams, 2 steps against the oracle's composition")
    layers, lm, dec = _device(ctx, model)
    caches, rings = _caches(ctx, B, 24000)
    x0 = synth.f32_normal(synth.seed_of(24500), B * H).reshape(B, H)
    dx = ctx.to_device(x0)
    pos = np.array([G, G + 4, G + 40, G + 1], np.uint32)
    rows, toks, checked = [], 0, 0
    for step in range(2):
        want = dx.numpy()  # continue from the device's state (the rings hold the same steps)
        for li, lw in enumerate(lws):
            want = O.decoder_layer_step(want, (pos + step).tolist(), rings[li], lw)
        logits_w, _ = O.lm_head_i8(O.rms_norm(want, final), lm_w, lm_s, V, H)
        tok, logits = ctx.empty((B,), np.uint32), ctx.empty((B, V), np.float32)
        dec.step(caches, pos + step, dx, tok, logits)
        got = logits.numpy()
        assert np.isfinite(got).all()
        rel = (np.abs(got.astype(np.float64) - logits_w) /
               np.maximum(np.abs(logits_w), np.abs(logits_w).max(axis=1, keepdims=True) * 1e-2)).max(axis=1)
        rows.extend(rel.tolist())
        t = tok.numpy()
        assert np.array_equal(t, got.argmax(axis=1)), "tokens are the argmax of the logits the step wrote"
        srt = np.sort(logits_w, axis=1)
        margin = (srt[:, -1] - srt[:, -2]) / np.abs(logits_w).max(axis=1)
        sure = (margin > 2e-3) & (rel <= 1e-3)
        checked += int(sure.sum())
        toks += int((t[sure] == logits_w.argmax(axis=1)[sure]).sum())
    rows = np.array(rows)
    _say(f"logit rows within 1e-3: {np.mean(rows <= 1e-3):.2f}, median {np.median(rows):.2e}; "
         f"tokens {toks}/{checked} where the oracle's margin is clear")
    assert np.mean(rows <= 1e-3) >= 0.75 and np.median(rows) <= 1e-4, rows
    assert toks == checked
    for c in caches:
        c.free()
    dec.free()


def test_decoder_step_argument_errors(ctx, model):
    from franken_ocr_amd.engine import RingCache

    layers, lm, dec = _device(ctx, model)
    caches, _ = _caches(ctx, 2, 25000)
    x = ctx.to_device(synth.f32_normal(synth.seed_of(25500), 2 * H).reshape(2, H))
    tok = ctx.empty((2,), np.uint32)
    pos = np.array([G, G], np.uint32)
    with pytest.raises(ValueError, match="2 caches for 3 layers"):
        dec.step(caches[:2], pos, x, tok)
    other = RingCache(3, G, ctx=ctx)
    with pytest.raises(_abi.FocrHipError, match="layer 1 cache holds 3 streams"):
        dec.step([caches[0], other, caches[2]], pos, x, tok)
    before = x.numpy()
    with pytest.raises(_abi.FocrHipError, match="temperature>0"):
        dec.step_sample(caches, pos, x, tok, temperature=0.7)
    assert np.array_equal(x.numpy(), before), "refused before any layer ran"
    assert [caches[0].state(s) for s in range(2)] == [(G, 0, 0)] * 2
    for c in caches + [other]:
        c.free()
    dec.free()


def _ref_block(ctx, cache, seq):
    import ctypes as C

    reg = cache.regions(0)
    out = []
    for key in ("ref_k", "ref_v"):
        full = np.empty((10, seq, 128), np.float32)  # ref_capacity == seq
        _abi.call("focr_hip_d2h", ctx.handle, full.ctypes.data_as(C.c_void_p), C.c_void_p(reg[key]), full.nbytes)
        out.append(full)
    return out


@pytest.mark.parametrize("chunk", [64, None])
def test_decoder_prefill_equals_the_layer_calls(ctx, model, chunk):
    """focr_hip_decoder_prefill (prefill_with_cache_i8_chunked, decoder.rs:
    2428-2520) is the per-layer prefill issued chunk by chunk, every layer per
    chunk, then the final norm + LM head + argmax of the last row: the same
    bits (hidden rows, every layer's reference block, expert ids, logits,
    token). chunk None: the monolithic schedule, one chunk of all rows."""
    from franken_ocr_amd.engine import RingCache, lm_head_i8, prefill_chunk_bounds, rms_norm

    seq = 150
    _say(f"prefill of {seq} rows, chunk {chunk}: one call vs the layer calls")
    layers, lm, dec = _device(ctx, model)
    final_dev = ctx.to_device(model[1])
    x0 = synth.f32_normal(synth.seed_of(23000), seq * H).reshape(seq, H)
    ca = [RingCache(1, seq, ctx=ctx) for _ in range(3)]
    cb = [RingCache(1, seq, ctx=ctx) for _ in range(3)]
    xa, xb = ctx.to_device(x0), ctx.to_device(x0)
    moe = ["moe" in lw for lw in model[0]]
    ia = ctx.empty((3 * seq, K), np.uint32)
    ib = np.zeros((3, seq, K), np.uint32)
    ta, tb = ctx.empty((1,), np.uint32), ctx.empty((1, 1), np.uint32)
    la, lb = ctx.empty((1, V), np.float32), ctx.empty((1, V), np.float32)
    dec.prefill(ca, 0, xa, seq, chunk=chunk, token=ta, logits=la, route_idx=ia)
    for c0, c1 in prefill_chunk_bounds(seq, chunk or seq):
        for li, layer in enumerate(layers):
            ri = ctx.empty((c1 - c0, K), np.uint32) if moe[li] else None
            layer.prefill(cb[li], 0, xb.view_rows(c0, c1), c0, ri)
            if ri is not None:
                ib[li, c0:c1] = ri.numpy()
    xn = ctx.empty((1, H), np.float32)
    rms_norm(xb.view_rows(seq - 1, seq), xn, final_dev)
    lm_head_i8(lm, xn, tb, lb)
    assert np.array_equal(xa.numpy(), xb.numpy())
    assert np.array_equal(ta.numpy().ravel(), tb.numpy().ravel())
    assert np.array_equal(la.numpy(), lb.numpy())
    got_idx = ia.numpy().reshape(3, seq, K)
    for li in range(3):
        assert ca[li].state(0) == (seq, 0, 0)
        for a, b in zip(_ref_block(ctx, ca[li], seq), _ref_block(ctx, cb[li], seq)):
            assert np.array_equal(a, b), f"layer {li} reference block"
        if moe[li]:
            assert np.array_equal(got_idx[li], ib[li])
    assert np.isfinite(xa.numpy()).all()


def test_decoder_prefill_argument_errors(ctx, model):
    from franken_ocr_amd.engine import RingCache

    layers, lm, dec = _device(ctx, model)
    x = ctx.empty((40, H), np.float32)
    small = [RingCache(1, 32, ctx=ctx) for _ in range(3)]
    with pytest.raises(_abi.FocrHipError, match="exceeds ref_capacity"):
        dec.prefill(small, 0, x, 40)
    with pytest.raises(_abi.FocrHipError, match="stream 1 >= num_streams 1"):
        dec.prefill(small, 1, x, 16)
    with pytest.raises(ValueError, match="2 caches for 3 layers"):
        dec.prefill(small[:2], 0, x, 16)
