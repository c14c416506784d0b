"""Prefill attention (decoder.rs:568-640) and chunked prefill attention
(decoder.rs:1282-1340) on the f32 matrix cores, against the CPU oracle.

Tolerance: rel 1e-4 (the attention tolerance) against the oracle, which
evaluates the attention math in float64 and rounds once: the reference's
attention runs in ft-kernel-cpu (un-vendored, f32, unknown summation order),
and any f32 evaluation is about 1e-4 from the exact result at 1024 keys, so
the oracle is the exact attention they all approximate. The f32 restatement
of the reference's described order is measured beside it (its distance from
the oracle is printed; it is what the reference's own f32 result is expected
to look like). The error of an element is |got - want| / max(|want|, f), with
the floor f = 1e-2 * max|want| over the element's row: attention outputs are
convex blends of value rows and individual elements can be arbitrarily close
to 0, where a pure relative error measures only the cancellation. The plain
per-element maximum is printed beside it.
"""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from franken_ocr_amd.engine import prefill_chunk_bounds
from oracle import pyoracle as O

NH, D = 10, 128
DIM = NH * D


def test_prefill_chunk_bounds_cover_contiguously_in_order():
    # decoder.rs:3481-3497
    for seq in (0, 1, 2, 5, 7, 16, 17):
        for chunk in (1, 2, 3, 5, 7, 16, 64):
            cursor = 0
            for c0, c1 in prefill_chunk_bounds(seq, chunk):
                assert c0 == cursor and c1 > c0 and c1 - c0 <= chunk and c1 <= seq
                cursor = c1
            assert cursor == seq
    assert prefill_chunk_bounds(5, 0) == [(i, i + 1) for i in range(5)]  # clamped to >= 1


def _say(msg):
    print(f"[gpu-attn] {msg}", flush=True)


def _rel(got, want):
    want = np.asarray(want, np.float64)
    floor = np.max(np.abs(want), axis=-1, keepdims=True) * 1e-2
    err = np.abs(got.astype(np.float64) - want)
    plain = float(np.max(err / np.maximum(np.abs(want), 1e-30)))
    return float(np.max(err / np.maximum(np.abs(want), floor))), plain


def _check(got, q, k, v):
    st, want = O.prefill_attention(q, k, v, NH, D)
    assert st == 0
    st, f32 = O.prefill_attention_f32(q, k, v, NH, D)
    rel, plain = _rel(got, want)
    _say(f"  rel {rel:.2e} (plain per-element {plain:.2e}); f32 reference-order restatement vs oracle "
         f"{_rel(f32, want)[0]:.2e}")
    assert rel <= 1e-4


def _qkv(seed, seq):
    return [synth.f32_normal(synth.seed_of(seed + i), seq * DIM).reshape(seq, DIM) for i in range(3)]


@pytest.mark.gpu
@pytest.mark.parametrize("seq", [1, 5, 64, 100, 257, 1024])
def test_prefill_attention_matches_oracle(ctx, seq):
    from franken_ocr_amd.engine import prefill_attention

    _say(f"prefill_attention seq={seq}")
    q, k, v = _qkv(700 + seq, seq)
    out = ctx.empty((seq, DIM), np.float32)
    prefill_attention(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), NH, D, out)
    _check(out.numpy(), q, k, v)


@pytest.mark.gpu
@pytest.mark.parametrize("seq,chunk", [(300, 1), (300, 7), (300, 64), (300, 256), (300, 300), (2048, 256)])
def test_chunked_prefill_attention_matches_monolithic_oracle(ctx, seq, chunk):
    from franken_ocr_amd.engine import chunk_prefill_attention

    _say(f"chunk_prefill_attention seq={seq} chunk={chunk}")
    q, k, v = _qkv(800 + seq, seq)
    dk, dv = ctx.to_device(k), ctx.to_device(v)
    got = np.zeros((seq, DIM), np.float32)
    for c0, c1 in prefill_chunk_bounds(seq, chunk):
        out = ctx.empty((c1 - c0, DIM), np.float32)
        # the prefix views: the first c1 rows of the full K/V
        kp, vp = ctx.to_device(k[:c1]), ctx.to_device(v[:c1])
        chunk_prefill_attention(ctx.to_device(q[c0:c1]), kp, vp, NH, D, c0, out)
        got[c0:c1] = out.numpy()
    del dk, dv
    _check(got, q, k, v)


@pytest.mark.gpu
def test_rswa_prefill_chunk_fills_the_reference_block(ctx):
    from franken_ocr_amd.engine import RingCache

    G, chunk, cap = 600, 256, 1024
    _say(f"rswa_prefill_chunk G={G} chunk={chunk}")
    q, k, v = _qkv(900, G)
    cache = RingCache(2, cap, ctx=ctx)
    got = np.zeros((G, DIM), np.float32)
    for c0, c1 in prefill_chunk_bounds(G, chunk):
        out = ctx.empty((c1 - c0, DIM), np.float32)
        cache.prefill_chunk(1, ctx.to_device(q[c0:c1]), ctx.to_device(k[c0:c1]), ctx.to_device(v[c0:c1]), c0, out)
        got[c0:c1] = out.numpy()
    _check(got, q, k, v)
    assert cache.state(1)[:2] == (G, 0)
    # the reference block holds exactly record_prefill's head-major K/V
    regs = cache.regions(1)
    import ctypes as C

    from franken_ocr_amd import _abi

    def rd(ptr, n):
        a = np.empty(n, np.float32)
        _abi.call("focr_hip_d2h", ctx.handle, a.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), a.nbytes)
        return a

    ref_k = rd(regs["ref_k"], NH * cap * D).reshape(NH, cap, D)[:, :G]
    ref_v = rd(regs["ref_v"], NH * cap * D).reshape(NH, cap, D)[:, :G]
    assert np.array_equal(ref_k, k.reshape(G, NH, D).transpose(1, 0, 2))
    assert np.array_equal(ref_v, v.reshape(G, NH, D).transpose(1, 0, 2))
    # a decode step over the chunk-filled stream equals one over record_prefill
    other = RingCache(2, cap, ctx=ctx)
    kh = np.ascontiguousarray(k.reshape(G, NH, D).transpose(1, 0, 2))
    vh = np.ascontiguousarray(v.reshape(G, NH, D).transpose(1, 0, 2))
    other.record_prefill(1, ctx.to_device(kh), ctx.to_device(vh), G)
    other.record_prefill(0, ctx.to_device(kh), ctx.to_device(vh), G)
    cache.record_prefill(0, ctx.to_device(kh), ctx.to_device(vh), G)
    qs = synth.f32_normal(synth.seed_of(950), 2 * DIM).reshape(2, DIM)
    o1, o2 = ctx.empty((2, DIM), np.float32), ctx.empty((2, DIM), np.float32)
    cache.decode_attention(ctx.to_device(qs), o1)
    other.decode_attention(ctx.to_device(qs), o2)
    assert np.array_equal(o1.numpy(), o2.numpy())


@pytest.mark.gpu
def test_prefill_attention_contract_errors(ctx):
    from franken_ocr_amd import _abi
    from franken_ocr_amd.engine import RingCache, chunk_prefill_attention

    q = ctx.to_device(np.zeros((4, DIM), np.float32))
    kv = ctx.to_device(np.zeros((8, DIM), np.float32))
    out = ctx.empty((4, DIM), np.float32)
    with pytest.raises(_abi.ContractViolation, match=r"chunk_prefill_attention: chunk \[2, 6\) of 4 rows does not fit prefix 8"):
        chunk_prefill_attention(q, kv, kv, NH, D, 2, out)
    with pytest.raises(_abi.ContractViolation, match="head_dim 64 unsupported"):
        chunk_prefill_attention(q, kv, kv, 20, 64, 4, out)
    cache = RingCache(1, 16, ctx=ctx)
    with pytest.raises(_abi.StateError, match="chunk starts at 4"):
        cache.prefill_chunk(0, q, q, q, 4, out)
    with pytest.raises(_abi.StateError, match="exceeds ref_capacity 16"):
        big = ctx.to_device(np.zeros((20, DIM), np.float32))
        cache.prefill_chunk(0, big, big, big, 0, ctx.empty((20, DIM), np.float32))
