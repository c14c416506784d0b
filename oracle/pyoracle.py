"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg — never by the product package.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# FOCR_ORACLE_LIB selects another build of the oracle (the sanitized one in _san/).
LIB_PATH = Path(os.environ.get("FOCR_ORACLE_LIB") or HERE / "liboracle.so")

_P = C.c_void_p
_SZ = C.c_size_t

_SIGS = {
    "oracle_igemm_s8s8": ([_P, _P, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_igemm_u8s8": ([_P, _P, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_xs32": ([_P], C.c_uint32),
    "oracle_selftest_n_shapes": ([], _SZ),
    "oracle_selftest_shape": ([_SZ, _P, _P, _P, _P, _P], C.c_int),
    "oracle_selftest_fill_s8": ([_SZ, _P, _P], C.c_int),
    "oracle_selftest_fill_u8": ([_SZ, _P, _P], C.c_int),
    "oracle_quantize_row_i8": ([_P, _SZ, _P], C.c_float),
    "oracle_quantize_row_i8_te": ([_P, _SZ, _P], C.c_float),
    "oracle_gemv_i8_batched": ([_P, _SZ, _P, _P, _SZ, _SZ, _P, _P, _P, _P], None),
    "oracle_dequant_i8": ([_P, _SZ, _SZ, _P, _P, _P], None),
    "oracle_argmax_row": ([_P, _SZ, _P], C.c_int),
    "oracle_lm_head_i8": ([_P, _SZ, _P, _P, _SZ, _SZ, _P, _P], C.c_int),
    "oracle_ngram_bans": ([_P, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _P], _SZ),
    "oracle_sample": ([_P, _SZ, _P, _SZ, _SZ, _SZ, _P, _SZ, _P, _P], C.c_int),
    "oracle_route": ([_P, _SZ, _SZ, _P, _SZ, _SZ, C.c_int, C.c_float, _P, _P, _P], C.c_int),
    "oracle_silu": ([C.c_float], C.c_float),
    "oracle_expert_i8": ([_P, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P], None),
    "oracle_moe_decode": ([_P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, C.c_int, C.c_float,
                           _P, _P, _P, _P, _P, _P, _SZ, _P, _P, _P], C.c_int),
    "oracle_sign_extend_nibble": ([C.c_uint8], C.c_int8),
    "oracle_unpack_byte": ([C.c_uint8, _P, _P], None),
    "oracle_unpack_to_i8": ([_P, _SZ, _SZ, _P], C.c_int),
    "oracle_igemm_s4s8_packed": ([_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_s4s8_group_i32": ([_P, _P, _SZ, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_moe_prefill_i4": ([_P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P],
                              C.c_int),
    "oracle_quantize_row_dynamic": ([_P, _SZ, _P], C.c_float),
    "oracle_rms_norm": ([_P, _SZ, _P, C.c_float, _P], None),
    "oracle_rope": ([_P, _SZ, _SZ, _SZ, C.c_float], C.c_int),
    "oracle_linear_i8_dynamic": ([_P, _SZ, _SZ, _P, _P, _SZ, _P, _P, _P, _P], C.c_int),
    "oracle_moe_prefill_i8": ([_P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _SZ, _P], C.c_int),
    "oracle_quantize_int8_f32": ([_P, _SZ, _SZ, _P, _P], C.c_int),
    "oracle_pack_int4_f32": ([_P, _SZ, _SZ, _SZ, _P, _P], C.c_int),
    "oracle_ring_write": ([_P, _P, _P, _P, _P, _P, _P], C.c_int),
    "oracle_decode_attention": ([_P, _P, _SZ, _SZ, _P, _P, _SZ, _P, _P], C.c_int),
    "oracle_chunk_prefill_attention": ([_P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_prefill_attention": ([_P, _P, _P, _SZ, _SZ, _SZ, _P], C.c_int),
    "oracle_chunk_prefill_attention_f32": ([_P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _P], C.c_int),
    "cpu_detect_tier": ([], C.c_int),
    "cpu_tier_available": ([C.c_int], C.c_int),
    "cpu_tier_tag": ([C.c_int], C.c_char_p),
    "cpu_tier_feature": ([C.c_int], C.c_char_p),
    "cpu_set_threads": ([C.c_int], C.c_int),
    "cpu_threads": ([], C.c_int),
    "cpu_igemm_s8s8": ([C.c_int, _P, _P, _SZ, _SZ, _SZ, _P], None),
    "cpu_gemv_i8": ([C.c_int, _P, _SZ, _P, _P, _SZ, _SZ, _P], None),
    "cpu_lm_head_i8": ([C.c_int, _P, _SZ, _P, _P, _SZ, _SZ, _P, _P], None),
    "cpu_moe_decode": ([C.c_int, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, C.c_int, C.c_float,
                        _P, _P, _P], C.c_int),
    "cpu_igemm_s8s8_batched": ([C.c_int, _P, _P, _SZ, _SZ, _SZ, _SZ, _P], None),
    "cpu_linear_i8_dynamic": ([C.c_int, _P, _SZ, _SZ, _P, _P, _SZ, _P], None),
    "cpu_moe_decode_shared": ([C.c_int, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, C.c_int,
                               C.c_float, _P, _P, _P, _P, _P, _P, _SZ, _P, _P, _P], C.c_int),
    "cpu_decoder_layer_step": ([C.c_int, _P, _SZ, _P, _P, _P, _SZ, _P, _P, _P, _P, _P, _P, _P, C.c_float,
                                C.c_float, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                _P, _P, _SZ], C.c_int),
    "cpu_igemm_s4s8": ([C.c_int, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P], None),
    "cpu_moe_prefill_i4": ([C.c_int, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _SZ, _P, _P, _P, _P, _P, _P, _P],
                           C.c_int),
}

_lib = None


def build() -> Path:
    """Compile oracle/*.c into oracle/liboracle.so (gcc, via the Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = C.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = res
        _lib = h
    return _lib


def p(a: np.ndarray | None) -> C.c_void_p:
    if a is None:
        return C.c_void_p()
    return a.ctypes.data_as(C.c_void_p)


# ---- numpy-friendly wrappers ------------------------------------------------
def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def igemm_s8s8(a, b, m, k, n, out=None):
    out = np.zeros(m * n, np.int32) if out is None else out
    a, b = _c(a, np.int8), _c(b, np.int8)
    assert lib().oracle_igemm_s8s8(p(a), p(b), m, k, n, p(out)) == 0
    return out


def igemm_u8s8(a, b, m, k, n, out=None):
    out = np.zeros(m * n, np.int32) if out is None else out
    a, b = _c(a, np.uint8), _c(b, np.int8)
    assert lib().oracle_igemm_u8s8(p(a), p(b), m, k, n, p(out)) == 0
    return out


def selftest_case(i, unsigned=False):
    m, k, n, seed = C.c_size_t(), C.c_size_t(), C.c_size_t(), C.c_uint32()
    label = C.c_char_p()
    assert lib().oracle_selftest_shape(i, C.byref(label), C.byref(m), C.byref(k), C.byref(n), C.byref(seed)) == 0
    m, k, n = m.value, k.value, n.value
    a = np.zeros(m * k, np.uint8 if unsigned else np.int8)
    b = np.zeros(n * k, np.int8)
    f = lib().oracle_selftest_fill_u8 if unsigned else lib().oracle_selftest_fill_s8
    assert f(i, p(a), p(b)) == 0
    return label.value.decode(), m, k, n, seed.value, a, b


def quantize_row_i8(x, ties_even=False):
    x = _c(x, np.float32)
    q = np.zeros(x.size, np.int8)
    f = lib().oracle_quantize_row_i8_te if ties_even else lib().oracle_quantize_row_i8
    s = f(p(x), x.size, p(q))
    return q, np.float32(s)


def gemv_i8_batched(x, w, scales, n, k):
    x = _c(x, np.float32).reshape(-1, k)
    m = x.shape[0]
    xq = np.zeros(m * k, np.int8)
    a_s = np.zeros(m, np.float32)
    acc = np.zeros(m * n, np.int32)
    y = np.zeros(m * n, np.float32)
    lib().oracle_gemv_i8_batched(p(x), m, p(_c(w, np.int8)), p(_c(scales, np.float32)), n, k, p(xq), p(a_s), p(acc), p(y))
    return y.reshape(m, n), acc.reshape(m, n), xq.reshape(m, k), a_s


def argmax_row(logits):
    logits = _c(logits, np.float32)
    idx = C.c_uint32()
    st = lib().oracle_argmax_row(p(logits), logits.size, C.byref(idx))
    return st, idx.value


def lm_head_i8(x, w, scales, n, k):
    x = _c(x, np.float32).reshape(-1, k)
    m = x.shape[0]
    logits = np.zeros(m * n, np.float32)
    am = np.zeros(m, np.uint32)
    assert lib().oracle_lm_head_i8(p(x), m, p(_c(w, np.int8)), p(_c(scales, np.float32)), n, k, p(logits), p(am)) == 0
    return logits.reshape(m, n), am


def ngram_bans(seq, ngram, window, vocab, whitelist=()):
    """sampler.rs:191-235: the banned ids in scan order (repeats kept)."""
    seq = _c(seq, np.uint32)
    white = _c(list(whitelist), np.uint32)
    out = np.zeros(max(seq.size, 1), np.uint32)
    nb = lib().oracle_ngram_bans(p(seq) if seq.size else None, seq.size, ngram, window,
                                 p(white) if white.size else None, white.size, vocab, p(out))
    return out[:nb]


def sample(row, seq, ngram, window, whitelist=()):
    """sampler.rs:346-395 greedy sample: (status, token, masked row)."""
    row = _c(row, np.float32).reshape(-1)
    seq = _c(seq, np.uint32)
    white = _c(list(whitelist), np.uint32)
    masked = np.zeros(max(row.size, 1), np.float32)
    tok = C.c_uint32()
    st = lib().oracle_sample(p(row) if row.size else None, row.size, p(seq) if seq.size else None, seq.size, ngram,
                             window, p(white) if white.size else None, white.size, p(masked), C.byref(tok))
    return st, tok.value, masked[:row.size]


def route(hidden, gate, n_experts, top_k, norm_topk=False, routed_scale=1.0):
    hidden = _c(hidden, np.float32)
    t, h = hidden.shape
    idx = np.zeros(t * top_k, np.uint32)
    w = np.zeros(t * top_k, np.float32)
    probs = np.zeros(t * n_experts, np.float32)
    st = lib().oracle_route(p(hidden), t, h, p(_c(gate, np.float32)), n_experts, top_k, int(norm_topk),
                            float(routed_scale), p(idx), p(w), p(probs))
    return st, idx.reshape(t, top_k), w.reshape(t, top_k), probs.reshape(t, n_experts)


def expert_i8(x, h, inter, wg, sg, wu, su, wd, sd):
    x = _c(x, np.float32)
    y = np.zeros(h, np.float32)
    act = np.zeros(inter, np.float32)
    aq = np.zeros(inter, np.int8)
    as2 = C.c_float()
    lib().oracle_expert_i8(p(x), h, inter, p(_c(wg, np.int8)), p(_c(sg, np.float32)), p(_c(wu, np.int8)),
                           p(_c(su, np.float32)), p(_c(wd, np.int8)), p(_c(sd, np.float32)), p(y), p(act), p(aq),
                           C.byref(as2))
    return y, act, aq, np.float32(as2.value)


def moe_decode(hidden, router, wg, sg, wu, su, wd, sd, n_experts, top_k, inter, norm_topk=False, routed_scale=1.0,
               shared=None):
    hidden = _c(hidden, np.float32)
    t, h = hidden.shape
    out = np.zeros(t * h, np.float32)
    idx = np.zeros(t * top_k, np.uint32)
    gates = np.zeros(t * top_k, np.float32)
    if shared is None:
        sh = [None] * 6
        si = 0
    else:
        si = shared[0]
        sh = [_c(shared[1], np.int8), _c(shared[2], np.float32), _c(shared[3], np.int8), _c(shared[4], np.float32),
              _c(shared[5], np.int8), _c(shared[6], np.float32)]
    st = lib().oracle_moe_decode(p(hidden), t, h, inter, n_experts, top_k, p(_c(router, np.float32)),
                                 p(_c(wg, np.int8)), p(_c(sg, np.float32)), p(_c(wu, np.int8)),
                                 p(_c(su, np.float32)), p(_c(wd, np.int8)), p(_c(sd, np.float32)), int(norm_topk),
                                 float(routed_scale), *[p(a) for a in sh], si, p(out), p(idx), p(gates))
    return st, out.reshape(t, h), idx.reshape(t, top_k), gates.reshape(t, top_k)


def unpack_to_i8(packed, n, k):
    packed = _c(packed, np.uint8)
    out = np.zeros(n * k, np.int8)
    st = lib().oracle_unpack_to_i8(p(packed), n, k, p(out))
    return st, out


def igemm_s4s8_packed(a, b_packed, scales, group, m, k, n):
    out = np.zeros(m * n, np.float32)
    st = lib().oracle_igemm_s4s8_packed(p(_c(a, np.int8)), p(_c(b_packed, np.uint8)), p(_c(scales, np.float32)),
                                        group, m, k, n, p(out))
    return st, out


def s4s8_group_i32(a, b_packed, group, m, k, n):
    out = np.zeros(m * n * (k // group), np.int32)
    st = lib().oracle_s4s8_group_i32(p(_c(a, np.int8)), p(_c(b_packed, np.uint8)), group, m, k, n, p(out))
    return st, out


def quantize_int8_f32(w, n, k):
    w = _c(w, np.float32)
    q = np.zeros(n * k, np.int8)
    s = np.zeros(n, np.float32)
    st = lib().oracle_quantize_int8_f32(p(w), n, k, p(q), p(s))
    return st, q, s


def pack_int4_f32(w, n, k, group):
    w = _c(w, np.float32)
    packed = np.zeros(n * k // 2, np.uint8)
    s = np.zeros(n * (k // group), np.float32)
    st = lib().oracle_pack_int4_f32(p(w), n, k, group, p(packed), p(s))
    return st, packed, s


def moe_prefill_i4(x, idx, gates, group, wg, sg, wu, su, wd, sd, n_experts, inter):
    x = _c(x, np.float32)
    t, h = x.shape
    top_k = idx.shape[1]
    out = np.zeros(t * h, np.float32)
    xq = np.zeros(t * h, np.int8)
    xs = np.zeros(t, np.float32)
    st = lib().oracle_moe_prefill_i4(p(x), t, h, inter, n_experts, top_k, p(_c(idx, np.uint32)),
                                     p(_c(gates, np.float32)), group, p(_c(wg, np.uint8)), p(_c(sg, np.float32)),
                                     p(_c(wu, np.uint8)), p(_c(su, np.float32)), p(_c(wd, np.uint8)),
                                     p(_c(sd, np.float32)), p(out), p(xq), p(xs))
    return st, out.reshape(t, h), xq.reshape(t, h), xs


def quantize_row_dynamic(x):
    """docs/focrq-format.md:296-320 dynamic activation rule (ties-even, true division)."""
    x = _c(x, np.float32)
    q = np.zeros(x.size, np.int8)
    s = lib().oracle_quantize_row_dynamic(p(x), x.size, p(q))
    return q, np.float32(s)


def linear_i8_dynamic(x, w, w_scales, n, bias=None):
    """nn::linear_int8_dynamic (nn.rs:151-173): y [m, n], xq [m, k], x scales [m]."""
    x = _c(x, np.float32)
    m, k = x.shape
    y = np.zeros(m * n, np.float32)
    xq = np.zeros(m * k, np.int8)
    xs = np.zeros(m, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    st = lib().oracle_linear_i8_dynamic(p(x), m, k, p(_c(w, np.int8)), p(_c(w_scales, np.float32)), n,
                                        None if b is None else p(b), p(y), p(xq), p(xs))
    return st, y.reshape(m, n), xq.reshape(m, k), xs


def moe_prefill_i8(x, idx, gates, wg, sg, wu, su, wd, sd, n_experts, inter, shared=None):
    """moe_block_i8 (decoder.rs:2142-2181) over given routing, int8 experts."""
    x = _c(x, np.float32)
    t, h = x.shape
    top_k = idx.shape[1]
    out = np.zeros(t * h, np.float32)
    if shared is None:
        sh = [None] * 6
        si = 0
    else:
        si = shared[0]
        sh = [p(_c(a, np.int8 if i % 2 == 0 else np.float32)) for i, a in enumerate(shared[1:])]
    st = lib().oracle_moe_prefill_i8(p(x), t, h, inter, n_experts, top_k, p(_c(idx, np.uint32)),
                                     p(_c(gates, np.float32)), p(_c(wg, np.int8)), p(_c(sg, np.float32)),
                                     p(_c(wu, np.int8)), p(_c(su, np.float32)), p(_c(wd, np.int8)),
                                     p(_c(sd, np.float32)), *sh, si, p(out))
    return st, out.reshape(t, h)


def rms_norm(x, w=None, eps=1e-6):
    """nn::rms_norm as this build fixes it (f64 sum of squares); rows of x."""
    x = _c(x, np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros_like(rows)
    wc = None if w is None else _c(w, np.float32)
    for r in range(rows.shape[0]):
        lib().oracle_rms_norm(p(rows[r]), rows.shape[1], None if wc is None else p(wc), float(eps), p(out[r]))
    return out.reshape(x.shape)


def rope(x, pos, n_heads=10, head_dim=128, theta=10000.0):
    """RopeTable::build + apply_rope (decoder.rs:150-268) on one row."""
    y = np.array(_c(x, np.float32), copy=True)
    assert lib().oracle_rope(p(y), n_heads, head_dim, int(pos), float(theta)) == 0
    return y


def decoder_layer_step(x, positions, rings, lw, eps=1e-6, theta=10000.0):
    """One layer of batched_decode_step_i8_streams (decoder.rs:2812-2933) for
    rows x [B, H] (stream s at positions[s], its RingCache rings[s]):
    RMSNorm -> fused qkv GEMV -> RoPE -> ring write -> R-SWA -> o_proj ->
    residual -> RMSNorm -> decode_mlp_i8 (MoE: route_default + the shared
    expert; dense: one SwiGLU expert) -> residual. lw: dict with input_ln,
    post_ln, qkv (w, s), o (w, s) and either moe (router, wg, sg, wu, su, wd,
    sd, n_experts, top_k, inter, shared) or dense (wg, sg, wu, su, wd, sd, inter)."""
    x = _c(x, np.float32)
    B, H = x.shape
    D = 10 * 128
    out = np.zeros_like(x)
    normed = rms_norm(x, lw["input_ln"], eps)
    qkv = gemv_i8_batched(normed, lw["qkv"][0], lw["qkv"][1], 3 * D, H)[0]
    ctx = np.zeros((B, D), np.float32)
    for s in range(B):
        q = rope(qkv[s, :D], positions[s], theta=theta)
        k = rope(qkv[s, D:2 * D], positions[s], theta=theta)
        rings[s].write(k, qkv[s, 2 * D:])
        st, ctx[s] = rings[s].attend(q)
        assert st == 0
    attn = gemv_i8_batched(ctx, lw["o"][0], lw["o"][1], H, D)[0]
    h = (x + attn).astype(np.float32)
    normed2 = rms_norm(h, lw["post_ln"], eps)
    if "moe" in lw:
        m = lw["moe"]
        st, mlp, _, _ = moe_decode(normed2, m["router"], m["wg"], m["sg"], m["wu"], m["su"], m["wd"], m["sd"],
                                   m["n_experts"], m["top_k"], m["inter"], norm_topk=False, routed_scale=1.0,
                                   shared=m.get("shared"))
        assert st == 0
    else:
        d = lw["dense"]
        mlp = np.stack([expert_i8(normed2[s], H, d["inter"], d["wg"], d["sg"], d["wu"], d["su"], d["wd"], d["sd"])[0]
                        for s in range(B)])
    out[:] = (h + mlp).astype(np.float32)
    return out


def decoder_layer_prefill(x, c0, k_prev, v_prev, lw, eps=1e-6, theta=10000.0):
    """One layer of prefill_with_cache_i8_chunked (decoder.rs:2461-2486) for
    the chunk rows x [cs, H] at positions c0 .. c0 + cs - 1, given the
    earlier chunks' RoPE'd K / V k_prev, v_prev [c0, D] (token-major):
    RMSNorm -> q / k / v = linear_int8_dynamic -> RoPE -> chunk_prefill_attention
    over [0, c0 + cs) -> o_proj -> residual -> RMSNorm -> prefill_mlp_i8 ->
    residual. lw as decoder_layer_step's, with moe (router, wg, sg, wu, su,
    wd, sd, n_experts, top_k, inter, shared) or dense (wg, sg, wu, su, wd, sd,
    inter). Returns (out [cs, H], k [cs, D], v [cs, D], idx [cs, top_k] or None)."""
    x = _c(x, np.float32)
    cs, H = x.shape
    D = 10 * 128
    normed = rms_norm(x, lw["input_ln"], eps)
    st, qkv, _, _ = linear_i8_dynamic(normed, lw["qkv"][0], lw["qkv"][1], 3 * D)
    assert st == 0
    q = np.stack([rope(qkv[r, :D], c0 + r, theta=theta) for r in range(cs)])
    k = np.stack([rope(qkv[r, D:2 * D], c0 + r, theta=theta) for r in range(cs)])
    v = np.ascontiguousarray(qkv[:, 2 * D:])
    kp = np.concatenate([np.asarray(k_prev, np.float32).reshape(c0, D), k])
    vp = np.concatenate([np.asarray(v_prev, np.float32).reshape(c0, D), v])
    st, ctx = chunk_prefill_attention(q, kp, vp, 10, 128, c0)
    assert st == 0
    st, attn, _, _ = linear_i8_dynamic(ctx, lw["o"][0], lw["o"][1], H)
    assert st == 0
    h = (x + attn).astype(np.float32)
    normed2 = rms_norm(h, lw["post_ln"], eps)
    idx = None
    if "moe" in lw:
        m = lw["moe"]
        # route_default (moe.rs:273-280): norm_topk_prob false, scaling 1.0
        st, idx, gates, _ = route(normed2, m["router"], m["n_experts"], m["top_k"], norm_topk=False, routed_scale=1.0)
        assert st == 0
        st, mlp = moe_prefill_i8(normed2, idx, gates, m["wg"], m["sg"], m["wu"], m["su"], m["wd"], m["sd"],
                                 m["n_experts"], m["inter"], shared=m.get("shared"))
    else:
        d = lw["dense"]
        # expert_mlp_i8 (decoder.rs:2120-2135) is moe_block_i8's body for one
        # expert taking every row at weight 1.0 (w * y with w = 1 is exact)
        one_i = np.zeros((cs, 1), np.uint32)
        one_g = np.ones((cs, 1), np.float32)
        st, mlp = moe_prefill_i8(normed2, one_i, one_g, d["wg"], d["sg"], d["wu"], d["su"], d["wd"], d["sd"], 1,
                                 d["inter"])
    assert st == 0
    out = (h + mlp.reshape(cs, H)).astype(np.float32)
    return out, k, v, idx


class Ring:
    """One stream's RingCache regions in host memory (head-major f32)."""

    H, D, W = 10, 128, 128

    def __init__(self, ref_cap):
        self.ref_cap = ref_cap
        self.ref_k = np.zeros((self.H, ref_cap, self.D), np.float32)
        self.ref_v = np.zeros((self.H, ref_cap, self.D), np.float32)
        self.ring_k = np.zeros((self.H, self.W, self.D), np.float32)
        self.ring_v = np.zeros((self.H, self.W, self.D), np.float32)
        self.prefill_len = 0
        self.ring_len = C.c_uint32(0)
        self.ring_pos = C.c_uint32(0)

    def record_prefill(self, k, v, seq):
        self.ref_k[:, :seq] = k.reshape(self.H, seq, self.D)
        self.ref_v[:, :seq] = v.reshape(self.H, seq, self.D)
        self.prefill_len = seq
        self.ring_len.value = 0
        self.ring_pos.value = 0

    def write(self, k_step, v_step):
        slot = C.c_uint32()
        st = lib().oracle_ring_write(p(self.ring_k), p(self.ring_v), C.byref(self.ring_len), C.byref(self.ring_pos),
                                     p(_c(k_step, np.float32)), p(_c(v_step, np.float32)), C.byref(slot))
        assert st == 0
        return slot.value

    def attend(self, q):
        out = np.zeros(self.H * self.D, np.float32)
        st = lib().oracle_decode_attention(p(self.ref_k), p(self.ref_v), self.ref_cap, self.prefill_len,
                                           p(self.ring_k), p(self.ring_v), self.ring_len.value,
                                           p(_c(q, np.float32)), p(out))
        return st, out


def chunk_prefill_attention(q_chunk, k_prefix, v_prefix, num_heads, head_dim, c0):
    """decoder.rs:1282-1340: context [cs, num_heads*head_dim] of the chunk's queries."""
    q_chunk = _c(q_chunk, np.float32)
    cs = q_chunk.shape[0]
    c1 = k_prefix.shape[0]
    out = np.zeros((cs, num_heads * head_dim), np.float32)
    st = lib().oracle_chunk_prefill_attention(p(q_chunk), cs, p(_c(k_prefix, np.float32)), p(_c(v_prefix, np.float32)),
                                              c1, num_heads, head_dim, c0, p(out))
    return st, out


def prefill_attention_f32(q, k, v, num_heads, head_dim):
    """The f32 restatement in the reference's described order (ascending dims, keys)."""
    q = _c(q, np.float32)
    out = np.zeros(q.shape, np.float32)
    st = lib().oracle_chunk_prefill_attention_f32(p(q), q.shape[0], p(_c(k, np.float32)), p(_c(v, np.float32)),
                                                  q.shape[0], num_heads, head_dim, 0, p(out))
    return st, out


def prefill_attention(q, k, v, num_heads, head_dim):
    """decoder.rs:568-640: full causal multi-head attention [seq, num_heads*head_dim]."""
    q = _c(q, np.float32)
    out = np.zeros(q.shape, np.float32)
    st = lib().oracle_prefill_attention(p(q), p(_c(k, np.float32)), p(_c(v, np.float32)), q.shape[0], num_heads,
                                        head_dim, p(out))
    return st, out
