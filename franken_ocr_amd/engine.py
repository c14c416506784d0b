"""Device-resident engine ops: the decoder functions one level above the tier.

Mirrors, on uploaded weights and device arrays:

* ``QInt8`` (tensor.rs:149-179) uploaded once (DecoderWeightCacheI8::build,
  decoder.rs:2018-2116),
* ``gemv_i8`` / ``gemv_i8_batched`` (decoder.rs:1607-1640, :2703-2747),
* ``lm_head_i8`` + ``argmax_row`` (decoder.rs:2275-2296, :2943-2965;
  sampler.rs:168-186),
* ``MoeLayer.route`` / ``MoeLayer.decode`` (moe.rs:181-266,
  decoder.rs:2199-2268),
* ``RingCache`` (rswa.rs:121-152, :389-513, :894-939, :1320-1367).

All work is queued on the context's stream; results come back with
``DeviceArray.numpy()``.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi
from .device import Context, DeviceArray, default_context

NUM_HEADS = 10
HEAD_DIM = 128
RING_WINDOW = 128


def _p(x) -> C.c_void_p:
    if x is None:
        return C.c_void_p()
    if isinstance(x, DeviceArray):
        return x.c_ptr
    if isinstance(x, np.ndarray):
        return x.ctypes.data_as(C.c_void_p)
    if isinstance(x, C.c_void_p):
        return x
    return C.c_void_p(int(x))


class QInt8:
    """Per-output-channel int8 weight ``w [n, k]`` + ``scales [n]`` in HBM."""

    def __init__(self, w: np.ndarray | DeviceArray, scales: np.ndarray | DeviceArray, n: int, k: int,
                 ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.n, self.k = int(n), int(k)
        self._h = C.c_void_p()
        if isinstance(w, DeviceArray):
            self._keep = (w, scales)
            _abi.call("focr_hip_qint8_from_device", self.ctx.handle, w.c_ptr, scales.c_ptr, self.n, self.k,
                      C.byref(self._h))
        else:
            w = np.ascontiguousarray(w, dtype=np.int8).reshape(-1)
            s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
            if w.size != self.n * self.k or s.size != self.n:
                raise _abi.ContractViolation(_abi.E_SHAPE, f"QInt8: w len {w.size} != n*k {self.n * self.k}"
                                             if w.size != self.n * self.k else
                                             f"QInt8: scales len {s.size} != n {self.n}")
            _abi.call("focr_hip_qint8_upload", self.ctx.handle, _p(w), _p(s), self.n, self.k, C.byref(self._h))

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_qint8_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


QUANT_HALF_AWAY, QUANT_TIES_EVEN, QUANT_DYNAMIC = 0, 1, 2


def quantize_rows_i8(x: DeviceArray, xq: DeviceArray, a_scales: DeviceArray, ties_even: bool = False,
                     rule: int | None = None) -> None:
    """Per-row int8 quantization: quantize_row_i8 (decoder.rs:1588-1597),
    quantize_row_i8_te (ties_even, :1647-1656), or rule=QUANT_DYNAMIC, the
    dynamic activation rule of linear_int8_dynamic (true division)."""
    m, k = x.shape
    r = (QUANT_TIES_EVEN if ties_even else QUANT_HALF_AWAY) if rule is None else int(rule)
    _abi.call("focr_hip_quantize_rows_i8", x.ctx.handle, x.c_ptr, m, k, xq.c_ptr, a_scales.c_ptr, r)


def linear_i8_dynamic(w: QInt8, x: DeviceArray, y: DeviceArray, bias: DeviceArray | None = None) -> None:
    """nn::linear_int8_dynamic (nn.rs:151-173) on the matrix cores: x [m, k]
    f32 -> y [m, n] f32 (k a multiple of 64)."""
    m = x.shape[0] if len(x.shape) > 1 else 1
    _abi.call("focr_hip_linear_i8_dynamic", w.ctx.handle, w.handle, x.c_ptr, m, _p(bias), y.c_ptr)


def gemv_i8(w: QInt8, x: DeviceArray, y: DeviceArray) -> None:
    """y[m, n] = dequant(quantize_row_i8(x[m]) . W^T) for m <= 32 rows."""
    m = x.shape[0] if len(x.shape) > 1 else 1
    _abi.call("focr_hip_gemv_i8", w.ctx.handle, w.handle, x.c_ptr, m, y.c_ptr)


def gemv_i8_prequant(w: QInt8, xq: DeviceArray, a_scales: DeviceArray, y: DeviceArray,
                     acc: DeviceArray | None = None) -> None:
    m = xq.shape[0] if len(xq.shape) > 1 else 1
    _abi.call("focr_hip_gemv_i8_prequant", w.ctx.handle, w.handle, xq.c_ptr, a_scales.c_ptr, m, y.c_ptr, _p(acc))


def lm_head_i8(w: QInt8, x: DeviceArray, argmax: DeviceArray, logits: DeviceArray | None = None) -> None:
    """LM head on already-normed rows: logits (optional) and argmax ids."""
    m = x.shape[0] if len(x.shape) > 1 else 1
    _abi.call("focr_hip_lm_head_i8", w.ctx.handle, w.handle, x.c_ptr, m, _p(logits), argmax.c_ptr)


def argmax_rows(logits: DeviceArray, argmax: DeviceArray) -> None:
    m, n = logits.shape
    _abi.call("focr_hip_argmax_rows", logits.ctx.handle, logits.c_ptr, m, n, argmax.c_ptr)


# sampler.rs:33-36 defaults: no_repeat_ngram_size 35, ngram_window 128
# (single image; 1024 multi-image), EOS id 1.
DEFAULT_NO_REPEAT_NGRAM_SIZE = 35
NGRAM_WINDOW_SINGLE = 128
NGRAM_WINDOW_MULTI = 1024
DEFAULT_EOS_TOKEN_ID = 1


def _sampler_args(history, history_len, ngram_size, window, whitelist, temperature, eos, append):
    cap = history.shape[1] if history is not None else 0
    nw = whitelist.shape[0] if whitelist is not None else 0
    return [_p(history), cap, _p(history_len), int(ngram_size), int(window), _p(whitelist), nw, float(temperature),
            int(eos), 1 if append else 0]


def lm_head_sample_i8(w: QInt8, x: DeviceArray, tokens: DeviceArray, history: DeviceArray | None = None,
                      history_len: DeviceArray | None = None, ngram_size: int = DEFAULT_NO_REPEAT_NGRAM_SIZE,
                      window: int = NGRAM_WINDOW_SINGLE, whitelist: DeviceArray | None = None,
                      temperature: float = 0.0, eos: int = DEFAULT_EOS_TOKEN_ID, append: bool = False,
                      logits: DeviceArray | None = None, is_eos: DeviceArray | None = None,
                      check: bool = False) -> None:
    """Greedy decode step with the no-repeat-ngram ban in the LM-head epilogue
    (decoder.rs:2319-2400, sampler.rs:191-235, :426-460) for m streams:
    history [m, cap] u32 and history_len [m] u32 live on the device."""
    m = x.shape[0]
    _abi.call("focr_hip_lm_head_sample_i8", w.ctx.handle, w.handle, x.c_ptr, m,
              *_sampler_args(history, history_len, ngram_size, window, whitelist, temperature, eos, append),
              _p(logits), tokens.c_ptr, _p(is_eos), 1 if check else 0)


def sample_rows(logits: DeviceArray, tokens: DeviceArray, history: DeviceArray | None = None,
                history_len: DeviceArray | None = None, ngram_size: int = DEFAULT_NO_REPEAT_NGRAM_SIZE,
                window: int = NGRAM_WINDOW_SINGLE, whitelist: DeviceArray | None = None, temperature: float = 0.0,
                eos: int = DEFAULT_EOS_TOKEN_ID, append: bool = False, is_eos: DeviceArray | None = None,
                check: bool = False) -> None:
    """sampler.rs:491-545 batched_sample / batched_decode_step over device logits [m, n]."""
    m, n = logits.shape
    _abi.call("focr_hip_sample_rows", logits.ctx.handle, logits.c_ptr, m, n,
              *_sampler_args(history, history_len, ngram_size, window, whitelist, temperature, eos, append),
              tokens.c_ptr, _p(is_eos), 1 if check else 0)


class MoeLayer:
    """A MoE layer's router (f32) and int8 experts, uploaded once.

    Host arrays: router [E, hidden] f32; wg/wu [E, inter, hidden] i8 with
    sg/su [E, inter]; wd [E, hidden, inter] i8 with sd [E, hidden]. Passing
    DeviceArrays borrows them instead of copying.
    """

    def __init__(self, hidden: int, inter: int, n_experts: int, top_k: int, router, wg, sg, wu, su, wd, sd,
                 ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hidden, self.inter, self.n_experts, self.top_k = int(hidden), int(inter), int(n_experts), int(top_k)
        self._h = C.c_void_p()
        arrs = [router, wg, sg, wu, su, wd, sd]
        from_dev = isinstance(router, DeviceArray)
        if from_dev:
            self._keep = arrs
            ptrs = [a.c_ptr for a in arrs]
        else:
            dts = [np.float32, np.int8, np.float32, np.int8, np.float32, np.int8, np.float32]
            host = [np.ascontiguousarray(a, dtype=dt) for a, dt in zip(arrs, dts)]
            self._host = host
            ptrs = [_p(a) for a in host]
        _abi.call("focr_hip_moe_layer_create", self.ctx.handle, self.hidden, self.inter, self.n_experts, self.top_k,
                  *ptrs, 1 if from_dev else 0, C.byref(self._h))
        if not from_dev:
            del self._host

    @classmethod
    def adopt(cls, ctx: Context, handle: C.c_void_p, hidden: int, inter: int, n_experts: int,
              top_k: int) -> "MoeLayer":
        """Wrap a layer handle created by the library (e.g. from a .focrq)."""
        m = cls.__new__(cls)
        m.ctx, m._h = ctx, handle
        m.hidden, m.inter, m.n_experts, m.top_k = int(hidden), int(inter), int(n_experts), int(top_k)
        return m

    def set_shared(self, shared_inter: int, wg, sg, wu, su, wd, sd) -> None:
        arrs = [wg, sg, wu, su, wd, sd]
        from_dev = isinstance(wg, DeviceArray)
        if from_dev:
            self._keep_shared = arrs
            ptrs = [a.c_ptr for a in arrs]
        else:
            dts = [np.int8, np.float32, np.int8, np.float32, np.int8, np.float32]
            host = [np.ascontiguousarray(a, dtype=dt) for a, dt in zip(arrs, dts)]
            ptrs = [_p(a) for a in host]
        _abi.call("focr_hip_moe_layer_set_shared", self._h, int(shared_inter), *ptrs, 1 if from_dev else 0)

    def route(self, hidden: DeviceArray, idx: DeviceArray, gates: DeviceArray, probs: DeviceArray | None = None,
              norm_topk: bool = False, routed_scale: float = 1.0) -> None:
        t = hidden.shape[0]
        _abi.call("focr_hip_moe_route", self.ctx.handle, self._h, hidden.c_ptr, t, 1 if norm_topk else 0,
                  float(routed_scale), idx.c_ptr, gates.c_ptr, _p(probs))

    def decode(self, hidden: DeviceArray, out: DeviceArray, idx: DeviceArray | None = None,
               gates: DeviceArray | None = None, norm_topk: bool = False, routed_scale: float = 1.0,
               with_shared: bool = False, check_route: bool = True) -> None:
        t = hidden.shape[0]
        _abi.call("focr_hip_moe_decode", self.ctx.handle, self._h, hidden.c_ptr, t, 1 if norm_topk else 0,
                  float(routed_scale), 1 if with_shared else 0, out.c_ptr, _p(idx), _p(gates),
                  1 if check_route else 0)

    def decode_noalloc(self, hidden: DeviceArray, out: DeviceArray, idx: DeviceArray | None = None,
                       gates: DeviceArray | None = None, norm_topk: bool = False, routed_scale: float = 1.0,
                       with_shared: bool = False, check_route: bool = True, ctx: Context | None = None) -> None:
        """`decode` with every intermediate in the library's static per-GPU
        scratch: no device allocation (for graph capture and serving loops).
        `ctx` issues it on another context's stream of the same device (the
        library orders the calls that share the device's scratch)."""
        t = hidden.shape[0]
        _abi.call("focr_hip_moe_decode_noalloc", (ctx or self.ctx).handle, self._h, hidden.c_ptr, t,
                  1 if norm_topk else 0, float(routed_scale), 1 if with_shared else 0, out.c_ptr, _p(idx), _p(gates),
                  1 if check_route else 0)

    def prefill(self, x: DeviceArray, idx: DeviceArray, gates: DeviceArray, out: DeviceArray,
                with_shared: bool = False, check_idx: bool = True) -> None:
        """moe_block_i8 (decoder.rs:2142-2181) on the matrix cores for prefill
        rows x [t, hidden] with routing idx/gates [t, top_k]; out [t, hidden]."""
        t = idx.shape[0]
        _abi.call("focr_hip_moe_prefill_i8", self.ctx.handle, self._h, x.c_ptr, t, idx.c_ptr, gates.c_ptr,
                  1 if with_shared else 0, out.c_ptr, 1 if check_idx else 0)

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_moe_layer_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


class MoeLayerI4:
    """A MoE layer of int4 experts for chunked prefill, uploaded once.

    Host arrays (simd::int4 packed layout, low nibble = even k): wg/wu
    [E, inter, hidden/2] u8 with sg/su [E, inter, hidden/group] f32; wd
    [E, hidden, inter/2] u8 with sd [E, hidden, inter/group]. DeviceArrays are
    borrowed instead of copied.
    """

    def __init__(self, hidden: int, inter: int, n_experts: int, group: int, wg, sg, wu, su, wd, sd,
                 ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hidden, self.inter, self.n_experts, self.group = int(hidden), int(inter), int(n_experts), int(group)
        self._h = C.c_void_p()
        arrs = [wg, sg, wu, su, wd, sd]
        from_dev = isinstance(wg, DeviceArray)
        if from_dev:
            self._keep = arrs
            ptrs = [a.c_ptr for a in arrs]
        else:
            dts = [np.uint8, np.float32, np.uint8, np.float32, np.uint8, np.float32]
            host = [np.ascontiguousarray(a, dtype=dt) for a, dt in zip(arrs, dts)]
            ptrs = [_p(a) for a in host]
        _abi.call("focr_hip_moe_layer_i4_create", self.ctx.handle, self.hidden, self.inter, self.n_experts,
                  self.group, *ptrs, 1 if from_dev else 0, C.byref(self._h))

    @classmethod
    def adopt(cls, ctx: Context, handle: C.c_void_p, hidden: int, inter: int, n_experts: int,
              group: int) -> "MoeLayerI4":
        """Wrap a layer handle created by the library (e.g. from a .focrq)."""
        m = cls.__new__(cls)
        m.ctx, m._h = ctx, handle
        m.hidden, m.inter, m.n_experts, m.group = int(hidden), int(inter), int(n_experts), int(group)
        return m

    def prefill(self, x: DeviceArray, idx: DeviceArray, gates: DeviceArray, out: DeviceArray,
                check_idx: bool = True) -> None:
        """decoder.rs:2142-2181 grouped MoE over int4 experts for x [t, hidden]
        with routing idx/gates [t, top_k]; out [t, hidden]."""
        t, top_k = idx.shape
        _abi.call("focr_hip_moe_prefill_i4", self.ctx.handle, self._h, x.c_ptr, t, top_k, idx.c_ptr, gates.c_ptr,
                  out.c_ptr, 1 if check_idx else 0)

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_moe_layer_i4_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


class RingCache:
    """``n_streams`` R-SWA ring caches of one layer on the device."""

    def __init__(self, n_streams: int, ref_capacity: int, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.n_streams, self.ref_capacity = int(n_streams), int(ref_capacity)
        self._h = C.c_void_p()
        _abi.call("focr_hip_rswa_create", self.ctx.handle, self.n_streams, self.ref_capacity, C.byref(self._h))

    def record_prefill(self, stream: int, k: DeviceArray, v: DeviceArray, seq: int) -> None:
        _abi.call("focr_hip_rswa_record_prefill", self.ctx.handle, self._h, stream, _p(k), _p(v), seq)

    def write_decode_step(self, k_steps: DeviceArray, v_steps: DeviceArray) -> list:
        slots = np.zeros(self.n_streams, dtype=np.uint32)
        _abi.call("focr_hip_rswa_write_decode_step", self.ctx.handle, self._h, k_steps.c_ptr, v_steps.c_ptr, _p(slots))
        return [int(s) for s in slots]

    def decode_attention(self, q: DeviceArray, out: DeviceArray) -> None:
        _abi.call("focr_hip_rswa_decode_attention", self.ctx.handle, self._h, q.c_ptr, out.c_ptr)

    def step(self, q: DeviceArray, k_steps: DeviceArray, v_steps: DeviceArray, out: DeviceArray) -> None:
        _abi.call("focr_hip_rswa_step", self.ctx.handle, self._h, q.c_ptr, k_steps.c_ptr, v_steps.c_ptr, out.c_ptr)

    def prefill_chunk(self, stream: int, q_chunk: DeviceArray, k_chunk: DeviceArray, v_chunk: DeviceArray,
                      c0: int, out: DeviceArray) -> None:
        """One chunk of prefill_with_cache_chunked (decoder.rs:1400-1447) for one
        layer: the chunk's K/V [cs, 1280] go to the stream's reference block at
        [c0, c0 + cs) and its queries attend causally over ref[0 .. c0 + cs)."""
        cs = q_chunk.shape[0]
        _abi.call("focr_hip_rswa_prefill_chunk", self.ctx.handle, self._h, stream, q_chunk.c_ptr, k_chunk.c_ptr,
                  v_chunk.c_ptr, cs, c0, out.c_ptr)

    def state(self, stream: int) -> tuple:
        p, rl, rp = C.c_uint32(), C.c_uint32(), C.c_uint32()
        _abi.call("focr_hip_rswa_get_state", self._h, stream, C.byref(p), C.byref(rl), C.byref(rp))
        return int(p.value), int(rl.value), int(rp.value)

    def set_state(self, stream: int, ring_len: int, ring_pos: int) -> None:
        _abi.call("focr_hip_rswa_set_state", self._h, stream, int(ring_len), int(ring_pos))

    def regions(self, stream: int) -> dict:
        ptrs = [C.c_void_p() for _ in range(4)]
        _abi.call("focr_hip_rswa_regions", self._h, stream, *[C.byref(p) for p in ptrs])
        return dict(zip(("ref_k", "ref_v", "ring_k", "ring_v"), (int(p.value) for p in ptrs)))

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_rswa_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


def prefill_chunk_bounds(seq: int, chunk: int) -> list:
    """decoder.rs:1246-1256: contiguous ascending [c0, c1) tiles of at most
    `chunk` tokens covering [0, seq) (chunk clamped to >= 1)."""
    chunk = max(int(chunk), 1)
    return [(c0, min(c0 + chunk, seq)) for c0 in range(0, seq, chunk)]


def chunk_prefill_attention(q_chunk: DeviceArray, k_prefix: DeviceArray, v_prefix: DeviceArray, num_heads: int,
                            head_dim: int, c0: int, out: DeviceArray) -> None:
    """decoder.rs:1282-1340: the chunk's queries (positions [c0, c0 + cs)) attend
    causally over the prefix [c1 = c0 + cs, num_heads*head_dim]; out [cs, dim]."""
    _abi.call("focr_hip_chunk_prefill_attention", q_chunk.ctx.handle, q_chunk.c_ptr, q_chunk.shape[0],
              k_prefix.c_ptr, v_prefix.c_ptr, k_prefix.shape[0], num_heads, head_dim, c0, out.c_ptr)


def prefill_attention(q: DeviceArray, k: DeviceArray, v: DeviceArray, num_heads: int, head_dim: int,
                      out: DeviceArray) -> None:
    """decoder.rs:568-640: full causal multi-head attention over the sequence."""
    _abi.call("focr_hip_prefill_attention", q.ctx.handle, q.c_ptr, k.c_ptr, v.c_ptr, q.shape[0], num_heads, head_dim,
              out.c_ptr)


def rms_norm(x: DeviceArray, y: DeviceArray, w: DeviceArray | None = None, eps: float = 1e-6) -> None:
    """nn::rms_norm (nn.rs:240-253) of the rows of x [rows, n] into y."""
    rows, n = x.shape
    _abi.call("focr_hip_rms_norm", x.ctx.handle, x.c_ptr, rows, n, _p(w), float(eps), y.c_ptr)


class DecoderLayer:
    """One decoder layer for decode steps (decoder.rs:2542-2627 per stream,
    :2812-2933 batched): input RMSNorm, fused qkv GEMV, RoPE, ring write +
    R-SWA attention, o_proj, residual, post-attention RMSNorm, the MoE layer
    (route_default + its shared expert) or the dense SwiGLU MLP, residual.

    Borrows the weight handles (kept alive by this object); input_ln and
    post_ln are host f32 [hidden]."""

    def __init__(self, hidden: int, input_ln, post_ln, qkv: QInt8, o_proj: QInt8, moe: MoeLayer | None = None,
                 dense: tuple[QInt8, QInt8, QInt8] | None = None, n_heads: int = 10, head_dim: int = 128,
                 eps: float = 1e-6, rope_theta: float = 10000.0, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hidden = int(hidden)
        self._keep = (qkv, o_proj, moe, dense)
        self._h = C.c_void_p()
        ln1 = np.ascontiguousarray(input_ln, dtype=np.float32)
        ln2 = np.ascontiguousarray(post_ln, dtype=np.float32)
        g, u, d = dense if dense is not None else (None, None, None)
        _abi.call("focr_hip_decoder_layer_create", self.ctx.handle, self.hidden, int(n_heads), int(head_dim),
                  ln1.ctypes.data_as(C.c_void_p), ln2.ctypes.data_as(C.c_void_p), qkv.handle, o_proj.handle,
                  moe._h if moe is not None else None, g.handle if g else None, u.handle if u else None,
                  d.handle if d else None, float(eps), float(rope_theta), C.byref(self._h))

    def step(self, cache: "RingCache", positions, x: DeviceArray, route_idx: DeviceArray | None = None,
             check_route: bool = True) -> None:
        """x [n_streams, hidden] (device) updated in place; positions: each
        stream's absolute position; route_idx [n_streams, top_k] (optional)
        receives a MoE layer's expert ids."""
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        _abi.call("focr_hip_decoder_layer_step", self.ctx.handle, self._h, cache._h, pos.ctypes.data_as(C.c_void_p),
                  x.c_ptr, _p(route_idx), 1 if check_route else 0)

    def prefill(self, cache: "RingCache", stream: int, x: DeviceArray, c0: int, route_idx: DeviceArray | None = None,
                check_route: bool = True) -> None:
        """One chunk of prefill_with_cache_i8_chunked (decoder.rs:2461-2486) for
        this layer: x [cs, hidden] (device; the rows of positions c0 .. c0 + cs
        - 1 of stream `stream`) updated in place; the chunk's K / V land in the
        stream's reference block. route_idx [cs, top_k] (optional) receives a
        MoE layer's expert ids."""
        cs = x.shape[0]
        _abi.call("focr_hip_decoder_layer_prefill", self.ctx.handle, self._h, cache._h, int(stream), x.c_ptr, cs,
                  int(c0), _p(route_idx), 1 if check_route else 0)

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_decoder_layer_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


class Decoder:
    """The decode spine of DecoderWeightCacheI8 as one device call per token:
    the layers in order (borrowed and kept alive here), the final RMSNorm
    weight (host f32 [hidden]) and the int8 LM head."""

    def __init__(self, layers: list[DecoderLayer], final_norm, lm_head: QInt8, eps: float = 1e-6,
                 ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self._keep = (list(layers), lm_head)
        self.n_layers = len(layers)
        self._h = C.c_void_p()
        handles = (C.c_void_p * len(layers))(*[layer._h.value for layer in layers])
        fn = np.ascontiguousarray(final_norm, dtype=np.float32)
        _abi.call("focr_hip_decoder_create", self.ctx.handle, len(layers), C.cast(handles, C.c_void_p),
                  fn.ctypes.data_as(C.c_void_p), float(eps), lm_head.handle, C.byref(self._h))

    def _caches(self, caches):
        if len(caches) != self.n_layers:
            raise ValueError(f"{len(caches)} caches for {self.n_layers} layers")
        return (C.c_void_p * len(caches))(*[c._h.value for c in caches])

    def step(self, caches: list["RingCache"], positions, x: DeviceArray, tokens: DeviceArray,
             logits: DeviceArray | None = None, route_idx: DeviceArray | None = None,
             check_route: bool = False) -> None:
        """batched_decode_step_i8 + batched_lm_head_i8 + argmax_row for every
        stream (decoder.rs:2812-2965, sampler.rs:168-186): x [n_streams, hidden]
        (device) holds the token embeddings and receives the last layer's
        hidden rows; tokens [n_streams] the argmax ids; logits (optional)
        [n_streams, vocab]; route_idx (optional) [n_layers, n_streams, top_k]."""
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        cs = self._caches(caches)
        _abi.call("focr_hip_decoder_step", self.ctx.handle, self._h, C.cast(cs, C.c_void_p),
                  pos.ctypes.data_as(C.c_void_p), x.c_ptr, _p(logits), tokens.c_ptr, _p(route_idx),
                  1 if check_route else 0)

    def step_sample(self, caches: list["RingCache"], positions, x: DeviceArray, tokens: DeviceArray,
                    history: DeviceArray | None = None, history_len: DeviceArray | None = None,
                    ngram_size: int = DEFAULT_NO_REPEAT_NGRAM_SIZE, window: int = NGRAM_WINDOW_SINGLE,
                    whitelist: DeviceArray | None = None, temperature: float = 0.0, eos: int = DEFAULT_EOS_TOKEN_ID,
                    append: bool = False, logits: DeviceArray | None = None, is_eos: DeviceArray | None = None,
                    route_idx: DeviceArray | None = None, check_route: bool = False) -> None:
        """The same step with the no-repeat-ngram greedy sampler in the
        LM-head epilogue (sampler.rs:426-460, :491-545) instead of the argmax."""
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        cs = self._caches(caches)
        _abi.call("focr_hip_decoder_step_sample", self.ctx.handle, self._h, C.cast(cs, C.c_void_p),
                  pos.ctypes.data_as(C.c_void_p), x.c_ptr,
                  *_sampler_args(history, history_len, ngram_size, window, whitelist, temperature, eos, append),
                  _p(logits), tokens.c_ptr, _p(is_eos), _p(route_idx), 1 if check_route else 0)

    def prefill(self, caches: list["RingCache"], stream: int, x: DeviceArray, seq: int, chunk: int | None = None,
                token: DeviceArray | None = None, logits: DeviceArray | None = None,
                route_idx: DeviceArray | None = None, check_route: bool = False) -> None:
        """prefill_with_cache_i8_chunked (decoder.rs:2428-2520) of one stream:
        x [seq, hidden] (device) holds the input embeddings and receives the
        last layer's hidden rows; every layer's chunk K / V go to caches[l]'s
        stream; chunk None is the monolithic schedule. token / logits
        (optional): the first generated token from the last position (final
        norm, LM head, argmax); route_idx (optional) [n_layers, seq, top_k]."""
        cs = self._caches(caches)
        _abi.call("focr_hip_decoder_prefill", self.ctx.handle, self._h, C.cast(cs, C.c_void_p), int(stream), x.c_ptr,
                  int(seq), int(chunk or 0), _p(logits), _p(token), _p(route_idx), 1 if check_route else 0)

    def free(self) -> None:
        if self._h:
            _abi.lib().focr_hip_decoder_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass
