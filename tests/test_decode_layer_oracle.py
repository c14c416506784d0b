"""The oracle's decode-step decoder layer (pyoracle.decoder_layer_step,
decoder.rs:2812-2933 batched, :2542-2627 per stream) against an independent
float64 numpy restatement of the same wiring: RMSNorm with the input /
post-attention weights, quantize_row_i8 (decoder.rs:1647-1656: scale
amax / 127, round half away from zero) ahead of every int8 GEMV, RoPE at
each stream's own position, the new K / V appended to the stream's ring and
softmax attention over the reference block and the ring, the residuals,
route_default (softmax over the experts, top-k by probability, weights the
probabilities) with the shared expert at weight 1, and the dense SwiGLU
expert for layer 0.

Only the int8 rule is kept exact in the restatement. The f32 path and the
f64 one round an activation differently by an ulp now and then; where that
value sits on an int8 rounding boundary one code flips and that row moves
(by ~1e-3 of its row max, spread further by the quantizations after it). So
the criterion is on the rows: the median row within 1e-5 of its row max and
most rows within 1e-4. A wiring mistake moves every row by far more; the
last test checks that swapping the two norm weights, shifting the position
by one or dropping the ring's new token is rejected by the same criterion.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pyoracle as O

H, NH, HD = 1280, 10, 128
D = NH * HD
G = 24  # reference-block tokens per stream


def _weights(rng, moe: bool, E=8, K=3, inter=128, si=256, dense_inter=256):
    i8 = lambda n: rng.integers(-127, 128, n).astype(np.int8)  # noqa: E731
    # per-row scales that keep the layer's gain near 1 (a 1280-wide int8 dot
    # of unit rows has std ~ 73 sqrt(1280) scale)
    sc = lambda n: rng.uniform(2e-4, 6e-4, n).astype(np.float32)  # noqa: E731
    lw = {"input_ln": rng.uniform(0.5, 1.5, H).astype(np.float32), "post_ln": rng.uniform(0.5, 1.5, H).astype(np.float32),
          "qkv": (i8(3 * D * H), sc(3 * D)), "o": (i8(H * D), sc(H))}
    if moe:
        lw["moe"] = {"router": (rng.standard_normal((E, H)) * 0.02).astype(np.float32), "wg": i8(E * inter * H),
                     "sg": sc(E * inter), "wu": i8(E * inter * H), "su": sc(E * inter), "wd": i8(E * H * inter),
                     "sd": sc(E * H), "n_experts": E, "top_k": K, "inter": inter,
                     "shared": (si, i8(si * H), sc(si), i8(si * H), sc(si), i8(H * si), sc(H))}
    else:
        lw["dense"] = {"wg": i8(dense_inter * H), "sg": sc(dense_inter), "wu": i8(dense_inter * H),
                       "su": sc(dense_inter), "wd": i8(H * dense_inter), "sd": sc(H), "inter": dense_inter}
    return lw


def _refs(rng, B):
    """Each stream's reference block, head-major [NH, G, HD] (K already RoPE'd)."""
    return [(rng.standard_normal((NH, G, HD)).astype(np.float32), rng.standard_normal((NH, G, HD)).astype(np.float32))
            for _ in range(B)]


def _oracle_steps(x0, pos0, refs, lw, steps):
    rings = [O.Ring(G) for _ in refs]
    for r, (k, v) in zip(rings, refs):
        r.record_prefill(k, v, G)
    x, outs = x0, []
    for t in range(steps):
        x = O.decoder_layer_step(x, [p + t for p in pos0], rings, lw)
        outs.append(x)
    return outs


class _F64Layer:
    """The layer restated in float64 from the reference's text."""

    def __init__(self, refs, lw, eps=1e-6, theta=10000.0, pos_shift=0, keep_new_token=True):
        self.lw, self.eps, self.theta = lw, eps, theta
        self.pos_shift, self.keep_new = pos_shift, keep_new_token
        # token-major keys / values per stream: [G + ring, NH, HD]
        self.keys = [k.transpose(1, 0, 2).astype(np.float64) for k, _ in refs]
        self.vals = [v.transpose(1, 0, 2).astype(np.float64) for _, v in refs]

    def norm(self, a, w):
        return a / np.sqrt((a * a).mean(axis=-1, keepdims=True) + self.eps) * w.astype(np.float64)

    @staticmethod
    def lin(a, w, s, n):
        """quantize_row_i8 of each row, the i32 product, ((acc * a_s) * w_s)."""
        a = np.atleast_2d(a)
        a32 = a.astype(np.float32)
        amax = np.abs(a32).max(axis=1, keepdims=True)
        sa = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
        v = a32 * (np.float32(1.0) / sa)
        q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -127, 127).astype(np.int64)
        return (q @ w.reshape(n, -1).astype(np.int64).T) * sa.astype(np.float64) * s.astype(np.float64)

    def rope(self, a, pos):
        half = HD // 2
        inv = 1.0 / self.theta ** (np.arange(half) * 2.0 / HD)
        ang = pos * inv
        a = a.reshape(NH, HD)
        lo, hi = a[:, :half], a[:, half:]
        c, s = np.cos(ang), np.sin(ang)
        return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1)

    def mlp(self, a, wg, sg, wu, su, wd, sd, inter):
        g = self.lin(a, wg, sg, inter)
        return self.lin(g / (1.0 + np.exp(-g)) * self.lin(a, wu, su, inter), wd, sd, H)

    def step(self, x, positions):
        lw = self.lw
        x = x.astype(np.float64)
        B = x.shape[0]
        qkv = self.lin(self.norm(x, lw["input_ln"]), *lw["qkv"], 3 * D)
        ctx = np.zeros((B, D))
        for s in range(B):
            p = positions[s] + self.pos_shift
            q, k = self.rope(qkv[s, :D], p), self.rope(qkv[s, D:2 * D], p)
            v = qkv[s, 2 * D:].reshape(NH, HD)
            if self.keep_new:
                self.keys[s] = np.concatenate([self.keys[s], k[None]])
                self.vals[s] = np.concatenate([self.vals[s], v[None]])
            for h in range(NH):
                sc = self.keys[s][:, h] @ q[h] / np.sqrt(HD)
                w = np.exp(sc - sc.max())
                ctx[s, h * HD:(h + 1) * HD] = (w / w.sum()) @ self.vals[s][:, h]
        h1 = x + self.lin(ctx, *lw["o"], H)
        n2 = self.norm(h1, lw["post_ln"])
        if "moe" in lw:
            m = lw["moe"]
            E, K, I = m["n_experts"], m["top_k"], m["inter"]
            lg = n2 @ m["router"].astype(np.float64).T
            pr = np.exp(lg - lg.max(axis=1, keepdims=True))
            pr /= pr.sum(axis=1, keepdims=True)
            out = np.zeros_like(x)
            for t in range(B):
                for e in np.argsort(-pr[t], kind="stable")[:K]:
                    r = lambda a: a.reshape(E, -1)[e]  # noqa: E731
                    out[t] += pr[t, e] * self.mlp(n2[t], r(m["wg"]), r(m["sg"]), r(m["wu"]), r(m["su"]),
                                                  r(m["wd"]), r(m["sd"]), I)[0]
            si, *sw = m["shared"]
            out += self.mlp(n2, *sw, si)
        else:
            d = lw["dense"]
            out = self.mlp(n2, d["wg"], d["sg"], d["wu"], d["su"], d["wd"], d["sd"], d["inter"])
        return h1 + out


def _f64_steps(x0, pos0, refs, lw, steps, **kw):
    f = _F64Layer(refs, lw, **kw)
    x, outs = x0.astype(np.float64), []
    for t in range(steps):
        x = f.step(x, [p + t for p in pos0])
        outs.append(x)
    return outs


def _row_rel(got, want):
    return (np.abs(got - want) / np.maximum(np.abs(want), np.abs(want).max(axis=1, keepdims=True) * 1e-2)).max(axis=1)


def _close(got_steps, want_steps):
    rel = np.concatenate([_row_rel(g, w) for g, w in zip(got_steps, want_steps)])
    return bool(np.median(rel) < 1e-5 and np.mean(rel < 1e-4) >= 0.75), rel


def _case(rng, moe):
    lw = _weights(rng, moe)
    B = 4
    refs = _refs(rng, B)
    x0 = rng.standard_normal((B, H)).astype(np.float32)
    pos0 = [G, G + 7, G + 100, G + 3]
    return lw, refs, x0, pos0


@pytest.mark.parametrize("moe", [True, False], ids=["moe", "dense"])
def test_decode_layer_matches_a_float64_restatement(moe, rng):
    lw, refs, x0, pos0 = _case(rng, moe)
    got = _oracle_steps(x0, pos0, refs, lw, 3)
    ok, rel = _close(got, _f64_steps(x0, pos0, refs, lw, 3))
    assert ok, rel


def test_the_restatement_rejects_wiring_mistakes(rng):
    lw, refs, x0, pos0 = _case(rng, True)
    got = _oracle_steps(x0, pos0, refs, lw, 3)
    swapped = dict(lw, input_ln=lw["post_ln"], post_ln=lw["input_ln"])
    for name, want in (("norm weights swapped", _f64_steps(x0, pos0, refs, swapped, 3)),
                       ("position off by one", _f64_steps(x0, pos0, refs, lw, 3, pos_shift=1)),
                       ("new token not attended", _f64_steps(x0, pos0, refs, lw, 3, keep_new_token=False))):
        ok, rel = _close(got, want)
        assert not ok, f"{name}: median {np.median(rel):.2e}"
