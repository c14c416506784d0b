"""Seeded synthetic inputs for the benchmark configs (numpy, vectorised).

A counter-based generator: value ``i`` of the stream for tensor seed ``s``
is splitmix64's i-th output, ``mix(s + (i + 1) * 0x9E3779B97F4A7C15)``, so a
tensor of any size is generated in one vectorised pass and any slice can be
regenerated independently. Derived draws:

* int8 uniform in [-127, 127]: ``(u % 255) - 127``
* byte uniform in [0, 255]: ``u & 0xFF`` (int4-packed weights)
* f32 uniform U(a, b): ``a + (b - a) * (u >> 40) * 2**-24`` (f32 arithmetic)
* f32 normal N(mu, sigma): Box-Muller in float64 on two 53-bit uniforms,
  rounded to f32.

Tests feed the very same arrays to the GPU and to the oracle, so no
cross-machine bit reproducibility of the float transcendental draws is
assumed.
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SEED_BASE = 0xF0C00000


def seed_of(tensor_id: int) -> int:
    return SEED_BASE + int(tensor_id)


def u64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def int8_uniform(seed: int, n: int) -> np.ndarray:
    return ((u64(seed, n) % np.uint64(255)).astype(np.int16) - 127).astype(np.int8)


def bytes_uniform(seed: int, n: int) -> np.ndarray:
    return (u64(seed, n) & np.uint64(0xFF)).astype(np.uint8)


def f32_uniform(seed: int, n: int, a: float, b: float) -> np.ndarray:
    u = (u64(seed, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    a32, b32 = np.float32(a), np.float32(b)
    return a32 + (b32 - a32) * u


def f32_normal(seed: int, n: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    z = u64(seed, 2 * n)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mu + sigma * g).astype(np.float32)


def int_uniform(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive)."""
    span = np.uint64(hi - lo + 1)
    return (u64(seed, n) % span).astype(np.int64) + lo


def zipf_routing(seed: int, t: int, n_experts: int = 64, top_k: int = 6, s: float = 1.1):
    """Synthetic prefill routing: per token, top_k distinct experts drawn
    without replacement from Zipf(s) over ranks 1..n_experts (p_r ∝ r^-s),
    through a seeded rank -> expert-id permutation; gates U(0.1, 1)
    renormalised to sum 1 in f32. Returns idx [t, top_k] u32, gates
    [t, top_k] f32. Deterministic in (seed, t, n_experts, top_k, s)."""
    perm = np.argsort(u64(seed, n_experts), kind="stable")  # rank -> expert id
    w = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    draws = (u64(seed + 1, t * top_k) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    idx = np.zeros((t, top_k), np.uint32)
    for tok in range(t):
        avail = np.ones(n_experts, bool)
        for j in range(top_k):
            p = np.where(avail, w, 0.0)
            c = np.cumsum(p)
            r = int(np.searchsorted(c, draws[tok * top_k + j] * c[-1], side="right"))
            r = min(r, n_experts - 1)
            while not avail[r]:  # guards the c[-1] edge only
                r -= 1
            avail[r] = False
            idx[tok, j] = perm[r]
    g = f32_uniform(seed + 2, t * top_k, 0.1, 1.0).reshape(t, top_k)
    gates = (g / g.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return idx, gates
