"""GPU parity for the decoder's RMSNorm entry point (nn.rs:240-253 rms_norm,
the final norm before the LM head, decoder.rs:2275-2296) against the oracle's
restatement: y = (x * rstd) * w with rstd = (float)(1 / sqrt(mean(x^2) + eps))
from an f64 sum of squares. The f32 operations per element are the oracle's;
the f64 sum runs in another order, which can move rstd by one f32 ulp only
when the f64 value sits on a rounding boundary, hence rel 1e-6 (one ulp of
rstd is ~6e-8 relative)."""

from __future__ import annotations

import numpy as np
import pytest

from franken_ocr_amd import synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


# rows, n, weighted: the register form (n % 4 == 0, up to 2048 and 4096
# floats per row), the staged-row form (n % 4 != 0), no weight
@pytest.mark.parametrize("rows,n,weighted", [(8, 1280, True), (3, 4096, True), (5, 1282, True), (2, 1280, False),
                                             (1, 7, True), (4, 2048, False)])
def test_rms_norm_matches_oracle(ctx, rows, n, weighted):
    from franken_ocr_amd.engine import rms_norm

    print(f"[gpu-norm] rows={rows} n={n} weighted={weighted}", flush=True)
    x = synth.f32_normal(synth.seed_of(9100 + n), rows * n).reshape(rows, n) * 3.0
    w = synth.f32_uniform(synth.seed_of(9200 + n), n, 0.5, 1.5) if weighted else None
    dy = ctx.empty((rows, n), np.float32)
    rms_norm(ctx.to_device(x), dy, ctx.to_device(w) if weighted else None, eps=1e-6)
    want = O.rms_norm(x, w, 1e-6)
    np.testing.assert_allclose(dy.numpy(), want, rtol=1e-6, atol=0)


def test_rms_norm_zero_row_and_scale(ctx):
    """A zero row gives zeros (rstd = 1/sqrt(eps), times 0); with eps = 0, a
    row scaled by 2^10 normalises to the same values (the f64 sum of squares,
    its sqrt and the reciprocal all scale exactly by powers of two)."""
    from franken_ocr_amd.engine import rms_norm

    n = 1280
    dz = ctx.empty((1, n), np.float32)
    rms_norm(ctx.to_device(np.zeros((1, n), np.float32)), dz, None, eps=1e-6)
    assert (dz.numpy() == 0).all()
    base = synth.f32_normal(synth.seed_of(9300), n)
    x = np.stack([base, base * np.float32(1024.0)])
    dy = ctx.empty((2, n), np.float32)
    rms_norm(ctx.to_device(x), dy, None, eps=0.0)
    y = dy.numpy()
    np.testing.assert_array_equal(y[0], y[1])
