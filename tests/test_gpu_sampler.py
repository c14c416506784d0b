"""GPU parity for the greedy sampler (sampler.rs:168-545) and its fusion into
the LM-head epilogue (decoder.rs:2319-2400).

Tokens and EOS flags are bit-exact against oracle_sample; the masked logits
of the fused LM head are bit-exact against the oracle's LM-head logits with
the oracle's ban applied; a device-resident multi-step loop (append = 1)
reproduces a host loop over the oracle token for token.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from franken_ocr_amd import _abi, synth
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu
INF = float("inf")


def _say(msg):
    print(f"[gpu-sampler] {msg}", flush=True)


def _hist(ctx, seqs, cap):
    h = np.zeros((len(seqs), cap), np.uint32)
    ln = np.zeros(len(seqs), np.uint32)
    for i, s in enumerate(seqs):
        h[i, :len(s)] = s
        ln[i] = len(s)
    return ctx.to_device(h), ctx.to_device(ln)


def _sample_dev(ctx, rows, seqs, n, w, white=(), cap=None, eos=1):
    from franken_ocr_amd.engine import sample_rows

    rows = np.asarray(rows, np.float32)
    m = rows.shape[0]
    cap = cap or max(1, max(len(s) for s in seqs) + 1)
    dh, dl = _hist(ctx, seqs, cap)
    dw = ctx.to_device(np.asarray(white, np.uint32)) if len(white) else None
    tok, eos_f = ctx.empty((m,), np.uint32), ctx.empty((m,), np.uint8)
    sample_rows(ctx.to_device(rows), tok, dh, dl, n, w, dw, eos=eos, is_eos=eos_f, check=True)
    return tok.numpy(), eos_f.numpy()


# (row, seq, ngram, window, whitelist, expected) — sampler.rs:617-925
KNOWN = [
    ([0.1, -2.0, 3.5, 3.4, 0.0], [], 35, 128, (), 2),
    ([0.0, 5.0, 1.0, 5.0], [], 0, 0, (), 1),
    ([math.nan, -INF, 2.0, 1.0], [], 0, 0, (), 2),
    ([math.nan] * 3, [], 0, 0, (), 0),
    ([10.0, 5.0, 5.0], [0, 0], 1, 8, (), 1),
    ([0.0, 0.0, 0.0, 9.0, 1.0], [7, 3, 7], 2, 16, (), 4),
    ([9.0, 1.0, 0.0], [5, 0, 5], 2, 0, (), 1),
    ([3.0, 2.0, 1.0], [0, 1, 2], 1, 8, (), 0),
    ([0.0, 0.0, 9.0, 0.0], [1, 2, 9], 2, 16, (), 2),
    ([0.0, 0.0, 9.0, 1.0], [0, 2, 0], 2, 16, (), 3),
    ([0.0] * 5 + [9.0], [5, 0, 5], 2, 2, (), 5),
    ([9.0, 0.0, 0.0], [0, 0, 0], 35, 128, (), 0),
    ([1.0, 2.0, 3.0], [99, 99], 1, 8, (), 2),
    ([1.0, 2.0, 3.0], [2, 2], 1, 8, (2,), 2),
]


@pytest.mark.parametrize("case", range(len(KNOWN)))
def test_known_answers(ctx, case):
    row, seq, n, w, white, want = KNOWN[case]
    _say(f"known case {case}")
    tok, eos = _sample_dev(ctx, [row], [seq], n, w, white)
    assert tok[0] == want and eos[0] == (want == 1)


def test_35gram_window_boundaries(ctx):
    row = np.zeros(128, np.float32)
    row[7], row[6] = 10.0, 9.0
    for window, cases in ((128, [(127, 6), (128, 6), (129, 7)]), (1024, [(1023, 6), (1024, 6), (1025, 7)])):
        seqs = []
        for total, _ in cases:
            prefix = list(range(20, 54))
            seqs.append(prefix + [7] + [99] * (total - 69) + prefix)
        tok, _ = _sample_dev(ctx, [row] * 3, seqs, 35, window)
        assert tok.tolist() == [c[1] for c in cases]


@pytest.mark.parametrize("vocab", [7, 1000, 129280])
def test_sample_rows_random_against_oracle(ctx, vocab):
    _say(f"sample_rows vocab={vocab}")
    rng = np.random.default_rng(vocab)
    m = 16
    alpha = min(vocab, 12)  # small alphabet: frequent repeated n-grams
    seqs, rows, params = [], [], []
    for i in range(m):
        L = int(rng.integers(0, 400))
        seqs.append(rng.integers(0, alpha, L).tolist())
        r = rng.standard_normal(vocab).astype(np.float32)
        r[: alpha] += 4.0  # make the repeated ids the likely argmax so bans matter
        if i % 5 == 0:
            r[int(rng.integers(0, vocab))] = math.nan
        if i % 7 == 0:
            r[1] = r.max()  # a tie with the lowest index winning
        rows.append(r)
    for n, w, white in ((1, 8, ()), (2, 16, ()), (3, 0, (0,)), (35, 128, ()), (2, 1024, (1, 2))):
        tok, eos = _sample_dev(ctx, rows, seqs, n, w, white)
        for i in range(m):
            st, want, _ = O.sample(rows[i], np.asarray(seqs[i], np.uint32), n, w, white)
            assert st == 0 and tok[i] == want, (n, w, i)
            assert eos[i] == (want == 1)


def test_lm_head_sample_fused_matches_oracle(ctx):
    from franken_ocr_amd.engine import QInt8, lm_head_sample_i8

    n, k, m = 129280, 1280, 8
    _say(f"lm_head_sample_i8 n={n} k={k} m={m}")
    w = synth.int8_uniform(synth.seed_of(900), n * k)
    s = synth.f32_uniform(synth.seed_of(901), n, 1e-3, 2e-2)
    x = synth.f32_normal(synth.seed_of(902), m * k).reshape(m, k)
    logits, argmax = O.lm_head_i8(x, w, s, n, k)
    rng = np.random.default_rng(903)
    seqs = []
    for r in range(m):
        # stream r repeats a 35-gram whose completion is its raw argmax, so the
        # ban must move the choice (rows 0..5), or a 2-gram (6), or nothing (7)
        top = int(argmax[r])
        body = rng.integers(2, n, 60).tolist()
        if r < 6:
            pre = rng.integers(2, n, 34).tolist()
            seqs.append(body + pre + [top] + rng.integers(2, n, 20).tolist() + pre)
        elif r == 6:
            seqs.append(body + [5, top, 9, 5])
        else:
            seqs.append(body)
    ngrams = [35] * 6 + [2, 35]
    q = QInt8(w, s, n, k, ctx)
    cap = 256
    for n_gram in (35, 2):
        dh, dl = _hist(ctx, seqs, cap)
        tok, eos = ctx.empty((m,), np.uint32), ctx.empty((m,), np.uint8)
        dlog = ctx.empty((m, n), np.float32)
        lm_head_sample_i8(q, ctx.to_device(x), tok, dh, dl, n_gram, 128, logits=dlog, is_eos=eos, check=True)
        got_logits, got = dlog.numpy(), tok.numpy()
        for r in range(m):
            st, want, masked = O.sample(logits[r], np.asarray(seqs[r], np.uint32), n_gram, 128)
            assert st == 0
            assert got[r] == want, (n_gram, r)
            assert np.array_equal(got_logits[r].view(np.uint32), masked.view(np.uint32)), (n_gram, r)
            if ngrams[r] == n_gram and r < 7:
                assert want != argmax[r]  # the ban changed the pick


def test_device_decode_loop_appends_history(ctx):
    from franken_ocr_amd.engine import QInt8, lm_head_sample_i8

    n, k, m, steps, cap = 4096, 256, 4, 40, 128
    _say(f"device loop n={n} steps={steps}")
    w = synth.int8_uniform(synth.seed_of(910), n * k)
    s = synth.f32_uniform(synth.seed_of(911), n, 1e-3, 2e-2)
    x = synth.f32_normal(synth.seed_of(912), m * k).reshape(m, k)
    logits, _ = O.lm_head_i8(x, w, s, n, k)
    q = QInt8(w, s, n, k, ctx)
    seqs = [[3, 4], [], [7] * 10, [1, 2, 3]]
    dh, dl = _hist(ctx, seqs, cap)
    dx = ctx.to_device(x)
    tok = ctx.empty((m,), np.uint32)
    # fixed logits each step: the 1-gram ban over the window forces a new token
    for _ in range(steps):
        lm_head_sample_i8(q, dx, tok, dh, dl, 1, 32, append=True)
    hist, lens = dh.numpy(), dl.numpy()
    for r in range(m):
        ref = list(seqs[r])
        for _ in range(steps):
            st, t, _ = O.sample(logits[r], np.asarray(ref, np.uint32), 1, 32)
            ref.append(t)
        assert lens[r] == len(ref)
        assert hist[r, :len(ref)].tolist() == ref


def test_sampler_errors(ctx):
    from franken_ocr_amd.engine import sample_rows

    rows = ctx.to_device(np.zeros((2, 8), np.float32))
    tok = ctx.empty((2,), np.uint32)
    with pytest.raises(_abi.NotImplementedPath):
        sample_rows(rows, tok, ngram_size=0, temperature=0.7)
    dh = ctx.to_device(np.zeros((2, 4), np.uint32))
    dl = ctx.to_device(np.array([2, 9], np.uint32))  # row 1 claims 9 > cap 4
    with pytest.raises(_abi.ContractViolation) as e:
        sample_rows(rows, tok, dh, dl, 2, 16, check=True)
    assert "exceeds history_cap" in str(e.value)
    dl2 = ctx.to_device(np.array([4, 1], np.uint32))  # row 0 full
    with pytest.raises(_abi.ContractViolation) as e:
        sample_rows(rows, tok, dh, dl2, 2, 16, append=True, check=True)
    assert "full" in str(e.value)
    assert dl2.numpy().tolist() == [4, 2]
    # NaN temperature is greedy (sampler.rs:96-100)
    sample_rows(rows, tok, ngram_size=0, temperature=math.nan)
    assert tok.numpy().tolist() == [0, 0]
