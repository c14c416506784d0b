"""Regenerate the committed golden fixtures from the C oracle.

    python tests/golden/make_golden.py

Writes small seeded instances of every benchmark config (inputs + the
oracle's outputs) as compressed .npz, the 24 self-test i32 vectors of
dispatch.rs:352-429, and the reference's in-code known answers as JSON.
The reference (Rust) cannot run here; its known answers are copied as data
with their file:line, and the oracle that produced the .npz outputs is
itself pinned by tests/test_oracle.py.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from franken_ocr_amd import synth  # noqa: E402
from oracle import pyoracle as O  # noqa: E402

KNOWN_ANSWERS = {
    "igemm_s8s8": [
        {"a": [1, 2, 3, 4, 5, 6], "b": [1, 0, 1, 0, 1, 0], "m": 2, "k": 3, "n": 2, "out0": [0, 0, 0, 0],
         "want": [4, 2, 10, 5], "src": "src/simd/scalar.rs:176-183"},
        {"a": [1, 2, 3], "b": [1, 1, 1], "m": 1, "k": 3, "n": 1, "out0": [100], "want": [106],
         "src": "src/simd/scalar.rs:186-195"},
        {"a": [-2, 3], "b": [-1, -1, 4, -2], "m": 1, "k": 2, "n": 2, "out0": [0, 0], "want": [-1, -14],
         "src": "src/simd/scalar.rs:210-220"},
    ],
    "igemm_u8s8": [
        {"a": [10, 20, 30], "b": [2, -1, 1], "m": 1, "k": 3, "n": 1, "out0": [0], "want": [30],
         "src": "src/simd/scalar.rs:200-207"},
    ],
    "k6848_extremes": [
        {"a": 127, "b": 127, "unsigned": False, "want": 110451392, "src": "src/simd/scalar.rs:227-236"},
        {"a": -128, "b": -128, "unsigned": False, "want": 112197632, "src": "src/simd/scalar.rs:240-249"},
        {"a": 255, "b": 127, "unsigned": True, "want": 221772480, "src": "src/simd/scalar.rs:253-262"},
        {"a": 255, "b": -128, "unsigned": True, "want": -223518720, "src": "src/simd/dispatch.rs:604-618"},
    ],
    "int4_sign_extend": {"want": [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1],
                         "src": "src/simd/int4.rs:660-670"},
    "int4_unpack": [
        {"packed": [33], "n": 1, "k": 2, "want": [1, 2], "src": "src/simd/int4.rs:677"},
        {"packed": [135], "n": 1, "k": 2, "want": [7, -8], "src": "src/simd/int4.rs:679"},
        {"packed": [240], "n": 1, "k": 2, "want": [0, -1], "src": "src/simd/int4.rs:680"},
        {"packed": [136], "n": 1, "k": 2, "want": [-8, -8], "src": "src/simd/int4.rs:682"},
        {"packed": [33, 67, 101, 135], "n": 2, "k": 4, "want": [1, 2, 3, 4, 5, 6, 7, -8],
         "src": "src/simd/int4.rs:692-695"},
    ],
    "int4_adversarial_cell": {"weights_byte": 136, "a": -127, "m": 2, "k": 32, "n": 3, "group": 16, "want": 32512.0,
                              "src": "src/simd/int4.rs:879-891"},
    "quantize_int8_f32": [
        {"w": [127.0, -127.0, 0.0, 64.0], "n": 1, "k": 4, "q": [127, -127, 0, 64], "scales": [1.0],
         "src": "src/quant/int8.rs:300-307"},
        {"w": [254.0, -2.0, 100.0], "n": 1, "k": 3, "q": [127, -1, 50], "scales": [2.0],
         "src": "src/quant/int8.rs:310-315"},
        {"w": [127.0, 0.5, 1.5, 2.5], "n": 1, "k": 4, "q": [127, 0, 2, 2], "scales": [1.0],
         "src": "src/quant/int8.rs:337-343"},
        {"w": [-127.0, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 127.0], "n": 1, "k": 8,
         "q": [-127, -2, -2, 0, 0, 2, 2, 127], "scales": [1.0], "src": "src/quant/int8.rs:346-356"},
    ],
    "argmax_row": [
        {"logits": [0.1, -2.0, 3.5, 3.4, 0.0], "want": 2, "src": "src/native_engine/sampler.rs:618-621"},
        {"logits": [0.0, 5.0, 1.0, 5.0], "want": 1, "src": "src/native_engine/sampler.rs:624-634"},
        {"logits": ["nan", "-inf", 2.0, 1.0], "want": 2, "src": "src/native_engine/sampler.rs:637-645"},
    ],
    "route_top6": {"boost": {"10": 10.0, "11": 9.0, "12": 8.0, "13": 7.0, "14": 6.0, "15": 5.0},
                   "want": [10, 11, 12, 13, 14, 15], "src": "src/native_engine/moe.rs:777-820"},
    "rswa": [
        {"case": "single key returns V", "want": 7.0, "src": "src/native_engine/rswa.rs:1475-1488"},
        {"case": "equal scores average V rows 2 and 4", "want": 3.0, "src": "src/native_engine/rswa.rs:1493-1507"},
    ],
}


def selftest_vectors():
    out = {}
    for i in range(12):
        for unsigned in (False, True):
            label, m, k, n, seed, a, b = O.selftest_case(i, unsigned)
            f = O.igemm_u8s8 if unsigned else O.igemm_s8s8
            out[f"{'u8s8' if unsigned else 's8s8'}|{label}"] = f(a, b, m, k, n)
    return out


def cfg1(path):
    M, N, K = 16, 64, 1280
    a = synth.int8_uniform(synth.seed_of(9001), M * K)
    w = synth.int8_uniform(synth.seed_of(9002), N * K)
    ws = synth.f32_uniform(synth.seed_of(9003), N, 1e-3, 2e-2)
    as_ = synth.f32_uniform(synth.seed_of(9004), M, 1e-3, 2e-2)
    acc = O.igemm_s8s8(a, w, M, K, N)
    y = np.zeros(M * N, np.float32)
    L = O.lib()
    L.oracle_dequant_i8(O.p(acc), M, N, O.p(as_), O.p(ws), O.p(y))
    np.savez_compressed(path, a=a, w=w, ws=ws, as_=as_, acc=acc, y=y, M=M, N=N, K=K)


def cfg2(path):
    M, N, K = 8, 257, 1280
    w = synth.int8_uniform(synth.seed_of(9011), N * K)
    s = synth.f32_uniform(synth.seed_of(9012), N, 1e-3, 2e-2)
    x = synth.f32_normal(synth.seed_of(9013), M * K).reshape(M, K)
    logits, am = O.lm_head_i8(x, w, s, N, K)
    np.savez_compressed(path, w=w, s=s, x=x, logits=logits, argmax=am, M=M, N=N, K=K)


def cfg3(path):
    T, H, I, E, K = 4, 64, 32, 16, 6
    router = synth.f32_normal(synth.seed_of(9021), E * H, 0.0, 0.02).reshape(E, H)
    wg = synth.int8_uniform(synth.seed_of(9022), E * I * H)
    wu = synth.int8_uniform(synth.seed_of(9023), E * I * H)
    wd = synth.int8_uniform(synth.seed_of(9024), E * H * I)
    sg = synth.f32_uniform(synth.seed_of(9025), E * I, 1e-3, 2e-2)
    su = synth.f32_uniform(synth.seed_of(9026), E * I, 1e-3, 2e-2)
    sd = synth.f32_uniform(synth.seed_of(9027), E * H, 1e-3, 2e-2)
    x = synth.f32_normal(synth.seed_of(9028), T * H).reshape(T, H)
    st, out, idx, gates = O.moe_decode(x, router, wg, sg, wu, su, wd, sd, E, K, I, norm_topk=True)
    assert st == 0
    np.savez_compressed(path, router=router, wg=wg, wu=wu, wd=wd, sg=sg, su=su, sd=sd, x=x, out=out, idx=idx,
                        gates=gates, T=T, H=H, I=I, E=E, K=K)


def cfg4(path):
    m, k, n, g = 6, 256, 24, 32
    a = synth.int8_uniform(synth.seed_of(9031), m * k)
    b = synth.bytes_uniform(synth.seed_of(9032), n * k // 2)
    s = synth.f32_uniform(synth.seed_of(9033), n * (k // g), 1e-3, 2e-2)
    st, out = O.igemm_s4s8_packed(a, b, s, g, m, k, n)
    st2, parts = O.s4s8_group_i32(a, b, g, m, k, n)
    assert st == 0 and st2 == 0
    np.savez_compressed(path, a=a, b=b, s=s, out=out, parts=parts, m=m, k=k, n=n, group=g)


def cfg5(path):
    G = 8
    r = O.Ring(G)
    k = synth.f32_normal(synth.seed_of(9041), 10 * G * 128)
    v = synth.f32_normal(synth.seed_of(9042), 10 * G * 128)
    r.record_prefill(k, v, G)
    slots = []
    for step in range(140):  # wraps the 128-slot ring
        ks = synth.f32_normal(synth.seed_of(9100 + step), 10 * 128)
        vs = synth.f32_normal(synth.seed_of(9300 + step), 10 * 128)
        slots.append(r.write(ks, vs))
    q = synth.f32_normal(synth.seed_of(9043), 10 * 128)
    st, out = r.attend(q)
    assert st == 0
    np.savez_compressed(path, k=k, v=v, q=q, out=out, slots=np.array(slots, np.uint32), G=G, steps=140,
                        ring_len=r.ring_len.value, ring_pos=r.ring_pos.value)


def main():
    (HERE / "known_answers.json").write_text(json.dumps(KNOWN_ANSWERS, indent=1) + "\n")
    np.savez_compressed(HERE / "selftest_i32.npz", **selftest_vectors())
    cfg1(HERE / "cfg1_igemm_small.npz")
    cfg2(HERE / "cfg2_lmhead_small.npz")
    cfg3(HERE / "cfg3_moe_small.npz")
    cfg4(HERE / "cfg4_int4_small.npz")
    cfg5(HERE / "cfg5_rswa_small.npz")
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
