"""Writes the golden fixtures of this directory: small seeded inputs and the
outputs of the C oracle (oracle/oracle.c, the restatement of weightstream-ref
quant.rs / actquant.rs / moe.rs / num.rs and of moe_dispatch_kernel's
contract) for them. Test infrastructure: the fixtures are data (inputs and
expected outputs); tests/test_golden.py checks that the oracle still
reproduces them bit for bit, tests/test_gpu_golden.py runs the GPU path on
the same inputs.

Before writing, the oracle is checked against a few of the reference's
known-answer values (the full set is tests/test_oracle_quant.py).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

SEED = 20261202


def check_kats():
    # quant.rs:233-240, :259-269; actquant.rs:181-193
    assert O.f32_to_e4m3(1.0) == 0x38 and O.f32_to_e4m3(-1.0) == 0xB8
    assert O.f32_to_e4m3(448.0) == 0x7E and O.f32_to_e4m3(1000.0) == 0x7E
    assert O.e4m3_to_f32(0x01) == 2.0 ** -9
    assert O.log2_ceil(1.0 / 448.0) == -8 and O.log2_ceil(448.0) == 9
    assert O.ue8m0_round_scale(100.0, 448.0) == 0.25
    x = np.zeros(32, np.float32)
    x[:4] = [100.0, -100.0, 3.0, 0.001]
    assert list(O.fp8_snap(x)[:4]) == [96.0, -96.0, 3.0, 0.0009765625]


def quant_cases(rng):
    x = rng.standard_normal((4, 256)).astype(np.float32)
    x[0, :32] = np.linspace(-500.0, 500.0, 32, dtype=np.float32)       # saturation
    x[1, :32] = np.linspace(0.0140, 0.0160, 32, dtype=np.float32)      # the 2^-6 carry quirk
    x[2, ::7] *= 20.0                                                  # outliers
    x[3, 32:64] = 0.0                                                  # a zero block
    aq, as_ = O.fp8_act_emit(x)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[3, 5] = 7.0
    w[40:64, 64:96] = 0.0
    w8, s8 = O.weight_quant_fp8(w)
    w4, s4 = O.weight_quant_fp4(w)
    return dict(x=x, aq=aq, as_=as_, w=w, w8=w8, s8=s8, w4=w4, s4=s4)


def gemm_cases(rng):
    m, n, k = 5, 64, 512
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random((m, k)) < 0.01] *= 20.0
    aq, as_ = O.fp8_act_emit(x)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w8, s8 = O.weight_quant_fp8(w)
    w4, s4 = O.weight_quant_fp4(w)
    y8 = O.gemm_q(aq, as_, m, w8, s8, n, k, False)
    y4 = O.gemm_q(aq, as_, m, w4, s4, n, k, True)
    return dict(aq=aq, as_=as_, w8=w8, s8=s8, w4=w4, s4=s4, y8=y8, y4=y4,
                shape=np.array([m, n, k], np.int32))


def route_cases(rng):
    rows, e, k = 3, 384, 8
    logits = rng.standard_normal((rows, e)).astype(np.float32)
    bias = (rng.standard_normal(e) * 0.1).astype(np.float32)
    logits[2, 10] = logits[2, 11]            # an exact tie
    out = dict(logits=logits, bias=bias)
    for sf in (O.SCORE_SOFTMAX, O.SCORE_SIGMOID, O.SCORE_SQRTSOFTPLUS):
        idx = np.empty((rows, k), np.int32)
        wts = np.empty((rows, k), np.float32)
        for r in range(rows):
            idx[r], wts[r] = O.route(O.score(logits[r], sf, 1.0), bias, k, True, 2.5)
        out["idx_%d" % sf], out["w_%d" % sf] = idx, wts
    return out


def dispatch_cases(rng):
    m, k, e = 20, 8, 64
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(m)]).astype(np.int32)
    idx[3, 2] = -1                           # a pick another rank owns
    w = rng.random((m, k)).astype(np.float32)
    tiles = (m * k + 31) // 32 + min(m * k, e)
    d = O.dispatch(idx, w, e, tiles)
    return dict(idx=idx, w=w, tiles=np.array([tiles], np.int32), experts=np.array([e], np.int32),
                **{"out_" + key: np.asarray(v) for key, v in d.items()})


def moe_cases(rng):
    e, dim, inter, k = 4, 128, 128, 3
    def enc4(rows, cols):
        return O.weight_quant_fp4((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    w1, s1 = enc4(e * inter, dim)
    w3, s3 = enc4(e * inter, dim)
    w2, s2 = enc4(e * dim, inter)
    x = rng.standard_normal(dim).astype(np.float32)
    idx = np.array([2, 0, 3], np.int32)
    w = np.array([0.5, 0.3, 0.2], np.float32)
    y = O.moe_routed(w1, s1, w3, s3, w2, s2, dim, inter, x, idx, w)
    def enc8(rows, cols):
        return O.weight_quant_fp8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    f1, g1 = enc8(inter, dim)
    f3, g3 = enc8(inter, dim)
    f2, g2 = enc8(dim, inter)
    ys = O.shared_fp8(f1, g1, f3, g3, f2, g2, dim, inter, x)
    return dict(w1=w1, s1=s1, w3=w3, s3=s3, w2=w2, s2=s2, x=x, idx=idx, w=w, y=y,
                f1=f1, g1=g1, f3=f3, g3=g3, f2=f2, g2=g2, ys=ys,
                shape=np.array([e, dim, inter, k], np.int32))


CASES = {"quant": quant_cases, "gemm": gemm_cases, "route": route_cases,
         "dispatch": dispatch_cases, "moe": moe_cases}


def make(name):
    """The fixture `name` as the oracle computes it now (same seed)."""
    rng = np.random.default_rng(SEED + sorted(CASES).index(name))
    return CASES[name](rng)


def main():
    O.set_threads(1)
    check_kats()
    for name in CASES:
        np.savez(os.path.join(HERE, name + ".npz"), **make(name))
        print("wrote", name + ".npz")


if __name__ == "__main__":
    main()
