"""GPU parity of the FP8 block quantisers on blocks holding infinities, NaN
and values near FLT_MAX, bit for bit against the oracle.

A block holding an infinity has amax = inf, so the reference's scale is
2^log2_ceil(inf / 448) = 2^128 = inf (scale byte 0xFF): dividing by it sends
every finite element to a signed zero and an infinity to the x86
invalid-operation NaN (sign bit set, byte 0xFF); a NaN element stays NaN
(actquant.rs:21-45 with quant.rs:103-137). The device kernels compute
x / 2^e as x * 2^-e, so these blocks are the case where that rewrite needs
its own rule. test_oracle_quant.py pins the oracle's bytes for them from the
IEEE arithmetic.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, announce, dev, host
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu

FMAX = np.finfo(np.float32).max


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def _nonfinite_acts(rng, nblk, block=32):
    x = rng.standard_normal(nblk * block).astype(np.float32)
    b = lambda i: slice(i * block, (i + 1) * block)
    x[b(0)][3] = np.inf                            # finite values -> +-0, inf -> 0xFF
    x[b(1)][0] = -np.inf
    x[b(2)][5], x[b(2)][6] = np.inf, np.nan        # NaN stays NaN
    x[b(3)][:] = FMAX * np.sign(rng.standard_normal(block)).astype(np.float32)
    x[b(4)][7] = np.float32(-FMAX)                 # largest finite scale, e = 120
    x[b(4)][8] = np.float32(2.0 ** 118)
    x[b(5)][:] = np.inf                            # all infinite
    x[b(6)][:] = np.nan                            # all NaN: amax floor
    x[b(7)][1], x[b(7)][2] = -np.inf, np.inf
    x[b(7)][3] = -0.0
    return x


def test_emit8_snap8_nonfinite_blocks():
    rng = np.random.default_rng(900)
    n = 32 * 64
    x = _nonfinite_acts(rng, n // 32)
    q_ref, s_ref = O.fp8_act_emit(x)
    assert q_ref[3] == 0xFF and s_ref[0] == 0xFF     # the rule this file states
    announce("emit8 nonfinite n=%d" % n)
    q = torch.empty(n, dtype=torch.uint8, device=DEV)
    s = torch.empty(n // 32, dtype=torch.uint8, device=DEV)
    L.emit8(dev(x), q, s, n)
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(host(s), s_ref)
    announce("emit8_packed nonfinite n=%d" % n)
    raw = n // 32
    off = (raw + 15) // 16 * 16
    q2 = torch.empty(n, dtype=torch.uint8, device=DEV)
    s2 = torch.zeros(off + raw, dtype=torch.uint8, device=DEV)
    L.emit8_packed(dev(x), q2, s2, n)
    assert np.array_equal(host(q2), q_ref)
    assert np.array_equal(host(s2)[:raw], s_ref)
    announce("snap8 nonfinite n=%d" % n)
    dx = dev(x)
    L.snap8(dx, n)
    got = host(dx)
    want = O.fp8_snap(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_act_quant_f32s_nonfinite_blocks():
    rng = np.random.default_rng(901)
    m, k = 2, 1024
    x = _nonfinite_acts(rng, m * k // 128, 128).reshape(m, k)
    aq_ref, as_ref = O.act_quant_f32s(x, 128)
    announce("act_quant_f32s nonfinite m=%d k=%d" % (m, k))
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 128), dtype=torch.float32, device=DEV)
    L.act_quant_f32s(dev(x), aq, as_, m, k)
    assert np.array_equal(host(aq).ravel(), aq_ref.ravel())
    assert np.array_equal(host(as_).view(np.uint32).ravel(), as_ref.view(np.uint32).ravel())


def test_weight_quant_fp8_nonfinite_blocks():
    rng = np.random.default_rng(902)
    rows, cols = 96, 128
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, 0] = np.inf
    w[40, 70] = -np.inf
    w[70, 100] = FMAX
    q_ref, s_ref = O.weight_quant_fp8(w)
    announce("weight_quant_fp8 nonfinite %dx%d" % (rows, cols))
    q = torch.empty((rows, cols), dtype=torch.uint8, device=DEV)
    s = torch.empty((rows // 32, cols // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(dev(w), q, s, rows, cols)
    assert np.array_equal(host(q).ravel(), q_ref.ravel())
    assert np.array_equal(host(s).ravel(), s_ref.ravel())


@pytest.mark.parametrize("m", [1, 4])
def test_fused_gemv_nonfinite_token_matches_unfused(m):
    """The in-kernel 1x32 quantisation of the fused GEMV (four values per
    lane) against emit8 -> fp8_gemm -> acc_f32: NaN where the unfused chain
    gives NaN, the same bits elsewhere."""
    n, k = 256, 1024
    gen = torch.Generator(device=DEV).manual_seed(903)
    wf = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    w = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    sw = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(wf, w, sw, n, k)
    rng = np.random.default_rng(904)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, 100] = np.inf                              # every output of row 0 NaN
    if m > 1:
        x[1, 200] = np.float32(FMAX)                # finite, e = 120
    dx = dev(x)
    h0 = torch.randn((m, n), device=DEV, generator=gen)
    announce("fp8_gemv_acc nonfinite m=%d" % m)
    xq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    xs = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    o = torch.empty((m, n), device=DEV)
    want = h0.clone()
    L.emit8(dx, xq, xs, m * k)
    L.fp8_gemm(xq, xs, w, sw, o, m, n, k)
    L.acc_f32(o, want, m * n)
    got = h0.clone()
    L.fp8_gemv_acc(dx, w, sw, got, m, n, k)
    g, wt = host(got), host(want)
    assert np.isnan(wt[0]).all()
    assert np.array_equal(np.isnan(g), np.isnan(wt))
    ok = ~np.isnan(wt)
    assert np.array_equal(g[ok].view(np.uint32), wt[ok].view(np.uint32))
