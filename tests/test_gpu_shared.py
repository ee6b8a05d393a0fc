"""GPU parity of the shared FP8 expert (weightstream-ref moe.rs:210-250,
shared_expert_hidden) and acc_f32 (gemv.cu:63), called through the C ABI and
checked against the C oracle on the same seeded inputs.

Tolerance: max relative error <= 1e-3 on the f32 output (floor at 1% of the
output scale). The GEMM sums differ from the oracle's sequential order by f32
reassociation; re-quantising h to FP8 can move a value that sits on a
rounding boundary by one e4m3 step, which the tolerance covers. acc_f32 is one
f32 add per element: bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, announce, assert_close, dev, host
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def _fp8_weights(rng, rows, cols):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    return O.weight_quant_fp8(w)


@pytest.mark.parametrize("m,dim,inter,limit", [(1, 4096, 2048, 10.0), (3, 512, 256, 10.0),
                                               (64, 1024, 512, 10.0), (5, 256, 384, 0.0)])
@pytest.mark.parametrize("split_k", [False, True])
def test_shared_expert_matches_oracle(m, dim, inter, limit, split_k):
    rng = np.random.default_rng(7000 + m + dim + inter)
    w1, s1 = _fp8_weights(rng, inter, dim)
    w3, s3 = _fp8_weights(rng, inter, dim)
    w2, s2 = _fp8_weights(rng, dim, inter)
    # gate/up outputs large enough that the +-L clamps bite on some elements
    x = (rng.standard_normal((m, dim)) * 4.0).astype(np.float32)
    want = np.stack([O.shared_fp8(w1, s1, w3, s3, w2, s2, dim, inter, x[t], limit)
                     for t in range(m)])
    announce("shared_expert_fp8 m=%d dim=%d inter=%d limit=%g split_k=%d"
             % (m, dim, inter, limit, split_k))
    gws = None
    if split_k:
        gws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
        L.set_gemm_workspace(gws)
    try:
        ws = torch.empty(L.shared_expert_workspace_size(m, dim, inter), dtype=torch.uint8,
                         device=DEV)
        y = torch.full((m, dim), float("nan"), dtype=torch.float32, device=DEV)
        d = [dev(a) for a in (w1, s1, w3, s3, w2, s2)]
        L.shared_expert_fp8(dev(x), *d, y, m, dim, inter, ws, swiglu_limit=limit)
        got = host(y)
    finally:
        torch.cuda.synchronize()
        if gws is not None:
            L.set_gemm_workspace(None)
    assert_close(got, want, TOL, "shared_expert_fp8 m=%d dim=%d inter=%d" % (m, dim, inter))


@pytest.mark.parametrize("m,dim,inter", [(1, 4096, 2048), (6, 5120, 2304), (64, 1024, 512)])
def test_shared_expert_w13_matches_oracle(m, dim, inter):
    """w1 and w3 fused row-wise (the engine's shared_w13): the same expert."""
    rng = np.random.default_rng(7100 + m + dim)
    w1, s1 = _fp8_weights(rng, inter, dim)
    w3, s3 = _fp8_weights(rng, inter, dim)
    w2, s2 = _fp8_weights(rng, dim, inter)
    x = (rng.standard_normal((m, dim)) * 4.0).astype(np.float32)
    want = np.stack([O.shared_fp8(w1, s1, w3, s3, w2, s2, dim, inter, x[t], 10.0)
                     for t in range(m)])
    announce("shared_expert_fp8_w13 m=%d dim=%d inter=%d" % (m, dim, inter))
    gws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    L.set_gemm_workspace(gws)
    try:
        ws = torch.empty(L.shared_expert_workspace_size(m, dim, inter), dtype=torch.uint8,
                         device=DEV)
        y = torch.full((m, dim), float("nan"), dtype=torch.float32, device=DEV)
        L.shared_expert_fp8_w13(dev(x), dev(np.concatenate([w1, w3])), dev(np.concatenate([s1, s3])),
                                dev(w2), dev(s2), y, m, dim, inter, ws)
        got = host(y)
    finally:
        torch.cuda.synchronize()
        L.set_gemm_workspace(None)
    assert_close(got, want, TOL, "shared_expert_fp8_w13 m=%d dim=%d inter=%d" % (m, dim, inter))


def test_shared_expert_rejects_bad_shapes():
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    b = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    f = torch.zeros(1 << 14, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        L.shared_expert_fp8(f, b, b, b, b, b, b, f, 1, 100, 128, ws)   # dim % 128
    with pytest.raises(RuntimeError):
        L.shared_expert_fp8(f, b, b, b, b, b, b, f, 1, 128, 128, ws[:16])  # workspace too small


@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_acc_f32_bit_exact(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    announce("acc_f32 n=%d" % n)
    dy = dev(y0)
    L.acc_f32(dev(x), dy, n)
    want = (y0 + x).astype(np.float32)
    assert np.array_equal(host(dy).view(np.uint32), want.view(np.uint32))


def test_shared_expert_w13_rejects_bad_shapes():
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    b = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    f = torch.zeros(1 << 14, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        L.shared_expert_fp8_w13(f, b, b, b, b, f, 1, 128, 100, ws)  # inter % 128
    with pytest.raises(RuntimeError):
        L.shared_expert_fp8_w13(f, b, b, b, b, f, 1, 128, 128, ws[:16])  # workspace too small
