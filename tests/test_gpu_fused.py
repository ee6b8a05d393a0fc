"""GPU checks of the fused block steps against the unfused launches they
replace, bit for bit (both are the same FP8 GEMV sums, in the same order):

  ws_fp8_gemv_acc              == emit8 -> fp8_gemm -> acc_f32 (launch.rs:1175)
  ws_fp8_gemm_acc              == fp8_gemm -> acc_f32
  ws_shared_expert_fp8_w13_acc == ws_shared_expert_fp8_w13 -> acc_f32(ys, yr)
                                  -> acc_f32(yr, h)   (engine.rs:4532)
  ws_moe_gate_shared_w13 + ws_shared_expert_down_acc
                               == ws_moe_gate_logits + the line above
  ws_moe_decode_route_shared   == ws_moe_decode_route + ws_shared_expert_down_acc

The unfused chains are themselves checked against the oracle
(test_gpu_kernels.py, test_gpu_block.py). Both math modes."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


@pytest.fixture(params=[L.MATH_EXACT, L.MATH_NATIVE], ids=["exact", "native"])
def mode(request):
    prev = L.set_math_mode(request.param)
    yield request.param
    L.set_math_mode(prev)


def _fp8(gen, rows, cols):
    w = torch.empty((rows, cols), dtype=torch.float32, device=DEV).normal_(0.0, 0.02,
                                                                          generator=gen)
    q = torch.empty((rows, cols), dtype=torch.uint8, device=DEV)
    s = torch.empty((rows // 32, cols // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(w, q, s, rows, cols)
    return q, s


def _x(gen, m, k):
    x = torch.randn((m, k), device=DEV, generator=gen)
    x[:, ::97] *= 20.0                          # outliers, as BASELINE config 2
    return x


@pytest.mark.parametrize("m,n,k", [(1, 4096, 8192), (8, 4096, 8192), (16, 2048, 4096),
                                   (3, 512, 2048), (1, 4096, 128)])
def test_gemv_acc_bit_exact(mode, m, n, k):
    announce("fp8_gemv_acc mode=%d m=%d n=%d k=%d" % (mode, m, n, k))
    gen = torch.Generator(device=DEV).manual_seed(m * 7 + n + k)
    w, sw = _fp8(gen, n, k)
    x = _x(gen, m, k)
    h0 = torch.randn((m, n), device=DEV, generator=gen)
    xq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    xs = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    o = torch.empty((m, n), device=DEV)
    want = h0.clone()
    L.emit8(x, xq, xs, m * k)
    L.fp8_gemm(xq, xs, w, sw, o, m, n, k)
    L.acc_f32(o, want, m * n)
    got = h0.clone()
    L.fp8_gemv_acc(x, w, sw, got, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (8, 4096, 8192), (20, 512, 1024),
                                   (64, 4096, 8192), (64, 12288, 4096), (48, 2048, 2304),
                                   (128, 4096, 4096), (128, 2048, 4096)])
def test_gemm_acc_bit_exact(mode, m, n, k):
    """ws_fp8_gemm_acc == emit8 -> fp8_gemm -> acc_f32 on the shapes where
    both run the same kernel (no split-K workspace registered): column strips
    (m <= 64), the line kernel (32 x 32 and 64 x 32 tiles)."""
    announce("fp8_gemm_acc mode=%d m=%d n=%d k=%d" % (mode, m, n, k))
    gen = torch.Generator(device=DEV).manual_seed(m * 5 + n + k)
    w, sw = _fp8(gen, n, k)
    x = _x(gen, m, k)
    h0 = torch.randn((m, n), device=DEV, generator=gen)
    xq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    xs = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    L.emit8(x, xq, xs, m * k)
    o = torch.empty((m, n), device=DEV)
    want = h0.clone()
    L.fp8_gemm(xq, xs, w, sw, o, m, n, k)
    L.acc_f32(o, want, m * n)
    got = h0.clone()
    L.fp8_gemm_acc(xq, xs, w, sw, got, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("m,limit", [(1, 10.0), (1, 0.0), (8, 10.0), (16, 10.0), (20, 10.0),
                                     (64, 10.0), (64, 0.0)])
def test_shared_w13_acc_bit_exact(mode, m, limit):
    dim, inter = 4096, 2048
    announce("shared_expert_fp8_w13_acc mode=%d m=%d limit=%g" % (mode, m, limit))
    gen = torch.Generator(device=DEV).manual_seed(100 + m)
    w13, s13 = _fp8(gen, 2 * inter, dim)
    w2, s2 = _fp8(gen, dim, inter)
    h0 = torch.randn((m, dim), device=DEV, generator=gen)
    yr0 = torch.randn((m, dim), device=DEV, generator=gen)
    ws = torch.empty(L.shared_expert_workspace_size(m, dim, inter), dtype=torch.uint8,
                     device=DEV)
    ys = torch.empty((m, dim), device=DEV)
    # unfused: x is h itself, as in the block
    want, yr = h0.clone(), yr0.clone()
    L.shared_expert_fp8_w13(want, w13, s13, w2, s2, ys, m, dim, inter, ws, swiglu_limit=limit)
    L.acc_f32(ys, yr, m * dim)
    L.acc_f32(yr, want, m * dim)
    got, yr2 = h0.clone(), yr0.clone()
    L.shared_expert_fp8_w13_acc(got, w13, s13, w2, s2, yr2, got, m, dim, inter, ws,
                                swiglu_limit=limit)
    torch.cuda.synchronize()
    assert torch.equal(yr2, yr0)                # yr is not written
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("m,limit", [(1, 10.0), (1, 0.0), (4, 10.0), (8, 10.0)])
def test_gate_shared_split_bit_exact(mode, m, limit):
    dim, inter, E = 4096, 2048, 384
    announce("moe_gate_shared_w13 + shared_expert_down_acc mode=%d m=%d limit=%g" % (mode, m, limit))
    gen = torch.Generator(device=DEV).manual_seed(200 + m)
    w13, s13 = _fp8(gen, 2 * inter, dim)
    w2, s2 = _fp8(gen, dim, inter)
    gw = torch.empty((E, dim), device=DEV).normal_(0.0, 0.02, generator=gen)
    h0 = torch.randn((m, dim), device=DEV, generator=gen)
    yr = torch.randn((m, dim), device=DEV, generator=gen)
    ws = torch.empty(L.shared_expert_workspace_size(m, dim, inter), dtype=torch.uint8,
                     device=DEV)
    lg_want = torch.empty((m, E), device=DEV)
    want = h0.clone()
    L.moe_gate_logits(want, gw, lg_want, m, dim, E)
    L.shared_expert_fp8_w13_acc(want, w13, s13, w2, s2, yr, want, m, dim, inter, ws,
                                swiglu_limit=limit)
    lg = torch.full((m, E), float("nan"), device=DEV)
    hs = torch.empty((m, inter), device=DEV)
    got = h0.clone()
    L.moe_gate_shared_w13(got, gw, lg, w13, s13, hs, m, dim, E, inter, swiglu_limit=limit)
    L.shared_expert_down_acc(hs, w2, s2, yr, got, m, dim, inter)
    torch.cuda.synchronize()
    assert torch.equal(lg.view(torch.int32), lg_want.view(torch.int32))
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def _slabs(gen, E, dim, inter):
    """Packed FP4 expert slabs (w1, s1, w3, s3, w2, s2) of E experts."""
    def enc(rows, cols):
        w = torch.empty((rows, cols), device=DEV).normal_(0.0, 0.02, generator=gen)
        q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=DEV)
        sc = torch.empty((rows, cols // 32), dtype=torch.uint8, device=DEV)
        L.weight_quant_fp4(w, q, sc, rows, cols)
        return L.prepack_fp4_new(q, sc, rows, cols)
    return enc(E * inter, dim) + enc(E * inter, dim) + enc(E * dim, inter)


@pytest.mark.parametrize("E,score,limit", [(64, L.SCORE_SIGMOID, 10.0),
                                           (96, L.SCORE_SQRTSOFTPLUS, 0.0)])
def test_decode_route_shared_bit_exact(mode, E, score, limit):
    dim, inter, k, si = 4096, 2048, 8, 2048
    announce("moe_decode_route_shared mode=%d E=%d score=%d" % (mode, E, score))
    gen = torch.Generator(device=DEV).manual_seed(300 + E)
    routed = _slabs(gen, E, dim, inter)
    w2s, s2s = _fp8(gen, dim, si)
    logits = torch.randn(E, device=DEV, generator=gen)
    bias = torch.randn(E, device=DEV, generator=gen) * 0.1
    x = torch.randn(dim, device=DEV, generator=gen)
    hsf = torch.randn(si, device=DEV, generator=gen) * 0.1
    h0 = torch.randn(dim, device=DEV, generator=gen)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    outs = []
    for fused in (False, True):
        y = torch.full((dim,), float("nan"), device=DEV)
        idx = torch.full((k,), -5, dtype=torch.int32, device=DEV)
        w = torch.full((k,), float("nan"), device=DEV)
        h = h0.clone()
        if fused:
            ys = torch.full((dim,), float("nan"), device=DEV)
            L.moe_decode_route_shared(logits, bias, score, 1.0, 1, 2.5, x, *routed, y, idx, w, dim,
                                      inter, E, k, hsf, w2s, s2s, si, ys, h, ws,
                                      swiglu_limit=limit)
        else:
            L.moe_decode_route(logits, bias, score, 1.0, 1, 2.5, x, *routed, y, idx, w, dim,
                               inter, E, k, ws, swiglu_limit=limit)
            L.shared_expert_down_acc(hsf, w2s, s2s, y, h, 1, dim, si)
        torch.cuda.synchronize()
        outs.append((y, idx, w, h))
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_fused_rejects_bad_shapes():
    x = torch.zeros((17, 256), device=DEV)
    w = torch.zeros((32, 256), dtype=torch.uint8, device=DEV)
    sw = torch.zeros((1, 8), dtype=torch.uint8, device=DEV)
    h = torch.zeros((17, 32), device=DEV)
    with pytest.raises(RuntimeError):
        L.fp8_gemv_acc(x, w, sw, h, 17, 32, 256)        # m > 16
    with pytest.raises(RuntimeError):
        L.fp8_gemv_acc(x, w, sw, h, 1, 32, 200)         # k % 128
