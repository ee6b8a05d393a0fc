"""The GPU path on the committed golden fixtures (tests/golden/*.npz, seeded
inputs with the C oracle's outputs): quantisation, routing and dispatch bit
for bit, GEMM and MoE outputs within the parity tolerance (max relative error
1e-3, floor at 1% of the output scale; bf16 2^-8 + 1e-3)."""
import os

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, dev, host
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_golden_quantisation_bit_exact():
    g = load("quant")
    announce("golden quant")
    x, w = g["x"], g["w"]
    q = torch.empty(x.shape, dtype=torch.uint8, device=DEV)
    s = torch.empty((x.shape[0], x.shape[1] // 32), dtype=torch.uint8, device=DEV)
    L.emit8(dev(x), q, s, x.size)
    assert np.array_equal(host(q), g["aq"]) and np.array_equal(host(s), g["as_"])
    r, c = w.shape
    q8 = torch.empty((r, c), dtype=torch.uint8, device=DEV)
    s8 = torch.empty(((r + 31) // 32, c // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(dev(w), q8, s8, r, c)
    assert np.array_equal(host(q8), g["w8"]) and np.array_equal(host(s8), g["s8"])
    q4 = torch.empty((r, c // 2), dtype=torch.uint8, device=DEV)
    s4 = torch.empty((r, c // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp4(dev(w), q4, s4, r, c)
    assert np.array_equal(host(q4), g["w4"]) and np.array_equal(host(s4), g["s4"])


def test_golden_gemm():
    g = load("gemm")
    m, n, k = (int(v) for v in g["shape"])
    announce("golden gemm %dx%dx%d" % (m, n, k))
    aq, as_ = dev(g["aq"]), dev(g["as_"])
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(aq, as_, dev(g["w8"]), dev(g["s8"]), out, m, n, k)
    assert_close(host(out), g["y8"], TOL, "golden fp8_gemm")
    L.fp4_gemm(aq, as_, dev(g["w4"]), dev(g["s4"]), out, m, n, k)
    assert_close(host(out), g["y4"], TOL, "golden fp4_gemm")
    ob = torch.empty((m, n), dtype=torch.int16, device=DEV)
    L.fp8_gemm_bf16(aq, as_, dev(g["w8"]), dev(g["s8"]), ob, m, n, k)
    got = (host(ob).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    assert_close(got, g["y8"], 2.0 ** -8 + TOL, "golden fp8_gemm_bf16")


@pytest.mark.parametrize("score", [L.SCORE_SOFTMAX, L.SCORE_SIGMOID, L.SCORE_SQRTSOFTPLUS])
def test_golden_routing_bit_exact(score):
    g = load("route")
    rows, e = g["logits"].shape
    k = g["idx_%d" % score].shape[1]
    announce("golden route score=%d" % score)
    idx = torch.empty((rows, k), dtype=torch.int32, device=DEV)
    w = torch.empty((rows, k), dtype=torch.float32, device=DEV)
    L.moe_topk(dev(g["logits"]), dev(g["bias"]), None, idx, w, rows, e, k, score, 1.0, True, 2.5)
    assert np.array_equal(host(idx), g["idx_%d" % score])
    assert np.array_equal(host(w).view(np.uint32), g["w_%d" % score].view(np.uint32))


@pytest.mark.parametrize("ids", [np.int32, np.int64])
def test_golden_dispatch_bit_exact(ids):
    g = load("dispatch")
    m, k = g["idx"].shape
    e, tiles = int(g["experts"][0]), int(g["tiles"][0])
    announce("golden dispatch")
    i32 = lambda n: torch.full((n,), -7, dtype=torch.int32, device=DEV)
    order, lw = i32(tiles * 32), torch.full((tiles * 32,), -7.0, device=DEV)
    rp, te, cnt, off, ps, nt = i32(m * k), i32(tiles), i32(e), i32(e), i32(e), i32(1)
    L.moe_dispatch_tl(dev(g["idx"].astype(ids)), dev(g["w"]), order, lw, rp, te, cnt, off, ps, nt, m, k,
                      tiles, e)
    assert int(host(nt)[0]) == int(g["out_num_tiles"])
    used = int(g["out_num_tiles"]) * 32
    for key, t in (("route_pos", rp), ("tile_expert", te), ("count", cnt), ("offset", off),
                   ("psum", ps)):
        assert np.array_equal(host(t), g["out_" + key]), key
    assert np.array_equal(host(order)[:used], g["out_order"][:used])
    assert np.array_equal(host(lw)[:used].view(np.uint32), g["out_layout_w"][:used].view(np.uint32))


def test_golden_moe_decode_and_shared_expert():
    g = load("moe")
    e, dim, inter, k = (int(v) for v in g["shape"])
    announce("golden moe decode E=%d dim=%d inter=%d k=%d" % (e, dim, inter, k))
    p1 = L.prepack_fp4_new(dev(g["w1"]), dev(g["s1"]), e * inter, dim)
    p3 = L.prepack_fp4_new(dev(g["w3"]), dev(g["s3"]), e * inter, dim)
    p2 = L.prepack_fp4_new(dev(g["w2"]), dev(g["s2"]), e * dim, inter)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    y = torch.empty(dim, dtype=torch.float32, device=DEV)
    L.moe_decode(dev(g["x"]), dev(g["idx"]), dev(g["w"]), *p1, *p3, *p2, y, dim, inter, e, k, ws)
    assert_close(host(y), g["y"], TOL, "golden moe_decode")
    sws = torch.empty(L.shared_expert_workspace_size(1, dim, inter), dtype=torch.uint8,
                      device=DEV)
    ys = torch.empty(dim, dtype=torch.float32, device=DEV)
    L.shared_expert_fp8(dev(g["x"]), dev(g["f1"]), dev(g["g1"]), dev(g["f3"]), dev(g["g3"]),
                        dev(g["f2"]), dev(g["g2"]), ys, 1, dim, inter, sws)
    assert_close(host(ys), g["ys"], TOL, "golden shared_expert_fp8")
