"""GPU tests of the launch.rs-shaped entry points (weightstream-gpu/src/
launch.rs), each against the fused entry points the bench runs (bit for bit:
the same arithmetic) and against the C oracle:

- the decode chain moe_local_slots -> expert_glu -> expert_quant ->
  expert_reduce (engine.rs:4341-4400), also for an expert-parallel rank that
  owns a slice of the experts (e_start, e_len);
- moe_dispatch_ids -> moe_dispatch_tl (int64 ids) and the grouped chain
  moe_grouped_tl(GateUp, w1) / (GateUp, w3) -> moe_swiglu_route ->
  emit8_packed -> moe_grouped_tl(Down) -> moe_combine_f32 (engine.rs:
  4125-4243);
- fp8_gemm_tl for every TlGemm kind with the packed scale words and the
  upload-time packed weight table (engine.rs:842-853);
- split-K GEMMs on two streams at once, each with its own workspace.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, activations, announce, assert_close, dev, host, rand_fp4_weights
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def _i32(n):
    return torch.empty(n, dtype=torch.int32, device=DEV)


def _slabs(gen, E, dim, inter):
    w1, s1 = rand_fp4_weights(gen, E * inter, dim)
    w3, s3 = rand_fp4_weights(gen, E * inter, dim)
    w2, s2 = rand_fp4_weights(gen, E * dim, inter)
    return w1, s1, w3, s3, w2, s2


def _packed(raw, E, dim, inter):
    w1, s1, w3, s3, w2, s2 = raw
    return (L.prepack_fp4_new(w1, s1, E * inter, dim) + L.prepack_fp4_new(w3, s3, E * inter, dim)
            + L.prepack_fp4_new(w2, s2, E * dim, inter))


def _local_slots_ref(ids, e_start, e_len):
    """moe_grouped.cu:23-58: stable insertion sort of the local picks."""
    loc = [(int(e), s) for s, e in enumerate(ids) if e_start <= e < e_start + e_len]
    loc.sort(key=lambda t: t[0])  # Python's sort is stable
    return [s for _, s in loc], [e - e_start for e, _ in loc]


@pytest.mark.parametrize("ids,e_start,e_len", [([20, 3, 31, 0, 7], 0, 32),
                                               ([20, 3, 31, 0, 7, 3], 0, 32),
                                               ([20, 3, 31, 0, 7, 9, 12, 8], 8, 16),
                                               ([40, 41, 42], 0, 32)])
def test_moe_local_slots_and_dispatch_ids(ids, e_start, e_len):
    ids = np.array(ids, np.int32)
    k = ids.size
    announce("moe_local_slots / moe_dispatch_ids k=%d e_start=%d" % (k, e_start))
    ls, le, lc = _i32(k), _i32(k), _i32(1)
    L.moe_local_slots(dev(ids), ls, le, lc, k, e_start, e_len)
    want_s, want_e = _local_slots_ref(ids, e_start, e_len)
    n = int(host(lc)[0])
    assert n == len(want_s)
    assert list(host(ls)[:n]) == want_s and list(host(le)[:n]) == want_e
    di = torch.empty(k, dtype=torch.int64, device=DEV)
    L.moe_dispatch_ids(dev(ids), di, k, e_start, e_len)
    want = [e - e_start if e_start <= e < e_start + e_len else -1 for e in ids]
    assert list(host(di)) == want


@pytest.mark.parametrize("E,dim,inter,ids,e_start,e_len",
                         [(32, 1024, 512, [20, 3, 31, 0, 7], 0, 32),
                          (384, 4096, 2048, [300, 7, 81, 199, 5, 383, 42, 256], 0, 384),
                          (32, 1024, 256, [20, 3, 31, 0, 7, 9, 12, 8], 8, 16)])
def test_reference_decode_chain_matches_moe_decode(E, dim, inter, ids, e_start, e_len):
    """engine.rs:4341-4400: local slots -> expert_glu (f32 h per slot) ->
    expert_quant -> expert_reduce gives ws_moe_decode's bits on the rank's
    picks (picks another rank owns given as -1), with the rank's slice of
    the slabs."""
    ids = np.array(ids, np.int32)
    k = ids.size
    rng = np.random.default_rng(1300 + E)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(1300 + E)
    raw = _slabs(gen, E, dim, inter)
    full = _packed(raw, E, dim, inter)
    # the rank's slice of the experts, packed on its own
    sl = lambda t, rows: t[e_start * rows:(e_start + e_len) * rows]
    part = _packed((sl(raw[0], inter), sl(raw[1], inter), sl(raw[2], inter), sl(raw[3], inter),
                    sl(raw[4], dim), sl(raw[5], dim)), e_len, dim, inter)
    x = rng.standard_normal(dim).astype(np.float32)
    wts = rng.random(k).astype(np.float32)
    announce("reference decode chain E=%d k=%d e_start=%d" % (E, k, e_start))
    xq = torch.empty(dim, dtype=torch.uint8, device=DEV)
    xs = torch.empty(dim // 32, dtype=torch.uint8, device=DEV)
    L.emit8(dev(x), xq, xs, dim)
    ls, le, lc = _i32(k), _i32(k), _i32(1)
    L.moe_local_slots(dev(ids), ls, le, lc, k, e_start, e_len)
    h = torch.zeros((k, inter), dtype=torch.float32, device=DEV)
    L.expert_glu(xq, xs, part[0], part[1], part[2], part[3], dev(wts), ls, le, lc, h, inter, dim,
                 k, e_len)
    q = torch.zeros((k, inter), dtype=torch.uint8, device=DEV)
    qs = torch.zeros((k, inter // 32), dtype=torch.uint8, device=DEV)
    L.expert_quant(h, ls, lc, q, qs, inter, k)
    y = torch.empty(dim, dtype=torch.float32, device=DEV)
    L.expert_reduce(q, qs, part[4], part[5], dev(ids), ls, lc, y, dim, inter, k, e_start, e_len)
    # the fused path on the full slabs with non-local picks dropped
    own = np.where((ids >= e_start) & (ids < e_start + e_len), ids, -1).astype(np.int32)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    y2 = torch.empty(dim, dtype=torch.float32, device=DEV)
    L.moe_decode(dev(x), dev(own), dev(wts), *full, y2, dim, inter, E, k, ws)
    assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))
    # expert_quant's bytes are the fused kernel's for every local slot
    hq2 = torch.zeros((k, inter), dtype=torch.uint8, device=DEV)
    hs2 = torch.zeros((k, inter // 32), dtype=torch.uint8, device=DEV)
    L.expert_glu_quant(xq, xs, dev(own), dev(wts), *full[:4], hq2, hs2, inter, dim, E, k)
    for s in host(ls)[:int(host(lc)[0])]:
        assert torch.equal(q[s], hq2[s]) and torch.equal(qs[s], hs2[s])
    # and the oracle on the rank's picks
    keep = own >= 0
    picked = sorted(set(int(e) for e in own[keep]))
    hostw = [t.view(E, -1)[picked].cpu().numpy() for t in raw]
    remap = np.array([picked.index(int(e)) for e in own[keep]], np.int32)
    want = O.moe_routed(*hostw, dim, inter, x, remap, wts[keep])
    assert_close(host(y), want, TOL, "reference decode chain")


def _pack_weight_scales(sb, n, k):
    """engine.rs:842-853: row r gets the words of its 32-row block."""
    return np.ascontiguousarray(np.repeat(sb, 32, axis=0)[:n]).view(np.uint32).reshape(n, k // 128)


@pytest.mark.parametrize("kind", list(range(10)))
@pytest.mark.parametrize("m", [1, 6])
def test_fp8_gemm_tl_every_kind(kind, m):
    """fp8_gemm_tl(kind) with the packed activation words (emit8_packed's
    tail) and the packed per-row weight table equals fp8_gemm on the raw
    bytes bit for bit, and the oracle within tolerance (m = 1)."""
    n, k = L.tl_gemm_shape(kind)
    rng = np.random.default_rng(1400 + kind + m)
    x = activations(rng, m, k)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(1400 + kind)
    wf = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    wq = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    ws = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(wf, wq, ws, n, k)
    del wf
    announce("fp8_gemm_tl kind=%d (%d x %d) m=%d" % (kind, n, k, m))
    raw = m * k // 32
    tail = (raw + 15) // 16 * 16
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    sa = torch.zeros(tail + raw + 16, dtype=torch.uint8, device=DEV)
    L.emit8_packed(dev(x), aq, sa, m * k)
    words = sa[tail:tail + raw].clone()            # the packed-word half
    table = dev(_pack_weight_scales(host(ws), n, k).view(np.int32))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm_tl(kind, aq, words, wq, table, out, m)
    ref = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(aq, sa[:raw], wq, ws, ref, m, n, k)
    assert np.array_equal(host(out).view(np.uint32), host(ref).view(np.uint32))
    if m == 1:
        want = O.gemm_q(host(aq), host(sa[:raw]), m, host(wq), host(ws), n, k, False)
        assert_close(host(out), want, TOL, "fp8_gemm_tl kind %d" % kind)


@pytest.mark.parametrize("m,E,dim,inter,k", [(40, 64, 1024, 512, 6), (132, 384, 4096, 2048, 8)])
def test_reference_grouped_chain_matches_oracle(m, E, dim, inter, k):
    """engine.rs:4125-4243 step by step: moe_dispatch_ids -> moe_dispatch_tl
    (int64 ids; the same arrays as the int32 dispatch) -> moe_grouped_tl
    GateUp with w1 and with w3 -> moe_swiglu_route -> emit8_packed ->
    moe_grouped_tl Down -> moe_combine_f32; each token's row against the
    oracle's routed MoE."""
    rng = np.random.default_rng(1500 + m)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(1500 + m)
    raw = _slabs(gen, E, dim, inter)
    P = _packed(raw, E, dim, inter)
    logits = rng.standard_normal((m, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    idx = _i32(m * k).view(m, k)
    w = torch.empty((m, k), dtype=torch.float32, device=DEV)
    L.moe_topk(dev(logits), dev(bias), None, idx, w, m, E, k, O.SCORE_SIGMOID, 1.0, True, 1.0)
    x = rng.standard_normal((m, dim)).astype(np.float32)
    announce("reference grouped chain m=%d E=%d" % (m, E))
    routes, tiles = m * k, L.moe_tiles(m * k, E)
    di = torch.empty(routes, dtype=torch.int64, device=DEV)
    L.moe_dispatch_ids(idx, di, routes, 0, E)
    # slots past the used tiles are not written: both runs start from -7
    arrs = [torch.full((n,), -7, dtype=dt, device=DEV)
            for n, dt in [(tiles * 32, torch.int32), (tiles * 32, torch.float32), (routes, torch.int32),
                          (tiles, torch.int32), (E, torch.int32), (E, torch.int32), (E, torch.int32),
                          (1, torch.int32)]]
    arrs32 = [a.clone() for a in arrs]
    L.moe_dispatch_tl(di, w, *arrs, m, k, tiles, E)
    L.moe_dispatch_tl(idx, w, *arrs32, m, k, tiles, E)
    for a, b in zip(arrs, arrs32):
        assert torch.equal(a, b)
    order, lw, route_pos, tile_expert = arrs[:4]
    xq = torch.empty((m, dim), dtype=torch.uint8, device=DEV)
    xs = torch.empty((m, dim // 32), dtype=torch.uint8, device=DEV)
    L.emit8(dev(x), xq, xs, m * dim)
    gate = torch.zeros((tiles * 32, inter), dtype=torch.float32, device=DEV)
    up = torch.zeros((tiles * 32, inter), dtype=torch.float32, device=DEV)
    L.moe_grouped_tl(L.TL_MOE_GATE_UP, xq, xs, P[0], P[1], order, tile_expert, gate, tiles, m, k,
                     inter, dim, E)
    L.moe_grouped_tl(L.TL_MOE_GATE_UP, xq, xs, P[2], P[3], order, tile_expert, up, tiles, m, k,
                     inter, dim, E)
    L.moe_swiglu_route(gate, up, lw, gate, inter, tiles * 32)
    n = tiles * 32 * inter
    tail = (n // 32 + 15) // 16 * 16
    hq = torch.empty((tiles * 32, inter), dtype=torch.uint8, device=DEV)
    hs = torch.empty(tail + n // 32, dtype=torch.uint8, device=DEV)
    L.emit8_packed(gate, hq, hs, n)
    down = torch.zeros((tiles * 32, dim), dtype=torch.float32, device=DEV)
    L.moe_grouped_tl(L.TL_MOE_DOWN, hq, hs[tail:], P[4], P[5], order, tile_expert, down, tiles, m,
                     k, dim, inter, E)
    y = torch.empty((m, dim), dtype=torch.float32, device=DEV)
    L.moe_combine_f32(down, route_pos, y, dim, k, m, tiles)
    gi, gw, gy = host(idx), host(w), host(y)
    rows = range(m) if m <= 40 else [0, 17, 64, 131]
    for r in rows:
        picked = sorted(set(int(e) for e in gi[r]))
        hostw = [t.view(E, -1)[picked].cpu().numpy() for t in raw]
        remap = np.array([picked.index(int(e)) for e in gi[r]], np.int32)
        want = O.moe_routed(*hostw, dim, inter, x[r], remap, gw[r])
        assert_close(gy[r], want, TOL, "reference grouped chain row %d" % r)


def test_moe_swiglu_route_bit_exact():
    rng = np.random.default_rng(1600)
    rows, inter = 64, 512
    g = (rng.standard_normal((rows, inter)) * 8).astype(np.float32)
    u = (rng.standard_normal((rows, inter)) * 8).astype(np.float32)
    lw = rng.random(rows).astype(np.float32)
    lw[::5] = 0.0                                     # padding slots
    announce("moe_swiglu_route")
    out = torch.empty((rows, inter), dtype=torch.float32, device=DEV)
    L.moe_swiglu_route(dev(g), dev(u), dev(lw), out, inter, rows)
    got = host(out)
    for r in range(rows):
        if lw[r] == 0.0:
            assert not got[r].any()
            continue
        want = np.array([np.float32(np.float32(O.silu(float(min(a, np.float32(10)))) *
                                               np.float32(np.clip(b, -10, 10))) * lw[r])
                         for a, b in zip(g[r], u[r])], np.float32)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r


def test_split_k_gemms_on_two_streams_are_independent():
    """Each stream has its own split-K workspace: GEMMs issued alternately on
    two streams, with no ordering between them, give the bits of the same
    GEMMs run one at a time on one stream."""
    rng = np.random.default_rng(1700)
    shapes = [(128, 4096, 4096), (128, 12288, 4096), (8, 1280, 15360), (200, 2048, 1024)]
    cases = []
    for (m, n, k) in shapes:
        aq, as_ = O.fp8_act_emit(activations(rng, m, k))
        gen = torch.Generator(device=DEV)
        gen.manual_seed(n + k)
        wf = torch.randn((n, k), device=DEV, generator=gen) * 0.02
        wq = torch.empty((n, k), dtype=torch.uint8, device=DEV)
        ws = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
        L.weight_quant_fp8(wf, wq, ws, n, k)
        cases.append((dev(aq), dev(as_), wq, ws, m, n, k))
    announce("split-K GEMMs on two streams")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    need = max(L.gemm_workspace_size(m, n, k) for (_, _, _, _, m, n, k) in cases)
    assert need > 0
    w1 = torch.empty(need, dtype=torch.uint8, device=DEV)
    w2 = torch.empty(need, dtype=torch.uint8, device=DEV)
    # one stream at a time
    ref = []
    L.set_gemm_workspace(w1, stream=s1)
    try:
        for a, sa, b, sb, m, n, k in cases:
            o = torch.empty((m, n), dtype=torch.float32, device=DEV)
            L.fp8_gemm(a, sa, b, sb, o, m, n, k, stream=s1)
            ref.append(o)
        s1.synchronize()
        L.set_gemm_workspace(w2, stream=s2)
        outs = [[torch.empty_like(r) for r in ref] for _ in range(2)]
        torch.cuda.synchronize()
        for rep in range(4):
            for i, (a, sa, b, sb, m, n, k) in enumerate(cases):
                L.fp8_gemm(a, sa, b, sb, outs[0][i], m, n, k, stream=s1)
                L.fp8_gemm(a, sa, b, sb, outs[1][i], m, n, k, stream=s2)
        torch.cuda.synchronize()
        for i in range(len(cases)):
            for j in range(2):
                assert torch.equal(outs[j][i], ref[i]), (shapes[i], j)
    finally:
        torch.cuda.synchronize()
        L.set_gemm_workspace(None, stream=s1)
        L.set_gemm_workspace(None, stream=s2)
