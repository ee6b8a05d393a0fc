"""Pin the oracle's routing, expert and dispatch restatements
(weightstream-ref/src/moe.rs, num.rs; moe_dispatch.cu's contract)."""
import math

import numpy as np
import pytest

import oracle_lib as O


# ---- num.rs --------------------------------------------------------------
def test_num_special_points():
    assert O.sigmoid(0.0) == 0.5
    assert O.silu(0.0) == 0.0
    assert O.softplus(25.0) == 25.0                      # threshold 20
    assert abs(O.softplus(0.0) - math.log(2.0)) < 1e-7
    assert O.sigmoid(-200.0) == 0.0 and O.sigmoid(200.0) == 1.0
    x = np.array([1.0, 2.0, 3.0], np.float32)
    s = O.softmax(x)
    e = np.exp(x.astype(np.float64) - 3)
    assert np.allclose(s, e / e.sum(), rtol=1e-6)


def test_dot_is_sequential():
    # (1e8 + 1) - 1e8 evaluated left to right in f32 loses the 1
    a = np.array([1e8, 1.0, -1e8], np.float32)
    b = np.ones(3, np.float32)
    assert O.dot(a, b) == 0.0
    assert O.dot(a[[0, 2, 1]], b) == 1.0


# ---- moe.rs:45-69 routing -----------------------------------------------
def _brute_route(scores, bias, k, norm, route_scale):
    """Rank each expert by counting how many beat it under (value desc,
    index asc), with -0.0 < +0.0 as in f32::total_cmp."""
    biased = (scores + bias).astype(np.float32)

    def beats(j, i):
        a, b = float(biased[j]), float(biased[i])
        if a != b:
            return a > b
        sa, sb = math.copysign(1, a), math.copysign(1, b)
        if sa != sb:
            return sa > sb
        return j < i

    n = len(scores)
    rank = [sum(beats(j, i) for j in range(n) if j != i) for i in range(n)]
    order = sorted(range(n), key=lambda i: rank[i])[:k]
    w = [np.float32(scores[i]) for i in order]
    if norm and k > 1:
        tot = np.float32(-0.0)
        for v in w:
            tot = np.float32(tot + v)
        w = [np.float32(v / np.float32(tot + np.float32(1e-20))) for v in w]
    w = [np.float32(v * np.float32(route_scale)) for v in w]
    return np.array(order, np.int32), np.array(w, np.float32)


@pytest.mark.parametrize("score_func", [O.SCORE_SIGMOID, O.SCORE_SOFTMAX, O.SCORE_SQRTSOFTPLUS])
def test_route_matches_bruteforce_with_ties(score_func):
    rng = np.random.default_rng(21)
    E, k = 64, 8
    for trial in range(20):
        logits = rng.standard_normal(E).astype(np.float32)
        bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
        if trial % 2:
            # inject exact ties on the biased score, including +0/-0
            s = O.score(logits, score_func)
            bias[5] = np.float32(s[9] + bias[9] - s[5])
            bias[17] = np.float32(s[3] + bias[3] - s[17])
        scores = O.score(logits, score_func)
        if trial == 3:
            scores[:] = 0.0
            bias[:] = 0.0
            bias[7] = -0.0
            scores[11] = -0.0
        idx, w = O.route(scores, bias, k, True, 1.5)
        bi, bw = _brute_route(scores, bias, k, True, 1.5)
        assert np.array_equal(idx, bi)
        assert np.array_equal(w.view(np.uint32), bw.view(np.uint32))


def test_score_functions_closed_form():
    x = np.array([-3.0, 0.0, 0.5, 25.0], np.float32)
    sig = O.score(x, O.SCORE_SIGMOID)
    assert np.allclose(sig, 1 / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6)
    ssp = O.score(x, O.SCORE_SQRTSOFTPLUS)
    want = np.sqrt(np.where(x > 20, x, np.log1p(np.exp(x.astype(np.float64)))))
    assert np.allclose(ssp, want, rtol=1e-6)
    t = O.score(x, O.SCORE_SIGMOID, 2.0)
    assert np.allclose(t, 1 / (1 + np.exp(-x.astype(np.float64) / 2)), rtol=1e-6)


# ---- experts ---------------------------------------------------------------
def test_grouped_closed_form_of_reference_gpu_test():
    """weightstream-gpu/src/tests.rs:837-1020 at small K: all-0x11 FP4
    weights (every value 0.5, unit scales) and x = 0.01 give gate = up =
    K * 0.5 * e4m3_snap(0.01); the final routed sum of two experts with
    weight 1 is 2 * h * 0.5 * inter where h is the FP8-snapped SwiGLU."""
    dim, inter, E = 1024, 256, 4
    w_up = np.full((E, inter, dim // 2), 0x11, np.uint8)
    s_up = np.full((E, inter, dim // 32), 127, np.uint8)
    w_dn = np.full((E, dim, inter // 2), 0x11, np.uint8)
    s_dn = np.full((E, dim, inter // 32), 127, np.uint8)
    x = np.full(dim, 0.01, np.float32)
    xa = np.float32(0.009765625)                 # e4m3 snap of 0.01, scale 2^-15
    assert O.fp8_snap(x[:32])[0] == xa
    g = np.float32(dim * 0.5 * xa)                # exact: 5.0 at dim=1024
    gc = min(g, np.float32(10))
    h = np.float32(np.float32(gc * np.float32(1 / (1 + math.exp(-float(gc))))) * min(g, 10))
    sc = 2.0 ** math.ceil(math.log2(h / 448.0))
    hq = O.e4m3_to_f32(O.f32_to_e4m3(float(h / sc))) * sc
    want = 2.0 * hq * 0.5 * inter
    y = O.moe_routed(w_up, s_up, w_up, s_up, w_dn, s_dn, dim, inter, x,
                     np.array([2, 0], np.int32), np.array([1.0, 1.0], np.float32))
    assert np.all(np.abs(y - want) <= 1e-6 * want)


def _rand_experts(rng, E, dim, inter):
    def q(rows, cols):
        return O.weight_quant_fp4((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    w1 = [q(inter, dim) for _ in range(E)]
    w3 = [q(inter, dim) for _ in range(E)]
    w2 = [q(dim, inter) for _ in range(E)]
    st = lambda L, i: np.stack([a[i] for a in L])
    return (st(w1, 0), st(w1, 1), st(w3, 0), st(w3, 1), st(w2, 0), st(w2, 1))


def test_routing_weight_applies_before_w2():
    """moe.rs:267-298: expert(1.5 w) != 1.5 expert(w)."""
    rng = np.random.default_rng(22)
    dim, inter = 256, 64
    W = _rand_experts(rng, 1, dim, inter)
    x = np.array([((i % 7) - 3.0) * 0.11 for i in range(dim)], np.float32)
    a = O.expert_fp4(*[v[0] for v in W], dim, inter, x, 1.0)
    b = O.expert_fp4(*[v[0] for v in W], dim, inter, x, 1.5)
    assert not np.array_equal(b, np.float32(1.5) * a)
    assert np.all(np.isfinite(b))


def test_moe_routed_is_ascending_sum_of_experts():
    rng = np.random.default_rng(23)
    E, dim, inter, k = 6, 256, 64, 3
    W = _rand_experts(rng, E, dim, inter)
    x = rng.standard_normal(dim).astype(np.float32)
    idx = np.array([4, 1, 3], np.int32)
    w = np.array([0.5, 0.3, 0.2], np.float32)
    y = O.moe_routed(*W, dim, inter, x, idx, w)
    acc = np.zeros(dim, np.float32)
    for e, rw in sorted(zip(idx, w)):
        acc = acc + O.expert_fp4(*[v[e] for v in W], dim, inter, x, float(rw))
    assert np.array_equal(y.view(np.uint32), acc.view(np.uint32))


# ---- dispatch ---------------------------------------------------------------
def test_dispatch_hand_example():
    # routes: 0->e3, 1->e1, 2->e3, 3->dropped, 4->e0, 5->e1
    idx = np.array([3, 1, 3, -1, 0, 1], np.int32)
    w = np.array([.1, .2, .3, .4, .5, .6], np.float32)
    d = O.dispatch(idx, w, 4, 6)
    assert list(d["count"]) == [1, 2, 0, 2]
    assert list(d["offset"]) == [0, 32, 64, 64]
    assert list(d["psum"]) == [1, 34, 64, 66]
    assert d["num_tiles"] == 3
    assert list(d["tile_expert"]) == [0, 1, 3, -1, -1, -1]
    assert list(d["route_pos"]) == [64, 32, 65, -1, 0, 33]
    o = d["order"]
    assert o[0] == 4 and o[32] == 1 and o[33] == 5 and o[64] == 0 and o[65] == 2
    assert np.all(o[1:32] == -1) and np.all(o[34:64] == -1) and np.all(o[66:96] == -1)
    assert d["layout_w"][65] == np.float32(.3) and d["layout_w"][1] == 0.0


def test_dispatch_invariants_zipf():
    rng = np.random.default_rng(24)
    E, M, k = 384, 132, 8
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    logits = rng.standard_normal((M, E)) + np.log(pop)[rng.permutation(E)]
    idx = np.argsort(-logits, axis=1)[:, :k].astype(np.int32)
    w = rng.random((M, k)).astype(np.float32)
    routes = M * k
    tiles = (routes + 31) // 32 + min(routes, E)
    d = O.dispatch(idx, w, E, tiles)
    cnt, off = d["count"], d["offset"]
    assert cnt.sum() == routes and np.array_equal(cnt, np.bincount(idx.ravel(), minlength=E))
    assert np.all(off % 32 == 0) and np.all(np.diff(off) >= 0)
    assert np.all(np.diff(off) == (cnt[:-1] + 31) // 32 * 32)
    rp, order = d["route_pos"], d["order"]
    assert np.array_equal(order[rp], np.arange(routes))
    flat = idx.ravel()
    for e in np.flatnonzero(cnt):
        seg = order[off[e]:off[e] + cnt[e]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)
    nt = d["num_tiles"]
    assert nt == ((cnt + 31) // 32).sum() <= tiles
    te = d["tile_expert"]
    assert np.all(te[nt:] == -1) and np.all(np.diff(te[:nt]) >= 0)


def test_threaded_oracle_is_bit_identical():
    """The timing baseline's threaded GEMV rows give the scalar loop's bits."""
    rng = np.random.default_rng(31)
    E, dim, inter, k = 8, 512, 256, 4
    w1, s1 = O.weight_quant_fp4((rng.standard_normal((E * inter, dim)) * 0.02).astype(np.float32))
    w3, s3 = O.weight_quant_fp4((rng.standard_normal((E * inter, dim)) * 0.02).astype(np.float32))
    w2, s2 = O.weight_quant_fp4((rng.standard_normal((E * dim, inter)) * 0.02).astype(np.float32))
    x = rng.standard_normal(dim).astype(np.float32)
    idx = np.array([5, 1, 7, 2], np.int32)
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    want = O.moe_routed(w1, s1, w3, s3, w2, s2, dim, inter, x, idx, w)
    try:
        O.set_threads(4)
        got = O.moe_routed(w1, s1, w3, s3, w2, s2, dim, inter, x, idx, w)
    finally:
        O.set_threads(1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_expert_hidden_composes_to_the_routed_expert():
    """or_expert_hidden_fp4 is the hidden state or_moe_routed feeds its down
    GEMV: the down projection of it equals a one-pick routed MoE bit for bit,
    and it equals silu(min(g, L)) * clamp(u, +-L) * rw of the two GEMVs to
    f32 rounding."""
    rng = np.random.default_rng(12)
    dim, inter = 256, 128
    w1, w3 = (rng.integers(0, 256, (inter, dim // 2), dtype=np.uint8) for _ in range(2))
    s1, s3 = (rng.integers(118, 124, (inter, dim // 32), dtype=np.uint8) for _ in range(2))
    w2 = rng.integers(0, 256, (dim, inter // 2), dtype=np.uint8)
    s2 = rng.integers(118, 124, (dim, inter // 32), dtype=np.uint8)
    x = rng.standard_normal(dim).astype(np.float32)
    h = O.expert_hidden_fp4(w1, s1, w3, s3, dim, inter, x, 0.7, 2.0)
    y = O.fp4_gemv(w2, s2, dim, inter, h)
    y1 = O.moe_routed(w1[None], s1[None], w3[None], s3[None], w2[None], s2[None], dim, inter, x,
                      np.array([0], np.int32), np.array([0.7], np.float32), 2.0)
    assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))
    g = O.fp4_gemv(w1, s1, inter, dim, x).astype(np.float64)
    u = O.fp4_gemv(w3, s3, inter, dim, x).astype(np.float64)
    g, u = np.minimum(g, 2.0), np.clip(u, -2.0, 2.0)
    ref = g / (1.0 + np.exp(-g)) * u * 0.7
    assert np.allclose(h, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
