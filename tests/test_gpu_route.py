"""GPU parity of MoE routing (weightstream-ref moe.rs:20-69): device expf and
logf, gate logits, scores, top-k selection and weights are bit-exact with the
C oracle for sigmoid, softmax and sqrtsoftplus, ties and near-ties at the
top-k cut included."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, announce, dev, host
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def test_device_expf_equals_glibc_on_every_input():
    """All 2^32 inputs: the device digest equals glibc's, and 2^24 inputs
    spread over the whole range are compared value by value. The probe also
    evaluates the lane-table variant used by the routing kernels and marks
    any input where the two differ."""
    lib = L._lib.load()
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int32, device=DEV)
    total = 0
    for c in range(16):
        lo = c * chunk
        announce("expf probe chunk %d" % c)
        L._lib.check("ws_expf_probe", lib.ws_expf_probe(lo, chunk, out.data_ptr(),
                                                         torch.cuda.current_stream().cuda_stream))
        # the lane-table variant (routing kernels) agrees with ws_expf
        assert int((out == 0x7FBADBAD).sum().item()) == 0
        r = out.to(torch.int64) & 0xFFFFFFFF
        # canonical NaN, as the host digest does
        nan = ((r & 0x7F800000) == 0x7F800000) & ((r & 0x7FFFFF) != 0)
        r = torch.where(nan, torch.full_like(r, 0x7FC00000), r)
        u = torch.arange(lo, lo + chunk, dtype=torch.int64, device=DEV)
        mixed = (r ^ ((u * 0x9E3779B1) & 0xFFFFFFFF)) * (2 * u + 1)
        total = (total + int(mixed.sum().item())) & ((1 << 64) - 1)
    want = O.expfcheck().glibc_expf_digest(0, 1 << 32)
    assert total == want
    # direct comparison on a strided sample
    lo, n = 0x3C000000, 1 << 24
    L._lib.check("ws_expf_probe", lib.ws_expf_probe(lo, n, out.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream))
    got = host(out[:n]).view(np.uint32)
    ref = np.empty(n, np.uint32)
    O.expfcheck().glibc_expf_bits(lo, n, ref.ctypes.data)
    nan = (got & 0x7F800000 == 0x7F800000) & (got & 0x7FFFFF != 0)
    got = np.where(nan, np.uint32(0x7FC00000), got)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("m,dim,E", [(3, 4096, 384), (1, 4096, 384), (40, 1024, 100), (1, 1000, 64), (5, 768, 50),
                                     (17, 256, 33), (6, 5120, 384), (8, 4096, 384), (9, 4096, 384),
                                     (2, 512, 7)])
def test_gate_logits_bit_exact(bf16, m, dim, E):
    """dim % 256 == 0: up to 8 tokens the producer/consumer kernel (4 experts
    per workgroup), more tokens the pipelined kernel (8 x 8 blocks of experts
    x tokens), partial blocks at the edges; otherwise the per-lane kernel.
    (6, 5120, 384): the DS4.1F gate for a verify batch."""
    rng = np.random.default_rng(200 + bf16 + m + dim)
    x = rng.standard_normal((m, dim)).astype(np.float32)
    w = (rng.standard_normal((E, dim)) * 0.02).astype(np.float32)
    if bf16:
        bits = w.view(np.uint32)  # finite values: RNE to bf16 (quant.rs:95-101)
        wb = ((bits + (((bits >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)
        assert wb[0, 0] == O.f32_to_bf16(float(w[0, 0]))
        w = (wb.astype(np.uint32) << 16).view(np.float32)
        dw = dev(wb.view(np.int16))
    else:
        dw = dev(w)
    announce("gate_logits bf16=%d m=%d dim=%d E=%d" % (bf16, m, dim, E))
    logits = torch.empty((m, E), dtype=torch.float32, device=DEV)
    L.moe_gate_logits(dev(x), dw, logits, m, dim, E)
    got = host(logits)
    for r in range(m):
        want = O.gemv_f32(w, x[r])
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32))


def _rows_with_ties(rng, m, E, score_func):
    logits = rng.standard_normal((m, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    # exact ties of score+bias between experts (9, 5) and (3, 17) on row 0
    s0 = O.score(logits[0], score_func)
    bias[5] = np.float32(s0[9] + bias[9] - s0[5])
    logits[1, 40] = logits[1, 41]                  # equal logits, equal scores
    bias[40] = bias[41]
    if E > 71:
        # row 2: four exact ties at the very top, on different lanes (10, 20)
        # and on one lane (7, 71 = 7 + 64): picked by ascending index
        logits[2, [7, 10, 20, 71]] = 6.0
        bias[[7, 10, 20, 71]] = 0.25
    return logits, bias


@pytest.mark.parametrize("score_func", [O.SCORE_SIGMOID, O.SCORE_SOFTMAX, O.SCORE_SQRTSOFTPLUS])
@pytest.mark.parametrize("E,k", [(384, 8), (256, 6), (64, 1), (1000, 16)])
def test_topk_bit_exact(score_func, E, k):
    rng = np.random.default_rng(300 + E + k + score_func)
    m = 48
    logits, bias = _rows_with_ties(rng, m, E, score_func)
    temp, rscale = (1.0, 1.0) if k != 6 else (1.7, 2.5)
    announce("moe_topk E=%d k=%d f=%d" % (E, k, score_func))
    idx = torch.empty((m, k), dtype=torch.int32, device=DEV)
    w = torch.empty((m, k), dtype=torch.float32, device=DEV)
    sc = torch.empty((m, E), dtype=torch.float32, device=DEV)
    L.moe_topk(dev(logits), dev(bias), sc, idx, w, m, E, k, score_func, temp, True, rscale)
    gi, gw, gs = host(idx), host(w), host(sc)
    if E > 71 and score_func == O.SCORE_SIGMOID:
        assert list(gi[2][:4]) == [7, 10, 20, 71][:k]
    for r in range(m):
        s = O.score(logits[r], score_func, temp)
        assert np.array_equal(gs[r].view(np.uint32), s.view(np.uint32))
        ri, rw = O.route(s, bias, k, True, rscale)
        assert np.array_equal(gi[r], ri), (r, gi[r], ri)
        assert np.array_equal(gw[r].view(np.uint32), rw.view(np.uint32))


def _near_tied_rows(rng, m, E, k, score_func):
    """Rows whose top-k cut falls between score+bias values 0 and 1 ulp apart
    (and 2 ulp, and ties across several experts), set through the bias from
    the oracle's scores so that the tie is exact in f32."""
    logits = rng.standard_normal((m, E)).astype(np.float32)
    bias = np.zeros((m, E), np.float32)
    for r in range(m):
        s = O.score(logits[r], score_func)
        order = np.argsort(-s, kind="stable")
        a, b = order[k - 1], order[k]           # last pick, first non-pick
        target = np.float32(s[a])
        gap = r % 4                              # 0: tie, 1-2: ulps apart, 3: b above
        want = target
        for _ in range(gap if gap < 3 else 1):
            want = np.nextafter(want, np.float32(-np.inf) if gap < 3 else np.float32(np.inf))
        bb = np.float32(want - s[b])
        # adjust so that s[b] + bb lands exactly on want in f32
        for _ in range(8):
            got = np.float32(s[b] + bb)
            if got == want:
                break
            bb = np.nextafter(bb, np.float32(np.inf) if got < want else np.float32(-np.inf))
        bias[r, b] = bb
    return logits, bias


@pytest.mark.parametrize("score_func", [O.SCORE_SQRTSOFTPLUS, O.SCORE_SIGMOID])
@pytest.mark.parametrize("E,k", [(384, 6), (384, 8), (1000, 16)])
def test_topk_near_ties_at_the_cut_bit_exact(score_func, E, k):
    """ws_moe_topk picks and weights equal the oracle's bit for bit when the
    k-th and (k+1)-th score+bias are tied or 1-2 ulp apart (the bias is per
    row here, so each row runs as its own one-token call)."""
    rng = np.random.default_rng(400 + E + k + score_func)
    m = 16
    logits, bias = _near_tied_rows(rng, m, E, k, score_func)
    announce("moe_topk near ties E=%d k=%d f=%d" % (E, k, score_func))
    for r in range(m):
        idx = torch.empty(k, dtype=torch.int32, device=DEV)
        w = torch.empty(k, dtype=torch.float32, device=DEV)
        sc = torch.empty(E, dtype=torch.float32, device=DEV)
        L.moe_topk(dev(logits[r]), dev(bias[r]), sc, idx, w, 1, E, k, score_func, 1.0, True, 1.5)
        s = O.score(logits[r], score_func)
        assert np.array_equal(host(sc).view(np.uint32), s.view(np.uint32))
        ri, rw = O.route(s, bias[r], k, True, 1.5)
        assert np.array_equal(host(idx), ri), (r, host(idx), ri)
        assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))


def test_device_logf_and_sqrtsoftplus_equal_glibc_on_every_input():
    """All 2^32 inputs: the digests of the device ws_logf and of the
    sqrtsoftplus score (score_fn and the routing kernels' wave variant) equal
    the host glibc digests; 2^24 inputs are also compared value by value."""
    lib = L._lib.load()
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for fn in (0, 1):
        total = 0
        for c in range(16):
            lo = c * chunk
            announce("math probe fn %d chunk %d" % (fn, c))
            L._lib.check("ws_math_probe", lib.ws_math_probe(fn, lo, chunk, out.data_ptr(), stream))
            assert int((out == 0x7FBADBAD).sum().item()) == 0
            r = out.to(torch.int64) & 0xFFFFFFFF
            nan = ((r & 0x7F800000) == 0x7F800000) & ((r & 0x7FFFFF) != 0)
            r = torch.where(nan, torch.full_like(r, 0x7FC00000), r)
            u = torch.arange(lo, lo + chunk, dtype=torch.int64, device=DEV)
            mixed = (r ^ ((u * 0x9E3779B1) & 0xFFFFFFFF)) * (2 * u + 1)
            total = (total + int(mixed.sum().item())) & ((1 << 64) - 1)
        assert total == O.expfcheck().glibc_math_digest(fn, 0, 1 << 32), fn
        lo, n = 0x3E000000 if fn == 0 else 0xC0000000, 1 << 24
        L._lib.check("ws_math_probe", lib.ws_math_probe(fn, lo, n, out.data_ptr(), stream))
        got = host(out[:n]).view(np.uint32)
        ref = np.empty(n, np.uint32)
        O.expfcheck().glibc_math_bits(fn, lo, n, ref.ctypes.data)
        nan = (got & 0x7F800000 == 0x7F800000) & (got & 0x7FFFFF != 0)
        got = np.where(nan, np.uint32(0x7FC00000), got)
        assert np.array_equal(got, ref), fn


def test_reference_gate_select_route_contract():
    """moe_gate (bf16, sqrtsoftplus scores), moe_select (always-normalised
    top-k of given scores) and the fused moe_route agree with each other and
    with the oracle's selection on the same scores."""
    rng = np.random.default_rng(500)
    dim, E, k = 512, 96, 6
    x = rng.standard_normal(dim).astype(np.float32)
    wf = (rng.standard_normal((E, dim)) * 0.05).astype(np.float32)
    wb = np.array([O.f32_to_bf16(float(v)) for v in wf.ravel()], np.uint16).reshape(E, dim)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    dx, dwb, db = dev(x), dev(wb.view(np.int16)), dev(bias)
    announce("moe_gate/moe_select/moe_route")
    scores = torch.empty(E, dtype=torch.float32, device=DEV)
    L.moe_gate(dx, dwb, db, scores, dim, E)
    w1 = torch.empty(k, dtype=torch.float32, device=DEV)
    i1 = torch.empty(k, dtype=torch.int32, device=DEV)
    L.moe_select(scores, db, w1, i1, E, k, 1.5)
    w2 = torch.empty(k, dtype=torch.float32, device=DEV)
    i2 = torch.empty(k, dtype=torch.int32, device=DEV)
    L.moe_route(dx, dwb, db, w2, i2, dim, E, k, 1.5)
    s = host(scores)
    ri, rw = O.route(s, bias, k, True, 1.5)
    assert np.array_equal(host(i1), ri) and np.array_equal(host(i2), ri)
    assert np.array_equal(host(w1).view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(host(w2).view(np.uint32), rw.view(np.uint32))
    wdense = (wb.astype(np.uint32) << 16).view(np.float32)
    ref_s = O.score(O.gemv_f32(wdense, x), O.SCORE_SQRTSOFTPLUS)
    assert np.array_equal(s.view(np.uint32), ref_s.view(np.uint32))


def test_swiglu_bit_exact():
    rng = np.random.default_rng(600)
    n = 4096
    g = (rng.standard_normal(n) * 8).astype(np.float32)
    u = (rng.standard_normal(n) * 8).astype(np.float32)
    announce("swiglu")
    out = torch.empty(n, dtype=torch.float32, device=DEV)
    L.swiglu(dev(g), dev(u), out, n, 0.37)
    got = host(out)
    gc = np.minimum(g, np.float32(10))
    uc = np.clip(u, np.float32(-10), np.float32(10))
    want = np.array([np.float32(np.float32(O.silu(float(a)) * b) * np.float32(0.37))
                     for a, b in zip(gc, uc)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_device_e4m3_and_activation_scale_equal_oracle_on_every_input():
    """All 2^32 inputs: the digests of the device e4m3 encoder (f32_to_e4m3,
    branch-free), of the activation quantisation's scale byte for a block
    maximum |x| (the exponent taken from the bits of amax, no division) and of
    the e4m3 rounding without the byte (e4m3_round_value) equal the oracle's
    (quant.rs:103-137, actquant.rs:21-45); 2^24 inputs around the subnormal /
    normal boundary are also compared value by value."""
    lib = L._lib.load()
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for fn in (2, 3, 4):
        total = 0
        for c in range(16):
            lo = c * chunk
            announce("quant probe fn %d chunk %d" % (fn, c))
            L._lib.check("ws_math_probe", lib.ws_math_probe(fn, lo, chunk, out.data_ptr(), stream))
            r = out.to(torch.int64) & 0xFFFFFFFF
            if fn == 4:  # canonical NaN, as the oracle's bytes
                nan = ((r & 0x7F800000) == 0x7F800000) & ((r & 0x7FFFFF) != 0)
                r = torch.where(nan, torch.full_like(r, 0x7FC00000), r)
            u = torch.arange(lo, lo + chunk, dtype=torch.int64, device=DEV)
            mixed = (r ^ ((u * 0x9E3779B1) & 0xFFFFFFFF)) * (2 * u + 1)
            total = (total + int(mixed.sum().item())) & ((1 << 64) - 1)
        assert total == O.lib.or_probe_digest(fn, 0, 1 << 32), fn
        lo, n = 0x3C000000, 1 << 24
        L._lib.check("ws_math_probe", lib.ws_math_probe(fn, lo, n, out.data_ptr(), stream))
        got = host(out[:n]).view(np.uint32).copy()
        if fn == 4:
            got[((got & 0x7F800000) == 0x7F800000) & ((got & 0x7FFFFF) != 0)] = 0x7FC00000
        ref = np.empty(n, np.uint32)
        O.lib.or_probe_bytes(fn, lo, n, ref.ctypes.data)
        assert np.array_equal(got, ref), fn
