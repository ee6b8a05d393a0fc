"""GPU parity: activation/weight quantisation and the block-scaled GEMMs,
called through the C ABI (weightstream_amd.launch) and checked against the
C oracle on the same seeded inputs.

Tolerances: quantisation is integer/byte work and must be bit-exact. GEMM
outputs are f32 sums of exact fp8 x fp8 (or fp8 x fp4) products; the MFMA
accumulation order differs from the oracle's sequential per-32-block order,
so outputs are compared with max relative error <= 1e-3 (floor at 1% of the
output scale, see gpu_util.rel_err_stats); observed errors are ~1e-6.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, activations, announce, assert_close, dev, host
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


@pytest.fixture(params=["single_pass", "split_k"])
def gemm_path(request):
    """Run a GEMM test with no split-K workspace (single-pass kernels) and
    with one (M > 64, and M <= 16 when the column strips leave CUs idle,
    split K across workgroups)."""
    ws = None
    if request.param == "split_k":
        ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
        L.set_gemm_workspace(ws)
    yield request.param
    if ws is not None:
        torch.cuda.synchronize()
        L.set_gemm_workspace(None)


def _wide_range_acts(rng, n):
    x = rng.standard_normal(n).astype(np.float32)
    x *= np.repeat(10.0 ** rng.uniform(-7, 4, n // 32), 32).astype(np.float32)
    x[:32] = 0.0                                   # zero block -> amax floor
    x[32:64] = np.float32(15.2 / 1024) * np.sign(rng.standard_normal(32))  # carry quirk
    x[32] = 448.0                                  # scale 1: the rest sit in [15/1024, 2^-6)
    x[70] = np.float32(np.nan)
    x[100] = np.float32(1e30)
    return x


def test_emit8_and_snap8_bit_exact():
    rng = np.random.default_rng(100)
    n = 32 * 4096
    x = _wide_range_acts(rng, n)
    q_ref, s_ref = O.fp8_act_emit(x)
    announce("emit8 n=%d" % n)
    dx = dev(x)
    q = torch.empty(n, dtype=torch.uint8, device=DEV)
    s = torch.empty(n // 32, dtype=torch.uint8, device=DEV)
    L.emit8(dx, q, s, n)
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(host(s), s_ref)
    announce("snap8 n=%d" % n)
    L.snap8(dx, n)
    got = host(dx)
    want = O.fp8_snap(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_emit8_packed_and_pack_scales():
    rng = np.random.default_rng(101)
    n = 32 * 100
    x = rng.standard_normal(n).astype(np.float32)
    q_ref, s_ref = O.fp8_act_emit(x)
    raw = n // 32
    off = (raw + 15) // 16 * 16
    announce("emit8_packed n=%d" % n)
    q = torch.empty(n, dtype=torch.uint8, device=DEV)
    s = torch.zeros(off + raw, dtype=torch.uint8, device=DEV)
    L.emit8_packed(dev(x), q, s, n)
    sh = host(s)
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(sh[:raw], s_ref) and np.array_equal(sh[off:off + raw], s_ref)
    n2 = 128 * 7
    src = rng.integers(0, 256, n2 // 32).astype(np.uint8)
    dst = torch.empty(n2 // 128, dtype=torch.int32, device=DEV)
    L.pack_scales(dev(src), dst, n2)
    assert np.array_equal(host(dst).view(np.uint32), src.view("<u4"))


def test_weight_quant_bit_exact():
    rng = np.random.default_rng(102)
    rows, cols = 200, 512
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[3, 5] = 7.0
    w[40:72, 64:96] = 0.0
    announce("weight_quant fp4/fp8 %dx%d" % (rows, cols))
    q4 = torch.empty((rows, cols // 2), dtype=torch.uint8, device=DEV)
    s4 = torch.empty((rows, cols // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp4(dev(w), q4, s4, rows, cols)
    q4r, s4r = O.weight_quant_fp4(w)
    assert np.array_equal(host(q4), q4r) and np.array_equal(host(s4), s4r)
    q8 = torch.empty((rows, cols), dtype=torch.uint8, device=DEV)
    s8 = torch.empty(((rows + 31) // 32, cols // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(dev(w), q8, s8, rows, cols)
    q8r, s8r = O.weight_quant_fp8(w)
    assert np.array_equal(host(q8), q8r) and np.array_equal(host(s8), s8r)


def _quantised_case(rng, m, n, k, fp4):
    x = activations(rng, m, k)
    aq, as_ = O.fp8_act_emit(x)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq, ws = O.weight_quant_fp4(wf) if fp4 else O.weight_quant_fp8(wf)
    return aq, as_, wq, ws


GEMM_SHAPES = [(1, 4096, 4096), (1, 1024, 2048), (4, 256, 512), (16, 512, 1024),
               (17, 96, 384), (64, 256, 1024), (128, 512, 4096), (130, 48, 256),
               (300, 160, 640), (65, 1024, 4096)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_fp8_gemm_matches_oracle(m, n, k, gemm_path):
    rng = np.random.default_rng(1000 + m + n + k)
    aq, as_, wq, ws = _quantised_case(rng, m, n, k, False)
    want = O.gemm_q(aq, as_, m, wq, ws, n, k, False)
    announce("fp8_gemm %s m=%d n=%d k=%d" % (gemm_path, m, n, k))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(dev(aq), dev(as_), dev(wq), dev(ws), out, m, n, k)
    assert_close(host(out), want, GEMM_TOL, "fp8_gemm %dx%dx%d" % (m, n, k))
    announce("fp8_gemm_bf16 m=%d n=%d k=%d" % (m, n, k))
    ob = torch.empty((m, n), dtype=torch.int16, device=DEV)
    L.fp8_gemm_bf16(dev(aq), dev(as_), dev(wq), dev(ws), ob, m, n, k)
    got = (host(ob).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    # bf16 keeps 8 significant bits: RNE error <= 2^-8 relative; and the
    # output equals the oracle's f32 rounded to bf16 except where the two f32
    # values straddle a rounding boundary
    assert_close(got, want, 2.0 ** -8 + GEMM_TOL, "fp8_gemm_bf16 %dx%dx%d" % (m, n, k))
    want_b = np.array([O.f32_to_bf16(float(v)) for v in want.ravel()], np.uint16)
    same = np.mean(host(ob).astype(np.uint16).ravel() == want_b)
    assert same >= 0.999, same


@pytest.mark.parametrize("m", [1, 8, 64])
def test_fp8_gemm_out_projection_shape_matches_oracle(m, gemm_path):
    """The config-5 attention out-projection shape, N=4096, K=8192, at the
    block's M in {1, 8, 64}: f32 and bf16 outputs against the oracle's
    dequantise-then-f32 GEMM (or_gemm_q) on sampled rows."""
    n, k = 4096, 8192
    rng = np.random.default_rng(1500 + m)
    aq, as_, wq, ws = _quantised_case(rng, m, n, k, False)
    rows = sorted({0, m // 2, m - 1})
    want = O.gemm_q(np.ascontiguousarray(aq[rows]), np.ascontiguousarray(as_[rows]), len(rows),
                    wq, ws, n, k, False)
    announce("fp8_gemm out-projection %s m=%d" % (gemm_path, m))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(dev(aq), dev(as_), dev(wq), dev(ws), out, m, n, k)
    assert_close(host(out)[rows], want, GEMM_TOL, "fp8_gemm %dx%dx%d" % (m, n, k))
    ob = torch.empty((m, n), dtype=torch.int16, device=DEV)
    L.fp8_gemm_bf16(dev(aq), dev(as_), dev(wq), dev(ws), ob, m, n, k)
    got = (host(ob).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    assert_close(got[rows], want, 2.0 ** -8 + GEMM_TOL, "fp8_gemm_bf16 %dx%dx%d" % (m, n, k))


@pytest.mark.parametrize("m,n,k", [(1, 2048, 4096), (8, 512, 1024), (128, 256, 2048),
                                   (33, 80, 512), (200, 192, 1024), (130, 8192, 256)])
def test_fp4_gemm_matches_oracle(m, n, k, gemm_path):
    rng = np.random.default_rng(2000 + m + n + k)
    aq, as_, wq, ws = _quantised_case(rng, m, n, k, True)
    want = O.gemm_q(aq, as_, m, wq, ws, n, k, True)
    announce("fp4_gemm %s m=%d n=%d k=%d" % (gemm_path, m, n, k))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp4_gemm(dev(aq), dev(as_), dev(wq), dev(ws), out, m, n, k)
    assert_close(host(out), want, GEMM_TOL, "fp4_gemm %dx%dx%d" % (m, n, k))


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (128, 384, 4096), (20, 256, 512),
                                   (5, 64, 1152), (257, 320, 1280), (128, 8192, 512)])  # K/128 = 9: the general kernel
def test_fp8_gemm_f32s_matches_oracle(m, n, k, gemm_path):
    rng = np.random.default_rng(3000 + m + n + k)
    x = activations(rng, m, k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq, ws = O.weight_quant_fp8_f32s(wf, 128)
    aq_ref, as_ref = O.act_quant_f32s(x, 128)
    want = O.gemm_f32s(aq_ref, as_ref, wq, ws, 128)
    announce("act_quant_f32s + fp8_gemm_f32s m=%d n=%d k=%d" % (m, n, k))
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 128), dtype=torch.float32, device=DEV)
    L.act_quant_f32s(dev(x), aq, as_, m, k)
    assert np.array_equal(host(aq), aq_ref)
    assert np.array_equal(host(as_).view(np.uint32), as_ref.view(np.uint32))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm_f32s(aq, as_, dev(wq), dev(ws), out, m, n, k)
    assert_close(host(out), want, GEMM_TOL, "fp8_gemm_f32s %dx%dx%d" % (m, n, k))


@pytest.mark.parametrize("n", [4096, 12288, 2048])
def test_config2_fp8_gemm_f32s_full_size_matches_oracle(n, gemm_path):
    """BASELINE config 2 in its own scale scheme at full size: M=128, K=4096,
    N in {4096, 12288, 2048}; weights N(0, 0.02) quantised with 128x128 f32
    scales amax/448 (or_weight_quant_fp8_f32s), activations N(0, 1) with 1%
    outliers x20 quantised per 1x128 on the device (bit-exact with the
    oracle); f32 and bf16 outputs against the oracle's sequential
    dequantise-then-f32-accumulate GEMM (or_gemm_f32s) on every row. Runs
    with and without the split-K workspace (the line kernel takes all three
    N: 128 x 48 tiles at N = 12288, 64 x 32 at N = 4096, 32 x 32 at
    N = 2048; the split-K pipeline is covered by the model shapes below)."""
    m, k = 128, 4096
    rng = np.random.default_rng(3100 + n)
    x = activations(rng, m, k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq, ws = O.weight_quant_fp8_f32s(wf, 128)
    del wf
    aq_ref, as_ref = O.act_quant_f32s(x, 128)
    O.set_threads(16)
    try:
        want = O.gemm_f32s(aq_ref, as_ref, wq, ws, 128)
    finally:
        O.set_threads(1)
    announce("config 2 act_quant_f32s + fp8_gemm_f32s %s m=%d n=%d k=%d" % (gemm_path, m, n, k))
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 128), dtype=torch.float32, device=DEV)
    L.act_quant_f32s(dev(x), aq, as_, m, k)
    assert np.array_equal(host(aq), aq_ref)
    assert np.array_equal(host(as_).view(np.uint32), as_ref.view(np.uint32))
    dwq, dws = dev(wq), dev(ws)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm_f32s(aq, as_, dwq, dws, out, m, n, k)
    assert_close(host(out), want, GEMM_TOL, "config 2 f32s %dx%dx%d f32 out" % (m, n, k))
    ob = torch.empty((m, n), dtype=torch.int16, device=DEV)
    L.fp8_gemm_f32s(aq, as_, dwq, dws, ob, m, n, k, out_bf16=True)
    bits = host(ob).astype(np.uint16)
    got = (bits.astype(np.uint32) << 16).view(np.float32)
    assert_close(got, want, 2.0 ** -8 + GEMM_TOL, "config 2 f32s %dx%dx%d bf16 out" % (m, n, k))
    # bf16 out is the f32 result rounded to nearest even (quant.rs:95-101):
    # equal to the oracle's f32 rounded to bf16 except at rounding boundaries
    wb = want.view(np.uint32)
    want_b = ((wb + (((wb >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)
    same = np.mean(bits == want_b)
    print("[config 2 bf16 n=%d] %.5f of outputs equal bf16(oracle)" % (n, same), flush=True)
    assert same >= 0.999, same


@pytest.mark.parametrize("n", [4096, 12288, 2048])
def test_fp8_gemm_full_size_vs_fp64_dequant(n, gemm_path):
    """BASELINE config 2 shapes (M=128, K=4096) against an f64 matmul of the
    dequantised operands on the device (too large for the scalar oracle)."""
    m, k = 128, 4096
    gen = torch.Generator(device=DEV)
    gen.manual_seed(n)
    announce("fp8_gemm full %s m=%d n=%d k=%d" % (gemm_path, m, n, k))
    x = torch.randn((m, k), device=DEV, generator=gen)
    x = torch.where(torch.rand((m, k), device=DEV, generator=gen) < 0.01, x * 20, x)
    w = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    L.emit8(x, aq, as_, m * k)
    wq = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    ws = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(w, wq, ws, n, k)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(aq, as_, wq, ws, out, m, n, k)
    table = torch.from_numpy(O.e4m3_decode_table().astype(np.float64)).to(DEV)
    pw = lambda s: torch.pow(2.0, s.to(torch.float64) - 127)
    da = table[aq.long()] * pw(as_).repeat_interleave(32, 1)
    dw = table[wq.long()] * pw(ws).repeat_interleave(32, 0).repeat_interleave(32, 1)
    want = (da @ dw.T).cpu().numpy()
    assert_close(host(out), want, GEMM_TOL, "fp8_gemm full %dx%dx%d" % (m, n, k))


# The engine's FP8 projection shapes (N, K) (weightstream-gpu engine.rs:3388-3398:
# q_a, q_b, wkv, wo_b, shared w1/w3, fused w13, shared w2, engram wkv, drafter).
MODEL_SHAPES = [(1280, 5120), (8192, 1280), (512, 5120), (5120, 2048), (2304, 5120),
                (4608, 5120), (5120, 2304), (25600, 5120), (1280, 15360)]


@pytest.mark.parametrize("n,k", MODEL_SHAPES)
@pytest.mark.parametrize("m", [1, 6, 128])
def test_fp8_gemm_model_shapes_vs_fp64_dequant(m, n, k, gemm_path):
    """The real projection shapes through the dispatch (every kernel family
    and the fallbacks for K/128 not a multiple of 4), against an f64 matmul of
    the dequantised operands on the device."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(m * 7 + n + k)
    announce("fp8_gemm model shape %s m=%d n=%d k=%d" % (gemm_path, m, n, k))
    x = torch.randn((m, k), device=DEV, generator=gen)
    w = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    L.emit8(x, aq, as_, m * k)
    wq = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    ws = torch.empty(((n + 31) // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(w, wq, ws, n, k)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(aq, as_, wq, ws, out, m, n, k)
    table = torch.from_numpy(O.e4m3_decode_table().astype(np.float64)).to(DEV)
    pw = lambda s: torch.pow(2.0, s.to(torch.float64) - 127)
    da = table[aq.long()] * pw(as_).repeat_interleave(32, 1)
    dw = table[wq.long()] * pw(ws).repeat_interleave(32, 0)[:n].repeat_interleave(32, 1)
    want = (da @ dw.T).cpu().numpy()
    assert_close(host(out), want, GEMM_TOL, "fp8_gemm %dx%dx%d" % (m, n, k))


def test_gemm_rejects_bad_shapes():
    a = torch.zeros(256, dtype=torch.uint8, device=DEV)
    out = torch.zeros(256, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        L.fp8_gemm(a, a, a, a, out, 1, 16, 100)     # K % 128 != 0
    with pytest.raises(RuntimeError, match="unsupported shape"):
        L.fp8_gemm(a, a, a, a, out, 1, 10, 128)     # N % 16 != 0


def test_split_k_is_deterministic_and_reusable():
    """Split-K tickets reset themselves: repeated calls (and a different shape
    in between) give bit-identical results."""
    rng = np.random.default_rng(4000)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    L.set_gemm_workspace(ws)
    try:
        outs = []
        for m, n, k in [(128, 512, 4096), (40, 192, 2048), (128, 512, 4096), (128, 512, 4096)]:
            aq, as_, wq, ws_ = _quantised_case(np.random.default_rng(4000 + m + n), m, n, k, False)
            announce("split-k repeat m=%d n=%d k=%d" % (m, n, k))
            out = torch.empty((m, n), dtype=torch.float32, device=DEV)
            L.fp8_gemm(dev(aq), dev(as_), dev(wq), dev(ws_), out, m, n, k)
            outs.append(host(out))
        assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
        assert np.array_equal(outs[0].view(np.uint32), outs[3].view(np.uint32))
    finally:
        torch.cuda.synchronize()
        L.set_gemm_workspace(None)
    del rng


@pytest.mark.parametrize("m,n,k", [(1, 1280, 15360), (6, 512, 12288)])
def test_long_k_strip_split_matches_single_pass(m, n, k):
    """M <= 16 with few column strips and K > 8192 splits K over workgroups
    when a workspace is set: the same sums up to f32 reassociation (within
    the GEMM tolerance of the single-pass result), and repeated calls give
    the same bits."""
    aq, as_, wq, ws_ = _quantised_case(np.random.default_rng(4100 + m + n), m, n, k, False)
    announce("strip split m=%d n=%d k=%d" % (m, n, k))
    args = [dev(aq), dev(as_), dev(wq), dev(ws_)]
    single = torch.empty((m, n), dtype=torch.float32, device=DEV)
    L.fp8_gemm(*args, single, m, n, k)
    ws = torch.empty(max(L.gemm_workspace_size(m, n, k), 256), dtype=torch.uint8, device=DEV)
    L.set_gemm_workspace(ws)
    try:
        outs = []
        for _ in range(2):
            out = torch.empty((m, n), dtype=torch.float32, device=DEV)
            L.fp8_gemm(*args, out, m, n, k)
            outs.append(host(out))
    finally:
        torch.cuda.synchronize()
        L.set_gemm_workspace(None)
    assert L.gemm_workspace_size(m, n, k) > 0
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert_close(outs[0], host(single), GEMM_TOL, "strip split m=%d n=%d k=%d" % (m, n, k))


def test_workspace_registered_under_one_mode_serves_both():
    """set_gemm_workspace registers with both library builds: a NATIVE-mode
    GEMM on a stream whose workspace was set while EXACT was active takes the
    split-K path (it writes partials into the workspace) and gives the bits
    of the same NATIVE GEMM registered under NATIVE."""
    m, n, k = 128, 8192, 2304     # the split-K pipeline's shape (K not a multiple of 512)
    gen = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn((m, k), device=DEV, generator=gen)
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    asc = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    L.emit8(x, aq, asc, m * k)
    wf = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    w = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    sw = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(wf, w, sw, n, k)
    ws = torch.full((L.gemm_workspace_size(m, n, k),), 0xAB, dtype=torch.uint8, device=DEV)
    outs = []
    try:
        for reg_mode in (L.MATH_EXACT, L.MATH_NATIVE):
            L.set_math_mode(reg_mode)
            L.set_gemm_workspace(ws)
            ws.fill_(0xAB)
            L.set_math_mode(L.MATH_NATIVE)
            announce("native fp8_gemm after a workspace set in mode %d" % reg_mode)
            out = torch.empty((m, n), dtype=torch.float32, device=DEV)
            L.fp8_gemm(aq, asc, w, sw, out, m, n, k)
            torch.cuda.synchronize()
            assert (ws != 0xAB).any(), "the split-K path did not run"
            outs.append(out)
            L.set_gemm_workspace(None)
    finally:
        L.set_math_mode(L.MATH_EXACT)
        torch.cuda.synchronize()
        L.set_gemm_workspace(None)
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))


@pytest.mark.parametrize("m,n,k", [(100, 4096, 4096), (65, 3072, 2048), (128, 5120, 1024),
                                   (127, 3104, 4096), (100, 2048, 4096), (40, 4096, 2048),
                                   (120, 12288, 4096), (128, 9216, 768),
                                   # K > 4096, N > 4096 or few tiles
                                   (64, 4096, 8192), (96, 5120, 5120), (24, 2048, 4096),
                                   (64, 12288, 4096), (128, 1280, 8192)])
@pytest.mark.parametrize("native", [False, True])
def test_line_gemm_ragged_rows_vs_fp64_dequant(m, n, k, native):
    """The line kernel (K a multiple of 512): 64 x 32 tiles for M in 65-128
    with 192-384 workgroups, 32 x 32 tiles for 32-row blocks (n = 2048 at
    M = 100; M = 40), 128 x 48 tiles for wide N (12288; 9216 at K = 768,
    three 256-K stages); ragged last row blocks, the XCD-paired tile order and
    (n = 3104: 194 workgroups) the plain order; the other shapes it stages
    (K > 4096, N > 4096, few tiles: 32 x 32 tiles when they fit one round of
    workgroups, else 64 x 32; at most 32 rows, 32 x 32 with 64 or more
    tiles), UE8M0 and f32 scales, f32
    and bf16 outputs, against an f64 matmul of the dequantised operands.
    EXACT within 1e-3; NATIVE within its own 5e-2 (tests/test_gpu_native.py)."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(m + n + k)
    tol = 5e-2 if native else GEMM_TOL
    announce("line gemm m=%d n=%d k=%d native=%d" % (m, n, k, native))
    x = torch.randn((m, k), device=DEV, generator=gen)
    x = torch.where(torch.rand((m, k), device=DEV, generator=gen) < 0.01, x * 20, x)
    w = torch.randn((n, k), device=DEV, generator=gen) * 0.02
    aq = torch.empty((m, k), dtype=torch.uint8, device=DEV)
    as_ = torch.empty((m, k // 32), dtype=torch.uint8, device=DEV)
    L.emit8(x, aq, as_, m * k)
    wq = torch.empty((n, k), dtype=torch.uint8, device=DEV)
    ws = torch.empty((n // 32, k // 32), dtype=torch.uint8, device=DEV)
    L.weight_quant_fp8(w, wq, ws, n, k)
    table = torch.from_numpy(O.e4m3_decode_table().astype(np.float64)).to(DEV)
    pw = lambda s: torch.pow(2.0, s.to(torch.float64) - 127)
    da = table[aq.long()] * pw(as_).repeat_interleave(32, 1)
    dw = table[wq.long()] * pw(ws).repeat_interleave(32, 0).repeat_interleave(32, 1)
    want = (da @ dw.T).cpu().numpy()
    # f32 scales: the same codes with per-block f32 scales (128 x 128 / 1 x 128)
    af = torch.rand((m, k // 128), device=DEV, generator=gen) * 0.01 + 1e-3
    wf = torch.rand((n // 128 + (n % 128 > 0), k // 128), device=DEV, generator=gen) * 1e-4 + 1e-5
    daf = table[aq.long()] * af.double().repeat_interleave(128, 1)
    dwf = table[wq.long()] * wf.double().repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)
    want_f = (daf @ dwf.T).cpu().numpy()
    prev = L.set_math_mode(L.MATH_NATIVE if native else L.MATH_EXACT)
    try:
        out = torch.empty((m, n), dtype=torch.float32, device=DEV)
        L.fp8_gemm(aq, as_, wq, ws, out, m, n, k)
        assert_close(host(out), want, tol, "line gemm %dx%dx%d" % (m, n, k))
        ob = torch.empty((m, n), dtype=torch.int16, device=DEV)
        L.fp8_gemm_bf16(aq, as_, wq, ws, ob, m, n, k)
        got = (host(ob).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
        assert_close(got, want, 2.0 ** -8 + tol, "line gemm bf16 %dx%dx%d" % (m, n, k))
        outf = torch.empty((m, n), dtype=torch.float32, device=DEV)
        L.fp8_gemm_f32s(aq, af, wq, wf, outf, m, n, k)
        assert_close(host(outf), want_f, tol, "line gemm f32s %dx%dx%d" % (m, n, k))
    finally:
        L.set_math_mode(prev)
