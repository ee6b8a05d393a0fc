"""Pin the oracle's GEMV/GEMM restatements (weightstream-ref/src/actquant.rs:
110-173) and the f32-scale generalisation.

Checks: the reference's own "GEMV == dense dequant" tests (actquant.rs:
225-270), an f64 brute-force dot bounded by the f32 summation error bound
(catches a dropped scale, a transposed operand or a wrong nibble order), and
the quantised-activation entry (or_gemm_q) against the f32-input GEMV.
"""
import numpy as np

import oracle_lib as O


def _f32_sum_bound(abs_terms_sum, n):
    # |fl(sum) - sum| <= (n-1) u sum|terms| (+ product rounding), u = 2^-24
    return 1.2 * n * 2.0 ** -24 * abs_terms_sum + 1e-30


# ---- actquant.rs:225-252 -------------------------------------------------
def test_fp8_gemv_matches_dense_dequant():
    rows = cols = 32
    w = np.array([(i % 200) for i in range(rows * cols)], np.uint8)
    w[w == 0x7F] = 0x7E
    s = np.full(1, 127, np.uint8)
    x = np.array([((i * 0.01) - 0.15) * 448.0 / 200.0 for i in range(cols)], np.float32)
    y = O.fp8_gemv(w, s, rows, cols, x)
    qa = O.fp8_snap(x)
    table = O.e4m3_decode_table()
    for n in range(rows):
        want = np.float32(0)
        for c in range(cols):
            want = np.float32(want + qa[c] * table[w[n * cols + c]])
        assert abs(y[n] - want) < 1e-4


# ---- actquant.rs:254-270 -------------------------------------------------
def test_fp4_gemv_matches_dense_dequant():
    rows, cols = 4, 64
    w = np.array([i % 251 for i in range(rows * cols // 2)], np.uint8)
    s = np.full(rows * 2, 127, np.uint8)
    x = np.array([(i * 0.02 - 0.6) * 6.0 / 4.0 for i in range(cols)], np.float32)
    y = O.fp4_gemv(w, s, rows, cols, x)
    qa = O.fp8_snap(x)
    dense = O.dequant_fp4_packed(w, s, rows, cols)
    for n in range(rows):
        assert abs(y[n] - O.dot(dense[n], qa)) < 1e-4


def _rand_case(rng, rows, cols, fp4):
    wf = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    x[rng.integers(0, cols, cols // 100 + 1)] *= 20
    if fp4:
        q, s = O.weight_quant_fp4(wf)
        dense = O.dequant_fp4_packed(q, s, rows, cols)
    else:
        q, s = O.weight_quant_fp8(wf)
        dense = O.dequant_fp8_blockwise(q, s, rows, cols)
    return wf, q, s, dense, x


def test_gemv_f64_bruteforce_bound():
    rng = np.random.default_rng(11)
    for fp4 in (False, True):
        rows, cols = 96, 512
        wf, q, s, dense, x = _rand_case(rng, rows, cols, fp4)
        y = (O.fp4_gemv if fp4 else O.fp8_gemv)(q, s, rows, cols, x)
        qa = O.fp8_snap(x).astype(np.float64)
        exact = dense.astype(np.float64) @ qa
        bound = _f32_sum_bound(np.abs(dense.astype(np.float64)) @ np.abs(qa), cols)
        assert np.all(np.abs(y - exact) <= bound)
        # and the quantised weights are close to the f32 weights they encode
        assert np.abs(dense - wf).max() <= np.abs(wf).max() * (0.26 if fp4 else 0.07)


def test_gemm_q_equals_gemv_rows():
    rng = np.random.default_rng(12)
    M, N, K = 5, 64, 256
    for fp4 in (False, True):
        xs = rng.standard_normal((M, K)).astype(np.float32)
        _, q, s, _, _ = _rand_case(rng, N, K, fp4)
        aq, as_ = O.fp8_act_emit(xs)
        y = O.gemm_q(aq, as_, M, q, s, N, K, fp4)
        for m in range(M):
            want = (O.fp4_gemv if fp4 else O.fp8_gemv)(q, s, N, K, xs[m])
            assert np.array_equal(y[m].view(np.uint32), want.view(np.uint32))


def test_f32s_gemm_bruteforce_and_pow2_reduction():
    rng = np.random.default_rng(13)
    M, N, K, B = 3, 256, 512, 128
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wq, ws = O.weight_quant_fp8_f32s(wf, B)
    aq, as_ = O.act_quant_f32s(x, B)
    y = O.gemm_f32s(aq, as_, wq, ws, B)
    t = O.e4m3_decode_table().astype(np.float64)
    da = t[aq] * np.repeat(as_.astype(np.float64), B, axis=1)
    dw = t[wq] * np.repeat(np.repeat(ws.astype(np.float64), B, axis=0)[:N], B, axis=1)
    exact = da @ dw.T
    bound = _f32_sum_bound(np.abs(da) @ np.abs(dw).T, K) * 4
    assert np.all(np.abs(y - exact) <= bound)
    # quantisation error of the scheme itself: e4m3 keeps 3 mantissa bits
    assert np.abs(da - x).max() <= np.abs(x).max() / 16 * 1.01

    # with power-of-two scales the f32-scale GEMM equals the UE8M0 path
    # regrouped: pick B=32, scales 2^e, and compare to or_gemm_q
    B = 32
    aq2, as2 = O.fp8_act_emit(x)
    wq2, ws2 = O.weight_quant_fp8(wf)
    as2f = np.ldexp(np.float32(1), as2.astype(np.int32) - 127).astype(np.float32)
    ws2f = np.ldexp(np.float32(1), ws2.astype(np.int32) - 127).astype(np.float32)
    y2 = O.gemm_f32s(aq2, as2f, wq2, ws2f, B)
    y3 = O.gemm_q(aq2, as2, M, wq2, ws2, N, K, False)
    assert np.array_equal(y2.view(np.uint32), y3.view(np.uint32))


def test_weight_quant_fp8_uses_full_block_amax():
    """A single large value in row 0 sets the scale of the whole 32x32 block
    (store.rs's test encoder used the last row's amax instead)."""
    w = np.full((32, 32), 0.01, np.float32)
    w[0, 0] = 100.0
    q, s = O.weight_quant_fp8(w)
    assert s[0, 0] == O.log2_ceil(100.0 / 448.0) + 127
    dec = O.dequant_fp8_blockwise(q, s, 32, 32)
    assert dec[0, 0] == 96.0
