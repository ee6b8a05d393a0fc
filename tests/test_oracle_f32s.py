"""Pin the oracle's f32-scale quantisers (or_act_quant_f32s,
or_weight_quant_fp8_f32s), the scale scheme of BASELINE configs 1-2.

The reference has no f32-scale path; the scheme generalises the block rule of
weightstream-ref actquant.rs:21-45 (per-block amax floored at 1e-4, scale
from amax/448, each element divided by the scale and e4m3-encoded) with an
f32 scale instead of a UE8M0 power of two. Nothing here restates the C code:
the checker recomputes every block's amax in numpy over the block it must
cover, forms the scale and the division in numpy f32, and encodes with
torch's e4m3fn cast (round to nearest even), with the reference encoder's
subnormal carry (quant.rs:120-122, pinned in test_oracle_quant.py) patched in.
A UE8M0-rounded scale, a multiply by the reciprocal, the last row's amax
(store.rs:372-383) and a ragged block that ignores its partial rows are each
shown to fail the checker.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O


def _e4m3_ref(v):
    """Independent encoder: torch's RNE e4m3fn cast plus the reference's
    carry quirk (inputs in [15/1024, 2^-6) encode as sign | 0x38)."""
    v = np.asarray(v, np.float32)
    out = torch.from_numpy(v.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
    a = np.abs(v)
    carry = (a >= np.float32(15.0 / 1024)) & (a < np.float32(2.0 ** -6))
    out[carry] = np.where(np.signbit(v[carry]), 0xB8, 0x38)
    return out


def _scale(amax):
    amax = np.maximum(np.float32(amax), np.float32(1e-4))
    return np.float32(amax) / np.float32(448.0)


def _check_blocks(x, q, s, rb, cb):
    """x [R, K] f32, blocks of rb rows x cb columns (ragged last row block).
    Returns None when (q, s) follow the scheme, else a description."""
    R, K = x.shape
    nrb = (R + rb - 1) // rb
    if s.shape != (nrb, K // cb):
        return f"scale shape {s.shape}"
    for i in range(nrb):
        r0, r1 = i * rb, min(R, (i + 1) * rb)
        for j in range(K // cb):
            blk = x[r0:r1, j * cb:(j + 1) * cb]
            sc = _scale(np.abs(blk).max())
            if s[i, j].view(np.uint32) != sc.view(np.uint32):
                return f"scale ({i},{j}) {s[i, j]!r} != {sc!r}"
            v = np.clip(blk / sc, np.float32(-448.0), np.float32(448.0)).astype(np.float32)
            want = _e4m3_ref(v)
            if not np.array_equal(q[r0:r1, j * cb:(j + 1) * cb], want):
                return f"bytes of block ({i},{j})"
    return None


def _plant_midpoints(rng, blk):
    """Make blk's amax 7.0422525 and plant values x for which x / s lands on
    an e4m3 rounding midpoint while x * (1 / s) does not (or the reverse)."""
    f = np.float32
    amax = f(7.0422525)
    blk[:] = np.clip(blk, -f(6), f(6))
    blk[0] = amax
    sc = amax / f(448)
    enc = lambda v: _e4m3_ref(np.array([v], f))[0]
    k = 1
    while k < 9:
        e, m = rng.integers(2, 8), rng.integers(0, 8)
        x = f(f((1 + (2 * m + 1) / 16) * 2.0 ** e) * sc)
        for xx in (x, np.nextafter(x, f(np.inf)), np.nextafter(x, f(-np.inf))):
            if abs(xx) < amax and enc(xx / sc) != enc(xx * (f(1) / sc)):
                blk[k] = xx if k % 2 else -xx
                k += 1
                break


def _act_case(rng, M=5, K=512):
    x = rng.standard_normal((M, K)).astype(np.float32)
    _plant_midpoints(rng, x[0, 0:128])
    # 1% outliers x20
    mask = rng.random((M, K)) < 0.01
    x[mask] *= 20
    x[1, 128:256] = 0.0                     # all-zero block: amax floor
    x[2, 256:384] *= np.float32(1e-6)       # below the floor
    if M > 3 and K >= 512:
        x[3, 384:512] *= np.float32(1e3)    # large-magnitude block
    if M > 4:
        x[4, 0:128] = np.float32(2.0 ** -9) * rng.standard_normal(128).astype(np.float32)
    return x


def test_act_quant_f32s_follows_scheme():
    rng = np.random.default_rng(31)
    x = _act_case(rng)
    q, s = O.act_quant_f32s(x, 128)
    assert _check_blocks(x, q.reshape(x.shape), s.reshape(x.shape[0], -1), 1, 128) is None


@pytest.mark.parametrize("N", [256, 300])
def test_weight_quant_fp8_f32s_follows_scheme(N):
    """128x128 blocks; N = 300 leaves a ragged last row block of 44 rows.
    Block (0,0) has its amax in row 0, block (0,1) in row 127, block (1,2)
    in the block's last row: a last-row or first-row amax rule fails."""
    rng = np.random.default_rng(N)
    K = 384
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, 5] = 3.0
    w[127, 200] = -2.5
    w[min(N, 256) - 1, 300] = 1.75
    if N > 256:
        w[N - 1, 10] = 4.0                  # amax in the ragged block's last row
    q, s = O.weight_quant_fp8_f32s(w, 128)
    q = q.reshape(N, K)
    s = s.reshape(-1, K // 128)
    assert _check_blocks(w, q, s, 128, 128) is None
    # the outliers decode back to themselves within e4m3 precision
    t = O.e4m3_decode_table()
    assert abs(t[q[0, 5]] * s[0, 0] - 3.0) <= 3.0 / 16
    assert t[q[0, 5]] == 448.0 and t[q[127, 200]] == -448.0


def test_checker_rejects_plausible_variants():
    """The slips a rewrite could make each fail the checker on this data."""
    rng = np.random.default_rng(7)
    x = _act_case(rng, M=4, K=384)
    M, K = x.shape

    def quant(scale_fn, divide=True):
        q = np.zeros_like(x, np.uint8)
        s = np.zeros((M, K // 128), np.float32)
        for m in range(M):
            for j in range(K // 128):
                blk = x[m, j * 128:(j + 1) * 128]
                sc = scale_fn(np.abs(blk).max())
                s[m, j] = sc
                v = blk / sc if divide else blk * (np.float32(1) / sc)
                q[m, j * 128:(j + 1) * 128] = _e4m3_ref(np.clip(v, -448, 448).astype(np.float32))
        return q, s

    good_q, good_s = quant(_scale)
    assert _check_blocks(x, good_q, good_s, 1, 128) is None
    # UE8M0-rounded scale 2^ceil(log2(amax/448)): the other rule of this codebase
    ue = lambda a: np.float32(2.0) ** np.float32(np.ceil(np.log2(max(a, 1e-4) / 448.0)))
    assert _check_blocks(x, *quant(ue), 1, 128) is not None
    # multiply by the reciprocal instead of dividing: scales equal, bytes differ
    assert _check_blocks(x, *quant(_scale, divide=False), 1, 128) is not None
    # no amax floor
    nofloor = lambda a: np.float32(a) / np.float32(448.0) if a > 0 else np.float32(1e-30)
    assert _check_blocks(x, *quant(nofloor), 1, 128) is not None

    # weight-side slips: the last row's amax, and a ragged block quantised
    # with the amax of its full-size neighbour
    N = 300
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, 5] = 3.0
    w[N - 1, 10] = 4.0
    q, s = O.weight_quant_fp8_f32s(w, 128)
    q = q.reshape(N, K)
    s = s.reshape(-1, K // 128)
    s_last = s.copy()
    s_last[0, 0] = _scale(np.abs(w[127, 0:128]).max())
    assert _check_blocks(w, q, s_last, 128, 128) is not None
    s_rag = s.copy()
    s_rag[2, 0] = _scale(np.abs(w[256:300, 0:128][:-1]).max())
    assert _check_blocks(w, q, s_rag, 128, 128) is not None


def test_f32s_reduces_to_ue8m0_rule_on_pow2_amax():
    """When amax/448 is an exact power of two the f32 scale equals the UE8M0
    scale of the reference rule (actquant.rs:36-44, block 32), so the bytes of
    the two quantisers coincide block by block."""
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (4, 128)).astype(np.float32)
    for m, e in enumerate([-3, 0, 2, 5]):
        x[m] *= np.float32(448.0 * 2.0 ** e) / np.abs(x[m]).max()
        x[m, 17::32] = np.float32(448.0 * 2.0 ** e)   # every 32-block's amax
    q, s = O.act_quant_f32s(x, 32)
    aq, as_ = O.fp8_act_emit(x)
    assert np.array_equal(q.reshape(aq.shape), aq)
    sf = np.ldexp(np.float32(1), as_.astype(np.int32) - 127).astype(np.float32)
    assert np.array_equal(s.reshape(sf.shape), sf)
