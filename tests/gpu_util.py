"""Helpers of the GPU parity tests: device tensors, seeded synthetic data,
and the error statistics reported next to every tolerance check."""
import sys

import numpy as np
import torch

DEV = "cuda:0"


def announce(msg):
    """Name the case before a GPU step, so a fault report says what ran."""
    print("[gpu-case] " + msg, flush=True)
    sys.stdout.flush()


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err_stats(got, want):
    """|got - want| / max(|want|, 1e-2 * max|want|): relative error with a
    floor at 1% of the output's scale so that outputs near zero do not turn
    absolute noise into huge ratios. Returns (max, p50, p99)."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    floor = 1e-2 * max(np.abs(want).max(), 1e-30)
    r = np.abs(got - want) / np.maximum(np.abs(want), floor)
    return float(r.max()), float(np.median(r)), float(np.quantile(r, 0.99))


def raw_rel_err_stats(got, want):
    """|got - want| / |want| with no floor, over the outputs with want != 0:
    the unfloored distribution (max, p50, p99, p99.9), reported beside the
    floored one. Outputs that cancel to near zero dominate its maximum."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    nz = want != 0
    if not nz.any():
        return 0.0, 0.0, 0.0, 0.0
    r = np.abs(got[nz] - want[nz]) / np.abs(want[nz])
    return (float(r.max()), float(np.median(r)), float(np.quantile(r, 0.99)),
            float(np.quantile(r, 0.999)))


def assert_close(got, want, tol, what):
    mx, p50, p99 = rel_err_stats(got, want)
    rmx, rp50, rp99, rp999 = raw_rel_err_stats(got, want)
    print("[%s] rel err max %.3g p50 %.3g p99 %.3g (tol %.1g, floor 1%% of max|want|); "
          "unfloored max %.3g p50 %.3g p99 %.3g p99.9 %.3g"
          % (what, mx, p50, p99, tol, rmx, rp50, rp99, rp999), flush=True)
    assert mx <= tol, "%s: max rel err %.3g > %.1g" % (what, mx, tol)


def rand_fp4_weights(gen, rows, cols, scale_lo=118, scale_hi=123):
    """Random packed e2m1 bytes + UE8M0 scales on the device."""
    w = torch.randint(0, 256, (rows, cols // 2), dtype=torch.uint8, device=DEV, generator=gen)
    s = torch.randint(scale_lo, scale_hi, (rows, cols // 32), dtype=torch.uint8, device=DEV,
                      generator=gen)
    return w, s


def activations(rng, m, k, outliers=True):
    """N(0,1) with 1% of entries x20."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        idx = rng.random((m, k)) < 0.01
        x[idx] *= 20.0
    return x
