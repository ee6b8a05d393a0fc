"""The allocation-free decode step (ws_moe_decode_route_noalloc, called
through the C ABI) gives ws_moe_decode_route's picks, weights and output bit
for bit, on two calls in a row, the second with a smaller problem (the
library's scratch keeps the first call's bytes), and rejects nothing that
ws_moe_decode_route accepts. Runs last: it shares the library's one scratch
array with nothing else."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, dev, host, rand_fp4_weights
from weightstream_amd import _lib
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def _case(seed, E, dim, inter):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    w1, s1 = rand_fp4_weights(gen, E * inter, dim)
    w3, s3 = rand_fp4_weights(gen, E * inter, dim)
    w2, s2 = rand_fp4_weights(gen, E * dim, inter)
    packed = (L.prepack_fp4_new(w1, s1, E * inter, dim) + L.prepack_fp4_new(w3, s3, E * inter, dim)
              + L.prepack_fp4_new(w2, s2, E * dim, inter))
    rng = np.random.default_rng(seed)
    logits = dev(rng.standard_normal(E).astype(np.float32))
    bias = dev((rng.standard_normal(E) * 0.1).astype(np.float32))
    x = dev(rng.standard_normal(dim).astype(np.float32))
    return packed, logits, bias, x


def _noalloc(packed, logits, bias, x, score, dim, inter, E, k):
    """Straight through the C ABI (no Python-side buffers but the outputs)."""
    lib = _lib.load()
    y = torch.full((dim,), -1.0, dtype=torch.float32, device=DEV)
    idx = torch.full((k,), -5, dtype=torch.int32, device=DEV)
    w = torch.zeros(k, dtype=torch.float32, device=DEV)
    p = lambda t: t.data_ptr()
    rc = lib.ws_moe_decode_route_noalloc(
        p(logits), p(bias), score, C.c_float(1.0), 1, C.c_float(1.0), p(x),
        *[p(t) for t in packed], p(y), p(idx), p(w), dim, inter, E, k, C.c_float(10.0),
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.load().ws_error_string(rc)
    return y, idx, w


def _with_workspace(packed, logits, bias, x, score, dim, inter, E, k):
    y = torch.empty(dim, dtype=torch.float32, device=DEV)
    idx = torch.empty(k, dtype=torch.int32, device=DEV)
    w = torch.empty(k, dtype=torch.float32, device=DEV)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    L.moe_decode_route(logits, bias, score, 1.0, 1, 1.0, x, *packed, y, idx, w, dim, inter, E, k,
                       ws)
    return y, idx, w


def test_noalloc_decode_matches_workspace_decode_twice():
    # second call smaller than the first; the third (dim > 8192) also stages
    # the quantised token in the scratch; the fourth runs softmax scores
    # (ws_moe_topk first, then the two expert kernels)
    for (seed, E, dim, inter, k, score) in [(31, 384, 4096, 2048, 8, 1), (32, 64, 1024, 512, 4, 1),
                                            (33, 16, 10240, 256, 6, 2), (34, 32, 1024, 256, 3, 0)]:
        announce("noalloc decode E=%d dim=%d inter=%d k=%d score=%d" % (E, dim, inter, k, score))
        case = _case(seed, E, dim, inter)
        got = _noalloc(*case, score, dim, inter, E, k)
        want = _with_workspace(*case, score, dim, inter, E, k)
        assert torch.equal(got[1], want[1])
        assert np.array_equal(host(got[2]).view(np.uint32), host(want[2]).view(np.uint32))
        assert np.array_equal(host(got[0]).view(np.uint32), host(want[0]).view(np.uint32))


def test_noalloc_rejects_shapes_outside_the_scratch():
    lib = _lib.load()
    f = torch.zeros(16, dtype=torch.float32, device=DEV)
    b = torch.zeros(16, dtype=torch.uint8, device=DEV)
    i = torch.zeros(16, dtype=torch.int32, device=DEV)
    # top_k * inter above 32768: rejected before any launch
    rc = lib.ws_moe_decode_route_noalloc(f.data_ptr(), f.data_ptr(), 1, C.c_float(1.0), 1,
                                         C.c_float(1.0), f.data_ptr(), *[b.data_ptr()] * 6,
                                         f.data_ptr(), i.data_ptr(), f.data_ptr(), 1024, 4096, 64,
                                         16, C.c_float(10.0), None)
    assert rc == 1002
