"""Experts loaded from a synthetic safetensors checkpoint (weightstream_amd.
ingest), relaid out by ws_prepack_fp4 and run through ws_moe_decode: the
output matches the C oracle on the raw on-disk bytes (max relative error
<= 1e-3, as the other MoE parity tests)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, announce, assert_close, dev, host
from test_ingest import _make_ckpt
from weightstream_amd import ingest as I
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    L.Hip.global_()


def test_checkpoint_experts_through_decode(tmp_path):
    E, dim, inter, k = 3, 256, 128, 2
    raw, _ = _make_ckpt(str(tmp_path), E, dim, inter, seed=5)
    ck = I.Checkpoint(str(tmp_path))
    slabs = I.load_expert_slabs(ck, "layers.0", E, dim, inter, device=DEV)
    packed = I.pack_expert_slabs(slabs, E, dim, inter)
    ck.close()
    rng = np.random.default_rng(9)
    x = rng.standard_normal(dim).astype(np.float32)
    idx = np.array([2, 0], np.int32)
    w = np.array([0.7, 0.3], np.float32)
    announce("ingest -> prepack -> moe_decode E=%d dim=%d inter=%d" % (E, dim, inter))
    y = torch.empty(dim, dtype=torch.float32, device=DEV)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    L.moe_decode(dev(x), dev(idx), dev(w), *packed, y, dim, inter, E, k, ws)
    H = [np.stack([raw["layers.0.ffn.experts.%d.%s" % (e, wn)][j] for e in range(E)])
         for wn in ("w1", "w3", "w2") for j in (0, 1)]
    want = O.moe_routed(*H, dim, inter, x, idx, w)
    assert_close(host(y), want, 1e-3, "ingest decode")
