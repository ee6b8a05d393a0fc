"""Experts loaded from a synthetic safetensors checkpoint (weightstream_amd.
ingest), relaid out by ws_prepack_fp4 and run through ws_moe_decode: the
output matches the C oracle on the raw on-disk bytes (max relative error
<= 1e-3, as the other MoE parity tests)."""
import json
import os
import shutil

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DEV, announce, assert_close, dev, host, rel_err_stats
from test_gpu_prefill import _check_by_stages, _staged_hidden
from test_ingest import _make_ckpt
from weightstream_amd import ingest as I
from weightstream_amd import launch as L

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


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


def _ds41f_checkpoint(tmp, E, dim, inter, sinter, seed=41):
    """A two-shard checkpoint of one DS4.1F MoE layer with the reference's
    tensor names and dtypes (engine.rs:1346-1530): routed experts as raw
    I8/U8 (even experts) or F4_E2M1/F8_E8M0 (odd), the shared expert's FP8
    w1/w2/w3 (F8_E4M3 + F8_E8M0), the bf16 gate and the f32 gate bias. The
    experts draw random bytes (every e2m1 code), the FP8 weights random
    finite e4m3 codes. Returns the raw on-disk arrays."""
    rng = np.random.default_rng(seed)
    shards = ({}, {})
    raw = {}
    p = "layers.3"
    for e in range(E):
        for wn, (rows, cols) in (("w1", (inter, dim)), ("w3", (inter, dim)), ("w2", (dim, inter))):
            w = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
            s = rng.integers(118, 124, (rows, cols // 32), dtype=np.uint8)
            base = "%s.ffn.experts.%d.%s" % (p, e, wn)
            shards[e % 2][base + ".weight"] = ("I8" if e % 2 == 0 else "F4_E2M1", w.shape, w)
            shards[e % 2][base + ".scale"] = ("U8" if e % 2 == 0 else "F8_E8M0", s.shape, s)
            raw[(e, wn)] = (w, s)
    for wn, (rows, cols) in (("w1", (sinter, dim)), ("w3", (sinter, dim)), ("w2", (dim, sinter))):
        w = rng.integers(0, 0x7F, (rows, cols), dtype=np.uint8) | \
            (rng.integers(0, 2, (rows, cols), dtype=np.uint8) << 7)   # no NaN codes
        s = rng.integers(119, 124, (rows // 32, cols // 32), dtype=np.uint8)
        base = "%s.ffn.shared_experts.%s" % (p, wn)
        shards[0][base + ".weight"] = ("F8_E4M3", w.shape, w)
        shards[0][base + ".scale"] = ("F8_E8M0", s.shape, s)
        raw[("shared", wn)] = (w, s)
    gw = (rng.standard_normal((E, dim)) * 0.02).astype(np.float32)
    bits = gw.view(np.uint32)
    gb16 = ((bits + (((bits >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)  # RNE, quant.rs:95
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    shards[1][p + ".ffn.gate.weight"] = ("BF16", (E, dim), gb16.view(np.uint8))
    shards[1][p + ".ffn.gate.bias"] = ("F32", (E,), bias.view(np.uint8))
    raw["gate"] = ((gb16.astype(np.uint32) << 16).view(np.float32), bias)
    names = ("model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors")
    wm = {}
    for fname, t in zip(names, shards):
        I.write_safetensors(os.path.join(tmp, fname), t, {"format": "pt"})
        wm.update({n: fname for n in t})
    with open(os.path.join(tmp, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    shutil.copy(os.path.join(GOLDEN, "config_1017_moe.json"), os.path.join(tmp, "config.json"))
    return p, raw


def test_ds41f_layer_checkpoint_through_decode_prefill_and_shared(tmp_path):
    """One MoE layer at the DS4.1F size (dim 5120, moe_intermediate_size 2304,
    top-6 sqrtsoftplus with routed_scaling_factor 1.5, from the reference's
    testdata/config-1017.json) but 24 of its 384 experts, on disk as the
    engine reads it (sharded index, the reference's names and dtypes):
    ingest -> ws_prepack_fp4 -> gate logits (bf16) -> ws_moe_decode_route
    for one token and ws_moe_topk + ws_moe_prefill for 16, and the shared
    expert through the fused w13; routing bit for bit and outputs within
    1e-3 of the oracle on the raw on-disk bytes."""
    E = 24
    tmp = str(tmp_path)
    announce("DS4.1F layer checkpoint: writing %d experts" % E)
    with open(os.path.join(GOLDEN, "config_1017_moe.json")) as f:
        c = json.load(f)["text_config"]
    dim, inter, k = c["hidden_size"], c["moe_intermediate_size"], c["num_experts_per_tok"]
    sinter = inter * c["n_shared_experts"]
    prefix, raw = _ds41f_checkpoint(tmp, E, dim, inter, sinter)
    cfg = I.read_config(tmp)
    assert (cfg["hidden_size"], cfg["moe_intermediate_size"], cfg["num_experts_per_tok"]) == \
        (dim, inter, k)
    assert cfg["scoring_func"] == "sqrtsoftplus" and cfg["model_type"] == "deepseek_v41"
    sf = {"sigmoid": O.SCORE_SIGMOID, "softmax": O.SCORE_SOFTMAX,
          "sqrtsoftplus": O.SCORE_SQRTSOFTPLUS}[cfg["scoring_func"]]
    rscale, limit = float(cfg["routed_scaling_factor"]), float(cfg["swiglu_limit"])

    ck = I.Checkpoint(tmp)
    layer = I.load_moe_layer(ck, prefix, E, dim, inter, sinter, device=DEV)
    ck.close()
    P = I.pack_expert_slabs(layer["experts"], E, dim, inter)
    H = [np.stack([raw[(e, wn)][j] for e in range(E)]) for wn in ("w1", "w3", "w2")
         for j in (0, 1)]
    gate_f32, bias = raw["gate"]

    # decode: one token
    rng = np.random.default_rng(43)
    x = rng.standard_normal(dim).astype(np.float32)
    announce("DS4.1F layer: gate logits + moe_decode_route")
    lg = torch.empty((1, E), dtype=torch.float32, device=DEV)
    L.moe_gate_logits(dev(x[None]), layer["gate_w"], lg, 1, dim, E)
    y = torch.empty(dim, dtype=torch.float32, device=DEV)
    idx = torch.empty(k, dtype=torch.int32, device=DEV)
    w = torch.empty(k, dtype=torch.float32, device=DEV)
    ws = torch.empty(L.moe_decode_workspace_size(dim, inter, k), dtype=torch.uint8, device=DEV)
    L.moe_decode_route(lg[0], layer["gate_bias"], sf, 1.0, int(cfg["norm_topk_prob"]), rscale,
                       dev(x), *P, y, idx, w, dim, inter, E, k, ws, swiglu_limit=limit)
    want_lg = O.gemv_f32(gate_f32, x)
    assert np.array_equal(host(lg)[0].view(np.uint32), want_lg.view(np.uint32))
    ri, rw = O.route(O.score(want_lg, sf), bias, k, True, rscale)
    assert np.array_equal(host(idx), ri)
    assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert_close(host(y), O.moe_routed(*H, dim, inter, x, ri, rw, limit), 1e-3,
                 "DS4.1F checkpoint decode")

    # prefill: 16 tokens
    m = 16
    xs = rng.standard_normal((m, dim)).astype(np.float32)
    announce("DS4.1F layer: gate logits + moe_topk + moe_prefill m=%d" % m)
    lgm = torch.empty((m, E), dtype=torch.float32, device=DEV)
    L.moe_gate_logits(dev(xs), layer["gate_w"], lgm, m, dim, E)
    im = torch.empty((m, k), dtype=torch.int32, device=DEV)
    wm = torch.empty((m, k), dtype=torch.float32, device=DEV)
    L.moe_topk(lgm, layer["gate_bias"], None, im, wm, m, E, k, sf, 1.0,
               bool(cfg["norm_topk_prob"]), rscale)
    ym = torch.empty((m, dim), dtype=torch.float32, device=DEV)
    pws = torch.empty(L.moe_prefill_workspace_size(m, dim, inter, k, E), dtype=torch.uint8,
                      device=DEV)
    L.moe_prefill(dev(xs), im, wm, *P, ym, m, dim, inter, E, k, pws, swiglu_limit=limit)
    glg, gi, gw, gy = host(lgm), host(im), host(wm), host(ym)
    O.set_threads(16)
    try:
        for r in range(m):
            wl = O.gemv_f32(gate_f32, xs[r])
            assert np.array_equal(glg[r].view(np.uint32), wl.view(np.uint32))
            ri, rw = O.route(O.score(wl, sf), bias, k, True, rscale)
            assert np.array_equal(gi[r], ri) and np.array_equal(gw[r].view(np.uint32),
                                                                rw.view(np.uint32))
            want = O.moe_routed(*H, dim, inter, xs[r], ri, rw, limit)
            if rel_err_stats(gy[r], want)[0] <= 1e-3:
                assert_close(gy[r], want, 1e-3, "DS4.1F checkpoint prefill row %d" % r)
            else:
                staged = _staged_hidden(xs, im, wm, P, m, E, dim, inter, k)
                _check_by_stages(gy[r], xs[r], gi[r], gw[r], H, staged, r, k, dim, inter)
    finally:
        O.set_threads(1)

    # the shared expert through the fused w13 (engine.rs:1520, :4067)
    announce("DS4.1F layer: shared expert w13 m=%d" % m)
    ys = torch.empty((m, dim), dtype=torch.float32, device=DEV)
    sws = torch.empty(L.shared_expert_workspace_size(m, dim, sinter), dtype=torch.uint8,
                      device=DEV)
    L.shared_expert_fp8_w13(dev(xs), *layer["shared_w13"], *layer["shared"]["w2"], ys, m, dim,
                            sinter, sws, swiglu_limit=limit)
    sh = [raw[("shared", wn)][j] for wn in ("w1", "w3", "w2") for j in (0, 1)]
    gys = host(ys)
    for r in (0, 7, 15):
        assert_close(gys[r], O.shared_fp8(*sh, dim, sinter, xs[r], limit), 1e-3,
                     "DS4.1F checkpoint shared row %d" % r)
