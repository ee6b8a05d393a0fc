"""Checkpoint ingest (weightstream_amd.ingest): safetensors parsing, the
dtype-by-name rules of weightstream-ref store.rs:105-123, and slab assembly,
on a synthetic two-shard checkpoint written here. CPU only; the GPU test in
test_gpu_ingest.py runs the loaded experts through the decode kernels."""
import json
import os

import numpy as np
import pytest
import torch

from weightstream_amd import ingest as I


def _make_ckpt(tmp, E=3, dim=256, inter=128, n=64, k=256, seed=0):
    rng = np.random.default_rng(seed)
    t1, t2, raw = {}, {}, {}
    for e in range(E):
        for wn, (rows, cols) in (("w1", (inter, dim)), ("w3", (inter, dim)), ("w2", (dim, inter))):
            w = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
            s = rng.integers(118, 124, (rows, cols // 32), dtype=np.uint8)
            base = "layers.0.ffn.experts.%d.%s" % (e, wn)
            # experts in two shards, raw I8/U8 dtypes (convert.py style) in one
            tgt = t1 if e % 2 == 0 else t2
            tgt[base + ".weight"] = ("I8" if e % 2 == 0 else "F4_E2M1", (rows, cols // 2), w)
            tgt[base + ".scale"] = ("U8" if e % 2 == 0 else "F8_E8M0", (rows, cols // 32), s)
            raw[base] = (w, s)
    wq = rng.integers(0, 126, (n, k), dtype=np.uint8)
    ws = rng.integers(118, 124, ((n + 31) // 32, k // 32), dtype=np.uint8)
    t1["layers.0.attn.wo_b.weight"] = ("F8_E4M3", (n, k), wq)
    t1["layers.0.attn.wo_b.scale"] = ("F8_E8M0", ((n + 31) // 32, k // 32), ws)
    I.write_safetensors(os.path.join(tmp, "model-00001-of-00002.safetensors"), t1,
                        {"format": "pt"})
    I.write_safetensors(os.path.join(tmp, "model-00002-of-00002.safetensors"), t2)
    wm = {n_: "model-00001-of-00002.safetensors" for n_ in t1}
    wm.update({n_: "model-00002-of-00002.safetensors" for n_ in t2})
    with open(os.path.join(tmp, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    return raw, (wq, ws)


def test_tensor_kind_rules():
    assert I.tensor_kind("a.attn.wq_a.weight", "F8_E4M3") == "e4m3"
    assert I.tensor_kind("a.attn.wq_a.scale", "U8") == "e8m0"
    assert I.tensor_kind("a.ffn.experts.3.w1.weight", "I8") == "e2m1"
    assert I.tensor_kind("a.ffn.experts.3.w1.scale", "I8") == "e8m0"
    assert I.tensor_kind("a.ffn.shared_experts.w1.weight", "U8") == "u8"
    assert I.tensor_kind("embed.weight", "BF16") == "bf16"
    assert I.tensor_kind("x.weight", "F4_E2M1") == "e2m1"
    with pytest.raises(ValueError, match="unsupported dtype"):
        I.tensor_kind("x", "F64")


def test_checkpoint_roundtrip_and_slabs(tmp_path):
    E, dim, inter = 3, 256, 128
    raw, (wq, ws) = _make_ckpt(str(tmp_path), E, dim, inter)
    ck = I.Checkpoint(str(tmp_path))
    assert len(list(ck.names())) == E * 6 + 2
    m = ck.meta("layers.0.ffn.experts.0.w1.weight")
    assert m["kind"] == "e2m1" and m["shape"] == [inter, dim // 2]
    for base, (w, s) in raw.items():
        assert np.array_equal(ck.bytes(base + ".weight"), w.ravel())
        assert np.array_equal(ck.bytes(base + ".scale"), s.ravel())
    w, s = I.load_fp8_linear(ck, "layers.0.attn.wo_b", 64, 256, device="cpu")
    assert np.array_equal(w.numpy(), wq) and np.array_equal(s.numpy(), ws)
    slabs = I.load_expert_slabs(ck, "layers.0", E, dim, inter, device="cpu")
    for i, wn in enumerate(("w1", "w3", "w2")):
        ws_ = np.concatenate([raw["layers.0.ffn.experts.%d.%s" % (e, wn)][0] for e in range(E)])
        ss_ = np.concatenate([raw["layers.0.ffn.experts.%d.%s" % (e, wn)][1] for e in range(E)])
        assert np.array_equal(slabs[2 * i].numpy(), ws_)
        assert np.array_equal(slabs[2 * i + 1].numpy(), ss_)
    with pytest.raises(ValueError, match="expected"):
        I.load_fp8_linear(ck, "layers.0.attn.wo_b", 64, 128, device="cpu")  # wrong size
    with pytest.raises(KeyError):
        ck.bytes("layers.9.missing.weight")
    ck.close()


def test_single_file_checkpoint(tmp_path):
    data = np.arange(64, dtype=np.uint8)
    I.write_safetensors(str(tmp_path / "model.safetensors"),
                        {"l.attn.wkv.weight": ("F8_E4M3", (2, 32), data)})
    ck = I.Checkpoint(str(tmp_path))
    assert np.array_equal(ck.bytes("l.attn.wkv.weight"), data)
    ck.close()


def test_rejects_bad_header(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
    with pytest.raises(ValueError, match="header length"):
        I.Shard(str(p))


def test_read_config_merges_text_config(tmp_path):
    """config.rs:109-130: a nested text_config wins; model_type, architectures
    and quantization_config survive from the top level unless redeclared."""
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                          "config_1017_moe.json")
    with open(golden) as f:
        c = json.load(f)
    c["quantization_config"] = {"fmt": "e4m3"}
    c["text_config"]["model_type"] = "inner"
    with open(tmp_path / "config.json", "w") as f:
        json.dump(c, f)
    cfg = I.read_config(str(tmp_path))
    assert cfg["hidden_size"] == 5120 and cfg["moe_intermediate_size"] == 2304
    assert cfg["num_experts_per_tok"] == 6 and cfg["scoring_func"] == "sqrtsoftplus"
    assert cfg["model_type"] == "inner"                       # redeclared inside
    assert cfg["architectures"] == ["DeepseekV41ForCausalLM"]   # from the top level
    assert cfg["quantization_config"] == {"fmt": "e4m3"}
    del c["text_config"]["hidden_size"]
    with open(tmp_path / "config.json", "w") as f:
        json.dump(c, f)
    with pytest.raises(ValueError, match="hidden_size"):
        I.read_config(str(tmp_path))


def test_load_moe_layer_assembles_gate_shared_and_w13(tmp_path):
    E, dim, inter, si = 2, 64, 64, 64
    rng = np.random.default_rng(3)
    t = {}
    for e in range(E):
        for wn, (rows, cols) in (("w1", (inter, dim)), ("w3", (inter, dim)), ("w2", (dim, inter))):
            base = "l.ffn.experts.%d.%s" % (e, wn)
            t[base + ".weight"] = ("U8", (rows, cols // 2),
                                   rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8))
            t[base + ".scale"] = ("U8", (rows, cols // 32),
                                  rng.integers(118, 124, (rows, cols // 32), dtype=np.uint8))
    sh = {}
    for wn, (rows, cols) in (("w1", (si, dim)), ("w3", (si, dim)), ("w2", (dim, si))):
        w = rng.integers(0, 126, (rows, cols), dtype=np.uint8)
        s = rng.integers(118, 124, (rows // 32, cols // 32), dtype=np.uint8)
        t["l.ffn.shared_experts.%s.weight" % wn] = ("F8_E4M3", w.shape, w)
        t["l.ffn.shared_experts.%s.scale" % wn] = ("F8_E8M0", s.shape, s)
        sh[wn] = (w, s)
    gw = rng.integers(0, 1 << 16, (E, dim), dtype=np.uint16)
    gb = rng.standard_normal(E).astype(np.float32)
    t["l.ffn.gate.weight"] = ("BF16", (E, dim), gw.view(np.uint8))
    t["l.ffn.gate.bias"] = ("F32", (E,), gb.view(np.uint8))
    I.write_safetensors(str(tmp_path / "model.safetensors"), t)
    ck = I.Checkpoint(str(tmp_path))
    lay = I.load_moe_layer(ck, "l", E, dim, inter, si, device="cpu")
    assert np.array_equal(lay["gate_w"].numpy().view(np.uint16), gw)
    assert np.array_equal(lay["gate_bias"].numpy(), gb)
    w13, s13 = lay["shared_w13"]
    # engine.rs:962-964: w1's rows then w3's, scales likewise
    assert np.array_equal(w13.numpy(), np.concatenate([sh["w1"][0], sh["w3"][0]]))
    assert np.array_equal(s13.numpy(), np.concatenate([sh["w1"][1], sh["w3"][1]]))
    for wn in ("w1", "w2", "w3"):
        assert np.array_equal(lay["shared"][wn][0].numpy(), sh[wn][0])
    assert len(lay["experts"]) == 6
    with pytest.raises(ValueError, match="n % 32"):
        I.load_fp8_combined_rows(ck, "l.ffn.shared_experts.w1", "l.ffn.shared_experts.w3", 48,
                                 dim, device="cpu")
    ck.close()
