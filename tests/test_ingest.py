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
