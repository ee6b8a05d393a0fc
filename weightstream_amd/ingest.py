"""On-disk checkpoint ingest for the quantized-matmul path.

Reads safetensors checkpoints in the layout weightstream's loader expects
(weightstream-core loader.rs:26-143, safetensors.rs:32-72): a directory with
`model.safetensors.index.json` (weight_map: tensor -> shard file) and the
shards, each an 8-byte little-endian header length, a JSON header
{name: {dtype, shape, data_offsets}} and the payload. Payloads are mapped,
not copied, and uploaded as raw bytes:

- FP8 linears: `<name>.weight` e4m3 [N, K] and `<name>.scale` UE8M0
  [ceil(N/32), K/32], read by ws_fp8_gemm as they are;
- routed experts: `<layer>.ffn.experts.<e>.w{1,2,3}.weight` packed e2m1
  [rows, cols/2] and `.scale` UE8M0 [rows, cols/32], concatenated into
  [E*rows, ...] slabs (engine.rs:1346-1353) and relaid out once by
  ws_prepack_fp4 for the routed-expert kernels (engine.rs:842-884 does its
  own relayout at the same point).

Dtype strings follow weightstream-ref store.rs:33-43 and 105-123: a raw
I8/U8 tensor is an e8m0 scale when its name ends in ".scale" and packed FP4
when it is an expert ".weight".
"""
import json
import mmap
import os

import numpy as np
import torch

from . import launch as L

# safetensors dtype string -> kind (store.rs:33-43)
_KINDS = {
    "BF16": "bf16", "BFLOAT16": "bf16",
    "F32": "f32", "FP32": "f32", "FLOAT32": "f32",
    "F8_E4M3": "e4m3", "FLOAT8_E4M3": "e4m3", "FP8": "e4m3",
    "F8_E8M0": "e8m0", "FLOAT8_E8M0": "e8m0",
    "F4_E2M1": "e2m1", "FLOAT4_E2M1": "e2m1", "F4": "e2m1",
    "I8": "u8", "U8": "u8", "INT8": "u8", "UINT8": "u8",
}


def tensor_kind(name, raw_dtype):
    """Kind of a checkpoint tensor from its dtype string and name
    (store.rs:105-123): raw bytes are e8m0 scales or packed FP4 experts."""
    kind = _KINDS.get(raw_dtype)
    if kind is None:
        raise ValueError("%s: unsupported dtype %s" % (name, raw_dtype))
    if kind == "u8":
        if name.endswith(".scale"):
            return "e8m0"
        if ".experts." in name and name.endswith(".weight"):
            return "e2m1"
    return kind


class Shard:
    """One safetensors file, memory-mapped (safetensors.rs:32-53)."""

    def __init__(self, path):
        self.path = path
        self._f = open(path, "rb")
        self._m = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        n = int.from_bytes(self._m[:8], "little")
        if n <= 0 or 8 + n > len(self._m):
            raise ValueError("%s: bad safetensors header length %d" % (path, n))
        hdr = json.loads(bytes(self._m[8:8 + n]))
        hdr.pop("__metadata__", None)
        self.tensors = hdr
        self.data_start = 8 + n

    def meta(self, name):
        return self.tensors[name]

    def bytes(self, name):
        """Zero-copy uint8 view of the payload (raw on-disk bytes)."""
        m = self.tensors[name]
        a, b = m["data_offsets"]
        if not (0 <= a <= b and self.data_start + b <= len(self._m)):
            raise ValueError("%s: data offsets out of the file" % name)
        return np.frombuffer(self._m, dtype=np.uint8, count=b - a, offset=self.data_start + a)

    def close(self):
        self._m.close()
        self._f.close()


class Checkpoint:
    """A checkpoint directory (loader.rs:26-143): index + lazily opened shards.
    A directory with a single model.safetensors and no index also works."""

    def __init__(self, path):
        self.dir = path
        idx = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(idx):
            with open(idx) as f:
                self.index = json.load(f)["weight_map"]
        else:
            single = os.path.join(path, "model.safetensors")
            sh = Shard(single)
            self.index = {n: "model.safetensors" for n in sh.tensors}
            self._shards = {"model.safetensors": sh}
            return
        self._shards = {}

    def _shard(self, name):
        fname = self.index.get(name)
        if fname is None:
            raise KeyError(name)
        if fname not in self._shards:
            self._shards[fname] = Shard(os.path.join(self.dir, fname))
        return self._shards[fname]

    def names(self):
        return self.index.keys()

    def meta(self, name):
        m = dict(self._shard(name).meta(name))
        m["kind"] = tensor_kind(name, m["dtype"])
        return m

    def bytes(self, name):
        return self._shard(name).bytes(name)

    def close(self):
        for s in self._shards.values():
            s.close()
        self._shards = {}


def _expect(ck, name, kind, nbytes):
    m = ck.meta(name)
    if m["kind"] != kind:
        raise ValueError("%s: %s, expected %s" % (name, m["kind"], kind))
    b = ck.bytes(name)
    if b.size != nbytes:
        raise ValueError("%s: %d bytes, expected %d" % (name, b.size, nbytes))
    return b


def load_fp8_linear(ck, name, n, k, device="cuda"):
    """`<name>.weight` e4m3 [n, k] and `<name>.scale` UE8M0 [ceil(n/32), k/32]
    as device uint8 tensors for ws_fp8_gemm."""
    w = _expect(ck, name + ".weight", "e4m3", n * k)
    s = _expect(ck, name + ".scale", "e8m0", ((n + 31) // 32) * (k // 32))
    return (torch.from_numpy(w.copy()).view(n, k).to(device),
            torch.from_numpy(s.copy()).view((n + 31) // 32, k // 32).to(device))


def load_fp8_combined_rows(ck, name_a, name_b, n, k, device="cuda"):
    """engine.rs:931-971 load_q8_combined_rows: two FP8 linears of the same K
    stacked by rows (a's rows, then b's) with their UE8M0 scale rows
    concatenated the same way: w [2n, k], s [2n/32, k/32]. n must be a
    multiple of 32 so that b's scale rows start a fresh 32-row block."""
    if n % 32:
        raise ValueError("combined rows need n %% 32 == 0 (n = %d)" % n)
    wa, sa = load_fp8_linear(ck, name_a, n, k, device)
    wb, sb = load_fp8_linear(ck, name_b, n, k, device)
    return torch.cat([wa, wb]), torch.cat([sa, sb])


def load_gate(ck, prefix, n_experts, dim, device="cuda"):
    """engine.rs:1482-1493: `<prefix>.ffn.gate.weight` bf16 [E, dim] (as the
    raw 16-bit words, for ws_moe_gate_logits with w_bf16 = 1) and
    `<prefix>.ffn.gate.bias` f32 [E]."""
    w = _expect(ck, prefix + ".ffn.gate.weight", "bf16", n_experts * dim * 2)
    b = _expect(ck, prefix + ".ffn.gate.bias", "f32", n_experts * 4)
    return (torch.from_numpy(w.copy().view(np.int16)).view(n_experts, dim).to(device),
            torch.from_numpy(b.copy().view(np.float32)).to(device))


def load_moe_layer(ck, prefix, n_experts, dim, inter, shared_inter, device="cuda"):
    """One MoE layer as engine.rs:1346-1530 assembles it: the gate (bf16
    weight + f32 bias), the routed experts' raw slabs (load_expert_slabs),
    the shared expert's FP8 w1 / w2 / w3 and the fused w13
    (load_fp8_combined_rows). Returns a dict of device tensors."""
    gate_w, gate_b = load_gate(ck, prefix, n_experts, dim, device)
    sp = prefix + ".ffn.shared_experts."
    shared = {wn: load_fp8_linear(ck, sp + wn, *(shape + (device,)))
              for wn, shape in (("w1", (shared_inter, dim)), ("w3", (shared_inter, dim)),
                                ("w2", (dim, shared_inter)))}
    w13 = load_fp8_combined_rows(ck, sp + "w1", sp + "w3", shared_inter, dim, device)
    return {"gate_w": gate_w, "gate_bias": gate_b,
            "experts": load_expert_slabs(ck, prefix, n_experts, dim, inter, device),
            "shared": shared, "shared_w13": w13}


def read_config(path):
    """The MoE fields of `config.json` (weightstream-core config.rs:19-130):
    a nested `text_config` (the DS4.1F-1017 layout) is merged over the top
    level as the reference does, model_type / architectures /
    quantization_config surviving from the top level unless redeclared."""
    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    inner = cfg.pop("text_config", None)
    if inner is not None:
        for key in ("model_type", "architectures", "quantization_config"):
            if key not in inner and key in cfg:
                inner[key] = cfg[key]
        cfg = inner
    for key in ("hidden_size", "qk_rope_head_dim", "vocab_size", "num_hidden_layers",
                "num_attention_heads"):
        if key not in cfg:
            raise ValueError("config.json lacks %s" % key)
    return cfg


def load_expert_slabs(ck, prefix, n_experts, dim, inter, device="cuda"):
    """Routed experts of one layer (`<prefix>.ffn.experts.<e>.w{1,2,3}`),
    concatenated into raw slabs (w1, s1, w3, s3, w2, s2): w1/w3 [E*inter,
    dim/2] + [E*inter, dim/32], w2 [E*dim, inter/2] + [E*dim, inter/32]."""
    shapes = {"w1": (inter, dim), "w3": (inter, dim), "w2": (dim, inter)}
    out = []
    for wn in ("w1", "w3", "w2"):
        rows, cols = shapes[wn]
        w = torch.empty((n_experts * rows, cols // 2), dtype=torch.uint8, device=device)
        s = torch.empty((n_experts * rows, cols // 32), dtype=torch.uint8, device=device)
        for e in range(n_experts):
            base = "%s.ffn.experts.%d.%s" % (prefix, e, wn)
            wb = _expect(ck, base + ".weight", "e2m1", rows * cols // 2)
            sb = _expect(ck, base + ".scale", "e8m0", rows * cols // 32)
            w[e * rows:(e + 1) * rows].copy_(torch.from_numpy(wb.copy()).view(rows, cols // 2))
            s[e * rows:(e + 1) * rows].copy_(torch.from_numpy(sb.copy()).view(rows, cols // 32))
        out += [w, s]
    return tuple(out)


def pack_expert_slabs(raw, n_experts, dim, inter):
    """Upload-time relayout of raw slabs (load_expert_slabs) into the
    fragment-major layout the routed-expert kernels read (ws_prepack_fp4):
    returns (w1, s1, w3, s3, w2, s2) packed."""
    w1, s1, w3, s3, w2, s2 = raw
    return (L.prepack_fp4_new(w1, s1, n_experts * inter, dim)
            + L.prepack_fp4_new(w3, s3, n_experts * inter, dim)
            + L.prepack_fp4_new(w2, s2, n_experts * dim, inter))


def write_safetensors(path, tensors, metadata=None):
    """Write {name: (dtype_string, shape, uint8 bytes)} as one safetensors
    file (header JSON + payload in name order). For tests and tools that
    build synthetic checkpoints."""
    hdr, payload, off = {}, [], 0
    if metadata:
        hdr["__metadata__"] = metadata
    for name in sorted(tensors):
        dt, shape, data = tensors[name]
        data = np.ascontiguousarray(data, dtype=np.uint8).ravel()
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + data.size]}
        payload.append(data)
        off += data.size
    js = json.dumps(hdr).encode()
    js += b" " * ((8 - len(js) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(js).to_bytes(8, "little"))
        f.write(js)
        for p in payload:
            f.write(p.tobytes())
