"""Converted-checkpoint loader: manifest.json + shard files -> device tensors.

The reference's loader is crates/engine/src/manifest.rs:5-95 (the manifest
schema and Manifest::parse's checks) plus Engine::new / Engine::upload_shard
(crates/engine/src/lib.rs:84-125,176-187: one buffer per tensor, each shard
read once and its tensors copied out by (offset, bytes)).  The files are the
ones tools/convert.py:122-158,224-233 writes: shard-NNN.bin with 256-byte
aligned tensors and a JSON index {shard, offset, bytes, dtype, shape}.

MI355X side: each shard is memory-mapped and its tensors are copied to the
device one at a time, so host memory holds at most one tensor beyond the
page cache; int4 weights become Q4Tensor views (.q u32 [N, K/8], .s u32
[N, K/G]) that the kernels take as they are.  Quant group 128 is admitted
besides the reference's 32 (manifest.rs:82 accepts 32 only).
"""
import json
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import ops

FORMAT = "webyiq-v2"
ARCHS = ("llama", "qwen3_5")
GROUPS = (32, 128)
CONFIG_KEYS = ("hidden_size", "intermediate_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
               "vocab_size", "rms_norm_eps", "rope_theta", "max_position_embeddings", "eos_token_ids")


@dataclass
class TensorInfo:
    shard: int
    offset: int
    bytes: int
    dtype: str
    shape: list


def _expected_bytes(t: TensorInfo):
    n = int(np.prod(t.shape)) if t.shape else 1
    if t.dtype == "q4":
        return n // 2
    if t.dtype in ("q4s", "f32", "u32"):
        return 4 * n
    raise ValueError(f"unknown dtype {t.dtype!r}")


class Manifest:
    def __init__(self, d):
        self.format = d["format"]
        self.arch = d["arch"]
        self.config = d["config"]
        self.quant = d["quant"]
        self.shards = list(d["shards"])
        self.tensors = {k: TensorInfo(**v) for k, v in d["tensors"].items()}

    @staticmethod
    def parse(text):
        """manifest.rs:78-85, with the index checked against itself."""
        try:
            d = json.loads(text)
            m = Manifest(d)
        except (ValueError, KeyError, TypeError) as e:
            raise ValueError(f"bad manifest: {e}") from None
        if m.format != FORMAT or m.arch not in ARCHS:
            raise ValueError(f"unsupported model: {m.format} / {m.arch}")
        if m.quant.get("bits") != 4 or m.quant.get("group") not in GROUPS:
            raise ValueError(f"unsupported quant: {m.quant}")
        missing = [k for k in CONFIG_KEYS if k not in m.config]
        if missing:
            raise ValueError(f"bad manifest: config lacks {', '.join(missing)}")
        G = m.group
        for name, t in m.tensors.items():
            if not 0 <= t.shard < len(m.shards):
                raise ValueError(f"{name}: shard {t.shard} not in the shard list")
            if t.offset < 0 or t.bytes != _expected_bytes(t):
                raise ValueError(f"{name}: {t.bytes} bytes do not match dtype {t.dtype} shape {t.shape}")
            if t.dtype == "q4" and (len(t.shape) != 2 or t.shape[1] % G):
                raise ValueError(f"{name}: shape {t.shape} is not [N, K] with K a multiple of {G}")
            if t.dtype == "q4s" and len(t.shape) != 2:
                raise ValueError(f"{name}: shape {t.shape} is not [N, K/G]")
        # every packed weight X.q pairs with its scale words X.s of shape
        # [N, K/G] for the manifest's group, and every X.s with an X.q: the
        # kernels read K/G words per row of .s with no bound of their own
        for name, t in m.tensors.items():
            if t.dtype == "q4":
                if not name.endswith(".q"):
                    raise ValueError(f"{name}: a q4 tensor must be named <weight>.q")
                sname = name[:-2] + ".s"
                s = m.tensors.get(sname)
                if s is None or s.dtype != "q4s":
                    raise ValueError(f"{name}: no q4s scale tensor {sname}")
                want = [t.shape[0], t.shape[1] // G]
                if list(s.shape) != want:
                    raise ValueError(f"{sname}: shape {s.shape} does not match {name} {t.shape} "
                                     f"at group {G} (want {want})")
            elif t.dtype == "q4s":
                qname = name[:-2] + ".q" if name.endswith(".s") else None
                if qname is None or qname not in m.tensors or m.tensors[qname].dtype != "q4":
                    raise ValueError(f"{name}: scale words without a q4 tensor <weight>.q")
        return m

    @property
    def group(self):
        return int(self.quant["group"])

    def shard_bytes(self):
        """manifest.rs:87-93: the bytes each shard must hold."""
        sizes = [0] * len(self.shards)
        for t in self.tensors.values():
            sizes[t.shard] = max(sizes[t.shard], t.offset + t.bytes)
        return sizes


class Model:
    """Tensors of a converted checkpoint on one device, by manifest name."""

    def __init__(self, manifest, tensors, device):
        self.manifest, self.device = manifest, device
        self.config = manifest.config
        self.G = manifest.group
        self.weights = ops.Weights()
        for name, t in tensors.items():
            info = manifest.tensors[name]
            if info.dtype == "q4":
                base = name[:-2]
                s = tensors[base + ".s"]
                self.weights[base] = ops.Q4Tensor(t, s, int(info.shape[1]), self.G)
            elif info.dtype in ("f32", "u32"):
                self.weights[name] = t
        self._draft = None

    def layer(self, i):
        """The names one decoder layer's linear sequence uses (graph.rs:257-328)."""
        w, p = self.weights, f"l{i}."
        out = ops.Weights()
        for k in ("qkv", "o", "gate_up", "down"):
            out[k] = w.w(p + k)
        out["attn_norm"] = w[p + "attn_norm"]
        out["mlp_norm"] = w[p + "ffn_norm"]
        return out

    def head(self):
        """lm_head, or the embedding when tied (convert.py:187-190)."""
        return self.weights.w("lm_head" if "lm_head" in self.weights else "embed")

    def draft_head(self, stream=None):
        """The reduced draft lm_head: embedding rows of mtp.head_ids, gathered
        on the device once (lib.rs:100-112, graph.rs:511-516)."""
        if self._draft is None:
            ids = self.weights["mtp.head_ids"]
            self._draft = ops.gather_rows(self.weights.w("embed"), ids, stream=stream)
        return self._draft


def load(path, device="cuda"):
    """Read manifest.json and every shard under `path` onto `device`."""
    with open(os.path.join(path, "manifest.json"), encoding="utf-8") as f:
        m = Manifest.parse(f.read())
    need = m.shard_bytes()
    by_shard = {}
    for name, t in m.tensors.items():
        by_shard.setdefault(t.shard, []).append(name)
    tensors = {}
    for i, fname in enumerate(m.shards):
        fp = os.path.join(path, fname)
        have = os.path.getsize(fp) if os.path.exists(fp) else -1
        if have < need[i]:
            raise ValueError(f"{fname}: {max(have, 0)} bytes, the manifest needs {need[i]}")
        if not by_shard.get(i):
            continue
        mm = np.memmap(fp, dtype=np.uint8, mode="r")
        for name in by_shard[i]:
            t = m.tensors[name]
            raw = np.array(mm[t.offset:t.offset + t.bytes])  # one tensor's bytes in host memory
            if t.dtype == "q4":
                arr = raw.view(np.int32).reshape(t.shape[0], t.shape[1] // 8)
            elif t.dtype == "q4s":
                arr = raw.view(np.int32).reshape(t.shape)
            elif t.dtype == "f32":
                arr = raw.view(np.float32).reshape(t.shape)
            else:  # u32, kept as int32 bits
                arr = raw.view(np.int32).reshape(t.shape)
            tensors[name] = torch.from_numpy(arr).to(device)
        del mm
    return Model(m, tensors, device)
