"""Writer of webyIQ's converted-checkpoint format, restated for tests.
TEST INFRASTRUCTURE ONLY: it produces the files the loader under test reads.

Restates tools/convert.py:
  :122-158  ShardWriter -- tensors appended to shard-NNN.bin files, each
            tensor's start aligned to 256 bytes (zero padding), a new shard
            started when the next tensor would pass the shard size (unless the
            shard is empty); every tensor recorded as
            {shard, offset, bytes, dtype, shape}; .q / .s pairs from add_q4
            with dtypes "q4" (shape [N, K]) and "q4s" (shape [N, K / group]);
  :172-187  llama layer names: l{i}.attn_norm (f32), l{i}.qkv, l{i}.o,
            l{i}.ffn_norm (f32), l{i}.gate_up, l{i}.down, then norm and
            lm_head (absent when tied);
  :216,219-221  embed, mtp.head_ids (u32, ascending);
  :224-233  manifest.json: format "webyiq-v2", arch, config, quant
            {bits: 4, group, scheme}, shards, tensors.
The shard hashes of :109-118 are omitted (the loader does not read them).
"""
import json
import os

import numpy as np

SHARD_BYTES = 128 << 20  # convert.py:23
ALIGN = 256              # convert.py:24


class ShardWriter:
    def __init__(self, out_dir, shard_bytes=SHARD_BYTES):
        self.out_dir = out_dir
        self.shard_bytes = shard_bytes
        self.index = -1
        self.f = None
        self.pos = 0
        self.tensors = {}
        self._next()

    def _next(self):
        if self.f:
            self.f.close()
        self.index += 1
        self.f = open(os.path.join(self.out_dir, f"shard-{self.index:03d}.bin"), "wb")
        self.pos = 0

    def add(self, name, arr, dtype, shape):
        data = np.ascontiguousarray(arr).tobytes()
        if self.pos > 0 and self.pos + len(data) > self.shard_bytes:
            self._next()
        pad = (-self.pos) % ALIGN
        self.f.write(b"\0" * pad)
        self.pos += pad
        self.tensors[name] = {"shard": self.index, "offset": self.pos, "bytes": len(data),
                              "dtype": dtype, "shape": list(shape)}
        self.f.write(data)
        self.pos += len(data)

    def add_q4(self, name, wq, ws, K, G):
        """Packed codes u32 [N, K/8] and scale words u32 [N, K/G]."""
        n = wq.shape[0]
        self.add(name + ".q", wq, "q4", (n, K))
        self.add(name + ".s", ws, "q4s", (n, K // G))

    def close(self):
        self.f.close()
        return self.index + 1


def write_llama(out_dir, rng, make_weight, hidden, inter, layers, heads, kv_heads, vocab, G,
                tied=True, draft_ids=None, shard_bytes=SHARD_BYTES):
    """A random llama-shaped checkpoint; returns (manifest dict, host arrays by name)."""
    os.makedirs(out_dir, exist_ok=True)
    w = ShardWriter(out_dir, shard_bytes)
    host = {}
    d = hidden // heads

    def q4(name, n, k):
        wq, ws = make_weight(rng, n, k, G)
        host[name] = (wq, ws)
        w.add_q4(name, wq, ws, k, G)

    def f32(name, n):
        v = rng.normal(1.0, 0.1, size=n).astype(np.float32)
        host[name] = v
        w.add(name, v, "f32", [n])

    q4("embed", vocab, hidden)
    for i in range(layers):
        f32(f"l{i}.attn_norm", hidden)
        q4(f"l{i}.qkv", (heads + 2 * kv_heads) * d, hidden)
        q4(f"l{i}.o", hidden, heads * d)
        f32(f"l{i}.ffn_norm", hidden)
        q4(f"l{i}.gate_up", 2 * inter, hidden)
        q4(f"l{i}.down", hidden, inter)
    f32("norm", hidden)
    if not tied:
        q4("lm_head", vocab, hidden)
    if draft_ids is not None:
        ids = np.sort(np.asarray(draft_ids, np.uint32))
        host["mtp.head_ids"] = ids
        w.add("mtp.head_ids", ids, "u32", [len(ids)])
    n = w.close()
    config = {"hidden_size": hidden, "intermediate_size": inter, "num_layers": layers, "num_heads": heads,
              "num_kv_heads": kv_heads, "head_dim": d, "vocab_size": vocab, "rms_norm_eps": 1e-6,
              "rope_theta": 10000.0, "max_position_embeddings": 4096, "bos_token_id": 1,
              "eos_token_ids": [2], "tie_word_embeddings": tied}
    if draft_ids is not None:
        config["mtp_layers"] = 1
    manifest = {"format": "webyiq-v2", "arch": "llama", "config": config,
                "quant": {"bits": 4, "group": G, "scheme": "asym-rtn"},
                "shards": [f"shard-{i:03d}.bin" for i in range(n)], "tensors": w.tensors}
    json.dump(manifest, open(os.path.join(out_dir, "manifest.json"), "w"), indent=1)
    return manifest, host
