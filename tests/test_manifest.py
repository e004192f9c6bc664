"""Converted-checkpoint loader (manifest.rs:5-95; Engine::new / upload_shard,
lib.rs:84-125,176-187) on checkpoints written by the restated ShardWriter of
convert.py:122-158,224-233 (oracle/checkpoint.py).  CPU: the index checks and
the byte-exact mapping of every tensor; GPU: a loaded layer and head through
the kernels against the oracle."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import checkpoint as ckpt
from oracle import oracle as orc
from oracle import reference as ref
from webyiq_amd import manifest as mf

SMALL = dict(hidden=256, inter=512, layers=2, heads=4, kv_heads=2, vocab=1000, G=128)


def write(tmp_path, **kw):
    args = dict(SMALL, shard_bytes=200_000)
    args.update(kw)
    rng = np.random.default_rng(3)
    return ckpt.write_llama(str(tmp_path), rng, ref.make_weight, **args)


def test_load_maps_every_tensor_byte_exact(tmp_path):
    m, host = write(tmp_path, tied=False, draft_ids=[5, 1, 900, 42])
    assert len(m["shards"]) > 2  # small shards: tensors spread over several files
    assert all(t["offset"] % 256 == 0 for t in m["tensors"].values())
    model = mf.load(str(tmp_path), device="cpu")
    assert model.G == 128 and model.config["num_layers"] == 2
    for name, v in host.items():
        if isinstance(v, tuple):
            w = model.weights.w(name)
            assert w.K == v[0].shape[1] * 8 and w.G == 128
            assert np.array_equal(w.q.numpy().view(np.uint32), v[0])
            assert np.array_equal(w.s.numpy().view(np.uint32), v[1])
        else:
            got = model.weights[name].numpy()
            assert np.array_equal(got.view(v.dtype) if v.dtype == np.uint32 else got, v)
    lw = model.layer(1)
    assert lw.w("down").K == SMALL["inter"] and lw.w("qkv").K == SMALL["hidden"]
    assert torch.equal(lw["mlp_norm"], model.weights["l1.ffn_norm"])
    assert model.head() is model.weights.w("lm_head")
    assert np.array_equal(model.weights["mtp.head_ids"].numpy().view(np.uint32), [1, 5, 42, 900])


def test_tied_head_is_the_embedding(tmp_path):
    write(tmp_path, tied=True, layers=1)
    model = mf.load(str(tmp_path), device="cpu")
    assert "lm_head" not in model.weights and model.head() is model.weights.w("embed")


def test_shard_bytes(tmp_path):
    m, _ = write(tmp_path, layers=1)
    man = mf.Manifest.parse(json.dumps(m))
    sizes = man.shard_bytes()
    for i, name in enumerate(m["shards"]):
        assert os.path.getsize(os.path.join(tmp_path, name)) == sizes[i]


@pytest.mark.parametrize("edit,msg", [
    (lambda d: d.update(format="webyiq-v1"), "unsupported model"),
    (lambda d: d.update(arch="gpt2"), "unsupported model"),
    (lambda d: d["quant"].update(bits=8), "unsupported quant"),
    (lambda d: d["quant"].update(group=64), "unsupported quant"),
    (lambda d: d["config"].pop("vocab_size"), "config lacks vocab_size"),
    (lambda d: d["tensors"]["l0.o.q"].update(bytes=12), "do not match"),
    (lambda d: d["tensors"]["norm"].update(shard=99), "not in the shard list"),
    (lambda d: d["tensors"]["l0.o.q"].update(shape=[256, 200], bytes=25600), "multiple of 128"),
    (lambda d: d["tensors"]["norm"].update(dtype="bf16"), "unknown dtype"),
    # scale words that do not pair with their packed weight at the group
    (lambda d: d["tensors"]["l0.o.s"].update(shape=[256, 8], bytes=8192), "does not match"),
    (lambda d: d["tensors"].pop("l0.o.s"), "no q4s scale tensor"),
    (lambda d: d["tensors"]["l0.o.q"].update(dtype="u32", bytes=4 * 256 * 256), "without a q4 tensor"),
])
def test_manifest_errors(tmp_path, edit, msg):
    m, _ = write(tmp_path, layers=1)
    d = json.loads(json.dumps(m))
    edit(d)
    with pytest.raises(ValueError, match=msg):
        mf.Manifest.parse(json.dumps(d))
    with pytest.raises(ValueError, match="bad manifest"):
        mf.Manifest.parse("{")


def test_group_32_checkpoint_and_truncated_shard(tmp_path):
    m, host = write(tmp_path, layers=1, G=32)
    model = mf.load(str(tmp_path), device="cpu")
    assert model.G == 32 and model.weights.w("l0.qkv").G == 32
    last = os.path.join(tmp_path, m["shards"][-1])
    with open(last, "r+b") as f:
        f.truncate(os.path.getsize(last) - 4)
    with pytest.raises(ValueError, match="the manifest needs"):
        mf.load(str(tmp_path), device="cpu")


@pytest.mark.gpu
def test_loaded_checkpoint_on_gpu(tmp_path):
    """A loaded layer's fused norm+quant+qkv and the tied head's greedy token,
    bit-exact against the oracle on the host arrays; the draft head gathered
    from the loaded embedding maps its winner back through the ids."""
    from webyiq_amd import ops
    print("[case] loaded checkpoint on gpu", flush=True)
    hidden, vocab, G = 2048, 4096, 128
    m, host = write(tmp_path, hidden=hidden, inter=1024, layers=1, heads=16, kv_heads=4, vocab=vocab, G=G,
                    tied=True, draft_ids=np.arange(7, vocab, 5), shard_bytes=4 << 20)
    model = mf.load(str(tmp_path), device="cuda")
    rng = np.random.default_rng(9)
    x = ref.make_activations(rng, 1, hidden)
    lw = model.layer(0)
    y, a = ops.quant_gemv(lw.w("qkv"), torch.from_numpy(x).cuda(), norm=lw["attn_norm"], eps=1e-6)
    xq, dx, xs = orc.quant_act(x, None, G, norm_w=host["l0.attn_norm"], eps=1e-6)
    want = orc.linear(*host["l0.qkv"], hidden, G, xq, dx, xs)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    tok = ops.lm_head_argmax(model.head(), a, workspace=ops.lm_head_workspace()).cpu().numpy()
    logits = orc.linear(*host["embed"], hidden, G, xq, dx, xs)
    assert int(tok[0]) == int(orc.argmax(logits)[0])
    ids = host["mtp.head_ids"]
    dt = ops.lm_head_argmax(model.draft_head(), a, ids=model.weights["mtp.head_ids"],
                            workspace=ops.lm_head_workspace()).cpu().numpy()
    assert int(dt[0]) == int(orc.argmax(logits[:, ids], ids)[0])
