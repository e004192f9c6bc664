"""Known-answer vectors (tests/golden/known_answers.json, written by
tests/golden/make_known_answers.py from the reference's definitions in exact
arithmetic): the CPU oracle reproduces every one, and so does the HIP path on
the GPU, bit for bit.

Cases: the `.q` packing (convert.py:8-12, with the comment's 0x73625140), the
activation quantiser's half-even ties, zero groups and power-of-two scales
(quant.wgsl:41-61) in four formats, the linear identity in modes 0 and 1 with
nibble-order probes (gemv_q4q8.wgsl:6) on the GEMV, the GEMM and the fused
lm_head argmax, argmax ties / NaN / -3e38 / id mapping (argmax.wgsl:14-43)
and the int4 embedding (embed.wgsl:13-27).
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))
K = KA["K"]


def u32(a):
    return np.asarray(a, dtype=np.uint32)


def f32(a):
    return np.asarray(a, dtype=np.float32)


def logits():
    return np.array([[np.nan if v == "nan" else v for v in r] for r in KA["argmax"]["logits"]], np.float32)


def quant_cases():
    return [pytest.param(c, id=c["name"]) for c in KA["quant"]]


def linear_cases():
    return [pytest.param(c, id=f"G{c['G']}_GA{c['GA']}") for c in KA["linear"]]


def ga_arg(c):
    return None if c["GA"] == K else c["GA"]


# ------------------------------------------------------------------ CPU -----

def test_oracle_pack_and_unpack():
    p = KA["pack"]
    codes = np.asarray(p["codes"], np.uint8)
    zeros = np.zeros((codes.shape[0], 1), np.uint16)
    wq, _ = orc.q4_pack(codes, zeros, zeros, K)
    assert np.array_equal(wq, u32(p["words"]))
    assert wq[0, 0] == 0x73625140
    assert np.array_equal(orc.q4_unpack(u32(p["words"]), K), codes)


@pytest.mark.parametrize("c", quant_cases())
def test_oracle_quant(c):
    xq, dx, xs = orc.quant_act(f32(c["x"]), ga_arg(c), c["G"])
    assert np.array_equal(xq, np.asarray(c["xq"], np.int8))
    assert np.array_equal(dx.view(np.uint32), f32(c["dx"]).view(np.uint32))
    assert np.array_equal(xs, np.asarray(c["xs"], np.int32))


@pytest.mark.parametrize("c", linear_cases())
def test_oracle_linear(c):
    args = (u32(c["words"]), u32(c["scale_words"]), K, c["G"], np.asarray(c["xq"], np.int8), f32(c["dx"]),
            np.asarray(c["xs"], np.int32))
    y0 = orc.linear(*args, mode=0, GA=c["GA"])
    assert np.array_equal(y0.view(np.uint32), f32(c["y_mode0"]).view(np.uint32))
    y1 = orc.linear(*args, mode=1, y=f32(c["y0"]), GA=c["GA"])
    assert np.array_equal(y1.view(np.uint32), f32(c["y_mode1"]).view(np.uint32))
    assert np.array_equal(orc.argmax(y0), u32(c["argmax_mode0"]))


def test_oracle_argmax():
    a = KA["argmax"]
    assert np.array_equal(orc.argmax(logits()), u32(a["tokens"]))
    assert np.array_equal(orc.argmax(logits(), u32(a["ids"])), u32(a["tokens_mapped"]))


def test_oracle_embed():
    e = KA["embed"]
    x = orc.embed(u32(e["words"]), u32(e["scale_words"]), K, e["G"], np.arange(3, dtype=np.uint32))
    assert np.array_equal(x.view(np.uint32), f32(e["x"]).view(np.uint32))


# ------------------------------------------------------------------ GPU -----

def _dev():
    import torch
    from webyiq_amd import ops
    return torch, ops


def _d(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _h(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("c", quant_cases())
def test_gpu_quant(c):
    torch, ops = _dev()
    print(f"[case] golden quant {c['name']}", flush=True)
    a = ops.quant(_d(torch, f32(c["x"])), GA=ga_arg(c), G=c["G"])
    assert np.array_equal(_h(torch, a.xq), np.asarray(c["xq"], np.int8))
    assert np.array_equal(_h(torch, a.dx).view(np.uint32), f32(c["dx"]).reshape(a.dx.shape).view(np.uint32))
    assert np.array_equal(_h(torch, a.xs), np.asarray(c["xs"], np.int32).reshape(a.xs.shape))


@pytest.mark.gpu
@pytest.mark.parametrize("c", linear_cases())
def test_gpu_linear_gemv_gemm_lm_head(c):
    torch, ops = _dev()
    print(f"[case] golden linear G={c['G']} GA={c['GA']}", flush=True)
    w = ops.Q4Tensor.from_numpy(u32(c["words"]), u32(c["scale_words"]), K, c["G"])
    dx = f32(c["dx"])
    a = ops.Acts(_d(torch, np.asarray(c["xq"], np.int8)), _d(torch, dx.reshape(4, -1)),
                 _d(torch, np.asarray(c["xs"], np.int32)), c["GA"], c["G"])
    want0, want1 = f32(c["y_mode0"]).view(np.uint32), f32(c["y_mode1"]).view(np.uint32)
    for fn in (ops.gemv, ops.gemm):
        assert np.array_equal(_h(torch, fn(w, a)).view(np.uint32), want0), fn.__name__
        y = _d(torch, f32(c["y0"]))
        fn(w, a, mode=ops.MODE_ACCUMULATE, y=y)
        assert np.array_equal(_h(torch, y).view(np.uint32), want1), fn.__name__
    tok = ops.lm_head_argmax(w, a, workspace=ops.lm_head_workspace())
    assert np.array_equal(_h(torch, tok).astype(np.uint32), u32(c["argmax_mode0"]))


@pytest.mark.gpu
def test_gpu_argmax():
    torch, ops = _dev()
    print("[case] golden argmax", flush=True)
    a = KA["argmax"]
    got = _h(torch, ops.argmax(_d(torch, logits()))).astype(np.uint32)
    assert np.array_equal(got, u32(a["tokens"]))
    ids = _d(torch, u32(a["ids"]).view(np.int32))
    got = _h(torch, ops.argmax(_d(torch, logits()), ids=ids)).astype(np.uint32)
    assert np.array_equal(got, u32(a["tokens_mapped"]))


@pytest.mark.gpu
def test_gpu_embed():
    torch, ops = _dev()
    print("[case] golden embed", flush=True)
    e = KA["embed"]
    w = ops.Q4Tensor.from_numpy(u32(e["words"]), u32(e["scale_words"]), K, e["G"])
    x = ops.embed(w, _d(torch, np.arange(3, dtype=np.int32)))
    assert np.array_equal(_h(torch, x).view(np.uint32), f32(e["x"]).view(np.uint32))
