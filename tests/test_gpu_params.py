"""Device step parameters (wq_params, the reference's Params uniform,
gemm_q4q8.wgsl:8-13 / attn_combine.wgsl:6-11) on the GPU, through the C ABI.

  * A prefill GEMM recorded for 128 tokens (captured in a HIP graph) covers
    the m tokens the Params buffer holds when it replays: rows 0 .. m-1
    against the oracle, the rows past m untouched (gemm_q4q8.wgsl:69,106).
  * A decode layer with the chunk merge, captured once, replayed at three
    positions with only the Params buffer rewritten between replays
    (lib.rs:312-314): each replay equals an eager run of the same layer at
    that position bit for bit, and its merged o-projection input equals the
    oracle's merge at that position bit for bit (partials with equal chunk
    maxima, so every chunk weight is exp(0)).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import reference as ref
from webyiq_amd import ops
from conftest import rel_err

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


@pytest.mark.parametrize("K,N,mode", [(2048, 1024, 0), (6144, 512, 1), (2048, 256, 2)])
def test_gemm_chunk_follows_params(K, N, mode):
    CAP, G = 128, 128
    note(f"gemm params K={K} N={N} mode={mode}")
    rng = np.random.default_rng(K + N + mode)
    rows = 2 * N if mode == 2 else N
    wq, ws = ref.make_weight(rng, rows, K, G)
    x = ref.make_activations(rng, CAP, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    y0 = rng.normal(size=(CAP, N)).astype(np.float32)
    want = orc.linear(wq, ws, K, G, xq, dx, xs, mode=mode, y=y0 if mode == 1 else None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = ops.Acts(dev(xq), dev(dx), dev(xs), K, G)
    params = ops.make_params(m=CAP)
    base = y0 if mode == 1 else np.full((CAP, N), np.nan, np.float32)
    y = dev(base)
    g = capture(lambda: ops.gemm(w, a, mode=mode, y=y, params=params))
    for m in (77, CAP, 1, 0):
        y.copy_(dev(base))
        ops.set_params(params, m=m)
        g.replay()
        got = host(y)
        if m:
            assert rel_err(got[:m], want[:m]) < 1e-5, f"m={m}"
        assert np.array_equal(got[m:].view(np.uint32), base[m:].view(np.uint32)), f"m={m}: rows past m written"


def test_decode_layer_positions_from_params():
    from webyiq_amd.layer import DecodeLayer
    M, H, Q, KV, F, G, D, CTX = 2, 1024, 1024, 256, 2048, 128, 128, 2048
    note("decode layer replayed at three positions from the Params buffer")
    rng = np.random.default_rng(33)
    shapes = {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H), "down": (H, F)}
    w = ops.Weights({n: ops.Q4Tensor.from_numpy(*ref.make_weight(rng, r, c, G), c, G)
                     for n, (r, c) in shapes.items()})
    w["attn_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    w["mlp_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    x0 = dev(ref.make_activations(rng, M, H))
    params = ops.make_params()
    layer = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, attention="combine", head_dim=D,
                        max_ctx=CTX, params=params)
    layer.part[..., D] = 0.75   # equal chunk maxima: the merge is exact, comparable bit for bit
    eager = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, attention="combine", head_dim=D,
                        max_ctx=CTX)
    eager.part.copy_(layer.part)

    def step():
        layer.x.copy_(x0)
        layer.run()
    g = capture(step)
    part_h = host(layer.part)
    for pos in (100, 1500, CTX - M):
        ops.set_params(params, pos=pos, seq_len=pos + M, m=M)
        g.replay()
        got = host(layer.x).copy()
        got_q, got_dx, got_xs = host(layer.a_att.xq), host(layer.a_att.dx), host(layer.a_att.xs)
        eager.pos = pos
        eager.x.copy_(x0)
        eager.run()
        assert np.array_equal(got.view(np.uint32), host(eager.x).view(np.uint32)), f"pos {pos}"
        cq, cdx, cxs = orc.attn_combine(part_h, pos)
        assert np.array_equal(got_q, cq), f"pos {pos}: merged codes"
        assert np.array_equal(got_dx.view(np.uint32), cdx.view(np.uint32)), f"pos {pos}: merged scales"
        assert np.array_equal(got_xs, cxs), f"pos {pos}: merged sums"
        # eager work between replays (lib.rs pipelines other submissions)
        ops.quant(dev(rng.normal(size=(3, 256)).astype(np.float32)))
    # a device position past the bound is clamped to it, never read past the context
    ops.set_params(params, pos=10 ** 6, m=M)
    g.replay()
    cq, _, _ = orc.attn_combine(part_h, CTX - M)
    assert np.array_equal(host(layer.a_att.xq), cq)
