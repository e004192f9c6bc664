"""GPU parity of the other producers of int8 activations, through the C ABI.

  * wq_mtp_in (mtp_in.wgsl): codes, dx, xs bit-exact against the oracle (the
    kernel's sums of squares and products run in the oracle's order).
  * wq_attn_combine (attn_combine.wgsl): bit-exact where every chunk weight
    is exp(0) = 1 and no gate is applied; otherwise the device expf and the
    host's may differ in the last bit, so dx within rel 1e-5, codes within
    one step (and equal in all but a 1e-3 fraction), xs the exact sums of
    the device's own codes.  Chunks past a token's positions hold NaN: a
    read of one would poison its head's output.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import reference as ref
from webyiq_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("M,K", [(1, 2048), (3, 4096), (2, 8192), (5, 2304)])
def test_mtp_in_bit_exact(M, K):
    note(f"mtp_in M={M} K={K}")
    rng = np.random.default_rng(100 + M + K)
    emb = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    x = rng.normal(0, 4, size=(M, K)).astype(np.float32)
    x[:, rng.choice(K, 4, replace=False)] *= 30.0
    nf, ne, nh = (rng.normal(1, 0.3, size=K).astype(np.float32) for _ in range(3))
    want = orc.mtp_in(emb, x, nf, ne, nh, eps=1e-6)
    a = ops.mtp_in(dev(emb), dev(x), dev(nf), dev(ne), dev(nh), eps=1e-6)
    for got, exp, name in zip((a.xq, a.dx, a.xs), want, ("xq", "dx", "xs")):
        assert np.array_equal(host(got), exp), name


def make_part(rng, M, H, D, nch, pos, equal_max):
    part = np.full((M, H, nch, D + 2), np.nan, np.float32)
    for m in range(M):
        n = (pos + m + 32) // 32
        part[m, :, :n, :D] = rng.normal(0, 3, size=(H, n, D))
        part[m, :, :n, D] = 0.75 if equal_max else rng.normal(0, 2, size=(H, n))
        part[m, :, :n, D + 1] = rng.uniform(1, 32, size=(H, n))
    return part


@pytest.mark.parametrize("D,M,H,nch,pos", [
    (64, 2, 3, 8, 100), (128, 2, 4, 8, 127), (256, 1, 2, 4, 31), (128, 3, 2, 130, 4000),
    (128, 2, 4, 8192, 262142),  # the host-checked maximum: 8192 chunks, last token at 262143
])
def test_attn_combine_equal_maxima_bit_exact(D, M, H, nch, pos):
    note(f"attn_combine exact D={D} M={M} H={H} nch={nch} pos={pos}")
    rng = np.random.default_rng(D + 7 * pos)
    part = make_part(rng, M, H, D, nch, pos, equal_max=True)
    want = orc.attn_combine(part, pos)
    a = ops.attn_combine(dev(part), pos)
    for got, exp, name in zip((a.xq, a.dx, a.xs), want, ("xq", "dx", "xs")):
        assert np.array_equal(host(got), exp), name


@pytest.mark.parametrize("D,gated", [(64, False), (128, True), (256, True)])
def test_attn_combine_random(D, gated):
    M, H, nch, pos = 4, 3, 16, 200
    note(f"attn_combine random D={D} gated={gated}")
    rng = np.random.default_rng(D + gated)
    part = make_part(rng, M, H, D, nch, pos, equal_max=False)
    stride = 2 * (H + 1) * D
    gate = rng.normal(0, 2, size=(M, stride)).astype(np.float32) if gated else None
    xq_r, dx_r, _ = orc.attn_combine(part, pos, gate, stride if gated else 0)
    a = ops.attn_combine(dev(part), pos, None if gate is None else dev(gate), stride if gated else 0)
    xq, dx, xs = host(a.xq), host(a.dx), host(a.xs)
    assert np.all(np.isfinite(dx))
    assert np.allclose(dx, dx_r, rtol=1e-5, atol=0)
    diff = np.abs(xq.astype(np.int32) - xq_r.astype(np.int32))
    assert diff.max() <= 1 and np.mean(diff != 0) < 1e-3
    assert np.array_equal(xs, xq.astype(np.int32).reshape(M, -1, 32).sum(-1))


def test_attn_combine_feeds_the_o_projection():
    """The combine's output is a per-32 activation tensor the GEMV takes as is."""
    M, H, D, nch, pos, N, G = 1, 16, 128, 8, 60, 256, 128
    note("attn_combine -> gemv")
    rng = np.random.default_rng(5)
    part = make_part(rng, M, H, D, nch, pos, equal_max=True)
    xq_r, dx_r, xs_r = orc.attn_combine(part, pos)
    wq, ws = ref.make_weight(rng, N, H * D, G)
    y_r = orc.linear(wq, ws, H * D, G, xq_r, dx_r, xs_r, GA=32)
    a = ops.attn_combine(dev(part), pos, G=G)
    y = ops.gemv(ops.Q4Tensor(dev(wq.view(np.int32)), dev(ws.view(np.int32)), H * D, G), a)
    assert np.array_equal(host(y), y_r)


def test_decode_layer_with_attention_combine():
    """The layer's decode order with the chunk merge (graph.rs:289-291):
    combine -> o (plain GEMV on per-32 activations) equals the oracle's
    combine and linear bit for bit, and graph replays reproduce the eager run."""
    from webyiq_amd.layer import DecodeLayer
    note("decode layer attention=combine")
    M, H, Q, KV, F, G, D, pos = 2, 1024, 1024, 256, 2048, 128, 128, 300
    rng = np.random.default_rng(31)
    shapes = {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H), "down": (H, F)}
    host_w = {n: ref.make_weight(rng, r, c, G) for n, (r, c) in shapes.items()}
    w = ops.Weights({n: ops.Q4Tensor.from_numpy(q, s, shapes[n][1], G) for n, (q, s) in host_w.items()})
    w["attn_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    w["mlp_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    x0 = dev(ref.make_activations(rng, M, H))
    layer = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, attention="combine", head_dim=D,
                        pos=pos, max_ctx=1024)
    part = make_part(rng, M, Q // D, D, 1024 // 32, pos, equal_max=True)
    layer.part.copy_(dev(part))

    # combine -> o alone against the oracle
    xq, dx, xs = orc.attn_combine(part, pos)
    a = ops.attn_combine(layer.part, pos)
    for got, exp in zip((a.xq, a.dx, a.xs), (xq, dx, xs)):
        assert np.array_equal(host(got), exp)
    y0 = host(x0).copy()
    y_want = orc.linear(*host_w["o"], Q, G, xq, dx, xs, mode=1, y=y0.copy(), GA=32)
    y = x0.clone()
    ops.gemv(w.w("o"), a, mode=ops.MODE_ACCUMULATE, y=y)
    assert np.array_equal(host(y).view(np.uint32), y_want.view(np.uint32))

    layer.x.copy_(x0)
    layer.run()
    want = host(layer.x).copy()
    assert np.all(np.isfinite(want))
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.x.copy_(x0)
        layer.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        layer.x.copy_(x0)
        layer.run()
    for i in range(3):
        g.replay()
        got = host(layer.x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i}"
        layer.x.add_(1.0)  # eager work between replays
        torch.cuda.synchronize()
