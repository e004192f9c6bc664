"""GPU parity of the per-GPU shard shapes: what one GPU computes when the path
is split over P GPUs, with the exchanges stood in for on the host.

  * decode GEMV (cfg 1) split along N: each shard's rows are bit-identical to
    the same rows of the unsharded product (rows are independent);
  * lm_head + argmax (cfg 5) split along V: each shard maps its local index to
    the global row through the ids table (the draft-vocabulary path of
    argmax.wgsl:41), and the host's max over the shards' (logit, -index)
    keys -- the all-gather a multi-GPU step would do -- is the unsharded
    token, ties to the lowest global index;
  * MLP block (cfg 2) split as gate_up along N and down along K: the down
    shards quantise with the token's global absmax (one 4-byte exchange per
    token), so their codes are the unsharded codes' columns; each gate_up
    shard's rows are bit-identical to the unsharded gate_up's; the partial
    sums, accumulated in mode 1, match the oracle run in the same order bit
    for bit and the unsharded block within rel 1e-5.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import reference as ref
from webyiq_amd import ops
from conftest import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
G = 128


def note(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("P", [2, 4, 8])
def test_gemv_row_shards(P):
    M, K, N = 1, 2048, 6144
    note(f"gemv row shards P={P} ({N // P} rows each)")
    rng = np.random.default_rng(100 + P)
    wq, ws = ref.make_weight(rng, N, K, G)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    want = orc.linear(wq, ws, K, G, xq, dx, xs)
    a = ops.Acts(dev(xq), dev(dx), dev(xs), K, G)
    n = N // P
    for p in range(P):
        w = ops.Q4Tensor.from_numpy(wq[p * n:(p + 1) * n], ws[p * n:(p + 1) * n], K, G)
        got = host(ops.gemv(w, a))
        assert np.array_equal(got.view(np.uint32), want[:, p * n:(p + 1) * n].view(np.uint32)), f"shard {p}"


@pytest.mark.parametrize("M", [1, 8])
def test_lm_head_vocab_shards(M):
    P, K, V = 8, 2048, 151936
    n = V // P
    note(f"lm_head vocab shards P={P} ({n} rows each) M={M}")
    rng = np.random.default_rng(200 + M)
    wq, ws = ref.make_weight(rng, V, K, G)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    # an exact tie across shards: the winner's row copied half a vocabulary away
    win = int(orc.argmax(orc.linear(wq, ws, K, G, xq[:1], dx[:1], xs[:1]))[0])
    twin = (win + V // 2) % V
    wq[twin], ws[twin] = wq[win], ws[win]
    logits = orc.linear(wq, ws, K, G, xq, dx, xs)
    want = orc.argmax(logits)
    assert want[0] == min(win, twin)

    a = ops.Acts(dev(xq), dev(dx), dev(xs), K, G)
    work = ops.lm_head_workspace()
    best_val = np.full(M, -np.inf, np.float32)
    best_idx = np.zeros(M, np.uint32)
    for p in range(P):
        r0 = p * n
        w = ops.Q4Tensor.from_numpy(wq[r0:r0 + n], ws[r0:r0 + n], K, G)
        ids = dev(np.arange(r0, r0 + n, dtype=np.uint32).view(np.int32))
        lg = torch.empty((M, n), dtype=torch.float32, device=DEV)
        tok = host(ops.lm_head_argmax(w, a, ids=ids, logits=lg, workspace=work)).astype(np.uint32)
        lgh = host(lg)
        assert np.array_equal(lgh.view(np.uint32), logits[:, r0:r0 + n].view(np.uint32)), f"shard {p} logits"
        assert np.array_equal(tok, orc.argmax(logits[:, r0:r0 + n]) + r0), f"shard {p} token"
        # host stand-in for the all-gather of (logit, index) keys
        val = lgh[np.arange(M), tok - r0]
        take = (val > best_val) | ((val == best_val) & (tok < best_idx))
        best_val = np.where(take, val, best_val)
        best_idx = np.where(take, tok, best_idx)
    assert np.array_equal(best_idx, want)


def test_mlp_shards():
    P, hd, F = 8, 2048, 6144
    n = F // P
    note(f"mlp shards P={P}: gate_up {2 * n} rows, down K={n}")
    rng = np.random.default_rng(300)
    wgu, sgu = ref.make_weight(rng, 2 * F, hd, G)
    wd, sd = ref.make_weight(rng, hd, F, G)
    x = ref.make_activations(rng, 1, hd)
    resid = rng.normal(size=(1, hd)).astype(np.float32)
    xq, dx, xs = orc.quant_act(x, None, G)
    a = ops.Acts(dev(xq), dev(dx), dev(xs), hd, G)
    # the unsharded gate_up on the GPU (mode 2 agrees with the oracle within
    # rel 1e-5: device expf), whose rows each shard must reproduce bit for bit
    h_want = host(ops.gemv(ops.Q4Tensor.from_numpy(wgu, sgu, hd, G), a, mode=2))
    assert rel_err(h_want, orc.linear(wgu, sgu, hd, G, xq, dx, xs, mode=2)) < 1e-5
    hq, hdx, hxs = orc.quant_act(h_want, None, G)
    y_full = orc.linear(wd, sd, F, G, hq, hdx, hxs, mode=1, y=resid)

    y = dev(resid)
    y_want = resid.copy()
    for p in range(P):
        c0, c1 = p * n, (p + 1) * n
        # gate_up along N: this shard's gate rows, then its up rows
        q = np.concatenate([wgu[c0:c1], wgu[F + c0:F + c1]])
        s = np.concatenate([sgu[c0:c1], sgu[F + c0:F + c1]])
        h = host(ops.gemv(ops.Q4Tensor.from_numpy(q, s, hd, G), a, mode=2))
        assert np.array_equal(h.view(np.uint32), h_want[:, c0:c1].view(np.uint32)), f"shard {p} h"
        # down along K: the slice's codes under the token's global scale
        qd = np.ascontiguousarray(wd[:, c0 // 8:c1 // 8])
        sdp = np.ascontiguousarray(sd[:, c0 // G:c1 // G])
        hp = (np.ascontiguousarray(hq[:, c0:c1]), hdx, np.ascontiguousarray(hxs[:, c0 // G:c1 // G]))
        ops.gemv(ops.Q4Tensor.from_numpy(qd, sdp, n, G), ops.Acts(dev(hp[0]), dev(hp[1]), dev(hp[2]), n, G),
                 mode=1, y=y)
        y_want = orc.linear(qd, sdp, n, G, *hp, mode=1, y=y_want)
    got = host(y)
    assert np.array_equal(got.view(np.uint32), y_want.view(np.uint32))
    assert rel_err(got - resid, y_full - resid) < 1e-5
