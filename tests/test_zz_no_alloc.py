"""wq_lm_head_argmax_noalloc (the entry point for callers that cannot
allocate) against wq_lm_head_argmax with a caller workspace, both through the
C ABI: two calls in a row on the library's static scratch, the second with a
smaller input (fewer tokens, a shorter vocabulary), tokens and logits
bit-identical, and the tokens equal to the oracle's."""
import numpy as np
import pytest

from oracle import oracle as orc
from oracle import reference as ref

K, G = 2048, 128


def case(seed, M, V, mapped):
    rng = np.random.default_rng(seed)
    wq, ws = ref.make_weight(rng, V, K, G)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    logits = orc.linear(wq, ws, K, G, xq, dx, xs)
    win = int(orc.argmax(logits)[0])
    lo = max(0, win // 2 - 1)  # an exact tie below the winner
    wq[lo], ws[lo] = wq[win], ws[win]
    logits = orc.linear(wq, ws, K, G, xq, dx, xs)
    ids = np.sort(rng.choice(151936, V, replace=False)).astype(np.uint32) if mapped else None
    return wq, ws, xq, dx, xs, ids, logits, orc.argmax(logits, ids)


@pytest.mark.gpu
@pytest.mark.parametrize("order", ["noalloc_first", "workspace_first"])
def test_noalloc_matches_workspace_entry(order):
    import torch
    from webyiq_amd import ops

    # 8 tokens on the MFMA GEMV with the id map, then 3 tokens on the dot4 GEMV
    for seed, M, V, mapped in ((21, 8, 32768, True), (22, 3, 5000, False)):
        print(f"[case] noalloc lm_head M={M} V={V} mapped={mapped} ({order})", flush=True)
        wq, ws, xq, dx, xs, ids, logits_want, tok_want = case(seed, M, V, mapped)
        w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
        a = ops.Acts(*(torch.from_numpy(v).cuda() for v in (xq, dx, xs)), K, G)
        d_ids = torch.from_numpy(ids.view(np.int32)).cuda() if mapped else None
        lg0 = torch.empty((M, V), dtype=torch.float32, device="cuda")
        lg1 = torch.empty((M, V), dtype=torch.float32, device="cuda")
        wsp = ops.lm_head_workspace()
        if order == "noalloc_first":
            t1 = ops.lm_head_argmax_noalloc(w, a, ids=d_ids, logits=lg1)
            t0 = ops.lm_head_argmax(w, a, ids=d_ids, logits=lg0, workspace=wsp)
        else:
            t0 = ops.lm_head_argmax(w, a, ids=d_ids, logits=lg0, workspace=wsp)
            t1 = ops.lm_head_argmax_noalloc(w, a, ids=d_ids, logits=lg1)
        # the same call again without logits: the scratch was left zeroed
        t2 = ops.lm_head_argmax_noalloc(w, a, ids=d_ids)
        torch.cuda.synchronize()
        got0 = t0.cpu().numpy().astype(np.uint32)
        assert np.array_equal(got0, tok_want)
        assert np.array_equal(t1.cpu().numpy().astype(np.uint32), got0)
        assert np.array_equal(t2.cpu().numpy().astype(np.uint32), got0)
        assert np.array_equal(lg1.cpu().numpy().view(np.uint32), lg0.cpu().numpy().view(np.uint32))
        assert np.array_equal(lg0.cpu().numpy().view(np.uint32), logits_want.view(np.uint32))


def test_noalloc_rejects_too_many_tokens():
    """Host-side limit: the scratch holds keys for at most 8 tokens."""
    import ctypes

    from webyiq_amd import _lib
    lib = _lib.load()
    P = ctypes.c_void_p
    fake = P(1 << 20)  # never dereferenced: the call fails validation first
    rc = lib.wq_lm_head_argmax_noalloc(None, fake, fake, 1024, 2048, 128, fake, fake, fake, 9, 2048, None,
                                       None, fake)
    assert rc == _lib.WQ_ESHAPE
    assert b"8" in lib.wq_last_error()


@pytest.mark.gpu
def test_noalloc_reset_then_calls():
    """wq_lm_head_noalloc_reset zeroes the static array with the fill kernel
    (stream-ordered); calls after it still give the oracle's tokens."""
    import ctypes

    import torch
    from webyiq_amd import _lib, ops
    lib = _lib.load()
    print("[case] noalloc reset, then M=2 V=4096 twice", flush=True)
    wq, ws, xq, dx, xs, _, _, tok_want = case(23, 2, 4096, False)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = ops.Acts(*(torch.from_numpy(v).cuda() for v in (xq, dx, xs)), K, G)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.wq_lm_head_noalloc_reset(s) == _lib.WQ_OK, lib.wq_last_error()
    t1 = ops.lm_head_argmax_noalloc(w, a)
    assert lib.wq_lm_head_noalloc_reset(s) == _lib.WQ_OK, lib.wq_last_error()
    t2 = ops.lm_head_argmax_noalloc(w, a)
    torch.cuda.synchronize()
    assert np.array_equal(t1.cpu().numpy().astype(np.uint32), tok_want)
    assert np.array_equal(t2.cpu().numpy().astype(np.uint32), tok_want)


def test_noalloc_reset_without_gpu_reports_error():
    """Without a usable device the reset launches nothing and returns
    WQ_EHIP with the runtime's message (CPU-only check)."""
    import torch

    from webyiq_amd import _lib
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU test covers the reset")
    lib = _lib.load()
    rc = lib.wq_lm_head_noalloc_reset(None)
    assert rc == _lib.WQ_EHIP
    assert b"wq_lm_head_noalloc_reset" in lib.wq_last_error()
