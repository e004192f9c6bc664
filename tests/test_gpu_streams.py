"""Re-entrancy of the C ABI on the GPU: two host threads, each on its own
stream (default priority) with its own buffers and lm_head workspace, issue
quantiser -> GEMV -> fused lm_head argmax chains concurrently; every result
matches the oracle bit for bit.  The engine itself is single-threaded
(lib.rs:267-273); the ABI promises that calls from different threads on
different streams do not interfere, since its only global state is the
thread-local error message."""
import threading

import numpy as np
import pytest

from oracle import oracle as orc
from oracle import reference as ref

K, N, V, G = 2048, 1024, 8192, 128
ITERS = 50


def case(seed):
    rng = np.random.default_rng(seed)
    wq, ws = ref.make_weight(rng, N, K, G)
    hq, hs = ref.make_weight(rng, V, K, G)
    x = ref.make_activations(rng, 2, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    y = orc.linear(wq, ws, K, G, xq, dx, xs)
    tok = orc.argmax(orc.linear(hq, hs, K, G, xq, dx, xs))
    return wq, ws, hq, hs, x, xq, y, tok


@pytest.mark.gpu
def test_two_threads_two_streams():
    import torch
    from webyiq_amd import ops

    print("[case] two host threads, two streams", flush=True)
    cases = [case(s) for s in (11, 12)]
    errors = []

    def worker(i):
        try:
            wq, ws, hq, hs, x, xq, y_want, tok_want = cases[i]
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
                h = ops.Q4Tensor.from_numpy(hq, hs, K, G)
                xd = torch.from_numpy(x).cuda()
                wsp = ops.lm_head_workspace(stream=st)
                outs = []
                for _ in range(ITERS):
                    a = ops.quant(xd, G=G, stream=st)
                    y = ops.gemv(w, a, stream=st)
                    tok = ops.lm_head_argmax(h, a, workspace=wsp, stream=st)
                    outs.append((a.xq, y, tok))
                st.synchronize()
            for xq_d, y_d, tok_d in outs:
                assert np.array_equal(xq_d.cpu().numpy(), xq)
                assert np.array_equal(y_d.cpu().numpy().view(np.uint32), y_want.view(np.uint32))
                assert np.array_equal(tok_d.cpu().numpy().astype(np.uint32), tok_want)
        except Exception as e:  # reported by the main thread
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=worker, args=(i,)) for i in (0, 1)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


@pytest.mark.gpu
def test_non_current_stream_temporaries():
    """Ops called with stream= a stream that is not current: the default
    lm_head workspace (freed when the call returns) and the outputs are
    allocated on that stream, so the current stream's allocations cannot
    reuse them while the kernels are still queued.  Between the calls the
    current stream allocates and fills blocks of the workspace's size with
    ones; a reused, unzeroed workspace would corrupt the tokens."""
    import torch
    from webyiq_amd import ops

    print("[case] ops on a non-current stream, default workspace", flush=True)
    wq, ws, hq, hs, x, xq, y_want, tok_want = case(13)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    h = ops.Q4Tensor.from_numpy(hq, hs, K, G)
    xd = torch.from_numpy(x).cuda()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    nbytes = ops._lib.load().wq_lm_head_workspace_bytes()
    outs, junk = [], []
    for _ in range(ITERS):
        a = ops.quant(xd, G=G, stream=st)
        y = ops.gemv(w, a, stream=st)
        tok = ops.lm_head_argmax(h, a, stream=st)
        outs.append((a.xq, y, tok))
        junk.append(torch.ones(nbytes, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
    for xq_d, y_d, tok_d in outs:
        assert np.array_equal(xq_d.cpu().numpy(), xq)
        assert np.array_equal(y_d.cpu().numpy().view(np.uint32), y_want.view(np.uint32))
        assert np.array_equal(tok_d.cpu().numpy().astype(np.uint32), tok_want)
