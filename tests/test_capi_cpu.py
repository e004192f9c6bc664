"""C-ABI checks that need no GPU: the library loads, exports every entry
point the header declares, and rejects bad arguments on the host (before any
launch) with the documented status codes and messages -- the analogue of the
engine's host-side shape checks (graph.rs:368-380, manifest.rs:82-84)."""
import ctypes
import re

import pytest

from webyiq_amd import _lib

L = _lib.load()
A16 = ctypes.c_void_p(0x10000)  # aligned non-null dummies: validation fails before any use
A4 = ctypes.c_void_p(0x10004)


def declared_symbols():
    text = open(_lib.HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\*?(wq_[a-z_0-9]+)\(", text, re.M)))


def test_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) == 20
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.PROTOTYPES)
    assert L.wq_abi_version() == 2
    assert L.wq_lm_head_workspace_bytes() >= 72


def gemv(*, wq=A16, ws=A4, N=64, K=2048, G=128, xq=A16, dx=A4, xs=A4, M=1, GA=None, mode=0, y=A4,
         fn="wq_gemv", params=None, workspace=None, wbytes=0):
    GA = K if GA is None else GA
    extra = [params, workspace, wbytes] if fn == "wq_gemm" else []
    return getattr(L, fn)(None, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, *extra)


def err():
    return L.wq_last_error().decode()


@pytest.mark.parametrize("fn", ["wq_gemv", "wq_gemm"])
def test_linear_argument_errors(fn):
    assert gemv(wq=None, fn=fn) == _lib.WQ_EINVAL and "wq is NULL" in err()
    assert gemv(y=None, fn=fn) == _lib.WQ_EINVAL
    assert gemv(mode=3, fn=fn) == _lib.WQ_EINVAL and "unknown mode" in err()
    assert gemv(K=2000, fn=fn) == _lib.WQ_ESHAPE and "multiple of 128" in err()
    assert gemv(K=64, fn=fn) == _lib.WQ_ESHAPE
    assert gemv(G=64, fn=fn) == _lib.WQ_ESHAPE and "quant group" in err()
    assert gemv(GA=64, fn=fn) == _lib.WQ_ESHAPE and "activation group" in err()
    assert gemv(N=0, fn=fn) == _lib.WQ_ESHAPE
    assert gemv(M=0, fn=fn) == _lib.WQ_ESHAPE
    assert gemv(wq=A4, fn=fn) == _lib.WQ_EALIGN and "16-byte" in err()
    assert gemv(xq=ctypes.c_void_p(0x10008), fn=fn) == _lib.WQ_EALIGN
    assert gemv(ws=ctypes.c_void_p(0x10002), fn=fn) == _lib.WQ_EALIGN


def test_gemv_token_and_k_limits():
    assert gemv(M=9) == _lib.WQ_ESHAPE and "M = 9" in err()
    assert gemv(K=2048 * 9) == _lib.WQ_ESHAPE
    # the GEMM takes any M (and the same K) ...
    assert gemv(M=9, mode=7, fn="wq_gemm") == _lib.WQ_EINVAL
    # ... while each operand stays within 4 GiB of 32-bit staging offsets
    assert gemv(M=1 << 20, K=8192, fn="wq_gemm") == _lib.WQ_ESHAPE and "4 GiB" in err()
    assert gemv(N=1 << 20, K=8192, mode=2, fn="wq_gemm") == _lib.WQ_ESHAPE
    # the step parameters are device words read by the kernel: 4-byte aligned
    assert gemv(params=ctypes.c_void_p(0x10002), fn="wq_gemm") == _lib.WQ_EALIGN and "params" in err()
    # the split-K workspace is 256-byte aligned
    assert gemv(workspace=ctypes.c_void_p(0x10040), wbytes=1 << 20, fn="wq_gemm") == _lib.WQ_EALIGN
    assert "workspace" in err()


def test_gemm_workspace_bytes():
    """The split plan's workspace: zero for shapes that never split (short K,
    per-32 activations, grids that fill the chip), flags plus 128 x width
    partial sums per tile otherwise."""
    wsb = L.wq_gemm_workspace_bytes
    assert wsb(6144, 2048, 128, 1024, 2048, 0) == 0          # K = 2048: 16 steps
    assert wsb(2048, 6144, 128, 1024, 32, 0) == 0            # per-32 activations
    n = wsb(2048, 6144, 128, 1024, 6144, 0)                  # width 128 split in pairs
    tiles = 8 * 16
    assert n == ((tiles * 64 + 255) // 256) * 256 + tiles * 128 * 128 * 4
    m512 = wsb(2048, 6144, 128, 512, 6144, 1)               # width 64 split in pairs
    assert m512 == ((4 * 32 * 64 + 255) // 256) * 256 + 4 * 32 * 128 * 64 * 4
    assert wsb(2048, 6144, 64, 1024, 6144, 0) == 0           # unsupported group: no plan


def test_matmul_paths():
    args = [A16, A4, 64, 2048, 128, A16, A4, A4, 2, 2048, 0, A4, None]
    assert L.wq_matmul(None, 7, *args) == _lib.WQ_EINVAL and "unknown path" in err()
    assert L.wq_matmul(None, _lib.PATH_DECODE, *args) == _lib.WQ_ESHAPE and "M = 1" in err()


def test_quant_errors():
    q = L.wq_quant_act
    assert q(None, None, None, 1e-6, 1, 2048, 2048, 128, A16, A4, A4) == _lib.WQ_EINVAL
    assert q(None, A16, None, 1e-6, 1, 2000, 2000, 128, A16, A4, A4) == _lib.WQ_ESHAPE
    assert q(None, A16, None, 1e-6, 1, 2048, 64, 128, A16, A4, A4) == _lib.WQ_ESHAPE
    assert q(None, A4, None, 1e-6, 1, 2048, 2048, 128, A16, A4, A4) == _lib.WQ_EALIGN
    assert q(None, A16, A16, -1.0, 1, 2048, 2048, 128, A16, A4, A4) == _lib.WQ_EINVAL
    assert q(None, A16, None, 1e-6, 1, 2048, 2048, 128, A4, A4, A4) == _lib.WQ_EALIGN and "xq" in err()


def test_quant_gemv_errors():
    f = L.wq_quant_gemv

    def call(x=A16, nw=None, eps=1e-6, wq=A16, N=64, K=2048, G=128, M=1, mode=0, xq=A16, dx=A4, xs=A4, y=A4):
        return f(None, x, nw, eps, wq, A4, N, K, G, M, mode, xq, dx, xs, y)

    assert call(x=None) == _lib.WQ_EINVAL and "x is NULL" in err()
    assert call(xq=None) == _lib.WQ_EINVAL  # the activations are required outputs
    assert call(y=None) == _lib.WQ_EINVAL
    assert call(M=9) == _lib.WQ_ESHAPE and "M = 9" in err()
    assert call(M=0) == _lib.WQ_ESHAPE
    assert call(K=2000) == _lib.WQ_ESHAPE
    assert call(K=2048 * 9) == _lib.WQ_ESHAPE
    assert call(G=64) == _lib.WQ_ESHAPE
    assert call(x=A4) == _lib.WQ_EALIGN and "x not 16" in err()
    assert call(nw=A4) == _lib.WQ_EALIGN
    assert call(nw=A16, eps=-1.0) == _lib.WQ_EINVAL and "eps" in err()
    assert call(mode=3) == _lib.WQ_EINVAL


def test_argmax_and_lm_head_errors():
    assert L.wq_argmax(None, None, 1, 10, None, A4) == _lib.WQ_EINVAL
    assert L.wq_argmax(None, A4, 1, 0, None, A4) == _lib.WQ_ESHAPE
    lm = L.wq_lm_head_argmax
    base = [None, A16, A4, 1000, 2048, 128, A16, A4, A4, 1, 2048, None, None, A4]
    assert lm(*base, None, 128) == _lib.WQ_EWORKSPACE and "workspace" in err()
    assert lm(*base, A16, 8) == _lib.WQ_EWORKSPACE
    base[-1] = None
    assert lm(*base, A16, 128) == _lib.WQ_EINVAL and "tok_out" in err()
    assert L.wq_workspace_clear(None, None, 16) == _lib.WQ_EINVAL


def test_python_wrapper_raises_wq_error():
    with pytest.raises(_lib.WqError) as e:
        _lib.call("wq_gemv", None, None, A4, 64, 2048, 128, A16, A4, A4, 1, 2048, 0, A4)
    assert e.value.code == _lib.WQ_EINVAL and "wq is NULL" in e.value.message


def test_embed_and_gather_errors():
    e = L.wq_embed
    assert e(None, None, A4, 100, 2048, 32, A4, 1, A16) == _lib.WQ_EINVAL and "eq is NULL" in err()
    assert e(None, A16, A4, 100, 2000, 32, A4, 1, A16) == _lib.WQ_ESHAPE
    assert e(None, A16, A4, 100, 2048, 64, A4, 1, A16) == _lib.WQ_ESHAPE
    assert e(None, A16, A4, 0, 2048, 32, A4, 1, A16) == _lib.WQ_ESHAPE
    assert e(None, A16, A4, 100, 2048, 32, A4, 0, A16) == _lib.WQ_ESHAPE
    assert e(None, A16, A4, 100, 2048, 32, A4, 1, A4) == _lib.WQ_EALIGN
    g = L.wq_gather_rows
    assert g(None, A16, A4, 100, 2048, 128, None, 4, A16, A4) == _lib.WQ_EINVAL
    assert g(None, A16, A4, 100, 2048, 128, A4, 0, A16, A4) == _lib.WQ_ESHAPE
    assert g(None, A16, A4, 100, 2048, 128, A4, 4, A4, A4) == _lib.WQ_EALIGN


def mtp_in(*, emb=A16, x=A16, nf=A16, ne=A16, nh=A16, eps=1e-6, M=1, K=2048, xq=A16, dx=A4, xs=A4):
    return L.wq_mtp_in(None, emb, x, nf, ne, nh, eps, M, K, xq, dx, xs)


def test_mtp_in_argument_errors():
    assert mtp_in(nh=None) == _lib.WQ_EINVAL and "norm_h is NULL" in err()
    assert mtp_in(K=2000) == _lib.WQ_ESHAPE and "multiple of 128" in err()
    assert mtp_in(M=0) == _lib.WQ_ESHAPE
    assert mtp_in(eps=-1.0) == _lib.WQ_EINVAL and "eps" in err()
    assert mtp_in(emb=A4) == _lib.WQ_EALIGN and "emb not 16-byte" in err()
    assert mtp_in(xq=ctypes.c_void_p(0x10008)) == _lib.WQ_EALIGN


def combine(*, part=A4, M=1, H=16, D=128, nch=128, pos=0, gate=None, gs=0, xq=A16, dx=A4, xs=A4, params=None):
    return L.wq_attn_combine(None, part, M, H, D, nch, pos, gate, gs, xq, dx, xs, params)


def test_attn_combine_argument_errors():
    assert combine(part=None) == _lib.WQ_EINVAL and "part is NULL" in err()
    assert combine(D=96) == _lib.WQ_ESHAPE and "head dim" in err()
    assert combine(M=0) == _lib.WQ_ESHAPE and combine(H=0) == _lib.WQ_ESHAPE
    assert combine(nch=8193) == _lib.WQ_ESHAPE and "chunks" in err()
    assert combine(nch=4, pos=128) == _lib.WQ_ESHAPE and "context" in err()
    assert combine(nch=4, pos=126, M=3) == _lib.WQ_ESHAPE     # token 2 at position 128
    assert combine(pos=-1) == _lib.WQ_ESHAPE
    assert combine(gate=A4, gs=2 * 16 * 128 - 1) == _lib.WQ_ESHAPE and "gate_stride" in err()
    assert combine(xq=ctypes.c_void_p(0x10008)) == _lib.WQ_EALIGN
    assert combine(part=ctypes.c_void_p(0x10002)) == _lib.WQ_EALIGN
    # with device params the host pos is the bound: it is checked the same way
    assert combine(nch=4, pos=128, params=A4) == _lib.WQ_ESHAPE and "context" in err()
    assert combine(params=ctypes.c_void_p(0x10002)) == _lib.WQ_EALIGN and "params" in err()


def test_last_error_is_per_thread():
    """wq_last_error() is thread-local: two threads failing with different
    messages, interleaved (ctypes releases the GIL around each call), each
    read back their own."""
    import threading
    start = threading.Barrier(2)
    bad = []

    def worker(kind):
        start.wait()
        for _ in range(2000):
            if kind == 0:
                rc, want = gemv(K=2000), "multiple of 128"
            else:
                rc, want = gemv(mode=5), "unknown mode"
            if rc >= 0 or want not in err():
                bad.append((kind, rc, err()))
                return

    ts = [threading.Thread(target=worker, args=(k,)) for k in (0, 1)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not bad, bad[:3]
