"""ctypes binding of the C oracle (q4q8_oracle.c).  TEST INFRASTRUCTURE ONLY.

Every function takes and returns numpy arrays in the layouts of the C-ABI:
  wq u32 [N, K/8], ws u32 [N, K/G], xq i8 [M, K], dx f32 [M, K/GA],
  xs i32 [M, K/Ge] with Ge = min(G, GA), y f32 [M, N].
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_q4q8.so")
_lib = None


def build():
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        src = os.path.join(_HERE, "q4q8_oracle.c")
        if not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        i32 = ctypes.c_int
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f32_to_f16_array.argtypes = [P, P, i64]
        L.or_q4_quantize.argtypes = [P, i64, i64, i32, P, P, P]
        L.or_q4_pack.argtypes = [P, P, P, i64, i64, i32, P, P]
        L.or_q4_unpack.argtypes = [P, i64, i64, P]
        L.or_quant_act.argtypes = [P, P, ctypes.c_float, i64, i64, i32, i32, P, P, P]
        L.or_group_acc.argtypes = [P, i64, i64, i32, P, i64, P]
        L.or_linear.argtypes = [P, P, i64, i64, i32, P, P, P, i64, i32, i32, P]
        L.or_linear.restype = ctypes.c_int
        L.or_argmax.argtypes = [P, i64, i64, P, P]
        L.or_embed.argtypes = [P, P, i64, i64, i32, P, i64, P]
        L.or_gather_rows.argtypes = [P, P, i64, i64, i32, P, i64, P, P]
        L.or_mtp_in.argtypes = [P, P, P, P, P, ctypes.c_float, i64, i64, P, P, P]
        L.or_attn_combine.argtypes = [P, i64, i64, i64, i64, i64, P, i64, P, P, P]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def f32_to_f16_bits(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h):
    return np.array([lib().or_f16_to_f32(int(v)) for v in np.asarray(h).ravel()],
                    np.float32).reshape(np.shape(h))


def q4_quantize(w, G, want_deq=False):
    """RTN int4 (tools/convert.py:78-106, search=False) -> (wq, ws[, deq])."""
    w = _c(w, np.float32)
    N, K = w.shape
    assert K % G == 0 and G % 8 == 0
    wq = np.empty((N, K // 8), np.uint32)
    ws = np.empty((N, K // G), np.uint32)
    deq = np.empty((N, K), np.float32) if want_deq else None
    lib().or_q4_quantize(_p(w), N, K, G, _p(wq), _p(ws), _p(deq))
    return (wq, ws, deq) if want_deq else (wq, ws)


def q4_pack(q, scale_bits, min_bits, G):
    q = _c(q, np.uint8)
    N, K = q.shape
    sc = _c(scale_bits, np.uint16)
    mn = _c(min_bits, np.uint16)
    wq = np.empty((N, K // 8), np.uint32)
    ws = np.empty((N, K // G), np.uint32)
    lib().or_q4_pack(_p(q), _p(sc), _p(mn), N, K, G, _p(wq), _p(ws))
    return wq, ws


def q4_unpack(wq, K):
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    q = np.empty((N, K), np.uint8)
    lib().or_q4_unpack(_p(wq), N, K, _p(q))
    return q


def ge_of(G, GA):
    return min(G, GA)


def quant_act(x, GA=None, G=128, norm_w=None, eps=1e-6):
    """Activation quantiser -> (xq i8 [M,K], dx f32 [M,K/GA], xs i32 [M,K/Ge]).
    GA=None means per token (GA = K)."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    M, K = x.shape
    GA = K if GA is None else GA
    Ge = ge_of(G, GA)
    xq = np.empty((M, K), np.int8)
    dx = np.empty((M, K // GA), np.float32)
    xs = np.empty((M, K // Ge), np.int32)
    nw = None if norm_w is None else _c(norm_w, np.float32)
    lib().or_quant_act(_p(x), _p(nw), ctypes.c_float(eps), M, K, GA, G, _p(xq), _p(dx), _p(xs))
    return xq, dx, xs


def group_acc(wq, K, Ge, xq):
    """Exact int32 group accumulators A [M, N, K/Ge]."""
    wq = _c(wq, np.uint32)
    xq = _c(xq, np.int8)
    N = wq.shape[0]
    M = xq.shape[0]
    acc = np.empty((M, N, K // Ge), np.int32)
    lib().or_group_acc(_p(wq), N, K, Ge, _p(xq), M, _p(acc))
    return acc


def linear(wq, ws, K, G, xq, dx, xs, mode=0, y=None, GA=None):
    """Canonical-order linear layer (modes 0/1/2) -> y f32 [M, N]."""
    wq = _c(wq, np.uint32)
    ws = _c(ws, np.uint32)
    xq = _c(xq, np.int8)
    dx = _c(dx, np.float32)
    xs = _c(xs, np.int32)
    M = xq.shape[0]
    GA = K if GA is None else GA
    rows = wq.shape[0]
    N = rows // 2 if mode == 2 else rows
    if mode == 1:
        assert y is not None
        out = _c(y, np.float32).copy()
    else:
        out = np.zeros((M, N), np.float32)
    rc = lib().or_linear(_p(wq), _p(ws), N, K, G, _p(xq), _p(dx), _p(xs), M, GA, mode, _p(out))
    if rc != 0:
        raise ValueError("oracle.linear: bad arguments")
    return out


def argmax(logits, ids=None):
    logits = _c(logits, np.float32)
    if logits.ndim == 1:
        logits = logits[None]
    M, N = logits.shape
    out = np.empty(M, np.uint32)
    idsa = None if ids is None else _c(ids, np.uint32)
    lib().or_argmax(_p(logits), M, N, _p(idsa), _p(out))
    return out


def embed(wq, ws, K, G, tok):
    wq = _c(wq, np.uint32)
    ws = _c(ws, np.uint32)
    tok = _c(tok, np.uint32).reshape(-1)
    x = np.empty((tok.size, K), np.float32)
    lib().or_embed(_p(wq), _p(ws), wq.shape[0], K, G, _p(tok), tok.size, _p(x))
    return x


def gather_rows(wq, ws, K, G, ids):
    wq = _c(wq, np.uint32)
    ws = _c(ws, np.uint32)
    ids = _c(ids, np.uint32).reshape(-1)
    dq = np.empty((ids.size, K // 8), np.uint32)
    ds = np.empty((ids.size, K // G), np.uint32)
    lib().or_gather_rows(_p(wq), _p(ws), wq.shape[0], K, G, _p(ids), ids.size, _p(dq), _p(ds))
    return dq, ds


def mtp_in(emb, x, nf, ne, nh, eps=1e-6):
    """MTP input stage -> (xq i8 [M, 2K], dx f32 [M, 2K/32], xs i32 [M, 2K/32])."""
    emb = _c(np.atleast_2d(emb), np.float32)
    x = _c(np.atleast_2d(x), np.float32)
    M, K = x.shape
    xq = np.empty((M, 2 * K), np.int8)
    dx = np.empty((M, 2 * K // 32), np.float32)
    xs = np.empty((M, 2 * K // 32), np.int32)
    nf, ne, nh = (_c(a, np.float32) for a in (nf, ne, nh))
    lib().or_mtp_in(_p(emb), _p(x), _p(nf), _p(ne), _p(nh), ctypes.c_float(eps), M, K, _p(xq), _p(dx), _p(xs))
    return xq, dx, xs


def attn_combine(part, pos, gate=None, gate_stride=0):
    """Chunk merge + per-32 quant -> (xq i8 [M, H*D], dx f32 [M, H*D/32], xs i32 [M, H*D/32])."""
    part = _c(part, np.float32)
    M, H, nch, D2 = part.shape
    D = D2 - 2
    K = H * D
    xq = np.empty((M, K), np.int8)
    dx = np.empty((M, K // 32), np.float32)
    xs = np.empty((M, K // 32), np.int32)
    g = None if gate is None else _c(gate, np.float32)
    lib().or_attn_combine(_p(part), M, H, D, nch, int(pos), _p(g), int(gate_stride), _p(xq), _p(dx), _p(xs))
    return xq, dx, xs
