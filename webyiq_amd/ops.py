"""Host-side operator API over the C ABI, on torch device tensors.

Mirrors the linear-layer operator interface of webyIQ's graph builder
(crates/engine/src/graph.rs:186-222, 476-486):

  reference (Rust)                                  here
  Builder::w(name) -> "{name}.q" / "{name}.s"      Weights.w(name) -> Q4Tensor
  Builder::quant(name, k, eps, x, norm, .., xq, xs) quant(x, norm, eps, GA, G) -> Acts
  Builder::gemv(name, w, k, n, mode, t, xq, xs, y)  gemv(w, acts, mode, y)
  Builder::gemm(name, w, k, n, mode, xq, xs, y, p)  gemm(w, acts, mode, y)
  Builder::matmul(path, ...)                        matmul(path, w, acts, mode, y)
  head_ops: quant + gemv(lm_head) + argmax          lm_head_argmax(w, acts, ids)

Errors raise WqError carrying the C status and message, as the Rust builder
returns Err(String).  Everything runs on the caller's current torch stream;
torch only provides device memory and streams.
"""
import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import (MODE_ACCUMULATE, MODE_SILU_MUL, MODE_STORE, PATH_DECODE,  # noqa: F401
                   PATH_PREFILL, PATH_SPEC, WqError)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


@dataclass
class Q4Tensor:
    """A packed int4 linear weight: `.q` u32 [rows, K/8] and `.s` u32 [rows, K/G]
    (tools/convert.py:8-12), held as int32 device tensors of the same bits."""
    q: torch.Tensor
    s: torch.Tensor
    K: int
    G: int

    @property
    def rows(self):
        return self.q.shape[0]

    @staticmethod
    def from_numpy(wq, ws, K, G, device="cuda"):
        q = torch.from_numpy(wq.view("int32")).to(device)
        s = torch.from_numpy(ws.view("int32")).to(device)
        return Q4Tensor(q, s, K, G)


class Weights(dict):
    """Named tensor map with the engine's lookup rule (graph.rs:186-188)."""

    def w(self, name) -> Q4Tensor:
        if name not in self:
            raise KeyError(f"missing tensor {name}")
        return self[name]


@dataclass
class Acts:
    """Quantised activations: xq i8 [M, K], dx f32 [M, K/GA], xs i32 [M, K/Ge]."""
    xq: torch.Tensor
    dx: torch.Tensor
    xs: torch.Tensor
    GA: int
    G: int

    @property
    def M(self):
        return self.xq.shape[0]

    @property
    def K(self):
        return self.xq.shape[1]


def empty_acts(M, K, GA=None, G=128, device="cuda"):
    GA = K if GA is None else GA
    Ge = min(G, GA)
    return Acts(torch.empty((M, K), dtype=torch.int8, device=device),
                torch.empty((M, K // GA), dtype=torch.float32, device=device),
                torch.empty((M, K // Ge), dtype=torch.int32, device=device), GA, G)


def quant(x, norm=None, eps=1e-6, GA=None, G=128, out: Optional[Acts] = None, stream=None) -> Acts:
    """Per-token (GA=None) or per-32 int8 quantisation of x f32 [M, K]
    (Builder::quant, quant.wgsl), optional RMSNorm with weight `norm`."""
    if x.dim() == 1:
        x = x[None]
    M, K = x.shape
    a = out if out is not None else empty_acts(M, K, GA, G, x.device)
    _lib.call("wq_quant_act", _stream(stream), _ptr(x), _ptr(norm), float(eps), M, K,
              a.GA, a.G, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs))
    return a


def _out(y, M, N, device, mode):
    if y is None:
        if mode == MODE_ACCUMULATE:
            raise ValueError("mode 1 (y += W x) needs y")
        y = torch.empty((M, N), dtype=torch.float32, device=device)
    return y


def _nrows(w, mode):
    return w.rows // 2 if mode == MODE_SILU_MUL else w.rows


def _linear(fn, w: Q4Tensor, a: Acts, mode, y, stream, acc=None):
    N = _nrows(w, mode)
    y = _out(y, a.M, N, a.xq.device, mode)
    args = [_stream(stream), _ptr(w.q), _ptr(w.s), N, w.K, w.G, _ptr(a.xq), _ptr(a.dx),
            _ptr(a.xs), a.M, a.GA, mode, _ptr(y)]
    if acc is not None:
        args.append(_ptr(acc))
    _lib.call(fn, *args)
    return y


def gemv(w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None):
    """Decode GEMV, M <= 8 (Builder::gemv, gemv_q4q8.wgsl)."""
    return _linear("wq_gemv", w, a, mode, y, stream)


def quant_gemv(w: Q4Tensor, x, norm=None, eps=1e-6, mode=MODE_STORE, y=None, out: Optional[Acts] = None,
               stream=None):
    """quant (per token) then gemv, M <= 8, in one launch for M <= 2; returns
    (y, the quantised activations) -- the norm_quant -> matmul pairs of the
    decode layer (graph.rs:266-269, 323-326)."""
    if x.dim() == 1:
        x = x[None]
    M, K = x.shape
    a = out if out is not None else empty_acts(M, K, None, w.G, x.device)
    if a.GA != K or a.G != w.G:
        raise ValueError("quant_gemv writes per-token activations for the weight's group")
    N = _nrows(w, mode)
    y = _out(y, M, N, x.device, mode)
    _lib.call("wq_quant_gemv", _stream(stream), _ptr(x), _ptr(norm), float(eps), _ptr(w.q), _ptr(w.s), N,
              w.K, w.G, M, mode, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), _ptr(y))
    return y, a


def gemm(w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None):
    """Prefill GEMM on int8 MFMA (Builder::gemm, gemm_q4q8.wgsl)."""
    return _linear("wq_gemm", w, a, mode, y, stream)


def matmul(path, w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None):
    """Builder::matmul: GEMM for the prefill path, GEMV otherwise."""
    N = _nrows(w, mode)
    y = _out(y, a.M, N, a.xq.device, mode)
    _lib.call("wq_matmul", _stream(stream), int(path), _ptr(w.q), _ptr(w.s), N, w.K, w.G,
              _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), a.M, a.GA, mode, _ptr(y))
    return y


def group_sums(path, w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None):
    """Run the GEMV (path != PREFILL) or GEMM kernel and return (y, A) with the
    exact int32 group sums A [M, rows, K/Ge] that the kernel folded into y."""
    Ge = min(w.G, a.GA)
    acc = torch.empty((a.M, w.rows, w.K // Ge), dtype=torch.int32, device=a.xq.device)
    fn = "wq_gemm_debug_acc" if path == PATH_PREFILL else "wq_gemv_debug_acc"
    y = _linear(fn, w, a, mode, y, stream, acc)
    return y, acc


def argmax(logits, ids=None, out=None, stream=None):
    """Greedy token per row (argmax.wgsl): ties to the lowest index."""
    if logits.dim() == 1:
        logits = logits[None]
    M, V = logits.shape
    out = torch.empty(M, dtype=torch.int32, device=logits.device) if out is None else out
    _lib.call("wq_argmax", _stream(stream), _ptr(logits), M, V, _ptr(ids), _ptr(out))
    return out


def lm_head_workspace(device="cuda", stream=None):
    n = _lib.load().wq_lm_head_workspace_bytes()
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.call("wq_workspace_clear", _stream(stream), _ptr(ws), n)
    return ws


def lm_head_argmax(w: Q4Tensor, a: Acts, ids=None, logits=None, workspace=None, out=None,
                   stream=None):
    """Fused lm_head GEMV + greedy argmax (head_ops' gemv + argmax in one launch)."""
    if workspace is None:
        workspace = lm_head_workspace(a.xq.device, stream)
    out = torch.empty(a.M, dtype=torch.int32, device=a.xq.device) if out is None else out
    _lib.call("wq_lm_head_argmax", _stream(stream), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G,
              _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), a.M, a.GA, _ptr(ids), _ptr(logits),
              _ptr(out), _ptr(workspace), workspace.numel())
    return out


def embed(w: Q4Tensor, tok, out=None, stream=None):
    """int4 embedding lookup (embed.wgsl): x[m] = dequantised row tok[m]."""
    M = tok.numel()
    x = torch.empty((M, w.K), dtype=torch.float32, device=tok.device) if out is None else out
    _lib.call("wq_embed", _stream(stream), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G, _ptr(tok), M, _ptr(x))
    return x


def mtp_in(emb, x, norm_f, norm_e, norm_h, eps=1e-6, out: Optional[Acts] = None, stream=None) -> Acts:
    """The MTP fc input (mtp_in.wgsl): per token, [quant(norm_e(emb)) |
    quant(norm_h(norm_f(x)))] as one [M, 2K] row with per-32 scales."""
    if emb.dim() == 1:
        emb, x = emb[None], x[None]
    M, K = x.shape
    a = out if out is not None else empty_acts(M, 2 * K, GA=32, G=32, device=x.device)
    _lib.call("wq_mtp_in", _stream(stream), _ptr(emb), _ptr(x), _ptr(norm_f), _ptr(norm_e), _ptr(norm_h),
              float(eps), M, K, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs))
    return a


def attn_combine(part, pos, gate=None, gate_stride=0, G=128, out: Optional[Acts] = None, stream=None) -> Acts:
    """Merge flash-decoding partials part f32 [M, H, nch, D + 2] into the o
    projection's int8 input (attn_combine.wgsl), per-32 scales; optional
    Qwen3.5 gate rows (gate of head h at h*2D + D of a token's row)."""
    M, H, nch, D2 = part.shape
    D = D2 - 2
    a = out if out is not None else empty_acts(M, H * D, GA=32, G=G, device=part.device)
    _lib.call("wq_attn_combine", _stream(stream), _ptr(part), M, H, D, nch, int(pos), _ptr(gate),
              int(gate_stride), _ptr(a.xq), _ptr(a.dx), _ptr(a.xs))
    return a


def gather_rows(w: Q4Tensor, ids, stream=None) -> Q4Tensor:
    """Packed rows ids of w as a new Q4Tensor (gather_rows.wgsl: the reduced
    draft lm_head)."""
    R = ids.numel()
    dq = torch.empty((R, w.K // 8), dtype=torch.int32, device=ids.device)
    ds = torch.empty((R, w.K // w.G), dtype=torch.int32, device=ids.device)
    _lib.call("wq_gather_rows", _stream(stream), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G, _ptr(ids), R,
              _ptr(dq), _ptr(ds))
    return Q4Tensor(dq, ds, w.K, w.G)
