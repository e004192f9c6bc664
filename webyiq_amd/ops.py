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
returns Err(String).  Tensor arguments are checked before anything is
launched (device, dtype, contiguity, size; ValueError otherwise): the C ABI
receives raw device pointers and cannot tell an int64 id tensor or a short
output buffer from a valid one.

Streams: every op runs on `stream` when given, else on the caller's current
torch stream.  Outputs and temporaries an op allocates are allocated while
that stream is current, so torch's caching allocator orders their reuse
after the op's kernels on that stream.  torch only provides device memory
and streams.
"""
import contextlib
import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import (MODE_ACCUMULATE, MODE_SILU_MUL, MODE_STORE, PATH_DECODE,  # noqa: F401
                   PATH_PREFILL, PATH_SPEC, WqError)

_ID_DTYPES = (torch.int32,) + ((torch.uint32,) if hasattr(torch, "uint32") else ())


def _check(t, name, dtypes, shape=None, min_numel=None, device=None):
    """Validate a tensor handed to a kernel; returns it unchanged."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if not isinstance(dtypes, tuple):
        dtypes = (dtypes,)
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {' or '.join(str(d) for d in dtypes)}")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: on {t.device}, the other operands are on {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: not contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if min_numel is not None and t.numel() < min_numel:
        raise ValueError(f"{name}: {t.numel()} elements, at least {min_numel} required")
    return t


def _cuda(t, name):
    """The operands share one device (checked per operand); it must be a GPU."""
    if t.device.type != "cuda":
        raise ValueError(f"{name}: on {t.device}, expected a cuda tensor")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _on(stream):
    """Make `stream` current for the op's allocations and launches."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _cur():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


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

    def check(self, name="w"):
        if self.G <= 0 or self.K % self.G or self.K % 8:
            raise ValueError(f"{name}: K = {self.K} is not a multiple of the group {self.G}")
        _check(self.q, f"{name}.q", torch.int32, shape=(self.rows, self.K // 8))
        _check(self.s, f"{name}.s", torch.int32, shape=(self.rows, self.K // self.G), device=self.q.device)
        return self


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

    def check(self, name="acts"):
        if self.xq.dim() != 2:
            raise ValueError(f"{name}.xq: expected [M, K], got shape {tuple(self.xq.shape)}")
        M, K = self.xq.shape
        Ge = min(self.G, self.GA)
        if self.GA <= 0 or Ge <= 0 or K % self.GA or K % Ge:
            raise ValueError(f"{name}: K = {K} is not a multiple of GA = {self.GA} and Ge = {Ge}")
        _check(self.xq, f"{name}.xq", torch.int8)
        d = self.xq.device
        _check(self.dx, f"{name}.dx", torch.float32, shape=(M, K // self.GA), device=d)
        _check(self.xs, f"{name}.xs", torch.int32, shape=(M, K // Ge), device=d)
        return self


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
    _check(x, "x", torch.float32)
    M, K = x.shape
    if norm is not None:
        _check(norm, "norm", torch.float32, shape=(K,), device=x.device)
    with _on(stream):
        a = out if out is not None else empty_acts(M, K, GA, G, x.device)
        a.check("out")
        if a.xq.shape != (M, K) or a.xq.device != x.device:
            raise ValueError(f"out: activations of shape {tuple(a.xq.shape)} for x of shape {(M, K)}")
        _cuda(x, "x")
        _lib.call("wq_quant_act", _cur(), _ptr(x), _ptr(norm), float(eps), M, K,
                  a.GA, a.G, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs))
    return a


def _nrows(w, mode):
    return w.rows // 2 if mode == MODE_SILU_MUL else w.rows


def _out(y, M, N, device, mode):
    if y is None:
        if mode == MODE_ACCUMULATE:
            raise ValueError("mode 1 (y += W x) needs y")
        y = torch.empty((M, N), dtype=torch.float32, device=device)
    return _check(y, "y", torch.float32, shape=(M, N), device=device)


def _check_linear(w: Q4Tensor, a: Acts):
    w.check("w")
    a.check("acts")
    # xs holds one sum per accumulation group Ge = min(G, GA) of the weight's G
    if a.K != w.K or min(a.G, a.GA) != min(w.G, a.GA):
        raise ValueError(f"acts (K = {a.K}, G = {a.G}, GA = {a.GA}) do not match the weight "
                         f"(K = {w.K}, G = {w.G})")
    if a.xq.device != w.q.device:
        raise ValueError(f"acts on {a.xq.device}, the weight on {w.q.device}")


def make_params(pos=0, seq_len=0, m=0, slot=0, device="cuda"):
    """The step parameters as a device tensor u32[4] {pos, seq_len, m, slot}
    (wq_params; the reference's Params uniform, gemm_q4q8.wgsl:8-13).  Kernels
    that take it read it when they run, so a recorded call follows its
    contents; rewrite it with set_params (a copy on the stream)."""
    return torch.tensor([pos, seq_len, m, slot], dtype=torch.int32, device=device)


def set_params(params, pos=0, seq_len=0, m=0, slot=0, stream=None):
    """Overwrite a make_params tensor in stream order (host -> device copy)."""
    _check_params(params, params.device)
    src = torch.tensor([pos, seq_len, m, slot], dtype=torch.int32)
    with _on(stream):
        params.copy_(src, non_blocking=False)
    return params


def _check_params(params, device):
    if params is None:
        return None
    return _check(params, "params", _ID_DTYPES, shape=(4,), device=device)


def _linear(fn, w: Q4Tensor, a: Acts, mode, y, stream, acc=None, params=None, pass_params=False, workspace=None):
    _check_linear(w, a)
    N = _nrows(w, mode)
    _check_params(params, a.xq.device)
    with _on(stream):
        y = _out(y, a.M, N, a.xq.device, mode)
        if acc is not None:
            _check(acc, "acc", torch.int32, shape=(a.M, w.rows, w.K // min(w.G, a.GA)), device=a.xq.device)
        _cuda(w.q, "w.q")
        args = [_cur(), _ptr(w.q), _ptr(w.s), N, w.K, w.G, _ptr(a.xq), _ptr(a.dx),
                _ptr(a.xs), a.M, a.GA, mode, _ptr(y)]
        if acc is not None:
            args.append(_ptr(acc))
        if pass_params:
            args.append(_ptr(params))
            if workspace is not None:
                _check(workspace, "workspace", torch.uint8, device=a.xq.device)
                args += [_ptr(workspace), workspace.numel()]
            else:
                args += [None, 0]
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
    w.check("w")
    _check(x, "x", torch.float32, device=w.q.device)
    M, K = x.shape
    if K != w.K:
        raise ValueError(f"x has K = {K}, the weight {w.K}")
    if norm is not None:
        _check(norm, "norm", torch.float32, shape=(K,), device=x.device)
    with _on(stream):
        a = out if out is not None else empty_acts(M, K, None, w.G, x.device)
        a.check("out")
        if a.GA != K or a.G != w.G or a.xq.shape != (M, K):
            raise ValueError("quant_gemv writes per-token activations for the weight's group")
        N = _nrows(w, mode)
        y = _out(y, M, N, x.device, mode)
        _cuda(x, "x")
        _lib.call("wq_quant_gemv", _cur(), _ptr(x), _ptr(norm), float(eps), _ptr(w.q), _ptr(w.s), N,
                  w.K, w.G, M, mode, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), _ptr(y))
    return y, a


def gemm(w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None, params=None, workspace=None):
    """Prefill GEMM on int8 MFMA (Builder::gemm, gemm_q4q8.wgsl).  params
    (make_params, optional): a.M is then the capacity and the kernel covers
    the params' m tokens, read when it runs; rows past them are not written.
    workspace (gemm_workspace, optional): lets the library split K between
    workgroup pairs on the shapes where that pays."""
    return _linear("wq_gemm", w, a, mode, y, stream, params=params, pass_params=True, workspace=workspace)


def gemm_workspace(N, K, G, M, GA=None, mode=MODE_STORE, device="cuda"):
    """A zeroed uint8 workspace of wq_gemm_workspace_bytes for this shape (a
    one-byte tensor when the shape never splits); reusable by later calls of
    the same or a smaller shape, not by overlapping ones."""
    nbytes = int(_lib.load().wq_gemm_workspace_bytes(N, K, G, M, K if GA is None else GA, mode))
    # 256-byte aligned: the caching allocator hands out 512-byte aligned blocks
    return torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)


def matmul(path, w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None, params=None):
    """Builder::matmul: GEMM for the prefill path (with params), GEMV otherwise."""
    _check_linear(w, a)
    N = _nrows(w, mode)
    _check_params(params, a.xq.device)
    with _on(stream):
        y = _out(y, a.M, N, a.xq.device, mode)
        _cuda(w.q, "w.q")
        _lib.call("wq_matmul", _cur(), int(path), _ptr(w.q), _ptr(w.s), N, w.K, w.G,
                  _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), a.M, a.GA, mode, _ptr(y), _ptr(params))
    return y


def group_sums(path, w: Q4Tensor, a: Acts, mode=MODE_STORE, y=None, stream=None):
    """Run the GEMV (path != PREFILL) or GEMM kernel and return (y, A) with the
    exact int32 group sums A [M, rows, K/Ge] that the kernel folded into y."""
    Ge = min(w.G, a.GA)
    with _on(stream):
        acc = torch.empty((a.M, w.rows, w.K // Ge), dtype=torch.int32, device=a.xq.device)
        fn = "wq_gemm_debug_acc" if path == PATH_PREFILL else "wq_gemv_debug_acc"
        y = _linear(fn, w, a, mode, y, None, acc)
    return y, acc


def _tok_out(out, M, device):
    if out is None:
        return torch.empty(M, dtype=torch.int32, device=device)
    return _check(out, "out", _ID_DTYPES, shape=(M,), device=device)


def argmax(logits, ids=None, out=None, stream=None):
    """Greedy token per row (argmax.wgsl): ties to the lowest index."""
    if logits.dim() == 1:
        logits = logits[None]
    _check(logits, "logits", torch.float32)
    M, V = logits.shape
    if ids is not None:
        _check(ids, "ids", _ID_DTYPES, min_numel=V, device=logits.device)
    with _on(stream):
        out = _tok_out(out, M, logits.device)
        _cuda(logits, "logits")
        _lib.call("wq_argmax", _cur(), _ptr(logits), M, V, _ptr(ids), _ptr(out))
    return out


def lm_head_workspace(device="cuda", stream=None):
    n = _lib.load().wq_lm_head_workspace_bytes()
    with _on(stream):
        ws = torch.empty(n, dtype=torch.uint8, device=device)
        _lib.call("wq_workspace_clear", _cur(), _ptr(ws), n)
    return ws


def lm_head_argmax(w: Q4Tensor, a: Acts, ids=None, logits=None, workspace=None, out=None,
                   stream=None):
    """Fused lm_head GEMV + greedy argmax (head_ops' gemv + argmax in one launch).
    Without `workspace` a fresh one is allocated (and cleared) on the op's stream."""
    _check_linear(w, a)
    d = a.xq.device
    if ids is not None:
        _check(ids, "ids", _ID_DTYPES, min_numel=w.rows, device=d)
    if logits is not None:
        _check(logits, "logits", torch.float32, shape=(a.M, w.rows), device=d)
    with _on(stream):
        if workspace is None:
            workspace = lm_head_workspace(d)
        _check(workspace, "workspace", torch.uint8, min_numel=_lib.load().wq_lm_head_workspace_bytes(), device=d)
        out = _tok_out(out, a.M, d)
        _cuda(w.q, "w.q")
        _lib.call("wq_lm_head_argmax", _cur(), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G,
                  _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), a.M, a.GA, _ptr(ids), _ptr(logits),
                  _ptr(out), _ptr(workspace), workspace.numel())
    return out


def lm_head_argmax_noalloc(w: Q4Tensor, a: Acts, ids=None, logits=None, out=None, stream=None):
    """lm_head_argmax without a workspace: the reduction runs in the library's
    own per-device scratch (wq_lm_head_argmax_noalloc).  Calls on one GPU must
    not overlap."""
    _check_linear(w, a)
    d = a.xq.device
    if ids is not None:
        _check(ids, "ids", _ID_DTYPES, min_numel=w.rows, device=d)
    if logits is not None:
        _check(logits, "logits", torch.float32, shape=(a.M, w.rows), device=d)
    with _on(stream):
        out = _tok_out(out, a.M, d)
        _cuda(w.q, "w.q")
        _lib.call("wq_lm_head_argmax_noalloc", _cur(), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G,
                  _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), a.M, a.GA, _ptr(ids), _ptr(logits), _ptr(out))
    return out


def embed(w: Q4Tensor, tok, out=None, stream=None):
    """int4 embedding lookup (embed.wgsl): x[m] = dequantised row tok[m]."""
    w.check("w")
    _check(tok, "tok", _ID_DTYPES, device=w.q.device)
    M = tok.numel()
    with _on(stream):
        if out is None:
            out = torch.empty((M, w.K), dtype=torch.float32, device=tok.device)
        _check(out, "out", torch.float32, shape=(M, w.K), device=tok.device)
        _cuda(w.q, "w.q")
        _lib.call("wq_embed", _cur(), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G, _ptr(tok), M, _ptr(out))
    return out


def mtp_in(emb, x, norm_f, norm_e, norm_h, eps=1e-6, out: Optional[Acts] = None, stream=None) -> Acts:
    """The MTP fc input (mtp_in.wgsl): per token, [quant(norm_e(emb)) |
    quant(norm_h(norm_f(x)))] as one [M, 2K] row with per-32 scales."""
    if emb.dim() == 1:
        emb, x = emb[None], x[None]
    _check(x, "x", torch.float32)
    M, K = x.shape
    _check(emb, "emb", torch.float32, shape=(M, K), device=x.device)
    for n, t in (("norm_f", norm_f), ("norm_e", norm_e), ("norm_h", norm_h)):
        _check(t, n, torch.float32, shape=(K,), device=x.device)
    with _on(stream):
        a = out if out is not None else empty_acts(M, 2 * K, GA=32, G=32, device=x.device)
        a.check("out")
        if a.xq.shape != (M, 2 * K) or a.GA != 32 or a.G != 32:
            raise ValueError(f"out: mtp_in writes [M, 2K] = {(M, 2 * K)} activations at GA = G = 32")
        _cuda(x, "x")
        _lib.call("wq_mtp_in", _cur(), _ptr(emb), _ptr(x), _ptr(norm_f), _ptr(norm_e), _ptr(norm_h),
                  float(eps), M, K, _ptr(a.xq), _ptr(a.dx), _ptr(a.xs))
    return a


def attn_combine(part, pos, gate=None, gate_stride=0, G=128, out: Optional[Acts] = None, stream=None,
                 params=None) -> Acts:
    """Merge flash-decoding partials part f32 [M, H, nch, D + 2] into the o
    projection's int8 input (attn_combine.wgsl), per-32 scales; optional
    Qwen3.5 gate rows (gate of head h at h*2D + D of a token's row).  params
    (make_params, optional): the position is read from it when the kernel
    runs, and `pos` is the largest it may be (larger values are clamped)."""
    _check(part, "part", torch.float32)
    if part.dim() != 4:
        raise ValueError(f"part: expected [M, H, nch, D + 2], got shape {tuple(part.shape)}")
    M, H, nch, D2 = part.shape
    D = D2 - 2
    if gate is not None:
        _check(gate, "gate", torch.float32, min_numel=(M - 1) * gate_stride + 2 * H * D, device=part.device)
    _check_params(params, part.device)
    with _on(stream):
        a = out if out is not None else empty_acts(M, H * D, GA=32, G=G, device=part.device)
        a.check("out")
        if a.xq.shape != (M, H * D) or a.GA != 32:
            raise ValueError(f"out: attn_combine writes [M, H*D] = {(M, H * D)} activations at GA = 32")
        _cuda(part, "part")
        _lib.call("wq_attn_combine", _cur(), _ptr(part), M, H, D, nch, int(pos), _ptr(gate),
                  int(gate_stride), _ptr(a.xq), _ptr(a.dx), _ptr(a.xs), _ptr(params))
    return a


def gather_rows(w: Q4Tensor, ids, stream=None) -> Q4Tensor:
    """Packed rows ids of w as a new Q4Tensor (gather_rows.wgsl: the reduced
    draft lm_head)."""
    w.check("w")
    _check(ids, "ids", _ID_DTYPES, device=w.q.device)
    R = ids.numel()
    with _on(stream):
        dq = torch.empty((R, w.K // 8), dtype=torch.int32, device=ids.device)
        ds = torch.empty((R, w.K // w.G), dtype=torch.int32, device=ids.device)
        _cuda(w.q, "w.q")
        _lib.call("wq_gather_rows", _cur(), _ptr(w.q), _ptr(w.s), w.rows, w.K, w.G, _ptr(ids), R,
                  _ptr(dq), _ptr(ds))
    return Q4Tensor(dq, ds, w.K, w.G)
