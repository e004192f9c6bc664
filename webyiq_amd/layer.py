"""One decoder layer's int4 x int8 op sequence, recorded once and replayed
(webyIQ crates/engine/src/graph.rs:257-328 builds it, lib.rs:222-228 replays
it): norm+quant -> qkv -> quant -> o (+= residual) -> norm+quant ->
gate_up (SiLU * up) -> quant -> down (+= residual).

The attention kernel that writes the flash-decoding partials (attn.wgsl)
is not part of this path.  With attention="combine" (the decode order of
graph.rs:289-291) a fixed buffer of synthetic chunk partials stands in for
its output: wq_attn_combine merges it and writes the o projection's per-32
int8 input, and o is a plain GEMV.  With attention="copy" the q columns of
the qkv output stand in for the attention output and o quantises them per
token.  With fused=True each quant -> matmul pair is one wq_quant_gemv call
(one launch for M <= 2); fused=False issues the quantiser and the GEMV
separately (bit-identical results).  All buffers are allocated up front;
`run()` only launches, on one stream, so the sequence can be captured into a
HIP graph and replayed.  With params (ops.make_params: the step's device
Params, the reference's uniform of graph.rs:413-416) the chunk merge reads
its position from that buffer when it runs (attn_combine.wgsl:35), so one
captured layer serves every position: only the buffer is rewritten between
replays (lib.rs:312-314, or the GPU itself on the speculative path,
lib.rs:325).
"""
import contextlib

import torch

from . import ops


class DecodeLayer:
    def __init__(self, w, M, hidden=2048, q_dim=2048, kv_dim=512, ffn=6144, G=128, eps=1e-6,
                 fused=True, x=None, device="cuda", attention="copy", head_dim=128, pos=511, max_ctx=4096,
                 params=None):
        """w: ops.Weights with 'qkv' (q_dim + 2 kv_dim rows), 'o', 'gate_up'
        (2 ffn rows) and 'down' Q4Tensors, plus float tensors 'attn_norm' and
        'mlp_norm'.  x: the residual stream f32 [M, hidden] to update in place
        (layers of one model share it); allocated when None.  attention:
        "copy" or "combine" (chunk partials of tokens at positions pos ..
        pos + M - 1 in a max_ctx context, head_dim per head).  params: the
        device step parameters; the merge then takes pos from them at run
        time (any position up to max_ctx - M) and `pos` is unused."""
        assert attention in ("copy", "combine")
        self.w, self.M, self.eps, self.fused, self.attention = w, M, eps, fused, attention
        self.q_dim, self.pos, self.params = q_dim, pos, params
        self.pos_bound = max_ctx - M  # the largest first position the context holds
        f32 = dict(dtype=torch.float32, device=device)
        self.x = torch.zeros((M, hidden), **f32) if x is None else x  # residual stream (in/out)
        self.qkv = torch.empty((M, q_dim + 2 * kv_dim), **f32)
        self.att = torch.empty((M, q_dim), **f32)
        self.h = torch.empty((M, ffn), **f32)
        self.a_in = ops.empty_acts(M, hidden, None, G, device)
        if attention == "combine":
            heads, nch = q_dim // head_dim, max_ctx // 32
            self.part = torch.randn((M, heads, nch, head_dim + 2), **f32)
            self.part[..., head_dim + 1].uniform_(1.0, 32.0)  # chunk weight sums
            self.a_att = ops.empty_acts(M, q_dim, 32, G, device)
        else:
            self.a_att = ops.empty_acts(M, q_dim, None, G, device)
        self.a_mlp = ops.empty_acts(M, hidden, None, G, device)
        self.a_h = ops.empty_acts(M, ffn, None, G, device)

    def _linear(self, name, x, a, norm=None, mode=ops.MODE_STORE, y=None, stream=None):
        w = self.w.w(name)
        if self.fused:
            ops.quant_gemv(w, x, norm=norm, eps=self.eps, mode=mode, y=y, out=a, stream=stream)
        else:
            ops.quant(x, norm=norm, eps=self.eps, G=w.G, out=a, stream=stream)
            ops.gemv(w, a, mode=mode, y=y, stream=stream)

    def run(self, stream=None):
        w = self.w
        self._linear("qkv", self.x, self.a_in, norm=w["attn_norm"], y=self.qkv, stream=stream)
        if self.attention == "combine":
            if self.params is not None:
                ops.attn_combine(self.part, self.pos_bound, out=self.a_att, stream=stream, params=self.params)
            else:
                ops.attn_combine(self.part, self.pos, out=self.a_att, stream=stream)
            ops.gemv(w.w("o"), self.a_att, mode=ops.MODE_ACCUMULATE, y=self.x, stream=stream)
        else:
            with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
                self.att.copy_(self.qkv[:, : self.q_dim])     # attention-core stand-in
            self._linear("o", self.att, self.a_att, mode=ops.MODE_ACCUMULATE, y=self.x, stream=stream)
        self._linear("gate_up", self.x, self.a_mlp, norm=w["mlp_norm"], mode=ops.MODE_SILU_MUL, y=self.h,
                     stream=stream)
        self._linear("down", self.h, self.a_h, mode=ops.MODE_ACCUMULATE, y=self.x, stream=stream)
        return self.x

    def weight_bytes(self):
        return sum(t.q.numel() * 4 + t.s.numel() * 4 for t in
                   (self.w.w(n) for n in ("qkv", "o", "gate_up", "down")))

