"""The reference's CPU torch fake-quant path, restated checkpoint-free.
TEST INFRASTRUCTURE ONLY (checker and reported CPU baseline, never the product).

Restates:
  tools/reference.py:35-40  weights replaced by their RTN int4 dequantisation
                            (q * scale + min, tools/convert.py:60-65) once, at load;
  tools/reference.py:43-48  fq_input: every linear input fake-quantised to int8
                            (dx = amax/127, round(x/dx)*dx), here with the
                            granularity GA (32 as the reference ships, or per token);
  then an fp32 torch matmul, plus SiLU(gate)*up / residual / argmax where the
  configuration has them.

Seeded inputs follow the benchmark protocol: numpy default_rng(seed);
W ~ N(0, 0.02); x ~ N(0, 1) with 8 outlier channels scaled by 20.
"""
import time

import numpy as np
import torch

from . import oracle as orc


def make_weight(rng, N, K, G, want_deq=False, chunk_rows=2048):
    """W ~ N(0, 0.02) [N, K] -> RTN int4 group-G (wq, ws[, deq]).  Drawn row
    chunk by row chunk so that large heads never hold the whole fp32 matrix."""
    wq = np.empty((N, K // 8), np.uint32)
    ws = np.empty((N, K // G), np.uint32)
    deq = np.empty((N, K), np.float32) if want_deq else None
    for r0 in range(0, N, chunk_rows):
        r1 = min(N, r0 + chunk_rows)
        w = rng.normal(0.0, 0.02, size=(r1 - r0, K)).astype(np.float32)
        out = orc.q4_quantize(w, G, want_deq=want_deq)
        wq[r0:r1], ws[r0:r1] = out[0], out[1]
        if want_deq:
            deq[r0:r1] = out[2]
    return (wq, ws, deq) if want_deq else (wq, ws)


def make_activations(rng, M, K, n_outliers=8, outlier_scale=20.0):
    """x ~ N(0, 1) [M, K] with n_outliers channels (same for every token) x20."""
    x = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    if n_outliers:
        idx = rng.choice(K, n_outliers, replace=False)
        x[:, idx] *= np.float32(outlier_scale)
    return x


def dequant_weight(wq, ws, K, G):
    """q * scale + min in fp32 (tools/convert.py:62-65), from the stored f16 words."""
    q = orc.q4_unpack(wq, K).astype(np.float32)
    N = q.shape[0]
    s = (ws & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    m = (ws >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    q = q.reshape(N, K // G, G)
    return (q * s[..., None] + m[..., None]).reshape(N, K)


def fq_input(x, GA=None):
    """tools/reference.py:43-48 with group GA (None = per token): returns x_deq."""
    x = torch.as_tensor(x, dtype=torch.float32)
    K = x.shape[-1]
    GA = K if GA is None else GA
    g = x.reshape(*x.shape[:-1], -1, GA)
    dx = g.abs().amax(-1, keepdim=True) / 127.0
    q = torch.where(dx > 0, torch.round(g / torch.where(dx > 0, dx, 1.0)), 0.0)
    return (q * dx).reshape(x.shape)


class FakeQuantLinear:
    """One linear layer of the torch fake-quant reference: W dequantised once at
    construction (as tools/reference.py:36-40 does at load), activations
    fake-quantised on every call."""

    def __init__(self, wq, ws, K, G, mode=0, GA=None):
        self.w = torch.from_numpy(dequant_weight(wq, ws, K, G))
        self.mode = mode
        self.GA = GA
        self.N = self.w.shape[0] // 2 if mode == 2 else self.w.shape[0]

    def __call__(self, x, y=None):
        xd = fq_input(x, self.GA)
        a = xd @ self.w.T
        if self.mode == 0:
            return a
        if self.mode == 1:
            return torch.as_tensor(y) + a
        gate, up = a[..., : self.N], a[..., self.N:]
        return torch.nn.functional.silu(gate) * up


def argmax_ref(logits):
    """Greedy token with the reference tie rule (argmax.wgsl:14-43) on torch:
    torch.argmax returns the first maximal index for finite inputs."""
    return torch.argmax(torch.as_tensor(logits), dim=-1)


def time_cpu(fn, warmup=3, iters=20, max_seconds=30.0):
    """Median wall time (s) of fn() after warm-up, bounded to max_seconds of
    work, on the torch thread count the caller set (torch.get_num_threads())."""
    for _ in range(warmup):
        fn()
    ts = []
    t_start = time.perf_counter()
    while len(ts) < iters and (time.perf_counter() - t_start) < max_seconds:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)
