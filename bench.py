"""Benchmark of the MI355X int4 x int8 path on BASELINE.json's metric:
"int4 GEMV us + HBM GB/s (M=1, 2048x6144); prefill GEMM int8 TOPS (M=1024)".

  python bench.py [--steps K] [--warmup W] [--copies R] [--no-cpu] [--gpus 1]

One step = one decode GEMV launch (M=1, K=2048, N=6144, int4 group-128 weights,
per-token int8 activations) on inputs already resident in HBM.  Launches rotate
over R weight copies (default 64 x 6.7 MB = 430 MB > the 256 MB MALL), so every
launch streams its weights from HBM.  The timed K steps run as HIP-graph
replays (no host gap between launches) bracketed by synchronize on both sides.

Printed JSON line:
  value       whole-job GEMV throughput, algorithmic GB/s over the K steps
  roofline    the GEMV kernel: algorithmic bytes / mean kernel duration
              (HIP events around single launches on the launch stream),
              against 8 TB/s; traffic = rocprofv3 FETCH+WRITE bytes per launch
              when profiles/gemv_traffic.json holds them
  prefill     the M=1024 GEMMs (K=2048 N=6144 and K=6144 N=2048): TOPS and
              fraction of the 5.0 POP/s dense int8 MFMA peak
  cpu_baseline the reference's torch fake-quant path (oracle/reference.py) on a
              bounded sample of the same workload on this host's cores
Algorithmic bytes: W = N*K/2, S = 4*N*K/G, x = M*K + 4*M + 4*M*K/G, y = 4*M*N.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def gemv_bytes(M, K, N, G):
    return N * K // 2 + 4 * N * K // G + M * K + 4 * M + 4 * M * K // G + 4 * M * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    return ap.parse_args()


class Launcher:
    """Pre-built ctypes argument lists so the timed loops pay no Python packing."""

    def __init__(self, lib, fn, args):
        self.f = getattr(lib, fn)
        self.args = args

    def __call__(self, stream):
        rc = self.f(stream, *self.args)
        if rc != 0:
            raise RuntimeError(f"launch failed [{rc}]")


def graph_time(torch, launches, reps):
    """Mean time per launch of `launches` captured in one HIP graph and
    replayed `reps` times back to back (seconds)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for ln in launches:
            ln(ctypes.c_void_p(s.cuda_stream))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for ln in launches:
            ln(cs)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (reps * len(launches))


def event_kernel_time(torch, launches, n):
    """Mean duration of single launches, each bracketed by HIP events recorded
    on the stream the kernel is launched on (seconds)."""
    stream = torch.cuda.current_stream()
    cs = ctypes.c_void_p(stream.cuda_stream)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        evs[i][0].record(stream)
        launches[i % len(launches)](cs)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) * 1e-3 for a, b in evs]
    return float(np.mean(ts)), float(np.median(ts))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md, not run", file=sys.stderr)
        sys.exit(2)
    import torch
    from webyiq_amd import _lib, ops

    lib = _lib.load()
    sys.path.insert(0, HERE)
    from oracle import oracle as orc
    from oracle import reference as ref

    dev = "cuda"
    M, K, N, G = 1, 2048, 6144, 128
    rng = np.random.default_rng(args.seed)
    wq, ws, deq = ref.make_weight(rng, N, K, G, want_deq=True)
    x = ref.make_activations(rng, M, K)

    # inputs resident in HBM: R weight copies at distinct addresses
    R = max(1, args.copies)
    q0 = torch.from_numpy(wq.view(np.int32)).to(dev)
    s0 = torch.from_numpy(ws.view(np.int32)).to(dev)
    qs = [q0] + [q0.clone() for _ in range(R - 1)]
    ss = [s0] + [s0.clone() for _ in range(R - 1)]
    a = ops.quant(torch.from_numpy(x).to(dev), G=G)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # parity gate before timing: bit-exact against the CPU oracle
    xq, dx, xs = orc.quant_act(x, None, G)
    ops.gemv(ops.Q4Tensor(qs[R - 1], ss[R - 1], K, G), a, y=y)
    want = orc.linear(wq, ws, K, G, xq, dx, xs)
    torch.cuda.synchronize()
    parity = bool(np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)))
    if not parity:
        print("bench.py: GEMV output differs from the oracle", file=sys.stderr)
        sys.exit(1)

    P = ctypes.c_void_p
    launches = [Launcher(lib, "wq_gemv", [P(qs[i].data_ptr()), P(ss[i].data_ptr()), N, K, G,
                                          P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                          M, K, 0, P(y.data_ptr())]) for i in range(R)]
    # warm-up, then the timed steps as graph replays
    reps_w = max(1, args.warmup // R)
    graph_time(torch, launches, reps_w)
    reps = max(1, args.steps // R)
    t_launch = graph_time(torch, launches, reps)
    steps = reps * R
    nbytes = gemv_bytes(M, K, N, G)
    value = nbytes / t_launch / 1e9
    t_kern_mean, t_kern_med = event_kernel_time(torch, launches, 512)
    achieved = nbytes / t_kern_mean / 1e9

    traffic = None
    tp = os.path.join(HERE, "profiles", "gemv_traffic.json")
    if os.path.exists(tp):
        traffic = json.load(open(tp)).get("bytes_per_launch")

    out = {
        "metric": "int4 GEMV us + HBM GB/s (M=1, 2048x6144); prefill GEMM int8 TOPS (M=1024)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * R,
        "ms_per_step": round(t_launch * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8->int32",
        "data": "synthetic: W~N(0,0.02) RTN int4 g128, x~N(0,1) with 8 outliers x20, seed %d" % args.seed,
        "config": {"workload": "decode GEMV M=1 K=2048 N=6144 G=128 per-token int8 (BASELINE configs[0] shape)",
                   "M": M, "K": K, "N": N, "G": G, "weight_copies": R,
                   "bytes_per_launch": nbytes, "parallelism": "single GPU"},
        "gemv_us_per_launch_graph": round(t_launch * 1e6, 3),
        "gemv_us_kernel_events": {"mean": round(t_kern_mean * 1e6, 3), "median": round(t_kern_med * 1e6, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "parity": {"gemv_vs_oracle_bit_exact": parity},
    }

    if not args.no_gemm:
        out["prefill"] = bench_gemm(torch, lib, ops, orc, ref, args)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(torch, ref, wq, ws, K, G, x, nbytes, args.cpu_seconds)

    print(json.dumps(out), flush=True)


def bench_gemm(torch, lib, ops, orc, ref, args):
    """M=1024 prefill GEMMs; TOPS = 2*M*N*K / time."""
    res = {}
    P = ctypes.c_void_p
    M = 1024
    for K, N in ((2048, 6144), (6144, 2048)):
        rng = np.random.default_rng(args.seed + K)
        wq, ws = ref.make_weight(rng, N, K, 128)
        x = ref.make_activations(rng, M, K)
        copies = 8  # 8 x 6.3 MB weights + outputs cycle well past the MALL with y
        q = [torch.from_numpy(wq.view(np.int32)).cuda() for _ in range(copies)]
        s = [torch.from_numpy(ws.view(np.int32)).cuda() for _ in range(copies)]
        a = ops.quant(torch.from_numpy(x).cuda(), G=128)
        ys = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(copies)]
        # parity on 8 sampled tokens against the oracle (bit-exact)
        ops.gemm(ops.Q4Tensor(q[0], s[0], K, 128), a, y=ys[0])
        idx = np.linspace(0, M - 1, 8).astype(int)
        xq, dx, xs = orc.quant_act(x[idx], None, 128)
        want = orc.linear(wq, ws, K, 128, xq, dx, xs)
        torch.cuda.synchronize()
        ok = bool(np.array_equal(ys[0].cpu().numpy()[idx].view(np.uint32), want.view(np.uint32)))
        launches = [Launcher(lib, "wq_gemm", [P(q[i].data_ptr()), P(s[i].data_ptr()), N, K, 128,
                                              P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                              M, K, 0, P(ys[i].data_ptr())]) for i in range(copies)]
        graph_time(torch, launches, 4)
        t = graph_time(torch, launches, 25)
        tk, _ = event_kernel_time(torch, launches, 64)
        ops_ = 2.0 * M * N * K
        res[f"K{K}_N{N}"] = {
            "us_graph": round(t * 1e6, 2), "us_kernel_events": round(tk * 1e6, 2),
            "TOPS": round(ops_ / tk / 1e12, 1),
            "frac_int8_peak": round(ops_ / tk / 1e12 / INT8_PEAK_TOPS, 4),
            "parity_sampled_rows_bit_exact": ok,
        }
        del q, s, ys
        torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, ref, wq, ws, K, G, x, nbytes, seconds):
    """The reference's CPU torch fake-quant path on the same GEMV workload."""
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    lin = ref.FakeQuantLinear(wq, ws, K, G)
    xt = torch.from_numpy(x)
    med, n = ref.time_cpu(lambda: lin(xt), warmup=3, iters=1000, max_seconds=seconds)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_gemv": round(med * 1e6, 1),
            "sample": f"median of {n} fake-quant GEMVs (M=1 K=2048 N=6144: fq_input + fp32 x@W^T, "
                      "W dequantised once as tools/reference.py:36-40), ~%.0f s bounded" % seconds}


if __name__ == "__main__":
    main()
