"""Benchmark of the MI355X int4 x int8 path on BASELINE.json's metric:
"int4 GEMV us + HBM GB/s (M=1, 2048x6144); prefill GEMM int8 TOPS (M=1024)".

  python bench.py [--steps K] [--warmup W] [--copies R] [--no-cpu] [--gpus 1]

One step = one decode GEMV launch (M=1, K=2048, N=6144, int4 group-128 weights,
per-token int8 activations) on inputs already resident in HBM.  W warm-up
launches, then exactly K timed launches; launch i uses weight copy i mod R
(default R = 64 x 6.7 MB = 430 MB > the 256 MB MALL), so every launch streams
its weights from HBM.  The W and the K launches are issued one by one (or,
with --launch graph, captured as two HIP graphs) on one stream behind a gate
of --settle untimed launches of the same GEMV replayed as a graph, so the
GPU runs them back to back with no host submission gap and at the clocks of
back-to-back decode launches (class Gate); HIP events on that stream around
the K launches time the region, which is synchronised on both sides.  The
events are created with hipEventDisableSystemFence (class TimingEvents: the
flag hip_runtime_api.h gives for events that only measure time), so
recording them adds no cache writeback and invalidate to the region;
--torch-events times with torch's default events instead.

Printed JSON line:
  value       whole-job GEMV throughput, algorithmic GB/s over the K steps
  roofline    the GEMV kernel: algorithmic bytes / mean duration per launch
              over the timed region, against 8 TB/s; traffic = HBM bytes per
              launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, scaled by
              a copy-kernel calibration) when profiles/gemv_traffic.json
              holds them; kernel_us = one launch's device-clock duration
              (first workgroup entry to last store, the timing build) and
              kernel_frac the same bytes over it
  prefill     the M=1024 GEMMs (K=2048 N=6144 and K=6144 N=2048): us, TOPS
              and fraction of the 5.0 POP/s dense int8 MFMA peak as flat
              keys <shape>_us/_TOPS/_frac; the same shapes at M=256 and 512
              under keys with _M256 / _M512; prefill_detail per shape
  configs     BASELINE configs 2, 3 and 5, the decode layer, the other
              producers, one GPU's shard shapes, the group-32 format
  cpu_baseline the reference's torch fake-quant path (oracle/reference.py) on a
              bounded sample of the same workload on this host's cores
Algorithmic bytes: W = N*K/2, S = 4*N*K/G, x = M*K + 4*M + 4*M*K/G, y = 4*M*N.
Parity gates before timing: the GEMV bit-exact against the CPU oracle; the
GEMM (per-token group-128, min term on the f16 MFMA) within rel 1e-5 on
sampled tokens; every cfg-2/3/5 instance and the one-token decode layer
(configs.parity_gates).
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
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config lines (decode MLP, verify shapes, lm_head)")
    ap.add_argument("--cpu-seconds", type=float, default=24.0)
    ap.add_argument("--gemm-copies", type=int, default=16,
                    help="weight/output copies the prefill GEMMs rotate over (16 = 504 MB, twice the MALL)")
    ap.add_argument("--gemm-warmup", type=int, default=400,
                    help="graph replays before the prefill GEMMs are timed (clocks settle within ~80 ms)")
    ap.add_argument("--launch", choices=("graph", "eager"), default="eager",
                    help="timed launches issued one by one (default) or as one captured HIP graph, "
                         "both queued behind the gate (a graph launch adds ~8 us to the timed region)")
    ap.add_argument("--settle", type=int, default=1000,
                    help="untimed GEMV launches (other weight copies), replayed as a graph ahead of "
                         "the warm-up: the gate that covers the host's enqueue and settles the clocks")
    ap.add_argument("--config-settle", type=int, default=512,
                    help="launches of the same graph queued right before each config timing "
                         "(0: none; keeps the dispatches in flight few, e.g. under rocprofv3 --pmc)")
    ap.add_argument("--torch-events", action="store_true",
                    help="time with torch's default events (a system-scope fence at each record) "
                         "instead of HIP events created with hipEventDisableSystemFence")
    ap.add_argument("--no-kernel-clock", action="store_true",
                    help="skip the device-clock duration of single launches (roofline.kernel_us)")
    ap.add_argument("--timeline", action="store_true",
                    help="also replay the GEMV from the timing build (libwebyiq_q4q8_timeline.so) and "
                         "report its per-workgroup phase stamps")
    ap.add_argument("--calib-mib", type=int, default=0,
                    help="after the timed region, copy a buffer of this many MiB 8 times "
                         "(the known-size kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def log(msg):
    """Progress on stderr (the JSON line is the only stdout output)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


class Launcher:
    """Pre-built ctypes argument lists so the timed loops pay no Python packing."""

    def __init__(self, lib, fn, args):
        self.f = getattr(lib, fn)
        self.args = args

    def __call__(self, stream):
        rc = self.f(stream, *self.args)
        if rc != 0:
            raise RuntimeError(f"launch failed [{rc}]")


class TimingEvents:
    """Two timing events (start, end) for one timed region.

    By default they are created on the HIP runtime that torch loaded with
    hipEventDisableSystemFence: the flag hip_runtime_api.h gives for events
    used only to measure time.  A default event performs a system-scope
    fence when it is recorded (a cache writeback and invalidate); its cost
    then lands in the timed region although it belongs to the event, not to
    the launches between the two events (measured at the driver's 20
    launches: 2.96-2.99 us per launch with these events, 3.04-3.19 with
    torch's default ones, alternating on one box).  --torch-events (or a
    torch build without that runtime file) uses torch's default events.
    Either way the region holds the same launches on the same stream, and
    the caller synchronises on both sides."""
    FLAGS = 0x20000000  # hipEventDisableSystemFence
    hip = None
    kind = "torch"

    @classmethod
    def configure(cls, torch, use_torch=False):
        cls.kind = "torch"
        if use_torch:
            return
        path = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        if not os.path.exists(path):
            return
        h = ctypes.CDLL(path)  # the runtime torch already loaded: the same file, the same handle
        h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        for f in ("hipEventCreateWithFlags", "hipEventRecord", "hipEventElapsedTime", "hipEventDestroy"):
            getattr(h, f).restype = ctypes.c_int
        cls.hip = h
        cls.kind = "hip_no_system_fence"

    def __init__(self, torch):
        self.native = self.kind != "torch"
        if not self.native:
            self.ev = [torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
            return
        self.ev = []
        for _ in range(2):
            e = ctypes.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(ctypes.byref(e), self.FLAGS)
            if rc:
                raise RuntimeError(f"hipEventCreateWithFlags failed [{rc}]")
            self.ev.append(e)

    def record(self, i, stream):
        """Record event i (0 = start, 1 = end) on `stream`, a torch stream."""
        if not self.native:
            self.ev[i].record(stream)
            return
        rc = self.hip.hipEventRecord(self.ev[i], ctypes.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError(f"hipEventRecord failed [{rc}]")

    def seconds(self):
        """Start-to-end time in seconds (the caller has synchronised)."""
        if not self.native:
            return self.ev[0].elapsed_time(self.ev[1]) * 1e-3
        ms = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1])
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed [{rc}]")
        return ms.value * 1e-3

    def __del__(self):
        if getattr(self, "native", False):
            for e in self.ev:
                self.hip.hipEventDestroy(e)


CONFIG_SETTLE = 512  # launches queued before each config timing (--config-settle)


def settle_reps(launches, n=None):
    """Replays of a graph of `launches` that make about n launches
    (default CONFIG_SETTLE): enough back-to-back load for the clocks to
    settle before a timing.  n = 0 gives none."""
    n = CONFIG_SETTLE if n is None else n
    return 0 if n <= 0 else max(2, -(-n // len(launches)))


def graph_time(torch, launches, reps, warm=0):
    """Mean time per launch of `launches` captured in one HIP graph and
    replayed `reps` times back to back (seconds).  `warm` untimed replays are
    queued right before the timed ones, with no synchronisation between, so
    the timing starts on a busy GPU at settled clocks."""
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
    ev = TimingEvents(torch)
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    for _ in range(warm):
        g.replay()
    ev.record(0, cur)
    for _ in range(reps):
        g.replay()
    ev.record(1, cur)
    torch.cuda.synchronize()
    return ev.seconds() / (reps * len(launches))


class Gate:
    """Host-independent timing of a launch sequence.  On one stream: a gate,
    then the warm-up launches, e0, the timed launches, e1.  The gate is either
    `settle`, untimed launches of the same kernel captured as one HIP graph
    and replayed, or (without them) read-only passes over a 512 MiB buffer;
    it lasts until the host has enqueued everything behind it (checked: its
    end event must still be pending when the host is done, else the gate is
    doubled and the run repeated), so the GPU runs the launches back to back
    with no host submission gap.  A settle gate also brings the GPU to the
    clocks of back-to-back launches: after other work the first ~200-1000
    launches of the headline GEMV run slower (measured: 20 timed launches
    averaged 3.84 us after a memory-bound gate, 3.57 us after 1000 settle
    launches, against 3.50 us over 2000).  Synchronised on both sides."""

    def __init__(self, torch, settle=()):
        self.torch = torch
        self.passes = 1
        self.settle = list(settle)
        self.gs = None
        self.flush = None
        if not self.settle:
            self.flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
            self.passes = 8

    def _graph(self, seq, s):
        torch = self.torch
        if not seq:
            return None
        with torch.cuda.stream(s):
            seq[0](ctypes.c_void_p(s.cuda_stream))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            cs = ctypes.c_void_p(s.cuda_stream)
            for ln in seq:
                ln(cs)
        return g

    def time(self, seq, graph=True, warm=()):
        """Seconds per launch of `seq` (callables taking a stream), after the
        gate and the `warm` launches on the same stream."""
        torch = self.torch
        warm = list(warm)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        if self.settle and self.gs is None:
            self.gs = self._graph(self.settle, s)
        gw = self._graph(warm, s) if graph else None
        gt = self._graph(seq, s) if graph else None
        for _ in range(6):
            torch.cuda.synchronize()
            eg = torch.cuda.Event()
            ev = TimingEvents(torch)
            with torch.cuda.stream(s):
                for _ in range(self.passes):
                    if self.gs is not None:
                        self.gs.replay()
                    else:
                        self.flush.sum()
                eg.record(s)
                cs = ctypes.c_void_p(s.cuda_stream)
                if gw is not None:
                    gw.replay()
                elif not graph:
                    for ln in warm:
                        ln(cs)
                ev.record(0, s)
                if gt is not None:
                    gt.replay()
                else:
                    for ln in seq:
                        ln(cs)
                ev.record(1, s)
            covered = not eg.query()  # the gate still ran when the host was done
            torch.cuda.synchronize()
            if covered:
                break
            self.passes *= 2
        self.covered = covered
        return ev.seconds() / len(seq)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards along the output rows, but no multi-GPU run is built", file=sys.stderr)
        sys.exit(2)
    import torch
    from webyiq_amd import _lib, ops

    TimingEvents.configure(torch, use_torch=args.torch_events)
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
    # warm-up: W launches on copies 0 .. W-1 (mod R); then exactly K timed
    # launches on copies W, W+1, ... (mod R): a copy comes back only after R
    # launches (430 MB), so every timed launch streams its weights from HBM
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    # the gate: settle launches on the copies after the timed ones, replayed
    # as a graph while the host enqueues the warm-up and timed launches
    gate = Gate(torch, [launches[(warmup + steps + j) % R] for j in range(args.settle)])
    graph = args.launch == "graph"
    t_launch = gate.time([launches[(warmup + i) % R] for i in range(steps)], graph=graph,
                         warm=[launches[i % R] for i in range(warmup)])
    gate_covered = gate.covered
    nbytes = gemv_bytes(M, K, N, G)
    value = nbytes / t_launch / 1e9
    # the kernel's mean duration per launch over the timed region (HIP events
    # on the launch stream around the K launches)
    achieved = nbytes / t_launch / 1e9

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
        "warmup": warmup,
        "ms_per_step": round(t_launch * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8->int32",
        "data": "synthetic: W~N(0,0.02) RTN int4 g128, x~N(0,1) with 8 outliers x20, seed %d" % args.seed,
        "config": {"workload": "decode GEMV M=1 K=2048 N=6144 G=128 per-token int8 (BASELINE configs[0] shape)",
                   "M": M, "K": K, "N": N, "G": G, "weight_copies": R,
                   "bytes_per_launch": nbytes, "parallelism": "single GPU"},
        "gemv_us_per_launch": round(t_launch * 1e6, 3),
        "launch": args.launch,
        "timing_events": TimingEvents.kind,
        "gate_covered_host_enqueue": gate_covered,
        "settle_launches": args.settle * gate.passes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "parity": {"gemv_vs_oracle_bit_exact": parity},
    }
    log(f"headline: {steps} timed launches, {t_launch * 1e6:.3f} us per launch")
    kc = None if args.no_kernel_clock else kernel_clock(
        torch, Gate(torch, [launches[j % R] for j in range(256)]), [ln.args for ln in launches])
    if kc is not None:
        # the device-clock duration of one launch (first workgroup entry to
        # last store, the timing build), beside the per-launch figure above
        out["roofline"]["kernel_us"] = kc["median_us"]
        out["roofline"]["kernel_frac"] = round(nbytes / (kc["median_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        out["kernel_clock"] = kc

    if args.timeline:
        out["timeline"] = bench_timeline(torch, [ln.args for ln in launches])

    if args.calib_mib > 0:
        nb = args.calib_mib << 20
        src = torch.empty(nb // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["calibration_copy_bytes"] = nb
        del src, dst

    if not args.no_gemm:
        log("prefill GEMMs")
        detail = bench_gemm(torch, lib, ops, orc, ref, args)
        # flat scalars per shape (us, TOP/s, fraction of the int8 peak); the
        # per-shape roofline blocks and parity figures under prefill_detail
        out["prefill"] = {f"{k}_{f}": v[src] for k, v in detail.items()
                          for f, src in (("us", "us_per_launch"), ("TOPS", "TOPS"), ("frac", "frac"))}
        out["prefill_detail"] = detail

    if not args.no_configs:
        global CONFIG_SETTLE
        CONFIG_SETTLE = max(0, args.config_settle)
        log("configs")
        out["configs"] = bench_configs(torch, lib, ops, orc)

    if not args.no_cpu:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(torch, ref, wq, ws, K, G, x, nbytes, args.cpu_seconds)

    print(json.dumps(out), flush=True)


def timeline_lib():
    """The timing build (libwebyiq_q4q8_timeline.so: the same kernels, the
    decode GEMV's thread 0 per workgroup stamping s_memrealtime, a 100 MHz
    clock), or None when it has not been built."""
    from webyiq_amd import _lib
    path = os.path.join(HERE, "webyiq_amd", "libwebyiq_q4q8_timeline.so")
    if not os.path.exists(path):
        return None
    T = ctypes.CDLL(path)
    T.wq_gemv.argtypes, T.wq_gemv.restype = _lib.PROTOTYPES["wq_gemv"]
    T.wq_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    T.wq_timeline_read.restype = ctypes.c_int
    return T


def read_stamps(T):
    buf = np.zeros(4096 * 8, dtype=np.uint64)
    if T.wq_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("wq_timeline_read failed")
    b = buf.reshape(4096, 8).astype(np.int64)
    return b[b[:, 0] > 0]


def kernel_clock(torch, gate, launch_args, n=32):
    """Device-clock duration of single headline launches: n launches of the
    timing build, each on a different weight copy after the gate, each from
    the first workgroup's entry stamp to the last workgroup's after-store
    stamp (us; median and range)."""
    T = timeline_lib()
    if T is None:
        return None
    durs = []
    for i in range(n):
        ln = Launcher(T, "wq_gemv", list(launch_args[i % len(launch_args)]))
        gate.time([ln], graph=False)
        b = read_stamps(T)
        durs.append((b[:, 4].max() - b[:, 0].min()) / 100.0)
    return {"median_us": round(float(np.median(durs)), 3), "min_us": round(float(np.min(durs)), 3),
            "max_us": round(float(np.max(durs)), 3), "launches": n,
            "how": "timing build, s_memrealtime (100 MHz): first workgroup entry to last workgroup's "
                   "after-store stamp, single launches each after the settle gate"}


def bench_timeline(torch, launch_args):
    """Phase stamps of the headline GEMV: the same launches (weight copies,
    activations, output) from the timing build, libwebyiq_q4q8_timeline.so
    (the kernels plus s_memrealtime stamps by thread 0 of each workgroup, a
    100 MHz clock), replayed as graphs; the stamps are those of the last
    launch.  Times in us from the first workgroup's entry, percentiles over
    the workgroups.  The per-launch time is the timing build's own."""
    from webyiq_amd import _lib
    path = os.path.join(HERE, "webyiq_amd", "libwebyiq_q4q8_timeline.so")
    if not os.path.exists(path):
        print("bench.py: --timeline needs webyiq_amd/libwebyiq_q4q8_timeline.so (python -m webyiq_amd.build)",
              file=sys.stderr)
        sys.exit(1)
    T = ctypes.CDLL(path)
    T.wq_gemv.argtypes, T.wq_gemv.restype = _lib.PROTOTYPES["wq_gemv"]
    T.wq_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    T.wq_timeline_read.restype = ctypes.c_int
    launches = [Launcher(T, "wq_gemv", list(a)) for a in launch_args]
    graph_time(torch, launches, 10)
    t = graph_time(torch, launches, 20)
    buf = np.zeros(4096 * 8, dtype=np.uint64)
    if T.wq_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("wq_timeline_read failed")
    b = buf.reshape(4096, 8).astype(np.int64)
    b = b[b[:, 0] > 0]
    t0 = b[:, 0].min()
    names = ["entry", "activations_landed", "first_row_landed", "products_done", "outputs_stored"]
    phases = {}
    for k, name in enumerate(names):
        d = (b[:, k] - t0) / 100.0
        phases[name] = {q: round(float(np.percentile(d, v)), 2) for q, v in
                        (("min", 0), ("p10", 10), ("median", 50), ("p90", 90), ("max", 100))}
    dur = (b[:, 4] - b[:, 0]) / 100.0
    return {"us_per_launch": round(t * 1e6, 3), "workgroups": int(len(b)), "phases_us": phases,
            "workgroup_duration_us": {"median": round(float(np.median(dur)), 2), "max": round(float(dur.max()), 2)},
            "clock": "s_memrealtime, 100 MHz"}


def bench_gemm(torch, lib, ops, orc, ref, args):
    """M=1024 prefill GEMMs; TOPS = 2*M*N*K / time."""
    res = {}
    P = ctypes.c_void_p
    # M = 1024 is BASELINE's shape; 256 and 512 (the smallest prefill sizes
    # the GEMM path serves) are reported beside it under their own keys
    for M, K, N in ((1024, 2048, 6144), (1024, 6144, 2048), (512, 2048, 6144), (512, 6144, 2048),
                    (256, 2048, 6144), (256, 6144, 2048)):
        rng = np.random.default_rng(args.seed + K + (0 if M == 1024 else M))
        wq, ws = ref.make_weight(rng, N, K, 128)
        x = ref.make_activations(rng, M, K)
        copies = max(1, args.gemm_copies)  # 16: 16 x (6.3 MB weights + 25.2 MB outputs) = 504 MB
        q = [torch.from_numpy(wq.view(np.int32)).cuda() for _ in range(copies)]
        s = [torch.from_numpy(ws.view(np.int32)).cuda() for _ in range(copies)]
        a = ops.quant(torch.from_numpy(x).cuda(), G=128)
        ys = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(copies)]
        # the split-K workspace (one byte when the shape is not split), shared
        # by the launches, which are stream-ordered
        wsp = ops.gemm_workspace(N, K, 128, M)
        split = wsp.numel() > 1
        # parity on 16 sampled tokens against the oracle (rel 1e-5, max-norm)
        ops.gemm(ops.Q4Tensor(q[0], s[0], K, 128), a, y=ys[0], workspace=wsp)
        idx = np.linspace(0, M - 1, 16).astype(int)
        xq, dx, xs = orc.quant_act(x[idx], None, 128)
        want = orc.linear(wq, ws, K, 128, xq, dx, xs)
        torch.cuda.synchronize()
        got = ys[0].cpu().numpy()[idx]
        rel = float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))
        if not rel < 1e-5:
            print(f"bench.py: GEMM K={K} N={N} differs from the oracle (rel {rel:.3g})", file=sys.stderr)
            sys.exit(1)
        launches = [Launcher(lib, "wq_gemm", [P(q[i].data_ptr()), P(s[i].data_ptr()), N, K, 128,
                                              P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                              M, K, 0, P(ys[i].data_ptr()), None, P(wsp.data_ptr()),
                                              wsp.numel()]) for i in range(copies)]
        # warm-up long enough for the clocks to settle (the first ~30-80 ms
        # of MFMA load run measurably slower), then the median of three timings
        graph_time(torch, launches, max(1, args.gemm_warmup))
        t = float(np.median([graph_time(torch, launches, 25) for _ in range(3)]))
        ops_ = 2.0 * M * N * K
        res[f"K{K}_N{N}" + ("" if M == 1024 else f"_M{M}")] = {
            "us_per_launch": round(t * 1e6, 2),
            "TOPS": round(ops_ / t / 1e12, 1),
            "frac": round(ops_ / t / 1e12 / INT8_PEAK_TOPS, 4),
            "roofline": {"bound": "mfma", "achieved": round(ops_ / t / 1e12, 1), "peak": INT8_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(ops_ / t / 1e12 / INT8_PEAK_TOPS, 4)},
            "parity_vs_oracle_rel": rel,
            "k_split_pairs": split,
        }
        del q, s, ys
        torch.cuda.empty_cache()
    return res


def rand_weights(torch, rows, K, G, copies):
    """Timing-only weights: random codes, finite f16 scale/min words (the
    values do not change the work; parity is the tests' job)."""
    q = torch.randint(-2**31, 2**31 - 1, (rows, K // 8), dtype=torch.int32, device="cuda")
    lo = torch.randint(0x1800, 0x2400, (rows, K // G), dtype=torch.int32, device="cuda")
    hi = torch.randint(0x9800, 0xA400, (rows, K // G), dtype=torch.int32, device="cuda")
    s = lo | (hi << 16)
    return [(q, s)] + [(q.clone(), s.clone()) for _ in range(copies - 1)]


def copies_for(nbytes, budget=512 << 20, cap=1024):
    """Enough weight copies that one rotation exceeds the 256 MB MALL
    (512 MB: the smallest verify shape, N = 512, takes ~940 copies)."""
    return max(2, min(cap, -(-budget // nbytes)))


def to_host_u32(t):
    return t.cpu().numpy().view(np.uint32)


def oracle_rows(orc, wq, ws, K, G, xq, dx, xs, threads=16):
    """orc.linear (mode 0) split along the weight rows over a thread pool
    (ctypes releases the GIL during the C oracle's calls)."""
    from concurrent.futures import ThreadPoolExecutor
    N = wq.shape[0]
    n = max(1, min(threads, os.cpu_count() or 1, N // 1024 or 1))
    cuts = np.linspace(0, N, n + 1).astype(int)
    with ThreadPoolExecutor(n) as ex:
        parts = ex.map(lambda i: orc.linear(wq[cuts[i]:cuts[i + 1]], ws[cuts[i]:cuts[i + 1]], K, G, xq, dx, xs),
                       range(n))
        return np.concatenate(list(parts), 1)


def parity_gate(name, ok, detail=""):
    """Stop the bench when a timed instance's output differs from the oracle."""
    if not ok:
        print(f"bench.py: {name} differs from the oracle {detail}", file=sys.stderr)
        sys.exit(1)
    return True


def bench_configs(torch, lib, ops, orc):
    """BASELINE configs 2, 3 and 5 (decode MLP block, M<=8 verify shapes,
    lm_head + argmax), one GPU's share of them when split over 2-8 GPUs, and
    the group-32 format on the cfg-1/2/4 shapes:
    us per launch (graph replays over weight copies, so weights stream from
    HBM) and algorithmic GB/s.  Before timing, every cfg-2/3/5 instance and
    the one-token decode layer are checked against the oracle on the timed
    inputs (one launch on the first weight copy): GEMV outputs bit-exact
    (mode 2 within rel 1e-5), argmax tokens exact, the fused layer
    bit-identical to the unfused one with its first projection bit-exact."""
    P = ctypes.c_void_p
    G = 128
    res = {}
    gates = {}
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731

    def host_acts(a):
        torch.cuda.synchronize()
        return a.xq.cpu().numpy(), a.dx.cpu().numpy(), a.xs.cpu().numpy()

    def acts(M, K):
        x = torch.randn((M, K), dtype=torch.float32, device="cuda")
        return ops.quant(x, G=G)

    def lin_bytes(M, K, N):
        return gemv_bytes(M, K, N, G)

    # cfg 3: the 7 linear shapes of one layer at M = 2, 4, 8
    shapes = {"q": (2048, 2048), "k": (2048, 512), "v": (2048, 512), "o": (2048, 2048),
              "gate": (2048, 6144), "up": (2048, 6144), "down": (6144, 2048)}
    verify = {}
    for M in (2, 4, 8):
        for name, (K, N) in shapes.items():
            nb = lin_bytes(M, K, N)
            R = copies_for(nb)
            ws = rand_weights(torch, N, K, G, R)
            a = acts(M, K)
            y = torch.empty((M, N), dtype=torch.float32, device="cuda")
            launches = [Launcher(lib, "wq_gemv", [P(q.data_ptr()), P(sc.data_ptr()), N, K, G,
                                                  P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                                  M, K, 0, P(y.data_ptr())]) for q, sc in ws]
            launches[0](cur())
            want = orc.linear(to_host_u32(ws[0][0]), to_host_u32(ws[0][1]), K, G, *host_acts(a))
            gates[f"cfg3_M{M}_{name}"] = parity_gate(
                f"cfg 3 M={M} {name}", np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)))
            t = graph_time(torch, launches, max(2, 256 // R), warm=settle_reps(launches))
            verify[f"M{M}_{name}_K{K}_N{N}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
            del ws
    res["cfg3_verify_gemv"] = verify

    # cfg 2: decode MLP block at M = 1: norm+quant, gate_up (mode 2), quant, down (mode 1)
    K1, F = 2048, 6144
    nb_gu, nb_dn = lin_bytes(1, K1, 2 * F) - 4 * F, lin_bytes(1, F, K1)
    nb_q = 4 * F + F + 4 + 4 * (F // G)
    R = copies_for(nb_gu + nb_dn)
    gu = rand_weights(torch, 2 * F, K1, G, R)
    dn = rand_weights(torch, K1, F, G, R)
    x = torch.randn((1, K1), dtype=torch.float32, device="cuda")
    nw = torch.ones(K1, dtype=torch.float32, device="cuda")
    a1 = ops.empty_acts(1, K1, None, G)
    a2 = ops.empty_acts(1, F, None, G)
    h = torch.empty((1, F), dtype=torch.float32, device="cuda")
    yres = torch.zeros((1, K1), dtype=torch.float32, device="cuda")
    fused = []
    for (qg, sg), (qd, sd) in zip(gu, dn):
        fused.append(Launcher(lib, "wq_quant_gemv", [P(x.data_ptr()), P(nw.data_ptr()), ctypes.c_float(1e-6),
                                                     P(qg.data_ptr()), P(sg.data_ptr()), F, K1, G, 1, 2,
                                                     P(a1.xq.data_ptr()), P(a1.dx.data_ptr()), P(a1.xs.data_ptr()),
                                                     P(h.data_ptr())]))
        fused.append(Launcher(lib, "wq_quant_gemv", [P(h.data_ptr()), None, ctypes.c_float(0.0),
                                                     P(qd.data_ptr()), P(sd.data_ptr()), K1, F, G, 1, 1,
                                                     P(a2.xq.data_ptr()), P(a2.dx.data_ptr()), P(a2.xs.data_ptr()),
                                                     P(yres.data_ptr())]))
    # gate: one block from a zero residual against the oracle chain
    yres.zero_()
    fused[0](cur())
    fused[1](cur())
    xh = x.cpu().numpy()
    q1, d1, s1 = orc.quant_act(xh, None, G, norm_w=nw.cpu().numpy(), eps=1e-6)
    h_want = orc.linear(to_host_u32(gu[0][0]), to_host_u32(gu[0][1]), K1, G, q1, d1, s1, mode=2)
    h_got = h.cpu().numpy()
    rel_h = float(np.max(np.abs(h_got - h_want)) / max(float(np.max(np.abs(h_want))), 1e-30))
    q2, d2, s2 = orc.quant_act(h_got, None, G)
    y_want = orc.linear(to_host_u32(dn[0][0]), to_host_u32(dn[0][1]), F, G, q2, d2, s2, mode=1,
                        y=np.zeros((1, K1), np.float32))
    gates["cfg2_block"] = parity_gate(
        "cfg 2 block", rel_h < 1e-5 and np.array_equal(host_acts(a2)[0], q2)
        and np.array_equal(yres.cpu().numpy().view(np.uint32), y_want.view(np.uint32)), f"(gate_up rel {rel_h:.3g})")
    t2 = graph_time(torch, fused, max(2, 128 // R), warm=settle_reps(fused)) * 2  # per block (2 launches)
    steps = []
    for (qg, sg), (qd, sd) in zip(gu, dn):
        steps.append(Launcher(lib, "wq_quant_act", [P(x.data_ptr()), P(nw.data_ptr()), ctypes.c_float(1e-6), 1, K1,
                                                    K1, G, P(a1.xq.data_ptr()), P(a1.dx.data_ptr()), P(a1.xs.data_ptr())]))
        steps.append(Launcher(lib, "wq_gemv", [P(qg.data_ptr()), P(sg.data_ptr()), F, K1, G, P(a1.xq.data_ptr()),
                                               P(a1.dx.data_ptr()), P(a1.xs.data_ptr()), 1, K1, 2, P(h.data_ptr())]))
        steps.append(Launcher(lib, "wq_quant_act", [P(h.data_ptr()), None, ctypes.c_float(0.0), 1, F, F, G,
                                                    P(a2.xq.data_ptr()), P(a2.dx.data_ptr()), P(a2.xs.data_ptr())]))
        steps.append(Launcher(lib, "wq_gemv", [P(qd.data_ptr()), P(sd.data_ptr()), K1, F, G, P(a2.xq.data_ptr()),
                                               P(a2.dx.data_ptr()), P(a2.xs.data_ptr()), 1, F, 1, P(yres.data_ptr())]))
    t4 = graph_time(torch, steps, max(2, 128 // R), warm=settle_reps(steps)) * 4  # per block (4 launches)
    nb_block = nb_gu + nb_q + nb_dn
    res["cfg2_decode_mlp_block"] = {"us": round(t2 * 1e6, 3), "bytes": nb_block,
                                    "GBps": round(nb_block / t2 / 1e9, 1), "launches": 2,
                                    "unfused_us": round(t4 * 1e6, 3), "unfused_launches": 4}
    del gu, dn

    # cfg 5: lm_head + fused argmax, M = 1 and 8, V = 151936 and 32768
    head = {}
    wsp = ops.lm_head_workspace()
    for V in (151936, 32768):
        nbw = V * 2048 // 2 + 4 * V * 2048 // G
        R = copies_for(nbw, budget=512 << 20, cap=16)
        ws = rand_weights(torch, V, 2048, G, R)
        for M in (1, 8):
            a = acts(M, 2048)
            tok = torch.empty(M, dtype=torch.int32, device="cuda")
            launches = [Launcher(lib, "wq_lm_head_argmax", [P(q.data_ptr()), P(sc.data_ptr()), V, 2048, G,
                                                            P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                                            M, 2048, None, None, P(tok.data_ptr()),
                                                            P(wsp.data_ptr()), wsp.numel()]) for q, sc in ws]
            launches[0](cur())
            logits = oracle_rows(orc, to_host_u32(ws[0][0]), to_host_u32(ws[0][1]), 2048, G, *host_acts(a))
            gates[f"cfg5_M{M}_V{V}"] = parity_gate(
                f"cfg 5 M={M} V={V}", np.array_equal(tok.cpu().numpy().view(np.uint32), orc.argmax(logits)))
            t = graph_time(torch, launches, max(2, 64 // R), warm=settle_reps(launches))
            nb = nbw + M * 2048 + 4 * M + 4 * M * 2048 // G + 4 * M
            head[f"M{M}_V{V}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1),
                                  "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
        del ws
    res["cfg5_lm_head_argmax"] = head

    # one GPU's share when the path is split over P GPUs (N-split GEMV and
    # lm_head, gate_up along N + down along K for the MLP); the exchanges
    # between GPUs are not built, so these are the per-GPU kernels alone
    shard = {}
    for Pn in (2, 4, 8):
        K, N = 2048, 6144 // Pn
        nb = lin_bytes(1, K, N)
        R = copies_for(nb)
        ws = rand_weights(torch, N, K, G, R)
        a = acts(1, K)
        y = torch.empty((1, N), dtype=torch.float32, device="cuda")
        launches = [Launcher(lib, "wq_gemv", [P(q.data_ptr()), P(sc.data_ptr()), N, K, G, P(a.xq.data_ptr()),
                                              P(a.dx.data_ptr()), P(a.xs.data_ptr()), 1, K, 0, P(y.data_ptr())])
                    for q, sc in ws]
        t = graph_time(torch, launches, max(2, 256 // R), warm=settle_reps(launches))
        shard[f"cfg1_P{Pn}_N{N}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
        del ws
    Vs = 151936 // 8
    nbw = Vs * 2048 // 2 + 4 * Vs * 2048 // G
    R = copies_for(nbw, budget=512 << 20, cap=64)
    ws = rand_weights(torch, Vs, 2048, G, R)
    ids = torch.arange(3 * Vs, 4 * Vs, dtype=torch.int32, device="cuda")  # shard 3's global rows
    for M in (1, 8):
        a = acts(M, 2048)
        tok = torch.empty(M, dtype=torch.int32, device="cuda")
        launches = [Launcher(lib, "wq_lm_head_argmax", [P(q.data_ptr()), P(sc.data_ptr()), Vs, 2048, G,
                                                        P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                                        M, 2048, P(ids.data_ptr()), None, P(tok.data_ptr()),
                                                        P(wsp.data_ptr()), wsp.numel()]) for q, sc in ws]
        t = graph_time(torch, launches, max(2, 128 // R), warm=settle_reps(launches))
        nb = nbw + M * 2048 + 4 * M + 4 * M * 2048 // G + 4 * M
        shard[f"cfg5_P8_M{M}_V{Vs}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
    del ws
    Fs = F // 8
    nb_gu, nb_dn = lin_bytes(1, K1, 2 * Fs) - 4 * Fs, lin_bytes(1, Fs, K1)
    R = copies_for(nb_gu + nb_dn)
    gu = rand_weights(torch, 2 * Fs, K1, G, R)
    dn = rand_weights(torch, K1, Fs, G, R)
    a1 = ops.empty_acts(1, K1, None, G)
    a2 = ops.empty_acts(1, Fs, None, G)
    hs = torch.empty((1, Fs), dtype=torch.float32, device="cuda")
    fused = []
    for (qg, sg), (qd, sd) in zip(gu, dn):
        fused.append(Launcher(lib, "wq_quant_gemv", [P(x.data_ptr()), P(nw.data_ptr()), ctypes.c_float(1e-6),
                                                     P(qg.data_ptr()), P(sg.data_ptr()), Fs, K1, G, 1, 2,
                                                     P(a1.xq.data_ptr()), P(a1.dx.data_ptr()), P(a1.xs.data_ptr()),
                                                     P(hs.data_ptr())]))
        fused.append(Launcher(lib, "wq_quant_gemv", [P(hs.data_ptr()), None, ctypes.c_float(0.0),
                                                     P(qd.data_ptr()), P(sd.data_ptr()), K1, Fs, G, 1, 1,
                                                     P(a2.xq.data_ptr()), P(a2.dx.data_ptr()), P(a2.xs.data_ptr()),
                                                     P(yres.data_ptr())]))
    t = graph_time(torch, fused, max(2, 128 // R), warm=settle_reps(fused)) * 2
    nb = nb_gu + 4 * Fs + Fs + 4 + 4 * (Fs // G) + nb_dn
    shard[f"cfg2_P8_gate_up_N{2 * Fs}_down_K{Fs}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1),
                                                     "launches": 2}
    del gu, dn
    res["shard_shapes"] = shard

    # the converter's native group size (G = 32, per-token activations) on
    # the cfg-1 / cfg-2 down GEMVs and the cfg-4 GEMM shape
    g32 = {}
    for M, K, N in ((1, 2048, 6144), (1, 6144, 2048), (8, 2048, 6144)):
        nb = gemv_bytes(M, K, N, 32)
        R = copies_for(nb)
        ws = rand_weights(torch, N, K, 32, R)
        a = ops.quant(torch.randn((M, K), dtype=torch.float32, device="cuda"), G=32)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        launches = [Launcher(lib, "wq_gemv", [P(q.data_ptr()), P(sc.data_ptr()), N, K, 32, P(a.xq.data_ptr()),
                                              P(a.dx.data_ptr()), P(a.xs.data_ptr()), M, K, 0, P(y.data_ptr())])
                    for q, sc in ws]
        t = graph_time(torch, launches, max(2, 256 // R), warm=settle_reps(launches))
        g32[f"gemv_M{M}_K{K}_N{N}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
        del ws
    M, K, N = 1024, 2048, 6144
    ws = rand_weights(torch, N, K, 32, 8)
    a = ops.quant(torch.randn((M, K), dtype=torch.float32, device="cuda"), G=32)
    ys = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(8)]
    launches = [Launcher(lib, "wq_gemm", [P(q.data_ptr()), P(sc.data_ptr()), N, K, 32, P(a.xq.data_ptr()),
                                          P(a.dx.data_ptr()), P(a.xs.data_ptr()), M, K, 0, P(ys[i].data_ptr()),
                                          None, None, 0])
                for i, (q, sc) in enumerate(ws)]
    graph_time(torch, launches, 50)
    t = graph_time(torch, launches, 10)
    g32[f"gemm_M{M}_K{K}_N{N}"] = {"us": round(t * 1e6, 2), "TOPS": round(2.0 * M * N * K / t / 1e12, 1)}
    del ws, ys
    res["group32"] = g32

    # the other producers of int8 activations: the MTP input stage
    # (mtp_in.wgsl, K = 2048) and the flash-decoding merge (attn_combine.wgsl,
    # 16 heads of 128, 4096-position context); inputs L2/MALL-resident, as
    # their producers just wrote them
    prod = {}
    Kh = 2048
    for M in (1, 2):
        emb = torch.randn((M, Kh), dtype=torch.float32, device="cuda")
        xh = torch.randn((M, Kh), dtype=torch.float32, device="cuda")
        nws = [torch.randn(Kh, dtype=torch.float32, device="cuda") for _ in range(3)]
        a = ops.empty_acts(M, 2 * Kh, 32, 32)
        ln = Launcher(lib, "wq_mtp_in", [P(emb.data_ptr()), P(xh.data_ptr())] + [P(t.data_ptr()) for t in nws] +
                      [ctypes.c_float(1e-6), M, Kh, P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr())])
        t = graph_time(torch, [ln] * 32, 8, warm=settle_reps([ln] * 32))
        nb = 4 * (2 * M * Kh + 3 * Kh) + 2 * M * Kh + 8 * (2 * M * Kh // 32)
        prod[f"mtp_in_M{M}_K{Kh}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
    Hh, Dh, nch = 16, 128, 128
    for M, pos in ((1, 511), (1, 4095 - 1), (2, 4094)):
        parts = []
        for _ in range(8):
            pt = torch.randn((M, Hh, nch, Dh + 2), dtype=torch.float32, device="cuda")
            pt[..., Dh + 1].uniform_(1.0, 32.0)
            parts.append(pt)
        a = ops.empty_acts(M, Hh * Dh, 32, G)
        lns = [Launcher(lib, "wq_attn_combine", [P(pt.data_ptr()), M, Hh, Dh, nch, pos, None, 0,
                                                 P(a.xq.data_ptr()), P(a.dx.data_ptr()), P(a.xs.data_ptr()),
                                                 None])
               for pt in parts]
        t = graph_time(torch, lns, 16, warm=settle_reps(lns))
        nread = sum(Hh * ((pos + m + 32) // 32) * (Dh + 2) * 4 for m in range(M))
        nb = nread + M * Hh * Dh + 8 * (M * Hh * Dh // 32)
        prod[f"attn_combine_M{M}_pos{pos}"] = {"us": round(t * 1e6, 3), "GBps": round(nb / t / 1e9, 1)}
        del parts
    res["producers"] = prod

    # decode step capture: 20 layers' linear sequences in one HIP graph
    # (webyiq_amd/layer.py: qkv, o, gate_up, down with their quantisers), the
    # layers sharing one residual stream
    from webyiq_amd.layer import DecodeLayer
    H, Q, KV, F, L = 2048, 2048, 512, 6144, 20
    step = {}
    for M, fuse, attention in ((1, True, "combine"), (2, True, "combine"), (4, True, "combine"),
                               (8, True, "combine"), (1, True, "copy"), (1, False, "copy")):
        x = torch.zeros((M, H), dtype=torch.float32, device="cuda")
        layers = []
        for _ in range(L):
            w = ops.Weights()
            for name, (r, c) in {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H),
                                 "down": (H, F)}.items():
                (q, sc), = rand_weights(torch, r, c, G, 1)
                w[name] = ops.Q4Tensor(q, sc, c, G)
            w["attn_norm"] = torch.ones(H, dtype=torch.float32, device="cuda")
            w["mlp_norm"] = torch.ones(H, dtype=torch.float32, device="cuda")
            layers.append(DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, fused=fuse, x=x,
                                      attention=attention))
        x0 = torch.randn((M, H), dtype=torch.float32, device="cuda")
        if M == 1 and fuse and attention == "combine":
            # gate: the first layer, fused, against the unfused sequence on the
            # same weights and partials (bit-identical) and its qkv against the
            # oracle (bit-exact)
            lay0 = layers[0]
            twin = DecodeLayer(lay0.w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, fused=False,
                               attention=attention)
            twin.part.copy_(lay0.part)
            x.copy_(x0)
            lay0.run()
            twin.x.copy_(x0)
            twin.run()
            torch.cuda.synchronize()
            wq0 = lay0.w.w("qkv")
            qq, qd, qs_ = orc.quant_act(x0.cpu().numpy(), None, G, norm_w=lay0.w["attn_norm"].cpu().numpy(),
                                        eps=1e-6)
            qkv_want = orc.linear(to_host_u32(wq0.q), to_host_u32(wq0.s), H, G, qq, qd, qs_)
            gates["decode_layer_M1"] = parity_gate(
                "decode layer M=1", np.array_equal(x.cpu().numpy().view(np.uint32),
                                                   twin.x.cpu().numpy().view(np.uint32))
                and np.array_equal(lay0.qkv.cpu().numpy().view(np.uint32), qkv_want.view(np.uint32)))
            del twin

        class Step:  # the graph_time launch protocol: one callable per captured unit
            def __call__(self, stream):
                x.copy_(x0)
                for lay in layers:
                    lay.run()
        # one replay is 100-160 launches: five replays settle the clocks
        t = graph_time(torch, [Step()], 10, warm=5 if CONFIG_SETTLE > 0 else 0)
        nbw = sum(lay.weight_bytes() for lay in layers)
        key = f"M{M}" + ("" if attention == "combine" else "_copy_attn") + ("" if fuse else "_unfused")
        # qkv, gate_up, down: quantiser + GEMV, one launch when fused and M <= 2;
        # o: a plain GEMV after the chunk merge, or quantiser + GEMV after the copy
        per_pair = 1 if fuse and M <= 2 else 2
        launches = 3 * per_pair + 1 + (1 if attention == "combine" else per_pair)
        step[key] = {"us_per_layer": round(t / L * 1e6, 3), "layers": L, "launches_per_layer": launches,
                     "attention_stand_in": attention, "weight_GBps": round(nbw / t / 1e9, 1)}
        del layers
    res["decode_step_graph"] = step
    res["parity_gates"] = {"checked": len(gates), "all_passed": all(gates.values())}
    torch.cuda.empty_cache()
    return res


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, plus the family
    and model numbers (a virtualised host may give only a generic name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k in ("model name", "cpu family", "model", "vendor_id") and k not in info:
                    info[k] = v.strip()
                if not line.strip() and info:
                    break
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    if "cpu family" in info:
        name += f" (family {info['cpu family']}, model {info.get('model', '?')})"
    return name


def cpu_baseline(torch, ref, wq, ws, K, G, x, nbytes, seconds):
    """The reference's CPU torch fake-quant path (tools/reference.py:35-52,
    restated in oracle/reference.py) on bounded samples of the BASELINE
    workloads, on this host's cores: the headline cfg 1 GEMV (about half of
    `seconds`) and, under "configs", cfg 2 (decode MLP chain), cfg 4 (the
    M=1024 prefill products) and cfg 5 (lm_head + argmax, V=151,936), each
    timed for about `seconds` / 6.

    Threads: the GPU pool gives each GPU's job a share of the host's cores
    (16 on a one-GPU box, exported as OMP_NUM_THREADS); os.cpu_count() there
    counts every core of the host, most of them other jobs'.  torch runs
    with OMP_NUM_THREADS threads, capped at the cores this process may run
    on (its affinity set); `cores` is the count torch used, and the line
    also states os.cpu_count() and the affinity count."""
    ncpu = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = ncpu
    threads = int(os.environ.get("OMP_NUM_THREADS", affinity))
    threads = max(1, min(threads, affinity))
    torch.set_num_threads(threads)
    used = torch.get_num_threads()
    lin = ref.FakeQuantLinear(wq, ws, K, G)
    xt = torch.from_numpy(x)
    med, n = ref.time_cpu(lambda: lin(xt), warmup=3, iters=1000, max_seconds=seconds / 2)
    out = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": used, "kind": "port",
           "cpu_model": cpu_model(), "os_cpu_count": ncpu, "affinity_cores": affinity,
           "threads_from": "OMP_NUM_THREADS (the pool's per-GPU core share)" if "OMP_NUM_THREADS" in os.environ
           else "affinity set",
           "us_per_gemv": round(med * 1e6, 1),
           "sample": f"median of {n} fake-quant GEMVs (M=1 K=2048 N=6144: fq_input + fp32 x@W^T, "
                     "W dequantised once as tools/reference.py:36-40), ~%.0f s bounded" % (seconds / 2)}

    # the other configurations: timing does not depend on the weight values,
    # so the dequantised weights (what tools/reference.py holds after load)
    # are random fp32 values directly instead of going through RTN
    g = torch.Generator().manual_seed(0)
    per = seconds / 6

    def weights(rows, cols):
        # a 4096-row random block tiled to size (drawing 300 M normals takes ~15 s)
        blk = torch.randn((min(rows, 4096), cols), generator=g) * 0.02
        return blk.repeat((rows + blk.shape[0] - 1) // blk.shape[0], 1)[:rows].contiguous()

    def fq_lin(xx, w):
        return ref.fq_input(xx) @ w.T

    cfgs = {}
    # cfg 2: norm-free decode MLP block at M=1: gate_up, SiLU*up, re-quant, down (+= residual)
    wgu = weights(2 * 6144, 2048)
    wdn = weights(2048, 6144)
    x1 = torch.randn((1, 2048), generator=g)
    res = torch.zeros((1, 2048))

    def mlp():
        a = fq_lin(x1, wgu)
        hh = torch.nn.functional.silu(a[:, :6144]) * a[:, 6144:]
        return res + fq_lin(hh, wdn)
    med, n = ref.time_cpu(mlp, warmup=2, iters=1000, max_seconds=per)
    cfgs["cfg2_decode_mlp_block"] = {"us": round(med * 1e6, 1), "GBps": round(20126156 / med / 1e9, 3),
                                     "sample": f"median of {n} blocks"}
    del wgu, wdn
    # cfg 4: the M=1024 prefill products
    for Kp, Np in ((2048, 6144), (6144, 2048)):
        w = weights(Np, Kp)
        xp = torch.randn((1024, Kp), generator=g)
        med, n = ref.time_cpu(lambda: fq_lin(xp, w), warmup=1, iters=50, max_seconds=per)
        cfgs[f"cfg4_prefill_K{Kp}_N{Np}"] = {"us": round(med * 1e6, 1),
                                             "TOPS": round(2.0 * 1024 * Np * Kp / med / 1e12, 4),
                                             "sample": f"median of {n} fake-quant products, M=1024"}
        del w, xp
    # cfg 5: lm_head + greedy argmax, M=1, V=151,936
    wh = weights(151936, 2048)
    med, n = ref.time_cpu(lambda: ref.argmax_ref(fq_lin(x1, wh)), warmup=1, iters=200, max_seconds=per)
    cfgs["cfg5_lm_head_argmax_M1_V151936"] = {"us": round(med * 1e6, 1),
                                              "GBps": round(165308488 / med / 1e9, 3),
                                              "sample": f"median of {n} heads"}
    del wh
    out["configs"] = cfgs
    return out


if __name__ == "__main__":
    main()
