"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle
on the same seeded inputs.

Bars (stated per test):
  * int8 codes, dx, xs, int32 group sums, argmax tokens: bit-exact;
  * GEMV fp32 outputs of modes 0/1: bit-exact against the oracle, which
    restates the GEMV's fold order;
  * GEMM fp32 outputs (per-token activations at G = 128 and 32 fold the min
    term separately on an f16 MFMA; per-32 activations fold one chain per
    output against the GEMV's chains and tree) and mode 2 (device expf vs
    libm expf): within rel 1e-5 (max-norm) of the oracle;
  * every fp32 output within rel 1e-3 (max-norm) of the torch fake-quant path.
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import reference as ref
from webyiq_amd import ops
from conftest import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def note(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def dev_acts(xq, dx, xs, GA, G):
    return ops.Acts(dev(xq), dev(dx), dev(xs), GA, G)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def setup_linear(seed, M, K, rows, G, GA):
    rng = np.random.default_rng(seed)
    wq, ws = ref.make_weight(rng, rows, K, G)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, GA, G)
    return wq, ws, x, xq, dx, xs


def oracle_linear_tokens(wq, ws, K, G, xq, dx, xs, mode=0, y=None, GA=None, threads=16):
    """orc.linear over token slices in a thread pool (the C oracle releases
    the GIL), for checks of every token of a prefill-sized product."""
    from concurrent.futures import ThreadPoolExecutor
    M = xq.shape[0]
    n = max(1, min(threads, os.cpu_count() or 1, M))
    cuts = np.linspace(0, M, n + 1).astype(int)

    def part(i):
        a, b = cuts[i], cuts[i + 1]
        return orc.linear(wq, ws, K, G, xq[a:b], dx[a:b], xs[a:b], mode=mode,
                          y=None if y is None else y[a:b], GA=GA)
    with ThreadPoolExecutor(n) as ex:
        return np.concatenate(list(ex.map(part, range(n))), 0)


# ------------------------------------------------------------- quantiser ----

@pytest.mark.parametrize("M,K,GA,G,norm", [
    (1, 2048, None, 128, False), (3, 6144, None, 128, False), (8, 2048, None, 32, False),
    (5, 1024, 32, 128, False), (2, 128, None, 128, False), (64, 2048, None, 128, False),
    (4, 2048, None, 128, True), (3, 6144, 32, 32, True),
    (1, 2176, None, 32, True), (2, 10240, None, 128, True),   # partial pass; rows past 4 passes
    (48, 4096, 32, 128, True), (40, 12288, None, 32, True),   # one wave per token: 2 and 6 passes
])
def test_quant_act_bit_exact(M, K, GA, G, norm):
    note(f"quant M={M} K={K} GA={GA} G={G} norm={norm}")
    rng = np.random.default_rng(M * 7 + K)
    x = ref.make_activations(rng, M, K)
    x[M - 1, : K // 2] = 0.0 if M > 1 else x[M - 1, : K // 2]
    nw = rng.normal(1.0, 0.2, size=K).astype(np.float32) if norm else None
    xq, dx, xs = orc.quant_act(x, GA, G, norm_w=nw, eps=1e-6)
    a = ops.quant(dev(x), norm=None if nw is None else dev(nw), eps=1e-6, GA=GA, G=G)
    assert np.array_equal(host(a.xq), xq)
    assert np.array_equal(host(a.dx).view(np.uint32), dx.view(np.uint32))
    assert np.array_equal(host(a.xs), xs)


def test_quant_zero_rows_and_ties():
    note("quant zero rows / ties")
    x = np.zeros((3, 256), np.float32)
    x[0, :6] = [127.0, 2.5, 3.5, -2.5, 0.5, -126.5]
    x[2] = np.linspace(-3, 3, 256, dtype=np.float32)
    for GA in (None, 32):
        xq, dx, xs = orc.quant_act(x, GA, 128)
        a = ops.quant(dev(x), GA=GA, G=128)
        assert np.array_equal(host(a.xq), xq)
        assert np.array_equal(host(a.dx), dx)
        assert np.array_equal(host(a.xs), xs)


def _half_boundary_rows(K):
    """Rows whose every 32-group starts with the row's absmax (so per-token
    and per-32 scales agree), followed by values within 3 ulps of the
    half-integer code boundaries (k + 0.5) * d: ties, and the cases where a
    quotient computed without a division would round the other way."""
    rows = []
    for amax in (np.float32(127.0), np.float32(3.7), np.float32(1e-3)):
        d = np.float32(amax / np.float32(127.0))
        vals = []
        for k in range(-127, 127):
            h = np.float32((np.float32(k) + np.float32(0.5)) * d)
            for j in range(-3, 4):
                v = h
                for _ in range(abs(j)):
                    v = np.nextafter(v, np.float32(np.inf if j > 0 else -np.inf), dtype=np.float32)
                if abs(v) <= amax:
                    vals.append(v)
        vals = np.array(vals, np.float32)
        row = np.resize(vals, (K // 32, 31))
        row = np.concatenate([np.full((K // 32, 1), amax, np.float32), row], 1).reshape(K)
        rows.append(row)
    return np.stack(rows)


def test_quant_half_boundaries():
    """Codes at and around the rounding boundaries, bit-exact against the
    oracle's IEEE division: quant_act (per token and per 32) and the fused
    quantiser of wq_quant_gemv."""
    note("quant half-integer boundaries")
    K, N = 2048, 256
    x = _half_boundary_rows(K)
    for GA in (None, 32):
        xq, dx, xs = orc.quant_act(x, GA, 128)
        a = ops.quant(dev(x), GA=GA, G=128)
        assert np.array_equal(host(a.xq), xq)
        assert np.array_equal(host(a.xs), xs)
    rng = np.random.default_rng(5)
    wq, ws = ref.make_weight(rng, N, K, 128)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, 128)
    xq, dx, xs = orc.quant_act(x[:2], None, 128)
    y, a = ops.quant_gemv(w, dev(x[:2]))
    assert np.array_equal(host(a.xq), xq)
    assert np.array_equal(host(y).view(np.uint32), orc.linear(wq, ws, K, 128, xq, dx, xs).view(np.uint32))


# ------------------------------------------------------------------ GEMV ----

GEMV_CASES = [
    # M, K, N, G, GA(None = per token), mode
    (1, 2048, 6144, 128, None, 0),   # BASELINE cfg 1 shape
    (1, 2048, 2048, 128, None, 1),
    (1, 6144, 2048, 128, None, 1),   # cfg 2 down
    (1, 2048, 6144, 128, None, 2),   # cfg 2 gate_up (2 x 6144 rows)
    (2, 2048, 512, 128, None, 0),    # cfg 3 k/v
    (3, 2048, 1000, 128, None, 0),   # ragged N, M rounded up to 4
    (4, 6144, 2048, 128, None, 0),
    (8, 2048, 6144, 128, None, 2),
    (8, 6144, 2048, 128, None, 1),
    (1, 128, 77, 128, None, 0),      # one group, partial pass
    (5, 1024, 300, 32, None, 0),
    (2, 2048, 256, 32, 32, 1),       # reference-native: G = 32, GA = 32
    (3, 4096, 130, 128, 32, 2),
    (7, 3072, 96, 32, None, 0),      # K not a multiple of 2048
    # 3..8 tokens, N >= 16384: the int8-MFMA GEMV (row blocks of 16, K split
    # between waves when K > 2048)
    (8, 2048, 16400, 128, None, 0),  # ragged last block
    (5, 6144, 16384, 128, None, 1),  # K split in 4
    (3, 2048, 20000, 128, None, 2),  # gate/up pairs
    (6, 1024, 16384, 128, None, 1),  # 8 groups per row, += residual
    (4, 4096, 16384, 128, None, 0),  # K split in 2
    (7, 2048, 16384, 128, None, 2),  # tokens 0..6 of the two-token lane map
    (4, 2048, 16500, 128, None, 1),
    # the limits the host checks: 8 tokens x K = 16384 (8 passes) on the dot4
    # kernel, the MFMA GEMV at its K = 8192, and K = 16384 in the
    # reference-native format
    (8, 16384, 512, 128, None, 1),
    (8, 8192, 16384, 128, None, 0),
    (1, 16384, 6144, 32, 32, 0),
    # three rows per wave: the plan for 2 x 768 < N / 4 <= 3 x 768 (K <= 2048)
    (1, 2048, 8192, 128, None, 0),
    (2, 2048, 8192, 128, None, 2),
    (8, 1536, 7000, 128, None, 1),   # partial pass, ragged last block
    # the o projection after the chunk merge (per-32 activations, += residual)
    # at the decode-layer shape, 1 and 8 tokens
    (1, 2048, 2048, 128, 32, 1),
    (8, 2048, 2048, 128, 32, 1),
    # the specialised one-pass kernel at 2..8 tokens (token slots 2, 4, 8;
    # padding slots re-read the last token and store nothing), within its
    # rule of at most eight folds per wave, ragged N included
    (2, 2048, 6144, 128, None, 1),
    (2, 2048, 6144, 128, None, 2),
    (4, 2048, 6144, 128, None, 0),   # two rows per wave
    (5, 2048, 2048, 128, None, 1),
    (6, 2048, 512, 128, None, 0),
    (7, 2048, 3000, 128, None, 0),
]


@pytest.mark.parametrize("M,K,N,G,GA,mode", GEMV_CASES)
def test_gemv_bit_exact(M, K, N, G, GA, mode):
    note(f"gemv M={M} K={K} N={N} G={G} GA={GA} mode={mode}")
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(M * 1000 + N, M, K, rows, G, GA)
    gaa = K if GA is None else GA
    y0 = np.random.default_rng(1).normal(size=(M, N)).astype(np.float32) if mode == 1 else None
    want = orc.linear(wq, ws, K, G, xq, dx, xs, mode=mode, y=y0, GA=gaa)
    acc_want = orc.group_acc(wq, K, min(G, gaa), xq)

    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, gaa, G)
    y = dev(y0) if mode == 1 else None
    y, acc = ops.group_sums(ops.PATH_SPEC, w, a, mode=mode, y=y)
    assert np.array_equal(host(acc), acc_want)
    got = host(y)
    if mode == 2:
        assert rel_err(got, want) < 1e-5
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the plain entry point computes the same values
    y2 = ops.gemv(w, a, mode=mode, y=dev(y0) if mode == 1 else None)
    assert np.array_equal(host(y2), got)
    # and the torch fake-quant reference agrees within the stated tolerance
    fq = ref.FakeQuantLinear(wq, ws, K, G, mode=mode, GA=GA)(x, y0).numpy()
    assert rel_err(got, fq) < 1e-3


# MTP speculative verify: the 7 linear shapes of one
# 2B-style layer at M = 2, 4, 8 -- q (2048 -> 2048), k and v (2048 -> 512),
# o (2048 -> 2048, += residual), gate and up (2048 -> 6144, as two plain
# products and as the fused gate_up pair), down (6144 -> 2048, += residual)
VERIFY_SHAPES = [("q", 2048, 2048, 0), ("k_v", 2048, 512, 0), ("o", 2048, 2048, 1),
                 ("gate_or_up", 2048, 6144, 0), ("gate_up", 2048, 6144, 2), ("down", 6144, 2048, 1)]


@pytest.mark.parametrize("M", [2, 4, 8])
@pytest.mark.parametrize("name,K,N,mode", VERIFY_SHAPES)
def test_cfg3_verify_shapes(M, name, K, N, mode):
    """Every (M, K x N) pair of configs[2] at group 128, per-token int8: int32
    group sums bit-exact, fp32 bit-exact against the oracle (mode 2 within
    rel 1e-5: device expf), within rel 1e-3 of the torch fake-quant path."""
    note(f"cfg3 {name} M={M} K={K} N={N} mode={mode}")
    G = 128
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(M * 7919 + K + N + mode, M, K, rows, G, None)
    y0 = np.random.default_rng(M + N).normal(size=(M, N)).astype(np.float32) if mode == 1 else None
    want = orc.linear(wq, ws, K, G, xq, dx, xs, mode=mode, y=y0)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, K, G)
    y, acc = ops.group_sums(ops.PATH_SPEC, w, a, mode=mode, y=dev(y0) if mode == 1 else None)
    assert np.array_equal(host(acc), orc.group_acc(wq, K, G, xq))
    got = host(y)
    if mode == 2:
        assert rel_err(got, want) < 1e-5
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y2 = host(ops.gemv(w, a, mode=mode, y=dev(y0) if mode == 1 else None))
    assert np.array_equal(y2.view(np.uint32), got.view(np.uint32))
    fq = ref.FakeQuantLinear(wq, ws, K, G, mode=mode)(x, y0).numpy()
    assert rel_err(got, fq) < 1e-3


# ------------------------------------------------------------------ GEMM ----

GEMM_CASES = [
    (256, 2048, 512, 128, None, 0),
    (100, 2048, 384, 128, None, 1),   # ragged M tile
    (130, 6144, 256, 128, None, 0),
    (64, 2048, 192, 128, None, 2),
    (33, 1024, 100, 128, None, 0),    # ragged N tile
    (96, 2048, 256, 32, 32, 0),       # reference-native groups
    (17, 512, 64, 32, None, 1),
    (48, 1024, 128, 128, 32, 2),
    (1, 128, 16, 128, None, 0),
    (200, 2048, 320, 128, None, 2),   # mode 2 at width 256
    (129, 1024, 130, 32, None, 0),
    (300, 6144, 2048, 128, None, 1),  # down-projection shape, tile width 64
    (64, 4096, 256, 128, None, 2),    # 32 steps: scale words preloaded, gate/up pairs
    (70, 3072, 192, 128, None, 0),    # 3 min-term blocks over two wave groups
    (40, 2176, 130, 128, None, 1),    # 17 groups: min-term blocks word by word
]


@pytest.mark.parametrize("M,K,N,G,GA,mode", GEMM_CASES)
def test_gemm_bit_exact(M, K, N, G, GA, mode):
    note(f"gemm M={M} K={K} N={N} G={G} GA={GA} mode={mode}")
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(M * 31 + N, M, K, rows, G, GA)
    gaa = K if GA is None else GA
    y0 = np.random.default_rng(2).normal(size=(M, N)).astype(np.float32) if mode == 1 else None
    want = orc.linear(wq, ws, K, G, xq, dx, xs, mode=mode, y=y0, GA=gaa)
    acc_want = orc.group_acc(wq, K, min(G, gaa), xq)

    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, gaa, G)
    y, acc = ops.group_sums(ops.PATH_PREFILL, w, a, mode=mode, y=dev(y0) if mode == 1 else None)
    assert np.array_equal(host(acc), acc_want)
    got = host(y)
    # f16-MFMA min term (per-token activations), device expf (mode 2), or
    # (per-32 activations) the GEMM's single fold chain against the GEMV's
    # chains-and-tree order
    assert rel_err(got, want) < 1e-5
    # the plain entry point (its own tile width) computes the same values
    y2 = host(ops.gemm(w, a, mode=mode, y=dev(y0) if mode == 1 else None))
    assert np.array_equal(y2.view(np.uint32), got.view(np.uint32))
    fq = ref.FakeQuantLinear(wq, ws, K, G, mode=mode, GA=GA)(x, y0).numpy()
    assert rel_err(got, fq) < 1e-3


# tile width the launcher picks for M = 1024 (8 tiles along M): 192, 256, 128,
# 256 (mode 2), 64; the other formats at width 128
WIDE_CASES = [
    (2048, 6144, 128, None, 0),
    (4096, 6144, 128, None, 0),   # tile width 192, min-term blocks reloaded
    (2048, 8192, 128, None, 0),
    (2048, 4096, 128, None, 0),
    (2048, 4096, 128, None, 2),
    (6144, 2048, 128, None, 1),
    (2048, 4096, 32, None, 0),
    (2048, 4096, 128, 32, 1),
]


@pytest.mark.parametrize("K,N,G,GA,mode", WIDE_CASES)
def test_gemm_wide_tiles(K, N, G, GA, mode):
    """Prefill shapes (M = 1024) on the production tile widths against the
    oracle: every row of the first and the last 128-token tile, and one row
    of every 8-row group of the other tiles (row 8 g + tile index), so each
    (wave, subtile, row group, lane) position of the tile layout is read."""
    M = 1024
    note(f"gemm wide M={M} K={K} N={N} G={G} GA={GA} mode={mode}")
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(K + N + G + mode, M, K, rows, G, GA)
    gaa = K if GA is None else GA
    y0 = np.random.default_rng(3).normal(size=(M, N)).astype(np.float32) if mode == 1 else None
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, gaa, G)
    got = host(ops.gemm(w, a, mode=mode, y=dev(y0) if mode == 1 else None))
    idx = np.unique(np.concatenate([np.arange(0, 128), np.arange(M - 128, M),
                                    np.arange(0, M, 8) + (np.arange(0, M, 8) // 128) % 8]))
    want = oracle_linear_tokens(wq, ws, K, G, xq[idx], dx[idx], xs[idx], mode=mode,
                                y=y0[idx] if mode == 1 else None, GA=gaa)
    assert rel_err(got[idx], want) < 1e-5
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("M", [256, 512, 2048])
@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048)])
def test_gemm_prefill_sizes(M, K, N):
    """The other prefill sizes, whose tile widths and grids differ from
    M = 1024's (width 128 at M = 512 and 192 at M = 2048 for N = 6144, 64
    elsewhere; two rounds of workgroups at M = 2048): every row of the first
    and the last tile and one row of every 8-row group, against the oracle."""
    note(f"gemm prefill M={M} K={K} N={N}")
    wq, ws, x, xq, dx, xs = setup_linear(K + N + M, M, K, N, 128, None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, 128)
    got = host(ops.gemm(w, dev_acts(xq, dx, xs, K, 128)))
    idx = np.unique(np.concatenate([np.arange(0, 128), np.arange(M - 128, M),
                                    np.arange(0, M, 8) + (np.arange(0, M, 8) // 128) % 8]))
    want = oracle_linear_tokens(wq, ws, K, 128, xq[idx], dx[idx], xs[idx])
    assert rel_err(got[idx], want) < 1e-5
    assert np.all(np.isfinite(got))


SPLIT_CASES = [
    # M, K, N, G, mode: shapes whose plan splits K between workgroup pairs
    (1024, 6144, 2048, 128, 0),   # width 128, 256 workgroups
    (512, 6144, 2048, 128, 1),    # width 64, += residual
    (256, 6144, 2048, 128, 0),
    (512, 4096, 1024, 128, 2),    # gate/up pairs (width 128)
    (384, 4096, 2048, 32, 0),     # per-token group 32
    (200, 8192, 640, 128, 1),     # ragged token and row tiles, 32 steps per half
]


@pytest.mark.parametrize("M,K,N,G,mode", SPLIT_CASES)
def test_gemm_split_k(M, K, N, G, mode):
    """K split between workgroup pairs (wq_gemm with a workspace): against the
    oracle within rel 1e-5 on every row of the first and last tile and one of
    every 8 elsewhere; within rel 1e-5 of the unsplit launch; bit-identical
    over repeated calls (the two partials are added in one fixed order); the
    workspace's flags zero again after every call; and with device Params at
    m below the capacity, the rows past m untouched."""
    note(f"gemm split-K M={M} K={K} N={N} G={G} mode={mode}")
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(M + K + N + mode, M, K, rows, G, None)
    y0 = np.random.default_rng(4).normal(size=(M, N)).astype(np.float32) if mode == 1 else None
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, K, G)
    nws = ops._lib.load().wq_gemm_workspace_bytes(N, K, G, M, K, mode)
    assert nws > 0, "this shape should split"
    wsp = ops.gemm_workspace(N, K, G, M, mode=mode)
    runs = [host(ops.gemm(w, a, mode=mode, y=dev(y0) if mode == 1 else None, workspace=wsp)) for _ in range(3)]
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    # the plan's tile count from the workspace size (flag lines, then 128 x
    # width partial sums per tile)
    plans = [(bn, ((M + 127) // 128) * -(-N // (bn // 2 if mode == 2 else bn))) for bn in (64, 128)]
    T = [t for bn, t in plans if -(-64 * t // 256) * 256 + t * 128 * bn * 4 == nws]
    assert len(T) == 1, (nws, plans)
    T = T[0]

    def flags_clear():
        return not host(wsp[: 64 * T]).view(np.uint32)[::16].any()
    assert flags_clear(), "flags left set"
    got = runs[0]
    unsplit = host(ops.gemm(w, a, mode=mode, y=dev(y0) if mode == 1 else None))
    assert rel_err(got, unsplit) < 1e-5
    idx = np.unique(np.concatenate([np.arange(0, min(128, M)), np.arange(max(0, M - 128), M),
                                    np.arange(0, M, 8) + (np.arange(0, M, 8) // 128) % 8]))
    idx = idx[idx < M]
    want = oracle_linear_tokens(wq, ws, K, G, xq[idx], dx[idx], xs[idx], mode=mode,
                                y=y0[idx] if mode == 1 else None)
    assert rel_err(got[idx], want) < 1e-5
    # device Params below the capacity: the pairs of tiles past m both end
    m = M // 2 + 3
    base = y0 if mode == 1 else np.full((M, N), np.nan, np.float32)
    y = dev(base)
    ops.gemm(w, a, mode=mode, y=y, workspace=wsp, params=ops.make_params(m=m))
    gp = host(y)
    assert np.array_equal(gp[:m].view(np.uint32), got[:m].view(np.uint32))
    assert np.array_equal(gp[m:].view(np.uint32), base[m:].view(np.uint32))
    assert flags_clear()


@pytest.mark.parametrize("M,mode,stride", [(2048, 0, 8), (4096, 2, 32)])
def test_gemm_group32_wide_widths(M, mode, stride):
    """Per-token activations at group 32 on the widths the launcher picks for
    long prompts: 192 at M = 2048, N = 6144 (three columns per wave, the
    columns' fragments read up front) and 256 in mode 2 at M = 4096 (four
    columns, read column by column).  Every row of the first and the last
    tile and one row per `stride` elsewhere (offset rotating with the tile),
    against the oracle at rel 1e-5."""
    K, N, G = 2048, 6144, 32
    note(f"gemm group-32 M={M} K={K} N={N} mode={mode}")
    rows = 2 * N if mode == 2 else N
    wq, ws, x, xq, dx, xs = setup_linear(M + mode, M, K, rows, G, None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    got = host(ops.gemm(w, dev_acts(xq, dx, xs, K, G), mode=mode))
    base = np.arange(0, M, stride)
    idx = np.unique(np.concatenate([np.arange(0, 128), np.arange(M - 128, M),
                                    base + (base // 128) % stride]))
    want = oracle_linear_tokens(wq, ws, K, G, xq[idx], dx[idx], xs[idx], mode=mode)
    assert rel_err(got[idx], want) < 1e-5
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048)])
def test_gemm_prefill_production_int32(K, N):
    """BASELINE configs[3] at the production tile width (the one the
    launcher picks for M = 1024): the int32 group sums of all 1,024 tokens
    bit-exact against an exact integer reference (one float64 product per
    group, exact for these magnitudes), and the fp32 output of all 1,024
    tokens within rel 1e-5 of the oracle.  The sums come from the dump
    hook, a sibling instance of the same template (DUMP set); its fp32
    output is checked bit-identical to the production instance's below,
    which ties the sums to the production kernel."""
    M, G = 1024, 128
    note(f"gemm production int32 M={M} K={K} N={N}")
    wq, ws, x, xq, dx, xs = setup_linear(K * 3 + N, M, K, N, G, None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, K, G)
    y, acc = ops.group_sums(ops.PATH_PREFILL, w, a)
    got_acc = host(acc)
    q = orc.q4_unpack(wq, K).astype(np.float64)
    xf = xq.astype(np.float64)
    for g in range(K // G):
        sl = slice(g * G, (g + 1) * G)
        exact = xf[:, sl] @ q[:, sl].T
        assert np.array_equal(got_acc[:, :, g], exact.astype(np.int32)), f"group {g}"
    del got_acc, acc
    got = host(y)
    want = oracle_linear_tokens(wq, ws, K, G, xq, dx, xs)
    assert rel_err(got, want) < 1e-5
    # the production instance (plain entry point) gives the same bits
    y2 = host(ops.gemm(w, a))
    assert np.array_equal(y2.view(np.uint32), got.view(np.uint32))


def test_gemm_long_rows_partial_tile_group():
    """K >= 4096 assigns tiles to XCDs in groups of 4 token tiles; M = 640
    has 5 token tiles, so one full group and a partial one.  Sampled tokens
    of every token tile against the oracle."""
    M, K, N = 640, 4096, 1024
    note(f"gemm long rows M={M} K={K} N={N}")
    wq, ws, x, xq, dx, xs = setup_linear(641, M, K, N, 128, None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, 128)
    got = host(ops.gemm(w, dev_acts(xq, dx, xs, K, 128)))
    idx = np.array([0, 127, 128, 255, 300, 383, 384, 511, 512, 600, 639])
    want = orc.linear(wq, ws, K, 128, xq[idx], dx[idx], xs[idx])
    assert rel_err(got[idx], want) < 1e-5
    assert np.all(np.isfinite(got))


def test_gemm_matches_gemv_rows():
    """Decode vs prefill cross-check (the reference's --ppl / --sequential
    harnesses, crates/cli/src/main.rs:209-250): each GEMM row matches the GEMV
    of that token to rel 1e-5 (the GEMM folds the min term on an f16 MFMA)."""
    note("gemm vs gemv rows")
    M, K, N = 40, 2048, 1024
    wq, ws, x, xq, dx, xs = setup_linear(5, M, K, N, 128, None)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, 128)
    a = dev_acts(xq, dx, xs, K, 128)
    yg = host(ops.matmul(ops.PATH_PREFILL, w, a))
    for t0 in range(0, M, 8):
        sub = dev_acts(xq[t0:t0 + 8], dx[t0:t0 + 8], xs[t0:t0 + 8], K, 128)
        yv = host(ops.matmul(ops.PATH_SPEC, w, sub))
        assert rel_err(yg[t0:t0 + 8], yv) < 1e-5


# -------------------------------------------------------------- argmax ------

def test_argmax_standalone():
    note("argmax standalone")
    rng = np.random.default_rng(3)
    v = rng.normal(size=(4, 151936)).astype(np.float32)
    v[1, [5, 77777, 150000]] = 50.0
    v[2, 9] = np.nan
    v[3, :] = -np.inf
    ids = np.arange(151936, dtype=np.uint32)[::-1].copy()
    got = host(ops.argmax(dev(v))).astype(np.uint32)
    assert np.array_equal(got, orc.argmax(v))
    got = host(ops.argmax(dev(v), ids=dev(ids.view(np.int32)))).astype(np.uint32)
    assert np.array_equal(got, orc.argmax(v, ids))


@pytest.mark.parametrize("M,V,G,mapped", [(1, 32768, 128, False), (8, 32768, 128, True),
                                          (3, 5000, 32, False), (1, 151936, 128, False),
                                          (5, 20000, 128, False), (8, 151936, 128, False)])
def test_lm_head_argmax(M, V, G, mapped):
    note(f"lm_head M={M} V={V} G={G} mapped={mapped}")
    K = 2048
    wq, ws, x, xq, dx, xs = setup_linear(V + M, M, K, V, G, None)
    # plant exact ties: duplicate the winner's row at a lower and a higher index
    logits = orc.linear(wq, ws, K, G, xq, dx, xs)
    win = int(orc.argmax(logits)[0])
    lo, hi = max(0, win // 2 - 1), min(V - 1, win + 3)
    wq[lo], ws[lo] = wq[win], ws[win]
    wq[hi], ws[hi] = wq[win], ws[win]
    logits = orc.linear(wq, ws, K, G, xq, dx, xs)
    ids = np.sort(np.random.default_rng(4).choice(151936, V, replace=False)).astype(np.uint32) if mapped else None
    want = orc.argmax(logits, ids)
    assert want[0] == (ids[lo] if mapped else lo)

    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    a = dev_acts(xq, dx, xs, K, G)
    lg = torch.empty((M, V), dtype=torch.float32, device=DEV)
    ws_dev = ops.lm_head_workspace()
    d_ids = dev(ids.view(np.int32)) if mapped else None
    tok = ops.lm_head_argmax(w, a, ids=d_ids, logits=lg, workspace=ws_dev)
    assert np.array_equal(host(tok).astype(np.uint32), want)
    assert np.array_equal(host(lg).view(np.uint32), logits.view(np.uint32))
    # second call on the same workspace (it must have been left zeroed), no logits
    tok2 = ops.lm_head_argmax(w, a, ids=d_ids, workspace=ws_dev)
    assert np.array_equal(host(tok2).astype(np.uint32), want)
    assert np.all(host(ws_dev) == 0)


# ------------------------------------------------------- MLP block (cfg 2) --

def test_decode_mlp_block():
    """gate_up (mode 2) -> per-token re-quant -> down (mode 1), graph.rs:318-328."""
    note("mlp block")
    hd, ffn = 2048, 6144
    rng = np.random.default_rng(11)
    wgu, sgu = ref.make_weight(rng, 2 * ffn, hd, 128)
    wd, sd = ref.make_weight(rng, hd, ffn, 128)
    x = ref.make_activations(rng, 1, hd)
    resid = rng.normal(size=(1, hd)).astype(np.float32)

    xq, dx, xs = orc.quant_act(x, None, 128)
    h_want = orc.linear(wgu, sgu, hd, 128, xq, dx, xs, mode=2)

    a = ops.quant(dev(x), G=128)
    h = ops.gemv(ops.Q4Tensor.from_numpy(wgu, sgu, hd, 128), a, mode=2)
    h_got = host(h)
    assert rel_err(h_got, h_want) < 1e-5
    # re-quant of the device h is bit-exact against the oracle on the same h
    a2 = ops.quant(h, G=128)
    hq, hdx, hxs = orc.quant_act(h_got, None, 128)
    assert np.array_equal(host(a2.xq), hq)
    y = dev(resid)
    ops.gemv(ops.Q4Tensor.from_numpy(wd, sd, ffn, 128), a2, mode=1, y=y)
    want = orc.linear(wd, sd, ffn, 128, hq, hdx, hxs, mode=1, y=resid)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    # torch fake-quant chain
    gu = ref.FakeQuantLinear(wgu, sgu, hd, 128, mode=2)(x)
    out = ref.FakeQuantLinear(wd, sd, ffn, 128, mode=1)(gu, resid).numpy()
    assert rel_err(host(y), out) < 1e-3


# ------------------------------------------- fused quantiser + GEMV -------

QUANT_GEMV_CASES = [
    # M, K, N, G, mode, norm
    (1, 2048, 6144, 128, 0, True),   # norm_quant -> qkv / lm_head shape
    (1, 6144, 2048, 128, 1, False),  # quant -> down (+= residual)
    (2, 2048, 6144, 128, 2, True),   # norm_quant -> gate_up (SiLU * up)
    (1, 128, 77, 128, 0, False),     # one group, partial pass
    (2, 3072, 96, 32, 0, True),      # K not a multiple of 2048, G = 32
    (1, 16384, 256, 128, 1, True),   # eight passes
    (5, 2048, 512, 128, 0, True),    # M > 2: quantiser and GEMV launches
    (4, 2048, 3072, 128, 2, True),   # 4 tokens, gate_up
    (8, 2048, 2048, 32, 1, False),   # 8 tokens, G = 32, += residual
    (3, 128, 300, 128, 0, True),     # 3 tokens, one group, partial pass
    (6, 6144, 512, 128, 1, False),
    # the instances the bench times (cfg 2 and the decode layers at
    # hidden 2048, q 2048, kv 512, ffn 6144): norm+quant -> qkv (3072 rows),
    # norm+quant -> gate_up (2 x 6144 rows), quant -> down, at 1, 2, 4, 8 tokens
    (1, 2048, 6144, 128, 2, True),   # cfg 2 gate_up, one launch (3 rows per wave)
    (1, 2048, 3072, 128, 0, True),
    (2, 2048, 3072, 128, 0, True),
    (2, 6144, 2048, 128, 1, False),
    (4, 2048, 3072, 128, 0, True),
    (4, 2048, 6144, 128, 2, True),
    (4, 6144, 2048, 128, 1, False),
    (8, 2048, 3072, 128, 0, True),
    (8, 2048, 6144, 128, 2, True),
    (8, 6144, 2048, 128, 1, False),
]


@pytest.mark.parametrize("M,K,N,G,mode,norm", QUANT_GEMV_CASES)
def test_quant_gemv_bit_exact(M, K, N, G, mode, norm):
    """quant -> matmul pairs of the decode layer in one call: y and the
    quantised activations are bit-identical to wq_quant_act + wq_gemv, and
    match the oracle (bit-exact; mode 2 within rel 1e-5, device expf)."""
    note(f"quant_gemv M={M} K={K} N={N} G={G} mode={mode} norm={norm}")
    rng = np.random.default_rng(M * 100 + K + N)
    rows = 2 * N if mode == 2 else N
    wq, ws = ref.make_weight(rng, rows, K, G)
    x = ref.make_activations(rng, M, K)
    nw = rng.normal(1.0, 0.2, size=K).astype(np.float32) if norm else None
    y0 = rng.normal(size=(M, N)).astype(np.float32)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    dnw = None if nw is None else dev(nw)
    y = dev(y0) if mode == 1 else None
    y, a = ops.quant_gemv(w, dev(x), norm=dnw, eps=1e-6, mode=mode, y=y)
    a2 = ops.quant(dev(x), norm=dnw, eps=1e-6, G=G)
    y2 = ops.gemv(w, a2, mode=mode, y=dev(y0) if mode == 1 else None)
    assert np.array_equal(host(a.xq), host(a2.xq))
    assert np.array_equal(host(a.dx).view(np.uint32), host(a2.dx).view(np.uint32))
    assert np.array_equal(host(a.xs), host(a2.xs))
    assert np.array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))
    xq, dx, xs = orc.quant_act(x, None, G, norm_w=nw, eps=1e-6)
    assert np.array_equal(host(a.xq), xq)
    want = orc.linear(wq, ws, K, G, xq, dx, xs, mode=mode, y=y0 if mode == 1 else None)
    if mode == 2:
        assert rel_err(host(y), want) < 1e-5
    else:
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))


# ------------------------------------------------ embedding, row gather ----

@pytest.mark.parametrize("G,M", [(32, 1), (128, 2), (32, 7), (128, 33)])
def test_embed_bit_exact(G, M):
    """int4 embedding lookup (embed.wgsl) against the oracle, bit for bit;
    ids past the vocabulary give zero rows."""
    note(f"embed G={G} M={M}")
    V, K = 4096, 2048
    rng = np.random.default_rng(G + M)
    wq, ws = ref.make_weight(rng, V, K, G)
    tok = rng.integers(0, V, M).astype(np.uint32)
    tok[-1] = V + 5 if M > 1 else tok[-1]
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    x = host(ops.embed(w, dev(tok.view(np.int32))))
    want = orc.embed(wq, ws, K, G, tok)
    assert np.array_equal(x.view(np.uint32), want.view(np.uint32))


def test_embed_full_vocabulary_edges():
    """The lookup at the real vocabulary (151,936 rows): the first and last
    rows, and ids V and 0xFFFFFFFF (zero rows), against the oracle."""
    V, K, G = 151936, 2048, 128
    note(f"embed V={V}")
    rng = np.random.default_rng(5)
    wq = rng.integers(0, 2**32, size=(V, K // 8), dtype=np.uint32)
    lo = rng.integers(0x1800, 0x2400, size=(V, K // G), dtype=np.uint32)
    hi = rng.integers(0x9800, 0xA400, size=(V, K // G), dtype=np.uint32)
    ws = lo | (hi << 16)
    tok = np.array([0, 1, V - 1, V - 2, V, 0xFFFFFFFF, 12345, V - 1], np.uint32)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    x = host(ops.embed(w, dev(tok.view(np.int32))))
    want = orc.embed(wq, ws, K, G, tok)
    assert np.array_equal(x.view(np.uint32), want.view(np.uint32))
    assert not np.any(x[4]) and not np.any(x[5])


def test_gather_rows_and_draft_head():
    """The reduced draft lm_head (graph.rs:511-522): gather the rows of the
    ascending draft ids, then the fused lm_head + argmax over them maps the
    winner back through ids -- the same token as the argmax of the full
    head's logits restricted to those rows."""
    note("gather rows + draft head")
    V, K, G, R = 20000, 2048, 128, 3000
    rng = np.random.default_rng(11)
    wq, ws = ref.make_weight(rng, V, K, G)
    ids = np.sort(rng.choice(V, R, replace=False)).astype(np.uint32)
    w = ops.Q4Tensor.from_numpy(wq, ws, K, G)
    d = ops.gather_rows(w, dev(ids.view(np.int32)))
    assert np.array_equal(host(d.q).view(np.uint32), wq[ids])
    assert np.array_equal(host(d.s).view(np.uint32), ws[ids])
    bad = ops.gather_rows(w, dev(np.array([3, V], np.uint32).view(np.int32)))
    assert np.array_equal(host(bad.q).view(np.uint32)[0], wq[3]) and not np.any(host(bad.q)[1])
    x = ref.make_activations(rng, 2, K)
    xq, dx, xs = orc.quant_act(x, None, G)
    a = dev_acts(xq, dx, xs, K, G)
    tok = host(ops.lm_head_argmax(d, a, ids=dev(ids.view(np.int32))))
    logits = orc.linear(wq[ids], ws[ids], K, G, xq, dx, xs)
    assert np.array_equal(tok.view(np.uint32), orc.argmax(logits, ids))


# ------------------------------------------------- decode-layer capture -----

def test_decode_layer_graph_replay():
    """One layer's linear sequence (graph.rs:257-328) recorded into a HIP graph
    and replayed (lib.rs:222-228): every replay, with eager work between them,
    reproduces the eager run bit for bit; the fused sequence equals the
    unfused one (separate quantiser launches) bit for bit; the first
    projection matches the oracle bit for bit."""
    from webyiq_amd.layer import DecodeLayer
    note("decode layer graph replay")
    M, H, Q, KV, F, G = 2, 1024, 1024, 256, 2048, 128
    rng = np.random.default_rng(21)
    shapes = {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H), "down": (H, F)}
    host_w = {n: ref.make_weight(rng, r, c, G) for n, (r, c) in shapes.items()}
    w = ops.Weights({n: ops.Q4Tensor.from_numpy(q, s, shapes[n][1], G) for n, (q, s) in host_w.items()})
    w["attn_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    w["mlp_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    x0 = dev(ref.make_activations(rng, M, H))

    plain = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, fused=False)
    plain.x.copy_(x0)
    plain.run()
    layer = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G)
    layer.x.copy_(x0)
    layer.run()
    want = host(layer.x).copy()
    assert np.array_equal(want.view(np.uint32), host(plain.x).view(np.uint32))
    # first projection against the oracle, bit for bit
    xq, dx, xs = orc.quant_act(host(x0), None, G, norm_w=host(w["attn_norm"]), eps=1e-6)
    qkv_want = orc.linear(*host_w["qkv"], H, G, xq, dx, xs)
    assert np.array_equal(host(layer.qkv).view(np.uint32), qkv_want.view(np.uint32))
    assert np.all(np.isfinite(want))

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.x.copy_(x0)
        layer.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        layer.x.copy_(x0)
        layer.run()
    for i in range(3):
        g.replay()
        got = host(layer.x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i}"
        ops.quant(dev(rng.normal(size=(3, 256)).astype(np.float32)))   # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_decode_layer_bench_shape(M):
    """The decode layer the bench times (hidden 2048, q 2048, kv 512, ffn
    6144, group 128, the chunk merge in place of attention) at its token
    counts: the fused sequence equals the unfused one (separate quantiser
    launches) bit for bit, and its first projection (norm+quant+qkv) and the
    o projection's merged input match the oracle."""
    from webyiq_amd.layer import DecodeLayer
    note(f"decode layer bench shape M={M}")
    H, Q, KV, F, G = 2048, 2048, 512, 6144, 128
    rng = np.random.default_rng(40 + M)
    shapes = {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H), "down": (H, F)}
    host_w = {n: ref.make_weight(rng, r, c, G) for n, (r, c) in shapes.items()}
    w = ops.Weights({n: ops.Q4Tensor.from_numpy(q, s, shapes[n][1], G) for n, (q, s) in host_w.items()})
    w["attn_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    w["mlp_norm"] = dev(rng.normal(1, 0.1, H).astype(np.float32))
    x0 = dev(ref.make_activations(rng, M, H))
    torch.manual_seed(M)
    layer = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, attention="combine")
    plain = DecodeLayer(w, M, hidden=H, q_dim=Q, kv_dim=KV, ffn=F, G=G, fused=False, attention="combine")
    plain.part.copy_(layer.part)
    for lay in (layer, plain):
        lay.x.copy_(x0)
        lay.run()
    got = host(layer.x)
    assert np.array_equal(got.view(np.uint32), host(plain.x).view(np.uint32))
    assert np.all(np.isfinite(got))
    xq, dx, xs = orc.quant_act(host(x0), None, G, norm_w=host(w["attn_norm"]), eps=1e-6)
    qkv_want = orc.linear(*host_w["qkv"], H, G, xq, dx, xs)
    assert np.array_equal(host(layer.qkv).view(np.uint32), qkv_want.view(np.uint32))
    cq, cdx, cxs = orc.attn_combine(host(layer.part), layer.pos)
    got_q = host(layer.a_att.xq).astype(np.int32)
    assert np.abs(got_q - cq.astype(np.int32)).max() <= 1
    assert rel_err(host(layer.a_att.dx), cdx) < 1e-5
