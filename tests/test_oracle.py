"""Pins of the CPU oracle (oracle/q4q8_oracle.c) -- CPU only.

The reference ships no golden vectors or unit tests for this path, so every
oracle function is pinned by something independent of its own formula:
numpy/torch library routines, closed forms, known answers from the
reference's own comments, invariants, and brute force.  Each test names the
mistake it is there to catch.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle import reference as ref
from conftest import rel_err


# ------------------------------------------------------------- f16 words ----

def test_f16_matches_numpy_random_and_edges(rng):
    """Scale/min words are f16 (convert.py:57); numpy's astype is the pin."""
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-30, 18, 200000))).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2**-24, 2**-25,
                      1.5 * 2**-25, 2**-14, 2**-14 * (1 - 2**-11), np.inf, -np.inf,
                      1.0 + 2**-11, 1.0 + 3 * 2**-11, 1.0 + 2**-11 + 2**-20], np.float32)
    for v in (x, edges):
        assert np.array_equal(orc.f32_to_f16_bits(v), v.astype(np.float16).view(np.uint16))
    nan = orc.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert (nan[0] & 0x7C00) == 0x7C00 and (nan[0] & 0x3FF) != 0


def test_f16_decode_all_finite_codes():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]
    ours = orc.f16_bits_to_f32(h)
    assert np.array_equal(ours.view(np.uint32), h.view(np.float16).astype(np.float32).view(np.uint32))


# --------------------------------------------------------------- packing ----

def test_pack_known_answer():
    """convert.py:8-11: codes 0..7 -> bytes 0x40 0x51 0x62 0x73 -> 0x73625140."""
    q = np.arange(8, dtype=np.uint8)[None]
    wq, ws = orc.q4_pack(q, np.array([[0x3C00]], np.uint16), np.array([[0xBC00]], np.uint16), 8)
    assert wq[0, 0] == 0x73625140
    assert ws[0, 0] == (0x3C00 | (0xBC00 << 16))  # low = scale, high = min (convert.py:74)


def test_unpack_is_embed_wgsl_order(rng):
    """embed.wgsl:22-24 reads code 8i+b from bits 8b and code 8i+4+b from 8b+4."""
    q = rng.integers(0, 16, size=(5, 256)).astype(np.uint8)
    wq, _ = orc.q4_pack(q, np.zeros((5, 2), np.uint16), np.zeros((5, 2), np.uint16), 128)
    # independent restatement of the shader loop
    out = np.zeros_like(q)
    for i in range(256 // 8):
        w = wq[:, i]
        for b in range(4):
            out[:, 8 * i + b] = (w >> (8 * b)) & 15
            out[:, 8 * i + 4 + b] = (w >> (8 * b + 4)) & 15
    assert np.array_equal(out, q)
    assert np.array_equal(orc.q4_unpack(wq, 256), q)
    # dot-product lanes: u & 0x0F0F0F0F holds codes 8i..8i+3 (convert.py:9-11)
    lo = (wq[:, 0] & 0x0F0F0F0F).view(np.uint8).reshape(5, 4)
    assert np.array_equal(lo, q[:, 0:4])


# ----------------------------------------------------------------- RTN ------

@pytest.mark.parametrize("G", [32, 128])
def test_rtn_closed_form_and_invariants(rng, G):
    w = rng.normal(0, 0.02, size=(64, 512)).astype(np.float32)
    wq, ws, deq = orc.q4_quantize(w, G, want_deq=True)
    q = orc.q4_unpack(wq, 512).astype(np.int64).reshape(64, -1, G)
    g = w.reshape(64, -1, G)
    s = (ws & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    m = (ws >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    # grid: s = f16((max-min)/15), m = f16(min)  (convert.py:55-57)
    assert np.array_equal(s, ((g.max(2) - g.min(2)) / np.float32(15)).astype(np.float16).astype(np.float32))
    assert np.array_equal(m, g.min(2).astype(np.float16).astype(np.float32))
    # the stored dequantisation is q*s + m (convert.py:65)
    assert np.array_equal(deq.reshape(64, -1, G), q * s[..., None] + m[..., None])
    # nearest grid point: error at most half a step (+ f16 rounding of m/s)
    slack = np.abs(s[..., None]) * 0.5 + np.abs(g.min(2, keepdims=True)) * 2**-10 + 16 * np.abs(s[..., None]) * 2**-10
    inside = (g >= m[..., None]) & (g <= m[..., None] + 15 * s[..., None])
    assert np.all(np.abs(deq.reshape(64, -1, G) - g)[inside] <= slack.repeat(G, 2)[inside] + 1e-9)
    # group extremes land on the grid ends; codes monotone in w within a group
    assert np.all(np.take_along_axis(q, g.argmax(2)[..., None], 2) >= 14)
    assert np.all(np.take_along_axis(q, g.argmin(2)[..., None], 2) <= 1)
    order = np.argsort(g, axis=2, kind="stable")
    assert np.all(np.diff(np.take_along_axis(q, order, 2), axis=2) >= 0)


def test_rtn_constant_group_uses_unit_divisor():
    """convert.py:64: s == 0 -> divide by 1, so every code is rint(w - m) = 0."""
    w = np.full((2, 128), 0.25, np.float32)
    wq, ws, deq = orc.q4_quantize(w, 128, want_deq=True)
    assert np.all(wq == 0) and np.all(deq == 0.25)
    assert np.all((ws & 0xFFFF) == 0) and np.all((ws >> 16) == 0x3400)  # f16(0.25)


# ------------------------------------------------------- activation quant ---

@pytest.mark.parametrize("GA", [None, 32])
def test_quant_act_matches_torch_round(rng, GA):
    """reference.py:45-47 with torch as the pin: dx = amax/127, round(x / dx)."""
    x = ref.make_activations(rng, 5, 1024)
    xq, dx, xs = orc.quant_act(x, GA, 128)
    t = torch.from_numpy(x)
    ga = 1024 if GA is None else GA
    g = t.reshape(5, -1, ga)
    d = g.abs().amax(-1, keepdim=True) / 127.0
    q = torch.where(d > 0, torch.round(g / torch.where(d > 0, d, 1.0)), 0.0).reshape(5, 1024)
    assert np.array_equal(xq, q.numpy().astype(np.int8))
    assert np.array_equal(dx, d.reshape(5, -1).numpy())
    ge = min(128, ga)
    assert np.array_equal(xs, xq.astype(np.int64).reshape(5, -1, ge).sum(2).astype(np.int32))
    fq = ref.fq_input(x, GA).numpy()  # the torch restatement agrees too
    assert np.array_equal(fq, (xq.astype(np.float32).reshape(5, -1, ga) * dx[..., None]).reshape(5, 1024))


def test_quant_act_ties_to_even_and_zero_row():
    """Half-way codes round to even (torch.round / RNE); an all-zero token gets
    dx = 0 and zero codes (quant.wgsl:53, reference.py:47)."""
    x = np.zeros((2, 128), np.float32)
    x[0, :6] = [127.0, 2.5, 3.5, -2.5, 0.5, -126.5]
    xq, dx, xs = orc.quant_act(x, None, 128)
    assert dx[0, 0] == 1.0
    assert list(xq[0, :6]) == [127, 2, 4, -2, 0, -126]
    assert dx[1, 0] == 0.0 and np.all(xq[1] == 0) and xs[1, 0] == 0
    assert xs[0, 0] == 127 + 2 + 4 - 2 + 0 - 126


def test_quant_act_amax_maps_to_127(rng):
    x = ref.make_activations(rng, 4, 2048)
    xq, dx, _ = orc.quant_act(x, None, 128)
    assert np.all(np.abs(xq.astype(np.int32)).max(1) == 127)
    assert np.all(np.abs(xq[np.arange(4), np.abs(x).argmax(1)]) == 127)


@pytest.mark.parametrize("K", [128, 2048, 2176, 6144])
def test_quant_act_rmsnorm_prologue(rng, K):
    """quant.wgsl:24-39: v = x * nw / sqrt(mean(x^2) + eps); checked in float64
    (partial and several 2048-element passes: every element counted once)."""
    x = rng.normal(0, 3, size=(3, K)).astype(np.float32)
    nw = rng.normal(1, 0.1, size=K).astype(np.float32)
    xq, dx, _ = orc.quant_act(x, None, 128, norm_w=nw, eps=1e-6)
    v = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * nw
    d = np.abs(v).max(1) / 127
    assert np.allclose(dx[:, 0], d, rtol=1e-6)
    # codes agree except where v/dx sits within float rounding of a .5 boundary
    frac = np.abs(np.abs(v / d[:, None]) % 1 - 0.5)
    exact = frac > 1e-4
    assert np.array_equal(xq[exact], np.rint(v / d[:, None])[exact].astype(np.int8))


# ------------------------------------------------- integer group sums -------

@pytest.mark.parametrize("Ge", [32, 128])
def test_group_acc_brute_force(rng, Ge):
    """A[t,n,e] = sum q*xq over the group, int64 brute force from raw codes."""
    q = rng.integers(0, 16, size=(48, 512)).astype(np.uint8)
    wq, _ = orc.q4_pack(q, np.zeros((48, 512 // Ge), np.uint16), np.zeros((48, 512 // Ge), np.uint16), Ge)
    xq = rng.integers(-127, 128, size=(3, 512)).astype(np.int8)
    acc = orc.group_acc(wq, 512, Ge, xq)
    bf = np.einsum("tek,nek->tne", xq.astype(np.int64).reshape(3, -1, Ge), q.astype(np.int64).reshape(48, -1, Ge))
    assert np.array_equal(acc, bf)
    # extreme magnitudes stay exact: 128 * 15 * 127 = 243840
    q2 = np.full((1, 128), 15, np.uint8)
    wq2, _ = orc.q4_pack(q2, np.zeros((1, 1), np.uint16), np.zeros((1, 1), np.uint16), 128)
    x2 = np.full((1, 128), -127, np.int8)
    assert orc.group_acc(wq2, 128, 128, x2)[0, 0, 0] == -243840


# ------------------------------------------------------------- linear -------

def fake_quant_f64(wq, ws, K, G, xq, dx, GA):
    """The fake-quant product of tools/reference.py:35-48 in float64:
    sum_k (q s + m)(xq dx) -- an independent formulation of the same value."""
    wd = ref.dequant_weight(wq, ws, K, G).astype(np.float64)
    ga = K if GA is None else GA
    xd = (xq.astype(np.float64).reshape(xq.shape[0], -1, ga) * dx.astype(np.float64)[..., None]).reshape(xq.shape)
    return xd @ wd.T


@pytest.mark.parametrize("G,GA", [(128, None), (32, None), (128, 32), (32, 32)])
def test_linear_matches_fake_quant_product(rng, G, GA):
    K, N, M = 1024, 96, 4
    wq, ws = ref.make_weight(rng, N, K, G)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, GA, G)
    y = orc.linear(wq, ws, K, G, xq, dx, xs, GA=GA)
    exact = fake_quant_f64(wq, ws, K, G, xq, dx, GA)
    assert rel_err(y, exact) < 2e-6
    # the torch fake-quant path (fp32) is within the stated 1e-3
    y_t = ref.FakeQuantLinear(wq, ws, K, G, GA=GA)(x).numpy()
    assert rel_err(y, y_t) < 1e-5


def test_linear_catches_dropped_min_term(rng):
    """A dropped m*X term or a sign error would be far outside the tolerance."""
    K, N = 512, 32
    wq, ws = ref.make_weight(rng, N, K, 128)
    x = ref.make_activations(rng, 1, K)
    xq, dx, xs = orc.quant_act(x, None, 128)
    y = orc.linear(wq, ws, K, 128, xq, dx, xs)
    ws_no_min = ws & 0xFFFF
    y_bad = orc.linear(wq, ws_no_min, K, 128, xq, dx, xs)
    assert rel_err(y_bad, y) > 1e-2


def test_linear_modes(rng):
    K, N, M = 512, 64, 2
    wq, ws = ref.make_weight(rng, 2 * N, K, 128)
    x = ref.make_activations(rng, M, K)
    xq, dx, xs = orc.quant_act(x, None, 128)
    full = fake_quant_f64(wq, ws, K, 128, xq, dx, None)
    y0 = orc.linear(wq[:N], ws[:N], K, 128, xq, dx, xs, mode=0)
    base = rng.normal(size=(M, N)).astype(np.float32)
    y1 = orc.linear(wq[:N], ws[:N], K, 128, xq, dx, xs, mode=1, y=base)
    assert np.array_equal(y1, base + y0)
    y2 = orc.linear(wq, ws, K, 128, xq, dx, xs, mode=2)
    g, u = full[:, :N], full[:, N:]
    assert rel_err(y2, g / (1 + np.exp(-g)) * u) < 1e-5
    y2t = torch.nn.functional.silu(torch.from_numpy(y0)) * torch.from_numpy(orc.linear(wq[N:], ws[N:], K, 128, xq, dx, xs))
    assert rel_err(y2, y2t.numpy()) < 1e-6


# ------------------------------------------------------------- argmax -------

def test_argmax_first_occurrence_and_ties(rng):
    v = rng.normal(size=(6, 5000)).astype(np.float32)
    assert np.array_equal(orc.argmax(v), np.argmax(v, 1).astype(np.uint32))
    v[2, [17, 900, 4000]] = 99.0      # exact tie: lowest index
    v[3, 10] = 0.0
    v[3, :] = np.minimum(v[3], -1.0)
    v[3, 10], v[3, 5] = 0.0, -0.0     # -0.0 == +0.0: lowest index
    v[4, 7] = np.nan                  # NaN never wins
    v[5, :] = -np.inf                 # nothing above -3e38 -> 0
    out = orc.argmax(v)
    assert out[2] == 17 and out[3] == 5 and out[4] == np.argmax(np.nan_to_num(v[4], nan=-1e9))
    assert out[5] == 0
    ids = np.arange(5000, dtype=np.uint32) * 3 + 1
    assert np.array_equal(orc.argmax(v, ids), ids[out])


# ------------------------------------------------- embedding, row gather ----

def _numpy_dequant_rows(wq, ws, K, G, rows):
    """embed.wgsl:19-27 restated with numpy bit operations (not the oracle's
    unpacker): byte b of word i holds code 8i+b (low nibble) and 8i+4+b."""
    w = wq[rows].astype(np.uint32)                       # [R, K/8]
    lo = np.stack([(w >> (8 * b)) & 15 for b in range(4)], -1)
    hi = np.stack([(w >> (8 * b + 4)) & 15 for b in range(4)], -1)
    q = np.concatenate([lo, hi], -1).reshape(len(rows), K).astype(np.float32)
    s = (ws[rows] & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    m = (ws[rows] >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    s = np.repeat(s, G, axis=1)
    m = np.repeat(m, G, axis=1)
    return (q * s) + m                                   # product rounded, then the sum


@pytest.mark.parametrize("G", [32, 128])
def test_embed_matches_numpy_dequant(rng, G):
    V, K = 300, 512
    wq, ws = ref.make_weight(rng, V, K, G)
    tok = np.array([0, 299, 17, 17, 150], np.uint32)
    x = orc.embed(wq, ws, K, G, tok)
    assert np.array_equal(x.view(np.uint32), _numpy_dequant_rows(wq, ws, K, G, tok).view(np.uint32))
    # an id past the vocabulary gives a zero row
    x2 = orc.embed(wq, ws, K, G, np.array([V, 2**32 - 1], np.uint32))
    assert not np.any(x2)


def test_gather_rows_is_row_indexing(rng):
    V, K, G = 200, 1024, 128
    wq, ws = ref.make_weight(rng, V, K, G)
    ids = np.sort(rng.choice(V, 64, replace=False)).astype(np.uint32)   # ascending (convert.py:328)
    dq, ds = orc.gather_rows(wq, ws, K, G, ids)
    assert np.array_equal(dq, wq[ids]) and np.array_equal(ds, ws[ids])
    dq, ds = orc.gather_rows(wq, ws, K, G, np.array([5, V + 3], np.uint32))
    assert np.array_equal(dq[0], wq[5]) and not np.any(dq[1]) and not np.any(ds[1])
