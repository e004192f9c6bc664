"""Pins of the oracle's other producers of int8 activations -- CPU only.

or_mtp_in (mtp_in.wgsl:45-89) and or_attn_combine (attn_combine.wgsl:36-82)
are pinned by what does not share their formula: exact small-integer
inputs through numpy float32 (every sum and product exact, so any order
gives the oracle's bits), the already-pinned per-token quantiser, float64
RMSNorm, and textbook softmax attention computed directly from q, K, V.
"""
import numpy as np
import pytest

from oracle import oracle as orc


def np_quant32(v):
    """Per-32 quantiser in numpy float32 (IEEE quotient, RNE): dx, xq, xs."""
    g = v.astype(np.float32).reshape(-1, 32)
    d = (np.abs(g).max(1) / np.float32(127)).astype(np.float32)
    safe = np.where(d > 0, d, np.float32(1))
    q = np.where(d[:, None] > 0, np.rint(g / safe[:, None]), 0).astype(np.int8)
    return q.reshape(-1), d, q.astype(np.int32).sum(1)


# ------------------------------------------------------------ MTP input ----

def test_mtp_in_exact_small_integers(rng):
    """emb, x = +-1 and power-of-two norm weights, eps = 0: both rms factors
    are exact (1 and 1/2), so numpy float32 reproduces the oracle bit for bit.
    Catches swapped halves, a missing second norm, the wrong weight per norm
    and the wrong row of the [M, 2K] output."""
    M, K = 3, 2048
    emb = rng.choice([-1.0, 1.0], size=(M, K)).astype(np.float32)
    x = rng.choice([-1.0, 1.0], size=(M, K)).astype(np.float32)
    ne = rng.choice([-2.0, -0.5, 0.25, 1.0, 4.0], size=K).astype(np.float32)
    nf = rng.choice([-2.0, 2.0], size=K).astype(np.float32)      # x * nf = +-2: rms 2
    nh = rng.choice([-1.0, 0.5, 0.125, 8.0], size=K).astype(np.float32)
    xq, dx, xs = orc.mtp_in(emb, x, nf, ne, nh, eps=0.0)
    for m in range(M):
        h0 = emb[m] * (np.float32(1.0) * ne)
        v1 = x[m] * (np.float32(1.0) * nf)
        h1 = v1 * (np.float32(0.5) * nh)
        for half, v in ((0, h0), (1, h1)):
            q, d, s = np_quant32(v)
            cols = slice(half * K, (half + 1) * K)
            gcols = slice(half * K // 32, (half + 1) * K // 32)
            assert np.array_equal(xq[m, cols], q)
            assert np.array_equal(dx[m, gcols], d)
            assert np.array_equal(xs[m, gcols], s)


def test_mtp_in_unit_weights_is_the_quantiser_with_norm(rng):
    """With ne = 1, half 0 is x * (r * 1) = (x * r) * 1: the per-32 quantiser
    with an RMSNorm prologue (pinned in test_oracle.py), bit for bit."""
    M, K = 2, 4096
    emb = rng.normal(0, 2, size=(M, K)).astype(np.float32)
    x = rng.normal(0, 2, size=(M, K)).astype(np.float32)
    one = np.ones(K, np.float32)
    nf, nh = (rng.normal(1, 0.2, size=K).astype(np.float32) for _ in range(2))
    xq, dx, xs = orc.mtp_in(emb, x, nf, one, nh, eps=1e-6)
    q0, d0, s0 = orc.quant_act(emb, 32, 32, norm_w=one, eps=1e-6)
    assert np.array_equal(xq[:, :K], q0)
    assert np.array_equal(dx[:, :K // 32], d0)
    assert np.array_equal(xs[:, :K // 32], s0)


@pytest.mark.parametrize("K", [2048, 6144])
def test_mtp_in_float64_double_norm(rng, K):
    """Random inputs against float64 RMSNorm (one pass, and the norm of a norm)."""
    M = 2
    emb = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    x = rng.normal(0, 5, size=(M, K)).astype(np.float32)
    nf, ne, nh = (rng.normal(1, 0.3, size=K).astype(np.float32) for _ in range(3))
    xq, dx, _ = orc.mtp_in(emb, x, nf, ne, nh, eps=1e-6)

    def norm(v, w):
        v = v.astype(np.float64)
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + 1e-6) * w

    ref = np.concatenate([norm(emb, ne), norm(norm(x, nf), nh)], axis=1)
    g = ref.reshape(M, -1, 32)
    d = np.abs(g).max(-1) / 127
    assert np.allclose(dx, d, rtol=1e-5)
    deq = xq.astype(np.float64).reshape(M, -1, 32) * dx[..., None]
    assert np.all(np.abs(deq - g) <= d[..., None] * 0.5001)


# ------------------------------------------------ attention chunk merge ----

def partials(q, k, v, n_pos, nch):
    """attn.wgsl:60-113 in float64 for one (token, head): per chunk of 32
    positions (positions >= n_pos masked), the chunk max score m_c, the
    weight sum l_c and the D weighted value sums; unused chunks are NaN
    (never read)."""
    D = q.shape[0]
    s = (k[:n_pos] @ q) / np.sqrt(D)
    out = np.full((nch, D + 2), np.nan)
    for c in range((n_pos + 31) // 32):
        sc = s[32 * c:32 * c + 32]
        m = sc.max()
        e = np.exp(sc - m)
        out[c, :D] = e @ v[32 * c:32 * c + len(sc)]
        out[c, D] = m
        out[c, D + 1] = e.sum()
    return out


def make_attention(rng, M, H, D, nch, pos, scale=1.0):
    T = pos + M
    q = rng.normal(0, scale, size=(M, H, D))
    k = rng.normal(0, 1, size=(H, T, D))
    v = rng.normal(0, 1, size=(H, T, D))
    part = np.stack([np.stack([partials(q[m, h], k[h], v[h], pos + m + 1, nch) for h in range(H)])
                     for m in range(M)]).astype(np.float32)
    direct = np.zeros((M, H, D))
    for m in range(M):
        for h in range(H):
            s = k[h, :pos + m + 1] @ q[m, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            direct[m, h] = p @ v[h, :pos + m + 1] / p.sum()
    return part, direct


def check_close_to(xq, dx, ref):
    """Dequantised output within half a code step (plus float slack) of ref."""
    M = ref.shape[0]
    g = ref.reshape(M, -1, 32)
    d = np.abs(g).max(-1) / 127
    assert np.allclose(dx, d, rtol=2e-5)
    deq = xq.astype(np.float64).reshape(M, -1, 32) * dx[..., None]
    assert np.all(np.abs(deq - g) <= d[..., None] * 0.502)


@pytest.mark.parametrize("D,pos", [(64, 5), (128, 100), (128, 127), (256, 300)])
def test_attn_combine_is_softmax_attention(rng, D, pos):
    """Merging the chunk partials equals softmax(q K^T / sqrt(D)) V computed
    directly.  Catches a wrong chunk count per token (token m covers
    positions 0 ..= pos + m: NaN chunks past it would poison the output),
    a dropped weight, or l taken from the wrong slot."""
    M, H, nch = 2, 3, 16
    part, direct = make_attention(rng, M, H, D, nch, pos)
    xq, dx, xs = orc.attn_combine(part, pos)
    check_close_to(xq, dx, direct.reshape(M, H * D))
    assert np.array_equal(xs, xq.astype(np.int32).reshape(M, -1, 32).sum(-1))


def test_attn_combine_gate(rng):
    """Qwen3.5 gate: o / (1 + exp(-g)), g at h*2D + D + i of the token's row."""
    M, H, D, nch, pos = 2, 2, 128, 8, 40
    part, direct = make_attention(rng, M, H, D, nch, pos)
    stride = 2 * (H + 1) * D   # rows of 2 (H + KVH) D with KVH = 1
    gate = rng.normal(0, 2, size=(M, stride)).astype(np.float32)
    xq, dx, _ = orc.attn_combine(part, pos, gate, stride)
    g = np.stack([gate[:, h * 2 * D + D:h * 2 * D + 2 * D] for h in range(H)], axis=1).astype(np.float64)
    check_close_to(xq, dx, (direct / (1 + np.exp(-g))).reshape(M, H * D))


def test_attn_combine_zero_values():
    """All-zero value sums: o = 0, so dx = 0 and every code and sum is 0."""
    M, H, D, nch = 1, 2, 64, 4
    part = np.zeros((M, H, nch, D + 2), np.float32)
    part[..., D + 1] = 1.0
    xq, dx, xs = orc.attn_combine(part, 50)
    assert not np.any(xq) and not np.any(dx) and not np.any(xs)
