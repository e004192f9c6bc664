"""Known-answer vectors for the int4 x int8 path (writes known_answers.json).

The reference ships no golden vectors for this path, so these are derived by
hand from its definitions, in exact rational arithmetic, without this
repository's oracle or kernels:

  pack    convert.py:8-12,68-75: byte b of word i = q[8i+b] | q[8i+4+b] << 4,
          little-endian words (the comment's known answer: codes 0..7 ->
          0x73625140)
  quant   quant.wgsl:41-61: dx = amax / 127, xq = round-half-even(v / dx),
          a zero group gives dx = 0 and zero codes; xs = sum of codes per
          accumulation group min(G, GA)
  linear  gemv_q4q8.wgsl:6: y[t,n] = sum_g dx[t,g] (s[n,g] A[t,n,g] +
          m[n,g] X[t,g]); mode 1 adds to y
  argmax  argmax.wgsl:14-43: strict > from -3e38, first index wins ties,
          NaN never wins, ids map the index
  embed   embed.wgsl:13-27: x = f32(q) * s + m

The values are chosen so that every quotient is exact (dx a power of two)
and every partial sum of the fp32 folds is exactly representable, which this
script asserts, so the expected outputs hold bit for bit in any evaluation
order.  Run from anywhere: python tests/golden/make_known_answers.py
"""
import json
import os
import struct
from fractions import Fraction as Fr

HERE = os.path.dirname(os.path.abspath(__file__))
K = 128


def is_f32(v):
    v = Fr(v)
    return Fr(struct.unpack("<f", struct.pack("<f", float(v)))[0]) == v


def f32(v):
    assert is_f32(v), v
    return float(v)


def f16_bits(v):
    v = Fr(v)
    b = struct.unpack("<H", struct.pack("<e", float(v)))[0]
    assert Fr(struct.unpack("<e", struct.pack("<H", b))[0]) == v, v
    return b


def rne(q):
    """round half to even of a Fraction"""
    f = q.numerator // q.denominator
    r = q - f
    if r > Fr(1, 2) or (r == Fr(1, 2) and f % 2 == 1):
        f += 1
    return f


def pack_row(codes):
    words = []
    for i in range(len(codes) // 8):
        w = 0
        for b in range(4):
            w |= (codes[8 * i + b] | (codes[8 * i + 4 + b] << 4)) << (8 * b)
        words.append(w)
    return words


def quant_row(x, GA, G):
    ge = min(G, GA)
    xq, dx = [], []
    for g0 in range(0, K, GA):
        grp = [Fr(v) for v in x[g0:g0 + GA]]
        amax = max(abs(v) for v in grp)
        d = amax / 127
        assert is_f32(d)
        dx.append(d)
        xq += [0 if d == 0 else rne(v / d) for v in grp]
    assert all(-127 <= q <= 127 for q in xq)
    xs = [sum(xq[g0:g0 + ge]) for g0 in range(0, K, ge)]
    return xq, dx, xs


def linear_row(codes, s, m, xq, dx, G, GA, y0=0):
    """exact y and an exactness check of every partial sum of the canonical
    fold: acc = fma(s d, A, acc); acc = fma(m d, X, acc) per group (d = 1 and
    a final y = acc * dx for per-token activations)"""
    ge = min(G, GA)
    acc = Fr(0)
    for e in range(K // ge):
        g = (e * ge) // G
        d = dx[(e * ge) // GA] if GA != K else Fr(1)
        A = sum(codes[i] * xq[i] for i in range(e * ge, (e + 1) * ge))
        X = sum(xq[e * ge:(e + 1) * ge])
        acc += s[g] * d * A
        assert is_f32(acc) and is_f32(s[g] * d)
        acc += m[g] * d * X
        assert is_f32(acc) and is_f32(m[g] * d)
    y = acc * dx[0] if GA == K else acc
    y = Fr(y0) + y
    assert is_f32(y)
    return y


def main():
    out = {"K": K, "about": __doc__.split("\n\n")[0]}

    # ---- pack
    code_rows = [[i % 16 for i in range(K)], [15 - i % 16 for i in range(K)], [(7 * i + 3) % 16 for i in range(K)]]
    words = [pack_row(r) for r in code_rows]
    assert words[0][0] == 0x73625140 and words[0][1] == 0xFBEAD9C8
    out["pack"] = {"codes": code_rows, "words": words}

    # ---- quantiser
    row_d1 = [127.0, -63.5, 0.5, 1.5, 2.5, -2.5, -0.5, 3.5, 100.25, -100.75] + [0.0] * (K - 10)
    row_zero = [0.0] * K
    row_d2 = [254.0, 3.0, 5.0, 7.0, -1.0, 1.0, 253.0, -253.0, 0.75, -9.0] + [0.0] * (K - 10)
    per32 = (row_d1[:32] + [254.0, 3.0, 5.0, 7.0, -1.0, 1.0] + [0.0] * 26 + [0.0] * 32
             + [63.5, 0.25, 0.75, 1.25, -31.75] + [0.0] * 27)
    quant = []
    for name, rows, GA, G in (("per_token_G128", [row_d1, row_zero, row_d2], K, 128),
                              ("per_token_G32", [row_d1, row_d2], K, 32),
                              ("per32_G32", [per32], 32, 32),
                              ("per32_G128", [per32], 32, 128)):
        res = [quant_row(r, GA, G) for r in rows]
        quant.append({"name": name, "GA": GA, "G": G, "x": [[f32(v) for v in r] for r in rows],
                      "xq": [r[0] for r in res], "dx": [[f32(d) for d in r[1]] for r in res],
                      "xs": [r[2] for r in res]})
    assert quant[0]["xq"][0][:10] == [127, -64, 0, 2, 2, -2, 0, 4, 100, -101]
    assert quant[0]["xq"][2][:10] == [127, 2, 2, 4, 0, 0, 126, -126, 0, -4]
    out["quant"] = quant

    # ---- linear (modes 0 and 1), 4 rows x 4 tokens
    w_codes = [[1] * K, [i % 16 for i in range(K)], [15 - i % 16 for i in range(K)], [(5 * i + 1) % 16 for i in range(K)]]
    base_s = [Fr(1), Fr(1, 2), Fr(1, 4), Fr(2)]
    base_m = [Fr(0), Fr(-2), Fr(1), Fr(-16)]
    tok_xq = [[1 if i == 5 else 0 for i in range(K)],
              [(i % 7) - 3 for i in range(K)],
              [127] * K,
              [-127 if i == 127 else (1 if i == 64 else 0) for i in range(K)]]
    tok_dx = [Fr(1), Fr(1, 2), Fr(1, 4), Fr(2)]
    y0 = [[1.0, -2.0, 0.5, 3.0], [0.0, 0.25, -1.5, 8.0], [-4.0, 2.0, 0.0, 1.0], [16.0, -0.5, 0.125, -3.0]]
    linear = []
    for G, GA in ((128, K), (32, K), (32, 32), (128, 32)):
        ng = K // G
        gs = [[base_s[n] * [1, Fr(1, 2), 2, 1][g % 4] for g in range(ng)] for n in range(4)]
        gm = [[base_m[n] + [0, 1, -1, Fr(1, 2)][g % 4] for g in range(ng)] for n in range(4)]
        if GA == K:
            dxs = [[d] for d in tok_dx]
        else:  # per-32 scales of each token: powers of two
            dxs = [[tok_dx[t] * [1, Fr(1, 2), 2, Fr(1, 4)][e] for e in range(K // 32)] for t in range(4)]
        ge = min(G, GA)
        xs = [[sum(xq[e * ge:(e + 1) * ge]) for e in range(K // ge)] for xq in tok_xq]
        case = {"G": G, "GA": GA, "codes": w_codes,
                "words": [pack_row(c) for c in w_codes],
                "scale_words": [[f16_bits(gs[n][g]) | (f16_bits(gm[n][g]) << 16) for g in range(ng)]
                                for n in range(4)],
                "xq": tok_xq, "dx": [[f32(d) for d in r] for r in dxs], "xs": xs, "y0": y0}
        for mode in (0, 1):
            case[f"y_mode{mode}"] = [[f32(linear_row(w_codes[n], gs[n], gm[n], tok_xq[t], dxs[t], G, GA,
                                                     y0[t][n] if mode == 1 else 0))
                                      for n in range(4)] for t in range(4)]
        # greedy token of each token's mode-0 logits (first index on ties)
        case["argmax_mode0"] = [max(range(4), key=lambda n, r=r: (r[n], -n)) for r in case["y_mode0"]]
        linear.append(case)
    out["linear"] = linear

    # ---- argmax
    V = 64
    rows = [[0.0] * V for _ in range(6)]
    rows[0][3] = rows[0][7] = 5.0                        # tie: first index
    rows[1][0] = float("nan"); rows[1][40] = 2.5         # NaN never wins
    rows[2] = [float("-inf")] * V                        # nothing above -3e38: index 0
    rows[3] = [-1e30] * V; rows[3][63] = 1e30            # last element
    rows[4] = [-3e38] * V                                # -3e38 itself never wins: index 0
    rows[5] = [-3e38] * V; rows[5][17] = -2.9e38         # just above the start value
    want = [3, 40, 0, 63, 0, 17]
    ids = [1000 + 2 * i for i in range(V)]
    out["argmax"] = {"logits": [[("nan" if v != v else v) for v in r] for r in rows], "tokens": want,
                     "ids": ids, "tokens_mapped": [ids[i] for i in want]}

    # ---- embed (dequantisation of the packed rows)
    es = [(Fr(1), Fr(0)), (Fr(1, 2), Fr(-4)), (Fr(-1, 4), Fr(3, 2))]
    emb = []
    for r, (s, m) in enumerate(es):
        emb.append([f32(Fr(c) * s + m) for c in code_rows[r]])
    out["embed"] = {"G": 128, "words": words, "scale_words": [[f16_bits(s) | (f16_bits(m) << 16)] for s, m in es],
                    "x": emb}

    path = os.path.join(HERE, "known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(path)


if __name__ == "__main__":
    main()
