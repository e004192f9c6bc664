/*
 * CPU oracle for webyIQ's fused int4 x int8 linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels in webyiq_amd/.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product path never calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the webyIQ repository root).  Build: oracle/Makefile (gcc, -ffp-contract=off
 * so that the only fused multiply-adds are the explicit fmaf() calls, which
 * the HIP kernels issue as v_fma_f32 in the same order).
 *
 * Parity pins (tests/test_oracle.py): f16 conversion against numpy's astype,
 * the packing known answer 0x73625140 and the embed.wgsl unpack order, RTN
 * against closed forms, activation quantisation against torch.round(x / dx),
 * group accumulators against int64 brute force, the linear epilogue against
 * the float64 fake-quant product (tools/reference.py:35-48), argmax against
 * numpy's first-occurrence argmax and planted exact ties.
 */
#include "q4q8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 ---- */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Round-to-nearest-even binary32 -> binary16, including subnormals, overflow
 * to infinity and NaN (numpy float32.astype(float16) semantics). */
uint16_t or_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t ex = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (ex == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    int32_t e = (int32_t)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        /* subnormal half (or zero): value = man24 * 2^(ex-150); unit = 2^-24 */
        if (e < -10) return sign;  /* below half of the smallest subnormal -> 0 */
        uint32_t m24 = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);  /* 2^(ex-150) / 2^-24 = 2^(ex-126) */
        uint32_t q = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* may carry into exponent/inf */
    return (uint16_t)(sign | q);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (ex == 0x1Fu) return bits_f32(sign | 0x7F800000u | (man << 13));
    if (ex == 0) {
        /* subnormal: man * 2^-24 is exact in binary32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((ex - 15u + 127u) << 23) | (man << 13));
}

void or_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_f16(in[i]);
}

/* ------------------------------------------------------- int4 weights ---- */

/* tools/convert.py:68-75: byte b of word i = q[8i+b] | q[8i+4+b] << 4;
 * word = low16 f16 scale | high16 f16 min. */
void or_q4_pack(const uint8_t* q, const uint16_t* scale, const uint16_t* mn,
                int64_t N, int64_t K, int G, uint32_t* wq, uint32_t* ws) {
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* qr = q + n * K;
        for (int64_t i = 0; i < K / 8; ++i) {
            uint32_t w = 0;
            for (int b = 0; b < 4; ++b) {
                uint32_t byte = (uint32_t)(qr[8 * i + b] & 15u) | ((uint32_t)(qr[8 * i + 4 + b] & 15u) << 4);
                w |= byte << (8 * b);
            }
            wq[n * (K / 8) + i] = w;
        }
        for (int64_t g = 0; g < K / G; ++g) {
            int64_t j = n * (K / G) + g;
            ws[j] = (uint32_t)scale[j] | ((uint32_t)mn[j] << 16);
        }
    }
}

/* Unpack order of crates/engine/src/shaders/embed.wgsl:22-24. */
void or_q4_unpack(const uint32_t* wq, int64_t N, int64_t K, uint8_t* q) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t i = 0; i < K / 8; ++i) {
            uint32_t w = wq[n * (K / 8) + i];
            for (int b = 0; b < 4; ++b) {
                q[n * K + 8 * i + b] = (uint8_t)((w >> (8 * b)) & 15u);
                q[n * K + 8 * i + 4 + b] = (uint8_t)((w >> (8 * b + 4)) & 15u);
            }
        }
}

/* tools/convert.py:55-65 and 78-106 with search=False:
 *   lo/hi = group min/max; s = f16((hi - lo) / 15), m = f16(lo)   (fp32 math)
 *   q = clip(rint((w - m) / (s == 0 ? 1 : s)), 0, 15); deq = q*s + m */
void or_q4_quantize(const float* w, int64_t N, int64_t K, int G,
                    uint32_t* wq, uint32_t* ws, float* deq) {
    int64_t NG = K / G;
    uint8_t* q = (uint8_t*)malloc((size_t)K);
    uint16_t* sc = (uint16_t*)malloc((size_t)NG * 2);
    uint16_t* mn = (uint16_t*)malloc((size_t)NG * 2);
    for (int64_t n = 0; n < N; ++n) {
        const float* row = w + n * K;
        for (int64_t g = 0; g < NG; ++g) {
            const float* gp = row + g * G;
            float lo = gp[0], hi = gp[0];
            for (int i = 1; i < G; ++i) {
                if (gp[i] < lo) lo = gp[i];
                if (gp[i] > hi) hi = gp[i];
            }
            float range = hi - lo;
            uint16_t hs = or_f32_to_f16(range / 15.0f);
            uint16_t hm = or_f32_to_f16(lo);
            sc[g] = hs;
            mn[g] = hm;
            float s = or_f16_to_f32(hs), m = or_f16_to_f32(hm);
            float div = (s == 0.0f) ? 1.0f : s;
            for (int i = 0; i < G; ++i) {
                float v = rintf((gp[i] - m) / div);
                if (v < 0.0f) v = 0.0f;
                if (v > 15.0f) v = 15.0f;
                q[g * G + i] = (uint8_t)v;
                if (deq) deq[n * K + g * G + i] = v * s + m;
            }
        }
        or_q4_pack(q, sc, mn, 1, K, G, wq + n * (K / 8), ws + n * NG);
    }
    free(q);
    free(sc);
    free(mn);
}

/* --------------------------------------------------- activation quant ---- */

/* RMSNorm prologue in the kernels' reduction order.  The row is read in
 * passes of 2048 elements: in load u (0..7) of pass j, lane l (0..63) holds
 * the float4 chunk 512 j + 64 u + l (coalesced).  Chunk u's partial c_u is
 * an fmaf chain over its 4 elements in index order; a lane's partial is the
 * pairwise tree ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), so that
 * waves holding 2, 4 or 8 of the loads can form it together.  The 64 lane
 * partials of a pass are combined by a pairwise tree with offsets 1, 2, ...,
 * 32 (p[i] += p[i + o] for i with bit o clear: the wavefront's xor
 * butterfly); chunks past K count as 0; the pass sums are added in pass
 * order.
 * quant.wgsl:24-39: r = 1/sqrt(mean(x^2) + eps); v = (x * r) * nw. */
static float rms_scale(const float* x, int64_t K, float eps) {
    float total = 0.0f;
    for (int64_t j = 0; 2048 * j < K; ++j) {
        float p[64];
        for (int l = 0; l < 64; ++l) {
            float c[8];
            for (int u = 0; u < 8; ++u) {
                const int64_t b = 4 * (512 * j + 64 * u + l);
                c[u] = 0.0f;
                if (b < K)
                    for (int e = 0; e < 4; ++e) c[u] = fmaf(x[b + e], x[b + e], c[u]);
            }
            p[l] = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
        }
        for (int o = 1; o < 64; o <<= 1)
            for (int i = 0; i < 64; ++i)
                if (!(i & o)) p[i] = p[i] + p[i + o];
        total = total + p[0];
    }
    return 1.0f / sqrtf(total / (float)K + eps);
}

/* quant.wgsl:41-61 and tools/reference.py:43-48 (fq_input):
 *   per activation group (GA elements): dx = amax / 127 (fp32);
 *   xq = dx > 0 ? rne(v / dx) : 0 (IEEE division); xs = sum xq per Ge group. */
void or_quant_act(const float* x, const float* norm_w, float eps,
                  int64_t M, int64_t K, int GA, int G,
                  int8_t* xq, float* dx, int32_t* xs) {
    int Ge = GA < G ? GA : G;
    float* v = (float*)malloc((size_t)K * 4);
    for (int64_t t = 0; t < M; ++t) {
        const float* xr = x + t * K;
        if (norm_w) {
            float r = rms_scale(xr, K, eps);
            for (int64_t k = 0; k < K; ++k) v[k] = (xr[k] * r) * norm_w[k];
        } else {
            memcpy(v, xr, (size_t)K * 4);
        }
        for (int64_t a = 0; a < K / GA; ++a) {
            float amax = 0.0f;
            for (int i = 0; i < GA; ++i) {
                float e = fabsf(v[a * GA + i]);
                if (e > amax) amax = e;
            }
            float d = amax / 127.0f;
            dx[t * (K / GA) + a] = d;
            for (int i = 0; i < GA; ++i) {
                float q = d > 0.0f ? rintf(v[a * GA + i] / d) : 0.0f;
                xq[t * K + a * GA + i] = (int8_t)q;
            }
        }
        for (int64_t e = 0; e < K / Ge; ++e) {
            int32_t s = 0;
            for (int i = 0; i < Ge; ++i) s += xq[t * K + e * Ge + i];
            xs[t * (K / Ge) + e] = s;
        }
    }
    free(v);
}

/* ------------------------------------------------------------- linear ---- */

static inline uint32_t code(const uint32_t* row, int64_t k) {
    /* element k of a packed row: word k/8, byte (k%8)&3, nibble k%8 >= 4 */
    uint32_t w = row[k >> 3];
    int j = (int)(k & 7);
    return (w >> (8 * (j & 3) + 4 * (j >> 2))) & 15u;
}

/* gemv_q4q8.wgsl:29-34,68: A = sum over the group of q * xq, exact int32. */
void or_group_acc(const uint32_t* wq, int64_t N, int64_t K, int Ge,
                  const int8_t* xq, int64_t M, int32_t* acc) {
    int64_t NE = K / Ge;
    for (int64_t t = 0; t < M; ++t)
        for (int64_t n = 0; n < N; ++n) {
            const uint32_t* row = wq + n * (K / 8);
            for (int64_t e = 0; e < NE; ++e) {
                int32_t a = 0;
                for (int i = 0; i < Ge; ++i) {
                    int64_t k = e * Ge + i;
                    a += (int32_t)code(row, k) * (int32_t)xq[t * K + k];
                }
                acc[(t * N + n) * NE + e] = a;
            }
        }
}

/* Per-group identity of gemv_q4q8.wgsl:6:  sum_i (q s + m)(xq dx) = dx (s A + m X).
 * Canonical fp32 order shared with the kernels (this build's own; the
 * reference's subgroup reductions cannot be run here):
 *   per token, G = 128:  per pass of 2048 codes (16 groups), eight chains,
 *                        chain i over the groups 16p + 2i, 16p + 2i + 1 that
 *                        exist: c = fma(s, A, c); c = fma(m, X, c) from c = 0;
 *                        T_p = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
 *                        the pass sums added left to right; a = total * dx
 *   per 32   (GA = 32):  per pass of 2048 codes (64 groups of 32), sixteen
 *                        chains, chain i over the groups 64p + 4i .. 64p + 4i + 3
 *                        that exist: c = fma(s*dx_e, A, c); c = fma(m*dx_e, X, c)
 *                        from c = 0; T_p = the pairwise tree over c_0 .. c_15;
 *                        the pass sums added left to right; a = total
 *   per token, G = 32:   the per-32 order with the token's scale outside:
 *                        c = fma(s, A, c); c = fma(m, X, c); a = total * dx */
static float row_value(const uint32_t* wrow, const uint32_t* srow, int64_t K, int G, int GA,
                       const int8_t* xrow, const float* dxrow, const int32_t* xsrow) {
    int Ge = GA < G ? GA : G;
    int64_t NE = K / Ge;
    if (GA >= K && G == 128) {
        float total = 0.0f;
        for (int64_t e0 = 0; e0 < NE; e0 += 16) {
            float c[8];
            for (int q = 0; q < 8; ++q) {
                c[q] = 0.0f;
                for (int k = 0; k < 2; ++k) {
                    int64_t e = e0 + 2 * q + k;
                    if (e >= NE) break;
                    int32_t a = 0;
                    for (int i = 0; i < Ge; ++i) {
                        int64_t kk = e * Ge + i;
                        a += (int32_t)code(wrow, kk) * (int32_t)xrow[kk];
                    }
                    uint32_t sw = srow[e];
                    float s = or_f16_to_f32((uint16_t)(sw & 0xFFFFu));
                    float m = or_f16_to_f32((uint16_t)(sw >> 16));
                    c[q] = fmaf(s, (float)a, c[q]);
                    c[q] = fmaf(m, (float)xsrow[e], c[q]);
                }
            }
            float t = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
            total = e0 == 0 ? t : total + t;
        }
        return total * dxrow[0];
    }
    if (GA < K || G == 32) {
        const int pt = GA >= K;
        float total = 0.0f;
        for (int64_t e0 = 0; e0 < NE; e0 += 64) {
            float c[16];
            for (int q = 0; q < 16; ++q) {
                c[q] = 0.0f;
                for (int k = 0; k < 4; ++k) {
                    int64_t e = e0 + 4 * q + k;
                    if (e >= NE) break;
                    int32_t a = 0;
                    for (int i = 0; i < Ge; ++i) {
                        int64_t kk = e * Ge + i;
                        a += (int32_t)code(wrow, kk) * (int32_t)xrow[kk];
                    }
                    uint32_t sw = srow[(e * Ge) / G];
                    float s = or_f16_to_f32((uint16_t)(sw & 0xFFFFu));
                    float m = or_f16_to_f32((uint16_t)(sw >> 16));
                    if (pt) {
                        c[q] = fmaf(s, (float)a, c[q]);
                        c[q] = fmaf(m, (float)xsrow[e], c[q]);
                    } else {
                        float d = dxrow[e];
                        c[q] = fmaf(s * d, (float)a, c[q]);
                        c[q] = fmaf(m * d, (float)xsrow[e], c[q]);
                    }
                }
            }
            for (int w = 16; w > 1; w /= 2)
                for (int k = 0; k < w / 2; ++k) c[k] = c[2 * k] + c[2 * k + 1];
            total = e0 == 0 ? c[0] : total + c[0];
        }
        return pt ? total * dxrow[0] : total;
    }
    return 0.0f;  /* not reached: G is 32 or 128 (checked by the callers) */
}

/* Output modes of gemv_q4q8.wgsl:122-129 / gemm_q4q8.wgsl:112-118. */
int or_linear(const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int G,
              const int8_t* xq, const float* dx, const int32_t* xs,
              int64_t M, int GA, int mode, float* y) {
    if ((G != 32 && G != 128) || K % G || (GA != 32 && GA != K) || mode < 0 || mode > 2) return -1;
    int Ge = GA < G ? GA : G;
    int64_t NE = K / Ge, KW = K / 8, NG = K / G;
    for (int64_t t = 0; t < M; ++t) {
        const int8_t* xr = xq + t * K;
        const float* dr = dx + t * (K / GA);
        const int32_t* sr = xs + t * NE;
        for (int64_t n = 0; n < N; ++n) {
            float a = row_value(wq + n * KW, ws + n * NG, K, G, GA, xr, dr, sr);
            float* o = y + t * N + n;
            if (mode == 0) {
                *o = a;
            } else if (mode == 1) {
                *o = *o + a;
            } else {
                float u = row_value(wq + (n + N) * KW, ws + (n + N) * NG, K, G, GA, xr, dr, sr);
                *o = a / (1.0f + expf(-a)) * u;
            }
        }
    }
    return 0;
}

/* argmax.wgsl:14-43: best starts at -3e38 with index 0, a strict > scan keeps
 * the first occurrence, so NaN and values <= -3e38 never win and ties go to
 * the lowest index; MAPPED returns ids[idx]. */
void or_argmax(const float* logits, int64_t M, int64_t N, const uint32_t* ids,
               uint32_t* tok_out) {
    for (int64_t t = 0; t < M; ++t) {
        float best = -3.0e38f;
        uint32_t idx = 0;
        for (int64_t i = 0; i < N; ++i) {
            float v = logits[t * N + i];
            if (v > best) {
                best = v;
                idx = (uint32_t)i;
            }
        }
        tok_out[t] = ids ? ids[idx] : idx;
    }
}

/* embed.wgsl:13-27.  Word i of a row holds codes 8i..8i+7 (byte b = code
 * 8i+b | code 8i+4+b << 4); each code is dequantised as f32(q) * s + m with
 * the (s, m) of its group, the product rounded before the sum. */
void or_embed(const uint32_t* eq, const uint32_t* es, int64_t V, int64_t K, int G,
              const uint32_t* tok, int64_t M, float* x) {
    for (int64_t m = 0; m < M; ++m) {
        float* xr = x + m * K;
        const uint32_t t = tok[m];
        if ((int64_t)t >= V) {
            for (int64_t k = 0; k < K; ++k) xr[k] = 0.0f;
            continue;
        }
        const uint32_t* qr = eq + (int64_t)t * (K / 8);
        const uint32_t* sr = es + (int64_t)t * (K / G);
        for (int64_t i = 0; i < K / 8; ++i) {
            const uint32_t w = qr[i];
            for (int b = 0; b < 4; ++b) {
                const int64_t k0 = 8 * i + b, k1 = 8 * i + 4 + b;
                const uint32_t s0 = sr[k0 / G], s1 = sr[k1 / G];
                const float p0 = (float)((w >> (8 * b)) & 15u) * or_f16_to_f32((uint16_t)(s0 & 0xFFFFu));
                const float p1 = (float)((w >> (8 * b + 4)) & 15u) * or_f16_to_f32((uint16_t)(s1 & 0xFFFFu));
                xr[k0] = p0 + or_f16_to_f32((uint16_t)(s0 >> 16));
                xr[k1] = p1 + or_f16_to_f32((uint16_t)(s1 >> 16));
            }
        }
    }
}

/* gather_rows.wgsl:13-24. */
void or_gather_rows(const uint32_t* sq, const uint32_t* ss, int64_t V, int64_t K, int G,
                    const uint32_t* ids, int64_t R, uint32_t* dq, uint32_t* ds) {
    const int64_t W = K / 8, WS = K / G;
    for (int64_t r = 0; r < R; ++r) {
        const uint32_t src = ids[r];
        const int ok = (int64_t)src < V;
        for (int64_t i = 0; i < W; ++i) dq[r * W + i] = ok ? sq[(int64_t)src * W + i] : 0u;
        for (int64_t i = 0; i < WS; ++i) ds[r * WS + i] = ok ? ss[(int64_t)src * WS + i] : 0u;
    }
}

/* ------------------------------------------------------------ MTP input ---- */

/* mtp_in.wgsl:45-89 (dispatch graph.rs:500-504): row m of the [M, 2K] output
 * is quant32(norm_e(emb[m])) then quant32(norm_h(norm_f(x[m]))).  Each norm
 * scales as the reference writes it, v * (r * w) (mtp_in.wgsl:56,65,70), with
 * r = 1 / sqrt(mean(v^2) + eps) from rms_scale's order over the values it
 * normalises; quant32 is or_quant_act's per-32 quantiser (GA = Ge = 32). */
void or_mtp_in(const float* emb, const float* x, const float* nf, const float* ne,
               const float* nh, float eps, int64_t M, int64_t K,
               int8_t* xq, float* dx, int32_t* xs) {
    float* v = (float*)malloc((size_t)K * 4);
    for (int64_t m = 0; m < M; ++m) {
        for (int half = 0; half < 2; ++half) {
            const int64_t row = 2 * m + half;
            memcpy(v, (half ? x : emb) + m * K, (size_t)K * 4);
            const float* w0 = half ? nf : ne;
            float r = rms_scale(v, K, eps);
            for (int64_t k = 0; k < K; ++k) v[k] = v[k] * (r * w0[k]);
            if (half) {
                r = rms_scale(v, K, eps);
                for (int64_t k = 0; k < K; ++k) v[k] = v[k] * (r * nh[k]);
            }
            or_quant_act(v, NULL, eps, 1, K, 32, 32, xq + row * K, dx + row * (K / 32),
                         xs + row * (K / 32));
        }
    }
    free(v);
}

/* ------------------------------------------------ attention chunk merge ---- */

/* attn_combine.wgsl:36-82 (dispatch graph.rs:289-291) in the HIP kernel's
 * order.  part [M, H, nch, D + 2]: per chunk the D output sums, the chunk
 * max score and its weight sum (attn.wgsl:104-113); token m merges chunks
 * 0 .. (pos + m + 32) / 32 - 1.
 *   mx = max m_c; w_c = expf(m_c - mx)
 *   l: lane j (0..63) accumulates fmaf(w_c, l_c, .) over c = j, j + 64, ...,
 *      then the pairwise tree over the 64 lanes (as rms_scale)
 *   o[i] = ((o_0 + o_1) + (o_2 + o_3)) / l with o_w the fmaf chain of
 *      w_c * part_c[i] over c = w, w + 4, ... in order (four wavefronts)
 *   gated: o[i] = o[i] / (1 + expf(-g[i])), g at gate[m*gs + h*2D + D + i]
 *   per 32 dims: dx = amax / 127, xq = rint(o / dx), xs = sum xq.
 * The device's expf may differ from the host's in the last bit, so codes
 * are exact only where every weight is exp(0) (equal chunk maxima) and no
 * gate is applied; elsewhere the comparison carries a tolerance. */
void or_attn_combine(const float* part, int64_t M, int64_t H, int64_t D, int64_t nch,
                     int64_t pos, const float* gate, int64_t gs,
                     int8_t* xq, float* dx, int32_t* xs) {
    float* w = (float*)malloc((size_t)nch * 4);
    float* o = (float*)malloc((size_t)D * 4);
    const int64_t K = H * D;
    for (int64_t m = 0; m < M; ++m) {
        const int64_t n = (pos + m + 32) / 32;
        for (int64_t h = 0; h < H; ++h) {
            const float* hb = part + ((m * H + h) * nch) * (D + 2);
            float mx = -3.0e38f;
            for (int64_t c = 0; c < n; ++c) mx = fmaxf(mx, hb[c * (D + 2) + D]);
            float p[64];
            for (int j = 0; j < 64; ++j) p[j] = 0.0f;
            for (int64_t c = 0; c < n; ++c) {
                w[c] = expf(hb[c * (D + 2) + D] - mx);
                p[c % 64] = fmaf(w[c], hb[c * (D + 2) + D + 1], p[c % 64]);
            }
            for (int off = 1; off < 64; off <<= 1)
                for (int j = 0; j < 64; ++j)
                    if (!(j & off)) p[j] = p[j] + p[j + off];
            const float l = p[0];
            for (int64_t i = 0; i < D; ++i) {
                float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int64_t c = 0; c < n; ++c) acc[c % 4] = fmaf(w[c], hb[c * (D + 2) + i], acc[c % 4]);
                o[i] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) / l;
                if (gate) o[i] = o[i] / (1.0f + expf(-gate[m * gs + h * 2 * D + D + i]));
            }
            for (int64_t g = 0; g < D / 32; ++g) {
                float amax = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    const float e = fabsf(o[32 * g + i]);
                    if (e > amax) amax = e;
                }
                const float d = amax / 127.0f;
                int32_t sum = 0;
                for (int i = 0; i < 32; ++i) {
                    const float q = d > 0.0f ? rintf(o[32 * g + i] / d) : 0.0f;
                    xq[m * K + h * D + 32 * g + i] = (int8_t)q;
                    sum += (int32_t)q;
                }
                const int64_t gi = m * (K / 32) + (h * D + 32 * g) / 32;
                dx[gi] = d;
                xs[gi] = sum;
            }
        }
    }
    free(w);
    free(o);
}
