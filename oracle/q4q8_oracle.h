/*
 * CPU oracle for webyIQ's fused int4 x int8 linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This restatement of the reference arithmetic is
 * the checker for the HIP kernels; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  The product path never calls it.
 *
 * Conventions (shared with the HIP kernels, see each function):
 *   .q  u32 [N, K/8]   word i of row n: byte b = q[n,8i+b] | q[n,8i+4+b] << 4
 *   .s  u32 [N, K/G]   low 16 bits = f16 scale s, high 16 bits = f16 min m;
 *                      dequantised weight w = q*s + m
 *   xq  i8  [M, K]     per-token (GA = K) or per-32 (GA = 32) symmetric int8
 *   dx  f32 [M, K/GA]  activation scale, x ~= xq * dx
 *   xs  i32 [M, K/Ge]  sum of xq over each accumulation group, Ge = min(G, GA)
 *   A   i32 [M, N, K/Ge]  exact integer group accumulators sum q*xq
 */
#ifndef WEBYIQ_Q4Q8_ORACLE_H
#define WEBYIQ_Q4Q8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32 (round to nearest even), as numpy's astype. */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* RTN int4 quantiser + packer: tools/convert.py:55-106 (search=False). */
void or_q4_quantize(const float* w, int64_t N, int64_t K, int G,
                    uint32_t* wq, uint32_t* ws, float* deq /* nullable */);
/* Pack raw codes (0..15) + f16 scale/min: tools/convert.py:68-75. */
void or_q4_pack(const uint8_t* q, const uint16_t* scale, const uint16_t* mn,
                int64_t N, int64_t K, int G, uint32_t* wq, uint32_t* ws);
/* Inverse of or_q4_pack's code interleave (crates/engine/src/shaders/embed.wgsl:22-24). */
void or_q4_unpack(const uint32_t* wq, int64_t N, int64_t K, uint8_t* q);

/* Activation quantiser: quant.wgsl:41-61 / tools/reference.py:43-48 with
 * granularity GA (32 or K), IEEE division and round-half-even.
 * If norm_w != NULL an RMSNorm prologue (quant.wgsl:24-39) is applied first. */
void or_quant_act(const float* x, const float* norm_w, float eps,
                  int64_t M, int64_t K, int GA, int G,
                  int8_t* xq, float* dx, int32_t* xs);

/* Exact integer group accumulators A[t, n, e] (gemv_q4q8.wgsl:29-34,68). */
void or_group_acc(const uint32_t* wq, int64_t N, int64_t K, int Ge,
                  const int8_t* xq, int64_t M, int32_t* acc);

/* Linear layer, canonical epilogue (gemv_q4q8.wgsl:6,68,117-130;
 * gemm_q4q8.wgsl:96,104-119).  mode 0: y = a, 1: y += a,
 * 2: y = silu(a_n) * a_{n+N} with the up rows stored after the N gate rows.
 * y is [M, N]; wq/ws hold N rows (2N for mode 2). */
int or_linear(const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int G,
              const int8_t* xq, const float* dx, const int32_t* xs,
              int64_t M, int GA, int mode, float* y);

/* Greedy argmax with the reference tie rule (argmax.wgsl:14-43):
 * max over v > -3e38 (NaN never wins), ties -> lowest index, ids map if given. */
void or_argmax(const float* logits, int64_t M, int64_t N, const uint32_t* ids,
               uint32_t* tok_out);

/* int4 embedding lookup (embed.wgsl:13-27): x[m, k] = f32(q) * s + m of row
 * tok[m] (a product, then a sum); ids outside [0, V) give a zero row. */
void or_embed(const uint32_t* eq, const uint32_t* es, int64_t V, int64_t K, int G,
              const uint32_t* tok, int64_t M, float* x);

/* Packed row gather (gather_rows.wgsl:13-24): dst row r = src row ids[r];
 * ids outside [0, V) give zero rows. */
void or_gather_rows(const uint32_t* sq, const uint32_t* ss, int64_t V, int64_t K, int G,
                    const uint32_t* ids, int64_t R, uint32_t* dq, uint32_t* ds);

/* MTP input stage (mtp_in.wgsl:45-89): xq i8 [M, 2K], dx/xs [M, 2K/32]. */
void or_mtp_in(const float* emb, const float* x, const float* nf, const float* ne,
               const float* nh, float eps, int64_t M, int64_t K,
               int8_t* xq, float* dx, int32_t* xs);

/* Flash-decoding chunk merge + per-32 int8 groups (attn_combine.wgsl:36-82):
 * xq i8 [M, H*D], dx/xs [M, H*D/32]; gate nullable (row stride gs). */
void or_attn_combine(const float* part, int64_t M, int64_t H, int64_t D, int64_t nch,
                     int64_t pos, const float* gate, int64_t gs,
                     int8_t* xq, float* dx, int32_t* xs);

#ifdef __cplusplus
}
#endif
#endif
