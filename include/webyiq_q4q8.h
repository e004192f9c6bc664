/*
 * webyiq_q4q8.h -- C ABI of the MI355X (gfx950) int4 x int8 linear-layer path.
 *
 * Drop-in for the operator layer of webyIQ's Rust engine
 * (crates/engine/src/graph.rs:149-222 Builder::{gemv, gemm, matmul, quant},
 * graph.rs:476-486 head_ops) and the WGSL kernels it specialises
 * (crates/engine/src/shaders/{quant, gemv_q4q8, gemm_q4q8, argmax}.wgsl).
 * Only plain pointers and sizes cross the boundary: every pointer argument is
 * device memory (hipMalloc) owned by the caller; `stream` is a hipStream_t
 * (NULL = the default stream).  All calls are asynchronous and stream
 * ordered; no call synchronises the host or allocates memory.
 *
 * Tensor layout (webyIQ tools/convert.py:8-12, manifest quant.group = G):
 *   wq  u32 [N, K/8]   8 int4 codes per word; byte b of word i =
 *                      q[8i+b] | q[8i+4+b] << 4
 *   ws  u32 [N, K/G]   low 16 bits f16 scale s, high 16 bits f16 min m;
 *                      weight = q * s + m  (a zero point z is m = -z * s)
 *   xq  i8  [M, K]     int8 activations, x ~= xq * dx
 *   dx  f32 [M, K/GA]  activation scale; GA = K (per token) or 32 (per group,
 *                      as the reference ships, quant.wgsl:3)
 *   xs  i32 [M, K/Ge]  sum of xq over each accumulation group, Ge = min(G, GA)
 *   y   f32 [M, N]
 *
 * Output modes (gemv_q4q8.wgsl:4, gemm_q4q8.wgsl:3):
 *   WQ_MODE_STORE      y = W x
 *   WQ_MODE_ACCUMULATE y += W x            (residual add)
 *   WQ_MODE_SILU_MUL   y = silu(W[n] x) * W[n+N] x, gate rows 0..N-1 then up
 *                      rows N..2N-1 of one [2N, K] tensor (convert.py:184,231)
 *
 * Errors mirror the engine's Result<_, String>: a negative status code, and
 * wq_last_error() returns the message (thread-local, valid until the next call
 * on the same thread).  Arguments are validated on the host before anything
 * is launched; on error nothing is launched.
 */
#ifndef WEBYIQ_Q4Q8_H
#define WEBYIQ_Q4Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WQ_ABI_VERSION 2

/* status codes */
#define WQ_OK 0
#define WQ_EINVAL (-1)     /* null pointer, unknown mode/path */
#define WQ_ESHAPE (-2)     /* shape outside the supported set */
#define WQ_EALIGN (-3)     /* pointer alignment */
#define WQ_EHIP (-4)       /* HIP runtime error at launch */
#define WQ_EWORKSPACE (-5) /* workspace missing or too small */

/* output modes */
#define WQ_MODE_STORE 0
#define WQ_MODE_ACCUMULATE 1
#define WQ_MODE_SILU_MUL 2

/*
 * Step parameters read by the kernels at run time, the reference's Params
 * uniform (gemm_q4q8.wgsl:8-13, attn_combine.wgsl:6-11; written by the host
 * per step, lib.rs:312-314, or by the GPU itself on the speculative path,
 * lib.rs:325).  Passed as a pointer to 16 bytes of device memory, so a
 * recorded call (HIP graph, replayed op list) follows whatever the buffer
 * holds when the kernel runs.
 *   pos      position of the step's first token
 *   seq_len  attention length (not read by this library's kernels)
 *   m        tokens in the step
 *   slot     readback slot (not read by this library's kernels)
 */
typedef struct wq_params {
    uint32_t pos;
    uint32_t seq_len;
    uint32_t m;
    uint32_t slot;
} wq_params;

/* which dispatch list a product belongs to (graph.rs:127-146 Path) */
#define WQ_PATH_DECODE 0  /* one token: GEMV */
#define WQ_PATH_SPEC 1    /* speculative verify, M <= 8 tokens: GEMV */
#define WQ_PATH_PREFILL 2 /* a prompt chunk: GEMM on int8 MFMA */

/* Message of the last failed call on this thread ("" after success). */
const char* wq_last_error(void);

/* WQ_ABI_VERSION of the loaded library. */
int wq_abi_version(void);

/*
 * Activation quantiser.  Replaces Builder::quant (graph.rs:216-222) and
 * quant.wgsl:19-62; semantics of tools/reference.py:43-48 (fq_input).
 *   v = norm_w ? (x * r) * norm_w : x,  r = 1 / sqrt(mean(x^2) + eps)
 *   per activation group of GA elements: dx = max|v| / 127,
 *   xq = dx > 0 ? round_half_even(v / dx) : 0  (IEEE division)
 *   xs[e] = sum of xq over accumulation group e of Ge = min(G, GA) elements
 * x f32 [M, K], norm_w f32 [K] or NULL.  GA in {32, K}; G in {32, 128} is
 * the weight group of the linear layer that will consume xq.
 * Requires K % 128 == 0; x, norm_w and xq 16-byte aligned.
 */
int wq_quant_act(void* stream, const float* x, const float* norm_w, float eps,
                 int64_t M, int64_t K, int32_t GA, int32_t G,
                 int8_t* xq, float* dx, int32_t* xs);

/*
 * Decode GEMV, 1 <= M <= 8 tokens.  Replaces Builder::gemv (graph.rs:190-198)
 * and gemv_q4q8.wgsl:36-131.  Requires K % 128 == 0, G in {32, 128},
 * GA in {32, K}; wq and xq 16-byte aligned.  wq/ws hold 2N rows in
 * WQ_MODE_SILU_MUL.  Outputs of WQ_MODE_STORE / WQ_MODE_ACCUMULATE are
 * bit-reproducible, in one fixed fp32 order for every M and launch plan:
 * per-token activations at G = 128 fold each 2048-code pass as fma chains
 * over pairs of groups and a pairwise tree over the pairs, per-32
 * activations as chains over four groups and a tree over the 16 chains, the
 * passes in order; per-token activations at G = 32 the same chains and tree
 * with the token's dx applied to the total.
 */
int wq_gemv(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K,
            int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
            int64_t M, int32_t GA, int32_t mode, float* y);

/*
 * Quantiser + decode GEMV, 1 <= M <= 8, per-token activation scales
 * (GA = K).  Replaces the quant -> matmul pairs of the decode layer
 * (graph.rs:266+269, 285+293, 304+305, 313+314, 323+324, 325+326) and of the
 * head (graph.rs:482-483).  y and the quantised activations xq i8 [M, K],
 * dx f32 [M], xs i32 [M, K/G] (required outputs, read by the products that
 * share the input) are bit-identical to wq_quant_act(GA = K) followed by
 * wq_gemv.  M <= 2 is one launch: every workgroup quantises the tokens while
 * its weight loads are in flight, and workgroup 0 writes xq/dx/xs; larger M
 * is those two launches.  y must not overlap x.  Requirements of wq_gemv and
 * wq_quant_act (x, norm_w 16-byte aligned).
 */
int wq_quant_gemv(void* stream, const float* x, const float* norm_w, float eps,
                  const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int32_t G,
                  int64_t M, int32_t mode, int8_t* xq, float* dx, int32_t* xs, float* y);

/*
 * Prefill GEMM, any M >= 1 (tiles of 128 tokens).  Replaces Builder::gemm
 * (graph.rs:200-205, which binds the step's Params) and
 * gemm_q4q8.wgsl:46-121.  Same arguments and constraints as wq_gemv, plus
 * M * K and rows * K / 2 (rows = N, or 2N in WQ_MODE_SILU_MUL) below 4 GiB.
 * params (device memory, nullable): NULL -> the product covers M tokens.
 * Otherwise M is the capacity the launch is sized for (xq, dx, xs and y hold
 * M rows) and the kernel reads params->m when it runs: tokens
 * 0 .. min(params->m, M) - 1 are computed and stored, rows past them are
 * neither read beyond row M - 1 nor written, and token tiles past them end at
 * once (the reference clamps its tokens to p.m, gemm_q4q8.wgsl:69,106).
 * The int32 group sums are the GEMV's; with per-token activations (G = 128
 * or 32) the min term is summed on an f16 MFMA (exact products, fp32 sums in
 * hardware order) and per-32 activations fold one chain per output (the
 * GEMV: chains and a tree): the fp32 outputs agree with wq_gemv within
 * rel 1e-5.
 * workspace (device, nullable, 256-byte aligned; no counterpart in the
 * reference): when it holds at least wq_gemm_workspace_bytes(...) > 0 bytes
 * for the call's shape, the K steps of each output tile may be split between
 * two workgroups whose partial sums meet in it (the first half's added to
 * the second's, one fixed order: outputs are deterministic and within
 * rel 1e-5 of the unsplit launch).  It must be zero before its first use
 * (wq_workspace_clear) and every call leaves its flags zero again; calls
 * sharing one workspace must not overlap.  A partner's wait is bounded
 * (~0.5 s); if it ran out, that tile's outputs are NaN and the workspace is
 * to be cleared before the next call.  NULL, or fewer bytes: the unsplit
 * launch.
 */
int wq_gemm(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K,
            int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
            int64_t M, int32_t GA, int32_t mode, float* y, const wq_params* params,
            void* workspace, size_t workspace_bytes);

/* Bytes of workspace wq_gemm can use for this shape (M the capacity); 0
 * when the shape is never split. */
size_t wq_gemm_workspace_bytes(int64_t N, int64_t K, int32_t G, int64_t M, int32_t GA, int32_t mode);

/*
 * Builder::matmul (graph.rs:207-214): WQ_PATH_PREFILL -> wq_gemm (with
 * params, nullable), otherwise wq_gemv (WQ_PATH_DECODE requires M == 1,
 * WQ_PATH_SPEC M <= 8; params unused, as the reference's gemv binds none).
 */
int wq_matmul(void* stream, int32_t path, const uint32_t* wq, const uint32_t* ws,
              int64_t N, int64_t K, int32_t G, const int8_t* xq, const float* dx,
              const int32_t* xs, int64_t M, int32_t GA, int32_t mode, float* y,
              const wq_params* params);

/*
 * Greedy argmax over logits f32 [M, V] (argmax.wgsl:14-43): the maximum over
 * values > -3e38 (NaN never wins), ties to the lowest index, 0 when no value
 * qualifies; with ids != NULL the winning index i is mapped to ids[i]
 * (the draft vocabulary, MAPPED in argmax.wgsl:41).  tok_out u32 [M].
 */
int wq_argmax(void* stream, const float* logits, int64_t M, int64_t V,
              const uint32_t* ids, uint32_t* tok_out);

/*
 * lm_head GEMV with fused greedy argmax, 1 <= M <= 8.  Replaces the
 * gemv + argmax pair of head_ops (graph.rs:482-484) with one launch.  The
 * token is bit-identical to wq_gemv(WQ_MODE_STORE) followed by wq_argmax.
 * logits f32 [M, V] is written when non-NULL.  `workspace` (device, at least
 * wq_lm_head_workspace_bytes() bytes) carries the cross-workgroup reduction;
 * it must be zero before the first call (wq_workspace_clear) and every call
 * leaves it zero again.  Calls sharing one workspace must not overlap.
 * The final workgroup's wait for the others is bounded (~0.5 s, far beyond
 * any launch): if it ever runs out, every token is written as 0xFFFFFFFF
 * (never a valid index, V <= 0xFFFFFFFE) and the workspace may be left
 * non-zero; clear it (wq_workspace_clear, stream-ordered after the call)
 * before the next call.
 */
int wq_lm_head_argmax(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t V,
                      int64_t K, int32_t G, const int8_t* xq, const float* dx,
                      const int32_t* xs, int64_t M, int32_t GA, const uint32_t* ids,
                      float* logits, uint32_t* tok_out, void* workspace,
                      size_t workspace_bytes);

/*
 * wq_lm_head_argmax without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * cross-workgroup reduction runs in the library's own static device array of
 * wq_lm_head_workspace_bytes() bytes, one per GPU, held until the process
 * ends; its address is looked up on the first call per device.  Nothing is
 * allocated.  The array starts zeroed and every call leaves it zeroed.
 * Calls that overlap on one GPU (concurrent streams, or threads) race on the
 * array and must not be issued; use wq_lm_head_argmax with one workspace per
 * stream for that.  Limits: M <= 8 tokens (as wq_lm_head_argmax); other
 * arguments and the result as wq_lm_head_argmax, including the 0xFFFFFFFF
 * tokens of a wait that ran out, after which the array must be reset with
 * wq_lm_head_noalloc_reset before the next call.
 */
int wq_lm_head_argmax_noalloc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t V,
                              int64_t K, int32_t G, const int8_t* xq, const float* dx,
                              const int32_t* xs, int64_t M, int32_t GA, const uint32_t* ids,
                              float* logits, uint32_t* tok_out);

/*
 * Zero the current GPU's static array of wq_lm_head_argmax_noalloc with a
 * fill kernel on `stream` (no allocation, no hipMemset; safe inside graph
 * capture).  No counterpart in the reference.  Needed only after a call
 * returned 0xFFFFFFFF tokens; issue it stream-ordered after that call, with
 * no other wq_lm_head_argmax_noalloc call in flight on the GPU.
 */
int wq_lm_head_noalloc_reset(void* stream);

/* Bytes of workspace wq_lm_head_argmax needs (no counterpart in the
 * reference, whose argmax runs as a separate single-workgroup dispatch). */
size_t wq_lm_head_workspace_bytes(void);

/* Zero `bytes` of device memory with a fill kernel (safe inside HIP graph
 * capture, unlike hipMemsetAsync). */
int wq_workspace_clear(void* stream, void* workspace, size_t bytes);

/*
 * int4 embedding lookup: x[m, :] = dequantised row tok[m] of the packed
 * matrix (eq, es), x = q * s + m per code (a product, then a sum, as
 * f32(q) * s.x + s.y in embed.wgsl:13-27).  Replaces the embed op of the
 * decode and prefill graphs (graph.rs:439-443, 502).  Token ids outside
 * [0, V) give a zero row.  x f32 [M, K]; K % 128 == 0, G in {32, 128};
 * eq and x 16-byte aligned.
 */
int wq_embed(void* stream, const uint32_t* eq, const uint32_t* es, int64_t V, int64_t K,
             int32_t G, const uint32_t* tok, int64_t M, float* x);

/*
 * Row gather of a packed int4 matrix: row r of (dq, ds) = row ids[r] of
 * (sq, ss).  Replaces the one-time gather of the reduced draft lm_head
 * (gather_rows.wgsl:13-24, graph.rs:511-516; ids from convert.py:327-330).
 * Ids outside [0, V) give zero rows.  sq and dq 16-byte aligned.
 */
int wq_gather_rows(void* stream, const uint32_t* sq, const uint32_t* ss, int64_t V, int64_t K,
                   int32_t G, const uint32_t* ids, int64_t R, uint32_t* dq, uint32_t* ds);

/*
 * MTP input stage: the int8 input of the MTP fc projection, a [M, 2K] row
 * per token with per-32 activation scales (GA = 32, Ge = 32):
 *   columns [0, K)  = quant(norm_e(emb[m])),
 *   columns [K, 2K) = quant(norm_h(norm_f(x[m]))),
 * each norm v * (r * w) with r = 1 / sqrt(mean(v^2) + eps) over the values it
 * normalises (mtp_in.wgsl:45-89, dispatched by graph.rs:500-504; emb is the
 * embedding of the next token, x the last hidden state before the final
 * norm).  xq i8 [M, 2K], dx f32 [M, 2K/32], xs i32 [M, 2K/32];
 * K % 128 == 0; emb, x, the norms and xq 16-byte aligned.
 */
int wq_mtp_in(void* stream, const float* emb, const float* x, const float* norm_f,
              const float* norm_e, const float* norm_h, float eps, int64_t M, int64_t K,
              int8_t* xq, float* dx, int32_t* xs);

/*
 * Flash-decoding merge of attention partials, emitted as the int8 input of
 * the o projection with per-32 activation scales (attn_combine.wgsl:1-83,
 * dispatched per (token, head) by graph.rs:289-291).  part f32
 * [M, H, nch, D + 2]: per chunk of 32 positions the D weighted output sums,
 * the chunk's maximum score and its weight sum (attn.wgsl:104-113).  Token
 * m covers positions 0 ..= pos + m.  gate (nullable, Qwen3.5's gated
 * attention): the gate of (m, h, i) is gate[m * gate_stride + h * 2D + D + i]
 * and the output is divided by 1 + exp(-gate).  xq i8 [M, H*D],
 * dx f32 [M, H*D/32], xs i32 [M, H*D/32]; D in {64, 128, 256},
 * nch <= 8192, pos + M - 1 < 32 nch; xq 16-byte aligned.
 * params (device memory, nullable): when set, the position is read at run
 * time from params->pos, as the reference counts its chunks from p.pos
 * (attn_combine.wgsl:24,35), and the host `pos` is the largest position the
 * call may see: a device value above it is clamped to it, so no chunk past
 * nch is read.
 */
int wq_attn_combine(void* stream, const float* part, int64_t M, int64_t H, int64_t D,
                    int64_t nch, int64_t pos, const float* gate, int64_t gate_stride,
                    int8_t* xq, float* dx, int32_t* xs, const wq_params* params);

/*
 * Test hooks: wq_gemv / wq_gemm that also store the exact int32 group sums
 * A[t, row, e] = sum over group e of q[row, k] * xq[t, k] that the kernel
 * folded into y, into acc i32 [M, rows, K/Ge] (rows = N, or 2N in
 * WQ_MODE_SILU_MUL).  The reference exposes no such dump; its group sums are
 * internal to gemv_q4q8.wgsl:68 / gemm_q4q8.wgsl:96.
 */
int wq_gemv_debug_acc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N,
                      int64_t K, int32_t G, const int8_t* xq, const float* dx,
                      const int32_t* xs, int64_t M, int32_t GA, int32_t mode, float* y,
                      int32_t* acc);
int wq_gemm_debug_acc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N,
                      int64_t K, int32_t G, const int8_t* xq, const float* dx,
                      const int32_t* xs, int64_t M, int32_t GA, int32_t mode, float* y,
                      int32_t* acc);

#ifdef __cplusplus
}
#endif

#endif /* WEBYIQ_Q4Q8_H */
