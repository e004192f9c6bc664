// Internal launcher interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Arguments are already validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wq {

struct QuantArgs {
    const float* x;
    const float* norm_w;  // nullable: RMSNorm prologue when set
    float eps;
    int64_t M, K;
    int GA, G;  // GA: K (per token) or 32; xs group Ge = min(G, GA)
    int8_t* xq;
    float* dx;
    int32_t* xs;
};

struct LinearArgs {
    const uint32_t* wq;  // [rows, K/8], rows = N (2N for mode 2)
    const uint32_t* ws;  // [rows, K/G]
    int64_t N, K;
    int G;
    const int8_t* xq;  // [M, K]
    const float* dx;   // [M, K/GA]
    const int32_t* xs; // [M, K/Ge]
    int64_t M;
    int GA;
    int mode;
    float* y;            // [M, N]; nullable only for the lm_head argmax path
    int32_t* acc_dump;   // nullable: [M, rows, K/Ge] int32 group accumulators
    // nullable (the GEMM only): device wq_params {pos, seq_len, m, slot}; when
    // set, M is the capacity and the kernel covers min(m, M) tokens
    const uint32_t* params;
    // nullable (the GEMM only): caller workspace of a K-split launch (ready
    // flags, zero between calls, and partial sums)
    void* workspace;
    size_t workspace_bytes;
};
// word index of wq_params fields
constexpr int kParamPos = 0;
constexpr int kParamM = 2;

struct ArgmaxArgs {
    const uint32_t* ids;  // nullable id map (draft vocabulary)
    uint32_t* tok_out;    // [M]
    unsigned long long* keys;  // workspace: [kArgmaxSlots][8] running (value, index) keys
    unsigned int* ticket;      // workspace: [kArgmaxSlots] slot ticket counters (+ a spare line), one line each
};

// Input of a GEMV that quantises its own activations (per token).
struct QuantInArgs {
    const float* x;       // [M, K] f32
    const float* norm_w;  // nullable: RMSNorm prologue when set
    float eps;
    int8_t* xq;           // nullable outputs: the quantised activations
    float* dx;            //   (xq [M, K], dx [M], xs [M, K/G])
    int32_t* xs;
};

// MTP input stage: per token m, row 2m = per-32 quant of norm_e(emb[m]) and
// row 2m + 1 = per-32 quant of norm_h(norm_f(x[m])), each norm v * (r * w).
struct MtpInArgs {
    const float* emb;     // [M, K]
    const float* x;       // [M, K]
    const float* norm_f;  // [K] final norm
    const float* norm_e;  // [K]
    const float* norm_h;  // [K]
    float eps;
    int64_t M, K;
    int8_t* xq;           // [M, 2K]
    float* dx;            // [M, 2K/32]
    int32_t* xs;          // [M, 2K/32]
};

// Flash-decoding merge of per-chunk attention partials, emitted as per-32
// int8 groups for the o projection (nch <= kCombineMaxChunks: the chunk
// weights and three partial chains fit 64 KiB of LDS).
constexpr int kCombineMaxChunks = 8192;
struct AttnCombineArgs {
    const float* part;    // [M, H, nch, D + 2]: chunk output sums, chunk max, chunk sum
    int64_t M, H, D, nch;
    int64_t pos;          // position of token 0; token m covers positions 0 ..= pos + m
                          // (with params: the largest position the call may see)
    const uint32_t* params;  // nullable: device wq_params, pos read from it at run time
    const float* gate;    // nullable: gate of (m, h, i) at gate[m * gate_stride + h * 2D + D + i]
    int64_t gate_stride;
    int8_t* xq;           // [M, H * D]
    float* dx;            // [M, H * D / 32]
    int32_t* xs;          // [M, H * D / 32]
};

struct EmbedArgs {
    const uint32_t* q;    // [V, K/8] packed int4 rows
    const uint32_t* s;    // [V, K/G] (scale, min) words
    int64_t V, K;
    int G;
    const uint32_t* ids;  // [M] token ids
    int64_t M;
    float* x;             // [M, K]
};

struct GatherArgs {
    const uint32_t* q;    // source [V, K/8]
    const uint32_t* s;    // source [V, K/G]
    int64_t V, K;
    int G;
    const uint32_t* ids;  // [R] source rows
    int64_t R;
    uint32_t* dq;         // [R, K/8]
    uint32_t* ds;         // [R, K/G]
};

hipError_t launch_quant_act(const QuantArgs& a, hipStream_t s);
hipError_t launch_mtp_in(const MtpInArgs& a, hipStream_t s);
hipError_t launch_attn_combine(const AttnCombineArgs& a, hipStream_t s);
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);
hipError_t launch_gather_rows(const GatherArgs& a, hipStream_t s);
hipError_t launch_gemv(const LinearArgs& a, hipStream_t s);
// 3..8 tokens, per-token activations, group 128, K <= 8192: the int8-MFMA
// GEMV (am != nullptr: with the fused argmax)
bool gemv_mfma_fits(const LinearArgs& a);
hipError_t launch_gemv_mfma(const LinearArgs& a, const ArgmaxArgs* am, hipStream_t s);
hipError_t launch_gemv_quant_in(const LinearArgs& a, const QuantInArgs& q, hipStream_t s);
hipError_t launch_lm_head_argmax(const LinearArgs& a, const ArgmaxArgs& am, hipStream_t s);
hipError_t launch_gemm(const LinearArgs& a, hipStream_t s);
// Bytes of workspace the GEMM's K-split plan needs for this shape (0: the
// shape never splits).
size_t gemm_workspace_bytes(const LinearArgs& a);
hipError_t launch_argmax(const float* logits, int64_t M, int64_t V, const uint32_t* ids,
                         uint32_t* tok_out, hipStream_t s);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s);

// Decode GEMV: rows of one pass = 1 KiB of packed weights = 2048 codes.
constexpr int kGemvPassK = 2048;
// Largest token count of the decode GEMV (the M <= 8 speculative-verify case).
constexpr int kGemvMaxTokens = 8;
// Workspace of the fused lm_head argmax: kArgmaxSlots cache lines of 8 keys,
// then kArgmaxSlots lines holding one ticket counter each and a spare line.
constexpr int kArgmaxSlots = 64;
constexpr int kArgmaxSlotWords = 8;  // 64-bit words per 64-byte line
constexpr size_t kArgmaxKeyBytes = (size_t)kArgmaxSlots * kArgmaxSlotWords * 8;
constexpr size_t kArgmaxWorkspaceBytes = kArgmaxKeyBytes + (size_t)(kArgmaxSlots + 1) * 64;

}  // namespace wq
