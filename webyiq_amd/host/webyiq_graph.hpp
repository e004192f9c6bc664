// C++ host side of the int4 x int8 path: webyIQ's operator layer restated
// above the C ABI (include/webyiq_q4q8.h) for hosts without the engine's
// Rust toolchain.
//
//   Builder       crates/engine/src/graph.rs:117-222 (gemv, gemm, matmul by
//                 Path, quant, the weight lookup `w`), plus head_ops
//                 (graph.rs:476-486) and the fused quant -> matmul pair
//   OpDef         graph.rs:66-71: a recorded dispatch -- here the C-ABI call
//                 with its arguments bound, replayed on a HIP stream
//   Path          graph.rs:127-146 (Decode: 1 token, Spec: 2, Prefill: 128)
//   encode        Engine::encode (lib.rs:222-228): the ops in order
//
// Errors follow the engine's Result<_, String>: a build-time check fails
// with the message the engine would give (a missing tensor is
// "missing tensor {name}") and launches nothing; a launch error carries the
// op's name and the library's wq_last_error() text.  Buffers are device
// memory owned by the caller; their byte sizes are checked against the
// shapes at build time, as wgpu checks binding sizes.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace webyiq {

// Result<T, String>
template <class T>
class Result {
  public:
    static Result ok(T v) { return Result(std::move(v), std::string(), true); }
    static Result err(std::string e) { return Result(T(), std::move(e), false); }
    bool is_ok() const { return ok_; }
    const T& value() const { return v_; }
    T& value() { return v_; }
    const std::string& error() const { return e_; }

  private:
    Result(T v, std::string e, bool ok) : v_(std::move(v)), e_(std::move(e)), ok_(ok) {}
    T v_;
    std::string e_;
    bool ok_;
};

struct Unit {};

// A device buffer: pointer and size in bytes (caller-owned).
struct Buffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// Which dispatch list a product belongs to (graph.rs:127-146).
enum class Path { Decode, Spec, Prefill };
constexpr uint32_t kSpecTokens = 2;      // graph.rs:11 SPEC_TOKENS
constexpr uint32_t kPrefillChunk = 128;  // graph.rs:10 PREFILL_CHUNK
uint32_t tokens(Path p);

// The int8 activations of a path: the reference's (xq, xs) pair, with xs
// split into the f32 scales dx [t, K/ga] and the i32 group sums xs
// [t, K/min(G, ga)].  ga = 0 means per token (ga = K).
struct Acts {
    Buffer xq, dx, xs;
    uint32_t ga = 0;
};

// The step an op list is replayed for (Engine::resolve, lib.rs:207-214):
// seq_len positions in all, m tokens.  0 means "as built": an op then runs
// the token count it was built with.  Ops whose token count follows the step
// (the reference's Dims::Tokens / GemmTiles: quant, gemm, attn_combine) run
// min(m, built count) tokens; GEMV ops keep their path's count, as the
// reference's gemv bakes T into the pipeline.
struct Step {
    uint32_t seq_len = 0;
    uint32_t m = 0;
};

// One recorded dispatch (graph.rs:66-71): the C-ABI call with its arguments
// bound, resolved against the step when replayed.
struct OpDef {
    std::string name;
    std::function<int(void* stream, Step step)> launch;  // returns the C ABI's status
};

class Builder {
  public:
    // weights: the engine's name -> buffer map (graph.rs:119), int4 tensors as
    // "{w}.q" / "{w}.s" pairs (copied: the builder keeps its own map of the
    // caller's device pointers); group: the manifest's quant.group
    Builder(std::unordered_map<std::string, Buffer> weights, int32_t group);

    // graph.rs:186-188
    Result<Buffer> w(const std::string& name) const;

    // y (+)= W x for t tokens (graph.rs:190-198); mode 0 store, 1 accumulate,
    // 2 silu(gate) * up over the 2n rows of w
    Result<OpDef> gemv(const std::string& name, const std::string& w, uint32_t k, uint32_t n, uint32_t mode,
                       uint32_t t, const Acts& a, Buffer y);
    // the prefill product over up to m tokens (graph.rs:200-205); params
    // (optional): the step's Params buffer (wq_params, 16 bytes of device
    // memory) the kernel reads when it runs, so the tokens it covers follow
    // the buffer's m (at most m, the capacity the buffers hold); workspace
    // (optional, zeroed once): wq_gemm_workspace_bytes for the shape, so that
    // the library may split K between workgroup pairs
    Result<OpDef> gemm(const std::string& name, const std::string& w, uint32_t k, uint32_t n, uint32_t mode,
                       uint32_t m, const Acts& a, Buffer y, const Buffer* params = nullptr,
                       const Buffer* workspace = nullptr);
    // GEMM for Prefill, GEMV otherwise (graph.rs:207-214); m: the prefill
    // tokens (the other paths take theirs from the path); params as gemm's
    Result<OpDef> matmul(Path path, const std::string& name, const std::string& w, uint32_t k, uint32_t n,
                         uint32_t mode, const Acts& a, Buffer y, uint32_t m = kPrefillChunk,
                         const Buffer* params = nullptr);
    // int8 quantisation of t rows of x (k wide), optionally RMSNorm'ed with
    // norm (graph.rs:216-222); writes a's three buffers
    Result<OpDef> quant(const std::string& name, uint32_t k, double eps, Buffer x, const Buffer* norm, uint32_t t,
                        const Acts& a);
    // a quant -> decode matmul pair in one call (one launch for t <= 2)
    Result<OpDef> quant_gemv(const std::string& name, const std::string& w, uint32_t k, uint32_t n, uint32_t mode,
                             uint32_t t, double eps, Buffer x, const Buffer* norm, const Acts& a, Buffer y);
    // norm + lm_head + greedy argmax of t rows of x into tok (graph.rs:476-486),
    // fused into one launch after the quantiser; ids maps rows to tokens
    // (the draft head), logits (optional) receives the t x v logits;
    // workspace: wq_lm_head_workspace_bytes() bytes, zeroed once
    Result<std::vector<OpDef>> head_ops(const std::string& head, uint32_t k, uint32_t v, uint32_t t, double eps,
                                        Buffer x, Buffer norm, const Acts& a, const Buffer* ids, Buffer tok,
                                        Buffer workspace, const Buffer* logits = nullptr);

    // the other ops around the path (the survey's next rows):
    // int4 embedding lookup of t token ids into x [t, k] (graph.rs:439-443);
    // ids outside [0, v) give zero rows
    Result<OpDef> embed(const std::string& name, const std::string& table, uint32_t k, uint32_t v, uint32_t t,
                        Buffer tok, Buffer x);
    // the draft head's packed rows: dst row r = row ids[r] of table
    // (graph.rs:511-516); dq / ds hold r rows of the packed format
    Result<OpDef> gather_rows(const std::string& name, const std::string& table, uint32_t k, uint32_t v,
                              uint32_t r, Buffer ids, Buffer dq, Buffer ds);
    // flash-decoding chunk merge of t tokens x h heads of d dims over nch
    // chunks, positions up to pos + t - 1, optional output gate rows, into
    // per-32 int8 activations of k = h d (graph.rs:289-291); a.ga must be 32.
    // params (optional): the Params buffer; the position is then read from
    // it when the kernel runs (attn_combine.wgsl:35) and pos is its bound
    Result<OpDef> attn_combine(const std::string& name, Buffer part, uint32_t t, uint32_t h, uint32_t d,
                               uint32_t nch, int64_t pos, const Buffer* gate, int64_t gate_stride, const Acts& a,
                               const Buffer* params = nullptr);
    // MTP input stage: per-32 int8 activations [t, 2k] of the normed
    // embedding and hidden state (graph.rs:500-504); a.ga must be 32
    Result<OpDef> mtp_in(const std::string& name, uint32_t k, double eps, Buffer emb, Buffer x, Buffer norm_f,
                         Buffer norm_e, Buffer norm_h, uint32_t t, const Acts& a);

  private:
    struct Q4 {
        Buffer q, s;
    };
    Result<Q4> q4(const std::string& w, uint32_t rows, uint32_t k) const;
    std::string check_acts(const std::string& name, uint32_t k, uint32_t t, const Acts& a) const;

    std::unordered_map<std::string, Buffer> weights_;
    int32_t group_;
};

// Engine::encode (lib.rs:222-228) over Engine::resolve (lib.rs:207-214):
// launch the ops in order on stream for `step`; the first failing op ends
// the replay with "{op}: {message}".
Result<Unit> encode(const std::vector<OpDef>& ops, void* stream, Step step = Step{});

}  // namespace webyiq
