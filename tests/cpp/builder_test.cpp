// Tests of the C++ host side (webyiq_amd/host/webyiq_graph.hpp).
//
//   builder_test --cpu   build-time checks and error propagation; launches
//                        nothing (every op that reaches the C ABI is one its
//                        validation rejects)
//   builder_test --gpu   an MLP block and the greedy head built with Builder
//                        and replayed by encode on the GPU, on the Decode,
//                        Spec and Prefill paths, compared bit for bit with
//                        the CPU oracle (oracle/q4q8_oracle.h)
//
// Prints "builder_test <mode> ok" and exits 0 when every check passes.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/webyiq_q4q8.h"
#include "../../oracle/q4q8_oracle.h"
#include "../../webyiq_amd/host/webyiq_graph.hpp"

using namespace webyiq;

static int g_failures = 0;

#define CHECK(cond, ...)                                     \
    do {                                                     \
        if (!(cond)) {                                       \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                        \
            std::printf("\n");                               \
            ++g_failures;                                    \
        }                                                    \
    } while (0)

template <class T>
static void expect_err(const Result<T>& r, const std::string& want, const char* what) {
    CHECK(!r.is_ok(), "%s: expected an error containing '%s'", what, want.c_str());
    if (!r.is_ok())
        CHECK(r.error().find(want) != std::string::npos, "%s: error '%s' lacks '%s'", what, r.error().c_str(),
              want.c_str());
}

// ---------------------------------------------------------------- CPU mode

static Buffer fake(uintptr_t addr, size_t bytes) { return Buffer{reinterpret_cast<void*>(addr), bytes}; }

static void cpu_checks() {
    const uint32_t K = 256, N = 128, G = 128;
    std::unordered_map<std::string, Buffer> wts;
    wts["mlp.up.q"] = fake(0x10000, N * K / 2);
    wts["mlp.up.s"] = fake(0x20000, N * (K / G) * 4);
    wts["short.q"] = fake(0x30000, N * K / 2 - 4);
    wts["short.s"] = fake(0x40000, N * (K / G) * 4);
    wts["head.q"] = fake(0x50000, 1024 * K / 2);
    wts["head.s"] = fake(0x60000, 1024 * (K / G) * 4);
    Builder b(wts, G);

    Acts a;
    a.xq = fake(0x70000, 8 * K);
    a.dx = fake(0x71000, 8 * 4);
    a.xs = fake(0x72000, 8 * (K / G) * 4);
    const Buffer y = fake(0x80000, 8 * N * 4);

    // weight lookup (graph.rs:186-188)
    expect_err(b.w("nope"), "missing tensor nope", "w()");
    CHECK(b.w("mlp.up.q").is_ok() && b.w("mlp.up.q").value().ptr == wts["mlp.up.q"].ptr, "w() lookup");
    expect_err(b.gemv("up", "mlp.gate", K, N, 0, 1, a, y), "missing tensor mlp.gate.q", "gemv missing weight");

    // shapes
    expect_err(b.gemv("up", "mlp.up", 200, N, 0, 1, a, y), "up: K = 200", "K % 128");
    expect_err(b.gemv("up", "mlp.up", K, N, 3, 1, a, y), "unknown mode 3", "mode");
    expect_err(b.gemv("up", "mlp.up", K, N, 0, 9, a, y), "9 tokens", "t > 8");
    expect_err(b.gemv("up", "mlp.up", K, N, 2, 1, a, y), "mlp.up: the .q tensor holds", "mode 2 needs 2N rows");
    expect_err(b.gemv("up", "short", K, N, 0, 1, a, y), "the .q tensor holds 16380 bytes, the shape needs 16384",
               "short weight");
    expect_err(b.gemv("up", "mlp.up", K, N, 0, 8, a, fake(0x80000, 8 * N * 4 - 1)), "y holds", "short output");
    Acts noxs = a;
    noxs.xs = Buffer{};
    expect_err(b.gemv("up", "mlp.up", K, N, 0, 1, noxs, y), "xs is not bound", "unbound xs");
    Acts per32 = a;
    per32.ga = 32;
    expect_err(b.gemv("up", "mlp.up", K, N, 0, 2, per32, y), "dx holds 32 bytes, the shape needs 64",
               "per-32 scales need K/32 floats a token");
    Acts ga64 = a;
    ga64.ga = 64;
    expect_err(b.gemv("up", "mlp.up", K, N, 0, 1, ga64, y), "activation group 64", "GA");
    Builder b48(wts, 48);
    expect_err(b48.gemv("up", "mlp.up", K, N, 0, 1, a, y), "up: quant group 48", "G");
    expect_err(b48.quant("q", K, 1e-6, fake(0x90000, K * 4), nullptr, 1, a), "q: quant group 48", "G in quant");
    // the builder owns its map: one built from a temporary stays valid
    Builder bt({{"t.q", fake(0x10000, N * K / 2)}, {"t.s", fake(0x20000, N * (K / G) * 4)}}, G);
    CHECK(bt.gemv("t", "t", K, N, 0, 1, a, y).is_ok(), "builder over a temporary map");

    // matmul dispatch by path (graph.rs:207-214): Decode/Spec -> GEMV with the
    // path's tokens, Prefill -> GEMM over m tokens
    CHECK(tokens(Path::Decode) == 1 && tokens(Path::Spec) == 2 && tokens(Path::Prefill) == 128, "tokens()");
    CHECK(b.matmul(Path::Spec, "up", "mlp.up", K, N, 0, a, y).is_ok(), "Spec matmul builds");
    expect_err(b.matmul(Path::Prefill, "up", "mlp.up", K, N, 0, a, y), "xq holds 2048 bytes, the shape needs 32768",
               "Prefill matmul sizes the 128-token chunk");
    CHECK(b.matmul(Path::Prefill, "up", "mlp.up", K, N, 0, a, y, 8).is_ok(), "Prefill matmul with m = 8");

    // quant / quant_gemv / head_ops
    const Buffer x = fake(0x90000, 8 * K * 4), nw = fake(0xA0000, K * 4);
    expect_err(b.quant("q", K, 1e-6, fake(0x90000, K * 4 - 4), &nw, 1, a), "x holds", "short x");
    const Buffer short_nw = fake(0xA0000, K * 4 - 4);
    expect_err(b.quant("q", K, 1e-6, x, &short_nw, 1, a), "the norm weight holds", "short norm");
    expect_err(b.quant_gemv("qg", "mlp.up", K, N, 0, 1, 1e-6, x, &nw, per32, y), "per-token", "fused per-32");
    const Buffer tok = fake(0xB0000, 32), wsp = fake(0xC0000, wq_lm_head_workspace_bytes());
    auto h = b.head_ops("head", K, 1024, 2, 1e-6, x, nw, a, nullptr, tok, wsp);
    CHECK(h.is_ok() && h.value().size() == 2 && h.value()[0].name == "norm_quant" && h.value()[1].name == "lm_head",
          "head_ops = norm_quant + lm_head");
    expect_err(b.head_ops("head", K, 1024, 2, 1e-6, x, nw, a, nullptr, tok, fake(0xC0000, 16)),
               "lm_head: the workspace holds 16 bytes", "small workspace");
    expect_err(b.head_ops("lm", K, 1024, 2, 1e-6, x, nw, a, nullptr, tok, wsp), "missing tensor lm.q",
               "missing head");

    // encode: the first op the C ABI rejects ends the replay with its name
    // and wq_last_error(); ops after it are not launched.  A weight
    // pointer off the ABI's alignment passes the builder's size checks and
    // fails the library's validation before any HIP call.
    std::unordered_map<std::string, Buffer> odd = wts;
    odd["mlp.up.q"] = fake(0x10002, N * K / 2);
    Builder bo(odd, G);
    auto op = bo.gemv("up_proj", "mlp.up", K, N, 0, 1, a, y);
    CHECK(op.is_ok(), "misaligned op still builds");
    int later = 0;
    std::vector<OpDef> ops{op.value(), OpDef{"after", [&](void*, Step) { ++later; return WQ_OK; }}};
    auto r = encode(ops, nullptr);
    CHECK(!r.is_ok(), "encode reports the rejected op");
    if (!r.is_ok())
        CHECK(r.error().rfind("up_proj: wq_gemv: wq", 0) == 0 && r.error().find("aligned") != std::string::npos,
              "encode error '%s'", r.error().c_str());
    CHECK(later == 0, "ops after a failure are not launched");
    // the ops around the path
    expect_err(b.embed("embed", "emb", K, 1024, 2, tok, x), "missing tensor emb.q", "embed table");
    expect_err(b.embed("embed", "head", K, 1024, 2, tok, fake(0x90000, 2 * K * 4 - 4)), "embed: x holds", "embed x");
    CHECK(b.embed("embed", "head", K, 1024, 2, tok, x).is_ok(), "embed builds");
    expect_err(b.gather_rows("gather", "head", K, 1024, 8, tok, fake(0xD0000, 8 * K / 2 - 16), wsp),
               "gather: dq holds", "gather dq");
    Acts p32 = a;
    p32.ga = 32;
    p32.dx = fake(0x71000, 8 * (K / 32) * 4);
    p32.xs = fake(0x72000, 8 * (K / 32) * 4);
    const Buffer part = fake(0xE0000, (size_t)2 * 2 * 4 * (128 + 2) * 4);
    CHECK(b.attn_combine("combine", part, 2, 2, 128, 4, 100, nullptr, 0, p32).is_ok(), "combine builds");
    expect_err(b.attn_combine("combine", part, 2, 2, 96, 4, 100, nullptr, 0, p32), "head dim 96", "combine D");
    expect_err(b.attn_combine("combine", part, 2, 2, 128, 4, 127, nullptr, 0, p32), "positions 0..128", "combine pos");
    expect_err(b.attn_combine("combine", part, 2, 2, 128, 4, 100, nullptr, 0, a), "per-32", "combine ga");
    expect_err(b.attn_combine("combine", part, 2, 2, 128, 5, 100, nullptr, 0, p32), "combine: part holds", "part");
    expect_err(b.attn_combine("combine", part, 2, 2, 128, 4, 100, &x, 511, p32), "gate_stride 511", "gate stride");
    const Buffer half = fake(0xA0000, K / 2 * 4);
    CHECK(b.mtp_in("mtp_in", K / 2, 1e-6, x, x, half, half, half, 2, p32).is_ok(), "mtp_in builds");
    expect_err(b.mtp_in("mtp_in", K / 2, 1e-6, x, x, half, half, half, 2, a), "per-32", "mtp_in ga");
    expect_err(b.mtp_in("mtp_in", K / 2, 1e-6, x, x, half, half, fake(0xA0000, 8), 2, p32), "norm_h holds", "norm_h");

    std::vector<OpDef> fine{OpDef{"a", [&](void*, Step) { ++later; return WQ_OK; }},
                            OpDef{"b", [&](void*, Step) { ++later; return WQ_OK; }}};
    CHECK(encode(fine, nullptr).is_ok() && later == 2, "encode runs every op in order");
    // encode hands every op the step it replays (Engine::resolve's seq_len, m)
    uint32_t seen_m = 0, seen_len = 0;
    std::vector<OpDef> stepped{OpDef{"s", [&](void*, Step st) {
        seen_m = st.m;
        seen_len = st.seq_len;
        return WQ_OK;
    }}};
    CHECK(encode(stepped, nullptr, Step{300, 77}).is_ok() && seen_m == 77 && seen_len == 300,
          "encode passes the step to its ops");
    // the Params buffer is 16 bytes of device memory
    const Buffer small_params = fake(0xF0000, 8);
    expect_err(b.gemm("gemm", "mlp.up", K, N, 0, 8, a, y, &small_params), "gemm: params holds 8 bytes",
               "params size");
    expect_err(b.attn_combine("combine", part, 2, 2, 128, 4, 100, nullptr, 0, p32, &small_params),
               "combine: params holds 8 bytes", "combine params size");
}

// ---------------------------------------------------------------- GPU mode

#define HIP_OK(x)                                                                          \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                                  \
        }                                                                                  \
    } while (0)

struct Dev {
    std::vector<void*> held;
    ~Dev() {
        for (void* p : held) (void)hipFree(p);
    }
    template <class T>
    Buffer put(const std::vector<T>& h) {
        void* p = nullptr;
        HIP_OK(hipMalloc(&p, h.size() * sizeof(T)));
        HIP_OK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
        held.push_back(p);
        return Buffer{p, h.size() * sizeof(T)};
    }
    Buffer zeros(size_t bytes) {
        void* p = nullptr;
        HIP_OK(hipMalloc(&p, bytes));
        HIP_OK(hipMemset(p, 0, bytes));
        held.push_back(p);
        return Buffer{p, bytes};
    }
};

template <class T>
static std::vector<T> get(Buffer b, size_t n) {
    std::vector<T> h(n);
    HIP_OK(hipMemcpy(h.data(), b.ptr, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

template <class T>
static bool same_bits(const std::vector<T>& a, const std::vector<T>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(T)) == 0;
}

// max |a - b| / max |b|
static double rel_err(const std::vector<float>& a, const std::vector<float>& b) {
    double num = 0.0, den = 1e-30;
    for (size_t i = 0; i < a.size(); ++i) {
        num = std::fmax(num, std::fabs((double)a[i] - (double)b[i]));
        den = std::fmax(den, std::fabs((double)b[i]));
    }
    return num / den;
}

struct Q4Host {
    std::vector<uint32_t> q, s;
};

static Q4Host make_weight(std::mt19937& rng, uint32_t rows, uint32_t k, int g) {
    std::normal_distribution<float> nd(0.0f, 0.02f);
    std::vector<float> w((size_t)rows * k);
    for (float& v : w) v = nd(rng);
    Q4Host out{std::vector<uint32_t>((size_t)rows * k / 8), std::vector<uint32_t>((size_t)rows * (k / g))};
    or_q4_quantize(w.data(), rows, k, g, out.q.data(), out.s.data(), nullptr);
    return out;
}

// One decode-style step on path p with t tokens: the MLP block
// (norm -> quant -> gate_up silu*up, quant -> down accumulated into the
// residual) then norm_quant -> lm_head -> argmax, built with Builder and
// checked against the oracle's chain of the same calls.  The silu * up
// epilogue calls the device's expf, which may differ from the host's in the
// last bit, so h is compared within rel 1e-5 (norm-wise) and the oracle
// continues from the device's h.  The Prefill GEMM's residual is within
// rel 1e-5 too (see below); every other value is compared bit for bit.
static void gpu_step(Path p, uint32_t t) {
    const uint32_t H = 1024, I = 2048, V = 4096;
    const int G = 128;
    const double eps = 1e-6;
    std::mt19937 rng(1234 + t);
    Q4Host gu = make_weight(rng, 2 * I, H, G), dn = make_weight(rng, H, I, G), hd = make_weight(rng, V, H, G);
    std::normal_distribution<float> nd(0.0f, 1.0f), nn(1.0f, 0.1f);
    std::vector<float> x((size_t)t * H), n1(H), n2(H);
    for (float& v : x) v = nd(rng);
    for (float& v : n1) v = nn(rng);
    for (float& v : n2) v = nn(rng);

    Dev d;
    std::unordered_map<std::string, Buffer> wts{{"mlp.gate_up.q", d.put(gu.q)}, {"mlp.gate_up.s", d.put(gu.s)},
                                                {"mlp.down.q", d.put(dn.q)},    {"mlp.down.s", d.put(dn.s)},
                                                {"lm_head.q", d.put(hd.q)},     {"lm_head.s", d.put(hd.s)}};
    Builder b(wts, G);
    const Buffer xr = d.put(x), bn1 = d.put(n1), bn2 = d.put(n2);
    auto acts = [&](uint32_t k) {
        Acts a;
        a.xq = d.zeros((size_t)t * k);
        a.dx = d.zeros((size_t)t * 4);
        a.xs = d.zeros((size_t)t * (k / G) * 4);
        return a;
    };
    const Acts a1 = acts(H), a2 = acts(I), a3 = acts(H);
    const Buffer hbuf = d.zeros((size_t)t * I * 4), tok = d.zeros((size_t)t * 4),
                 wsp = d.zeros(wq_lm_head_workspace_bytes());

    std::vector<OpDef> ops;
    auto add = [&](Result<OpDef> r) {
        CHECK(r.is_ok(), "build: %s", r.error().c_str());
        if (r.is_ok()) ops.push_back(r.value());
    };
    if (p == Path::Prefill) {
        add(b.quant("mlp_quant", H, eps, xr, &bn1, t, a1));
        add(b.matmul(p, "gate_up", "mlp.gate_up", H, I, WQ_MODE_SILU_MUL, a1, hbuf, t));
    } else {
        add(b.quant_gemv("gate_up", "mlp.gate_up", H, I, WQ_MODE_SILU_MUL, t, eps, xr, &bn1, a1, hbuf));
    }
    add(b.quant("down_quant", I, eps, hbuf, nullptr, t, a2));
    add(b.matmul(p, "down", "mlp.down", I, H, WQ_MODE_ACCUMULATE, a2, xr, t));
    const bool head = t <= 8;
    if (head) {
        auto hops = b.head_ops("lm_head", H, V, t, eps, xr, bn2, a3, nullptr, tok, wsp);
        CHECK(hops.is_ok(), "head_ops: %s", hops.error().c_str());
        if (hops.is_ok()) ops.insert(ops.end(), hops.value().begin(), hops.value().end());
    }
    auto r = encode(ops, nullptr);
    CHECK(r.is_ok(), "encode: %s", r.error().c_str());
    HIP_OK(hipDeviceSynchronize());

    // oracle
    std::vector<int8_t> q1((size_t)t * H), q2((size_t)t * I), q3((size_t)t * H);
    std::vector<float> d1(t), d2(t), d3(t), h((size_t)t * I), xo = x, logits((size_t)t * V);
    std::vector<int32_t> s1((size_t)t * (H / G)), s2((size_t)t * (I / G)), s3((size_t)t * (H / G));
    or_quant_act(x.data(), n1.data(), (float)eps, t, H, (int)H, G, q1.data(), d1.data(), s1.data());
    or_linear(gu.q.data(), gu.s.data(), I, H, G, q1.data(), d1.data(), s1.data(), t, (int)H, 2, h.data());
    const std::vector<float> hg = get<float>(hbuf, h.size());
    or_quant_act(hg.data(), nullptr, (float)eps, t, I, (int)I, G, q2.data(), d2.data(), s2.data());
    or_linear(dn.q.data(), dn.s.data(), H, I, G, q2.data(), d2.data(), s2.data(), t, (int)I, 1, xo.data());

    const char* pn = p == Path::Decode ? "Decode" : p == Path::Spec ? "Spec" : "Prefill";
    CHECK(same_bits(get<int8_t>(a1.xq, q1.size()), q1), "%s t=%u: norm+quant codes", pn, t);
    CHECK(rel_err(hg, h) < 1e-5, "%s t=%u: gate_up silu*up rel err %.3g", pn, t, rel_err(hg, h));
    CHECK(same_bits(get<int8_t>(a2.xq, q2.size()), q2), "%s t=%u: down_quant codes", pn, t);
    const std::vector<float> xg = get<float>(xr, xo.size());
    if (p == Path::Prefill) {
        // the GEMM's per-token G = 128 epilogue folds the min term on an f16
        // MFMA: rel 1e-5 (its int32 group sums are exact)
        const double e = rel_err(xg, xo);
        CHECK(e < 1e-5, "%s t=%u: residual += down rel err %.3g", pn, t, e);
    } else {
        CHECK(same_bits(xg, xo), "%s t=%u: residual += down", pn, t);
    }
    if (head) {
        std::vector<uint32_t> want(t);
        or_quant_act(xo.data(), n2.data(), (float)eps, t, H, (int)H, G, q3.data(), d3.data(), s3.data());
        or_linear(hd.q.data(), hd.s.data(), V, H, G, q3.data(), d3.data(), s3.data(), t, (int)H, 0, logits.data());
        or_argmax(logits.data(), t, V, nullptr, want.data());
        const std::vector<uint32_t> got = get<uint32_t>(tok, t);
        CHECK(same_bits(got, want), "%s t=%u: greedy tokens (first %u vs %u)", pn, t, got[0], want[0]);
    }
    std::printf("  %s t=%u: %zu ops replayed, compared with the oracle\n", pn, t, ops.size());
    std::fflush(stdout);
}

// embed, the chunk merge feeding a per-32 GEMV, and the MTP input stage,
// built with Builder and compared bit for bit with the oracle (the merge with
// equal chunk maxima, where every chunk weight is exp(0) exactly)
static void gpu_producers() {
    const uint32_t K = 1024, V = 4096, N = 256, H = 4, D = 128, NCH = 8, T = 2;
    const int G = 128;
    const int64_t POS = 100;
    std::mt19937 rng(77);
    Q4Host tab = make_weight(rng, V, K, G), wo = make_weight(rng, N, H * D, G);
    Dev d;
    Builder b({{"embed.q", d.put(tab.q)}, {"embed.s", d.put(tab.s)}, {"o.q", d.put(wo.q)}, {"o.s", d.put(wo.s)}}, G);
    auto acts32 = [&](uint32_t k) {
        Acts a;
        a.xq = d.zeros((size_t)T * k);
        a.dx = d.zeros((size_t)T * (k / 32) * 4);
        a.xs = d.zeros((size_t)T * (k / 32) * 4);
        a.ga = 32;
        return a;
    };
    // embed
    const std::vector<uint32_t> tok{7, V + 3};
    const Buffer dtok = d.put(tok), x = d.zeros((size_t)T * K * 4);
    // chunk partials [T, H, NCH, D + 2]: NaN past each token's chunks
    std::normal_distribution<float> nd(0.0f, 3.0f);
    std::uniform_real_distribution<float> ud(1.0f, 32.0f);
    std::vector<float> part((size_t)T * H * NCH * (D + 2), std::nanf(""));
    for (uint32_t m = 0; m < T; ++m)
        for (uint32_t h = 0; h < H; ++h)
            for (uint32_t c = 0; c < (POS + m + 32) / 32; ++c) {
                float* p = &part[(((size_t)m * H + h) * NCH + c) * (D + 2)];
                for (uint32_t i = 0; i < D; ++i) p[i] = nd(rng);
                p[D] = 0.75f;
                p[D + 1] = ud(rng);
            }
    const Acts ao = acts32(H * D);
    const Buffer y = d.zeros((size_t)T * N * 4);
    // MTP input
    std::normal_distribution<float> n1(0.0f, 1.0f), nw(1.0f, 0.1f);
    std::vector<float> emb((size_t)T * K), hid((size_t)T * K), nf(K), ne(K), nh(K);
    for (float& v : emb) v = n1(rng);
    for (float& v : hid) v = n1(rng);
    for (auto* w : {&nf, &ne, &nh})
        for (float& v : *w) v = nw(rng);
    const Acts am = acts32(2 * K);

    std::vector<OpDef> ops;
    auto add = [&](Result<OpDef> r) {
        CHECK(r.is_ok(), "build: %s", r.error().c_str());
        if (r.is_ok()) ops.push_back(r.value());
    };
    add(b.embed("embed", "embed", K, V, T, dtok, x));
    add(b.attn_combine("attn_combine", d.put(part), T, H, D, NCH, POS, nullptr, 0, ao));
    add(b.gemv("o_proj", "o", H * D, N, WQ_MODE_STORE, T, ao, y));
    add(b.mtp_in("mtp_in", K, 1e-6, d.put(emb), d.put(hid), d.put(nf), d.put(ne), d.put(nh), T, am));
    // draft-head rows: two in range, one past the table (zero rows)
    const std::vector<uint32_t> gids{3, V - 1, V};
    const Buffer dq = d.zeros((size_t)3 * K / 2), ds = d.zeros((size_t)3 * (K / G) * 4);
    add(b.gather_rows("gather_rows", "embed", K, V, 3, d.put(gids), dq, ds));
    auto r = encode(ops, nullptr);
    CHECK(r.is_ok(), "encode: %s", r.error().c_str());
    HIP_OK(hipDeviceSynchronize());

    std::vector<float> xw((size_t)T * K);
    or_embed(tab.q.data(), tab.s.data(), V, K, G, tok.data(), T, xw.data());
    CHECK(same_bits(get<float>(x, xw.size()), xw), "embed");
    const uint32_t KO = H * D;
    std::vector<int8_t> cq((size_t)T * KO);
    std::vector<float> cd((size_t)T * KO / 32), yo((size_t)T * N);
    std::vector<int32_t> cs((size_t)T * KO / 32);
    or_attn_combine(part.data(), T, H, D, NCH, POS, nullptr, 0, cq.data(), cd.data(), cs.data());
    CHECK(same_bits(get<int8_t>(ao.xq, cq.size()), cq), "attn_combine codes");
    CHECK(same_bits(get<float>(ao.dx, cd.size()), cd), "attn_combine scales");
    CHECK(same_bits(get<int32_t>(ao.xs, cs.size()), cs), "attn_combine sums");
    or_linear(wo.q.data(), wo.s.data(), N, KO, G, cq.data(), cd.data(), cs.data(), T, 32, 0, yo.data());
    CHECK(same_bits(get<float>(y, yo.size()), yo), "o projection on per-32 activations");
    std::vector<int8_t> mq((size_t)T * 2 * K);
    std::vector<float> md((size_t)T * 2 * K / 32);
    std::vector<int32_t> ms((size_t)T * 2 * K / 32);
    or_mtp_in(emb.data(), hid.data(), nf.data(), ne.data(), nh.data(), 1e-6f, T, K, mq.data(), md.data(), ms.data());
    CHECK(same_bits(get<int8_t>(am.xq, mq.size()), mq), "mtp_in codes");
    CHECK(same_bits(get<float>(am.dx, md.size()), md), "mtp_in scales");
    CHECK(same_bits(get<int32_t>(am.xs, ms.size()), ms), "mtp_in sums");
    const std::vector<uint32_t> gq = get<uint32_t>(dq, 3 * K / 8), gs = get<uint32_t>(ds, 3 * (K / G));
    bool rows_ok = true;
    for (int r = 0; r < 3; ++r)
        for (uint32_t i = 0; i < K / 8; ++i)
            rows_ok &= gq[r * (K / 8) + i] == (r < 2 ? tab.q[(size_t)gids[r] * (K / 8) + i] : 0u);
    for (int r = 0; r < 3; ++r)
        for (uint32_t i = 0; i < K / G; ++i)
            rows_ok &= gs[r * (K / G) + i] == (r < 2 ? tab.s[(size_t)gids[r] * (K / G) + i] : 0u);
    CHECK(rows_ok, "gather_rows");
    std::printf("  embed, attn_combine -> o_proj, mtp_in, gather_rows: %zu ops replayed, compared with the oracle\n",
                ops.size());
    std::fflush(stdout);
}

// Device step parameters (wq_params): a prefill chunk's list recorded for
// 128 tokens runs the m tokens the Params buffer holds when it replays, and a
// chunk-merge op recorded once follows the position written into the buffer,
// each against the oracle; the host-resolved step (encode's Step) sizes the
// same ops without the buffer.
static void gpu_params() {
    const uint32_t H = 1024, N = 512, CAP = kPrefillChunk;
    const int G = 128;
    std::mt19937 rng(91);
    Q4Host w = make_weight(rng, N, H, G);
    Dev d;
    Builder b({{"w.q", d.put(w.q)}, {"w.s", d.put(w.s)}}, G);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<float> x((size_t)CAP * H);
    for (float& v : x) v = nd(rng);
    const Buffer xr = d.put(x);
    Acts a;
    a.xq = d.zeros((size_t)CAP * H);
    a.dx = d.zeros((size_t)CAP * 4);
    a.xs = d.zeros((size_t)CAP * (H / G) * 4);
    const std::vector<float> sentinel((size_t)CAP * N, std::nanf(""));
    const Buffer y = d.put(sentinel);
    wq_params hp{0, 0, CAP, 0};
    const Buffer prm = d.put(std::vector<wq_params>{hp});

    std::vector<OpDef> ops;
    auto add = [&](std::vector<OpDef>& list, Result<OpDef> r) {
        CHECK(r.is_ok(), "build: %s", r.error().c_str());
        if (r.is_ok()) list.push_back(r.value());
    };
    add(ops, b.quant("quant", H, 1e-6, xr, nullptr, CAP, a));
    add(ops, b.matmul(Path::Prefill, "gemm", "w", H, N, WQ_MODE_STORE, a, y, CAP, &prm));
    // oracle over all 128 tokens (the quantiser runs per token)
    std::vector<int8_t> q((size_t)CAP * H);
    std::vector<float> dx(CAP), want((size_t)CAP * N);
    std::vector<int32_t> xs((size_t)CAP * (H / G));
    or_quant_act(x.data(), nullptr, 1e-6f, CAP, H, (int)H, G, q.data(), dx.data(), xs.data());
    or_linear(w.q.data(), w.s.data(), N, H, G, q.data(), dx.data(), xs.data(), CAP, (int)H, 0, want.data());
    auto rows_match = [&](const std::vector<float>& got, uint32_t m) {
        std::vector<float> g0(got.begin(), got.begin() + (size_t)m * N), w0(want.begin(), want.begin() + (size_t)m * N);
        bool rest_untouched = true;
        for (size_t i = (size_t)m * N; i < got.size(); ++i) rest_untouched &= std::isnan(got[i]);
        return std::make_pair(rel_err(g0, w0), rest_untouched);
    };
    for (uint32_t m : {77u, 128u, 1u}) {
        HIP_OK(hipMemcpy(y.ptr, sentinel.data(), sentinel.size() * 4, hipMemcpyHostToDevice));
        hp.m = m;
        HIP_OK(hipMemcpy(prm.ptr, &hp, sizeof hp, hipMemcpyHostToDevice));  // only the Params buffer changes
        auto r = encode(ops, nullptr);
        CHECK(r.is_ok(), "encode: %s", r.error().c_str());
        HIP_OK(hipDeviceSynchronize());
        auto [e, untouched] = rows_match(get<float>(y, sentinel.size()), m);
        CHECK(e < 1e-5 && untouched, "params m=%u: rows 0..m-1 rel err %.3g, rows past m untouched %d", m, e,
              (int)untouched);
    }
    // the host-resolved step sizes the same ops (params left at 128)
    hp.m = CAP;
    HIP_OK(hipMemcpy(prm.ptr, &hp, sizeof hp, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(y.ptr, sentinel.data(), sentinel.size() * 4, hipMemcpyHostToDevice));
    auto r = encode(ops, nullptr, Step{0, 50});
    CHECK(r.is_ok(), "encode step: %s", r.error().c_str());
    HIP_OK(hipDeviceSynchronize());
    auto [e50, u50] = rows_match(get<float>(y, sentinel.size()), 50);
    CHECK(e50 < 1e-5 && u50, "Step m=50: rel err %.3g, rows past m untouched %d", e50, (int)u50);

    // chunk merge recorded once, replayed at three positions
    const uint32_t HH = 4, D = 128, NCH = 16, T = 2;
    const int64_t BOUND = 32 * NCH - T;
    std::normal_distribution<float> pn(0.0f, 3.0f);
    std::uniform_real_distribution<float> ud(1.0f, 32.0f);
    std::vector<float> part((size_t)T * HH * NCH * (D + 2));
    for (size_t i = 0; i < part.size(); ++i) {
        const size_t c = i % (D + 2);
        part[i] = c == D ? 0.75f : c == D + 1 ? ud(rng) : pn(rng);
    }
    Acts ao;
    ao.xq = d.zeros((size_t)T * HH * D);
    ao.dx = d.zeros((size_t)T * HH * D / 32 * 4);
    ao.xs = d.zeros((size_t)T * HH * D / 32 * 4);
    ao.ga = 32;
    std::vector<OpDef> comb;
    add(comb, b.attn_combine("attn_combine", d.put(part), T, HH, D, NCH, BOUND, nullptr, 0, ao, &prm));
    for (uint32_t pos : {40u, 300u, 7u}) {
        hp.pos = pos;
        HIP_OK(hipMemcpy(prm.ptr, &hp, sizeof hp, hipMemcpyHostToDevice));
        auto rc = encode(comb, nullptr);
        CHECK(rc.is_ok(), "encode combine: %s", rc.error().c_str());
        HIP_OK(hipDeviceSynchronize());
        const uint32_t KO = HH * D;
        std::vector<int8_t> cq((size_t)T * KO);
        std::vector<float> cd((size_t)T * KO / 32);
        std::vector<int32_t> cs((size_t)T * KO / 32);
        or_attn_combine(part.data(), T, HH, D, NCH, pos, nullptr, 0, cq.data(), cd.data(), cs.data());
        CHECK(same_bits(get<int8_t>(ao.xq, cq.size()), cq) && same_bits(get<float>(ao.dx, cd.size()), cd) &&
                  same_bits(get<int32_t>(ao.xs, cs.size()), cs),
              "params pos=%u: attn_combine codes, scales, sums", pos);
    }
    std::printf("  params: prefill list for 128 tokens at m = 77, 128, 1 and Step m = 50; "
                "chunk merge at positions 40, 300, 7: compared with the oracle\n");
    std::fflush(stdout);
}

static void gpu_checks() {
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (n < 1) {
        std::printf("no GPU\n");
        std::exit(2);
    }
    gpu_step(Path::Decode, 1);
    gpu_step(Path::Spec, 2);
    gpu_step(Path::Prefill, 128);
    gpu_producers();
    gpu_params();
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "--cpu";
    if (mode == "--cpu") cpu_checks();
    else if (mode == "--gpu") gpu_checks();
    else {
        std::printf("usage: builder_test --cpu | --gpu\n");
        return 2;
    }
    if (g_failures) {
        std::printf("builder_test %s: %d failures\n", mode.c_str() + 2, g_failures);
        return 1;
    }
    std::printf("builder_test %s ok\n", mode.c_str() + 2);
    return 0;
}
