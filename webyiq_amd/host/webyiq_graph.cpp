// Builder, OpDef and encode over the C ABI (see webyiq_graph.hpp).
#include "webyiq_graph.hpp"

#include <cstdarg>
#include <cstdio>

#include "../../include/webyiq_q4q8.h"

namespace webyiq {
namespace {

std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// Shape rules of the path (graph.rs:368-380 requires K % 128; the GEMV
// holds at most 8 tokens)
std::string check_kn(const std::string& name, uint32_t k, uint32_t n, uint32_t mode) {
    if (k == 0 || k % 128 != 0) return fmt("%s: K = %u is not a positive multiple of 128", name.c_str(), k);
    if (n == 0) return fmt("%s: N = 0", name.c_str());
    if (mode > 2) return fmt("%s: unknown mode %u", name.c_str(), mode);
    return {};
}

std::string check_size(const std::string& name, const char* what, Buffer b, size_t need) {
    if (b.ptr == nullptr) return fmt("%s: %s is not bound", name.c_str(), what);
    if (b.bytes < need)
        return fmt("%s: %s holds %zu bytes, the shape needs %zu", name.c_str(), what, b.bytes, need);
    return {};
}

// Tokens an op built for `built` tokens runs at step.m (0: as built).
uint32_t step_tokens(Step st, uint32_t built) { return st.m == 0 || st.m > built ? built : st.m; }

}  // namespace

uint32_t tokens(Path p) {
    switch (p) {
        case Path::Decode: return 1;
        case Path::Spec: return kSpecTokens;
        default: return kPrefillChunk;
    }
}

Builder::Builder(std::unordered_map<std::string, Buffer> weights, int32_t group)
    : weights_(std::move(weights)), group_(group) {}

Result<Buffer> Builder::w(const std::string& name) const {
    auto it = weights_.find(name);
    if (it == weights_.end()) return Result<Buffer>::err("missing tensor " + name);
    return Result<Buffer>::ok(it->second);
}

Result<Builder::Q4> Builder::q4(const std::string& w, uint32_t rows, uint32_t k) const {
    if (group_ != 32 && group_ != 128)
        return Result<Q4>::err(fmt("%s: quant group %d (32 or 128)", w.c_str(), group_));
    auto q = this->w(w + ".q");
    if (!q.is_ok()) return Result<Q4>::err(q.error());
    auto s = this->w(w + ".s");
    if (!s.is_ok()) return Result<Q4>::err(s.error());
    std::string e = check_size(w, "the .q tensor", q.value(), (size_t)rows * k / 2);
    if (e.empty()) e = check_size(w, "the .s tensor", s.value(), (size_t)rows * (k / group_) * 4);
    if (!e.empty()) return Result<Q4>::err(e);
    return Result<Q4>::ok(Q4{q.value(), s.value()});
}

std::string Builder::check_acts(const std::string& name, uint32_t k, uint32_t t, const Acts& a) const {
    if (group_ != 32 && group_ != 128) return fmt("%s: quant group %d (32 or 128)", name.c_str(), group_);
    const uint32_t ga = a.ga == 0 ? k : a.ga;
    if (ga != k && ga != 32) return fmt("%s: activation group %u (32 or per token)", name.c_str(), ga);
    const uint32_t ge = ga < (uint32_t)group_ ? ga : (uint32_t)group_;
    std::string e = check_size(name, "xq", a.xq, (size_t)t * k);
    if (e.empty()) e = check_size(name, "dx", a.dx, (size_t)t * (k / ga) * 4);
    if (e.empty()) e = check_size(name, "xs", a.xs, (size_t)t * (k / ge) * 4);
    return e;
}

Result<OpDef> Builder::gemv(const std::string& name, const std::string& w, uint32_t k, uint32_t n, uint32_t mode,
                            uint32_t t, const Acts& a, Buffer y) {
    std::string e = check_kn(name, k, n, mode);
    if (e.empty() && (t == 0 || t > 8)) e = fmt("%s: %u tokens (the GEMV takes 1..8)", name.c_str(), t);
    if (e.empty()) e = check_acts(name, k, t, a);
    if (e.empty()) e = check_size(name, "y", y, (size_t)t * n * 4);
    if (!e.empty()) return Result<OpDef>::err(e);
    auto wt = q4(w, mode == 2 ? 2 * n : n, k);
    if (!wt.is_ok()) return Result<OpDef>::err(wt.error());
    const Q4 q = wt.value();
    const int32_t g = group_, ga = (int32_t)(a.ga == 0 ? k : a.ga);
    const Acts in = a;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step) {
        return wq_gemv(s, (const uint32_t*)q.q.ptr, (const uint32_t*)q.s.ptr, n, k, g, (const int8_t*)in.xq.ptr,
                       (const float*)in.dx.ptr, (const int32_t*)in.xs.ptr, t, ga, (int32_t)mode, (float*)y.ptr);
    }});
}

Result<OpDef> Builder::gemm(const std::string& name, const std::string& w, uint32_t k, uint32_t n, uint32_t mode,
                            uint32_t m, const Acts& a, Buffer y, const Buffer* params, const Buffer* workspace) {
    std::string e = check_kn(name, k, n, mode);
    if (e.empty() && m == 0) e = fmt("%s: 0 tokens", name.c_str());
    if (e.empty()) e = check_acts(name, k, m, a);
    if (e.empty()) e = check_size(name, "y", y, (size_t)m * n * 4);
    if (e.empty() && params) e = check_size(name, "params", *params, sizeof(wq_params));
    if (!e.empty()) return Result<OpDef>::err(e);
    auto wt = q4(w, mode == 2 ? 2 * n : n, k);
    if (!wt.is_ok()) return Result<OpDef>::err(wt.error());
    const Q4 q = wt.value();
    const int32_t g = group_, ga = (int32_t)(a.ga == 0 ? k : a.ga);
    const Acts in = a;
    const wq_params* pp = params ? (const wq_params*)params->ptr : nullptr;
    const Buffer wsb = workspace ? *workspace : Buffer{};
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step st) {
        return wq_gemm(s, (const uint32_t*)q.q.ptr, (const uint32_t*)q.s.ptr, n, k, g, (const int8_t*)in.xq.ptr,
                       (const float*)in.dx.ptr, (const int32_t*)in.xs.ptr, step_tokens(st, m), ga, (int32_t)mode,
                       (float*)y.ptr, pp, wsb.ptr, wsb.bytes);
    }});
}

Result<OpDef> Builder::matmul(Path path, const std::string& name, const std::string& w, uint32_t k, uint32_t n,
                              uint32_t mode, const Acts& a, Buffer y, uint32_t m, const Buffer* params) {
    if (path == Path::Prefill) return gemm(name, w, k, n, mode, m, a, y, params);
    return gemv(name, w, k, n, mode, tokens(path), a, y);
}

Result<OpDef> Builder::quant(const std::string& name, uint32_t k, double eps, Buffer x, const Buffer* norm,
                             uint32_t t, const Acts& a) {
    std::string e = check_kn(name, k, 1, 0);
    if (e.empty() && t == 0) e = fmt("%s: 0 tokens", name.c_str());
    if (e.empty()) e = check_size(name, "x", x, (size_t)t * k * 4);
    if (e.empty() && norm) e = check_size(name, "the norm weight", *norm, (size_t)k * 4);
    if (e.empty()) e = check_acts(name, k, t, a);
    if (!e.empty()) return Result<OpDef>::err(e);
    const void* nw = norm ? norm->ptr : nullptr;
    const int32_t g = group_, ga = (int32_t)(a.ga == 0 ? k : a.ga);
    const Acts out = a;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step st) {
        return wq_quant_act(s, (const float*)x.ptr, (const float*)nw, (float)eps, step_tokens(st, t), k, ga, g,
                            (int8_t*)out.xq.ptr, (float*)out.dx.ptr, (int32_t*)out.xs.ptr);
    }});
}

Result<OpDef> Builder::quant_gemv(const std::string& name, const std::string& w, uint32_t k, uint32_t n,
                                  uint32_t mode, uint32_t t, double eps, Buffer x, const Buffer* norm,
                                  const Acts& a, Buffer y) {
    if (a.ga != 0 && a.ga != k)
        return Result<OpDef>::err(fmt("%s: the fused quantiser writes per-token activations", name.c_str()));
    std::string e = check_kn(name, k, n, mode);
    if (e.empty() && (t == 0 || t > 8)) e = fmt("%s: %u tokens (the GEMV takes 1..8)", name.c_str(), t);
    if (e.empty()) e = check_size(name, "x", x, (size_t)t * k * 4);
    if (e.empty() && norm) e = check_size(name, "the norm weight", *norm, (size_t)k * 4);
    if (e.empty()) e = check_acts(name, k, t, a);
    if (e.empty()) e = check_size(name, "y", y, (size_t)t * n * 4);
    if (!e.empty()) return Result<OpDef>::err(e);
    auto wt = q4(w, mode == 2 ? 2 * n : n, k);
    if (!wt.is_ok()) return Result<OpDef>::err(wt.error());
    const Q4 q = wt.value();
    const void* nw = norm ? norm->ptr : nullptr;
    const int32_t g = group_;
    const Acts out = a;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step) {
        return wq_quant_gemv(s, (const float*)x.ptr, (const float*)nw, (float)eps, (const uint32_t*)q.q.ptr,
                             (const uint32_t*)q.s.ptr, n, k, g, t, (int32_t)mode, (int8_t*)out.xq.ptr,
                             (float*)out.dx.ptr, (int32_t*)out.xs.ptr, (float*)y.ptr);
    }});
}

Result<std::vector<OpDef>> Builder::head_ops(const std::string& head, uint32_t k, uint32_t v, uint32_t t, double eps,
                                             Buffer x, Buffer norm, const Acts& a, const Buffer* ids, Buffer tok,
                                             Buffer workspace, const Buffer* logits) {
    using R = Result<std::vector<OpDef>>;
    auto nq = quant("norm_quant", k, eps, x, &norm, t, a);
    if (!nq.is_ok()) return R::err(nq.error());
    const std::string name = "lm_head";
    std::string e = check_kn(name, k, v, 0);
    if (e.empty() && (t == 0 || t > 8)) e = fmt("%s: %u tokens (the GEMV takes 1..8)", name.c_str(), t);
    if (e.empty()) e = check_size(name, "tok", tok, (size_t)t * 4);
    if (e.empty() && ids) e = check_size(name, "ids", *ids, (size_t)v * 4);
    if (e.empty() && logits) e = check_size(name, "logits", *logits, (size_t)t * v * 4);
    if (e.empty()) e = check_size(name, "the workspace", workspace, wq_lm_head_workspace_bytes());
    if (!e.empty()) return R::err(e);
    auto wt = q4(head, v, k);
    if (!wt.is_ok()) return R::err(wt.error());
    const Q4 q = wt.value();
    const int32_t g = group_, ga = (int32_t)(a.ga == 0 ? k : a.ga);
    const void* idp = ids ? ids->ptr : nullptr;
    void* lgp = logits ? logits->ptr : nullptr;
    const Acts in = a;
    std::vector<OpDef> ops;
    ops.push_back(nq.value());
    ops.push_back(OpDef{name, [=](void* s, Step) {
        return wq_lm_head_argmax(s, (const uint32_t*)q.q.ptr, (const uint32_t*)q.s.ptr, v, k, g,
                                 (const int8_t*)in.xq.ptr, (const float*)in.dx.ptr, (const int32_t*)in.xs.ptr, t,
                                 ga, (const uint32_t*)idp, (float*)lgp, (uint32_t*)tok.ptr, workspace.ptr,
                                 workspace.bytes);
    }});
    return R::ok(std::move(ops));
}

Result<OpDef> Builder::embed(const std::string& name, const std::string& table, uint32_t k, uint32_t v, uint32_t t,
                             Buffer tok, Buffer x) {
    std::string e = check_kn(name, k, v, 0);
    if (e.empty() && t == 0) e = fmt("%s: 0 tokens", name.c_str());
    if (e.empty()) e = check_size(name, "tok", tok, (size_t)t * 4);
    if (e.empty()) e = check_size(name, "x", x, (size_t)t * k * 4);
    if (!e.empty()) return Result<OpDef>::err(e);
    auto wt = q4(table, v, k);
    if (!wt.is_ok()) return Result<OpDef>::err(wt.error());
    const Q4 q = wt.value();
    const int32_t g = group_;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step) {
        return wq_embed(s, (const uint32_t*)q.q.ptr, (const uint32_t*)q.s.ptr, v, k, g, (const uint32_t*)tok.ptr, t,
                        (float*)x.ptr);
    }});
}

Result<OpDef> Builder::gather_rows(const std::string& name, const std::string& table, uint32_t k, uint32_t v,
                                   uint32_t r, Buffer ids, Buffer dq, Buffer ds) {
    std::string e = check_kn(name, k, v, 0);
    if (e.empty() && r == 0) e = fmt("%s: 0 rows", name.c_str());
    if (e.empty() && group_ != 32 && group_ != 128) e = fmt("%s: quant group %d (32 or 128)", name.c_str(), group_);
    if (e.empty()) e = check_size(name, "ids", ids, (size_t)r * 4);
    if (e.empty()) e = check_size(name, "dq", dq, (size_t)r * k / 2);
    if (e.empty()) e = check_size(name, "ds", ds, (size_t)r * (k / group_) * 4);
    if (!e.empty()) return Result<OpDef>::err(e);
    auto wt = q4(table, v, k);
    if (!wt.is_ok()) return Result<OpDef>::err(wt.error());
    const Q4 q = wt.value();
    const int32_t g = group_;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step) {
        return wq_gather_rows(s, (const uint32_t*)q.q.ptr, (const uint32_t*)q.s.ptr, v, k, g,
                              (const uint32_t*)ids.ptr, r, (uint32_t*)dq.ptr, (uint32_t*)ds.ptr);
    }});
}

Result<OpDef> Builder::attn_combine(const std::string& name, Buffer part, uint32_t t, uint32_t h, uint32_t d,
                                    uint32_t nch, int64_t pos, const Buffer* gate, int64_t gate_stride,
                                    const Acts& a, const Buffer* params) {
    std::string e;
    if (d != 64 && d != 128 && d != 256) e = fmt("%s: head dim %u (64, 128 or 256)", name.c_str(), d);
    if (e.empty() && (t == 0 || h == 0 || nch == 0)) e = fmt("%s: empty shape", name.c_str());
    if (e.empty() && (pos < 0 || pos + t - 1 >= 32 * (int64_t)nch))
        e = fmt("%s: positions 0..%lld exceed the %u chunks", name.c_str(), (long long)(pos + t - 1), nch);
    if (e.empty() && a.ga != 32) e = fmt("%s: the chunk merge writes per-32 activations (ga = 32)", name.c_str());
    if (e.empty()) e = check_size(name, "part", part, (size_t)t * h * nch * (d + 2) * 4);
    if (e.empty() && gate) {
        if (gate_stride < 2 * (int64_t)h * d) e = fmt("%s: gate_stride %lld < 2 h d", name.c_str(), (long long)gate_stride);
        else e = check_size(name, "gate", *gate, ((size_t)(t - 1) * gate_stride + 2 * (size_t)h * d) * 4);
    }
    if (e.empty()) e = check_acts(name, h * d, t, a);
    if (e.empty() && params) e = check_size(name, "params", *params, sizeof(wq_params));
    if (!e.empty()) return Result<OpDef>::err(e);
    const void* gp = gate ? gate->ptr : nullptr;
    const Acts out = a;
    const wq_params* pp = params ? (const wq_params*)params->ptr : nullptr;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step st) {
        return wq_attn_combine(s, (const float*)part.ptr, step_tokens(st, t), h, d, nch, pos, (const float*)gp,
                               gate_stride, (int8_t*)out.xq.ptr, (float*)out.dx.ptr, (int32_t*)out.xs.ptr, pp);
    }});
}

Result<OpDef> Builder::mtp_in(const std::string& name, uint32_t k, double eps, Buffer emb, Buffer x, Buffer norm_f,
                              Buffer norm_e, Buffer norm_h, uint32_t t, const Acts& a) {
    std::string e = check_kn(name, k, 1, 0);
    if (e.empty() && t == 0) e = fmt("%s: 0 tokens", name.c_str());
    if (e.empty() && a.ga != 32) e = fmt("%s: the MTP input is per-32 activations (ga = 32)", name.c_str());
    if (e.empty()) e = check_size(name, "emb", emb, (size_t)t * k * 4);
    if (e.empty()) e = check_size(name, "x", x, (size_t)t * k * 4);
    if (e.empty()) e = check_size(name, "norm_f", norm_f, (size_t)k * 4);
    if (e.empty()) e = check_size(name, "norm_e", norm_e, (size_t)k * 4);
    if (e.empty()) e = check_size(name, "norm_h", norm_h, (size_t)k * 4);
    if (e.empty()) e = check_acts(name, 2 * k, t, a);
    if (!e.empty()) return Result<OpDef>::err(e);
    const Acts out = a;
    return Result<OpDef>::ok(OpDef{name, [=](void* s, Step) {
        return wq_mtp_in(s, (const float*)emb.ptr, (const float*)x.ptr, (const float*)norm_f.ptr,
                         (const float*)norm_e.ptr, (const float*)norm_h.ptr, (float)eps, t, k, (int8_t*)out.xq.ptr,
                         (float*)out.dx.ptr, (int32_t*)out.xs.ptr);
    }});
}

Result<Unit> encode(const std::vector<OpDef>& ops, void* stream, Step step) {
    for (const OpDef& op : ops) {
        const int rc = op.launch(stream, step);
        if (rc != WQ_OK) return Result<Unit>::err(op.name + ": " + wq_last_error());
    }
    return Result<Unit>::ok(Unit{});
}

}  // namespace webyiq
