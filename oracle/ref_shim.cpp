// C entry points over the reference's own CPU sources (quant.cpp, gguf.cpp,
// backend.cpp from /root/reference/v1.1/src), compiled unchanged into
// oracle/_ref/libemprise_ref.so by oracle/Makefile. TEST INFRASTRUCTURE ONLY: used by
// tests/ to pin the oracle restatement against the reference's compiled code.
// The reference's Model and Tokenizer are wrapped by ref_model_shim.cpp in a library of
// their own (libemprise_refmodel.so, with PCRE2 and utf8proc).
#include "emprise/backend.hpp"
#include "emprise/gguf.hpp"

#include <cstring>
#include <memory>
#include <span>
#include <string>

using namespace emprise;

namespace {
thread_local std::string g_error;
template <class F> int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}
}

extern "C" {
const char* ref_last_error() { return g_error.c_str(); }

float ref_half_to_float(uint16_t h) { return half_to_float(h); }

int ref_encoded_bytes(uint32_t type, uint64_t n, uint64_t* out) {
    return guarded([&] { *out = encoded_bytes(static_cast<WeightType>(type), n); });
}

int ref_dequantize(uint32_t type, const void* in, size_t in_len, float* out, size_t n) {
    return guarded([&] {
        dequantize(static_cast<WeightType>(type), std::span(static_cast<const std::byte*>(in), in_len),
                   std::span(out, n));
    });
}

int ref_matvec(uint32_t type, const void* w, size_t w_len, const float* x, size_t cols, float* y, size_t rows) {
    return guarded([&] {
        matvec(static_cast<WeightType>(type), std::span(static_cast<const std::byte*>(w), w_len),
               std::span(x, cols), std::span(y, rows));
    });
}

// ---- GGUF + CPU backend (backend.cpp) over a model file ----
struct ref_model {
    std::unique_ptr<Gguf> gguf;
    std::unique_ptr<Backend> cpu;
};

ref_model* ref_open(const char* path, uint64_t ram_budget) {
    ref_model* m = nullptr;
    if (guarded([&] {
            auto g = std::make_unique<Gguf>(path);
            g->configure_storage(DiskPolicy::automatic, ram_budget);
            m = new ref_model{std::move(g), cpu_backend()};
        }))
        return nullptr;
    return m;
}
void ref_close(ref_model* m) { delete m; }

int ref_tensor_info(ref_model* m, const char* name, uint32_t* type, uint64_t* shape, uint32_t* ndim, uint64_t* bytes) {
    return guarded([&] {
        const Tensor& t = m->gguf->tensor(name);
        *type = static_cast<uint32_t>(t.type);
        *ndim = static_cast<uint32_t>(t.shape.size());
        for (size_t i = 0; i < t.shape.size(); ++i) shape[i] = t.shape[i];
        *bytes = t.bytes;
    });
}

int ref_tensor_read(ref_model* m, const char* name, void* out, uint64_t len) {
    return guarded([&] {
        const Tensor& t = m->gguf->tensor(name);
        m->gguf->read(t, 0, std::span(static_cast<std::byte*>(out), len));
    });
}

int ref_metadata_json(ref_model* m, char* out, size_t cap) {
    return guarded([&] {
        const std::string& s = m->gguf->metadata_json();
        if (s.size() + 1 > cap) throw std::runtime_error("metadata buffer too small");
        std::memcpy(out, s.c_str(), s.size() + 1);
    });
}

int ref_linear(ref_model* m, const char* name, const float* x, size_t cols, float* y, size_t rows) {
    return guarded([&] { m->cpu->linear(*m->gguf, m->gguf->tensor(name), std::span(x, cols), std::span(y, rows)); });
}

int ref_feed_forward(ref_model* m, const char* gate, const char* up, const char* down, const float* x, size_t hidden,
                     float* y) {
    return guarded([&] {
        m->cpu->feed_forward(*m->gguf, m->gguf->tensor(gate), m->gguf->tensor(up), m->gguf->tensor(down),
                             std::span(x, hidden), std::span(y, hidden));
    });
}

// Backend::delta_net (backend.cpp:19-60); the Gguf argument is unused by the CPU path.
int ref_delta_net(ref_model* m, int key_heads, int value_heads, int state_dim, int conv_width, float eps,
                  const float* qkv, const float* gate, const float* alpha, const float* beta, const float* conv,
                  const float* ssm_a, const float* dt, const float* norm, float* conv_state, float* rec_state,
                  float* out) {
    return guarded([&] {
        const size_t kd = size_t(key_heads) * state_dim, vd = size_t(value_heads) * state_dim, ch = 2 * kd + vd;
        Backend::DeltaNet d;
        d.key_heads = key_heads; d.value_heads = value_heads; d.state_dim = state_dim; d.conv_width = conv_width;
        d.eps = eps; d.slot = 0;
        d.qkv = std::span(qkv, ch); d.gate = std::span(gate, vd);
        d.alpha = std::span(alpha, size_t(value_heads)); d.beta = std::span(beta, size_t(value_heads));
        d.conv = std::span(conv, ch * conv_width); d.ssm_a = std::span(ssm_a, size_t(value_heads));
        d.dt = std::span(dt, size_t(value_heads)); d.norm = std::span(norm, size_t(state_dim));
        d.conv_state = std::span(conv_state, ch * conv_width); d.rec_state = std::span(rec_state, vd * state_dim);
        d.out = std::span(out, vd);
        m->cpu->delta_net(*m->gguf, d);
    });
}

// Backend::recurrent_block (backend.cpp:61-77) on the tensors of layer `prefix`.
int ref_recurrent_block(ref_model* m, const char* prefix, int key_heads, int value_heads, int state_dim,
                        int conv_width, float eps, const float* conv, const float* ssm_a, const float* dt,
                        const float* norm, const float* x, size_t hidden, float* conv_state, float* rec_state,
                        float* out) {
    return guarded([&] {
        const std::string p(prefix);
        const size_t kd = size_t(key_heads) * state_dim, vd = size_t(value_heads) * state_dim, ch = 2 * kd + vd;
        Backend::RecurrentBlock b;
        b.qkv_w = &m->gguf->tensor(p + "attn_qkv.weight");
        b.gate_w = &m->gguf->tensor(p + "attn_gate.weight");
        b.alpha_w = &m->gguf->tensor(p + "ssm_alpha.weight");
        b.beta_w = &m->gguf->tensor(p + "ssm_beta.weight");
        b.out_w = &m->gguf->tensor(p + "ssm_out.weight");
        b.conv = std::span(conv, ch * conv_width); b.ssm_a = std::span(ssm_a, size_t(value_heads));
        b.dt = std::span(dt, size_t(value_heads)); b.norm = std::span(norm, size_t(state_dim));
        b.key_heads = key_heads; b.value_heads = value_heads; b.state_dim = state_dim; b.conv_width = conv_width;
        b.eps = eps; b.slot = 0;
        b.x = std::span(x, hidden);
        b.conv_state = std::span(conv_state, ch * conv_width); b.rec_state = std::span(rec_state, vd * state_dim);
        b.out = std::span(out, hidden);
        m->cpu->recurrent_block(*m->gguf, b);
    });
}
}
