// C entry points over the reference's own Model and Tokenizer (model.cpp, tokenizer.cpp,
// backend.cpp, quant.cpp, gguf.cpp, cuda.cpp, hardware.cpp from
// /root/reference/v1.1/src, compiled unchanged, with PCRE2 10.45 and utf8proc from its
// third_party/), built into oracle/_ref/libemprise_refmodel.so by oracle/Makefile.
// TEST INFRASTRUCTURE ONLY: tests/ use it to pin the oracle's model composition
// (attention, RoPE, the MTP head, the trace points) and its tokenizer against the
// reference's compiled code. The model always runs on the reference's CPU backend
// (ModelOptions::cuda = false): this is the CPU path the oracle restates.
#include "emprise/model.hpp"

#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

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
typedef void (*refm_trace_fn)(void* user, uint64_t position, const char* name, const float* data, uint64_t n);
struct Handle {
    refm_trace_fn fn = nullptr;
    void* user = nullptr;
    std::unique_ptr<Model> model;
};
}  // namespace

extern "C" {

const char* refm_last_error(void) { return g_error.c_str(); }

// A Model over `path` on the CPU backend with `threads` OpenMP threads (0: the
// reference's default). The trace hook forwards to refm_set_trace's fn.
void* refm_open(const char* path, uint64_t context, unsigned threads) {
    auto h = std::make_unique<Handle>();
    Handle* raw = h.get();
    const int rc = guarded([&] {
        ModelOptions o;
        o.context = static_cast<size_t>(context);
        o.cuda = false;
        o.threads = threads;
        o.disk = DiskPolicy::disabled;
        o.trace = [raw](size_t pos, const std::string& name, std::span<const float> x) {
            if (raw->fn) raw->fn(raw->user, pos, name.c_str(), x.data(), x.size());
        };
        h->model = std::make_unique<Model>(path, o);
    });
    return rc ? nullptr : h.release();
}

void refm_close(void* p) { delete static_cast<Handle*>(p); }

void refm_set_trace(void* p, refm_trace_fn fn, void* user) {
    Handle* h = static_cast<Handle*>(p);
    h->fn = fn;
    h->user = user;
}

int refm_reset(void* p) {
    return guarded([&] { static_cast<Handle*>(p)->model->reset(); });
}

// Model::evaluate; logits (vocab floats) may be NULL (then the output head is skipped).
int refm_evaluate(void* p, int token, float* logits, uint64_t vocab) {
    return guarded([&] {
        auto v = static_cast<Handle*>(p)->model->evaluate(token, logits != nullptr);
        if (logits) {
            if (v.size() != vocab) throw std::runtime_error("vocab size");
            std::memcpy(logits, v.data(), v.size() * sizeof(float));
        }
    });
}

// Model::evaluate_block: n rows of vocab floats.
int refm_evaluate_block(void* p, const int* tokens, uint64_t n, float* logits, uint64_t vocab) {
    return guarded([&] {
        auto rows = static_cast<Handle*>(p)->model->evaluate_block(std::vector<int>(tokens, tokens + n));
        if (rows.size() != n) throw std::runtime_error("block size");
        for (uint64_t i = 0; i < n; ++i) {
            if (rows[i].size() != vocab) throw std::runtime_error("vocab size");
            std::memcpy(logits + i * vocab, rows[i].data(), vocab * sizeof(float));
        }
    });
}

// Model::prefill: the last position's logits.
int refm_prefill(void* p, const int* tokens, uint64_t n, float* logits, uint64_t vocab) {
    return guarded([&] {
        auto v = static_cast<Handle*>(p)->model->prefill(std::vector<int>(tokens, tokens + n));
        if (v.size() != vocab) throw std::runtime_error("vocab size");
        std::memcpy(logits, v.data(), vocab * sizeof(float));
    });
}

// Model::last_hidden (raw = 0) or last_hidden_raw (raw = 1).
int refm_last_hidden(void* p, int raw, float* out, uint64_t n) {
    return guarded([&] {
        Model& m = *static_cast<Handle*>(p)->model;
        auto v = raw ? m.last_hidden_raw() : m.last_hidden();
        if (v.size() != n) throw std::runtime_error("hidden size");
        std::memcpy(out, v.data(), n * sizeof(float));
    });
}

int refm_mtp_draft(void* p, const float* hidden, uint64_t n, int token, uint64_t position, float* logits,
                   uint64_t vocab) {
    return guarded([&] {
        auto v = static_cast<Handle*>(p)->model->mtp_draft(std::vector<float>(hidden, hidden + n), token,
                                                           static_cast<size_t>(position));
        if (v.size() != vocab) throw std::runtime_error("vocab size");
        std::memcpy(logits, v.data(), vocab * sizeof(float));
    });
}

int refm_mtp_hidden(void* p, float* out, uint64_t n) {
    return guarded([&] {
        auto v = static_cast<Handle*>(p)->model->mtp_hidden();
        if (v.size() != n) throw std::runtime_error("hidden size");
        std::memcpy(out, v.data(), n * sizeof(float));
    });
}

int refm_reset_mtp(void* p) {
    return guarded([&] { static_cast<Handle*>(p)->model->reset_mtp(); });
}

// Tokenizer::encode of the model's vocabulary: writes up to cap ids, returns the count
// (or -1).
int64_t refm_encode(void* p, const char* text, uint64_t len, int parse_special, int* ids, uint64_t cap) {
    int64_t n = -1;
    guarded([&] {
        auto v = static_cast<Handle*>(p)->model->tokenizer().encode(std::string(text, len), parse_special != 0);
        n = static_cast<int64_t>(v.size());
        for (uint64_t i = 0; i < v.size() && i < cap; ++i) ids[i] = v[i];
    });
    return n;
}

// Tokenizer::decode of one id: writes up to cap bytes, returns the length (or -1).
int64_t refm_decode(void* p, int id, char* out, uint64_t cap) {
    int64_t n = -1;
    guarded([&] {
        auto s = static_cast<Handle*>(p)->model->tokenizer().decode(id);
        n = static_cast<int64_t>(s.size());
        std::memcpy(out, s.data(), s.size() < cap ? s.size() : cap);
    });
    return n;
}

// Tokenizer::chat_prompt.
int64_t refm_chat_prompt(void* p, const char* user, uint64_t len, char* out, uint64_t cap) {
    int64_t n = -1;
    guarded([&] {
        auto s = static_cast<Handle*>(p)->model->tokenizer().chat_prompt(std::string(user, len));
        n = static_cast<int64_t>(s.size());
        std::memcpy(out, s.data(), s.size() < cap ? s.size() : cap);
    });
    return n;
}

}  // extern "C"
