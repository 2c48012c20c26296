// C ABI of the host library (include/emprise_host.h).
#include <algorithm>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>

#include "emprise_host.h"
#include "gguf.hpp"
#include "model.hpp"
#include "tokenizer.hpp"

namespace emprise {
void synth_write(const emprise_synth_config& c, const std::string& path);
void synth_prompt(uint64_t seed, int vocab, size_t n, int* ids);
}  // namespace emprise

// A tokenizer handle: one opened from a file (owning the GGUF mapping) or the view of a
// model's own tokenizer.
struct emprise_tokenizer {
    std::unique_ptr<emprise::Gguf> file;
    std::unique_ptr<emprise::Tokenizer> owned;
    const emprise::Tokenizer* tok = nullptr;
};

struct emprise_model {
    std::unique_ptr<emprise::Model> model;
    std::string name;
    emprise_tokenizer tokenizer;
};

namespace {
thread_local std::string g_error;

template <class F> emprise_status guarded(F&& f) {
    try {
        f();
        return EMPRISE_OK;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return EMPRISE_EINVAL;
    } catch (const std::out_of_range& e) {
        g_error = e.what();
        return EMPRISE_EINVAL;
    } catch (const std::bad_alloc&) {
        g_error = "out of host memory";
        return EMPRISE_ENOMEM;
    } catch (const std::exception& e) {
        g_error = e.what();
        return EMPRISE_EDEVICE;
    }
}
// Tokenizer calls fail only on their input (invalid UTF-8, an unknown id) or on the
// file's vocabulary: every error is EINVAL.
template <class F> emprise_status guarded_input(F&& f) {
    try {
        f();
        return EMPRISE_OK;
    } catch (const std::bad_alloc&) {
        g_error = "out of host memory";
        return EMPRISE_ENOMEM;
    } catch (const std::exception& e) {
        g_error = e.what();
        return EMPRISE_EINVAL;
    }
}
}  // namespace

extern "C" {

const char* emprise_host_last_error(void) { return g_error.c_str(); }

emprise_status emprise_gguf_inspect(const char* path, uint64_t* tensors, uint64_t* metadata) {
    if (!path) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    try {
        emprise::Gguf g(path);
        if (tensors) *tensors = g.tensors().size();
        if (metadata) *metadata = g.metadata_count();
        return EMPRISE_OK;
    } catch (const std::exception& e) {
        g_error = e.what();
        return EMPRISE_EINVAL;
    }
}

emprise_status emprise_model_open(const emprise_model_options* o, emprise_model** out) {
    if (!o || !o->path || !out) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    *out = nullptr;
    return guarded([&] {
        emprise::ModelOptions opt;
        opt.path = o->path;
        opt.context = o->context ? o->context : 4096;
        opt.device = o->device;
        opt.weight_vram_budget = o->weight_vram_budget;
        opt.quantize_activations = o->quantize_activations != 0;
        opt.fused = o->fused != 0;
        opt.graph = o->graph != 0;
        opt.batch_prefill_min = o->batch_prefill < 0 ? 0 : o->batch_prefill == 0 ? 64 : static_cast<size_t>(o->batch_prefill);
        auto m = std::make_unique<emprise_model>();
        m->model = std::make_unique<emprise::Model>(opt);
        m->name = m->model->backend_name();
        m->tokenizer.tok = m->model->tokenizer();
        *out = m.release();
    });
}

const emprise_tokenizer* emprise_model_tokenizer(const emprise_model* m) {
    return m && m->tokenizer.tok ? &m->tokenizer : nullptr;
}

emprise_status emprise_tokenizer_open(const char* path, emprise_tokenizer** out) {
    if (!path || !out) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    *out = nullptr;
    return guarded([&] {
        auto t = std::make_unique<emprise_tokenizer>();
        t->file = std::make_unique<emprise::Gguf>(path);
        try {
            t->owned = std::make_unique<emprise::Tokenizer>(*t->file);
        } catch (const std::runtime_error& e) {
            throw std::invalid_argument(e.what());  // a file without a usable tokenizer
        }
        t->tok = t->owned.get();
        *out = t.release();
    });
}

void emprise_tokenizer_close(emprise_tokenizer* t) {
    if (t && t->owned) delete t;  // a model's view is owned by the model
}

emprise_status emprise_tokenizer_encode(const emprise_tokenizer* t, const char* text, size_t len, int parse_special,
                                        int* ids, size_t cap, size_t* n) {
    if (!t || !t->tok || (!text && len) || (!ids && cap) || !n) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded_input([&] {
        const auto v = t->tok->encode(std::string(text ? text : "", len), parse_special != 0);
        std::copy(v.begin(), v.begin() + static_cast<std::ptrdiff_t>(std::min(cap, v.size())), ids);
        *n = v.size();
    });
}

emprise_status emprise_tokenizer_decode(const emprise_tokenizer* t, int token, char* out, size_t cap, size_t* n) {
    if (!t || !t->tok || (!out && cap) || !n) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded_input([&] {
        const std::string s = t->tok->decode(token);
        std::memcpy(out, s.data(), std::min(cap, s.size()));
        *n = s.size();
    });
}

emprise_status emprise_tokenizer_chat_prompt(const emprise_tokenizer* t, const char* user, size_t len, char* out,
                                             size_t cap, size_t* n) {
    if (!t || !t->tok || (!user && len) || (!out && cap) || !n) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded_input([&] {
        const std::string s = t->tok->chat_prompt(std::string(user ? user : "", len));
        std::memcpy(out, s.data(), std::min(cap, s.size()));
        *n = s.size();
    });
}

void emprise_model_close(emprise_model* m) { delete m; }

const char* emprise_model_backend_name(const emprise_model* m) { return m ? m->name.c_str() : ""; }


emprise_status emprise_model_get_info(const emprise_model* m, emprise_model_info* info) {
    if (!m || !info) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    *info = m->model->info();
    return EMPRISE_OK;
}

emprise_status emprise_model_reset(emprise_model* m) {
    if (!m) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] { m->model->reset(); });
}

emprise_status emprise_model_evaluate(emprise_model* m, int token, float* logits) {
    if (!m) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto v = m->model->evaluate(token, logits != nullptr);
        if (logits) std::memcpy(logits, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_set_trace(emprise_model* m, emprise_trace_fn fn, void* user) {
    if (!m) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] { m->model->set_trace(fn, user); });
}

emprise_status emprise_model_prefill(emprise_model* m, const int* tokens, size_t n, float* logits) {
    if (!m || (!tokens && n)) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto v = m->model->prefill(std::vector<int>(tokens, tokens + n), logits != nullptr);
        if (logits) std::memcpy(logits, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_last_hidden(emprise_model* m, float* hidden) {
    if (!m || !hidden) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto v = m->model->last_hidden();
        std::memcpy(hidden, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_last_hidden_normed(emprise_model* m, float* hidden) {
    if (!m || !hidden) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto v = m->model->last_hidden_normed();
        std::memcpy(hidden, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_evaluate_block(emprise_model* m, const int* tokens, size_t n, float* logits) {
    if (!m || !tokens || !logits) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        const auto rows = m->model->evaluate_block(std::vector<int>(tokens, tokens + n));
        for (size_t i = 0; i < rows.size(); ++i)
            std::memcpy(logits + i * rows[i].size(), rows[i].data(), rows[i].size() * sizeof(float));
    });
}

int emprise_model_has_mtp(const emprise_model* m) { return m && m->model->has_mtp() ? 1 : 0; }

emprise_status emprise_model_mtp_draft(emprise_model* m, const float* hidden, int token, size_t position,
                                       float* logits) {
    if (!m || !hidden || !logits) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    if (!m->model->has_mtp()) {
        g_error = "The model has no MTP (nextn) block";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        const size_t H = static_cast<size_t>(m->model->info().hidden);
        auto v = m->model->mtp_draft(std::vector<float>(hidden, hidden + H), token, position);
        std::memcpy(logits, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_mtp_hidden(emprise_model* m, float* hidden) {
    if (!m || !hidden) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    if (!m->model->has_mtp()) {
        g_error = "The model has no MTP (nextn) block";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto v = m->model->mtp_hidden();
        std::memcpy(hidden, v.data(), v.size() * sizeof(float));
    });
}

emprise_status emprise_model_reset_mtp(emprise_model* m) {
    if (!m) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] { m->model->reset_mtp(); });
}

emprise_status emprise_model_generate(emprise_model* m, const int* prompt, size_t prompt_len, size_t count, int* tokens,
                                      size_t* emitted, double* arrivals) {
    if (!m || (!prompt && prompt_len) || (!tokens && count) || !emitted) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        std::vector<double> arr;
        auto out = m->model->generate(std::vector<int>(prompt, prompt + prompt_len), count, &arr);
        std::memcpy(tokens, out.data(), out.size() * sizeof(int));
        if (arrivals) std::memcpy(arrivals, arr.data(), arr.size() * sizeof(double));
        *emitted = out.size();
    });
}

emprise_status emprise_model_get_profile(const emprise_model* m, emprise_model_profile* out) {
    if (!m || !out) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] { *out = m->model->profile(); });
}

emprise_status emprise_model_trace_step(emprise_model* m, int token, emprise_hip_trace_record* records, size_t cap,
                                        size_t* n) {
    if (!m || !n || (!records && cap)) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] {
        auto rec = m->model->trace_step(token);
        const size_t k = std::min(cap, rec.size());
        std::memcpy(records, rec.data(), k * sizeof(emprise_hip_trace_record));
        *n = k;
    });
}

emprise_status emprise_synth_write(const emprise_synth_config* c, const char* path) {
    if (!c || !path) {
        g_error = "null argument";
        return EMPRISE_EINVAL;
    }
    return guarded([&] { emprise::synth_write(*c, path); });
}

emprise_status emprise_synth_prompt(uint64_t seed, int vocab, size_t n, int* ids) {
    if ((!ids && n) || vocab < 1) {
        g_error = "bad argument";
        return EMPRISE_EINVAL;
    }
    emprise::synth_prompt(seed, vocab, n, ids);
    return EMPRISE_OK;
}

}  // extern "C"
