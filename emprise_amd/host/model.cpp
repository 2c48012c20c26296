// qwen35 decode graph (reference src/model.cpp) on the HIP backend.
#include "model.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace emprise {

namespace {
uint32_t type_id(WeightType t) { return static_cast<uint32_t>(t); }
}  // namespace

emprise_weight Model::upload(const std::string& name, uint64_t cols, uint64_t rows) {
    const Tensor& t = gguf_->tensor(name);
    if (t.shape.size() != 2 || t.shape[0] != cols || (rows && t.shape[1] != rows))
        throw std::runtime_error("Expected matrix: " + name);
    info_.weight_bytes += t.bytes;
    return backend_->resident(type_id(t.type), t.shape[0], t.shape[1], gguf_->data(t), t.bytes);
}

// Small parameters (model.cpp:80-89) are decoded to FP32 on the host once, like the
// reference's parameter cache, and kept on the device as F32 vectors.
emprise_weight Model::upload_vector(const std::string& name, uint64_t n) {
    const Tensor& t = gguf_->tensor(name);
    if (t.elements != n) throw std::runtime_error("Parameter dimensions: " + name);
    if (t.bytes > 16ull * 1024 * 1024) throw std::runtime_error("Unexpected non-matrix parameter size");
    info_.weight_bytes += t.bytes;
    std::vector<float> v(n);
    const uint8_t* p = gguf_->data(t);
    if (t.type == WeightType::f32) {
        std::memcpy(v.data(), p, n * 4);
    } else if (t.type == WeightType::f16 || t.type == WeightType::bf16) {
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t b;
            std::memcpy(&b, p + 2 * i, 2);
            uint32_t u;
            if (t.type == WeightType::bf16) {
                u = uint32_t(b) << 16;
            } else {
                // exact fp16 -> fp32 (quant.cpp:8-17)
                const uint32_t sign = uint32_t(b & 0x8000) << 16, ex = (b >> 10) & 31, frac = b & 1023;
                if (ex == 0) {
                    float f = std::ldexp(static_cast<float>(frac), -24);
                    if (sign) f = -f;
                    std::memcpy(&u, &f, 4);
                } else {
                    u = sign | (ex == 31 ? 0x7f800000u : (ex + 112) << 23) | (frac << 13);
                }
            }
            std::memcpy(&v[i], &u, 4);
        }
    } else {
        throw std::runtime_error("Unsupported parameter encoding: " + name);
    }
    return backend_->resident(EMPRISE_F32, n, 1, v.data(), n * 4);
}

Model::Model(const ModelOptions& options) : opt_(options) {
    const auto start = std::chrono::steady_clock::now();
    gguf_ = std::make_unique<Gguf>(opt_.path);
    const Gguf& g = *gguf_;
    const MetaValue* arch = g.meta("general.architecture");
    if (!arch || arch->text != "qwen35") throw std::runtime_error("Only qwen35 is implemented");
    try {
        tokenizer_ = std::make_unique<Tokenizer>(g);
    } catch (const std::exception& e) {
        tokenizer_error_ = e.what();  // token ids still work; text calls report this
    }
    auto integer = [&](const char* key) { return g.meta_int(std::string("qwen35.") + key); };
    emprise_model_info& d = info_;
    d.hidden = integer("embedding_length");
    const MetaValue* nextn = g.meta("qwen35.nextn_predict_layers");
    d.layers = integer("block_count") - (nextn ? static_cast<int>(nextn->number) : 0);
    d.heads = integer("attention.head_count");
    d.kv_heads = integer("attention.head_count_kv");
    d.head_dim = integer("attention.key_length");
    d.rotary = integer("rope.dimension_count");
    d.key_heads = integer("ssm.group_count");
    d.value_heads = integer("ssm.time_step_rank");
    d.state_dim = integer("ssm.state_size");
    d.conv_width = integer("ssm.conv_kernel");
    d.eos = g.meta_int("tokenizer.ggml.eos_token_id");
    d.eps = g.meta_float("qwen35.attention.layer_norm_rms_epsilon");
    d.rope_base = g.meta_float("qwen35.rope.freq_base");
    d.context = opt_.context;
    // model.cpp:67-70
    if (std::min({d.hidden, d.layers, d.heads, d.kv_heads, d.head_dim, d.rotary, d.key_heads, d.value_heads,
                  d.state_dim, d.conv_width}) <= 0 ||
        d.heads % d.kv_heads || d.value_heads % d.key_heads || d.rotary > d.head_dim || d.rotary % 2 ||
        opt_.context == 0 || opt_.context > static_cast<size_t>(integer("context_length")))
        throw std::runtime_error("Unsupported or invalid Qwen dimensions/context");

    backend_ = std::make_unique<HipBackend>(opt_.device, opt_.weight_vram_budget, opt_.quantize_activations);
    const uint64_t H = d.hidden;
    const Tensor& emb = g.tensor("token_embd.weight");
    if (emb.shape.size() != 2 || emb.shape[0] != H) throw std::runtime_error("token_embd shape");
    d.vocab = static_cast<int>(emb.shape[1]);
    embd_ = upload("token_embd.weight", H, 0);
    output_ = upload("output.weight", H, static_cast<uint64_t>(d.vocab));  // required: no tied fallback (model.cpp:252)
    output_norm_ = upload_vector("output_norm.weight", H);
    const uint64_t kd = uint64_t(d.key_heads) * d.state_dim, vd = uint64_t(d.value_heads) * d.state_dim;
    const uint64_t ch = 2 * kd + vd, qd = uint64_t(d.heads) * d.head_dim * 2, kvd = uint64_t(d.kv_heads) * d.head_dim;
    uint64_t per_token = encoded_bytes(emb.type, H) + g.tensor("output.weight").bytes + g.tensor("output_norm.weight").bytes;
    layers_.resize(static_cast<size_t>(d.layers));
    for (int l = 0; l < d.layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Layer& L = layers_[static_cast<size_t>(l)];
        L.recurrent = g.has(p + "ssm_a");  // layer type from its tensors (model.cpp:75-78)
        L.attn_norm = upload_vector(p + "attn_norm.weight", H);
        L.post_norm = upload_vector(p + "post_attention_norm.weight", H);
        const Tensor& fg = g.tensor(p + "ffn_gate.weight");
        if (l == 0) d.ffn = static_cast<int>(fg.shape.at(1));
        if (fg.shape.size() != 2 || static_cast<int>(fg.shape[1]) != d.ffn) throw std::runtime_error("FFN dimensions");
        L.gate = upload(p + "ffn_gate.weight", H, d.ffn);
        L.up = upload(p + "ffn_up.weight", H, d.ffn);
        L.down = upload(p + "ffn_down.weight", d.ffn, H);
        std::vector<std::string> names = {"attn_norm.weight", "post_attention_norm.weight", "ffn_gate.weight",
                                          "ffn_up.weight", "ffn_down.weight"};
        if (L.recurrent) {
            L.qkv = upload(p + "attn_qkv.weight", H, ch);
            L.zgate = upload(p + "attn_gate.weight", H, vd);
            L.alpha = upload(p + "ssm_alpha.weight", H, d.value_heads);
            L.beta = upload(p + "ssm_beta.weight", H, d.value_heads);
            L.out = upload(p + "ssm_out.weight", vd, H);
            L.conv = upload_vector(p + "ssm_conv1d.weight", ch * d.conv_width);
            L.ssm_a = upload_vector(p + "ssm_a", d.value_heads);
            L.dt = upload_vector(p + "ssm_dt.bias", d.value_heads);
            L.ssm_norm = upload_vector(p + "ssm_norm.weight", d.state_dim);
            L.conv_state = backend_->dev_alloc(ch * d.conv_width * 4);
            L.rec_state = backend_->dev_alloc(vd * d.state_dim * 4);
            names.insert(names.end(), {"attn_qkv.weight", "attn_gate.weight", "ssm_alpha.weight", "ssm_beta.weight",
                                       "ssm_out.weight", "ssm_conv1d.weight", "ssm_a", "ssm_dt.bias", "ssm_norm.weight"});
        } else {
            L.q = upload(p + "attn_q.weight", H, qd);
            L.k = upload(p + "attn_k.weight", H, kvd);
            L.v = upload(p + "attn_v.weight", H, kvd);
            L.o = upload(p + "attn_output.weight", uint64_t(d.heads) * d.head_dim, H);
            L.q_norm = upload_vector(p + "attn_q_norm.weight", d.head_dim);
            L.k_norm = upload_vector(p + "attn_k_norm.weight", d.head_dim);
            L.keys = backend_->dev_alloc(opt_.context * kvd * 4);
            L.values = backend_->dev_alloc(opt_.context * kvd * 4);
            names.insert(names.end(), {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                                       "attn_q_norm.weight", "attn_k_norm.weight"});
        }
        for (const auto& n : names) per_token += g.tensor(p + n).bytes;
    }
    d.token_weight_bytes = per_token;
    // the MTP block after the main layers, named blk.<layers> (blk.32 at the 9B shape,
    // the name model.cpp:378-392 uses); not part of a decode step's weights
    const std::string mp = "blk." + std::to_string(d.layers) + ".";
    if (g.has(mp + "nextn.eh_proj.weight")) {
        Mtp& M = mtp_;
        Layer& L = M.layer;
        M.eh = upload(mp + "nextn.eh_proj.weight", 2 * H, H);
        M.enorm = upload_vector(mp + "nextn.enorm.weight", H);
        M.hnorm = upload_vector(mp + "nextn.hnorm.weight", H);
        M.head_norm = upload_vector(mp + "nextn.shared_head_norm.weight", H);
        L.attn_norm = upload_vector(mp + "attn_norm.weight", H);
        L.post_norm = upload_vector(mp + "post_attention_norm.weight", H);
        L.q = upload(mp + "attn_q.weight", H, qd);
        L.k = upload(mp + "attn_k.weight", H, kvd);
        L.v = upload(mp + "attn_v.weight", H, kvd);
        L.o = upload(mp + "attn_output.weight", uint64_t(d.heads) * d.head_dim, H);
        L.q_norm = upload_vector(mp + "attn_q_norm.weight", d.head_dim);
        L.k_norm = upload_vector(mp + "attn_k_norm.weight", d.head_dim);
        L.gate = upload(mp + "ffn_gate.weight", H, d.ffn);
        L.up = upload(mp + "ffn_up.weight", H, d.ffn);
        L.down = upload(mp + "ffn_down.weight", d.ffn, H);
        L.keys = backend_->dev_alloc(opt_.context * kvd * 4);
        L.values = backend_->dev_alloc(opt_.context * kvd * 4);
        M.cat = backend_->dev_alloc(2 * H * 4);
        M.cur = backend_->dev_alloc(H * 4);
        M.x = backend_->dev_alloc(H * 4);
        M.in = backend_->dev_alloc(H * 4);
        M.ctl = backend_->dev_alloc(4 * sizeof(int));
        backend_->dev_fill(M.x, 0.f, H);
        M.present = true;
    }
    // activations
    const uint64_t wide = std::max<uint64_t>({H, qd + 2 * kvd, uint64_t(d.heads) * d.head_dim, vd});
    for (auto& x : x_) x = backend_->dev_alloc(H * 4);
    hid_ = backend_->dev_alloc(H * 4);
    backend_->dev_fill(hid_, 0.f, H);
    delta_attn_ = backend_->dev_alloc(H * 4);
    delta_ffn_ = backend_->dev_alloc(H * 4);
    norm_ = backend_->dev_alloc(wide * 4);
    tmp_ = backend_->dev_alloc(wide * 4);
    qkv_ = backend_->dev_alloc((qd + 2 * kvd) * 4);
    attn_out_ = backend_->dev_alloc(uint64_t(d.heads) * d.head_dim * 4);
    logits_ = backend_->dev_alloc(uint64_t(d.vocab) * 4);
    dev_state_ = backend_->dev_alloc(4 * sizeof(int));
    dev_next_ = backend_->dev_alloc(sizeof(int));
    dev_prompt_ = backend_->dev_alloc((opt_.context + 1) * sizeof(int));
    dev_history_ = backend_->dev_alloc((opt_.context + 1) * sizeof(int));
    reset();
    // one eager step sizes every backend scratch buffer before any graph capture
    set_state(0, 0, 0);
    enqueue_step(true);
    backend_->sync();
    backend_->dev_fill(hid_, 0.f, static_cast<size_t>(H));
    reset();
    d.load_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
}

Model::~Model() = default;

void Model::reset() {
    for (const Layer& L : layers_) {
        if (!L.recurrent) continue;
        const uint64_t kd = uint64_t(info_.key_heads) * info_.state_dim, vd = uint64_t(info_.value_heads) * info_.state_dim;
        backend_->dev_fill(L.conv_state, 0.f, (2 * kd + vd) * info_.conv_width);
        backend_->dev_fill(L.rec_state, 0.f, vd * info_.state_dim);
    }
    position_ = 0;
    set_state(0, 0, 0);
}

void Model::set_state(int position, int token, int prompt_len) {
    const int s[4] = {position, token, prompt_len, 0};
    backend_->dev_upload(dev_state_, s, sizeof s);
}

// One position. Token and position come from dev_state_ = {position, token,
// prompt_len}; the last call advances them on the device.
// Copies n floats of src to the host and calls the trace hook with them under `name` at
// the current position (ModelOptions::trace, model.cpp:118-120).
void Model::emit(const char* name, emprise_dev src, uint64_t n, std::vector<float>* keep) {
    std::vector<float> local;
    std::vector<float>& v = keep ? *keep : local;
    v.resize(static_cast<size_t>(n));
    backend_->dev_download(v.data(), src, n * 4);
    trace_fn_(trace_user_, position_, name, v.data(), n);
}

void Model::enqueue_step(bool logits, bool traced) {
    HipBackend& b = *backend_;
    const emprise_model_info& d = info_;
    const int H = d.hidden;
    const emprise_dev pos = dev_state_, token = dev_state_ + sizeof(int);
    const uint64_t qd = uint64_t(d.heads) * d.head_dim * 2, kvd = uint64_t(d.kv_heads) * d.head_dim;
    auto recurrent_params = [&](const Layer& L) {
        emprise_hip_recurrent_params p{};
        p.qkv_w = L.qkv;
        p.gate_w = L.zgate;
        p.alpha_w = L.alpha;
        p.beta_w = L.beta;
        p.out_w = L.out;
        p.conv = L.conv;
        p.ssm_a = L.ssm_a;
        p.dt = L.dt;
        p.norm = L.ssm_norm;
        p.key_heads = d.key_heads;
        p.value_heads = d.value_heads;
        p.state_dim = d.state_dim;
        p.conv_width = d.conv_width;
        p.eps = d.eps;
        p.conv_state = L.conv_state;
        p.rec_state = L.rec_state;
        return p;
    };
    auto attention_params = [&](const Layer& L) {
        emprise_hip_attention_params p{};
        p.heads = d.heads;
        p.kv_heads = d.kv_heads;
        p.head_dim = d.head_dim;
        p.rotary = d.rotary;
        p.context = static_cast<int>(opt_.context);
        p.eps = d.eps;
        p.rope_base = d.rope_base;
        p.q_norm = L.q_norm;
        p.k_norm = L.k_norm;
        p.keys = L.keys;
        p.values = L.values;
        p.position = pos;
        return p;
    };
    const emprise_dev qkv_parts[3] = {qkv_, qkv_ + qd * 4, qkv_ + (qd + kvd) * 4};

    b.dev_embed(embd_, token, x_[0]);
    if (opt_.fused) {
        // The residual adds and RMSNorms ride in the projections' prologues:
        // x_next = x + delta; input = rms(x_next) * norm (model.cpp:217, :226-228, :243, :249).
        int cur = 0;
        emprise_dev pending = 0;
        std::vector<float> xs, ds;  // traced: the stream and the feed-forward output
        for (size_t l = 0; l < layers_.size(); ++l) {
            const Layer& L = layers_[l];
            const std::string n = std::to_string(l);
            emprise_hip_input in{x_[cur], pending, pending ? x_[cur ^ 1] : 0, L.attn_norm, d.eps};
            if (pending) cur ^= 1;
            if (L.recurrent) {
                const auto p = recurrent_params(L);
                b.dev_recurrent(p, &in, 0, delta_attn_);
            } else {
                const emprise_weight w[3] = {L.q, L.k, L.v};
                b.dev_linear_norm(in, 3, w, qkv_parts);
                b.dev_attention(attention_params(L), qkv_, attn_out_);
                b.dev_linear(L.o, attn_out_, delta_attn_);
            }
            // x_[cur] now holds the block's input stream (its first projection wrote it)
            if (traced) {
                b.dev_rmsnorm(x_[cur], L.attn_norm, norm_, H, d.eps);
                emit(("attn_norm-" + n).c_str(), norm_, H);
            }
            emprise_hip_input in2{x_[cur], delta_attn_, x_[cur ^ 1], L.post_norm, d.eps};
            cur ^= 1;
            b.dev_ffn(&in2, 0, L.gate, L.up, L.down, delta_ffn_);
            pending = delta_ffn_;
            if (traced) {
                emit(("attn_residual-" + n).c_str(), x_[cur], H, &xs);
                ds.resize(static_cast<size_t>(H));
                b.dev_download(ds.data(), delta_ffn_, static_cast<uint64_t>(H) * 4);
                // the add the next projection's staging makes (one FP32 add per element)
                for (int i = 0; i < H; ++i) xs[static_cast<size_t>(i)] += ds[static_cast<size_t>(i)];
                trace_fn_(trace_user_, position_, ("l_out-" + n).c_str(), xs.data(), static_cast<uint64_t>(H));
            }
        }
        if (logits) {
            // the head's input staging writes the final stream to hid_, the hidden vector the
            // reference keeps from positions with logits only (model.cpp:247-251)
            emprise_hip_input in{x_[cur], pending, hid_, output_norm_, d.eps};
            hip_check(emprise_hip_lm_head(b.get(), &in, output_, logits_, dev_next_), "lm_head");
            if (traced) {
                b.dev_rmsnorm(hid_, output_norm_, norm_, H, d.eps);
                emit("result_norm", norm_, H);
                emit("logits", logits_, static_cast<uint64_t>(d.vocab));
            }
        }
    } else {
        // One op per launch, in the order of evaluate_device (model.cpp:422-472).
        const emprise_dev x = x_[0];
        for (size_t l = 0; l < layers_.size(); ++l) {
            const Layer& L = layers_[l];
            const std::string n = std::to_string(l);
            b.dev_rmsnorm(x, L.attn_norm, norm_, H, d.eps);
            if (traced) emit(("attn_norm-" + n).c_str(), norm_, H);
            if (L.recurrent) {
                const auto p = recurrent_params(L);
                b.dev_recurrent(p, nullptr, norm_, tmp_);
            } else {
                b.dev_linear(L.q, norm_, qkv_parts[0]);
                b.dev_linear(L.k, norm_, qkv_parts[1]);
                b.dev_linear(L.v, norm_, qkv_parts[2]);
                b.dev_attention(attention_params(L), qkv_, attn_out_);
                b.dev_linear(L.o, attn_out_, tmp_);
            }
            b.dev_add(x, tmp_, H);
            if (traced) emit(("attn_residual-" + n).c_str(), x, H);
            b.dev_rmsnorm(x, L.post_norm, norm_, H, d.eps);
            b.dev_ffn(nullptr, norm_, L.gate, L.up, L.down, tmp_);
            b.dev_add(x, tmp_, H);
            if (traced) emit(("l_out-" + n).c_str(), x, H);
        }
        if (logits) {
            b.dev_fill(hid_, 0.f, H);
            b.dev_add(hid_, x, H);
            b.dev_rmsnorm(x, output_norm_, norm_, H, d.eps);
            if (traced) emit("result_norm", norm_, H);
            b.dev_linear(output_, norm_, logits_);
            if (traced) emit("logits", logits_, static_cast<uint64_t>(d.vocab));
            b.dev_argmax(logits_, d.vocab, dev_next_);
        }
    }
    hip_check(emprise_hip_advance(b.get(), dev_state_, dev_prompt_, logits ? dev_history_ : 0, logits ? dev_next_ : 0),
              "advance");
}

emprise_graph Model::step_graph(bool logits) {
    bool& have = logits ? have_graph_full_ : have_graph_prefill_;
    emprise_graph& g = logits ? graph_full_ : graph_prefill_;
    if (!have) {
        backend_->graph_begin();
        try {
            enqueue_step(logits);
        } catch (...) {
            emprise_graph dead = 0;
            (void)emprise_hip_graph_end(backend_->get(), &dead);
            throw;
        }
        g = backend_->graph_end();
        have = true;
    }
    return g;
}

std::vector<float> Model::evaluate(int token, bool want_logits) {
    if (position_ >= opt_.context) throw std::runtime_error("Context budget exhausted");
    if (token < 0 || token >= info_.vocab) throw std::out_of_range("Token ID");
    set_state(static_cast<int>(position_), token, 0);
    if (trace_fn_) enqueue_step(want_logits, true);
    else if (opt_.graph) backend_->graph_launch(step_graph(want_logits));
    else enqueue_step(want_logits);
    ++position_;
    ++evaluated_;
    if (want_logits) ++decode_steps_;
    std::vector<float> out;
    if (want_logits) {
        out.resize(static_cast<size_t>(info_.vocab));
        backend_->dev_download(out.data(), logits_, out.size() * 4);
    } else {
        backend_->sync();
    }
    return out;
}

std::vector<emprise_hip_trace_record> Model::trace_step(int token) {
    if (position_ >= opt_.context) throw std::runtime_error("Context budget exhausted");
    if (token < 0 || token >= info_.vocab) throw std::out_of_range("Token ID");
    set_state(static_cast<int>(position_), token, 0);
    backend_->sync();
    hip_check(emprise_hip_trace_begin(backend_->get()), "trace_begin");
    enqueue_step(true);
    std::vector<emprise_hip_trace_record> rec(4096);
    size_t n = 0;
    hip_check(emprise_hip_trace_end(backend_->get(), rec.data(), rec.size(), &n), "trace_end");
    rec.resize(n);
    // the step's kernel time by kind, for profile()
    step_matrix_ms_ = step_norm_ms_ = step_attention_ms_ = step_recurrent_ms_ = step_other_ms_ = 0;
    for (const auto& r : rec) {
        const std::string k = r.kernel;
        if (k.rfind("matvec", 0) == 0 || k.rfind("gemm", 0) == 0) step_matrix_ms_ += r.ms;
        else if (k == "rmsnorm" || k == "add_rmsnorm") step_norm_ms_ += r.ms;
        else if (k.rfind("attention", 0) == 0) step_attention_ms_ += r.ms;
        else if (k.rfind("gdn", 0) == 0 || k == "delta_conv") step_recurrent_ms_ += r.ms;
        else step_other_ms_ += r.ms;
    }
    ++traced_steps_;  // a measurement: not counted as an evaluated token or decode step
    // attention reads K and V rows 0..position of its layer
    const uint64_t kv = uint64_t(position_ + 1) * info_.kv_heads * info_.head_dim * 4 * 2;
    for (auto& r : rec)
        if (std::string(r.kernel) == "attention") r.bytes = kv;
    ++position_;
    return rec;
}

std::vector<float> Model::last_hidden() {
    std::vector<float> h(static_cast<size_t>(info_.hidden));
    backend_->dev_download(h.data(), hid_, h.size() * 4);
    return h;
}

std::vector<float> Model::last_hidden_normed() {
    const int H = info_.hidden;
    backend_->dev_rmsnorm(hid_, output_norm_, tmp_, H, info_.eps);
    std::vector<float> h(static_cast<size_t>(H));
    backend_->dev_download(h.data(), tmp_, h.size() * 4);
    return h;
}

// Model::Impl::mtp_step (model.cpp:376-397): cur = eh_proj [enorm(embed(token)) |
// hnorm(hidden)]; the block's attention (its own cache, one more row per call, rotary
// position `position`) and FFN add to cur, which is kept as mtp_hidden; logits = output
// head of the shared head norm of cur. The reference's unfused FFN (mm, silu * up, mm)
// runs here as the fused feed-forward op, the same arithmetic per element.
std::vector<float> Model::mtp_draft(const std::vector<float>& hidden, int token, size_t position) {
    const emprise_model_info& d = info_;
    if (!mtp_.present) throw std::runtime_error("The model has no MTP (nextn) block");
    if (hidden.size() != static_cast<size_t>(d.hidden)) throw std::invalid_argument("MTP hidden size");
    if (token < 0 || token >= d.vocab) throw std::out_of_range("Token ID");
    if (position >= opt_.context) throw std::invalid_argument("MTP position outside the context");
    if (mtp_.length >= opt_.context) throw std::runtime_error("MTP context budget exhausted");
    HipBackend& b = *backend_;
    Mtp& M = mtp_;
    const Layer& L = M.layer;
    const uint64_t H = d.hidden, qd = uint64_t(d.heads) * d.head_dim * 2, kvd = uint64_t(d.kv_heads) * d.head_dim;
    const int ctl[4] = {static_cast<int>(M.length), static_cast<int>(position), token, 0};
    b.dev_upload(M.ctl, ctl, sizeof ctl);
    b.dev_upload(M.in, hidden.data(), H * 4);
    b.dev_embed(embd_, M.ctl + 2 * sizeof(int), tmp_);
    b.dev_rmsnorm(tmp_, M.enorm, M.cat, static_cast<int>(H), d.eps);
    b.dev_rmsnorm(M.in, M.hnorm, M.cat + H * 4, static_cast<int>(H), d.eps);
    b.dev_linear(M.eh, M.cat, M.cur);
    const emprise_hip_input in{M.cur, 0, 0, L.attn_norm, d.eps};
    const emprise_weight w[3] = {L.q, L.k, L.v};
    const emprise_dev parts[3] = {qkv_, qkv_ + qd * 4, qkv_ + (qd + kvd) * 4};
    b.dev_linear_norm(in, 3, w, parts);
    emprise_hip_attention_params p{};
    p.heads = d.heads;
    p.kv_heads = d.kv_heads;
    p.head_dim = d.head_dim;
    p.rotary = d.rotary;
    p.context = static_cast<int>(opt_.context);
    p.eps = d.eps;
    p.rope_base = d.rope_base;
    p.q_norm = L.q_norm;
    p.k_norm = L.k_norm;
    p.keys = L.keys;
    p.values = L.values;
    p.position = M.ctl;
    p.rope_position = M.ctl + sizeof(int);
    b.dev_attention(p, qkv_, attn_out_);
    b.dev_linear(L.o, attn_out_, delta_attn_);
    const emprise_hip_input fin{M.cur, delta_attn_, M.x, L.post_norm, d.eps};
    b.dev_ffn(&fin, 0, L.gate, L.up, L.down, delta_ffn_);
    b.dev_add(M.x, delta_ffn_, static_cast<int>(H));
    const emprise_hip_input hin{M.x, 0, 0, M.head_norm, d.eps};
    b.dev_linear_norm(hin, 1, &output_, &logits_);
    ++M.length;
    std::vector<float> out(static_cast<size_t>(d.vocab));
    b.dev_download(out.data(), logits_, out.size() * 4);
    return out;
}

std::vector<float> Model::mtp_hidden() {
    if (!mtp_.present) throw std::runtime_error("The model has no MTP (nextn) block");
    std::vector<float> h(static_cast<size_t>(info_.hidden));
    backend_->dev_download(h.data(), mtp_.x, h.size() * 4);
    return h;
}

// Every position's logits (Model::evaluate_block, model.cpp:274-354, which batches the
// block's projections the same way); a single token is a decode step.
std::vector<std::vector<float>> Model::evaluate_block(const std::vector<int>& tokens) {
    if (tokens.empty()) throw std::invalid_argument("Empty block");
    if (tokens.size() > opt_.context - std::min(position_, opt_.context))
        throw std::runtime_error("Context budget exhausted");
    for (int t : tokens)
        if (t < 0 || t >= info_.vocab) throw std::out_of_range("Token ID");
    std::vector<std::vector<float>> out;
    if (tokens.size() == 1) {
        out.push_back(evaluate(tokens[0], true));
        return out;
    }
    // all positions in one batched pass: every projection reads its weights once for the
    // block (the small-batch matvec up to 7 positions, the GEMM from 8), the recurrent
    // and attention steps run position by position, then the head over every row
    const size_t n = tokens.size(), start = position_;
    backend_->dev_upload(dev_prompt_ + start * sizeof(int), tokens.data(), n * sizeof(int));
    std::vector<float> flat;
    prefill_batched(start, n, &flat);
    position_ = start + n;
    evaluated_ += n;
    const size_t V = static_cast<size_t>(info_.vocab);
    out.reserve(n);
    for (size_t i = 0; i < n; ++i)
        out.emplace_back(flat.begin() + static_cast<std::ptrdiff_t>(i * V),
                         flat.begin() + static_cast<std::ptrdiff_t>((i + 1) * V));
    return out;
}

// Positions [start, start + count) of the tokens at dev_prompt_ (token of position p at
// index p), in chunks of up to kPrefillChunk
// tokens: every projection runs once per chunk as a GEMM on the matrix cores (the
// reference batches 4 positions, model.cpp:355-366; here the whole chunk), the
// projections of one input stacked into one GEMM (q|k|v; qkv|z|alpha|beta), the RMSNorms,
// residual adds and SwiGLU run over all rows at once, the GDN conv + state update runs
// as one scan over the chunk's positions (emprise_hip_delta_net_batch), and attention
// runs over the chunk at once as FP32 GEMMs with a causal softmax
// (emprise_hip_attention_batch). Op order is that of the unfused decode step.
void Model::prefill_batched(size_t start, size_t count, std::vector<float>* logits) {
    constexpr size_t kPrefillChunk = 2048;
    HipBackend& b = *backend_;
    const emprise_model_info& d = info_;
    const uint64_t H = d.hidden, kd = uint64_t(d.key_heads) * d.state_dim, vd = uint64_t(d.value_heads) * d.state_dim;
    const uint64_t ch = 2 * kd + vd, vh = d.value_heads, F = d.ffn;
    const uint64_t qd = uint64_t(d.heads) * d.head_dim * 2, kvd = uint64_t(d.kv_heads) * d.head_dim,
                   ao = uint64_t(d.heads) * d.head_dim;
    const uint64_t wa = std::max({ch + vd + 2 * vh, qd + 2 * kvd, F}), wb = std::max({vd, ao, F});
    const size_t rows = std::min(count, kPrefillChunk);
    if (pf_rows_ < rows) {
        for (emprise_dev* p : {&pf_x_, &pf_xn_, &pf_a_, &pf_b_, &pf_c_})
            if (*p) b.dev_free(*p), *p = 0;
        pf_x_ = b.dev_alloc(rows * H * 4);
        pf_xn_ = b.dev_alloc(rows * H * 4);
        pf_a_ = b.dev_alloc(rows * wa * 4);
        pf_b_ = b.dev_alloc(rows * wb * 4);
        pf_c_ = b.dev_alloc(rows * H * 4);
        pf_rows_ = rows;
    }
    for (size_t p0 = 0; p0 < count; p0 += rows) {
        const int T = static_cast<int>(std::min(rows, count - p0));
        b.dev_embed_rows(embd_, dev_prompt_ + (start + p0) * sizeof(int), T, pf_x_);
        // each residual add (model.cpp:226, :243) runs in the pass of the RMSNorm after it
        bool pending = false;  // pf_c_ holds a delta not yet added to pf_x_
        auto norm_rows = [&](emprise_weight w) {
            if (pending) b.dev_add_rmsnorm_rows(pf_x_, pf_c_, w, pf_xn_, static_cast<int>(H), T, d.eps);
            else b.dev_rmsnorm_rows(pf_x_, w, pf_xn_, static_cast<int>(H), T, d.eps);
            pending = false;
        };
        for (const Layer& L : layers_) {
            norm_rows(L.attn_norm);
            if (L.recurrent) {
                const uint64_t W = ch + vd + 2 * vh;
                b.dev_linear_batch_many({L.qkv, L.zgate, L.alpha, L.beta}, pf_xn_, H, pf_a_, W, T);
                emprise_hip_delta_net_params p{};
                p.key_heads = d.key_heads;
                p.value_heads = d.value_heads;
                p.state_dim = d.state_dim;
                p.conv_width = d.conv_width;
                p.eps = d.eps;
                p.conv = L.conv;
                p.ssm_a = L.ssm_a;
                p.dt = L.dt;
                p.norm = L.ssm_norm;
                p.conv_state = L.conv_state;
                p.rec_state = L.rec_state;
                p.qkv = pf_a_;
                p.gate = pf_a_ + ch * 4;
                p.alpha = pf_a_ + (ch + vd) * 4;
                p.beta = pf_a_ + (ch + vd + vh) * 4;
                p.out = pf_b_;
                b.dev_delta_net_batch(p, T, W, vd);
                b.dev_linear_batch(L.out, pf_b_, vd, pf_c_, H, T);
            } else {
                const uint64_t W = qd + 2 * kvd;
                b.dev_linear_batch_many({L.q, L.k, L.v}, pf_xn_, H, pf_a_, W, T);
                emprise_hip_attention_params p{};
                p.heads = d.heads;
                p.kv_heads = d.kv_heads;
                p.head_dim = d.head_dim;
                p.rotary = d.rotary;
                p.context = static_cast<int>(opt_.context);
                p.eps = d.eps;
                p.rope_base = d.rope_base;
                p.q_norm = L.q_norm;
                p.k_norm = L.k_norm;
                p.keys = L.keys;
                p.values = L.values;
                b.dev_attention_batch(p, pf_a_, T, W, static_cast<int>(start + p0), pf_b_, ao);
                b.dev_linear_batch(L.o, pf_b_, ao, pf_c_, H, T);
            }
            pending = true;
            norm_rows(L.post_norm);
            b.dev_ffn_gate_up_batch(L.gate, L.up, pf_xn_, H, pf_a_, F, T);
            b.dev_linear_batch(L.down, pf_a_, F, pf_c_, H, T);
            pending = true;
        }
        if (logits) {
            norm_rows(output_norm_);
        } else if (pending) {
            b.dev_add(pf_x_, pf_c_, static_cast<int>(T * H));
        }
        if (logits) {
            // the output norm and head over the chunk's rows, kHeadRows at a time
            constexpr int kHeadRows = 64;
            const uint64_t V = static_cast<uint64_t>(d.vocab);
            if (!pf_logits_) pf_logits_ = b.dev_alloc(kHeadRows * V * 4);
            for (int r0 = 0; r0 < T; r0 += kHeadRows) {
                const int n = std::min(kHeadRows, T - r0);
                b.dev_linear_batch(output_, pf_xn_ + static_cast<uint64_t>(r0) * H * 4, H, pf_logits_, V, n);
                const size_t at = logits->size();
                logits->resize(at + static_cast<size_t>(n) * V);
                b.dev_download(logits->data() + at, pf_logits_, static_cast<size_t>(n) * V * 4);
            }
            if (p0 + T == count) {
                // the last position's residual, as a decode step with logits leaves it
                b.dev_fill(hid_, 0.f, H);
                b.dev_add(hid_, pf_x_ + static_cast<uint64_t>(T - 1) * H * 4, static_cast<int>(H));
            }
        }
    }
}

std::vector<int> Model::generate(const std::vector<int>& prompt, size_t count, std::vector<double>* arrivals) {
    if (prompt.empty()) throw std::invalid_argument("Empty prompt");
    if (prompt.size() > opt_.context || count > opt_.context - prompt.size())
        throw std::invalid_argument("Prompt plus output exceeds context budget");
    for (int t : prompt)
        if (t < 0 || t >= info_.vocab) throw std::out_of_range("Token ID");
    reset();
    if (!count) return {};
    const int n = static_cast<int>(prompt.size());
    backend_->dev_upload(dev_prompt_, prompt.data(), prompt.size() * sizeof(int));
    backend_->event(0);
    // prefill: every prompt position but the last skips the output head
    if (opt_.batch_prefill_min && static_cast<size_t>(n - 1) >= opt_.batch_prefill_min) {
        prefill_batched(0, static_cast<size_t>(n - 1));
        set_state(n - 1, prompt[static_cast<size_t>(n - 1)], n);
    } else {
        set_state(0, prompt[0], n);
        for (int i = 0; i + 1 < n; ++i) {
            if (opt_.graph) backend_->graph_launch(step_graph(false));
            else enqueue_step(false);
        }
    }
    // then count steps with the output head: the first one reads the last prompt
    // token, each later one the previous greedy pick (model.cpp:497-502). The reference
    // evaluates count-1 tokens after the prompt; the last launch here only produces
    // the count-th pick.
    for (size_t i = 0; i < count; ++i) {
        if (opt_.graph) backend_->graph_launch(step_graph(true));
        else enqueue_step(true);
        backend_->event(static_cast<int>(1 + i));
    }
    backend_->sync();
    evaluated_ += static_cast<uint64_t>(n - 1) + count;
    decode_steps_ += count;
    std::vector<int> hist(count);
    backend_->dev_download(hist.data(), dev_history_ + static_cast<uint64_t>(n - 1) * sizeof(int), count * sizeof(int));
    std::vector<int> out;
    for (size_t i = 0; i < count; ++i) {
        if (hist[i] == info_.eos) break;  // model.cpp:500
        out.push_back(hist[i]);
        if (arrivals) arrivals->push_back(backend_->elapsed(0, static_cast<int>(1 + i)) * 1e-3);
    }
    // The reference evaluates the prompt and every emitted token but the last
    // (model.cpp:497-502): n + count - 1 positions, and fewer when EOS stops it. The
    // device ran all count steps (the count-th only picked the last token), so without
    // EOS its state is the reference's. After EOS it has moved past the reference's
    // stopping point; the state is rebuilt by evaluating the prompt and the emitted
    // tokens again (n + emitted positions, as the reference leaves it).
    if (out.size() == count) {
        position_ = static_cast<size_t>(n) + count - 1;
    } else {
        std::vector<int> seq(prompt);
        seq.insert(seq.end(), out.begin(), out.end());
        replay(seq);
    }
    return out;
}

// Leaves the model as if every token of seq had been evaluated in order from position 0
// (no logits): the prompt path of generate over the whole sequence.
void Model::replay(const std::vector<int>& seq) {
    reset();
    prefill(seq, false);
}

// Model::prefill (model.cpp:355-366): the tokens from the current position on, all but
// the last in batches (GEMM projections) or as replayed steps without the output head,
// then the last one as a decode step; returns its logits (empty when not wanted).
std::vector<float> Model::prefill(const std::vector<int>& tokens, bool want_logits) {
    if (tokens.empty()) throw std::invalid_argument("Empty prompt");
    if (tokens.size() > opt_.context - std::min(position_, opt_.context))
        throw std::runtime_error("Context budget exhausted");
    for (int t : tokens)
        if (t < 0 || t >= info_.vocab) throw std::out_of_range("Token ID");
    const size_t n = tokens.size(), start = position_;
    backend_->dev_upload(dev_prompt_ + start * sizeof(int), tokens.data(), n * sizeof(int));
    if (n > 1) {
        if (opt_.batch_prefill_min && n - 1 >= opt_.batch_prefill_min) {
            prefill_batched(start, n - 1);
        } else {
            set_state(static_cast<int>(start), tokens[0], static_cast<int>(start + n));
            for (size_t i = 0; i + 1 < n; ++i) {
                if (opt_.graph) backend_->graph_launch(step_graph(false));
                else enqueue_step(false);
            }
        }
        position_ = start + n - 1;
        evaluated_ += n - 1;
    }
    return evaluate(tokens[n - 1], want_logits);
}

// Model::profile (model.hpp:21-25); see emprise_model_get_profile in emprise_host.h.
emprise_model_profile Model::profile() const {
    emprise_model_profile p{};
    p.evaluated_tokens = evaluated_;
    p.decode_steps = decode_steps_;
    p.traced_steps = traced_steps_;
    // projections per decode step, one per weight as the reference counts them (mms and mm,
    // model.cpp:90-115; feed_forward as 3, model.cpp:236)
    uint64_t per_step = 1;  // the output head
    for (const Layer& L : layers_) per_step += L.recurrent ? 5 + 3 : 4 + 3;
    p.matrix_calls = per_step * decode_steps_;
    if (traced_steps_) {
        const double s = 1e-3 * static_cast<double>(decode_steps_);
        p.matrix_seconds = step_matrix_ms_ * s;
        p.norm_seconds = step_norm_ms_ * s;
        p.attention_seconds = step_attention_ms_ * s;
        p.recurrent_seconds = step_recurrent_ms_ * s;
        p.non_matrix_seconds = (step_norm_ms_ + step_attention_ms_ + step_recurrent_ms_ + step_other_ms_) * s;
    }
    return p;
}

}  // namespace emprise
