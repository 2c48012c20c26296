// qwen35 decode graph on the HIP backend: the reference's Model (include/emprise/
// model.hpp:26-55, src/model.cpp) with its device path (evaluate_device,
// model.cpp:422-472) extended so attention, the embedding row and the greedy pick also
// stay on the device, and the whole step replays as one hipGraph.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "emprise_host.h"
#include "gguf.hpp"
#include "hip_backend.hpp"
#include "tokenizer.hpp"

namespace emprise {

struct ModelOptions {
    std::string path;
    size_t context = 4096;
    int device = 0;
    uint64_t weight_vram_budget = 0;
    bool quantize_activations = false;
    bool fused = true;
    bool graph = true;
    // prompts of at least this many tokens prefill in batches (GEMM projections); 0 = never
    size_t batch_prefill_min = 64;
};

class Model {
public:
    explicit Model(const ModelOptions& options);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    std::string backend_name() const { return backend_->name(); }
    // Model::tokenizer (model.hpp:33): null when the file has no qwen35 GPT-2 BPE
    // tokenizer (tokenizer_error() says why); the reference requires one to load
    const Tokenizer* tokenizer() const { return tokenizer_.get(); }
    const std::string& tokenizer_error() const { return tokenizer_error_; }
    emprise_model_info info() const { return info_; }
    void reset();
    std::vector<float> evaluate(int token, bool want_logits = true);
    void set_trace(emprise_trace_fn fn, void* user) {
        trace_fn_ = fn;
        trace_user_ = user;
    }
    std::vector<float> last_hidden();
    std::vector<emprise_hip_trace_record> trace_step(int token);
    emprise_model_profile profile() const;
    // prefill + greedy loop; arrivals[i] = seconds from the first launch to token i
    std::vector<int> generate(const std::vector<int>& prompt, size_t count, std::vector<double>* arrivals);
    // Model::prefill: tokens from the current position on; the last one's logits
    std::vector<float> prefill(const std::vector<int>& tokens, bool want_logits = true);
    // Model::evaluate_block (model.cpp:274-354, every position's logits): the tokens from
    // the current position on, in order; one row of logits per token
    std::vector<std::vector<float>> evaluate_block(const std::vector<int>& tokens);
    // Model::last_hidden (model.cpp:483): the last residual through the output norm
    // (last_hidden() above is last_hidden_raw)
    std::vector<float> last_hidden_normed();
    // The MTP (next-n) draft head, Model::mtp_draft / mtp_hidden / reset_mtp
    // (model.cpp:376-397, :485-487), when the file has the block
    bool has_mtp() const { return mtp_.present; }
    std::vector<float> mtp_draft(const std::vector<float>& hidden, int token, size_t position);
    std::vector<float> mtp_hidden();
    void reset_mtp() { mtp_.length = 0; }

private:
    struct Layer {
        bool recurrent = false;
        emprise_weight attn_norm = 0, post_norm = 0, gate = 0, up = 0, down = 0;
        emprise_weight qkv = 0, zgate = 0, alpha = 0, beta = 0, out = 0, conv = 0, ssm_a = 0, dt = 0, ssm_norm = 0;
        emprise_weight q = 0, k = 0, v = 0, o = 0, q_norm = 0, k_norm = 0;
        emprise_dev conv_state = 0, rec_state = 0, keys = 0, values = 0;
    };
    emprise_weight upload(const std::string& name, uint64_t cols, uint64_t rows);
    emprise_weight upload_vector(const std::string& name, uint64_t n);
    // one position, reading token/position from dev_state_; `traced`: eager, with the
    // trace hook called at the reference's points
    void enqueue_step(bool logits, bool traced = false);
    void emit(const char* name, emprise_dev src, uint64_t n, std::vector<float>* keep = nullptr);
    // positions [start, start + count) of the tokens at dev_prompt_ in batches; with
    // logits, every position's output-head row is appended to it (count x vocab)
    void prefill_batched(size_t start, size_t count, std::vector<float>* logits = nullptr);
    void set_state(int position, int token, int prompt_len);
    // evaluates seq from position 0 (no logits), leaving position_ = seq.size()
    void replay(const std::vector<int>& seq);
    emprise_graph step_graph(bool logits);

    ModelOptions opt_;
    std::unique_ptr<Gguf> gguf_;
    std::unique_ptr<Tokenizer> tokenizer_;
    std::string tokenizer_error_;
    std::unique_ptr<HipBackend> backend_;
    emprise_model_info info_{};
    std::vector<Layer> layers_;
    emprise_weight embd_ = 0, output_ = 0, output_norm_ = 0;
    emprise_dev x_[2] = {0, 0}, delta_attn_ = 0, delta_ffn_ = 0, norm_ = 0, tmp_ = 0, qkv_ = 0, attn_out_ = 0, logits_ = 0;
    emprise_dev dev_state_ = 0, dev_next_ = 0, dev_prompt_ = 0, dev_history_ = 0;
    emprise_dev hid_ = 0;  // the stream after the last position evaluated with logits
    emprise_trace_fn trace_fn_ = nullptr;
    void* trace_user_ = nullptr;
    size_t position_ = 0;
    // Model::profile: positions evaluated and decode steps run since open, and the per-step
    // kernel time by kind (ms) from the last traced step
    uint64_t evaluated_ = 0, decode_steps_ = 0, traced_steps_ = 0;
    double step_matrix_ms_ = 0, step_norm_ms_ = 0, step_attention_ms_ = 0, step_recurrent_ms_ = 0, step_other_ms_ = 0;
    emprise_graph graph_full_ = 0, graph_prefill_ = 0;
    // batched prefill buffers, sized for pf_rows_ tokens on first use
    size_t pf_rows_ = 0;
    emprise_dev pf_x_ = 0, pf_xn_ = 0, pf_a_ = 0, pf_b_ = 0, pf_c_ = 0, pf_logits_ = 0;
    bool have_graph_full_ = false, have_graph_prefill_ = false;
    // the MTP block: its weights (an attention layer + FFN in `layer`), its own K/V cache
    // of `length` rows, and buffers: cat = [enorm(e) | hnorm(h)], cur = eh_proj(cat), x =
    // the block's output (Model::mtp_hidden), in = the caller's hidden, ctl = {cache row,
    // rotary position, token}
    struct Mtp {
        bool present = false;
        emprise_weight enorm = 0, hnorm = 0, eh = 0, head_norm = 0;
        Layer layer;
        size_t length = 0;
        emprise_dev cat = 0, cur = 0, x = 0, in = 0, ctl = 0;
    } mtp_;

};

}  // namespace emprise
