// C++ face of the HIP C ABI for the host: the device half of the reference's
// emprise::Backend (include/emprise/backend.hpp:55-68) plus the fused and graph calls.
// Status codes become the reference's exception types (invalid_argument for shapes,
// runtime_error otherwise, cuda.cpp:49-51).
#pragma once
#include <stdexcept>
#include <string>
#include <vector>
#include <initializer_list>

#include "emprise_hip.h"

namespace emprise {

inline void hip_check(emprise_status s, const char* what) {
    if (s == EMPRISE_OK) return;
    const std::string msg = std::string(what) + ": " + emprise_hip_last_error();
    if (s == EMPRISE_EINVAL) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

class HipBackend {
public:
    HipBackend(int device, uint64_t budget, bool q8) { hip_check(emprise_hip_create(device, budget, q8 ? 1 : 0, &h_), "create"); }
    ~HipBackend() { emprise_hip_destroy(h_); }
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;
    emprise_hip* get() const { return h_; }

    std::string name() const { return emprise_hip_name(h_); }
    bool device_path() const { return true; }
    uint64_t device_capacity() const { return emprise_hip_capacity(h_); }
    emprise_dev dev_alloc(size_t bytes) {
        emprise_dev d = 0;
        hip_check(emprise_hip_alloc(h_, bytes, &d), "dev_alloc");
        return d;
    }
    void dev_free(emprise_dev d) { hip_check(emprise_hip_free(h_, d), "dev_free"); }
    void dev_upload(emprise_dev d, const void* src, size_t n) { hip_check(emprise_hip_upload(h_, d, src, n), "dev_upload"); }
    void dev_download(void* dst, emprise_dev s, size_t n) { hip_check(emprise_hip_download(h_, dst, s, n), "dev_download"); }
    void dev_fill(emprise_dev d, float v, size_t n) { hip_check(emprise_hip_fill(h_, d, v, n), "fill"); }
    emprise_weight resident(uint32_t type, uint64_t cols, uint64_t rows, const void* data, size_t len) {
        emprise_weight w = 0;
        hip_check(emprise_hip_upload_weight(h_, type, cols, rows, data, len, &w), "upload weights");
        return w;
    }
    void dev_rmsnorm(emprise_dev x, emprise_weight w, emprise_dev out, int n, float eps) {
        hip_check(emprise_hip_rmsnorm(h_, x, w, out, n, eps), "rmsnorm");
    }
    void dev_add(emprise_dev x, emprise_dev y, int n) { hip_check(emprise_hip_add(h_, x, y, n), "add"); }
    void dev_linear(emprise_weight w, emprise_dev x, emprise_dev y) { hip_check(emprise_hip_linear(h_, w, x, y), "linear"); }
    void dev_linear_many(int n, const emprise_weight* w, emprise_dev x, const emprise_dev* y) {
        hip_check(emprise_hip_linear_many(h_, n, w, x, y), "linear_many");
    }
    void dev_linear_norm(const emprise_hip_input& in, int n, const emprise_weight* w, const emprise_dev* y) {
        hip_check(emprise_hip_linear_norm(h_, &in, n, w, y), "linear_norm");
    }
    void dev_ffn(const emprise_hip_input* in, emprise_dev x, emprise_weight g, emprise_weight u, emprise_weight d, emprise_dev y) {
        hip_check(emprise_hip_feed_forward(h_, in, x, g, u, d, y), "feed_forward");
    }
    void dev_recurrent(const emprise_hip_recurrent_params& p, const emprise_hip_input* in, emprise_dev x, emprise_dev y) {
        hip_check(emprise_hip_recurrent(h_, &p, in, x, y), "recurrent");
    }
    void dev_attention(const emprise_hip_attention_params& p, emprise_dev qkv, emprise_dev out) {
        hip_check(emprise_hip_attention(h_, &p, qkv, out), "attention");
    }
    void dev_attention_batch(const emprise_hip_attention_params& p, emprise_dev qkv, int count, uint64_t stride,
                             int first, emprise_dev out, uint64_t out_stride) {
        hip_check(emprise_hip_attention_batch(h_, &p, qkv, count, stride, first, out, out_stride), "attention_batch");
    }
    void dev_embed(emprise_weight w, emprise_dev token, emprise_dev out) { hip_check(emprise_hip_embed(h_, w, token, out), "embed"); }
    void dev_embed_rows(emprise_weight w, emprise_dev tokens, int count, emprise_dev out) {
        hip_check(emprise_hip_embed_rows(h_, w, tokens, count, out), "embed_rows");
    }
    void dev_rmsnorm_rows(emprise_dev x, emprise_weight w, emprise_dev out, int n, int rows, float eps) {
        hip_check(emprise_hip_rmsnorm_rows(h_, x, w, out, n, rows, eps), "rmsnorm_rows");
    }
    void dev_add_rmsnorm_rows(emprise_dev x, emprise_dev delta, emprise_weight w, emprise_dev out, int n, int rows,
                              float eps) {
        hip_check(emprise_hip_add_rmsnorm_rows(h_, x, delta, w, out, n, rows, eps), "add_rmsnorm_rows");
    }
    void dev_linear_batch(emprise_weight w, emprise_dev x, uint64_t ldx, emprise_dev y, uint64_t ldy, int k) {
        hip_check(emprise_hip_linear_batch_strided(h_, w, x, ldx, y, ldy, k), "linear_batch");
    }
    void dev_linear_batch_many(std::initializer_list<emprise_weight> ws, emprise_dev x, uint64_t ldx, emprise_dev y,
                               uint64_t ldy, int k) {
        const std::vector<emprise_weight> w(ws);
        hip_check(emprise_hip_linear_batch_many(h_, static_cast<int>(w.size()), w.data(), x, ldx, y, ldy, k),
                  "linear_batch_many");
    }
    void dev_ffn_gate_up_batch(emprise_weight gate, emprise_weight up, emprise_dev x, uint64_t ldx, emprise_dev y,
                               uint64_t ldy, int k) {
        hip_check(emprise_hip_ffn_gate_up_batch(h_, gate, up, x, ldx, y, ldy, k), "ffn_gate_up_batch");
    }
    void dev_swiglu(emprise_dev gate, emprise_dev up, int n) { hip_check(emprise_hip_swiglu(h_, gate, up, n), "swiglu"); }
    void dev_delta_net(const emprise_hip_delta_net_params& p) { hip_check(emprise_hip_delta_net(h_, &p), "delta_net"); }
    void dev_delta_net_batch(const emprise_hip_delta_net_params& p, int count, uint64_t stride, uint64_t out_stride) {
        hip_check(emprise_hip_delta_net_batch(h_, &p, count, stride, out_stride), "delta_net_batch");
    }
    void dev_argmax(emprise_dev logits, int n, emprise_dev index) { hip_check(emprise_hip_argmax(h_, logits, n, index), "argmax"); }
    void sync() { hip_check(emprise_hip_sync(h_), "sync"); }
    void graph_begin() { hip_check(emprise_hip_graph_begin(h_), "graph_begin"); }
    emprise_graph graph_end() {
        emprise_graph g = 0;
        hip_check(emprise_hip_graph_end(h_, &g), "graph_end");
        return g;
    }
    void graph_launch(emprise_graph g) { hip_check(emprise_hip_graph_launch(h_, g), "graph_launch"); }
    void event(int slot) { hip_check(emprise_hip_event_record(h_, slot), "event"); }
    float elapsed(int a, int b) {
        float ms = 0;
        hip_check(emprise_hip_event_elapsed(h_, a, b, &ms), "elapsed");
        return ms;
    }

private:
    emprise_hip* h_ = nullptr;
};

}  // namespace emprise
