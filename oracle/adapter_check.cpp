// Test infrastructure, not product: a harness that runs the reference-side adapter of
// INTEGRATION.md section 1 (the reference's Backend interface over libemprise_hip.so)
// next to the reference's own cpu_backend(). oracle/Makefile links it, the adapter text
// extracted from INTEGRATION.md, the reference's backend.cpp / quant.cpp / gguf.cpp and
// libemprise_hip.so into _ref/libemprise_adapter.so; only tests/test_gpu_adapter.py
// loads it.
//
// The call sequence is the reference's for a recurrent layer: its prefill calls
// Backend::delta_net once per prompt position on the layer's slot (model.cpp:301-306,
// :162-183), and decode then calls recurrent_block with the same slot (model.cpp:431-440),
// which continues from the state the prefill left (cuda.cpp:934-984 keeps it per slot).
#include "emprise/backend.hpp"

#include <cmath>
#include <cstdio>
#include <exception>
#include <random>
#include <string>
#include <vector>

namespace emprise {
std::unique_ptr<Backend> hip_backend(uint64_t weight_budget, bool quantize_activations);
}

using namespace emprise;

namespace {

std::vector<float> f32_tensor(Gguf& g, const std::string& name) {
    const Tensor& t = g.tensor(name);
    std::vector<std::byte> raw(static_cast<size_t>(t.bytes));
    g.read(t, 0, raw);
    std::vector<float> v(static_cast<size_t>(t.elements));
    dequantize(t.type, raw, v);
    return v;
}

// Seeded standard-normal values (Box-Muller over mt19937 words, so the inputs do not
// depend on the standard library's distribution code).
struct Normal {
    std::mt19937 rng;
    explicit Normal(uint32_t seed) : rng(seed) {}
    float operator()() {
        const double u1 = (rng() + 1.0) / 4294967297.0, u2 = rng() / 4294967296.0;
        return static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

}  // namespace

extern "C" {

// Runs `positions` delta_net calls (random qkv/gate/alpha/beta, seeded) on slot `layer`
// of the HIP adapter and of cpu_backend(), then one recurrent_block of that layer (random
// input x) on the same slot. Outputs: dn_* positions x value_heads*state_dim floats,
// rb_* hidden floats, where hidden is the layer's input width. Returns 0, or 1 with a
// message in err.
int adapter_recurrent_check(const char* path, uint64_t budget, int layer, int key_heads, int value_heads,
                            int state_dim, int conv_width, float eps, int positions, uint32_t seed, float* dn_hip,
                            float* dn_cpu, float* rb_hip, float* rb_cpu, uint64_t hidden, char* err, size_t errlen) {
    try {
        Gguf g(path);
        auto hip = hip_backend(budget, false);
        auto cpu = cpu_backend();
        const std::string p = "blk." + std::to_string(layer) + ".";
        const auto conv = f32_tensor(g, p + "ssm_conv1d.weight"), a = f32_tensor(g, p + "ssm_a");
        const auto dt = f32_tensor(g, p + "ssm_dt.bias"), nw = f32_tensor(g, p + "ssm_norm.weight");
        const size_t kd = size_t(key_heads) * state_dim, vd = size_t(value_heads) * state_dim, ch = 2 * kd + vd;
        // the CPU backend's state lives in these spans; the adapter is handed its own pair,
        // which it uses only where it falls back to the CPU (it keeps the slot on the device)
        std::vector<float> cpu_conv(ch * conv_width), cpu_rec(vd * state_dim);
        std::vector<float> hip_conv(cpu_conv.size()), hip_rec(cpu_rec.size());
        Normal rnd(seed);
        std::vector<float> qkv(ch), gate(vd), alpha(value_heads), beta(value_heads);
        for (int t = 0; t < positions; ++t) {
            for (auto& v : qkv) v = rnd();
            for (auto& v : gate) v = rnd();
            for (auto& v : alpha) v = rnd();
            for (auto& v : beta) v = rnd();
            Backend::DeltaNet d;
            d.key_heads = key_heads;
            d.value_heads = value_heads;
            d.state_dim = state_dim;
            d.conv_width = conv_width;
            d.eps = eps;
            d.slot = layer;
            d.qkv = qkv;
            d.gate = gate;
            d.alpha = alpha;
            d.beta = beta;
            d.conv = conv;
            d.ssm_a = a;
            d.dt = dt;
            d.norm = nw;
            d.conv_state = hip_conv;
            d.rec_state = hip_rec;
            d.out = std::span<float>(dn_hip + t * vd, vd);
            hip->delta_net(g, d);
            d.conv_state = cpu_conv;
            d.rec_state = cpu_rec;
            d.out = std::span<float>(dn_cpu + t * vd, vd);
            cpu->delta_net(g, d);
        }
        std::vector<float> x(hidden);
        for (auto& v : x) v = rnd();
        Backend::RecurrentBlock b;
        b.qkv_w = &g.tensor(p + "attn_qkv.weight");
        b.gate_w = &g.tensor(p + "attn_gate.weight");
        b.alpha_w = &g.tensor(p + "ssm_alpha.weight");
        b.beta_w = &g.tensor(p + "ssm_beta.weight");
        b.out_w = &g.tensor(p + "ssm_out.weight");
        b.conv = conv;
        b.ssm_a = a;
        b.dt = dt;
        b.norm = nw;
        b.key_heads = key_heads;
        b.value_heads = value_heads;
        b.state_dim = state_dim;
        b.conv_width = conv_width;
        b.eps = eps;
        b.slot = layer;
        b.x = x;
        b.conv_state = hip_conv;
        b.rec_state = hip_rec;
        b.out = std::span<float>(rb_hip, hidden);
        hip->recurrent_block(g, b);
        b.conv_state = cpu_conv;
        b.rec_state = cpu_rec;
        b.out = std::span<float>(rb_cpu, hidden);
        cpu->recurrent_block(g, b);
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, errlen, "%s", e.what());
        return 1;
    }
}

// The reference's fallback check (tests/core.cpp:145-147) for feed_forward: layer
// `layer`'s FFN on a seeded input through the adapter and through cpu_backend().
int adapter_ffn_check(const char* path, uint64_t budget, int layer, uint32_t seed, float* y_hip, float* y_cpu,
                      uint64_t hidden, char* err, size_t errlen) {
    try {
        Gguf g(path);
        auto hip = hip_backend(budget, false);
        auto cpu = cpu_backend();
        const std::string p = "blk." + std::to_string(layer) + ".";
        const Tensor& gw = g.tensor(p + "ffn_gate.weight");
        const Tensor& uw = g.tensor(p + "ffn_up.weight");
        const Tensor& dw = g.tensor(p + "ffn_down.weight");
        Normal rnd(seed);
        std::vector<float> x(hidden);
        for (auto& v : x) v = rnd();
        hip->feed_forward(g, gw, uw, dw, x, std::span<float>(y_hip, hidden));
        cpu->feed_forward(g, gw, uw, dw, x, std::span<float>(y_cpu, hidden));
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, errlen, "%s", e.what());
        return 1;
    }
}

}  // extern "C"
