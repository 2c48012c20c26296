// emprise-chat for the HIP backend (reference src/chat.cpp): loads a qwen35 GGUF,
// greedy-decodes from token ids, prints timings, writes the --report JSON with the
// reference's fields plus the weight-bytes roofline. Text tokenisation is outside
// this build, so prompts are token ids (--prompt-ids or a seeded --synthetic-prompt).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "emprise_host.h"

namespace {
void check(emprise_status s) {
    if (s != EMPRISE_OK) throw std::runtime_error(emprise_host_last_error());
}

std::vector<int> parse_ids(const std::string& s) {
    std::vector<int> ids;
    std::stringstream ss(s);
    std::string item;
    while (std::getline(ss, item, ',')) {
        if (item.empty()) continue;
        ids.push_back(std::stoi(item));
    }
    return ids;
}

// A JSON string literal: quotes, backslashes and control characters escaped.
std::string json_string(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += static_cast<char>(c);
        } else if (c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
        } else {
            o += static_cast<char>(c);
        }
    }
    return o + "\"";
}

template <class T> std::string json_list(const std::vector<T>& v) {
    std::ostringstream o;
    o.precision(9);
    o << '[';
    for (size_t i = 0; i < v.size(); ++i) o << (i ? "," : "") << v[i];
    o << ']';
    return o.str();
}
}  // namespace

int main(int argc, char** argv) {
    try {
        std::string model, report_file, ids;
        size_t count = 32, synthetic = 0;
        uint64_t seed = 0;
        emprise_model_options opt{};
        opt.context = 4096;
        opt.fused = 1;
        opt.graph = 1;
        for (int i = 1; i < argc; ++i) {
            const std::string arg = argv[i];
            auto value = [&] {
                if (i + 1 >= argc) throw std::invalid_argument("Missing value for " + arg);
                return std::string(argv[++i]);
            };
            if (arg == "--model") model = value();
            else if (arg == "--prompt-ids") ids = value();
            else if (arg == "--synthetic-prompt") synthetic = std::stoull(value());
            else if (arg == "--seed") seed = std::stoull(value());
            else if (arg == "--report") report_file = value();
            else if (arg == "--tokens") count = std::stoull(value());
            else if (arg == "--context") opt.context = std::stoull(value());
            else if (arg == "--vram-mib") opt.weight_vram_budget = std::stoull(value()) * 1024 * 1024;
            else if (arg == "--device") opt.device = std::stoi(value());
            else if (arg == "--fast-q8") opt.quantize_activations = 1;
            else if (arg == "--unfused") opt.fused = 0;
            else if (arg == "--no-graph") opt.graph = 0;
            else if (arg == "--no-batch-prefill") opt.batch_prefill = -1;
            else if (arg == "--step-program") opt.step_program = 1;
            else if (arg == "--cpu") throw std::invalid_argument("--cpu: this build runs on the MI355X backend only");
            else throw std::invalid_argument("Unknown option: " + arg);
        }
        if (model.empty())
            throw std::invalid_argument("Usage: emprise-chat --model MODEL.gguf (--prompt-ids 1,2,3 | --synthetic-prompt N "
                                        "[--seed S]) [--tokens N] [--context N] [--fast-q8] [--report FILE] [--unfused] "
                                        "[--no-graph] [--no-batch-prefill] [--step-program]");
        opt.path = model.c_str();
        const auto start = std::chrono::steady_clock::now();
        emprise_model* m = nullptr;
        check(emprise_model_open(&opt, &m));
        emprise_model_info info{};
        check(emprise_model_get_info(m, &info));
        std::cerr << "Backend: " << emprise_model_backend_name(m) << '\n';
        std::vector<int> prompt = parse_ids(ids);
        if (synthetic) {
            prompt.resize(synthetic);
            check(emprise_synth_prompt(seed, info.vocab, synthetic, prompt.data()));
        }
        const auto loaded = std::chrono::steady_clock::now();
        std::vector<int> tokens(count);
        std::vector<double> arrivals(count);
        size_t emitted = 0;
        check(emprise_model_generate(m, prompt.data(), prompt.size(), count, tokens.data(), &emitted, arrivals.data()));
        tokens.resize(emitted);
        arrivals.resize(emitted);
        for (size_t i = 0; i < emitted; ++i) std::cout << (i ? " " : "") << tokens[i];
        std::cout << '\n';
        const double load = std::chrono::duration<double>(loaded - start).count();
        const double first = emitted ? arrivals.front() : 0.0;
        const double rate = emitted > 1 ? double(emitted - 1) / (arrivals.back() - arrivals.front()) : 0.0;
        const double roofline = rate * double(info.token_weight_bytes) / 8.0e12;
        std::cerr << "Load: " << load << "s; first token after load: " << first << "s; generated: " << emitted
                  << "; decode: " << rate << " tokens/s (" << 100.0 * roofline << "% of the 8 TB/s weight roofline)\n";
        if (!report_file.empty()) {
            // The reference's --report fields (chat.cpp:77-84), then this build's roofline.
            // text: token ids are not detokenised here. matrix_seconds / matrix_calls /
            // non_matrix_seconds are the reference's host timers around each backend call;
            // the device path replays one graph per token and has no such calls: 0.
            std::ofstream f(report_file);
            if (!f) throw std::runtime_error("Cannot write report");
            f.precision(9);
            f << "{\n  \"engine\": \"emprise mi355x\",\n  \"backend\": " << json_string(emprise_model_backend_name(m))
              << ",\n  \"model\": " << json_string(model) << ",\n  \"prompt_tokens\": " << json_list(prompt)
              << ",\n  \"output_tokens\": " << json_list(tokens) << ",\n  \"text\": \"\",\n  \"load_seconds\": " << load
              << ",\n  \"first_token_seconds\": " << first << ",\n  \"generation_tokens_per_second\": " << rate
              << ",\n  \"content_arrivals_seconds\": " << json_list(arrivals)
              << ",\n  \"matrix_seconds\": 0,\n  \"matrix_calls\": 0,\n  \"non_matrix_seconds\": 0"
              << ",\n  \"context\": " << opt.context
              << ",\n  \"quantized_activations\": " << (opt.quantize_activations ? "true" : "false")
              << ",\n  \"fused_ffn\": " << (opt.fused ? "true" : "false")
              << ",\n  \"token_weight_bytes\": " << info.token_weight_bytes
              << ",\n  \"hbm_roofline_fraction\": " << roofline << "\n}\n";
        }
        emprise_model_close(m);
    } catch (const std::exception& e) {
        std::cerr << "Error: " << e.what() << '\n';
        return 1;
    }
}
