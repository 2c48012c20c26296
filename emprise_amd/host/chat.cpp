// emprise-chat for the HIP backend (reference src/chat.cpp): loads a qwen35 GGUF,
// greedy-decodes from a text prompt (--prompt / --prompt-file, through the file's
// tokenizer and chat template unless --raw), token ids (--prompt-ids) or a seeded
// --synthetic-prompt, prints the output and timings, writes the --report JSON with the
// reference's fields plus the weight-bytes roofline. --tokenize prints the prompt's ids
// without touching the device (chat.cpp:47-52).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <iterator>
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

// Length of the well-formed UTF-8 sequence at s[i], or 0.
size_t utf8_length(const std::string& s, size_t i) {
    const auto b = [&](size_t k) { return static_cast<unsigned char>(s[k]); };
    const unsigned char c = b(i);
    size_t n;
    uint32_t cp;
    if (c < 0x80) return 1;
    if ((c & 0xE0) == 0xC0) n = 2, cp = c & 0x1F;
    else if ((c & 0xF0) == 0xE0) n = 3, cp = c & 0x0F;
    else if ((c & 0xF8) == 0xF0) n = 4, cp = c & 0x07;
    else return 0;
    if (i + n > s.size()) return 0;
    for (size_t k = 1; k < n; ++k) {
        if ((b(i + k) & 0xC0) != 0x80) return 0;
        cp = (cp << 6) | (b(i + k) & 0x3F);
    }
    const uint32_t min = n == 2 ? 0x80 : n == 3 ? 0x800 : 0x10000;
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return 0;
    return n;
}

// A JSON string literal: quotes, backslashes and control characters escaped, and each
// byte that is not part of well-formed UTF-8 replaced by U+FFFD (the reference writes
// its report with nlohmann::json's error_handler_t::replace, chat.cpp:85).
std::string json_string(const std::string& s) {
    std::string o = "\"";
    for (size_t i = 0; i < s.size();) {
        const unsigned char c = static_cast<unsigned char>(s[i]);
        const size_t n = utf8_length(s, i);
        if (!n) {
            o += "\xEF\xBF\xBD";
            ++i;
        } else if (c == '"' || c == '\\') {
            o += '\\';
            o += static_cast<char>(c);
            ++i;
        } else if (c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
            ++i;
        } else {
            o.append(s, i, n);
            i += n;
        }
    }
    return o + "\"";
}

// The tokenizer's text as a std::string, or an exception with the library's message.
std::string take_string(emprise_status st, const std::vector<char>& buf, size_t n) {
    check(st);
    return std::string(buf.data(), n);
}

std::vector<int> encode(const emprise_tokenizer* t, const std::string& text) {
    size_t n = 0;
    check(emprise_tokenizer_encode(t, text.data(), text.size(), 1, nullptr, 0, &n));
    std::vector<int> ids(n);
    check(emprise_tokenizer_encode(t, text.data(), text.size(), 1, ids.data(), ids.size(), &n));
    return ids;
}

std::string chat_prompt(const emprise_tokenizer* t, const std::string& user) {
    size_t n = 0;
    check(emprise_tokenizer_chat_prompt(t, user.data(), user.size(), nullptr, 0, &n));
    std::vector<char> buf(n + 1);
    return take_string(emprise_tokenizer_chat_prompt(t, user.data(), user.size(), buf.data(), buf.size(), &n), buf, n);
}

std::string decode(const emprise_tokenizer* t, int id) {
    size_t n = 0;
    check(emprise_tokenizer_decode(t, id, nullptr, 0, &n));
    std::vector<char> buf(n + 1);
    return take_string(emprise_tokenizer_decode(t, id, buf.data(), buf.size(), &n), buf, n);
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
        std::string model, report_file, ids, text, prompt_file;
        bool have_text = false, raw = false, tokenize = false;
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
            else if (arg == "--prompt") text = value(), have_text = true;
            else if (arg == "--prompt-file") prompt_file = value(), have_text = true;
            else if (arg == "--raw") raw = true;
            else if (arg == "--tokenize") tokenize = true;
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
            else if (arg == "--cpu") throw std::invalid_argument("--cpu: this build runs on the MI355X backend only");
            else throw std::invalid_argument("Unknown option: " + arg);
        }
        if (model.empty())
            throw std::invalid_argument("Usage: emprise-chat --model MODEL.gguf (--prompt TEXT | --prompt-file FILE | "
                                        "--prompt-ids 1,2,3 | --synthetic-prompt N [--seed S]) [--raw] [--tokenize] "
                                        "[--tokens N] [--context N] [--fast-q8] [--report FILE] [--unfused] "
                                        "[--no-graph] [--no-batch-prefill]");
        if (!prompt_file.empty()) {
            std::ifstream f(prompt_file, std::ios::binary);
            if (!f) throw std::runtime_error("Cannot read prompt");
            text.assign(std::istreambuf_iterator<char>(f), {});
        }
        if (tokenize) {
            // the file's tokenizer alone, no device (chat.cpp:47-52)
            emprise_tokenizer* t = nullptr;
            check(emprise_tokenizer_open(model.c_str(), &t));
            const auto toks = encode(t, raw ? text : chat_prompt(t, text));
            emprise_tokenizer_close(t);
            std::cout << '[';
            for (size_t i = 0; i < toks.size(); ++i) std::cout << (i ? "," : "") << toks[i];
            std::cout << "]\n";
            return 0;
        }
        opt.path = model.c_str();
        const auto start = std::chrono::steady_clock::now();
        emprise_model* m = nullptr;
        check(emprise_model_open(&opt, &m));
        emprise_model_info info{};
        check(emprise_model_get_info(m, &info));
        std::cerr << "Backend: " << emprise_model_backend_name(m) << '\n';
        const emprise_tokenizer* tok = emprise_model_tokenizer(m);
        std::vector<int> prompt = parse_ids(ids);
        if (have_text) {
            if (!tok) throw std::runtime_error("The model file has no qwen35 GPT-2 BPE tokenizer");
            prompt = encode(tok, raw ? text : chat_prompt(tok, text));
        }
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
        std::string output_text;
        if (tok) {
            for (size_t i = 0; i < emitted; ++i) output_text += decode(tok, tokens[i]);
            std::cout << output_text << '\n';
        } else {
            for (size_t i = 0; i < emitted; ++i) std::cout << (i ? " " : "") << tokens[i];
            std::cout << '\n';
        }
        const double load = std::chrono::duration<double>(loaded - start).count();
        const double first = emitted ? arrivals.front() : 0.0;
        const double rate = emitted > 1 ? double(emitted - 1) / (arrivals.back() - arrivals.front()) : 0.0;
        const double roofline = rate * double(info.token_weight_bytes) / 8.0e12;
        std::cerr << "Load: " << load << "s; first token after load: " << first << "s; generated: " << emitted
                  << "; decode: " << rate << " tokens/s (" << 100.0 * roofline << "% of the 8 TB/s weight roofline)\n";
        // The profile (chat.cpp:72-76): the decode steps are replayed graphs, so the split by
        // kind comes from one more step launched eagerly with per-launch event timing after
        // the output is complete (emprise_model_get_profile), when the context has room.
        emprise_model_profile prof{};
        if (!tokens.empty() && prompt.size() + tokens.size() < opt.context) {
            std::vector<emprise_hip_trace_record> rec(4096);
            size_t nrec = 0;
            check(emprise_model_trace_step(m, tokens.back(), rec.data(), rec.size(), &nrec));
        }
        check(emprise_model_get_profile(m, &prof));
        std::cerr << "Matrix work (device kernels, " << prof.traced_steps << " traced step(s) x " << prof.decode_steps
                  << " decode steps): " << prof.matrix_seconds << "s in " << prof.matrix_calls
                  << " calls; other work: " << prof.non_matrix_seconds << "s\n";
        std::cerr << "Non-matrix: norm " << prof.norm_seconds << "s, attention " << prof.attention_seconds
                  << "s, recurrent " << prof.recurrent_seconds << "s\n";
        if (!report_file.empty()) {
            // The reference's --report fields (chat.cpp:77-84), then this build's roofline.
            // text: the decoded output ("" without a tokenizer). matrix_seconds / matrix_calls /
            // non_matrix_seconds: the profile above (device kernel time of the decode steps,
            // split by kind on a traced step; the reference's own device path leaves them at
            // the prefill's host timers).
            std::ofstream f(report_file);
            if (!f) throw std::runtime_error("Cannot write report");
            f.precision(9);
            f << "{\n  \"engine\": \"emprise mi355x\",\n  \"backend\": " << json_string(emprise_model_backend_name(m))
              << ",\n  \"model\": " << json_string(model) << ",\n  \"prompt_tokens\": " << json_list(prompt)
              << ",\n  \"output_tokens\": " << json_list(tokens) << ",\n  \"text\": " << json_string(output_text)
              << ",\n  \"load_seconds\": " << load
              << ",\n  \"first_token_seconds\": " << first << ",\n  \"generation_tokens_per_second\": " << rate
              << ",\n  \"content_arrivals_seconds\": " << json_list(arrivals)
              << ",\n  \"matrix_seconds\": " << prof.matrix_seconds << ",\n  \"matrix_calls\": " << prof.matrix_calls
              << ",\n  \"non_matrix_seconds\": " << prof.non_matrix_seconds
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
