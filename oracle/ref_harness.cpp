// Harness around the reference's own CPU path (CPULLM, cpu_llm.h:165-194),
// compiled from the reference sources by oracle/Makefile into oracle/_ref/.
// Test infrastructure only: it makes golden vectors and is the timed CPU
// baseline; the product never links it.
//
//   ref_cpullm MODEL.gguf --prompt 1,2,3 --tokens N [--max-sequence S]
//              [--logits FILE] [--no-time]
//
// Tokens follow chat.cpp:831-878 (generate) with no stop tokens: prefill,
// then up to N emitted tokens with a decode after each one except the last.
// With --logits, the forward is recomposed from the reference's public
// operators (embedding, cpu_prefill_layer, cpu_decode_layer, rmsnorm, gevmt:
// the same calls CPULLM::prefill/decode make, cpu_llm.cpp:978-1073) and the
// logits of every step are written as raw float32, step-major.
#include "cpu_llm.h"
#include "model.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

std::vector<int32_t> parse_ids(const char* text) {
    std::vector<int32_t> ids;
    const char* p = text;
    while (*p) {
        char* end = nullptr;
        long v = std::strtol(p, &end, 10);
        if (end == p) throw std::invalid_argument("bad token list");
        ids.push_back(static_cast<int32_t>(v));
        p = *end == ',' ? end + 1 : end;
    }
    return ids;
}

int32_t first_max(const llm::Vector& v) {
    return static_cast<int32_t>(std::max_element(v.values.begin(), v.values.end()) - v.values.begin());
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc < 2) throw std::invalid_argument("usage: ref_cpullm MODEL --prompt ids --tokens N");
        std::string model = argv[1];
        std::vector<int32_t> prompt;
        size_t tokens = 0, max_sequence = 0;
        std::string logits_path;
        for (int i = 2; i < argc; ++i) {
            std::string a = argv[i];
            if (a == "--prompt" && i + 1 < argc) prompt = parse_ids(argv[++i]);
            else if (a == "--tokens" && i + 1 < argc) tokens = std::strtoul(argv[++i], nullptr, 10);
            else if (a == "--max-sequence" && i + 1 < argc) max_sequence = std::strtoul(argv[++i], nullptr, 10);
            else if (a == "--logits" && i + 1 < argc) logits_path = argv[++i];
            else throw std::invalid_argument("unknown argument " + a);
        }
        using Clock = std::chrono::steady_clock;
        auto ms = [](Clock::time_point a, Clock::time_point b) {
            return std::chrono::duration<double, std::milli>(b - a).count();
        };

        std::vector<int32_t> generated;
        double load_ms = 0, prefill_ms = 0, decode_ms = 0;
        size_t decode_steps = 0;
        {
            auto t0 = Clock::now();
            llm::CPULLM backend(model, max_sequence);
            load_ms = ms(t0, Clock::now());
            const size_t limit = std::min(tokens, backend.max_sequence() - prompt.size());
            backend.reset();
            auto p0 = Clock::now();
            int32_t next = backend.prefill(prompt);
            prefill_ms = ms(p0, Clock::now());
            for (size_t step = 0; step < limit; ++step) {
                generated.push_back(next);
                if (step + 1 >= limit) break;
                auto d0 = Clock::now();
                next = backend.decode(next);
                decode_ms += ms(d0, Clock::now());
                ++decode_steps;
            }
        }

        std::vector<int32_t> recomposed;
        if (!logits_path.empty()) {
            llm::ModelFile file(model);
            const llm::ModelConfig cfg = file.config();
            llm::Matrix embd = file.load_token_embedding();
            llm::Vector out_norm = file.load_output_norm();
            llm::Matrix out_w = file.load_output_weight();
            std::vector<llm::Layer> layers;
            for (size_t i = 0; i < cfg.layer_count; ++i) layers.emplace_back(file, i);
            file.validate_all_tensors_loaded();
            std::vector<llm::CPUKVCache> cache(layers.size());
            FILE* f = std::fopen(logits_path.c_str(), "wb");
            if (!f) throw std::runtime_error("cannot write logits");
            llm::Matrix hidden = llm::embedding(prompt, embd);
            for (size_t i = 0; i < layers.size(); ++i) {
                hidden = llm::cpu_prefill_layer(hidden, layers[i], cfg.norm_epsilon, cfg.rotary_dimension,
                                                cfg.rope_theta, cfg.head_size, cache[i]);
            }
            hidden.rmsnorm(out_norm, cfg.norm_epsilon);
            llm::Vector logits = llm::gevmt(out_w, hidden.values.back());
            std::fwrite(logits.values.data(), 4, logits.values.size(), f);
            recomposed.push_back(first_max(logits));
            for (size_t step = 1; step < generated.size(); ++step) {
                llm::Vector h = llm::embedding({generated[step - 1]}, embd).values.front();
                for (size_t i = 0; i < layers.size(); ++i) {
                    h = llm::cpu_decode_layer(h, layers[i], cfg.norm_epsilon, cfg.rotary_dimension,
                                              cfg.rope_theta, cfg.head_size, cache[i]);
                }
                h.rmsnorm(out_norm, cfg.norm_epsilon);
                logits = llm::gevmt(out_w, h);
                std::fwrite(logits.values.data(), 4, logits.values.size(), f);
                recomposed.push_back(first_max(logits));
            }
            std::fclose(f);
        }

        std::printf("{\"tokens\": [");
        for (size_t i = 0; i < generated.size(); ++i) std::printf("%s%d", i ? ", " : "", generated[i]);
        std::printf("], \"recomposed_tokens\": [");
        for (size_t i = 0; i < recomposed.size(); ++i) std::printf("%s%d", i ? ", " : "", recomposed[i]);
        std::printf("], \"load_ms\": %.3f, \"prefill_ms\": %.3f, \"decode_ms\": %.3f, \"decode_steps\": %zu, "
                    "\"prompt_tokens\": %zu}\n",
                    load_ms, prefill_ms, decode_ms, decode_steps, prompt.size());
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_cpullm: %s\n", e.what());
        return 1;
    }
}
