// Generation loop and chat command over the HIP backends (chat.cpp:531-1040).
#include "hip_chat.h"

#include "gguf_reader.h"
#include "hip_llm.h"
#include "hip_moe.h"

#include <algorithm>
#include <chrono>
#include <filesystem>
#include <iomanip>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <type_traits>

namespace llm {
namespace chat {
namespace {

using Clock = std::chrono::steady_clock;

double ms_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

bool contains(const std::vector<std::int32_t>& v, std::int32_t t) { return std::find(v.begin(), v.end(), t) != v.end(); }

void record_expert_cache(const HipLLM&, GenerationStats&) {}
void record_expert_cache(const HipMoeLLM& backend, GenerationStats& s) {
    const HipExpertCacheStats c = backend.expert_cache_stats();
    s.has_expert_cache_stats = true;
    s.expert_cache_hits = c.hits;
    s.expert_cache_misses = c.misses;
}

template <typename Backend>
GenerationResult generate(Backend& backend, std::vector<std::int32_t> sequence, std::size_t max_new_tokens,
                          const std::vector<std::int32_t>& stop, const TokenSink& sink) {
    // Request checks of chat.cpp:675-699, in the same order and wording.
    if (sequence.empty()) throw std::invalid_argument("Generation requires at least one initial token");
    if (max_new_tokens == 0) throw std::invalid_argument("Generation requires max_new_tokens > 0");
    if (backend.max_sequence() == 0) throw std::runtime_error("Backend sequence capacity is zero");
    if (sequence.size() >= backend.max_sequence()) {
        throw std::invalid_argument("Initial token sequence leaves no room for generated tokens");
    }
    const GgufModelConfig& config = backend.config();
    if (config.layer_count == 0 || config.vocabulary_size == 0 || config.context_length == 0) {
        throw std::runtime_error("Backend model metadata is incomplete");
    }

    GenerationResult result;
    GenerationStats& s = result.stats;
    s.prompt_tokens = sequence.size();
    s.used_gpu = backend.uses_gpu();
    const std::size_t limit = std::min(max_new_tokens, backend.max_sequence() - sequence.size());
    const Clock::time_point t0 = Clock::now();
    backend.reset();

    std::int32_t next = backend.prefill(sequence);
    s.prefill_ms = ms_between(t0, Clock::now());
    for (std::size_t step = 0; step < limit; ++step) {
        if (contains(stop, next)) {
            s.stopped = true;
            break;
        }
        result.generated_tokens.push_back(next);
        ++s.generated_tokens;
        if (sink) sink(next);
        sequence.push_back(next);
        if (step + 1 >= limit) break;
        const Clock::time_point d0 = Clock::now();
        next = backend.decode(next);
        s.decode_ms += ms_between(d0, Clock::now());
        ++s.decode_steps;
    }
    s.total_ms = ms_between(t0, Clock::now());
    s.memory = backend.memory_stats();
    record_expert_cache(backend, s);
    return result;
}

struct Options {
    std::string model_path;
    int max_new_tokens = 32;
    std::size_t max_sequence = 0;
    std::size_t expert_cache_count = 8;
    bool raw_prompt = false;
    bool use_gpu = false;
    bool help_requested = false;
    bool profiling_enabled = true;
    bool kernel_profile = false;
    std::string profile_csv_path = "llm_profile.csv";
    std::string system_prompt = "You are a concise and helpful assistant.";
};

void usage(const char* program, std::ostream& err) {
    err << "Usage: " << program << " --model MODEL.gguf [options]\n"
        << "  --tokens N       Maximum generated tokens per input, default 32\n"
        << "  --max-sequence N Maximum sequence capacity (backend-specific default)\n"
        << "  --expert-cache N Per-layer routed-expert cache slots, default 8\n"
        << "  --system TEXT    System message used by ChatML\n"
        << "  --raw            Send input directly without ChatML wrapping\n"
        << "  --gpu            Use the HIP GPU backend (required: there is no CPU fallback)\n"
        << "  --profile-csv P  Write timing/statistics CSV under output/\n"
        << "                   (default output/llm_profile.csv)\n"
        << "  --profile-log P  Compatibility alias for --profile-csv\n"
        << "  --metal-kernel-profile, --kernel-profile\n"
        << "                   Record per-kernel GPU timestamps\n"
        << "                   (diagnostic mode; decode runs eagerly)\n"
        << "  --no-profile     Disable timing/statistics collection\n"
        << "  --help           Show this help\n";
}

std::size_t parse_size(const std::string& text, const char* name) {
    const unsigned long long v = std::stoull(text);
    if (v > static_cast<unsigned long long>(std::numeric_limits<std::size_t>::max())) {
        throw std::out_of_range(std::string(name) + " does not fit in size_t");
    }
    return static_cast<std::size_t>(v);
}

// chat.cpp:596-653. Returns false when the command line is incomplete.
bool parse_options(int argc, char** argv, Options& o, std::ostream& err) {
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&](const char* name) -> std::string {
            if (i + 1 >= argc) throw std::runtime_error(std::string("missing value for ") + name);
            return argv[++i];
        };
        if (a == "--model") {
            o.model_path = value("--model");
        } else if (a == "--tokens") {
            o.max_new_tokens = std::stoi(value("--tokens"));
        } else if (a == "--max-sequence") {
            o.max_sequence = parse_size(value("--max-sequence"), "--max-sequence");
        } else if (a == "--expert-cache") {
            o.expert_cache_count = parse_size(value("--expert-cache"), "--expert-cache");
        } else if (a == "--system") {
            o.system_prompt = value("--system");
        } else if (a == "--raw") {
            o.raw_prompt = true;
        } else if (a == "--gpu") {
            o.use_gpu = true;
        } else if (a == "--profile-csv") {
            o.profile_csv_path = value("--profile-csv");
        } else if (a == "--profile-log") {
            o.profile_csv_path = value("--profile-log");
        } else if (a == "--metal-kernel-profile" || a == "--kernel-profile") {
            o.kernel_profile = true;
        } else if (a == "--no-profile") {
            o.profiling_enabled = false;
        } else if (a == "--help" || a == "-h") {
            usage(argv[0], err);
            o.help_requested = true;
            return true;
        } else {
            throw std::runtime_error("unknown option: " + a);
        }
    }
    if (o.model_path.empty() || o.max_new_tokens <= 0) {
        usage(argv[0], err);
        return false;
    }
    return true;
}

double per_second(std::size_t n, double ms) { return n == 0 || ms <= 0.0 ? 0.0 : double(n) * 1000.0 / ms; }
double mib(std::uint64_t b) { return double(b) / (1024.0 * 1024.0); }

std::string describe(const HipLLM& b) { return "HIP device=" + b.device_name(); }
std::string describe(const HipMoeLLM& b) {
    return "HIP MoE device=" + b.device_name() + " expert_cache_per_layer=" + std::to_string(b.expert_cache_count());
}

template <typename Backend>
void run_turn(const Options& o, Backend& backend, const QwenTokenizer& tok, const std::vector<std::int32_t>& stop,
              const std::string& input, std::ostream& out, std::ostream& err) {
    const std::string prompt = o.raw_prompt ? input : chat_prompt(o.system_prompt, input);
    const std::vector<std::int32_t> ids = tok.encode(prompt);
    if (ids.empty()) {
        err << "[chat] tokenizer produced no tokens\n";
        return;
    }
    if (backend.max_sequence() == 0 || ids.size() >= backend.max_sequence()) {
        err << "[chat] prompt exceeds model context length\n";
        return;
    }
    err << "[chat] prompt_tokens=" << ids.size() << " ids=";
    for (const std::int32_t t : ids) err << t << ' ';
    err << '\n';
    err << "[assistant] " << std::flush;
    const GenerationResult r = run(backend, ids, static_cast<std::size_t>(o.max_new_tokens), stop,
                                   [&](std::int32_t t) { out << tok.decode_piece(t) << std::flush; });
    out << '\n' << std::flush;
    err << format_generation_stats(r.stats) << '\n';
}

template <typename Backend>
int run_interactive(const Options& o, Backend& backend, std::istream& in, std::ostream& out, std::ostream& err) {
    if (o.profiling_enabled) {
        backend.enable_profiling(o.profile_csv_path, o.kernel_profile);
        const std::filesystem::path primary(o.profile_csv_path);
        const std::filesystem::path parent = primary.parent_path();
        const std::string stem = primary.stem().empty() ? "llm_profile" : primary.stem().string();
        err << "[chat] profile_csv=" << o.profile_csv_path << "\n"
            << "[chat] metal_command_csv=" << (parent / (stem + "_metal_commands.csv")).string() << "\n"
            << "[chat] metal_kernel_csv=" << (parent / (stem + "_metal_kernels.csv")).string() << "\n"
            << "[chat] metal_operation_csv=" << (parent / (stem + "_metal_ops.csv")).string() << "\n";
    }
    const GgufModelConfig& config = backend.config();
    if (config.vocabulary.empty() || config.merges.empty()) {
        throw std::runtime_error("model does not contain Qwen tokenizer vocabulary/merges");
    }
    const QwenTokenizer tok(config.vocabulary, config.merges, config.tokenizer_pre);
    const std::int32_t im_end = tok.id("<|im_end|>");
    if (im_end < 0) throw std::runtime_error("model vocabulary has no <|im_end|> token");
    const std::int32_t slash_s = tok.id("</s>");

    err << "[chat] layers=" << config.layer_count << " embedding=" << config.embedding_size
        << " vocab=" << config.vocabulary_size << " merges=" << config.merges.size()
        << " context=" << config.context_length << " capacity=" << backend.max_sequence()
        << " backend=" << describe(backend) << "\n";
    out << "Enter text (/exit to quit, /clear is accepted):\n";
    const std::vector<std::int32_t> stop = make_stop_tokens(tok, config, im_end, slash_s);

    std::string line;
    while ((out << "> " << std::flush) && std::getline(in, line)) {
        if (line == "/exit" || line == "/quit") break;
        if (line == "/clear") {
            backend.reset();
            out << "[conversation cleared]\n";
            continue;
        }
        run_turn(o, backend, tok, stop, line, out, err);
    }
    out << "\n";
    return 0;
}

}  // namespace

GenerationResult run(HipLLM& backend, std::vector<std::int32_t> initial_sequence, std::size_t max_new_tokens,
                     const std::vector<std::int32_t>& stop_token_ids, TokenSink token_sink) {
    return generate(backend, std::move(initial_sequence), max_new_tokens, stop_token_ids, token_sink);
}

GenerationResult run(HipMoeLLM& backend, std::vector<std::int32_t> initial_sequence, std::size_t max_new_tokens,
                     const std::vector<std::int32_t>& stop_token_ids, TokenSink token_sink) {
    return generate(backend, std::move(initial_sequence), max_new_tokens, stop_token_ids, token_sink);
}

std::vector<std::int32_t> make_stop_tokens(const QwenTokenizer& tok, const GgufModelConfig& config,
                                           std::int32_t im_end, std::int32_t slash_s) {
    std::vector<std::int32_t> out;
    auto add = [&](std::int32_t t) {
        if (t >= 0 && !contains(out, t)) out.push_back(t);
    };
    add(config.eos_token_id);
    add(im_end);
    add(slash_s);
    for (std::size_t t = 0; t < config.vocabulary.size(); ++t) {
        if (tok.is_special(static_cast<std::int32_t>(t))) add(static_cast<std::int32_t>(t));
    }
    return out;
}

std::string format_generation_stats(const GenerationStats& s) {
    std::ostringstream o;
    o << std::fixed << std::setprecision(3) << "[chat] generation_stats mode=" << (s.used_gpu ? "gpu-kv" : "cpu-kv")
      << " prompt_tokens=" << s.prompt_tokens << " generated_tokens=" << s.generated_tokens
      << " decode_steps=" << s.decode_steps << " prefill_ms=" << s.prefill_ms
      << " prefill_tokens_per_sec=" << per_second(s.prompt_tokens, s.prefill_ms) << " decode_ms=" << s.decode_ms
      << " decode_tokens_per_sec=" << per_second(s.decode_steps, s.decode_ms) << " total_ms=" << s.total_ms
      << " weight_bytes=" << s.memory.weight_bytes << " weight_mib=" << mib(s.memory.weight_bytes)
      << " kv_cache_bytes=" << s.memory.kv_cache_bytes << " kv_cache_mib=" << mib(s.memory.kv_cache_bytes)
      << " recurrent_state_bytes=" << s.memory.recurrent_state_bytes
      << " recurrent_state_mib=" << mib(s.memory.recurrent_state_bytes)
      << " intermediate_bytes=" << s.memory.intermediate_bytes
      << " intermediate_mib=" << mib(s.memory.intermediate_bytes)
      << " intermediate_kind=" << (s.memory.intermediate_is_estimate ? "estimated" : "arena")
      << " peak_memory_bytes=" << s.memory.total_bytes() << " peak_memory_mib=" << mib(s.memory.total_bytes());
    if (s.has_expert_cache_stats) {
        const std::uint64_t requests = s.expert_cache_hits + s.expert_cache_misses;
        const double rate = requests == 0 ? 0.0 : 100.0 * double(s.expert_cache_hits) / double(requests);
        o << " expert_cache_requests=" << requests << " expert_cache_hits=" << s.expert_cache_hits
          << " expert_cache_misses=" << s.expert_cache_misses << " expert_cache_hit_rate=" << rate << '%';
    }
    o << " stopped=" << (s.stopped ? "true" : "false");
    return o.str();
}

std::string prepare_profile_output_path(const std::string& requested) {
    namespace fs = std::filesystem;
    if (requested.empty()) throw std::invalid_argument("Profile output filename cannot be empty");
    fs::path path(requested);
    if (!path.is_absolute()) {
        path = path.lexically_normal();
        const auto first = path.begin();
        if (first == path.end() || *first == "..") {
            throw std::invalid_argument("Relative profile output path cannot escape the output directory");
        }
        if (*first != "output") path = fs::path("output") / path;
    }
    const fs::path parent = path.parent_path();
    if (!parent.empty()) {
        std::error_code ec;
        fs::create_directories(parent, ec);
        if (ec) {
            throw std::runtime_error("Cannot create profile output directory " + parent.string() + ": " +
                                     ec.message());
        }
    }
    return path.string();
}

int run_cli(int argc, char** argv, std::istream& in, std::ostream& out, std::ostream& err) {
    try {
        Options o;
        if (!parse_options(argc, argv, o, err)) return 1;
        if (o.help_requested) return 0;
        if (o.kernel_profile && !o.use_gpu) throw std::invalid_argument("--metal-kernel-profile requires --gpu");
        if (o.kernel_profile && !o.profiling_enabled) {
            throw std::invalid_argument("--metal-kernel-profile cannot be combined with --no-profile");
        }
        if (o.profiling_enabled) o.profile_csv_path = prepare_profile_output_path(o.profile_csv_path);

        err << "[chat] loading model: " << o.model_path << "\n";
        if (!o.use_gpu) {
            throw std::invalid_argument("this build has only the HIP backend (no CPULLM); pass --gpu");
        }
        const std::string arch = GgufReader(o.model_path).config().architecture;
        if (arch == "qwen35moe") {
            HipMoeLLM backend(o.model_path, o.max_sequence, {}, o.expert_cache_count);
            return run_interactive(o, backend, in, out, err);
        }
        HipLLM backend(o.model_path, o.max_sequence);
        return run_interactive(o, backend, in, out, err);
    } catch (const std::exception& e) {
        err << "chat: " << e.what() << "\n";
        return 1;
    }
}

}  // namespace chat
}  // namespace llm
