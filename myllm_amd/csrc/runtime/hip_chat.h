// Greedy generation loop and the interactive chat front end over the HIP
// backends: the caller contract of chat.h:18-75 (GenerationStats,
// GenerationResult, run) and the command line of chat.cpp:531-1040
// (options, ChatML turns, stop tokens, stats line, profile CSV paths), with
// --gpu choosing HipLLM or HipMoeLLM by the GGUF architecture.
#pragma once

#include "backend_types.h"
#include "tokenizer.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <iosfwd>
#include <string>
#include <vector>

namespace llm {

class HipLLM;
class HipMoeLLM;
struct GgufModelConfig;

namespace chat {

using TokenSink = std::function<void(std::int32_t)>;

// Fields and meaning of chat.h:20-41.
struct GenerationStats {
    double prefill_ms = 0.0;  // prompt forward up to the first next token
    double decode_ms = 0.0;   // sum over single-token decode steps
    double total_ms = 0.0;
    std::size_t prompt_tokens = 0;
    std::size_t generated_tokens = 0;
    std::size_t decode_steps = 0;
    bool used_gpu = false;
    bool stopped = false;
    bool has_expert_cache_stats = false;
    std::uint64_t expert_cache_hits = 0;
    std::uint64_t expert_cache_misses = 0;
    MemoryStats memory;
};

struct GenerationResult {
    std::vector<std::int32_t> generated_tokens;
    GenerationStats stats;
};

// chat.cpp:831-878: validate, reset the backend's conversation state,
// prefill, then emit / decode until a stop token or the limit
// min(max_new_tokens, max_sequence - prompt length). A stop token is not
// emitted; the last emitted token is not decoded. token_sink sees every
// emitted token as soon as it is known.
GenerationResult run(HipLLM& backend, std::vector<std::int32_t> initial_sequence, std::size_t max_new_tokens,
                     const std::vector<std::int32_t>& stop_token_ids = {}, TokenSink token_sink = {});
GenerationResult run(HipMoeLLM& backend, std::vector<std::int32_t> initial_sequence, std::size_t max_new_tokens,
                     const std::vector<std::int32_t>& stop_token_ids = {}, TokenSink token_sink = {});

// chat.cpp:708-726: eos, <|im_end|>, </s> (when present), then every special
// token in id order, without repeats or negative ids.
std::vector<std::int32_t> make_stop_tokens(const QwenTokenizer& tokenizer, const GgufModelConfig& config,
                                           std::int32_t im_end, std::int32_t slash_s);

// The "[chat] generation_stats ..." line of chat.cpp:743-785 (no newline).
std::string format_generation_stats(const GenerationStats& stats);

// chat.cpp:562-594: a relative path goes under output/ (".." may not
// escape it); parent directories are created.
std::string prepare_profile_output_path(const std::string& requested_path);

// The chat command (chat.cpp:998-1040) reading turns from `in`, streaming
// the assistant text to `out` and diagnostics to `err`. Returns the exit
// status.
int run_cli(int argc, char** argv, std::istream& in, std::ostream& out, std::ostream& err);

}  // namespace chat
}  // namespace llm
