// HipLLM: the qwen2 inference backend for one MI355X.
//
// Same public contract as the reference's MetalLLM (metal_llm.h:20-52) and
// CPULLM (cpu_llm.h:165-194), so generate() (chat.cpp:831-878) drives it
// unchanged: reset(), prefill(ids) -> next token, decode(id) -> next token,
// config(), position(), max_sequence(), uses_gpu(), memory_stats(),
// available(), device_name(), enable_profiling(). Errors are the reference's
// exception types for the same conditions.
//
// The constructor streams native GGUF tensor bytes into one device weight
// arena (no dequantization, no repacking), allocates the fixed-capacity FP32
// KV cache and the activation arena, and builds the RoPE table. prefill and
// decode run hand-written HIP kernels on one stream and read back the 4-byte
// argmax token.
#pragma once

#include "gguf_reader.h"

#include <cstddef>
#include <cstdint>
#include <limits>
#include <memory>
#include <string>
#include <vector>

namespace llm {

// Byte accounting returned by every backend (memory_stats.h:11-37).
struct MemoryStats {
    std::uint64_t weight_bytes = 0;
    std::uint64_t kv_cache_bytes = 0;
    std::uint64_t recurrent_state_bytes = 0;
    std::uint64_t intermediate_bytes = 0;
    bool intermediate_is_estimate = false;

    std::uint64_t total_bytes() const noexcept {
        const std::uint64_t mx = std::numeric_limits<std::uint64_t>::max();
        std::uint64_t t = weight_bytes;
        for (std::uint64_t v : {kv_cache_bytes, recurrent_state_bytes, intermediate_bytes}) {
            if (v > mx - t) return mx;
            t += v;
        }
        return t;
    }
};

class HipLLM {
public:
    // device < 0 keeps the calling thread's current HIP device.
    explicit HipLLM(const std::string& gguf_path, std::size_t max_sequence = 0, int device = -1);
    ~HipLLM();

    HipLLM(const HipLLM&) = delete;
    HipLLM& operator=(const HipLLM&) = delete;
    HipLLM(HipLLM&&) noexcept;
    HipLLM& operator=(HipLLM&&) noexcept;

    void reset();
    std::int32_t prefill(const std::vector<std::int32_t>& token_ids);
    std::int32_t decode(std::int32_t token_id);

    void enable_profiling(const std::string& csv_path, bool detailed_kernel_timestamps = false);
    void disable_profiling();

    const ModelConfig& config() const;
    std::size_t position() const noexcept;
    std::size_t max_sequence() const noexcept;
    bool uses_gpu() const noexcept;
    MemoryStats memory_stats() const noexcept;

    bool available() const noexcept;
    const std::string& device_name() const noexcept;

    // Logits of the last prefill/decode (vocabulary_size floats), for parity
    // checks. Synchronous device-to-host copy.
    void copy_last_logits(float* destination, std::size_t count) const;
    // Prefill path selection: true = batched (GEMM) prefill, false = the
    // token-serial decode path for every prompt position.
    void set_batched_prefill(bool enabled);
    // Decode path: true (default) = each decode step is one replay of a
    // recorded HIP graph; false = the step's kernels are launched one by one.
    void set_decode_graphs(bool enabled);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace llm
