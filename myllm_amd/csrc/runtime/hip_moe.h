// HipMoeLLM: the qwen35moe (Qwen3.5/3.6 MoE, Gated DeltaNet) backend for one
// MI355X.
//
// Same public contract as the reference's MoeLLM (moe_llm.h:80-115):
// reset(), prefill(ids) -> next token, decode(id) -> next token, config(),
// position(), max_sequence(), uses_gpu(), memory_stats(), device_name(),
// expert_cache_count(). Errors are the reference's exception types for the
// same conditions (moe_llm.mm:3051-3141).
//
// Unlike the reference, every routed expert stays resident in HBM (the
// reference streams them through a per-layer LRU cache and reads the routes
// back to the host once per layer): the router's top-k ids stay on the
// device and the expert GEMVs index the resident weights directly, so a whole
// forward is one stream of kernels with a single 4-byte readback.
#pragma once

#include "gguf_reader.h"
#include "hip_llm.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace llm {

class HipMoeLLM {
public:
    // max_sequence 0 = min(context length, 1024), as the reference
    // (moe_llm.mm:1378-1380). expert_cache_count is accepted for interface
    // parity and validated like the reference (top-k <= n <= experts); all
    // experts are resident regardless.
    // device: as HipLLM's (the position of MoeLLM's shader path,
    // moe_llm.h:82-85), so `HipMoeLLM(path, max_sequence, {}, n)` reads like
    // run_cli's MoeLLM construction (chat.cpp:1026-1029).
    explicit HipMoeLLM(const std::string& gguf_path, std::size_t max_sequence = 0, const std::string& device = {},
                       std::size_t expert_cache_count = 8);
    ~HipMoeLLM();

    HipMoeLLM(const HipMoeLLM&) = delete;
    HipMoeLLM& operator=(const HipMoeLLM&) = delete;
    HipMoeLLM(HipMoeLLM&&) noexcept;
    HipMoeLLM& operator=(HipMoeLLM&&) noexcept;

    void reset();
    std::int32_t prefill(const std::vector<std::int32_t>& token_ids);
    std::int32_t decode(std::int32_t token_id);

    void enable_profiling(const std::string& csv_path, bool detailed_kernel_timestamps = false);
    void disable_profiling();

    const GgufModelConfig& config() const;
    std::size_t position() const noexcept;
    std::size_t max_sequence() const noexcept;
    bool uses_gpu() const noexcept;
    MemoryStats memory_stats() const noexcept;
    bool available() const noexcept;
    const std::string& device_name() const noexcept;
    std::size_t expert_cache_count() const noexcept;
    // Expert lookups since construction: tokens x routes x MoE layers of
    // every forward, all hits (every expert is resident).
    HipExpertCacheStats expert_cache_stats() const noexcept;
    // Decode path: true (default) = each decode step is one replay of a
    // recorded HIP graph; false = the step's kernels are launched one by one.
    void set_decode_graphs(bool enabled);
    // Prefill of 16 or more rows: true (default) = the dense projections run
    // as fp16 MFMA matmuls (the router stays FP32); false = FP32 GEMVs only.
    void set_matmul_prefill(bool enabled);

    void copy_last_logits(float* destination, std::size_t count) const;
    // Expert ids chosen for the last token of the last forward, layer-major
    // [layer_count, expert_used_count] (parity checks).
    void copy_last_routes(std::int32_t* destination, std::size_t count) const;
    // Route probe: when on, every forward keeps the router logits and the
    // shared-expert gate logit of its last row for each layer, readable as
    // [layer_count, expert_count + 1] floats (parity checks of near-tie
    // routes). Off by default; switching drops the recorded decode graph.
    void set_route_probe(bool enabled);
    void copy_last_router_logits(float* destination, std::size_t count) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace llm
