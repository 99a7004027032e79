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

#include "backend_types.h"
#include "gguf_reader.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace llm {

class HipLLM {
public:
    // The third parameter is where MetalLLM takes its shader path
    // (metal_llm.h:22-24), so run_cli's construction compiles unchanged; here
    // it selects the device: "" (default) keeps the calling thread's current
    // HIP device, "N" or "hip:N" picks visible device N.
    explicit HipLLM(const std::string& gguf_path, std::size_t max_sequence = 0, const std::string& device = {});
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

    const GgufModelConfig& config() const;
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
    // Decode GEMVs of Q4_K / Q6_K projections on the x16 tile-packed copies (the
    // int8-MFMA GEMV; on by default when the model has such projections) or
    // on the GGUF rows (the vector GEMV). Results agree to FP32 rounding.
    void set_packed_decode(bool enabled);
    bool packed_decode() const noexcept;
    // Decode RMSNorms folded into the neighbouring GEMVs where the model's
    // forms allow (true, default): the GEMV prologue for rows of up to 2048
    // values on GGUF rows, or the x16 GEMVs' norm data (producer epilogue,
    // consumer scaling); false = every norm is its own launch. Results agree
    // to FP32 rounding.
    void set_fused_norms(bool enabled);
    bool fused_norms() const noexcept;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace llm
