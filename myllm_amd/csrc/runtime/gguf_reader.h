// Streaming raw-tensor GGUF reader.
//
// Same contract as the reference's MetalRawModel (metal_model.h:78-162,
// metal_model.cpp:451-976): parse the header and tensor directory once,
// derive the model config from metadata, then hand out one tensor's native
// bytes at a time (never a dequantized or whole-file copy), with shape checks
// and consumed/ignored accounting so a loader can prove it mapped every
// tensor. The file is memory-mapped read-only; tensor bytes are copied out
// with memcpy (or pread when the mapping fails).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace llm {

// GGML tensor type ids, part of the GGUF format (metal_model.h:14-29).
enum class GgmlType : std::uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q3_K = 11,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
    BF16 = 30,
};

const char* ggml_type_name(GgmlType type) noexcept;
std::size_t ggml_block_size(GgmlType type);
std::size_t ggml_type_size(GgmlType type);
std::size_t ggml_row_bytes(GgmlType type, std::size_t columns);

// Model hyperparameters, same fields as MetalModelConfig (metal_model.h:37-72).
struct GgufModelConfig {
    std::string architecture;
    std::size_t tensor_count = 0;
    std::size_t parameter_count = 0;
    std::size_t stored_weight_bytes = 0;
    std::size_t layer_count = 0;
    std::size_t total_layer_count = 0;
    std::size_t nextn_layer_count = 0;
    std::size_t embedding_size = 0;
    std::size_t feed_forward_size = 0;
    std::size_t attention_head_count = 0;
    std::size_t kv_head_count = 0;
    std::size_t head_size = 0;
    std::size_t rotary_dimension = 0;
    std::size_t vocabulary_size = 0;
    std::size_t context_length = 0;
    std::int32_t eos_token_id = 0;
    float rope_theta = 1000000.0f;
    float norm_epsilon = 1e-6f;
    std::size_t full_attention_interval = 0;
    std::size_t expert_count = 0;
    std::size_t expert_used_count = 0;
    std::size_t expert_feed_forward_size = 0;
    std::size_t shared_expert_feed_forward_size = 0;
    std::size_t ssm_conv_kernel = 0;
    std::size_t ssm_state_size = 0;
    std::size_t ssm_group_count = 0;
    std::size_t ssm_time_step_rank = 0;
    std::size_t ssm_inner_size = 0;
    std::vector<std::string> vocabulary;
    std::vector<std::string> merges;
    std::string tokenizer_pre;
};

// A tensor that stays in the file: where it is and how it is laid out.
struct TensorDescriptor {
    std::string name;
    GgmlType type = GgmlType::F32;
    std::vector<std::uint64_t> dimensions;
    std::size_t rows = 0;
    std::size_t cols = 0;
    std::size_t row_bytes = 0;
    std::size_t data_offset = 0;  // absolute byte offset in the file
    std::size_t byte_size = 0;
};

class GgufReader {
public:
    explicit GgufReader(const std::string& path);
    ~GgufReader();
    GgufReader(const GgufReader&) = delete;
    GgufReader& operator=(const GgufReader&) = delete;

    const GgufModelConfig& config() const noexcept;
    bool has_tensor(const std::string& name) const noexcept;

    // Shape-checked descriptor; marks the tensor consumed (once only).
    TensorDescriptor take(const std::string& name, std::size_t rows, std::size_t cols);
    // Copies bytes [offset, offset + bytes) of a taken tensor into dst.
    void read(const TensorDescriptor& tensor, std::size_t offset, void* dst, std::size_t bytes) const;
    // Zero-copy view of a taken tensor's bytes while the reader lives (null
    // if the file could not be mapped).
    const std::uint8_t* mapped(const TensorDescriptor& tensor) const noexcept;

    void ignore(const std::string& name);
    void ignore_prefix(const std::string& prefix);
    void validate_all_consumed() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace llm
