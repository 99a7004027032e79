// Synthetic GGUF model writer: qwen2 schema with a per-role quant mix.
#pragma once

#include <cstdint>
#include <string>

namespace hipllm_tools {

// Plain-old-data so it can cross the C ABI unchanged (see include/hipllm_tools.h).
struct Qwen2Spec {
    uint32_t layers;
    uint32_t hidden;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t ffn;
    uint32_t vocab;
    uint32_t context;
    uint32_t eos_token_id;
    float rope_theta;
    float norm_eps;
    uint32_t type_embd;
    uint32_t type_attn_qkv;
    uint32_t type_attn_out;
    uint32_t type_ffn_gate_up;
    uint32_t type_ffn_down;
    uint32_t type_output;
    uint64_t seed;
    float stddev;
    float bias_stddev;
    uint32_t threads;
};

void write_qwen2(const std::string& path, const Qwen2Spec& spec);

}  // namespace hipllm_tools
