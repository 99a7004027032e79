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

// qwen35moe (text-only Qwen3.5/3.6 MoE with Gated DeltaNet layers): tensor
// schema of moe_model.cpp:151-234, metadata keys of metal_model.cpp:582-660.
struct Qwen35MoeSpec {
    uint32_t layers;
    uint32_t hidden;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;
    uint32_t vocab;
    uint32_t context;
    uint32_t eos_token_id;
    float rope_theta;
    float norm_eps;
    uint32_t experts;
    uint32_t experts_used;
    uint32_t expert_ffn;
    uint32_t shared_ffn;
    uint32_t full_attention_interval;
    uint32_t conv_kernel;
    uint32_t state_size;
    uint32_t group_count;
    uint32_t time_step_rank;
    uint32_t type_embd;
    uint32_t type_output;
    uint32_t type_attn_qgate;
    uint32_t type_attn_kv;
    uint32_t type_attn_out;
    uint32_t type_ssm_qkv;
    uint32_t type_ssm_gate;
    uint32_t type_ssm_out;
    uint32_t type_expert_gate_up;
    uint32_t type_expert_down;
    uint32_t type_shared;
    uint64_t seed;
    float stddev;
    float small_stddev;  // F32 router / alpha / beta / shared-router / dt bias
    float conv_stddev;   // depthwise conv taps
    uint32_t threads;
};

void write_qwen35moe(const std::string& path, const Qwen35MoeSpec& spec);

}  // namespace hipllm_tools
