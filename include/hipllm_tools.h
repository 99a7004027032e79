/*
 * C ABI of libhipllm_tools.so: host-only helpers that build synthetic inputs
 * (GGML block quantizers, a deterministic N(0, s) source and a qwen2 GGUF
 * writer). The reference has no counterpart: it only reads GGUF files made by
 * ggml (README.md:74, 91). Nothing here touches a GPU.
 */
#ifndef HIPLLM_TOOLS_H
#define HIPLLM_TOOLS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct HipllmQwen2Spec {
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
    uint32_t type_embd;        /* GGML type ids: 0 F32, 1 F16, 6 Q5_0, 8 Q8_0, 12 Q4_K, 14 Q6_K */
    uint32_t type_attn_qkv;
    uint32_t type_attn_out;
    uint32_t type_ffn_gate_up;
    uint32_t type_ffn_down;
    uint32_t type_output;
    uint64_t seed;
    float stddev;
    float bias_stddev;
    uint32_t threads;
} HipllmQwen2Spec;

/* Synthetic qwen35moe model (moe_model.cpp:151-234 schema): full-attention
 * layers where (i + 1) % full_attention_interval == 0, Gated DeltaNet layers
 * otherwise, routed + shared experts in every layer. */
typedef struct HipllmQwen35MoeSpec {
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
    float small_stddev;
    float conv_stddev;
    uint32_t threads;
} HipllmQwen35MoeSpec;

/* Bytes of one row of `cols` elements of GGML type `type`; 0 if unsupported
 * or not block aligned. */
size_t hipllm_tools_row_bytes(uint32_t type, size_t cols);

/* Quantizes rows x cols FP32 values (row-major) into dst, rows * row_bytes
 * bytes, using up to `threads` host threads. Returns 0 on success. */
int hipllm_tools_quantize_rows(uint32_t type, const float* src, size_t rows,
                               size_t cols, uint8_t* dst, uint32_t threads);

/* Deterministic N(0, stddev) values for indices [first, first + count). */
void hipllm_tools_fill_normal(uint64_t seed, uint64_t stream, uint64_t first,
                              size_t count, float stddev, float* dst);

/* Deterministic uniform integers in [0, bound). */
void hipllm_tools_fill_uniform_int(uint64_t seed, uint64_t stream,
                                   uint64_t first, size_t count,
                                   uint32_t bound, int32_t* dst);

/* Writes a qwen2 GGUF file. Returns 0 on success, else copies a message into
 * err (NUL terminated, at most errlen bytes) and returns -1. */
int hipllm_tools_write_qwen2(const char* path, const HipllmQwen2Spec* spec,
                             char* err, size_t errlen);

/* Writes a qwen35moe GGUF file; same error convention as the qwen2 writer. */
int hipllm_tools_write_qwen35moe(const char* path, const HipllmQwen35MoeSpec* spec,
                                 char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* HIPLLM_TOOLS_H */
