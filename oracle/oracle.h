/*
 * CPU oracle: a C++ restatement of the reference's CPULLM path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * CPU-baseline leg of bench.py may load liboracle.so, and only as the
 * checker or the timed CPU baseline; the HipLLM product path never calls it.
 *
 * What it restates (reference file:line):
 *   GGUF parsing            model.cpp:376-489 (whole file read into memory)
 *   half_to_float           model.cpp:500-522
 *   get_scale_min_k4        model.cpp:524-537
 *   dequant Q5_0/Q8_0/Q4_K/Q6_K/F32/F16   model.cpp:543-683
 *   qwen2 config + schema   model.cpp:720-776, 861-919
 *   operators               cpu_llm.cpp:101-235 (embedding, rmsnorm, softmax,
 *                           swiglu, rope), 453-665 (gevm/gevmts/gevmt/gevmtb,
 *                           gemm/gemmt/gemmts/gemmtb), 316-329 (causal mask)
 *   layer graphs            cpu_llm.cpp:774-841 (prefill), 843-914 (decode)
 *   lifecycle               cpu_llm.cpp:928-1073 (ctor, reset, prefill, decode)
 *   greedy_token            cpu_llm.cpp:34-48 (first maximum)
 * Every floating-point expression keeps the reference's operand order; the
 * library is built -O2 -ffp-contract=off with no -march so no FMA is formed,
 * as in the reference build (Makefile:4).
 *
 * Error codes mirror the reference's exception types:
 *   0 ok, 1 std::invalid_argument, 2 std::out_of_range, 3 std::length_error,
 *   4 std::runtime_error, 5 std::overflow_error.
 */
#ifndef HIPLLM_ORACLE_H
#define HIPLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OracleModel OracleModel;

typedef struct OracleConfig {
    uint64_t layer_count;
    uint64_t embedding_size;
    uint64_t feed_forward_size;
    uint64_t attention_head_count;
    uint64_t kv_head_count;
    uint64_t head_size;
    uint64_t rotary_dimension;
    uint64_t vocabulary_size;
    uint64_t context_length;
    uint64_t parameter_count;
    int32_t eos_token_id;
    float rope_theta;
    float norm_epsilon;
} OracleConfig;

int oracle_open(const char* gguf_path, size_t max_sequence, OracleModel** out,
                char* err, size_t errlen);
void oracle_close(OracleModel* model);
int oracle_config(const OracleModel* model, OracleConfig* out);
size_t oracle_position(const OracleModel* model);
size_t oracle_max_sequence(const OracleModel* model);
int oracle_reset(OracleModel* model, char* err, size_t errlen);
/* logits may be NULL; otherwise it receives vocabulary_size floats. */
int oracle_prefill(OracleModel* model, const int32_t* ids, size_t count,
                   int32_t* token, float* logits, char* err, size_t errlen);
int oracle_decode(OracleModel* model, int32_t id, int32_t* token,
                  float* logits, char* err, size_t errlen);

/* Dequantized copy of a named tensor (rows * cols floats). */
int oracle_tensor_f32(const OracleModel* model, const char* name, float* out,
                      size_t capacity, char* err, size_t errlen);

/* Operator-level entry points (same numerics as the model graph). */
int oracle_dequant_row(uint32_t type, const uint8_t* data, size_t cols, float* out);
float oracle_half_to_float(uint16_t bits);
void oracle_gevmt(const float* w, const float* x, const float* bias, size_t rows,
                  size_t cols, float* y);
void oracle_rmsnorm(float* x, const float* gamma, size_t n, float eps);
void oracle_softmax(float* x, size_t n);
void oracle_swiglu(float* gate, const float* up, size_t n);
/* The decode-layer FFN (cpu_llm.cpp:907-913) on a normalised row x[h]:
 * out[h] = Wd (silu(Wg x) * (Wu x)), weights row-major [f, h], [f, h], [h, f];
 * the same function the oracle's decode step calls. */
void oracle_ffn(const float* wg, const float* wu, const float* wd, const float* x, size_t h, size_t f, float* out);
void oracle_rope(float* x, size_t len, size_t position, float theta, size_t rot);
int32_t oracle_argmax(const float* x, size_t n);

#ifdef __cplusplus
}
#endif

#endif
