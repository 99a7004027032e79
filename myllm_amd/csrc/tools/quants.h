// Host-side GGML block quantizers used to build synthetic GGUF inputs.
//
// These restate the published GGML reference quantizers
// (ggml-quants.c: quantize_row_q4_K_ref, quantize_row_q6_K_ref,
// quantize_row_q8_0_ref, quantize_row_q5_0_ref, with make_qkx2_quants and
// make_qx_quants). The reference repository only consumes GGUF files made by
// those quantizers (README.md:74, 91) and pins no ggml version, so exact
// byte equality with any particular ggml release is not claimed. Parity of
// the inference path does not depend on it: the CPU oracle and the GPU both
// dequantize the same bytes.
#pragma once

#include <cstddef>
#include <cstdint>

namespace hipllm_tools {

enum : uint32_t {
    kTypeF32 = 0,
    kTypeF16 = 1,
    kTypeQ5_0 = 6,
    kTypeQ8_0 = 8,
    kTypeQ4_K = 12,
    kTypeQ6_K = 14,
};

// Bytes of one row of `cols` elements, or 0 when the type is unsupported or
// cols is not a multiple of the type's block size.
size_t row_bytes(uint32_t type, size_t cols);

// IEEE binary16 round-to-nearest-even conversion.
uint16_t float_to_half(float value);
float half_to_float(uint16_t value);

// Quantizes one row. Returns false for an unsupported type or shape.
bool quantize_row(uint32_t type, const float* src, size_t cols, uint8_t* dst);

// Deterministic N(0, stddev) values for element indices [first, first + count)
// of stream `stream` under `seed`. A counter-based hash (splitmix64 finaliser)
// feeds a Box-Muller transform, so any slice can be generated independently
// and in parallel with identical results.
void fill_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t count,
                 float stddev, float* dst);

// Deterministic uniform integers in [0, bound) for indices [first, first+count).
void fill_uniform_int(uint64_t seed, uint64_t stream, uint64_t first,
                      size_t count, uint32_t bound, int32_t* dst);

}  // namespace hipllm_tools
