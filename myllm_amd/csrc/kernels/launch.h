// Host-side launchers of the HipLLM kernels. Every launcher validates its
// arguments, launches on `stream` without allocating, and returns a status
// code from common.h (0 on success).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace hipllm {

int launch_dequant_rows(uint32_t type, const void* w, size_t row_bytes, size_t rows, size_t k, float* out,
                        hipStream_t stream);

int launch_prep_sums(const float* x, float* xs16, size_t k, hipStream_t stream);
int gemv_default_tiling(uint32_t n, uint32_t units, int mode);
int launch_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* xs16,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        hipStream_t stream);
int launch_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const float* xs16, float* y, float* ys16, size_t n, size_t k, hipStream_t stream);

int gemm_default_tile(uint32_t m, uint32_t n);
int launch_to_bf16(const float* x, size_t ldx, void* xb, size_t m, size_t k, hipStream_t stream);
int launch_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* bias,
                     const float* residual, float* y, size_t m, size_t n, size_t k, int tile, hipStream_t stream,
                     size_t ldy = 0);
int launch_attn_prefill(const float* q, size_t q_stride, const float* kcache, const float* vcache, float* out,
                        size_t out_stride, size_t rows, size_t hq, size_t hkv, size_t d, size_t pos0, float scale,
                        hipStream_t stream);

int launch_rmsnorm(const float* x, const float* gamma, float* y, float* ys16, size_t rows, size_t cols, float eps,
                   hipStream_t stream);
int launch_embed(uint32_t type, const void* table, size_t row_bytes, const int32_t* ids, size_t rows, size_t vocab,
                 size_t cols, float* out, hipStream_t stream);
int launch_rope_kv(float* qkv, const float* cos_sin, size_t rot, size_t hq, size_t hkv, size_t d, size_t pos0,
                   size_t rows, size_t row_stride, float* kcache, float* vcache, hipStream_t stream);
size_t attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len);
int launch_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, float* out16,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, hipStream_t stream);
size_t argmax_scratch_bytes(size_t n);
int launch_argmax(const float* x, size_t n, uint32_t* out, void* scratch, hipStream_t stream);
int launch_swiglu(const float* g, const float* u, float* y, float* y16, size_t n, hipStream_t stream);
int launch_add(const float* a, const float* b, float* y, size_t n, hipStream_t stream);

}  // namespace hipllm
