// Bit-exact dequantization of native GGUF rows to FP32 (model.cpp:543-683),
// one thread per output element. The parity hook for the weight formats, not
// a hot kernel; the element formulas live in formats.h.
#include "formats.h"

namespace hipllm {
namespace {

__global__ void dequant_rows_kernel(uint32_t type, const uint8_t* __restrict__ w, size_t row_bytes,
                                    uint32_t rows, uint32_t k, float* __restrict__ out) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t total = static_cast<size_t>(rows) * k;
    if (idx >= total) return;
    const uint32_t r = static_cast<uint32_t>(idx / k);
    const uint32_t c = static_cast<uint32_t>(idx % k);
    out[idx] = dequant_element(type, w + static_cast<size_t>(r) * row_bytes, c);
}

}  // namespace

int launch_dequant_rows(uint32_t type, const void* w, size_t row_bytes, size_t rows, size_t k,
                        float* out, hipStream_t stream) {
    const uint32_t be = block_elems(type);
    if (!w || !out || k == 0 || rows == 0 || k % be != 0) return kInvalidArgument;
    if (type != kF32 && type != kF16 && type != kQ5_0 && type != kQ8_0 && type != kQ4_K && type != kQ6_K) {
        return kInvalidArgument;
    }
    if (row_bytes < k / be * block_bytes(type)) return kInvalidArgument;
    if (rows > 0xffffffffull || k > 0xffffffffull) return kLengthError;
    const size_t total = rows * k;
    const uint32_t threads = 256;
    const size_t blocks = (total + threads - 1) / threads;
    if (blocks > 0x7fffffffull) return kLengthError;
    HIPLLM_LAUNCH(dequant_rows_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(threads), 0, stream,
                       type, static_cast<const uint8_t*>(w), row_bytes, static_cast<uint32_t>(rows),
                       static_cast<uint32_t>(k), out);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

}  // namespace hipllm
