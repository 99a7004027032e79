// C ABI wrapper over the synthetic-input tools.
#include "../../../include/hipllm_tools.h"

#include "quants.h"
#include "synth_gguf.h"

#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

static_assert(sizeof(HipllmQwen2Spec) == sizeof(hipllm_tools::Qwen2Spec),
              "C and C++ qwen2 spec layouts differ");

namespace {
void copy_error(const char* message, char* err, size_t errlen) {
    if (err == nullptr || errlen == 0) return;
    std::strncpy(err, message, errlen - 1);
    err[errlen - 1] = '\0';
}
}  // namespace

extern "C" size_t hipllm_tools_row_bytes(uint32_t type, size_t cols) {
    return hipllm_tools::row_bytes(type, cols);
}

extern "C" int hipllm_tools_quantize_rows(uint32_t type, const float* src, size_t rows,
                                          size_t cols, uint8_t* dst, uint32_t threads) {
    const size_t rb = hipllm_tools::row_bytes(type, cols);
    if (rb == 0 || src == nullptr || dst == nullptr) return -1;
    if (threads == 0) threads = 1;
    if (threads > rows) threads = static_cast<uint32_t>(rows ? rows : 1);
    std::vector<std::thread> pool;
    std::vector<int> status(threads, 0);
    for (uint32_t t = 0; t < threads; ++t) {
        pool.emplace_back([&, t] {
            for (size_t r = t; r < rows; r += threads) {
                if (!hipllm_tools::quantize_row(type, src + r * cols, cols, dst + r * rb)) {
                    status[t] = -1;
                    return;
                }
            }
        });
    }
    for (auto& th : pool) th.join();
    for (int s : status) {
        if (s) return s;
    }
    return 0;
}

extern "C" void hipllm_tools_fill_normal(uint64_t seed, uint64_t stream, uint64_t first,
                                         size_t count, float stddev, float* dst) {
    hipllm_tools::fill_normal(seed, stream, first, count, stddev, dst);
}

extern "C" void hipllm_tools_fill_uniform_int(uint64_t seed, uint64_t stream,
                                              uint64_t first, size_t count,
                                              uint32_t bound, int32_t* dst) {
    hipllm_tools::fill_uniform_int(seed, stream, first, count, bound, dst);
}

extern "C" int hipllm_tools_write_qwen2(const char* path, const HipllmQwen2Spec* spec,
                                        char* err, size_t errlen) {
    try {
        if (path == nullptr || spec == nullptr) throw std::invalid_argument("null argument");
        hipllm_tools::Qwen2Spec s;
        std::memcpy(&s, spec, sizeof(s));
        hipllm_tools::write_qwen2(path, s);
        return 0;
    } catch (const std::exception& e) {
        copy_error(e.what(), err, errlen);
        return -1;
    }
}

extern "C" int hipllm_tools_write_qwen35moe(const char* path, const HipllmQwen35MoeSpec* spec,
                                            char* err, size_t errlen) {
    try {
        if (path == nullptr || spec == nullptr) throw std::invalid_argument("null argument");
        static_assert(sizeof(HipllmQwen35MoeSpec) == sizeof(hipllm_tools::Qwen35MoeSpec), "spec layout");
        hipllm_tools::Qwen35MoeSpec s;
        std::memcpy(&s, spec, sizeof(s));
        hipllm_tools::write_qwen35moe(path, s);
        return 0;
    } catch (const std::exception& e) {
        copy_error(e.what(), err, errlen);
        return -1;
    }
}
