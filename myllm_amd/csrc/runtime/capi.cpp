// C ABI of libhipllm.so (declarations and reference citations in
// include/hipllm.h).
#include "../../../include/hipllm.h"

#include "../kernels/common.h"
#include "../kernels/launch.h"
#include "hip_llm.h"

#include <cstring>
#include <exception>
#include <new>
#include <stdexcept>
#include <string>

struct HipllmModel {
    llm::HipLLM model;
    explicit HipllmModel(const char* path, size_t max_sequence, int device) : model(path, max_sequence, device) {}
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* what) {
    g_last_error = what;
    return code;
}

int status(int code, const char* what) {
    if (code != hipllm::kOk) g_last_error = what;
    return code;
}

template <typename Fn>
int guarded(Fn fn) {
    try {
        fn();
        return HIPLLM_OK;
    } catch (const std::invalid_argument& e) {
        return fail(HIPLLM_INVALID_ARGUMENT, e.what());
    } catch (const std::out_of_range& e) {
        return fail(HIPLLM_OUT_OF_RANGE, e.what());
    } catch (const std::length_error& e) {
        return fail(HIPLLM_LENGTH_ERROR, e.what());
    } catch (const std::overflow_error& e) {
        return fail(HIPLLM_OVERFLOW_ERROR, e.what());
    } catch (const std::bad_alloc&) {
        return fail(HIPLLM_RUNTIME_ERROR, "host allocation failed");
    } catch (const std::exception& e) {
        return fail(HIPLLM_RUNTIME_ERROR, e.what());
    }
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

const char* hipllm_last_error(void) { return g_last_error.c_str(); }
const char* hipllm_version(void) { return "hipllm 0.1 (gfx950)"; }

int hipllm_dequant_rows(uint32_t type, const void* w, size_t row_bytes, size_t rows, size_t k, float* out,
                        void* stream) {
    return status(hipllm::launch_dequant_rows(type, w, row_bytes, rows, k, out, as_stream(stream)),
                  "hipllm_dequant_rows: invalid arguments or launch failure");
}

int hipllm_prep_sums(const float* x, float* xs16, size_t k, void* stream) {
    return status(hipllm::launch_prep_sums(x, xs16, k, as_stream(stream)), "hipllm_prep_sums failed");
}

size_t hipllm_gemv_workspace_bytes(size_t k) { return (k + 15) / 16 * sizeof(float); }

int hipllm_gemv(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* bias, float* y,
                size_t n, size_t k, void* workspace, void* stream) {
    if (!workspace) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemv: workspace is null");
    float* xs16 = static_cast<float*>(workspace);
    int rc = hipllm::launch_prep_sums(x, xs16, k, as_stream(stream));
    if (rc != hipllm::kOk) return status(rc, "hipllm_gemv: k must be a positive multiple of 16");
    return status(hipllm::launch_gemv_prepped(type, w, row_bytes, x, xs16, bias, nullptr, y, n, k, 0,
                                              as_stream(stream)),
                  "hipllm_gemv: invalid arguments or launch failure");
}

int hipllm_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* xs16,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        void* stream) {
    return status(hipllm::launch_gemv_prepped(type, w, row_bytes, x, xs16, bias, residual, y, n, k, tiling,
                                              as_stream(stream)),
                  "hipllm_gemv_prepped: invalid arguments or launch failure");
}

int hipllm_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const float* xs16, float* y, float* ys16, size_t n, size_t k, void* stream) {
    return status(hipllm::launch_gemv_swiglu(type, wg, wu, row_bytes, x, xs16, y, ys16, n, k, as_stream(stream)),
                  "hipllm_gemv_swiglu: invalid arguments or launch failure");
}

int hipllm_to_bf16(const float* x, size_t ldx, void* xb, size_t m, size_t k, void* stream) {
    return status(hipllm::launch_to_bf16(x, ldx, xb, m, k, as_stream(stream)),
                  "hipllm_to_bf16: invalid arguments (k % 8 == 0, 16-byte aligned buffers) or launch failure");
}

int hipllm_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* bias,
                     const float* residual, float* y, size_t m, size_t n, size_t k, int tile, void* stream) {
    return status(hipllm::launch_gemm_mfma(type, w, row_bytes, xb, bias, residual, y, m, n, k, tile,
                                           as_stream(stream)),
                  "hipllm_gemm_mfma: invalid arguments (k % 128 == 0, tile 0..3) or launch failure");
}

size_t hipllm_gemm_workspace_bytes(size_t m, size_t k) { return (m * k * 2 + 255) / 256 * 256; }

int hipllm_gemm(uint32_t type, const void* w, size_t row_bytes, const float* x, size_t ldx, const float* bias,
                float* y, size_t m, size_t n, size_t k, void* workspace, void* stream) {
    if (!workspace) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemm: workspace is null");
    const int rc = hipllm::launch_to_bf16(x, ldx, workspace, m, k, as_stream(stream));
    if (rc != hipllm::kOk) return status(rc, "hipllm_gemm: invalid activation arguments");
    return status(hipllm::launch_gemm_mfma(type, w, row_bytes, workspace, bias, nullptr, y, m, n, k, -1,
                                           as_stream(stream)),
                  "hipllm_gemm: invalid arguments (k % 128 == 0) or launch failure");
}

int hipllm_rmsnorm(const float* x, const float* gamma, float* y, float* ys16, size_t rows, size_t cols, float eps,
                   void* stream) {
    return status(hipllm::launch_rmsnorm(x, gamma, y, ys16, rows, cols, eps, as_stream(stream)),
                  "hipllm_rmsnorm: invalid arguments or launch failure");
}

int hipllm_embed(uint32_t type, const void* table, size_t row_bytes, const int32_t* ids, size_t rows, size_t vocab,
                 size_t cols, float* out, void* stream) {
    return status(hipllm::launch_embed(type, table, row_bytes, ids, rows, vocab, cols, out, as_stream(stream)),
                  "hipllm_embed: invalid arguments or launch failure");
}

int hipllm_rope_kv(float* qkv, const float* cos_sin, size_t rot, size_t hq, size_t hkv, size_t d, size_t pos0,
                   size_t rows, size_t row_stride, float* kcache, float* vcache, void* stream) {
    return status(hipllm::launch_rope_kv(qkv, cos_sin, rot, hq, hkv, d, pos0, rows, row_stride, kcache, vcache,
                                         as_stream(stream)),
                  "hipllm_rope_kv: invalid arguments or launch failure");
}

size_t hipllm_attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len) {
    return hipllm::attn_decode_scratch_floats(hq, d, max_len);
}

int hipllm_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, float* out16,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, void* stream) {
    return status(hipllm::launch_attn_decode(q, kcache, vcache, out, out16, scratch, hq, hkv, d, len, scale,
                                             as_stream(stream)),
                  "hipllm_attn_decode: invalid arguments or launch failure");
}

size_t hipllm_argmax_scratch_bytes(size_t n) { return hipllm::argmax_scratch_bytes(n); }

int hipllm_argmax(const float* x, size_t n, uint32_t* out, void* scratch, void* stream) {
    return status(hipllm::launch_argmax(x, n, out, scratch, as_stream(stream)),
                  "hipllm_argmax: invalid arguments or launch failure");
}

int hipllm_swiglu(const float* g, const float* u, float* y, float* y16, size_t n, void* stream) {
    return status(hipllm::launch_swiglu(g, u, y, y16, n, as_stream(stream)),
                  "hipllm_swiglu: invalid arguments or launch failure");
}

int hipllm_create(const char* path, size_t max_sequence, int device, HipllmModel** out) {
    if (!path || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_create: null argument");
    *out = nullptr;
    return guarded([&] { *out = new HipllmModel(path, max_sequence, device); });
}

void hipllm_destroy(HipllmModel* m) { delete m; }

int hipllm_reset(HipllmModel* m) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    return guarded([&] { m->model.reset(); });
}

int hipllm_prefill(HipllmModel* m, const int32_t* ids, size_t count, int32_t* next) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    if (!next || (!ids && count)) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_prefill: null argument");
    return guarded([&] { *next = m->model.prefill(std::vector<int32_t>(ids, ids + count)); });
}

int hipllm_decode(HipllmModel* m, int32_t id, int32_t* next) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    if (!next) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_decode: null argument");
    return guarded([&] { *next = m->model.decode(id); });
}

namespace {
void fill_config(const llm::ModelConfig& c, HipllmConfig* out) {
        std::memset(out, 0, sizeof(*out));
        out->layer_count = c.layer_count;
        out->embedding_size = c.embedding_size;
        out->feed_forward_size = c.feed_forward_size;
        out->attention_head_count = c.attention_head_count;
        out->kv_head_count = c.kv_head_count;
        out->head_size = c.head_size;
        out->rotary_dimension = c.rotary_dimension;
        out->vocabulary_size = c.vocabulary_size;
        out->context_length = c.context_length;
        out->parameter_count = c.parameter_count;
        out->stored_weight_bytes = c.stored_weight_bytes;
        out->eos_token_id = c.eos_token_id;
        out->rope_theta = c.rope_theta;
        out->norm_epsilon = c.norm_epsilon;
        std::strncpy(out->architecture, c.architecture.c_str(), sizeof(out->architecture) - 1);
}
}  // namespace

int hipllm_config(const HipllmModel* m, HipllmConfig* out) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_config: null argument");
    return guarded([&] { fill_config(m->model.config(), out); });
}

int hipllm_inspect_gguf(const char* path, HipllmConfig* out) {
    if (!path || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_inspect_gguf: null argument");
    return guarded([&] {
        llm::GgufReader reader(path);
        fill_config(reader.config(), out);
    });
}

size_t hipllm_position(const HipllmModel* m) { return m ? m->model.position() : 0; }
size_t hipllm_max_sequence(const HipllmModel* m) { return m ? m->model.max_sequence() : 0; }
int hipllm_uses_gpu(const HipllmModel* m) { return m && m->model.uses_gpu() ? 1 : 0; }

int hipllm_memory_stats(const HipllmModel* m, HipllmMemoryStats* out) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_memory_stats: null argument");
    const llm::MemoryStats s = m->model.memory_stats();
    out->weight_bytes = s.weight_bytes;
    out->kv_cache_bytes = s.kv_cache_bytes;
    out->recurrent_state_bytes = s.recurrent_state_bytes;
    out->intermediate_bytes = s.intermediate_bytes;
    out->intermediate_is_estimate = s.intermediate_is_estimate ? 1 : 0;
    return HIPLLM_OK;
}

const char* hipllm_device_name(const HipllmModel* m) { return m ? m->model.device_name().c_str() : ""; }

int hipllm_enable_profiling(HipllmModel* m, const char* csv_path) {
    if (!m || !csv_path) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_enable_profiling: null argument");
    return guarded([&] { m->model.enable_profiling(csv_path); });
}

int hipllm_disable_profiling(HipllmModel* m) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_disable_profiling: null argument");
    m->model.disable_profiling();
    return HIPLLM_OK;
}

int hipllm_copy_logits(const HipllmModel* m, float* out, size_t count) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_logits: null argument");
    return guarded([&] { m->model.copy_last_logits(out, count); });
}

int hipllm_set_batched_prefill(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_batched_prefill: null argument");
    return guarded([&] { m->model.set_batched_prefill(enabled != 0); });
}

}  // extern "C"
