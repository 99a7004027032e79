// C ABI of libhipllm.so (declarations and reference citations in
// include/hipllm.h).
#include "../../../include/hipllm.h"

#include "../kernels/common.h"
#include "../kernels/launch.h"
#include "hip_chat.h"
#include "hip_llm.h"
#include "hip_moe.h"
#include "tokenizer.h"

#include <cstring>
#include <exception>
#include <iostream>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>

// The handle holds the backend the CLI would pick for the file's
// architecture (chat.cpp:1019-1035): qwen35moe -> HipMoeLLM, qwen2 -> HipLLM.
struct HipllmModel {
    std::unique_ptr<llm::HipLLM> dense;
    std::unique_ptr<llm::HipMoeLLM> moe;

    template <typename Fn>
    decltype(auto) visit(Fn&& fn) {
        return dense ? fn(*dense) : fn(*moe);
    }
    template <typename Fn>
    decltype(auto) visit(Fn&& fn) const {
        return dense ? fn(static_cast<const llm::HipLLM&>(*dense)) : fn(static_cast<const llm::HipMoeLLM&>(*moe));
    }
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

static hipllm::XGroup* xg(void* p) { return static_cast<hipllm::XGroup*>(p); }
static const hipllm::XGroup* xgc(const void* p) { return static_cast<const hipllm::XGroup*>(p); }

int hipllm_prep_x(const float* x, void* xq, size_t k, void* stream) {
    return status(hipllm::launch_prep_x(x, xg(xq), k, as_stream(stream)),
                  "hipllm_prep_x: invalid arguments (k % 16 == 0, 16-byte aligned buffers) or launch failure");
}

size_t hipllm_gemv_workspace_bytes(size_t k) { return (k + 15) / 16 * sizeof(hipllm::XGroup); }

int hipllm_gemv(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* bias, float* y,
                size_t n, size_t k, void* workspace, void* stream) {
    if (!workspace) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemv: workspace is null");
    hipllm::XGroup* xq = xg(workspace);
    int rc = hipllm::launch_prep_x(x, xq, k, as_stream(stream));
    if (rc != hipllm::kOk) return status(rc, "hipllm_gemv: k must be a positive multiple of 16");
    return status(hipllm::launch_gemv_prepped(type, w, row_bytes, x, xq, bias, nullptr, y, n, k, 0,
                                              as_stream(stream)),
                  "hipllm_gemv: invalid arguments or launch failure");
}

// ------------------------------------------------ GEMV without allocation
// The XGroup form of x lives in a file-scope device array instead of a
// caller workspace. Its device address differs per GPU and is not the host
// name `scratch`, so each device's address comes from hipGetSymbolAddress
// once (the first call on that device, with it current) and is kept here.
static constexpr size_t kNoAllocMaxK = 65536;  // 4 bytes of XGroup form per value: 256 KiB per device
static __device__ __align__(256) unsigned char scratch[kNoAllocMaxK * 4];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's copy of `scratch`, or nullptr with the error set.
void* device_scratch(int* code, const char** what) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
        *code = HIPLLM_RUNTIME_ERROR;
        *what = "hipllm_gemv_noalloc: no usable current HIP device";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            *code = HIPLLM_RUNTIME_ERROR;
            *what = "hipllm_gemv_noalloc: hipGetSymbolAddress(scratch) failed";
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

int hipllm_gemv_noalloc(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* bias, float* y,
                        size_t n, size_t k, void* stream) {
    if (k > kNoAllocMaxK) {
        return fail(HIPLLM_LENGTH_ERROR, "hipllm_gemv_noalloc: k exceeds 65536, the capacity of its static scratch");
    }
    int code = HIPLLM_OK;
    const char* what = "";
    void* ptr = device_scratch(&code, &what);
    if (!ptr) return fail(code, what);
    hipllm::XGroup* xq = static_cast<hipllm::XGroup*>(ptr);
    const int rc = hipllm::launch_prep_x(x, xq, k, as_stream(stream));
    if (rc != hipllm::kOk) return status(rc, "hipllm_gemv_noalloc: k must be a positive multiple of 16");
    return status(hipllm::launch_gemv_prepped(type, w, row_bytes, x, xq, bias, nullptr, y, n, k, 0,
                                              as_stream(stream)),
                  "hipllm_gemv_noalloc: invalid arguments or launch failure");
}

int hipllm_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const void* xq,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        void* stream) {
    return status(hipllm::launch_gemv_prepped(type, w, row_bytes, x, xgc(xq), bias, residual, y, n, k, tiling,
                                              as_stream(stream)),
                  "hipllm_gemv_prepped: invalid arguments or launch failure");
}

int hipllm_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const void* xq, float* y, void* yq, size_t n, size_t k, int tiling, void* stream) {
    return status(hipllm::launch_gemv_swiglu(type, wg, wu, row_bytes, x, xgc(xq), y, xg(yq), n, k, tiling,
                                             as_stream(stream)),
                  "hipllm_gemv_swiglu: invalid arguments or launch failure");
}

int hipllm_gemv_norm(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* gamma, float eps,
                     const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                     void* stream) {
    return status(hipllm::launch_gemv_norm(type, w, row_bytes, x, gamma, eps, bias, residual, y, n, k, tiling,
                                           as_stream(stream)),
                  "hipllm_gemv_norm: invalid arguments or launch failure");
}

int hipllm_gemv_swiglu_norm(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                            const float* gamma, float eps, float* y, void* yq, size_t n, size_t k, int tiling,
                            void* stream) {
    return status(hipllm::launch_gemv_swiglu_norm(type, wg, wu, row_bytes, x, gamma, eps, y, xg(yq), n, k, tiling,
                                                  as_stream(stream)),
                  "hipllm_gemv_swiglu_norm: invalid arguments or launch failure");
}

int hipllm_gemv_multi_norm(const HipllmGemvJob* jobs, size_t count, const float* x, const float* gamma, float eps,
                           size_t k, float* norm, void* normq, void* stream) {
    hipllm::GemvJob js[hipllm::kMultiJobs];
    if (!jobs || count == 0 || count > hipllm::kMultiJobs) {
        return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemv_multi_norm: 1 to 3 jobs");
    }
    for (size_t i = 0; i < count; ++i) {
        const HipllmGemvJob& j = jobs[i];
        if (j.reserved != 0) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemv_multi_norm: reserved must be 0");
        js[i].type = j.type;
        js[i].mode = j.mode;
        js[i].w = j.w;
        js[i].w2 = j.w2;
        js[i].row_bytes = j.row_bytes;
        js[i].bias = j.bias;
        js[i].residual = j.residual;
        js[i].y = j.y;
        js[i].yq = xg(j.yq);
        js[i].n = j.n;
    }
    return status(hipllm::launch_gemv_multi_norm(js, count, x, gamma, eps, k, norm, xg(normq), as_stream(stream)),
                  "hipllm_gemv_multi_norm: invalid arguments (types, k % 32 == 0, k <= 8192, alignment) or launch "
                  "failure");
}

size_t hipllm_x16_bytes(uint32_t type, size_t n, size_t k) { return hipllm::x16_bytes(type, n, k); }

int hipllm_pack_x16(uint32_t type, const void* w, size_t row_bytes, size_t n, size_t k, void* packed, void* stream) {
    return status(hipllm::launch_pack_x16(type, w, row_bytes, n, k, packed, as_stream(stream)),
                  "hipllm_pack_x16: invalid arguments (Q4_K or Q6_K, k % 256 == 0, packed 16-byte aligned, Q4_K rows "
                  "16-byte and Q6_K rows 2-byte aligned) or launch failure");
}

namespace {
hipllm::X16Norm x16_norm(const HipllmX16Norm* n) {
    return hipllm::X16Norm{n->sumsq_in, n->eps, n->gamma_out, static_cast<hipllm::XGroup*>(n->yq_out), n->sumsq_out};
}
}  // namespace

int hipllm_gemv_x16(uint32_t type, const void* packed, const void* xq, const float* bias, const float* residual,
                    float* y, size_t n, size_t k, int waves, const HipllmX16Norm* norm, void* stream) {
    const hipllm::X16Norm nrm = norm ? x16_norm(norm) : hipllm::X16Norm{};
    return status(hipllm::launch_gemv_x16(type, packed, xgc(xq), bias, residual, y, n, k, waves, as_stream(stream),
                                          norm ? &nrm : nullptr),
                  "hipllm_gemv_x16: invalid arguments (Q4_K or Q6_K, k % 256 == 0, a known launch shape, 16-byte "
                  "aligned buffers, a norm before (k <= 8192) or after (n % 16 == 0) the product, not both) or launch "
                  "failure");
}

int hipllm_gemv_x16_swiglu(uint32_t type, const void* gate, const void* up, const void* xq, float* y, void* yq,
                           size_t n, size_t k, int waves, const HipllmX16Norm* norm, void* stream) {
    const hipllm::X16Norm nrm = norm ? x16_norm(norm) : hipllm::X16Norm{};
    return status(hipllm::launch_gemv_x16_swiglu(type, gate, up, xgc(xq), y, xg(yq), n, k, waves, as_stream(stream),
                                                 norm ? &nrm : nullptr),
                  "hipllm_gemv_x16_swiglu: invalid arguments (Q4_K or Q6_K, k % 256 == 0, n % 16 == 0 with yq, a "
                  "known launch shape, 16-byte aligned buffers, only a norm before the products, k <= 8192) or "
                  "launch failure");
}

int hipllm_gemv_x16_grouped(uint32_t type, const void* packed, const void* packed2, const void* xq, size_t ldx,
                            int x_routed, size_t routes, float* y, void* yq, size_t ldy, size_t n, size_t k,
                            size_t experts, const int32_t* order, const int32_t* groups, const uint32_t* ngroups,
                            size_t max_groups, void* stream) {
    return status(hipllm::launch_x16_grouped(type, packed, packed2, xgc(xq), ldx, x_routed, routes, y, xg(yq), ldy, n,
                                             k, experts, order, groups, ngroups, max_groups, as_stream(stream)),
                  "hipllm_gemv_x16_grouped: invalid arguments (Q4_K or Q6_K, k % 256 == 0, n % 16 == 0, 16-byte "
                  "aligned buffers, max_groups <= 65535) or launch failure");
}

int hipllm_gemv_x16_moe_down(uint32_t type_r, const void* down_packed, const int32_t* ids, size_t experts,
                             const void* xq, size_t ldx, size_t k_r, uint32_t type_s, const void* shared_packed,
                             const float* sx, size_t k_s, const float* weights, const float* sgate,
                             const float* residual, float* y, size_t n, size_t routes,
                             const HipllmX16Norm* norm_out, void* stream) {
    const hipllm::X16Norm nrm = norm_out ? x16_norm(norm_out) : hipllm::X16Norm{};
    return status(hipllm::launch_x16_moe_down(type_r, down_packed, ids, experts, xgc(xq), ldx, k_r, type_s,
                                              shared_packed, sx, k_s, weights, sgate, residual, y, n, routes,
                                              as_stream(stream), norm_out ? &nrm : nullptr),
                  "hipllm_gemv_x16_moe_down: invalid arguments (routed Q4_K / Q6_K, shared Q4_K / Q6_K / Q8_0, "
                  "k % 256 == 0, k_s <= 2048, n % 16 == 0, 1..8 routes, 16-byte aligned buffers) or launch failure");
}

int hipllm_gemv_x16_pair(uint32_t type_a, const void* packed_a, size_t n_a, float* y_a, uint32_t type_b,
                         const void* packed_b, size_t n_b, float* y_b, size_t k, const float* x, const float* gamma,
                         float eps, const float* conv_w, float* history, size_t ksize, const void* xq,
                         const double* sumsq, void* stream) {
    return status(hipllm::launch_gemv_x16_pair(type_a, packed_a, n_a, y_a, type_b, packed_b, n_b, y_b, k, x, gamma,
                                                eps, conv_w, history, ksize, as_stream(stream), xgc(xq), sumsq),
                  "hipllm_gemv_x16_pair: invalid arguments (Q4_K or Q6_K, k % 256 == 0, k <= 8192, 16-byte aligned "
                  "buffers, eps > 0, ksize 2..4 with a history) or launch failure");
}

int hipllm_gemv_x16_routed(uint32_t type, const void* packed, const void* packed2, const void* xq, size_t ldx,
                           int x_routed, float* y, void* yq, size_t ldy, size_t n, size_t k, size_t experts,
                           size_t routes, const int32_t* ids, const float* logits, int32_t* ids_out,
                           float* weights_out, int waves, void* stream) {
    return status(hipllm::launch_gemv_x16_routed(type, packed, packed2, xgc(xq), ldx, x_routed, y, xg(yq), ldy, n, k,
                                                 experts, routes, ids, logits, ids_out, weights_out, waves,
                                                 as_stream(stream)),
                  "hipllm_gemv_x16_routed: invalid arguments (Q4_K or Q6_K, k % 256 == 0, n % 16 == 0, routes <= 8, "
                  "experts <= 256 with logits, ids or logits, a known launch shape, 16-byte aligned buffers) or "
                  "launch failure");
}

int hipllm_to_f16(const float* x, size_t ldx, void* xh, float* xscale, size_t m, size_t k, void* stream) {
    return status(hipllm::launch_to_f16(x, ldx, xh, xscale, m, k, as_stream(stream)),
                  "hipllm_to_f16: invalid arguments (k % 8 == 0, 16-byte aligned buffers) or launch failure");
}

int hipllm_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xh, const float* xscale,
                     const float* bias, const float* residual, float* y, size_t m, size_t n, size_t k, int tile,
                     int splits, void* workspace, size_t workspace_bytes, void* stream) {
    return status(hipllm::launch_gemm_mfma(type, w, row_bytes, xh, xscale, bias, residual, y, m, n, k, tile, splits,
                                           as_stream(stream), 0, workspace, workspace_bytes),
                  "hipllm_gemm_mfma: invalid arguments (k % 128 == 0, tile -1..5, splits 0..1024, workspace for an "
                  "explicit split) or launch failure");
}

int hipllm_rmsnorm_f16(const float* x, const float* gamma, float* norm, void* xh, float* xscale, size_t rows,
                       size_t cols, float eps, void* stream) {
    return status(hipllm::launch_rmsnorm_f16(x, gamma, norm, xh, xscale, rows, cols, eps, as_stream(stream)),
                  "hipllm_rmsnorm_f16: invalid arguments (cols % 16 == 0, cols <= 8192, 16-byte aligned buffers, "
                  "eps > 0) or launch failure");
}

size_t hipllm_gemm_swiglu_workspace_bytes(size_t m, size_t n, size_t k) { return hipllm::gemm_swiglu_bytes(m, n, k); }

int hipllm_gemm_mfma_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xh,
                            const float* xscale, float* y, size_t m, size_t n, size_t k, void* workspace,
                            size_t workspace_bytes, void* stream) {
    return status(hipllm::launch_gemm_mfma_swiglu(type, wg, wu, row_bytes, xh, xscale, y, m, n, k, n, workspace,
                                                  workspace_bytes, as_stream(stream)),
                  "hipllm_gemm_mfma_swiglu: invalid arguments (Q4_K / Q6_K / Q8_0 / Q5_0 weights, k % 128 == 0, a "
                  "workspace of hipllm_gemm_swiglu_workspace_bytes) or launch failure");
}

int hipllm_gemm_mfma_swiglu_f16(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xh,
                                const float* xscale, void* yh, float* yscale, size_t m, size_t n, size_t k,
                                void* workspace, size_t workspace_bytes, void* stream) {
    if (!yh) return status(hipllm::kInvalidArgument, "hipllm_gemm_mfma_swiglu_f16: yh is required");
    return status(hipllm::launch_gemm_mfma_swiglu(type, wg, wu, row_bytes, xh, xscale, nullptr, m, n, k, n, workspace,
                                                  workspace_bytes, as_stream(stream), yh, yscale),
                  "hipllm_gemm_mfma_swiglu_f16: invalid arguments (as hipllm_gemm_mfma_swiglu, and n % 8 == 0, "
                  "n <= 32768, yh 16-byte aligned, yscale given) or launch failure");
}

size_t hipllm_gemm_mfma_workspace_bytes(size_t m, size_t n, size_t k, int tile, int splits) {
    return hipllm::gemm_split_bytes(m, n, k, tile, splits);
}

// Workspace: the fp16 rows (256-byte aligned), then the row scales.
size_t hipllm_gemm_workspace_bytes(size_t m, size_t k) { return (m * k * 2 + 255) / 256 * 256 + (m * 4 + 255) / 256 * 256; }

int hipllm_gemm(uint32_t type, const void* w, size_t row_bytes, const float* x, size_t ldx, const float* bias,
                float* y, size_t m, size_t n, size_t k, void* workspace, void* stream) {
    if (!workspace) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_gemm: workspace is null");
    float* xscale = reinterpret_cast<float*>(static_cast<char*>(workspace) + (m * k * 2 + 255) / 256 * 256);
    const int rc = hipllm::launch_to_f16(x, ldx, workspace, xscale, m, k, as_stream(stream));
    if (rc != hipllm::kOk) return status(rc, "hipllm_gemm: invalid activation arguments");
    return status(hipllm::launch_gemm_mfma(type, w, row_bytes, workspace, xscale, bias, nullptr, y, m, n, k, -1, 0,
                                           as_stream(stream)),
                  "hipllm_gemm: invalid arguments (k % 128 == 0) or launch failure");
}

int hipllm_rmsnorm(const float* x, const float* gamma, float* y, void* yq, size_t rows, size_t cols, float eps,
                   void* stream) {
    return status(hipllm::launch_rmsnorm(x, gamma, y, xg(yq), rows, cols, eps, as_stream(stream)),
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

int hipllm_attn_decode_rope(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                            float* out, void* outq, float* scratch, size_t hq, size_t hkv, size_t d, size_t pos,
                            float scale, void* stream) {
    return status(hipllm::launch_attn_decode_rope(qkv, cos_sin, rot, kcache, vcache, out, xg(outq), scratch, hq, hkv,
                                                  d, pos, scale, as_stream(stream)),
                  "hipllm_attn_decode_rope: invalid arguments or launch failure");
}

int hipllm_attn_decode_rope_gated(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                                  const float* gate, float* out, void* outq, float* scratch, size_t hq, size_t hkv,
                                  size_t d, size_t pos, float scale, void* stream) {
    if (!gate) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_attn_decode_rope_gated: gate is required");
    return status(hipllm::launch_attn_decode_rope(qkv, cos_sin, rot, kcache, vcache, out, xg(outq), scratch, hq, hkv,
                                                  d, pos, scale, as_stream(stream), nullptr, 0, gate),
                  "hipllm_attn_decode_rope_gated: invalid arguments or launch failure");
}

int hipllm_attn_decode_qgate(const float* mixed, const float* kv, const float* q_gamma, const float* k_gamma,
                             float eps, const float* cos_sin, size_t rot, float* kcache, float* vcache, float* out,
                             void* outq, size_t hq, size_t hkv, size_t d, size_t pos, float scale, void* stream) {
    return status(hipllm::launch_attn_decode_qgate(mixed, kv, q_gamma, k_gamma, eps, cos_sin, rot, kcache, vcache, out,
                                                   xg(outq), hq, hkv, d, pos, scale, as_stream(stream)),
                  "hipllm_attn_decode_qgate: invalid arguments (2 to 4 key chunks, d 64 / 128 / 256) or launch "
                  "failure");
}

size_t hipllm_attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len) {
    return hipllm::attn_decode_scratch_floats(hq, d, max_len);
}

int hipllm_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, void* outq,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, void* stream) {
    return status(hipllm::launch_attn_decode(q, kcache, vcache, out, xg(outq), scratch, hq, hkv, d, len, scale,
                                             as_stream(stream)),
                  "hipllm_attn_decode: invalid arguments or launch failure");
}

size_t hipllm_argmax_scratch_bytes(size_t n) { return hipllm::argmax_scratch_bytes(n); }

int hipllm_argmax(const float* x, size_t n, uint32_t* out, void* scratch, void* stream) {
    return status(hipllm::launch_argmax(x, n, out, scratch, as_stream(stream)),
                  "hipllm_argmax: invalid arguments or launch failure");
}

int hipllm_swiglu(const float* g, const float* u, float* y, void* yq, size_t n, void* stream) {
    return status(hipllm::launch_swiglu(g, u, y, xg(yq), n, as_stream(stream)),
                  "hipllm_swiglu: invalid arguments or launch failure");
}

int hipllm_create_ex(const char* path, size_t max_sequence, int device, size_t expert_cache_count,
                     HipllmModel** out) {
    if (!path || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_create: null argument");
    *out = nullptr;
    return guarded([&] {
        const std::string arch = llm::GgufReader(path).config().architecture;
        auto m = std::make_unique<HipllmModel>();
        const std::string spec = device < 0 ? std::string() : std::to_string(device);
        if (arch == "qwen35moe") {
            m->moe = std::make_unique<llm::HipMoeLLM>(path, max_sequence, spec, expert_cache_count);
        } else {
            m->dense = std::make_unique<llm::HipLLM>(path, max_sequence, spec);
        }
        *out = m.release();
    });
}

int hipllm_create(const char* path, size_t max_sequence, int device, HipllmModel** out) {
    return hipllm_create_ex(path, max_sequence, device, 8, out);
}

void hipllm_destroy(HipllmModel* m) { delete m; }

int hipllm_reset(HipllmModel* m) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    return guarded([&] { m->visit([](auto& b) { b.reset(); }); });
}

int hipllm_prefill(HipllmModel* m, const int32_t* ids, size_t count, int32_t* next) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    if (!next || (!ids && count)) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_prefill: null argument");
    return guarded([&] {
        const std::vector<int32_t> v(ids, ids + count);
        *next = m->visit([&](auto& b) { return b.prefill(v); });
    });
}

int hipllm_decode(HipllmModel* m, int32_t id, int32_t* next) {
    if (!m) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    if (!next) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_decode: null argument");
    return guarded([&] { *next = m->visit([&](auto& b) { return b.decode(id); }); });
}

namespace {
void fill_config(const llm::GgufModelConfig& c, HipllmConfig* out) {
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
        out->full_attention_interval = c.full_attention_interval;
        out->expert_count = c.expert_count;
        out->expert_used_count = c.expert_used_count;
        out->expert_feed_forward_size = c.expert_feed_forward_size;
        out->shared_expert_feed_forward_size = c.shared_expert_feed_forward_size;
        out->ssm_conv_kernel = c.ssm_conv_kernel;
        out->ssm_state_size = c.ssm_state_size;
        out->ssm_group_count = c.ssm_group_count;
        out->ssm_time_step_rank = c.ssm_time_step_rank;
        out->ssm_inner_size = c.ssm_inner_size;
}
}  // namespace

int hipllm_config(const HipllmModel* m, HipllmConfig* out) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_config: null argument");
    return guarded([&] { fill_config(m->visit([](const auto& b) -> const llm::GgufModelConfig& { return b.config(); }), out); });
}

int hipllm_inspect_gguf(const char* path, HipllmConfig* out) {
    if (!path || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_inspect_gguf: null argument");
    return guarded([&] {
        llm::GgufReader reader(path);
        fill_config(reader.config(), out);
    });
}

size_t hipllm_position(const HipllmModel* m) {
    return m ? m->visit([](const auto& b) { return b.position(); }) : 0;
}
size_t hipllm_max_sequence(const HipllmModel* m) {
    return m ? m->visit([](const auto& b) { return b.max_sequence(); }) : 0;
}
int hipllm_uses_gpu(const HipllmModel* m) { return m && m->visit([](const auto& b) { return b.uses_gpu(); }) ? 1 : 0; }

int hipllm_memory_stats(const HipllmModel* m, HipllmMemoryStats* out) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_memory_stats: null argument");
    const llm::MemoryStats s = m->visit([](const auto& b) { return b.memory_stats(); });
    out->weight_bytes = s.weight_bytes;
    out->kv_cache_bytes = s.kv_cache_bytes;
    out->recurrent_state_bytes = s.recurrent_state_bytes;
    out->intermediate_bytes = s.intermediate_bytes;
    out->intermediate_is_estimate = s.intermediate_is_estimate ? 1 : 0;
    return HIPLLM_OK;
}

const char* hipllm_device_name(const HipllmModel* m) {
    return m ? m->visit([](const auto& b) -> const std::string& { return b.device_name(); }).c_str() : "";
}

int hipllm_enable_profiling(HipllmModel* m, const char* csv_path, int detailed) {
    if (!m || !csv_path) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_enable_profiling: null argument");
    return guarded([&] { m->visit([&](auto& b) { b.enable_profiling(csv_path, detailed != 0); }); });
}

namespace {
const llm::GgufModelConfig* config_of(const HipllmModel* m) {
    return &m->visit([](const auto& b) -> const llm::GgufModelConfig& { return b.config(); });
}
}  // namespace

size_t hipllm_vocabulary_count(const HipllmModel* m) { return m ? config_of(m)->vocabulary.size() : 0; }

const char* hipllm_vocabulary_token(const HipllmModel* m, size_t index) {
    if (!m) return nullptr;
    const auto& v = config_of(m)->vocabulary;
    return index < v.size() ? v[index].c_str() : nullptr;
}

size_t hipllm_merge_count(const HipllmModel* m) { return m ? config_of(m)->merges.size() : 0; }

const char* hipllm_merge(const HipllmModel* m, size_t index) {
    if (!m) return nullptr;
    const auto& v = config_of(m)->merges;
    return index < v.size() ? v[index].c_str() : nullptr;
}

const char* hipllm_tokenizer_pre(const HipllmModel* m) { return m ? config_of(m)->tokenizer_pre.c_str() : ""; }

int hipllm_disable_profiling(HipllmModel* m) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_disable_profiling: null argument");
    m->visit([](auto& b) { b.disable_profiling(); });
    return HIPLLM_OK;
}

int hipllm_copy_logits(const HipllmModel* m, float* out, size_t count) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_logits: null argument");
    return guarded([&] { m->visit([&](const auto& b) { b.copy_last_logits(out, count); }); });
}

int hipllm_set_fused_norms(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_fused_norms: null argument");
    if (!m->dense) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_fused_norms: qwen2 models only");
    return guarded([&] { m->dense->set_fused_norms(enabled != 0); });
}

int hipllm_set_packed_decode(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_packed_decode: null argument");
    if (!m->dense) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_packed_decode: qwen2 models only");
    return guarded([&] { m->dense->set_packed_decode(enabled != 0); });
}

int hipllm_set_decode_graphs(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_decode_graphs: null argument");
    return guarded([&] { m->visit([&](auto& model) { model.set_decode_graphs(enabled != 0); }); });
}

int hipllm_set_batched_prefill(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_batched_prefill: null argument");
    return guarded([&] {
        if (m->dense) {
            m->dense->set_batched_prefill(enabled != 0);
        } else {
            m->moe->set_matmul_prefill(enabled != 0);
        }
    });
}

int hipllm_copy_routes(const HipllmModel* m, int32_t* out, size_t count) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_routes: null argument");
    if (!m->moe) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_routes: not a MoE model");
    return guarded([&] { m->moe->copy_last_routes(out, count); });
}

int hipllm_set_route_probe(HipllmModel* m, int enabled) {
    if (!m) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_route_probe: null argument");
    if (!m->moe) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_set_route_probe: not a MoE model");
    return guarded([&] { m->moe->set_route_probe(enabled != 0); });
}

int hipllm_copy_router_logits(const HipllmModel* m, float* out, size_t count) {
    if (!m || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_router_logits: null argument");
    if (!m->moe) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_copy_router_logits: not a MoE model");
    return guarded([&] { m->moe->copy_last_router_logits(out, count); });
}

size_t hipllm_expert_cache_count(const HipllmModel* m) { return m && m->moe ? m->moe->expert_cache_count() : 0; }

int hipllm_expert_cache_stats(const HipllmModel* m, uint64_t* hits, uint64_t* misses) {
    if (!m || !hits || !misses) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_expert_cache_stats: null argument");
    const llm::HipExpertCacheStats s = m->moe ? m->moe->expert_cache_stats() : llm::HipExpertCacheStats{};
    *hits = s.hits;
    *misses = s.misses;
    return HIPLLM_OK;
}

// ---------------------------------------------------------------- MoE kernels

int hipllm_gemv_batched(uint32_t type, const void* w, const void* wu, size_t row_bytes, const float* x,
                        const void* xq, const float* bias, const float* residual, float* y, void* yq, size_t n,
                        size_t k, size_t vectors, const int32_t* ids, size_t experts, size_t routes,
                        size_t expert_stride, int x_routed, size_t ldx, size_t ldy, void* stream) {
    return status(hipllm::launch_gemv_batched(type, w, wu, row_bytes, x, xgc(xq), bias, residual, y, xg(yq), n, k,
                                              vectors,
                                              ids, experts, routes, expert_stride, x_routed, ldx, ldy,
                                              as_stream(stream)),
                  "hipllm_gemv_batched: invalid arguments or launch failure");
}

int hipllm_gemv_routed_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                              const void* xq, size_t ldx, float* y, void* yq, size_t n, size_t k, size_t tokens,
                              const float* logits, size_t ld_logits, size_t experts, size_t routes,
                              size_t expert_stride, int32_t* ids_out, float* weights_out, void* stream) {
    return status(hipllm::launch_gemv_routed_swiglu(type, wg, wu, row_bytes, x,
                                                    static_cast<const hipllm::XGroup*>(xq), ldx, y, xg(yq), n, k,
                                                    tokens, logits, ld_logits, experts, routes, expert_stride,
                                                    ids_out, weights_out, as_stream(stream)),
                  "hipllm_gemv_routed_swiglu: invalid arguments (quantized weights, experts <= 256, routes <= 8) or "
                  "launch failure");
}

int hipllm_gemv_moe_combine(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* residual,
                            const float* down, const float* weights, const float* sgate, size_t routes, float* y,
                            size_t n, size_t k, void* stream) {
    return status(hipllm::launch_gemv_moe_combine(type, w, row_bytes, x, residual, down, weights, sgate, routes, y, n,
                                                  k, as_stream(stream)),
                  "hipllm_gemv_moe_combine: invalid arguments or launch failure");
}

size_t hipllm_matmul_f32_scratch_floats(size_t m, size_t n, size_t k) {
    return hipllm::matmul_f32_scratch_floats(m, n, k);
}

int hipllm_matmul_f32(const float* x, size_t ldx, const float* w, size_t ldw, float* y, size_t ldy, size_t m,
                      size_t n, size_t k, float* scratch, size_t scratch_floats, void* stream) {
    return status(hipllm::launch_matmul_f32(x, ldx, w, ldw, y, ldy, m, n, k, scratch, scratch_floats,
                                            as_stream(stream)),
                  "hipllm_matmul_f32: invalid arguments or launch failure");
}

size_t hipllm_route_groups_max(size_t n, size_t experts, size_t vmax) {
    return hipllm::route_groups_max(n, experts, vmax);
}

int hipllm_route_groups(const int32_t* ids, size_t n, size_t experts, size_t vmax, int32_t* order, int32_t* groups,
                        uint32_t* ngroups, void* stream) {
    return status(hipllm::launch_route_groups(ids, n, experts, vmax, order, groups, ngroups, as_stream(stream)),
                  "hipllm_route_groups: invalid arguments (n <= 16384, experts <= 1024) or launch failure");
}

int hipllm_gemm_gather(uint32_t type, const void* w, size_t row_bytes, const void* xh, const float* xscale, float* y,
                       size_t n, size_t k, size_t ldy, const int32_t* order, const int32_t* groups,
                       const uint32_t* ngroups, size_t max_groups, size_t expert_stride, size_t routes, int x_routed,
                       void* stream) {
    return status(hipllm::launch_gemm_gather(type, w, row_bytes, xh, xscale, y, n, k, ldy, order, groups, ngroups,
                                             max_groups, expert_stride, routes, x_routed, as_stream(stream)),
                  "hipllm_gemm_gather: invalid arguments (k % 128 == 0, max_groups <= 65535, alignment) or launch "
                  "failure");
}

int hipllm_router_topk(const float* logits, size_t ld, size_t tokens, size_t experts, size_t k, int32_t* ids,
                       float* weights, void* stream) {
    return status(hipllm::launch_router_topk(logits, ld, tokens, experts, k, ids, weights, as_stream(stream)),
                  "hipllm_router_topk: invalid arguments (k <= 8, experts <= 1024) or launch failure");
}

int hipllm_moe_combine_norm(const float* residual, const float* down, const float* w, const float* shared,
                            const float* sgate, size_t ld_sgate, float* out, const float* gamma, float* norm,
                            void* normq, size_t tokens, size_t h, size_t k, float eps, void* stream) {
    return status(hipllm::launch_moe_combine_norm(residual, down, w, shared, sgate, ld_sgate, out, gamma, norm,
                                                  static_cast<hipllm::XGroup*>(normq), tokens, h, k, eps,
                                                  as_stream(stream)),
                  "hipllm_moe_combine_norm: invalid arguments or launch failure");
}

int hipllm_moe_combine(const float* residual, const float* down, const float* w, const float* shared,
                       const float* sgate, size_t ld_sgate, float* out, size_t tokens, size_t h, size_t k,
                       void* stream) {
    return status(hipllm::launch_moe_combine(residual, down, w, shared, sgate, ld_sgate, out, tokens, h, k,
                                             as_stream(stream)),
                  "hipllm_moe_combine: invalid arguments or launch failure");
}

int hipllm_gdn_gates(const float* alpha, const float* beta_raw, size_t ld, const float* dt_bias, const float* a,
                     float* decay, float* beta, size_t tokens, size_t heads, void* stream) {
    return status(hipllm::launch_gdn_gates(alpha, beta_raw, ld, dt_bias, a, decay, beta, tokens, heads,
                                           as_stream(stream)),
                  "hipllm_gdn_gates: invalid arguments or launch failure");
}

int hipllm_conv1d_silu(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, void* stream) {
    return status(hipllm::launch_conv1d_silu(x, ldx, history, w, out, ldo, tokens, channels, ksize,
                                             as_stream(stream)),
                  "hipllm_conv1d_silu: invalid arguments (2 <= k <= 9, out != x) or launch failure");
}

int hipllm_l2norm_heads(float* x, size_t ld, size_t tokens, size_t heads, size_t d, float eps, void* stream) {
    return status(hipllm::launch_l2norm_heads(x, ld, tokens, heads, d, eps, as_stream(stream)),
                  "hipllm_l2norm_heads: invalid arguments or launch failure");
}

int hipllm_gdn_scan(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* decay,
                    const float* beta, float* state, float* out, size_t ldo, size_t tokens, size_t value_heads,
                    size_t key_heads, size_t d, void* stream) {
    return status(hipllm::launch_gdn_scan(q, k, ldqk, v, ldv, decay, beta, state, out, ldo, tokens, value_heads,
                                          key_heads, d, as_stream(stream)),
                  "hipllm_gdn_scan: invalid arguments (state size 64 or 128) or launch failure");
}

size_t hipllm_gdn_chunk_scratch_floats(size_t tokens, size_t value_heads) {
    return hipllm::gdn_chunk_scratch_floats(tokens, value_heads);
}

int hipllm_gdn_scan_chunked(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv,
                            const float* decay, const float* beta, float* state, float* out, size_t ldo,
                            size_t tokens, size_t value_heads, size_t key_heads, size_t d, float* scratch,
                            size_t scratch_floats, void* stream) {
    return status(hipllm::launch_gdn_scan_chunked(q, k, ldqk, v, ldv, decay, beta, state, out, ldo, tokens,
                                                  value_heads, key_heads, d, scratch, scratch_floats,
                                                  as_stream(stream)),
                  "hipllm_gdn_scan_chunked: invalid arguments (state size 64 or 128, scratch size) or launch "
                  "failure");
}

int hipllm_gated_rmsnorm(const float* o, size_t ldo, const float* gamma, const float* z, size_t ldz, float* y,
                         void* yq, size_t ldy, size_t tokens, size_t heads, size_t d, float eps, void* stream) {
    return status(hipllm::launch_gated_rmsnorm(o, ldo, gamma, z, ldz, y, xg(yq), ldy, tokens, heads, d, eps,
                                               as_stream(stream)),
                  "hipllm_gated_rmsnorm: invalid arguments or launch failure");
}

int hipllm_conv_l2norm(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, size_t norm_channels, size_t d, float eps,
                       void* stream) {
    return status(hipllm::launch_conv_l2norm(x, ldx, history, w, out, ldo, tokens, channels, ksize, norm_channels, d,
                                             eps, as_stream(stream)),
                  "hipllm_conv_l2norm: invalid arguments or launch failure");
}

int hipllm_gdn_scan_gated(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* alpha,
                          const float* beta_raw, size_t ld_ab, const float* dt_bias, const float* a, float* state,
                          const float* z, size_t ldz, const float* gamma, float* y, void* yq, size_t ldy,
                          size_t tokens, size_t value_heads, size_t key_heads, size_t d, float eps, void* stream) {
    return status(hipllm::launch_gdn_scan_gated(q, k, ldqk, v, ldv, alpha, beta_raw, ld_ab, dt_bias, a, state, z, ldz,
                                                gamma, y, xg(yq), ldy, tokens, value_heads, key_heads, d, eps,
                                                as_stream(stream)),
                  "hipllm_gdn_scan_gated: invalid arguments (state size 64 or 128) or launch failure");
}

int hipllm_gdn_decode(const float* qkv, const float* x, const float* x_gamma, const float* ab_w, size_t hidden,
                      const float* dt_bias, const float* a, float* state, const float* z, const float* gamma, float* y,
                      void* yq, size_t value_heads, size_t key_heads, size_t d, float eps, void* stream) {
    return status(hipllm::launch_gdn_decode(qkv, x, x_gamma, ab_w, hidden, dt_bias, a, state, z, gamma, y, xg(yq),
                                            value_heads, key_heads, d, eps, as_stream(stream)),
                  "hipllm_gdn_decode: invalid arguments (state size 64 or 128, hidden <= 4096) or launch failure");
}

int hipllm_split_qgate_norm(const float* mixed, size_t ldm, const float* kv, size_t ldkv, const float* q_gamma,
                            const float* k_gamma, float* qkv, size_t ldqkv, float* gate, size_t ldg, size_t tokens,
                            size_t hq, size_t hkv, size_t d, float eps, void* stream) {
    return status(hipllm::launch_split_qgate_norm(mixed, ldm, kv, ldkv, q_gamma, k_gamma, qkv, ldqkv, gate, ldg,
                                                  tokens, hq, hkv, d, eps, as_stream(stream)),
                  "hipllm_split_qgate_norm: invalid arguments or launch failure");
}

int hipllm_gate_mul(const float* a, const float* g, float* y, void* yq, size_t n, void* stream) {
    return status(hipllm::launch_gate_mul(a, g, y, xg(yq), n, as_stream(stream)),
                  "hipllm_gate_mul: invalid arguments (n % 16 == 0) or launch failure");
}

int hipllm_attn_prefill(const float* q, size_t q_stride, const float* kcache, const float* vcache, float* out,
                        size_t out_stride, size_t rows, size_t hq, size_t hkv, size_t d, size_t pos0, float scale,
                        void* stream) {
    return status(hipllm::launch_attn_prefill(q, q_stride, kcache, vcache, out, out_stride, rows, hq, hkv, d, pos0,
                                              scale, as_stream(stream)),
                  "hipllm_attn_prefill: invalid arguments or launch failure");
}

}  // extern "C"

// ------------------------------------------------------------ text front end

struct HipllmTokenizer {
    llm::QwenTokenizer impl;
};

namespace {

// Copy bytes out under the (capacity, *length) protocol.
int put_bytes(const std::string& s, char* out, size_t capacity, size_t* length, const char* what) {
    if (!length) return fail(HIPLLM_INVALID_ARGUMENT, what);
    *length = s.size();
    if (capacity < s.size() || (!out && !s.empty())) return fail(HIPLLM_LENGTH_ERROR, what);
    if (!s.empty()) std::memcpy(out, s.data(), s.size());
    return HIPLLM_OK;
}

template <typename T>
int put_values(const std::vector<T>& v, T* out, size_t capacity, size_t* count, const char* what) {
    if (!count) return fail(HIPLLM_INVALID_ARGUMENT, what);
    *count = v.size();
    if (capacity < v.size() || (!out && !v.empty())) return fail(HIPLLM_LENGTH_ERROR, what);
    std::copy(v.begin(), v.end(), out);
    return HIPLLM_OK;
}

void to_c(const llm::chat::GenerationStats& s, HipllmGenerationStats* o) {
    std::memset(o, 0, sizeof(*o));
    o->prefill_ms = s.prefill_ms;
    o->decode_ms = s.decode_ms;
    o->total_ms = s.total_ms;
    o->prompt_tokens = s.prompt_tokens;
    o->generated_tokens = s.generated_tokens;
    o->decode_steps = s.decode_steps;
    o->used_gpu = s.used_gpu ? 1 : 0;
    o->stopped = s.stopped ? 1 : 0;
    o->has_expert_cache_stats = s.has_expert_cache_stats ? 1 : 0;
    o->expert_cache_hits = s.expert_cache_hits;
    o->expert_cache_misses = s.expert_cache_misses;
    o->memory.weight_bytes = s.memory.weight_bytes;
    o->memory.kv_cache_bytes = s.memory.kv_cache_bytes;
    o->memory.recurrent_state_bytes = s.memory.recurrent_state_bytes;
    o->memory.intermediate_bytes = s.memory.intermediate_bytes;
    o->memory.intermediate_is_estimate = s.memory.intermediate_is_estimate ? 1 : 0;
}

llm::chat::GenerationStats from_c(const HipllmGenerationStats& o) {
    llm::chat::GenerationStats s;
    s.prefill_ms = o.prefill_ms;
    s.decode_ms = o.decode_ms;
    s.total_ms = o.total_ms;
    s.prompt_tokens = o.prompt_tokens;
    s.generated_tokens = o.generated_tokens;
    s.decode_steps = o.decode_steps;
    s.used_gpu = o.used_gpu != 0;
    s.stopped = o.stopped != 0;
    s.has_expert_cache_stats = o.has_expert_cache_stats != 0;
    s.expert_cache_hits = o.expert_cache_hits;
    s.expert_cache_misses = o.expert_cache_misses;
    s.memory.weight_bytes = o.memory.weight_bytes;
    s.memory.kv_cache_bytes = o.memory.kv_cache_bytes;
    s.memory.recurrent_state_bytes = o.memory.recurrent_state_bytes;
    s.memory.intermediate_bytes = o.memory.intermediate_bytes;
    s.memory.intermediate_is_estimate = o.memory.intermediate_is_estimate != 0;
    return s;
}

}  // namespace

extern "C" {

int hipllm_tokenizer_create(const char* const* vocabulary, size_t vocabulary_count, const char* const* merges,
                            size_t merge_count, const char* tokenizer_pre, HipllmTokenizer** out) {
    if (!out || (!vocabulary && vocabulary_count) || (!merges && merge_count)) {
        return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_tokenizer_create: null argument");
    }
    *out = nullptr;
    return guarded([&] {
        std::vector<std::string> v, m;
        v.reserve(vocabulary_count);
        m.reserve(merge_count);
        for (size_t i = 0; i < vocabulary_count; ++i) {
            if (!vocabulary[i]) throw std::invalid_argument("hipllm_tokenizer_create: null vocabulary entry");
            v.emplace_back(vocabulary[i]);
        }
        for (size_t i = 0; i < merge_count; ++i) {
            if (!merges[i]) throw std::invalid_argument("hipllm_tokenizer_create: null merge entry");
            m.emplace_back(merges[i]);
        }
        *out = new HipllmTokenizer{llm::QwenTokenizer(v, m, tokenizer_pre ? tokenizer_pre : "")};
    });
}

int hipllm_tokenizer_from_model(const HipllmModel* model, HipllmTokenizer** out) {
    if (!model || !out) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_tokenizer_from_model: null argument");
    *out = nullptr;
    return guarded([&] {
        const llm::GgufModelConfig& c = *config_of(model);
        if (c.vocabulary.empty() || c.merges.empty()) {
            throw std::runtime_error("model does not contain Qwen tokenizer vocabulary/merges");
        }
        *out = new HipllmTokenizer{llm::QwenTokenizer(c.vocabulary, c.merges, c.tokenizer_pre)};
    });
}

void hipllm_tokenizer_destroy(HipllmTokenizer* t) { delete t; }

int hipllm_tokenize(const HipllmTokenizer* t, const char* text, size_t length, int32_t* ids, size_t capacity,
                    size_t* count) {
    if (!t || (!text && length)) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_tokenize: null argument");
    int rc = HIPLLM_OK;
    const int g = guarded([&] {
        const std::vector<int32_t> v = t->impl.encode(std::string(text ? text : "", length));
        rc = put_values(v, ids, capacity, count, "hipllm_tokenize: capacity is smaller than the token count");
    });
    return g != HIPLLM_OK ? g : rc;
}

int32_t hipllm_token_id(const HipllmTokenizer* t, const char* token) {
    return t && token ? t->impl.id(token) : -1;
}

int hipllm_token_is_special(const HipllmTokenizer* t, int32_t token) { return t && t->impl.is_special(token) ? 1 : 0; }

int hipllm_decode_piece(const HipllmTokenizer* t, int32_t token, char* out, size_t capacity, size_t* length) {
    if (!t) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_decode_piece: null argument");
    return put_bytes(t->impl.decode_piece(token), out, capacity, length,
                     "hipllm_decode_piece: null length or capacity too small");
}

int hipllm_pretokenize(const HipllmTokenizer* t, const char* text, size_t length, size_t* ranges, size_t capacity,
                       size_t* count) {
    if (!t || (!text && length) || !count) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_pretokenize: null argument");
    int rc = HIPLLM_OK;
    const int g = guarded([&] {
        const auto pieces = t->impl.pieces(std::string(text ? text : "", length));
        std::vector<size_t> flat;
        flat.reserve(pieces.size() * 2);
        for (const auto& p : pieces) {
            flat.push_back(p.first);
            flat.push_back(p.second);
        }
        rc = put_values(flat, ranges, capacity, count, "hipllm_pretokenize: capacity is smaller than 2 * pieces");
        *count = pieces.size();
    });
    return g != HIPLLM_OK ? g : rc;
}

int hipllm_chat_prompt(const char* system, const char* user, char* out, size_t capacity, size_t* length) {
    if (!system || !user) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_chat_prompt: null argument");
    return put_bytes(llm::chat_prompt(system, user), out, capacity, length,
                     "hipllm_chat_prompt: null length or capacity too small");
}

int hipllm_stop_tokens(const HipllmModel* model, const HipllmTokenizer* t, int32_t* out, size_t capacity,
                       size_t* count) {
    if (!model || !t) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_stop_tokens: null argument");
    int rc = HIPLLM_OK;
    const int g = guarded([&] {
        const int32_t im_end = t->impl.id("<|im_end|>");
        if (im_end < 0) throw std::runtime_error("model vocabulary has no <|im_end|> token");
        const auto v = llm::chat::make_stop_tokens(t->impl, *config_of(model), im_end, t->impl.id("</s>"));
        rc = put_values(v, out, capacity, count, "hipllm_stop_tokens: capacity is smaller than the stop list");
    });
    return g != HIPLLM_OK ? g : rc;
}

int hipllm_run(HipllmModel* model, const int32_t* ids, size_t count, size_t max_new_tokens, const int32_t* stop_ids,
               size_t stop_count, HipllmTokenSink sink, void* user, int32_t* tokens, size_t capacity,
               size_t* generated, HipllmGenerationStats* stats) {
    if (!model) return fail(HIPLLM_RUNTIME_ERROR, "HIP model is not initialized");
    if ((!ids && count) || (!stop_ids && stop_count)) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_run: null argument");
    return guarded([&] {
        std::vector<int32_t> prompt(ids, ids + count);
        const std::vector<int32_t> stop(stop_ids, stop_ids + stop_count);
        llm::chat::TokenSink fn;
        if (sink) fn = [sink, user](int32_t t) { sink(t, user); };
        const llm::chat::GenerationResult r =
            model->visit([&](auto& b) { return llm::chat::run(b, std::move(prompt), max_new_tokens, stop, fn); });
        if (tokens) {
            std::copy_n(r.generated_tokens.begin(), std::min(capacity, r.generated_tokens.size()), tokens);
        }
        if (generated) *generated = r.generated_tokens.size();
        if (stats) to_c(r.stats, stats);
    });
}

int hipllm_format_generation_stats(const HipllmGenerationStats* stats, char* out, size_t capacity, size_t* length) {
    if (!stats) return fail(HIPLLM_INVALID_ARGUMENT, "hipllm_format_generation_stats: null argument");
    return put_bytes(llm::chat::format_generation_stats(from_c(*stats)), out, capacity, length,
                     "hipllm_format_generation_stats: null length or capacity too small");
}

int hipllm_chat_main(int argc, char** argv) {
    return llm::chat::run_cli(argc, argv, std::cin, std::cout, std::cerr);
}

}  // extern "C"
