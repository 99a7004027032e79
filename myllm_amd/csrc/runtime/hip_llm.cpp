// HipLLM implementation: weight upload, device state, and the per-token
// graph of HIP kernels (see hip_llm.h).
//
// Per decode token (MetalLLM::decode, metal_llm.mm:3295-3385; layer graph
// cpu_llm.cpp:843-914), all on one stream:
//   embed -> L x [ rmsnorm(+xq) -> QKV GEMV(+bias) -> RoPE + KV write
//                  -> attention(+xq) -> O GEMV(+residual)
//                  -> rmsnorm(+xq) -> gate/up GEMV + SwiGLU(+xq)
//                  -> down GEMV(+residual) ]
//   -> rmsnorm(+xq) -> LM-head GEMV -> argmax -> 4-byte readback.
#include "hip_llm.h"

#include "../kernels/launch.h"
#include "device_common.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>

namespace llm {
namespace {

struct DevLayer {
    const float* attn_norm = nullptr;
    DevMatrix q, k, v;          // q/k/v are contiguous when fused_qkv
    bool fused_qkv = false;
    const float* qkv_bias = nullptr;  // [bq | bk | bv]
    DevMatrix o;
    const float* ffn_norm = nullptr;
    DevMatrix gate, up, down;
    bool fused_gate_up = false;
    // Q4_K / Q6_K decode weights in the x16 tile-packed form (nullptr: not
    // packed): the fused QKV rows, the attention output, the FFN gate, up
    // and down.
    const void* qkv_x16 = nullptr;
    const void* o_x16 = nullptr;
    const void* gate_x16 = nullptr;
    const void* up_x16 = nullptr;
    const void* down_x16 = nullptr;
};

// Device activation buffers (one token row; the serial prefill reuses them).
struct Activations {
    float* hidden[2] = {nullptr, nullptr};
    float* norm = nullptr;
    hipllm::XGroup* normq = nullptr;
    float* qkv = nullptr;
    float* attn = nullptr;
    hipllm::XGroup* attnq = nullptr;
    float* ffn = nullptr;
    hipllm::XGroup* ffnq = nullptr;
    float* gate_tmp = nullptr;
    float* logits = nullptr;
    float* attn_scratch = nullptr;
    void* argmax_scratch = nullptr;
    std::int32_t* ids = nullptr;
    std::uint32_t* token = nullptr;
    std::uint32_t* step = nullptr;  // decode step inputs: [token id, position]
    double* sumsq = nullptr;        // per-16-value sums of squares of the row to normalise next
};

// Device buffers of the batched prefill: T prompt rows each.
struct PrefillActivations {
    float* hidden[2] = {nullptr, nullptr};  // [T, H]
    float* norm = nullptr;                  // [T, H]
    float* qkv = nullptr;                   // [T, H + 2 kv]
    float* attn = nullptr;                  // [T, H]
    float* gate = nullptr;                  // [T, F]
    float* up = nullptr;                    // [T, F]
    void* xb = nullptr;                     // fp16 [T, max(H, F)] matmul operands
    float* xscale = nullptr;                // [T] their row scales
    void* split = nullptr;                  // K-split partial sums of one matmul
    std::size_t split_bytes = 0;
};

}  // namespace

struct HipLLM::Impl {
    int device = 0;
    std::string device_name;
    hipStream_t stream = nullptr;
    GgufModelConfig config;
    std::size_t max_sequence = 0;
    std::size_t sequence_length = 0;
    bool batched_prefill = false;
    // Narrow models (H <= 2048, quantized fused QKV and gate/up): the decode
    // GEMVs that read the raw hidden row normalise it in their prologue
    // instead of a separate RMSNorm launch. Every block of such a GEMV
    // re-reads and normalises the whole row, which costs more than the saved
    // launch once rows are long (measured decode: 0.5B +8%; 7B -3% and 14B
    // -7% with both GEMVs fused, 7B 0% and 14B -5% with the QKV one alone).
    bool fused_norms = false;
    bool fused_ffn_norm = false;
    // The RMSNorms between x16 GEMVs ride in them: the attention output and
    // FFN down GEMVs write the next norm's input data, QKV, gate / up and the
    // LM head apply it.
    bool norm_epilogues = false;
    bool norm_fusion = true;  // switch for both fused forms

    WeightArena weights;
    std::size_t weight_bytes = 0;  // sum of GGUF tensor payloads
    // Decode copies of the Q4_K / Q6_K projections in the x16 tile-packed
    // form read by the int8-MFMA GEMV (the GGUF rows stay for the prefill
    // matmuls).
    void* x16_arena = nullptr;
    std::size_t x16_bytes = 0;
    const void* output_x16 = nullptr;  // the LM head's x16 copy
    bool packed_decode = false;
    DevMatrix embedding, output;
    const float* output_norm = nullptr;
    std::vector<DevLayer> layers;

    float* kv_arena = nullptr;
    std::size_t kv_cache_bytes = 0;
    std::size_t kv_dim = 0;
    float* rope_table = nullptr;

    void* act_arena = nullptr;
    std::size_t act_bytes = 0;
    Activations act;
    std::size_t prompt_capacity = 0;

    void* pre_arena = nullptr;
    std::size_t pre_bytes = 0;
    std::size_t pre_rows = 0;
    PrefillActivations pre;

    std::int32_t* host_ids = nullptr;      // pinned
    std::uint32_t* host_token = nullptr;   // pinned
    std::uint32_t* host_step = nullptr;    // pinned [token id, position]

    // One decode step recorded as a HIP graph (kernels read the token and
    // position from act.step) and replayed per token.
    bool decode_graphs = true;
    hipGraph_t decode_graph = nullptr;
    hipGraphExec_t decode_exec = nullptr;

    std::unique_ptr<RunProfiler> prof;
    GraphKernels decode_graph_kernels;

    ~Impl() {
        if (stream) hipStreamSynchronize(stream);
        drop_decode_graph();
        if (host_step) hipHostFree(host_step);
        prof.reset();
        weights.release();
        if (x16_arena) hipFree(x16_arena);
        if (kv_arena) hipFree(kv_arena);
        if (rope_table) hipFree(rope_table);
        if (act_arena) hipFree(act_arena);
        if (pre_arena) hipFree(pre_arena);
        if (host_ids) hipHostFree(host_ids);
        if (host_token) hipHostFree(host_token);
        if (stream) hipStreamDestroy(stream);
    }

    float* kcache(std::size_t layer) const { return kv_arena + (2 * layer) * max_sequence * kv_dim; }
    float* vcache(std::size_t layer) const { return kv_arena + (2 * layer + 1) * max_sequence * kv_dim; }

    void load(const std::string& path, std::size_t capacity, int dev);
    void upload(GgufReader& reader);
    void pack_decode_weights();
    void choose_decode_forms();
    void allocate_state();
    void build_rope_table();
    void ensure_prompt_capacity(std::size_t n);
    void ensure_prefill_rows(std::size_t n);
    bool batched_shapes() const;

    void gemv(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, const float* bias, const float* residual,
              float* y, std::size_t rows_override = 0) const;
    void layer_step(std::size_t li, std::size_t pos, float* hidden, float* next_hidden, const std::uint32_t* dpos);
    void token_step(const std::int32_t* device_id, std::size_t pos, bool head, const std::uint32_t* dpos = nullptr);
    void capture_decode();
    void drop_decode_graph();
    void norm_f16(const float* x, const float* gamma, std::size_t rows) const;
    void gemm(const DevMatrix& w, const void* xb, const float* bias, const float* residual, float* y,
              std::size_t rows, std::size_t ldy, std::size_t n_override = 0) const;
    void prefill_layer(std::size_t li, std::size_t rows, float* hidden, float* next_hidden);
    void prefill_batched(std::size_t rows);
    void head_step(const float* hidden_row);
    void head_logits(bool norm_in = false);
    std::int32_t read_token();
};

void HipLLM::Impl::load(const std::string& path, std::size_t capacity, int dev) {
    int count = 0;
    hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (count <= 0) throw std::runtime_error("no HIP device is available");
    if (dev < 0) hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev >= count) throw std::invalid_argument("HIP device index is outside the visible devices");
    device = dev;
    hip_check(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    device_name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");

    GgufReader reader(path);
    GgufModelConfig cfg = reader.config();
    if (cfg.architecture != "qwen2") {
        throw std::runtime_error("HipLLM supports qwen2 GGUF models, got " + cfg.architecture);
    }
    if (cfg.layer_count == 0 || cfg.embedding_size == 0 || cfg.feed_forward_size == 0 ||
        cfg.attention_head_count == 0 || cfg.kv_head_count == 0 || cfg.head_size == 0 ||
        cfg.vocabulary_size == 0 || cfg.context_length == 0) {
        throw std::runtime_error("HIP model metadata is incomplete");
    }
    if (capacity == 0) capacity = cfg.context_length;
    if (capacity > cfg.context_length) {
        throw std::invalid_argument("HIP maximum sequence exceeds the model context length");
    }
    if (cfg.embedding_size % 16 != 0 || cfg.feed_forward_size % 16 != 0 || cfg.head_size % 16 != 0 ||
        cfg.head_size > 256) {
        throw std::invalid_argument("HIP kernels need hidden, FFN and head sizes that are multiples of 16 "
                                    "(head size at most 256)");
    }
    config = std::move(cfg);
    max_sequence = capacity;
    upload(reader);
    pack_decode_weights();
    allocate_state();
    build_rope_table();
    batched_prefill = batched_shapes();
    choose_decode_forms();
}

// The decode forms: the x16 MFMA GEMVs read the XGroup form of their input,
// so with packed weights the norms run as their own launches; otherwise
// short rows fold the norm into the GEMVs' prologue.
void HipLLM::Impl::choose_decode_forms() {
    auto quantized = [](std::uint32_t t) {
        return t == hipllm::kQ4_K || t == hipllm::kQ6_K || t == hipllm::kQ8_0 || t == hipllm::kQ5_0;
    };
    const std::size_t H = config.embedding_size;
    fused_norms = norm_fusion && H % 16 == 0 && H <= 2048 && !packed_decode;
    fused_ffn_norm = fused_norms;
    norm_epilogues = norm_fusion && packed_decode && H % 16 == 0 && H <= 8192 && output_x16 != nullptr;
    for (const DevLayer& L : layers) {
        norm_epilogues = norm_epilogues && L.qkv_x16 && L.o_x16 && L.gate_x16 && L.down_x16;
    }
    for (const DevLayer& L : layers) {
        fused_norms = fused_norms && L.fused_qkv && quantized(L.q.type);
        fused_ffn_norm = fused_ffn_norm && L.fused_gate_up && quantized(L.gate.type);
    }
    fused_ffn_norm = fused_ffn_norm && fused_norms;
}

// Q4_K and Q6_K projections whose rows hold whole super-blocks get an x16
// copy: the fused QKV rows, the attention output, the FFN gate / up pair,
// the FFN down projection and the LM head.
void HipLLM::Impl::pack_decode_weights() {
    auto packable = [](const DevMatrix& m) {
        return m.cols % 256 == 0 && ((m.type == hipllm::kQ4_K && m.row_bytes % 16 == 0) ||
                                     (m.type == hipllm::kQ6_K && m.row_bytes % 2 == 0));
    };
    const std::size_t H = config.embedding_size;
    struct Job {
        const DevMatrix* m;
        std::size_t rows;
        const void** dst;
        std::size_t off;
    };
    std::vector<Job> jobs;
    std::size_t total = 0;
    auto add = [&](const DevMatrix& m, std::size_t rows, const void** dst) {
        jobs.push_back({&m, rows, dst, total});
        total = align_up(total + hipllm::x16_bytes(m.type, rows, m.cols), 256);
    };
    for (DevLayer& L : layers) {
        if (L.fused_qkv && packable(L.q)) add(L.q, H + 2 * kv_dim, &L.qkv_x16);
        if (packable(L.o)) add(L.o, L.o.rows, &L.o_x16);
        if (L.fused_gate_up && packable(L.gate)) {
            add(L.gate, L.gate.rows, &L.gate_x16);
            add(L.up, L.up.rows, &L.up_x16);
        }
        if (packable(L.down)) add(L.down, L.down.rows, &L.down_x16);
    }
    if (packable(output)) add(output, output.rows, &output_x16);
    if (jobs.empty()) return;
    hip_check(hipMalloc(&x16_arena, total), "hipMalloc(x16 decode weights)");
    x16_bytes = total;
    auto* base = static_cast<std::uint8_t*>(x16_arena);
    for (const Job& j : jobs) {
        *j.dst = base + j.off;
        launch_check(hipllm::launch_pack_x16(j.m->type, j.m->ptr, j.m->row_bytes, j.rows, j.m->cols, base + j.off,
                                             stream),
                     "x16 packing");
    }
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    packed_decode = true;
}

void HipLLM::Impl::upload(GgufReader& reader) {
    const GgufModelConfig& c = config;
    const std::size_t H = c.embedding_size, F = c.feed_forward_size, V = c.vocabulary_size;
    kv_dim = c.kv_head_count * c.head_size;
    WeightArena& A = weights;

    // Every tensor is taken (shape-checked, consumed once) up front so the
    // arena layout is known. Q/K/V weights (and their biases) are packed back
    // to back when their formats match, so one GEMV / matmul covers them.
    auto require_f32 = [&](std::size_t idx) {
        if (A.tensor(idx).type != GgmlType::F32) {
            throw std::invalid_argument("HIP norm and bias tensors must be F32: " + A.tensor(idx).name);
        }
    };
    auto supported = [&](std::size_t idx) {
        const GgmlType t = A.tensor(idx).type;
        if (t != GgmlType::F32 && t != GgmlType::F16 && t != GgmlType::Q5_0 && t != GgmlType::Q8_0 &&
            t != GgmlType::Q4_K && t != GgmlType::Q6_K) {
            throw std::invalid_argument(std::string("HIP backend does not support ") + ggml_type_name(t) +
                                        " weights: " + A.tensor(idx).name);
        }
    };
    const std::size_t i_embd = A.place(reader, "token_embd.weight", V, H);
    const std::size_t i_onorm = A.place(reader, "output_norm.weight", 1, H);
    const std::size_t i_out = A.place(reader, "output.weight", V, H);
    supported(i_embd);
    supported(i_out);
    require_f32(i_onorm);
    struct LayerIdx {
        std::size_t an, q, k, v, bq, bk, bv, o, fn, g, u, d;
    };
    std::vector<LayerIdx> li(c.layer_count);
    for (std::size_t l = 0; l < c.layer_count; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        LayerIdx& x = li[l];
        x.an = A.place(reader, p + "attn_norm.weight", 1, H);
        x.q = A.place(reader, p + "attn_q.weight", H, H);
        x.k = A.place(reader, p + "attn_k.weight", kv_dim, H, true);
        x.v = A.place(reader, p + "attn_v.weight", kv_dim, H, true);
        x.bq = A.place(reader, p + "attn_q.bias", 1, H);
        x.bk = A.place(reader, p + "attn_k.bias", 1, kv_dim, true);
        x.bv = A.place(reader, p + "attn_v.bias", 1, kv_dim, true);
        x.o = A.place(reader, p + "attn_output.weight", H, H);
        x.fn = A.place(reader, p + "ffn_norm.weight", 1, H);
        x.g = A.place(reader, p + "ffn_gate.weight", F, H);
        x.u = A.place(reader, p + "ffn_up.weight", F, H);
        x.d = A.place(reader, p + "ffn_down.weight", H, F);
        for (std::size_t idx : {x.an, x.bq, x.bk, x.bv, x.fn}) require_f32(idx);
        for (std::size_t idx : {x.q, x.k, x.v, x.o, x.g, x.u, x.d}) supported(idx);
        if (!A.contiguous(x.bq, x.bk) || !A.contiguous(x.bk, x.bv)) {
            throw std::runtime_error("HIP Q/K/V biases must pack contiguously");
        }
    }
    reader.validate_all_consumed();
    if (A.payload_bytes() != c.stored_weight_bytes) {
        throw std::runtime_error("HIP uploaded weight bytes do not match GGUF tensor bytes");
    }
    weight_bytes = A.payload_bytes();
    A.upload(reader, stream);

    embedding = A.matrix(i_embd);
    output = A.matrix(i_out);
    output_norm = A.vec(i_onorm);
    layers.resize(c.layer_count);
    for (std::size_t l = 0; l < c.layer_count; ++l) {
        const LayerIdx& x = li[l];
        DevLayer& L = layers[l];
        L.attn_norm = A.vec(x.an);
        L.q = A.matrix(x.q);
        L.k = A.matrix(x.k);
        L.v = A.matrix(x.v);
        L.fused_qkv = A.contiguous(x.q, x.k) && A.contiguous(x.k, x.v);
        L.qkv_bias = A.vec(x.bq);
        L.o = A.matrix(x.o);
        L.ffn_norm = A.vec(x.fn);
        L.gate = A.matrix(x.g);
        L.up = A.matrix(x.u);
        L.down = A.matrix(x.d);
        L.fused_gate_up = A.tensor(x.g).type == A.tensor(x.u).type;
    }
}

void HipLLM::Impl::allocate_state() {
    const GgufModelConfig& c = config;
    const std::size_t L = c.layer_count;
    kv_cache_bytes = 2 * L * max_sequence * kv_dim * sizeof(float);
    hip_check(hipMalloc(reinterpret_cast<void**>(&kv_arena), kv_cache_bytes), "hipMalloc(KV cache)");
    // Rows at or past the current length are never part of a result, but a
    // fresh allocation can hold any bits (NaN/Inf from an earlier owner), so
    // the cache starts at zero: an in-bounds read of a row past the length
    // that is then weighted by 0 stays 0. Set once here, outside any graph
    // capture; reset() keeps the bytes, as the reference does.
    hip_check(hipMemsetAsync(kv_arena, 0, kv_cache_bytes, stream), "hipMemsetAsync(KV cache)");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_token), 64, hipHostMallocDefault), "hipHostMalloc(token)");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_step), 64, hipHostMallocDefault), "hipHostMalloc(step)");
    ensure_prompt_capacity(1);
}

// Activation arena: one token row plus prompt ids. Reallocated only when a
// longer prompt arrives.
void HipLLM::Impl::ensure_prompt_capacity(std::size_t n) {
    if (n <= prompt_capacity && act_arena) return;
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    drop_decode_graph();  // it points into the arena
    if (act_arena) hipFree(act_arena);
    if (host_ids) hipHostFree(host_ids);
    act_arena = nullptr;
    host_ids = nullptr;
    const GgufModelConfig& c = config;
    const std::size_t H = c.embedding_size, F = c.feed_forward_size, V = c.vocabulary_size;
    const std::size_t qkv = H + 2 * kv_dim;
    std::size_t off = 0;
    auto reserve = [&](std::size_t bytes) {
        const std::size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    const std::size_t xg = sizeof(hipllm::XGroup);
    const std::size_t o_h0 = reserve(H * 4), o_h1 = reserve(H * 4), o_norm = reserve(H * 4),
                      o_normq = reserve(H / 16 * xg), o_qkv = reserve(qkv * 4), o_attn = reserve(H * 4),
                      o_attnq = reserve(H / 16 * xg), o_ffn = reserve(F * 4), o_ffnq = reserve(F / 16 * xg),
                      o_gtmp = reserve(F * 4), o_logits = reserve(V * 4),
                      o_as = reserve(hipllm::attn_decode_scratch_floats(c.attention_head_count, c.head_size,
                                                                          max_sequence) * 4),
                      o_am = reserve(hipllm::argmax_scratch_bytes(V)), o_ids = reserve(n * 4), o_tok = reserve(64),
                      o_step = reserve(16), o_ssq = reserve((H + 15) / 16 * sizeof(double));
    act_bytes = off;
    hip_check(hipMalloc(&act_arena, act_bytes), "hipMalloc(activations)");
    auto* base = static_cast<std::uint8_t*>(act_arena);
    act.hidden[0] = reinterpret_cast<float*>(base + o_h0);
    act.hidden[1] = reinterpret_cast<float*>(base + o_h1);
    act.norm = reinterpret_cast<float*>(base + o_norm);
    act.normq = reinterpret_cast<hipllm::XGroup*>(base + o_normq);
    act.qkv = reinterpret_cast<float*>(base + o_qkv);
    act.attn = reinterpret_cast<float*>(base + o_attn);
    act.attnq = reinterpret_cast<hipllm::XGroup*>(base + o_attnq);
    act.ffn = reinterpret_cast<float*>(base + o_ffn);
    act.ffnq = reinterpret_cast<hipllm::XGroup*>(base + o_ffnq);
    act.gate_tmp = reinterpret_cast<float*>(base + o_gtmp);
    act.logits = reinterpret_cast<float*>(base + o_logits);
    act.attn_scratch = reinterpret_cast<float*>(base + o_as);
    act.argmax_scratch = base + o_am;
    act.ids = reinterpret_cast<std::int32_t*>(base + o_ids);
    act.token = reinterpret_cast<std::uint32_t*>(base + o_tok);
    act.step = reinterpret_cast<std::uint32_t*>(base + o_step);
    act.sumsq = reinterpret_cast<double*>(base + o_ssq);
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_ids), n * 4, hipHostMallocDefault), "hipHostMalloc(ids)");
    prompt_capacity = n;
}

// cos/sin for every (position, pair) computed exactly as CPULLM's RoPE
// (cpu_llm.cpp:218-224): freq = powf(theta, -2 i / R), angle = pos * freq.
void HipLLM::Impl::build_rope_table() {
    const std::size_t R = config.rotary_dimension;
    const std::size_t half = R / 2;
    std::vector<float> table(max_sequence * half * 2);
    std::vector<float> freq(half);
    for (std::size_t p = 0; p < half; ++p) {
        freq[p] = std::pow(config.rope_theta, -2.0f * static_cast<float>(p) / static_cast<float>(R));
    }
    for (std::size_t pos = 0; pos < max_sequence; ++pos) {
        for (std::size_t p = 0; p < half; ++p) {
            const float angle = static_cast<float>(pos) * freq[p];
            table[2 * (pos * half + p)] = std::cos(angle);
            table[2 * (pos * half + p) + 1] = std::sin(angle);
        }
    }
    hip_check(hipMalloc(reinterpret_cast<void**>(&rope_table), table.size() * sizeof(float)), "hipMalloc(RoPE)");
    hip_check(hipMemcpy(rope_table, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice),
              "hipMemcpy(RoPE)");
}

void HipLLM::Impl::gemv(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, const float* bias,
                        const float* residual, float* y, std::size_t rows_override) const {
    const std::size_t n = rows_override ? rows_override : w.rows;
    launch_check(hipllm::launch_gemv_prepped(w.type, w.ptr, w.row_bytes, x, xq, bias, residual, y, n, w.cols, 0,
                                             stream),
                 "GEMV");
}

// dpos (device, nullable): the position read on the device (recorded decode
// step); pos is used otherwise.
void HipLLM::Impl::layer_step(std::size_t li, std::size_t pos, float* hidden, float* next_hidden,
                              const std::uint32_t* dpos) {
    const GgufModelConfig& c = config;
    const DevLayer& L = layers[li];
    const std::size_t H = c.embedding_size, F = c.feed_forward_size;
    const float eps = c.norm_epsilon;
    // Norm data that the x16 GEMVs pass along (norm_epilogues): the sums of
    // squares of the row, its XGroup form times the gain in act.normq.
    hipllm::X16Norm norm_in{};
    norm_in.sumsq_in = act.sumsq;
    norm_in.eps = eps;
    auto norm_out = [&](const float* gamma) {
        hipllm::X16Norm o{};
        o.gamma_out = gamma;
        o.yq_out = act.normq;
        o.sumsq_out = act.sumsq;
        return o;
    };
    if (packed_decode && L.qkv_x16) {
        // act.normq holds the XGroup form of rmsnorm(hidden) * attn_norm, or
        // (norm_epilogues past layer 0) of hidden * attn_norm with the sums
        // of squares of hidden.
        const bool in = norm_epilogues && li > 0;
        launch_check(hipllm::launch_gemv_x16(L.q.type, L.qkv_x16, act.normq, L.qkv_bias, nullptr, act.qkv,
                                             H + 2 * kv_dim, H, 0, stream, in ? &norm_in : nullptr),
                     "QKV GEMV");
    } else if (fused_norms) {
        // QKV of rmsnorm(hidden) * attn_norm, the norm in the GEMV's prologue.
        launch_check(hipllm::launch_gemv_norm(L.q.type, L.q.ptr, L.q.row_bytes, hidden, L.attn_norm, eps, L.qkv_bias,
                                              nullptr, act.qkv, H + 2 * kv_dim, H, 0, stream),
                     "QKV GEMV");
    } else if (L.fused_qkv) {
        // act.norm / act.normq hold rmsnorm(hidden) * attn_norm on entry.
        gemv(L.q, act.norm, act.normq, L.qkv_bias, nullptr, act.qkv, H + 2 * kv_dim);
    } else {
        gemv(L.q, act.norm, act.normq, L.qkv_bias, nullptr, act.qkv);
        gemv(L.k, act.norm, act.normq, L.qkv_bias + H, nullptr, act.qkv + H);
        gemv(L.v, act.norm, act.normq, L.qkv_bias + H + kv_dim, nullptr, act.qkv + H + kv_dim);
    }
    // RoPE of Q and K, the KV-cache write and the attention: one launch for
    // short capacities, else a launch pair (partials, merge).
    const float scale = 1.0f / std::sqrt(static_cast<float>(c.head_size));
    launch_check(hipllm::launch_attn_decode_rope(act.qkv, rope_table, c.rotary_dimension, kcache(li), vcache(li),
                                                 act.attn, act.attnq, act.attn_scratch, c.attention_head_count,
                                                 c.kv_head_count, c.head_size, pos, scale, stream, dpos, max_sequence),
                 "RoPE/KV write + attention");
    if (packed_decode && L.o_x16) {
        const hipllm::X16Norm out = norm_out(L.ffn_norm);
        launch_check(hipllm::launch_gemv_x16(L.o.type, L.o_x16, act.attnq, nullptr, hidden, next_hidden, H, H, 0,
                                             stream, norm_epilogues ? &out : nullptr),
                     "attention output GEMV");
    } else {
        gemv(L.o, act.attn, act.attnq, nullptr, hidden, next_hidden);
    }
    if (norm_epilogues) {
        launch_check(hipllm::launch_gemv_x16_swiglu(L.gate.type, L.gate_x16, L.up_x16, act.normq, act.ffn, act.ffnq, F,
                                                    H, 0, stream, &norm_in),
                     "gate/up GEMV");
    } else if (fused_ffn_norm) {
        launch_check(hipllm::launch_gemv_swiglu_norm(L.gate.type, L.gate.ptr, L.up.ptr, L.gate.row_bytes, next_hidden,
                                                     L.ffn_norm, eps, act.ffn, act.ffnq, F, H, 0, stream),
                     "gate/up GEMV");
    } else {
        launch_check(hipllm::launch_rmsnorm(next_hidden, L.ffn_norm, act.norm, act.normq, 1, H, eps, stream),
                     "RMSNorm");
        if (packed_decode && L.gate_x16) {
            launch_check(hipllm::launch_gemv_x16_swiglu(L.gate.type, L.gate_x16, L.up_x16, act.normq, act.ffn,
                                                        act.ffnq, F, H, 0, stream),
                         "gate/up GEMV");
        } else if (L.fused_gate_up) {
            launch_check(hipllm::launch_gemv_swiglu(L.gate.type, L.gate.ptr, L.up.ptr, L.gate.row_bytes, act.norm,
                                                    act.normq, act.ffn, act.ffnq, F, H, 0, stream),
                         "gate/up GEMV");
        } else {
            // Gate and up in different formats: two GEMVs, then SwiGLU.
            gemv(L.gate, act.norm, act.normq, nullptr, nullptr, act.gate_tmp);
            gemv(L.up, act.norm, act.normq, nullptr, nullptr, act.ffn);
            launch_check(hipllm::launch_swiglu(act.gate_tmp, act.ffn, act.ffn, act.ffnq, F, stream), "SwiGLU");
        }
    }
    // The layer output lands back in `hidden`, followed by its RMSNorm with
    // the next layer's attention gain (or the output norm after the last),
    // unless the next layer's QKV GEMV normalises it itself (its prologue, or
    // the norm data of this GEMV's epilogue).
    const float* next_gamma = li + 1 < layers.size() ? layers[li + 1].attn_norm : output_norm;
    if (packed_decode && L.down_x16) {
        const hipllm::X16Norm out = norm_out(next_gamma);
        launch_check(hipllm::launch_gemv_x16(L.down.type, L.down_x16, act.ffnq, nullptr, next_hidden, hidden, H, F, 0,
                                             stream, norm_epilogues ? &out : nullptr),
                     "down GEMV");
    } else {
        gemv(L.down, act.ffn, act.ffnq, nullptr, next_hidden, hidden);
    }
    if (!norm_epilogues && (!fused_norms || li + 1 == layers.size())) {
        launch_check(hipllm::launch_rmsnorm(hidden, next_gamma, act.norm, act.normq, 1, H, eps, stream), "RMSNorm");
    }
}

void HipLLM::Impl::token_step(const std::int32_t* device_id, std::size_t pos, bool head,
                              const std::uint32_t* dpos) {
    const GgufModelConfig& c = config;
    const std::size_t H = c.embedding_size;
    float* h = act.hidden[0];
    float* tmp = act.hidden[1];
    launch_check(hipllm::launch_embed(embedding.type, embedding.ptr, embedding.row_bytes, device_id, 1,
                                      c.vocabulary_size, H, h, stream),
                 "embedding");
    if (!fused_norms) {
        launch_check(hipllm::launch_rmsnorm(h, layers[0].attn_norm, act.norm, act.normq, 1, H, c.norm_epsilon,
                                            stream),
                     "RMSNorm");
    }
    for (std::size_t l = 0; l < layers.size(); ++l) layer_step(l, pos, h, tmp, dpos);
    // The last layer already produced the output norm's input (normalised,
    // or with the norm data for the LM head GEMV).
    if (head) head_logits(norm_epilogues);
}

// Records one decode step (embedding of act.step[0] at position act.step[1],
// every layer, LM head, argmax) as a graph. No allocation, copy or memset is
// recorded: the host writes act.step with an ordinary copy before each replay.
void HipLLM::Impl::capture_decode() {
    hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
        token_step(reinterpret_cast<const std::int32_t*>(act.step), 0, true, act.step + 1);
    } catch (...) {
        hipGraph_t g = nullptr;
        hipStreamEndCapture(stream, &g);
        if (g) hipGraphDestroy(g);
        throw;
    }
    hip_check(hipStreamEndCapture(stream, &decode_graph), "hipStreamEndCapture");
    hip_check(hipGraphInstantiate(&decode_exec, decode_graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    decode_graph_kernels = graph_kernels(decode_graph);
}

void HipLLM::Impl::drop_decode_graph() {
    if (decode_exec) hipGraphExecDestroy(decode_exec);
    if (decode_graph) hipGraphDestroy(decode_graph);
    decode_exec = nullptr;
    decode_graph = nullptr;
}

// Batched prefill buffers, grown to the longest prompt seen.
void HipLLM::Impl::ensure_prefill_rows(std::size_t n) {
    if (n <= pre_rows && pre_arena) return;
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (pre_arena) hipFree(pre_arena);
    pre_arena = nullptr;
    pre_rows = 0;
    const GgufModelConfig& c = config;
    const std::size_t H = c.embedding_size, F = c.feed_forward_size;
    std::size_t off = 0;
    auto reserve = [&](std::size_t bytes) {
        const std::size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    const std::size_t o_h0 = reserve(n * H * 4), o_h1 = reserve(n * H * 4), o_norm = reserve(n * H * 4),
                      o_qkv = reserve(n * (H + 2 * kv_dim) * 4), o_attn = reserve(n * H * 4),
                      o_gate = reserve(n * F * 4), o_up = reserve(n * F * 4),
                      o_xb = reserve(n * std::max(H, F) * 2), o_xs = reserve(n * 4);
    // The largest K-split workspace any layer matmul takes at up to n rows.
    std::size_t split_bytes = 0;
    for (std::size_t m = 1; m <= n; ++m) {
        split_bytes = std::max({split_bytes, hipllm::gemm_split_bytes(m, H + 2 * kv_dim, H, -1, 0),
                                hipllm::gemm_split_bytes(m, H, H, -1, 0), hipllm::gemm_split_bytes(m, F, H, -1, 0),
                                hipllm::gemm_split_bytes(m, H, F, -1, 0), hipllm::gemm_swiglu_bytes(m, F, H)});
    }
    const std::size_t o_split = reserve(split_bytes);
    pre_bytes = off;
    hip_check(hipMalloc(&pre_arena, pre_bytes), "hipMalloc(prefill activations)");
    auto* base = static_cast<std::uint8_t*>(pre_arena);
    pre.hidden[0] = reinterpret_cast<float*>(base + o_h0);
    pre.hidden[1] = reinterpret_cast<float*>(base + o_h1);
    pre.norm = reinterpret_cast<float*>(base + o_norm);
    pre.qkv = reinterpret_cast<float*>(base + o_qkv);
    pre.attn = reinterpret_cast<float*>(base + o_attn);
    pre.gate = reinterpret_cast<float*>(base + o_gate);
    pre.up = reinterpret_cast<float*>(base + o_up);
    pre.xb = base + o_xb;
    pre.xscale = reinterpret_cast<float*>(base + o_xs);
    pre.split = split_bytes ? base + o_split : nullptr;
    pre.split_bytes = split_bytes;
    pre_rows = n;
}

// The MFMA prefill matmul steps K by 128.
bool HipLLM::Impl::batched_shapes() const {
    return config.embedding_size % 128 == 0 && config.feed_forward_size % 128 == 0;
}

// RMSNorm of `rows` hidden rows into pre.norm and its fp16 operand form
// (pre.xb, pre.xscale): one launch where the row fits it.
void HipLLM::Impl::norm_f16(const float* x, const float* gamma, std::size_t rows) const {
    const std::size_t H = config.embedding_size;
    const float eps = config.norm_epsilon;
    if (H % 16 == 0 && H <= 8192) {
        launch_check(hipllm::launch_rmsnorm_f16(x, gamma, pre.norm, pre.xb, pre.xscale, rows, H, eps, stream),
                     "RMSNorm + fp16 activations");
        return;
    }
    launch_check(hipllm::launch_rmsnorm(x, gamma, pre.norm, nullptr, rows, H, eps, stream), "RMSNorm");
    launch_check(hipllm::launch_to_f16(pre.norm, H, pre.xb, pre.xscale, rows, H, stream), "fp16 activations");
}

void HipLLM::Impl::gemm(const DevMatrix& w, const void* xb, const float* bias, const float* residual, float* y,
                        std::size_t rows, std::size_t ldy, std::size_t n_override) const {
    const std::size_t n = n_override ? n_override : w.rows;
    launch_check(hipllm::launch_gemm_mfma(w.type, w.ptr, w.row_bytes, xb, pre.xscale, bias, residual, y, rows, n,
                                          w.cols, -1, 0, stream, ldy, pre.split, pre.split_bytes),
                 "prefill matmul");
}

// One decoder layer over `rows` prompt rows (cpu_prefill_layer,
// cpu_llm.cpp:774-841): every projection is one fp16 MFMA matmul over the
// native weights; attention is causal over the rows just written to the cache.
void HipLLM::Impl::prefill_layer(std::size_t li, std::size_t rows, float* hidden, float* next_hidden) {
    const GgufModelConfig& c = config;
    const DevLayer& L = layers[li];
    const std::size_t H = c.embedding_size, F = c.feed_forward_size;
    const std::size_t qkv_w = H + 2 * kv_dim;
    const float eps = c.norm_epsilon;
    norm_f16(hidden, L.attn_norm, rows);
    if (L.fused_qkv) {
        gemm(L.q, pre.xb, L.qkv_bias, nullptr, pre.qkv, rows, qkv_w, qkv_w);
    } else {
        gemm(L.q, pre.xb, L.qkv_bias, nullptr, pre.qkv, rows, qkv_w);
        gemm(L.k, pre.xb, L.qkv_bias + H, nullptr, pre.qkv + H, rows, qkv_w);
        gemm(L.v, pre.xb, L.qkv_bias + H + kv_dim, nullptr, pre.qkv + H + kv_dim, rows, qkv_w);
    }
    launch_check(hipllm::launch_rope_kv(pre.qkv, rope_table, c.rotary_dimension, c.attention_head_count,
                                        c.kv_head_count, c.head_size, 0, rows, qkv_w, kcache(li), vcache(li), stream),
                 "RoPE/KV write");
    const float scale = 1.0f / std::sqrt(static_cast<float>(c.head_size));
    launch_check(hipllm::launch_attn_prefill(pre.qkv, qkv_w, kcache(li), vcache(li), pre.attn, H, rows,
                                             c.attention_head_count, c.kv_head_count, c.head_size, 0, scale, stream),
                 "prefill attention");
    launch_check(hipllm::launch_to_f16(pre.attn, H, pre.xb, pre.xscale, rows, H, stream), "fp16 activations");
    gemm(L.o, pre.xb, nullptr, hidden, next_hidden, rows, H);
    norm_f16(next_hidden, L.ffn_norm, rows);
    if (L.gate.type == L.up.type && L.gate.row_bytes == L.up.row_bytes &&
        (L.gate.type == hipllm::kQ4_K || L.gate.type == hipllm::kQ6_K || L.gate.type == hipllm::kQ8_0 ||
         L.gate.type == hipllm::kQ5_0)) {
        // Gate and up keep their partial planes; one launch reduces both,
        // applies the SwiGLU and (F % 8 == 0, F <= 32768) writes the down
        // projection's fp16 rows directly, after the matmuls have read xb.
        const bool f16 = F % 8 == 0 && F <= 32768;
        launch_check(hipllm::launch_gemm_mfma_swiglu(L.gate.type, L.gate.ptr, L.up.ptr, L.gate.row_bytes, pre.xb,
                                                     pre.xscale, pre.gate, rows, F, L.gate.cols, F, pre.split,
                                                     pre.split_bytes, stream, f16 ? pre.xb : nullptr,
                                                     f16 ? pre.xscale : nullptr),
                     "prefill gate / up + SwiGLU");
        if (!f16) {
            launch_check(hipllm::launch_to_f16(pre.gate, F, pre.xb, pre.xscale, rows, F, stream), "fp16 activations");
        }
    } else {
        gemm(L.gate, pre.xb, nullptr, nullptr, pre.gate, rows, F);
        gemm(L.up, pre.xb, nullptr, nullptr, pre.up, rows, F);
        launch_check(hipllm::launch_swiglu(pre.gate, pre.up, pre.gate, nullptr, rows * F, stream), "SwiGLU");
        launch_check(hipllm::launch_to_f16(pre.gate, F, pre.xb, pre.xscale, rows, F, stream), "fp16 activations");
    }
    gemm(L.down, pre.xb, nullptr, next_hidden, hidden, rows, H);
}

// Final norm, LM head and argmax on one hidden row (decode kernels).
void HipLLM::Impl::head_step(const float* hidden_row) {
    const GgufModelConfig& c = config;
    launch_check(hipllm::launch_rmsnorm(hidden_row, output_norm, act.norm, act.normq, 1, c.embedding_size,
                                        c.norm_epsilon, stream),
                 "final RMSNorm");
    head_logits();
}

// LM head and argmax on the normalised row in act.norm / act.normq, or
// (norm_in) on act.normq = XGroup(hidden * output_norm) with the sums of
// squares of hidden in act.sumsq.
void HipLLM::Impl::head_logits(bool norm_in) {
    const GgufModelConfig& c = config;
    if (packed_decode && output_x16) {
        hipllm::X16Norm in{};
        in.sumsq_in = act.sumsq;
        in.eps = c.norm_epsilon;
        launch_check(hipllm::launch_gemv_x16(output.type, output_x16, act.normq, nullptr, nullptr, act.logits,
                                             c.vocabulary_size, c.embedding_size, 0, stream, norm_in ? &in : nullptr),
                     "LM head GEMV");
    } else {
        gemv(output, act.norm, act.normq, nullptr, nullptr, act.logits);
    }
    launch_check(hipllm::launch_argmax(act.logits, c.vocabulary_size, act.token, act.argmax_scratch, stream),
                 "argmax");
}

// Whole-prompt prefill: embedding of all rows, L batched layers, then the LM
// head on the last row only (metal_llm.mm:3266-3277; cpu_llm.cpp:1019-1020).
void HipLLM::Impl::prefill_batched(std::size_t rows) {
    ensure_prefill_rows(rows);
    const GgufModelConfig& c = config;
    const std::size_t H = c.embedding_size;
    float* h = pre.hidden[0];
    float* tmp = pre.hidden[1];
    launch_check(hipllm::launch_embed(embedding.type, embedding.ptr, embedding.row_bytes, act.ids, rows,
                                      c.vocabulary_size, H, h, stream),
                 "embedding");
    for (std::size_t l = 0; l < layers.size(); ++l) prefill_layer(l, rows, h, tmp);
    head_step(h + (rows - 1) * H);
}

std::int32_t HipLLM::Impl::read_token() {
    hip_check(hipMemcpyAsync(host_token, act.token, 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(token)");
    hip_check(hipStreamSynchronize(stream), "HIP forward");
    const std::uint32_t t = host_token[0];
    if (t > static_cast<std::uint32_t>(std::numeric_limits<std::int32_t>::max())) {
        throw std::overflow_error("HIP token id does not fit in int32_t");
    }
    return static_cast<std::int32_t>(t);
}

// Logical traffic of one forward, from shapes, for the operator table: the
// operator list of the reference backend's estimate (metal_llm.mm:307-433),
// in FP32 tensor bytes whatever the weights' storage.
namespace {
OpTraffic layer_traffic(const GgufModelConfig& c, std::size_t rows, std::size_t keys, bool prompt) {
    const std::size_t H = c.embedding_size, F = c.feed_forward_size, D = c.head_size;
    const std::size_t q = c.attention_head_count * D, kv = c.kv_head_count * D;
    auto proj = [&](std::size_t out, std::size_t in, bool bias) {
        return prompt ? traffic_matmul(rows, out, in, bias) : traffic_gemv(in, out);
    };
    OpTraffic t;
    t += traffic_elementwise(rows * H, 5, 3, 1);  // RMSNorm
    t += proj(q, H, true);
    t += proj(kv, H, true);
    t += proj(kv, H, true);
    t += traffic_elementwise(rows * (q + kv), 6, 1, 1);  // RoPE
    t += traffic_copy(static_cast<std::uint64_t>(rows) * kv * 4 * 2, 1);  // KV write
    for (std::size_t h = 0; h < c.attention_head_count; ++h) {
        if (prompt) {
            OpTraffic qk = traffic_matmul(rows, rows, D);
            qk.flops += static_cast<std::uint64_t>(rows) * rows;  // scale
            t += qk;
            t += traffic_elementwise(rows * rows, 4, 3, 2);  // mask + softmax
            t += traffic_matmul(rows, D, rows);
        } else {
            t += traffic_gemv(D, keys);
            t += traffic_elementwise(keys, 4, 3, 2);
            t += traffic_gemv(keys, D);
        }
    }
    t += prompt ? traffic_matmul(rows, H, q) : traffic_gemv(q, H);
    t += traffic_copy(static_cast<std::uint64_t>(rows) * H * 4, 1);  // residual
    t += traffic_elementwise(rows * H, 5, 3, 1);
    t += proj(F, H, false);
    t += proj(F, H, false);
    t += traffic_elementwise(rows * F, 8, 2, 1);  // SwiGLU
    t += prompt ? traffic_matmul(rows, H, F) : traffic_gemv(F, H);
    t += traffic_copy(static_cast<std::uint64_t>(rows) * H * 4, 1);
    return t;
}

OpTraffic head_traffic(const GgufModelConfig& c, std::size_t rows) {
    OpTraffic t = traffic_elementwise(rows * c.embedding_size, 5, 2, 1);  // final norm
    t += traffic_gemv(c.embedding_size, c.vocabulary_size);              // LM head, last row
    t += traffic_elementwise(c.vocabulary_size, 1, 1, 0);                // argmax
    return t;
}

OpTraffic prefill_traffic(const GgufModelConfig& c, std::size_t rows) {
    OpTraffic t = traffic_copy(static_cast<std::uint64_t>(rows) * c.embedding_size * 4, 1);  // embedding
    for (std::size_t l = 0; l < c.layer_count; ++l) t += layer_traffic(c, rows, rows, true);
    t += head_traffic(c, rows);
    return t;
}

OpTraffic decode_traffic(const GgufModelConfig& c, std::size_t keys) {
    OpTraffic t = traffic_copy(static_cast<std::uint64_t>(c.embedding_size) * 4, 1);
    for (std::size_t l = 0; l < c.layer_count; ++l) t += layer_traffic(c, 1, keys, false);
    t += head_traffic(c, 1);
    return t;
}
}  // namespace

int parse_device_spec(const std::string& spec) {
    if (spec.empty()) return -1;
    const std::string digits = spec.rfind("hip:", 0) == 0 ? spec.substr(4) : spec;
    if (digits.empty() || digits.size() > 6 ||
        digits.find_first_not_of("0123456789") != std::string::npos) {
        throw std::invalid_argument("HIP device must be \"\", \"N\" or \"hip:N\", got \"" + spec + "\"");
    }
    return std::stoi(digits);
}

HipLLM::HipLLM(const std::string& gguf_path, std::size_t max_sequence, const std::string& device)
    : impl_(std::make_unique<Impl>()) {
    impl_->load(gguf_path, max_sequence, parse_device_spec(device));
}

HipLLM::~HipLLM() = default;
HipLLM::HipLLM(HipLLM&&) noexcept = default;
HipLLM& HipLLM::operator=(HipLLM&&) noexcept = default;

void HipLLM::reset() {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    // KV bytes need no clearing: attention reads only [0, position].
    impl_->sequence_length = 0;
}

std::int32_t HipLLM::prefill(const std::vector<std::int32_t>& ids) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    Impl& m = *impl_;
    if (ids.empty()) throw std::invalid_argument("HIP prefill requires at least one token id");
    if (m.sequence_length != 0) throw std::invalid_argument("HIP prefill requires an empty conversation; call reset first");
    if (ids.size() > m.max_sequence) throw std::length_error("HIP prefill exceeds the allocated sequence capacity");
    for (std::int32_t id : ids) {
        if (id < 0 || static_cast<std::size_t>(id) >= m.config.vocabulary_size) {
            throw std::out_of_range("HIP prefill token id is outside the vocabulary");
        }
    }
    hip_check(hipSetDevice(m.device), "hipSetDevice");
    if (m.prof) m.prof->begin("prefill", ids.size(), "prefill.gpu_resident");
    m.ensure_prompt_capacity(ids.size());
    std::memcpy(m.host_ids, ids.data(), ids.size() * 4);
    hip_check(hipMemcpyAsync(m.act.ids, m.host_ids, ids.size() * 4, hipMemcpyHostToDevice, m.stream), "hipMemcpy(ids)");
    if (m.batched_prefill) {
        m.prefill_batched(ids.size());
    } else {
        for (std::size_t t = 0; t < ids.size(); ++t) m.token_step(m.act.ids + t, t, t + 1 == ids.size());
    }
    if (m.prof) m.prof->mark_gpu_end();
    const std::int32_t token = m.read_token();
    m.sequence_length = ids.size();
    if (m.prof) m.prof->end(prefill_traffic(m.config, ids.size()));
    return token;
}

std::int32_t HipLLM::decode(std::int32_t id) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    Impl& m = *impl_;
    if (m.sequence_length == 0) throw std::invalid_argument("HIP decode requires a completed prefill");
    if (id < 0 || static_cast<std::size_t>(id) >= m.config.vocabulary_size) {
        throw std::out_of_range("HIP decode token id is outside the vocabulary");
    }
    const std::size_t pos = m.sequence_length;
    if (pos >= m.max_sequence) throw std::length_error("HIP decode exceeds the allocated sequence capacity");
    hip_check(hipSetDevice(m.device), "hipSetDevice");
    if (m.prof) m.prof->begin("decode", pos + 1, "decode.gpu_resident");
    m.host_step[0] = static_cast<std::uint32_t>(id);
    m.host_step[1] = static_cast<std::uint32_t>(pos);
    hip_check(hipMemcpyAsync(m.act.step, m.host_step, 8, hipMemcpyHostToDevice, m.stream), "hipMemcpy(step)");
    // Detailed profiling times every launch, so the step runs eagerly.
    const bool graph = m.decode_graphs && !(m.prof && m.prof->detailed());
    if (graph) {
        if (!m.decode_exec) m.capture_decode();
        hip_check(hipGraphLaunch(m.decode_exec, m.stream), "hipGraphLaunch(decode)");
    } else {
        m.token_step(reinterpret_cast<const std::int32_t*>(m.act.step), pos, true);
    }
    if (m.prof) m.prof->mark_gpu_end();
    const std::int32_t token = m.read_token();
    m.sequence_length = pos + 1;
    if (m.prof) m.prof->end(decode_traffic(m.config, pos + 1), graph ? &m.decode_graph_kernels : nullptr);
    return token;
}

void HipLLM::enable_profiling(const std::string& csv_path, bool detailed_kernel_timestamps) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    disable_profiling();
    hip_check(hipSetDevice(impl_->device), "hipSetDevice");
    impl_->prof = std::make_unique<RunProfiler>(csv_path, detailed_kernel_timestamps, impl_->stream);
}

void HipLLM::disable_profiling() {
    if (impl_) impl_->prof.reset();
}

const GgufModelConfig& HipLLM::config() const {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    return impl_->config;
}

std::size_t HipLLM::position() const noexcept { return impl_ ? impl_->sequence_length : 0; }
std::size_t HipLLM::max_sequence() const noexcept { return impl_ ? impl_->max_sequence : 0; }
bool HipLLM::uses_gpu() const noexcept { return available(); }
bool HipLLM::available() const noexcept { return impl_ && impl_->weights.base() && impl_->stream; }

const std::string& HipLLM::device_name() const noexcept {
    static const std::string empty;
    return impl_ ? impl_->device_name : empty;
}

MemoryStats HipLLM::memory_stats() const noexcept {
    if (!impl_) return {};
    MemoryStats s;
    s.weight_bytes = impl_->weight_bytes + impl_->x16_bytes;
    s.kv_cache_bytes = impl_->kv_cache_bytes;
    s.recurrent_state_bytes = 0;
    s.intermediate_bytes = impl_->act_bytes;
    s.intermediate_is_estimate = false;
    return s;
}

void HipLLM::copy_last_logits(float* dst, std::size_t count) const {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    if (count != impl_->config.vocabulary_size) throw std::invalid_argument("logits buffer must hold the vocabulary");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    hip_check(hipMemcpy(dst, impl_->act.logits, count * 4, hipMemcpyDeviceToHost), "hipMemcpy(logits)");
}

void HipLLM::set_decode_graphs(bool enabled) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    impl_->decode_graphs = enabled;
    if (!enabled) impl_->drop_decode_graph();
}

void HipLLM::set_packed_decode(bool enabled) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    if (enabled && !impl_->x16_arena) throw std::invalid_argument("the model has no Q4_K or Q6_K projections to pack");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    impl_->packed_decode = enabled;
    impl_->choose_decode_forms();
    impl_->drop_decode_graph();  // recorded with the other forms
}

bool HipLLM::packed_decode() const noexcept { return impl_ && impl_->packed_decode; }

void HipLLM::set_fused_norms(bool enabled) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    impl_->norm_fusion = enabled;
    impl_->choose_decode_forms();
    impl_->drop_decode_graph();  // recorded with the other forms
}

bool HipLLM::fused_norms() const noexcept { return impl_ && (impl_->fused_norms || impl_->norm_epilogues); }

void HipLLM::set_batched_prefill(bool enabled) {
    if (!impl_) throw std::runtime_error("HIP model is not initialized");
    if (enabled && !impl_->batched_shapes()) {
        throw std::invalid_argument("batched prefill needs hidden and FFN sizes that are multiples of 128");
    }
    impl_->batched_prefill = enabled;
}

}  // namespace llm
