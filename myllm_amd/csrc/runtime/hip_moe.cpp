// HipMoeLLM implementation (see hip_moe.h).
//
// One forward over T rows (the whole prompt, or one decode token), on one
// stream (MoeLLM::forward, moe_llm.mm:2887-3039, restated without its 41 host
// round trips):
//   embed -> L x [ RMSNorm -> (gated attention | Gated DeltaNet) (+residual)
//                  -> RMSNorm -> router + top-k -> routed experts (gate/up +
//                  SwiGLU, down) + shared expert -> combine (+residual) ]
//   -> RMSNorm(last row) -> LM-head GEMV -> argmax -> 4-byte readback.
// Projections are FP32-accumulating GEMVs over the native weights: a batched
// launch covers all T rows (blockIdx.y = row), and the routed experts are the
// same kernel indexed by the device-resident top-k ids.
#include "hip_moe.h"

#include "../kernels/launch.h"
#include "device_common.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <stdexcept>


namespace llm {
namespace {

// From this many rows on, the dense projections of a forward run as fp16
// MFMA matmuls (the weights are read once per 64-row tile instead of once per
// row).
constexpr std::size_t kMatmulRows = 16;

// Up to this many rows the DeltaNet runs as two fused launches (conv + L2
// norm, scan + gates + gated norm); beyond it, as five launches that spread
// the per-row work over more blocks.
constexpr std::size_t kFusedDeltaNetRows = 4;

// A decode step (one row) runs the projections that read the same normalised
// row as one grouped GEMV launch with the norm in its prologue: DeltaNet
// QKV + z + alpha/beta, attention Q/gate + K/V, router + shared gate/up.
constexpr std::size_t kGroupedRows = 1;

// From this many rows the router logits run as a tiled FP32 matmul (each
// weight row read once per 32 rows) instead of a GEMV per row.
constexpr std::size_t kRouterMatmulRows = 8;

struct MoeLayer {
    bool full = false;
    const float* attn_norm = nullptr;
    const float* post_norm = nullptr;
    // gated full attention
    DevMatrix qgate, k, v, o;
    bool fused_kv = false;
    DevMatrix kv;  // K and V rows as one matrix when fused_kv (for its x16 copy)
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    float* kcache = nullptr;
    float* vcache = nullptr;
    // Gated DeltaNet
    DevMatrix qkv, z, alpha, beta, ssm_out;
    bool fused_ab = false;
    const float* conv = nullptr;
    const float* dt_bias = nullptr;
    const float* a = nullptr;
    const float* ssm_norm = nullptr;
    float* state = nullptr;
    float* history = nullptr;
    // experts
    DevMatrix router, shexp_router;  // F32 [E, H] and [1, H], packed -> one GEMV of E + 1 rows
    bool fused_router = false;
    DevMatrix gate_exps, up_exps, down_exps;  // per expert rows; expert_stride between experts
    DevMatrix sh_gate, sh_up, sh_down;
};

// Activation rows for up to `rows` tokens.
struct MoeActivations {
    float* hidden[2] = {nullptr, nullptr};  // [T, H]
    float* norm = nullptr;                  // [T, H]
    hipllm::XGroup* normq = nullptr;        // [T, H / 16] XGroup form of norm
    float* wide = nullptr;                  // [T, max(2 Hq D, qkv_w)]  Q+gate mix / DeltaNet QKV
    float* wide2 = nullptr;                 // [T, max((Hq + 2 Hkv) D, qkv_w)]  attention QKV / conv output
    float* kv = nullptr;                    // [T, 2 Hkv D]
    float* feat = nullptr;                  // [T, max(Hq D, inner)]  attention gate / DeltaNet z
    float* feat2 = nullptr;                 // [T, max(Hq D, inner)]  attention / recurrence output
    float* gated = nullptr;                 // [T, max(Hq D, inner)]
    hipllm::XGroup* gatedq = nullptr;
    float* ab = nullptr;                    // [T, 2 Hv]
    float* decay = nullptr;                 // [T, Hv]  (multi-row DeltaNet path)
    float* beta = nullptr;                  // [T, Hv]
    float* rlog = nullptr;                  // [T, E + 1] router logits | shared gate
    float* rweight = nullptr;               // [T, k]
    float* act = nullptr;                   // [T k, FF]
    hipllm::XGroup* actq = nullptr;
    float* down = nullptr;                  // [T k, H]
    float* sh_act = nullptr;                // [T, FFs]
    hipllm::XGroup* sh_actq = nullptr;
    hipllm::XGroup* inq = nullptr;          // [H / 16] next layer's input norm data (one token): x * gamma
    double* in_sumsq = nullptr;             // [H / 16] and its per-16 sums of squares
    float* sh_gate = nullptr;               // [T, FFs] shared gate projection (prefill matmul form)
    void* xb = nullptr;                     // [T, max(H, inner, Hq D, FFs)] fp16 matmul input
    float* xscale = nullptr;                // [T] its row scales
    float* sh_down = nullptr;               // [T, H]
    float* logits = nullptr;                // [V]
    float* attn_scratch = nullptr;
    void* argmax_scratch = nullptr;
    std::int32_t* ids = nullptr;            // [T] prompt / decode ids
    std::uint32_t* token = nullptr;
    std::uint32_t* step = nullptr;          // decode step inputs: [token id, position]
    std::int32_t* route_order = nullptr;    // [T k] routed vectors sorted by expert (prefill matmul path)
    std::int32_t* route_groups = nullptr;   // [route_groups_max(T k, E, 64)][2] expert groups
    std::uint32_t* route_ngroups = nullptr;
    float* gate_act = nullptr;              // [T k, FF] expert gate products (prefill matmul path)
    void* act_b = nullptr;                  // [T k, FF] fp16 SwiGLU outputs for the expert down matmul
    float* act_bscale = nullptr;            // [T k] their row scales
    float* mm_scratch = nullptr;            // router matmul partial sums (K split)
    std::size_t mm_scratch_floats = 0;
    void* split = nullptr;  // K-split partial sums of one fp16 matmul
    std::size_t split_bytes = 0;
};

}  // namespace

struct HipMoeLLM::Impl {
    int device = 0;
    std::uint64_t expert_lookups = 0;  // tokens x routes x MoE layers, all resident
    std::string device_name;
    hipStream_t stream = nullptr;
    GgufModelConfig config;
    std::size_t capacity = 0;
    std::size_t sequence_length = 0;
    std::size_t expert_cache = 0;

    WeightArena weights;
    std::size_t weight_bytes = 0;
    // Decode copies of Q4_K / Q6_K projections in the x16 tile-packed form
    // (the GGUF rows stay for the prefill matmuls).
    void* x16_arena = nullptr;
    std::size_t x16_bytes = 0;
    DevMatrix embedding, output;
    const float* output_norm = nullptr;
    std::vector<MoeLayer> layers;

    std::size_t H = 0, D = 0, Hq = 0, Hkv = 0, E = 0, K = 0, FF = 0, FFs = 0;
    std::size_t S = 0, G = 0, Hv = 0, inner = 0, qkv_w = 0, kv_w = 0, q_w = 0;

    void* state_arena = nullptr;
    std::size_t kv_cache_bytes = 0, recurrent_bytes = 0;
    float* rope_table = nullptr;
    std::int32_t* route_ids = nullptr;  // [L, rows, K]

    void* act_arena = nullptr;
    std::size_t act_bytes = 0;
    std::size_t act_rows = 0;
    MoeActivations act;
    std::int32_t* host_ids = nullptr;
    std::uint32_t* host_token = nullptr;
    std::uint32_t* host_step = nullptr;  // pinned [token id, position]
    std::size_t host_ids_cap = 0;
    std::size_t last_rows = 0;
    std::unique_ptr<RunProfiler> prof;
    GraphKernels decode_graph_kernels;

    // One decode step recorded as a HIP graph (kernels read the token and
    // position from act.step) and replayed per token.
    bool decode_graphs = true;
    bool matmul_prefill = true;  // multi-row projections as fp16 MFMA matmuls
    hipGraph_t decode_graph = nullptr;
    hipGraphExec_t decode_exec = nullptr;
    // Route probe (parity checks): the last row's router logits and shared
    // gate of every layer, [L, E + 1], copied after each router when on.
    float* probe = nullptr;
    bool probe_on = false;

    ~Impl() {
        if (stream) hipStreamSynchronize(stream);
        drop_decode_graph();
        if (host_step) hipHostFree(host_step);
        prof.reset();
        weights.release();
        if (x16_arena) hipFree(x16_arena);
        if (state_arena) hipFree(state_arena);
        if (rope_table) hipFree(rope_table);
        if (act_arena) hipFree(act_arena);
        if (route_ids) hipFree(route_ids);
        if (probe) hipFree(probe);
        if (host_ids) hipHostFree(host_ids);
        if (host_token) hipHostFree(host_token);
        if (stream) hipStreamDestroy(stream);
    }

    void load(const std::string& path, std::size_t max_sequence, int dev, std::size_t cache_count);
    void upload(GgufReader& reader);
    void pack_decode_weights();
    void allocate_state();
    void build_rope_table();
    void zero_state();
    void ensure_rows(std::size_t rows);

    void proj(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, std::size_t ldx, std::size_t rows, float* y,
              std::size_t ldy, const float* residual = nullptr, std::size_t n_override = 0,
              const void* xb = nullptr) const;
    const void* f16_rows(const float* x, std::size_t ldx, std::size_t k, std::size_t rows) const;
    void proj_out_norm(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, std::size_t ldx,
                       std::size_t rows, float* next, const float* hidden, const float* gamma, bool norm) const;
    void grouped(const hipllm::GemvJob* jobs, std::size_t count, const float* x, const float* gamma,
                 bool store_norm, const char* what) const;
    bool grouped_mixer(const MoeLayer& L, std::size_t rows) const;
    bool x16_deltanet(const MoeLayer& L, std::size_t rows) const;
    bool x16_attention_in(const MoeLayer& L, std::size_t rows) const;
    // Set by a MoE launch that left the next layer's input norm data in
    // act.inq / act.in_sumsq (one token), taken by that layer's x16 input
    // projections.
    bool in_norm = false;
    bool gathered_experts(const MoeLayer& L, std::size_t rows, const void* xb) const;
    bool grouped_moe(const MoeLayer& L, std::size_t rows) const;
    void attention_layer(std::size_t li, std::size_t rows, std::size_t pos0, float* hidden, float* next,
                         const std::uint32_t* dpos);
    void deltanet_layer(std::size_t li, std::size_t rows, float* hidden, float* next);
    void moe_layer(std::size_t li, std::size_t rows, float* hidden, float* next, const float* next_gamma,
                   bool next_norm);
    void forward(std::size_t rows, std::size_t pos0, const std::int32_t* ids, const std::uint32_t* dpos = nullptr);
    void capture_decode();
    void drop_decode_graph();
    std::int32_t read_token();
};

void HipMoeLLM::Impl::load(const std::string& path, std::size_t max_sequence, int dev, std::size_t cache_count) {
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
    const GgufModelConfig& c = reader.config();
    if (c.architecture != "qwen35moe") throw std::runtime_error("HipMoeLLM requires qwen35moe, got " + c.architecture);
    // require_qwen35_config (moe_model.cpp:39-80).
    if (c.layer_count == 0 || c.full_attention_interval == 0 || c.embedding_size == 0 ||
        c.attention_head_count == 0 || c.kv_head_count == 0 || c.head_size == 0 || c.rotary_dimension == 0 ||
        c.expert_count == 0 || c.expert_used_count == 0 || c.expert_used_count > c.expert_count ||
        c.expert_feed_forward_size == 0 || c.shared_expert_feed_forward_size == 0 || c.ssm_conv_kernel == 0 ||
        c.ssm_state_size == 0 || c.ssm_group_count == 0 || c.ssm_time_step_rank == 0 || c.ssm_inner_size == 0) {
        throw std::runtime_error("incomplete qwen35moe GGUF metadata");
    }
    if (c.rotary_dimension > c.head_size || c.rotary_dimension % 2 != 0) {
        throw std::runtime_error("qwen35moe rotary dimension must be even and fit one head");
    }
    if (c.expert_used_count > 8) throw std::runtime_error("qwen35moe currently supports at most eight selected experts");
    if (c.ssm_conv_kernel > 9 || c.ssm_conv_kernel < 2) {
        throw std::runtime_error("qwen35moe convolution kernel exceeds the history limit");
    }
    if (c.ssm_inner_size % c.ssm_time_step_rank != 0 || c.ssm_inner_size / c.ssm_time_step_rank != c.ssm_state_size) {
        throw std::runtime_error("qwen35moe DeltaNet value-head dimensions are inconsistent");
    }
    if (c.ssm_time_step_rank % c.ssm_group_count != 0) {
        throw std::runtime_error("qwen35moe DeltaNet value heads must group key heads evenly");
    }
    // What these kernels cover.
    if (c.ssm_state_size != 64 && c.ssm_state_size != 128) {
        throw std::invalid_argument("HIP DeltaNet kernels support state sizes 64 and 128");
    }
    if (c.head_size > 256 || c.head_size % 16 != 0 || c.embedding_size % 16 != 0 || c.expert_count > 1024 ||
        c.expert_feed_forward_size % 16 != 0 || c.shared_expert_feed_forward_size % 16 != 0) {
        throw std::invalid_argument("HIP MoE kernels need head size <= 256 and widths that are multiples of 16");
    }
    capacity = max_sequence == 0 ? std::min<std::size_t>(c.context_length, 1024) : max_sequence;
    if (capacity == 0 || capacity > c.context_length) {
        throw std::invalid_argument("MoE sequence capacity is outside the model context length");
    }
    if (cache_count < c.expert_used_count || cache_count > c.expert_count) {
        throw std::invalid_argument("per-layer expert cache count must be between top-k (" +
                                    std::to_string(c.expert_used_count) + ") and expert count (" +
                                    std::to_string(c.expert_count) + ")");
    }
    expert_cache = cache_count;
    config = c;
    H = c.embedding_size;
    D = c.head_size;
    Hq = c.attention_head_count;
    Hkv = c.kv_head_count;
    E = c.expert_count;
    K = c.expert_used_count;
    FF = c.expert_feed_forward_size;
    FFs = c.shared_expert_feed_forward_size;
    S = c.ssm_state_size;
    G = c.ssm_group_count;
    Hv = c.ssm_time_step_rank;
    inner = c.ssm_inner_size;
    qkv_w = 2 * G * S + inner;
    kv_w = Hkv * D;
    q_w = Hq * D;
    for (std::size_t l = c.layer_count; l < c.total_layer_count; ++l) {
        reader.ignore_prefix("blk." + std::to_string(l) + ".");  // NextN / MTP blocks (moe_model.cpp:84-94)
    }
    upload(reader);
    pack_decode_weights();
    allocate_state();
    build_rope_table();
    zero_state();
}

// x16 copies of the one-row decode GEMVs that read an XGroup input: the
// attention / DeltaNet output projections, the LM head, and every layer's
// routed expert blocks (gate, up, down; all experts of a projection packed
// as one matrix of experts x rows rows, so expert e's tiles start at e times
// its rows / 16).
void HipMoeLLM::Impl::pack_decode_weights() {
    struct Job {
        DevMatrix* m;
        std::size_t rows;  // rows packed: the matrix's, or every expert's
        bool q8 = false;   // a Q8_0 copy (the shared down projection)
    };
    std::vector<Job> jobs = {{&output, output.rows}};
    auto expert_block = [&](DevMatrix& m) {
        return x16_packable(m) && m.rows % 16 == 0 && m.expert_stride == m.rows * m.row_bytes;
    };
    for (MoeLayer& L : layers) {
        jobs.push_back({L.full ? &L.o : &L.ssm_out, (L.full ? L.o : L.ssm_out).rows});
        if (!L.full && x16_packable(L.qkv) && x16_packable(L.z)) {
            jobs.push_back({&L.qkv, L.qkv.rows});
            jobs.push_back({&L.z, L.z.rows});
        }
        // The shared expert's down projection, for the launch that runs it
        // with the routed down projections and the combine (Q8_0 too).
        // The attention's Q / gate and K / V projections, for the paired
        // launch that normalises the input in every block (K / V: Q8_0 too).
        if (L.full && L.fused_kv && x16_packable(L.qgate)) {
            L.kv = L.k;
            L.kv.rows = L.k.rows + L.v.rows;
            const bool kv8 = L.kv.type == hipllm::kQ8_0 && L.kv.cols % 256 == 0 && L.kv.row_bytes % 2 == 0;
            if (x16_packable(L.kv) || kv8) {
                jobs.push_back({&L.qgate, L.qgate.rows});
                jobs.push_back({&L.kv, L.kv.rows, kv8});
            }
        }
        const DevMatrix& sd = L.sh_down;
        const bool q8 = sd.type == hipllm::kQ8_0 && sd.cols % 256 == 0 && sd.row_bytes % 2 == 0;
        if (sd.rows % 16 == 0 && sd.cols <= 2048 && (x16_packable(sd) || q8)) jobs.push_back({&L.sh_down, sd.rows, q8});
        if (expert_block(L.gate_exps) && expert_block(L.up_exps) && L.gate_exps.type == L.up_exps.type &&
            expert_block(L.down_exps)) {
            jobs.push_back({&L.gate_exps, E * L.gate_exps.rows});
            jobs.push_back({&L.up_exps, E * L.up_exps.rows});
            jobs.push_back({&L.down_exps, E * L.down_exps.rows});
        }
    }
    std::vector<std::size_t> offs;
    std::size_t total = 0;
    for (const Job& j : jobs) {
        offs.push_back(total);
        if (j.q8 || x16_packable(*j.m)) total = align_up(total + hipllm::x16_bytes(j.m->type, j.rows, j.m->cols), 256);
    }
    if (total == 0) return;
    hip_check(hipMalloc(&x16_arena, total), "hipMalloc(x16 decode weights)");
    x16_bytes = total;
    auto* base = static_cast<std::uint8_t*>(x16_arena);
    for (std::size_t i = 0; i < jobs.size(); ++i) {
        DevMatrix& m = *jobs[i].m;
        if (!jobs[i].q8 && !x16_packable(m)) continue;
        launch_check(hipllm::launch_pack_x16(m.type, m.ptr, m.row_bytes, jobs[i].rows, m.cols, base + offs[i], stream),
                     "x16 packing");
        m.x16 = base + offs[i];
    }
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

void HipMoeLLM::Impl::upload(GgufReader& reader) {
    const GgufModelConfig& c = config;
    WeightArena& A = weights;
    auto require = [&](std::size_t idx, std::initializer_list<GgmlType> ok, const char* what) {
        const GgmlType t = A.tensor(idx).type;
        for (GgmlType g : ok) {
            if (t == g) return;
        }
        throw std::invalid_argument(std::string("HIP MoE backend does not support ") + ggml_type_name(t) + " for " +
                                    what + ": " + A.tensor(idx).name);
    };
    const std::initializer_list<GgmlType> mats = {GgmlType::F32, GgmlType::F16, GgmlType::Q5_0, GgmlType::Q8_0,
                                                  GgmlType::Q4_K, GgmlType::Q6_K};
    const std::initializer_list<GgmlType> f32 = {GgmlType::F32};
    const std::size_t V = c.vocabulary_size;
    const std::size_t i_embd = A.place(reader, "token_embd.weight", V, H);
    const std::size_t i_onorm = A.place(reader, "output_norm.weight", 1, H);
    const std::size_t i_out = A.place(reader, "output.weight", V, H);
    require(i_embd, mats, "the embedding");
    require(i_out, mats, "the output head");
    require(i_onorm, f32, "norms");
    struct Idx {
        std::size_t an, pn, qg, k, v, qn, kn, o, qkv, z, al, be, conv, dt, a, sn, so, r, shr, ge, ue, de, sg, su, sd;
    };
    std::vector<Idx> idx(c.layer_count);
    layers.resize(c.layer_count);
    for (std::size_t l = 0; l < c.layer_count; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Idx& x = idx[l];
        MoeLayer& L = layers[l];
        L.full = (l + 1) % c.full_attention_interval == 0;  // moe_model.cpp:164-166
        x.an = A.place(reader, p + "attn_norm.weight", 1, H);
        x.pn = A.place(reader, p + "post_attention_norm.weight", 1, H);
        require(x.an, f32, "norms");
        require(x.pn, f32, "norms");
        if (L.full) {
            x.qg = A.place(reader, p + "attn_q.weight", 2 * q_w, H);
            x.k = A.place(reader, p + "attn_k.weight", kv_w, H);
            x.v = A.place(reader, p + "attn_v.weight", kv_w, H, true);
            x.qn = A.place(reader, p + "attn_q_norm.weight", 1, D);
            x.kn = A.place(reader, p + "attn_k_norm.weight", 1, D);
            x.o = A.place(reader, p + "attn_output.weight", H, q_w);
            for (std::size_t i : {x.qg, x.k, x.v, x.o}) require(i, mats, "attention projections");
            require(x.qn, f32, "norms");
            require(x.kn, f32, "norms");
        } else {
            x.qkv = A.place(reader, p + "attn_qkv.weight", qkv_w, H);
            x.z = A.place(reader, p + "attn_gate.weight", inner, H);
            x.al = A.place(reader, p + "ssm_alpha.weight", Hv, H);
            x.be = A.place(reader, p + "ssm_beta.weight", Hv, H, true);
            x.conv = A.place(reader, p + "ssm_conv1d.weight", qkv_w, c.ssm_conv_kernel);
            x.dt = A.place(reader, p + "ssm_dt.bias", 1, Hv);
            x.a = A.place(reader, p + "ssm_a", 1, Hv);
            x.sn = A.place(reader, p + "ssm_norm.weight", 1, S);
            x.so = A.place(reader, p + "ssm_out.weight", H, inner);
            for (std::size_t i : {x.qkv, x.z, x.al, x.be, x.so}) require(i, mats, "DeltaNet projections");
            for (std::size_t i : {x.conv, x.dt, x.a, x.sn}) require(i, f32, "DeltaNet vectors");
        }
        x.r = A.place(reader, p + "ffn_gate_inp.weight", E, H);
        x.shr = A.place(reader, p + "ffn_gate_inp_shexp.weight", 1, H, true);
        x.ge = A.place(reader, p + "ffn_gate_exps.weight", FF * E, H);
        x.ue = A.place(reader, p + "ffn_up_exps.weight", FF * E, H);
        x.de = A.place(reader, p + "ffn_down_exps.weight", H * E, FF);
        x.sg = A.place(reader, p + "ffn_gate_shexp.weight", FFs, H);
        x.su = A.place(reader, p + "ffn_up_shexp.weight", FFs, H);
        x.sd = A.place(reader, p + "ffn_down_shexp.weight", H, FFs);
        require(x.r, mats, "the router");
        require(x.shr, mats, "the shared-expert gate");
        for (std::size_t i : {x.ge, x.ue, x.de}) require(i, {GgmlType::Q4_K, GgmlType::Q6_K}, "routed experts");
        for (std::size_t i : {x.sg, x.su, x.sd}) require(i, mats, "the shared expert");
        // Exact GGUF dimension vectors of the expert tensors (moe_model.cpp:21-37).
        const std::vector<std::uint64_t> gd = {H, FF, E}, dd = {FF, H, E};
        if (A.tensor(x.ge).dimensions != gd || A.tensor(x.ue).dimensions != gd || A.tensor(x.de).dimensions != dd) {
            throw std::runtime_error("unexpected GGUF dimensions for expert tensors of layer " + std::to_string(l));
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
    for (std::size_t l = 0; l < c.layer_count; ++l) {
        const Idx& x = idx[l];
        MoeLayer& L = layers[l];
        L.attn_norm = A.vec(x.an);
        L.post_norm = A.vec(x.pn);
        if (L.full) {
            L.qgate = A.matrix(x.qg);
            L.k = A.matrix(x.k);
            L.v = A.matrix(x.v);
            L.fused_kv = A.contiguous(x.k, x.v);
            L.q_norm = A.vec(x.qn);
            L.k_norm = A.vec(x.kn);
            L.o = A.matrix(x.o);
        } else {
            L.qkv = A.matrix(x.qkv);
            L.z = A.matrix(x.z);
            L.alpha = A.matrix(x.al);
            L.beta = A.matrix(x.be);
            L.fused_ab = A.contiguous(x.al, x.be);
            L.conv = A.vec(x.conv);
            L.dt_bias = A.vec(x.dt);
            L.a = A.vec(x.a);
            L.ssm_norm = A.vec(x.sn);
            L.ssm_out = A.matrix(x.so);
        }
        L.router = A.matrix(x.r);
        L.shexp_router = A.matrix(x.shr);
        L.fused_router = A.contiguous(x.r, x.shr);
        L.gate_exps = A.matrix(x.ge, E);
        L.up_exps = A.matrix(x.ue, E);
        L.down_exps = A.matrix(x.de, E);
        L.sh_gate = A.matrix(x.sg);
        L.sh_up = A.matrix(x.su);
        L.sh_down = A.matrix(x.sd);
    }
}

// KV caches of the full-attention layers, DeltaNet states and conv histories,
// and the per-layer route ids, in one allocation.
void HipMoeLLM::Impl::allocate_state() {
    std::size_t full = 0, dn = 0;
    for (const MoeLayer& L : layers) (L.full ? full : dn)++;
    const std::size_t cache_floats = capacity * kv_w;
    const std::size_t state_floats = Hv * S * S;
    const std::size_t hist_floats = (config.ssm_conv_kernel - 1) * qkv_w;
    kv_cache_bytes = full * 2 * cache_floats * 4;
    recurrent_bytes = dn * (state_floats + hist_floats) * 4;
    const std::size_t bytes = align_up(kv_cache_bytes, 256) + align_up(recurrent_bytes, 256) + 256;
    hip_check(hipMalloc(&state_arena, bytes), "hipMalloc(MoE state)");
    // The KV rows past the current length start at zero (a fresh allocation
    // can hold NaN/Inf bits); the recurrent part is zeroed on every reset().
    // Outside any graph capture.
    hip_check(hipMemsetAsync(state_arena, 0, bytes, stream), "hipMemsetAsync(MoE state)");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    float* p = static_cast<float*>(state_arena);
    for (MoeLayer& L : layers) {
        if (!L.full) continue;
        L.kcache = p;
        p += cache_floats;
        L.vcache = p;
        p += cache_floats;
    }
    p = reinterpret_cast<float*>(static_cast<std::uint8_t*>(state_arena) + align_up(kv_cache_bytes, 256));
    for (MoeLayer& L : layers) {
        if (L.full) continue;
        L.state = p;
        p += state_floats;
        L.history = p;
        p += hist_floats;
    }
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_token), 64, hipHostMallocDefault), "hipHostMalloc(token)");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_step), 64, hipHostMallocDefault), "hipHostMalloc(step)");
    ensure_rows(1);
}

// cos/sin for every (position, pair) of the rotary width R, with the
// reference's expression (metal_llm.metal:954-960): freq = pow(theta, -2i/R).
void HipMoeLLM::Impl::build_rope_table() {
    const std::size_t R = config.rotary_dimension, half = R / 2;
    std::vector<float> table(capacity * half * 2);
    for (std::size_t pos = 0; pos < capacity; ++pos) {
        for (std::size_t i = 0; i < half; ++i) {
            const float freq = std::pow(config.rope_theta, -2.0f * static_cast<float>(i) / static_cast<float>(R));
            const float ang = static_cast<float>(pos) * freq;
            table[2 * (pos * half + i)] = std::cos(ang);
            table[2 * (pos * half + i) + 1] = std::sin(ang);
        }
    }
    hip_check(hipMalloc(reinterpret_cast<void**>(&rope_table), table.size() * 4), "hipMalloc(RoPE)");
    hip_check(hipMemcpy(rope_table, table.data(), table.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(RoPE)");
}

// reset_state (moe_llm.mm:1531-1548): DeltaNet states and histories start at 0.
void HipMoeLLM::Impl::zero_state() {
    const std::size_t off = align_up(kv_cache_bytes, 256);
    if (recurrent_bytes) {
        hip_check(hipMemsetAsync(static_cast<std::uint8_t*>(state_arena) + off, 0, recurrent_bytes, stream),
                  "hipMemsetAsync(DeltaNet state)");
    }
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

void HipMoeLLM::Impl::ensure_rows(std::size_t n) {
    if (n <= act_rows && act_arena) return;
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    drop_decode_graph();  // it points into the arena
    if (act_arena) hipFree(act_arena);
    if (route_ids) hipFree(route_ids);
    if (host_ids) hipHostFree(host_ids);
    act_arena = nullptr;
    route_ids = nullptr;
    host_ids = nullptr;
    act_rows = 0;
    const std::size_t wide = std::max(2 * q_w, qkv_w), wide2 = std::max(q_w + 2 * kv_w, qkv_w);
    // The router matmul's K split needs the most scratch at some row count
    // below n (fewer rows, more splits): the largest over 1..n.
    std::size_t mm_floats = 0;
    for (std::size_t r = kRouterMatmulRows; r <= n; ++r) {
        mm_floats = std::max(mm_floats, hipllm::matmul_f32_scratch_floats(r, E + 1, H));
    }
    // Likewise the K-split partial sums of the fp16 projection matmuls.
    const std::size_t mm_shapes[][2] = {{2 * q_w, H}, {kv_w, H},   {2 * kv_w, H}, {qkv_w, H},
                                        {inner, H},   {Hv, H},     {2 * Hv, H},   {H, q_w},
                                        {H, inner},   {FFs, H},    {H, FFs}};
    std::size_t split_bytes = 0;
    for (std::size_t r = kMatmulRows; r <= n; ++r) {
        for (const auto& nk : mm_shapes) {
            if (nk[1] % 128 == 0) split_bytes = std::max(split_bytes, hipllm::gemm_split_bytes(r, nk[0], nk[1], -1, 0));
        }
        if (H % 128 == 0) split_bytes = std::max(split_bytes, hipllm::gemm_swiglu_bytes(r, FFs, H));
    }
    const std::size_t feat = std::max(q_w, inner);
    std::size_t off = 0;
    auto reserve = [&](std::size_t floats) {
        const std::size_t at = off;
        off = align_up(off + floats * 4, 256);
        return at;
    };
    const std::size_t o_h0 = reserve(n * H), o_h1 = reserve(n * H), o_norm = reserve(n * H),
                      o_normq = reserve(n * H), o_wide = reserve(n * wide), o_wide2 = reserve(n * wide2),
                      o_kv = reserve(n * 2 * kv_w), o_feat = reserve(n * feat), o_feat2 = reserve(n * feat),
                      o_gated = reserve(n * feat), o_gatedq = reserve(n * feat), o_ab = reserve(n * 2 * Hv),
                      o_decay = reserve(n * Hv), o_beta = reserve(n * Hv), o_rlog = reserve(n * (E + 1)),
                      o_rw = reserve(n * K), o_act = reserve(n * K * FF), o_actq = reserve(n * K * FF),
                      o_down = reserve(n * K * H), o_sha = reserve(n * FFs), o_shaq = reserve(n * FFs),
                      o_shd = reserve(n * H), o_logits = reserve(config.vocabulary_size),
                      o_as = reserve(hipllm::attn_decode_scratch_floats(Hq, D, capacity)),
                      o_am = reserve(hipllm::argmax_scratch_bytes(config.vocabulary_size) / 4 + 1),
                      o_ids = reserve(n), o_tok = reserve(16), o_step = reserve(4),
                      o_shg = reserve(n * FFs), o_xb = reserve((n * std::max({H, inner, q_w, FFs}) + 1) / 2),
                      o_ord = reserve(n * K),
                      o_grp = reserve(2 * std::max(hipllm::route_groups_max(n * K, E, hipllm::kGatherRows),
                                                   hipllm::route_groups_max(n * K, E, hipllm::kX16GroupRows))),
                      o_ngr = reserve(1), o_gact = reserve(n * K * FF), o_actb = reserve((n * K * FF + 1) / 2),
                      o_xs = reserve(n), o_abs = reserve(n * K),
                      o_mms = reserve(mm_floats), o_split = reserve(split_bytes / 4), o_inq = reserve(H),
                      o_inss = reserve(H / 8);
    act_bytes = off;
    hip_check(hipMalloc(&act_arena, act_bytes), "hipMalloc(MoE activations)");
    auto* b = static_cast<std::uint8_t*>(act_arena);
    auto f = [&](std::size_t o) { return reinterpret_cast<float*>(b + o); };
    auto g = [&](std::size_t o) { return reinterpret_cast<hipllm::XGroup*>(b + o); };  // 16 floats per group
    act.hidden[0] = f(o_h0);
    act.hidden[1] = f(o_h1);
    act.norm = f(o_norm);
    act.normq = g(o_normq);
    act.inq = g(o_inq);
    act.in_sumsq = reinterpret_cast<double*>(b + o_inss);
    act.wide = f(o_wide);
    act.wide2 = f(o_wide2);
    act.kv = f(o_kv);
    act.feat = f(o_feat);
    act.feat2 = f(o_feat2);
    act.gated = f(o_gated);
    act.gatedq = g(o_gatedq);
    act.ab = f(o_ab);
    act.decay = f(o_decay);
    act.beta = f(o_beta);
    act.rlog = f(o_rlog);
    act.rweight = f(o_rw);
    act.act = f(o_act);
    act.actq = g(o_actq);
    act.down = f(o_down);
    act.sh_act = f(o_sha);
    act.sh_actq = g(o_shaq);
    act.sh_gate = f(o_shg);
    act.xb = b + o_xb;
    act.xscale = f(o_xs);
    act.sh_down = f(o_shd);
    act.logits = f(o_logits);
    act.attn_scratch = f(o_as);
    act.argmax_scratch = b + o_am;
    act.ids = reinterpret_cast<std::int32_t*>(b + o_ids);
    act.token = reinterpret_cast<std::uint32_t*>(b + o_tok);
    act.step = reinterpret_cast<std::uint32_t*>(b + o_step);
    act.route_order = reinterpret_cast<std::int32_t*>(b + o_ord);
    act.route_groups = reinterpret_cast<std::int32_t*>(b + o_grp);
    act.route_ngroups = reinterpret_cast<std::uint32_t*>(b + o_ngr);
    act.gate_act = f(o_gact);
    act.act_b = b + o_actb;
    act.act_bscale = f(o_abs);
    act.mm_scratch = f(o_mms);
    act.mm_scratch_floats = mm_floats;
    act.split = split_bytes ? b + o_split : nullptr;
    act.split_bytes = split_bytes;
    hip_check(hipMalloc(reinterpret_cast<void**>(&route_ids), layers.size() * n * K * 4), "hipMalloc(routes)");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&host_ids), n * 4, hipHostMallocDefault), "hipHostMalloc(ids)");
    act_rows = n;
}

// y[rows, :] = W x[rows, :] (+ residual); one GEMV per row, batched over rows.
void HipMoeLLM::Impl::proj(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, std::size_t ldx, std::size_t rows,
                           float* y, std::size_t ldy, const float* residual, std::size_t n_override,
                           const void* xb) const {
    const std::size_t n = n_override ? n_override : w.rows;
    if (xb) {
        // Prefill rows through the fp16 MFMA matmul (xb: f16_rows of x, row
        // scales in act.xscale).
        launch_check(hipllm::launch_gemm_mfma(w.type, w.ptr, w.row_bytes, xb, act.xscale, nullptr, residual, y, rows, n,
                                              w.cols, -1, 0, stream, ldy, act.split, act.split_bytes),
                     "prefill matmul");
        return;
    }
    if (rows == 1) {
        if (w.x16 && xq && n == w.rows) {
            launch_check(hipllm::launch_gemv_x16(w.type, w.x16, xq, nullptr, residual, y, n, w.cols, 0, stream),
                         "GEMV");
            return;
        }
        launch_check(hipllm::launch_gemv_prepped(w.type, w.ptr, w.row_bytes, x, xq, nullptr, residual, y, n, w.cols,
                                                 0, stream),
                     "GEMV");
        return;
    }
    launch_check(hipllm::launch_gemv_batched(w.type, w.ptr, nullptr, w.row_bytes, x, xq, nullptr, residual, y,
                                             nullptr, n, w.cols, rows, nullptr, 1, 1, 0, 0, ldx, ldy, stream),
                 "batched GEMV");
}

// The fp16 copy of `rows` rows of x (k values, ld ldx) that the prefill
// matmul reads, in act.xb (row scales in act.xscale); nullptr when the rows go
// through the GEMV forms
// (few rows, or k not a multiple of the matmul's 128-k step). One copy per
// input: every projection of the same rows shares it until the next call.
const void* HipMoeLLM::Impl::f16_rows(const float* x, std::size_t ldx, std::size_t k, std::size_t rows) const {
    if (!matmul_prefill || rows < kMatmulRows || k % 128 != 0) return nullptr;
    launch_check(hipllm::launch_to_f16(x, ldx, act.xb, act.xscale, rows, k, stream), "fp16 activations");
    return act.xb;
}

// Output projection of a mixer block with the residual, next = hidden + W x,
// then (norm) act.norm = rmsnorm(next) * gamma (the post-mixer norm; the
// grouped router launch applies it otherwise).
void HipMoeLLM::Impl::proj_out_norm(const DevMatrix& w, const float* x, const hipllm::XGroup* xq, std::size_t ldx,
                                    std::size_t rows, float* next, const float* hidden, const float* gamma,
                                    bool norm) const {
    proj(w, x, xq, ldx, rows, next, H, hidden, 0, f16_rows(x, ldx, w.cols, rows));
    if (!norm) return;
    launch_check(hipllm::launch_rmsnorm(next, gamma, act.norm, act.normq, rows, H, config.norm_epsilon, stream),
                 "RMSNorm");
}

// One grouped GEMV launch over rmsnorm(x) * gamma (one row); store_norm:
// also write the normalised row and its XGroup form to act.norm / normq.
void HipMoeLLM::Impl::grouped(const hipllm::GemvJob* jobs, std::size_t count, const float* x, const float* gamma,
                              bool store_norm, const char* what) const {
    launch_check(hipllm::launch_gemv_multi_norm(jobs, count, x, gamma, config.norm_epsilon, H,
                                                store_norm ? act.norm : nullptr, store_norm ? act.normq : nullptr,
                                                stream),
                 what);
}

namespace {
hipllm::GemvJob job(const DevMatrix& w, float* y, std::size_t n) {
    hipllm::GemvJob j;
    j.type = w.type;
    j.w = w.ptr;
    j.row_bytes = w.row_bytes;
    j.y = y;
    j.n = static_cast<std::uint32_t>(n);
    return j;
}

// Weight types the grouped launch multiplies (mode 0; mode 1 quantized only).
bool groupable(const DevMatrix& w, bool swiglu = false) {
    const bool quant = w.type == hipllm::kQ4_K || w.type == hipllm::kQ6_K || w.type == hipllm::kQ8_0 ||
                       w.type == hipllm::kQ5_0;
    return quant || (!swiglu && w.type == hipllm::kF32);
}
}  // namespace

// Whether layer L's input-norm projections run as one grouped launch.
bool HipMoeLLM::Impl::grouped_mixer(const MoeLayer& L, std::size_t rows) const {
    if (rows != kGroupedRows || H % 256 != 0 || H > 8192) return false;
    if (L.full) return groupable(L.qgate) && groupable(L.k) && (L.fused_kv || groupable(L.v));
    return groupable(L.qkv) && groupable(L.z) && L.fused_ab && groupable(L.alpha);
}

// Whether DeltaNet layer L's decode step runs on the x16 copies: QKV (with
// the conv in its epilogue) and z as one paired launch that normalises the
// input in every block, then one launch per value head for alpha / beta,
// the L2 norms, the recurrence and the gated norm.
bool HipMoeLLM::Impl::x16_deltanet(const MoeLayer& L, std::size_t rows) const {
    return !L.full && rows == 1 && grouped_mixer(L, rows) && L.qkv.x16 && L.z.x16 &&
           L.alpha.type == hipllm::kF32 && L.fused_ab && H <= 4096 && (S == 64 || S == 128) &&
           config.ssm_conv_kernel >= 2 && config.ssm_conv_kernel <= 4;
}

// Whether attention layer L's decode step runs its Q / gate and K / V
// projections on the x16 copies as one paired launch.
bool HipMoeLLM::Impl::x16_attention_in(const MoeLayer& L, std::size_t rows) const {
    return L.full && rows == 1 && grouped_mixer(L, rows) && L.qgate.x16 && L.kv.x16 && H <= 8192;
}

// Whether layer L's routed experts run as gathered fp16 matmuls: a prompt
// whose dense projections already run as matmuls (xb holds its fp16 rows)
// and routes at least four vectors per expert on average. Each group block
// dequantizes a whole weight tile for its vectors, so with fewer the batched
// GEMV is faster (qwen35moe prefill, 256 experts top-8: 64 tokens 3.06k
// against 3.47k tok/s, 128 tokens 4.73k against 4.32k, 512 tokens 8.30k
// against 5.16k, 1024 tokens 8.85k against 4.92k).
bool HipMoeLLM::Impl::gathered_experts(const MoeLayer&, std::size_t rows, const void* xb) const {
    return xb && rows * K >= 4 * E && rows * K <= 16384 && E <= 1024 && H % 128 == 0 && FF % 128 == 0;
}

// Whether layer L's router and shared gate/up run as one grouped launch.
bool HipMoeLLM::Impl::grouped_moe(const MoeLayer& L, std::size_t rows) const {
    if (rows != kGroupedRows || H % 256 != 0 || H > 8192 || FFs % 16 != 0) return false;
    return groupable(L.router) && (L.fused_router || groupable(L.shexp_router)) && groupable(L.sh_gate, true) &&
           L.sh_gate.type == L.sh_up.type && L.sh_gate.row_bytes == L.sh_up.row_bytes &&
           groupable(L.sh_down, true) && FFs <= 8192;
}

// Gated full attention (moe_llm.mm:2238-2434) over `rows` rows at positions
// pos0.. ; next = hidden + out_proj(attention * sigmoid(gate)).
// dpos (device, nullable): the decode position read on the device (recorded
// decode step); pos0 is used otherwise.
void HipMoeLLM::Impl::attention_layer(std::size_t li, std::size_t rows, std::size_t pos0, float* hidden,
                                      float* next, const std::uint32_t* dpos) {
    const MoeLayer& L = layers[li];
    const float eps = config.norm_epsilon;
    const std::size_t ldqkv = q_w + 2 * kv_w;
    if (x16_attention_in(L, rows)) {
        // One token: Q / gate and K / V on their x16 copies in one launch,
        // from the norm data the previous MoE launch left, or with every
        // block normalising the input itself.
        launch_check(hipllm::launch_gemv_x16_pair(L.qgate.type, L.qgate.x16, L.qgate.rows, act.wide, L.kv.type,
                                                  L.kv.x16, L.kv.rows, act.kv, H, hidden, L.attn_norm, eps, nullptr,
                                                  nullptr, 0, stream, in_norm ? act.inq : nullptr,
                                                  in_norm ? act.in_sumsq : nullptr),
                     "input norm + Q/gate + K/V");
        in_norm = false;
    } else if (grouped_mixer(L, rows)) {
        hipllm::GemvJob jobs[3];
        std::size_t nj = 0;
        jobs[nj++] = job(L.qgate, act.wide, L.qgate.rows);
        if (L.fused_kv) {
            jobs[nj++] = job(L.k, act.kv, 2 * kv_w);
        } else {
            jobs[nj++] = job(L.k, act.kv, L.k.rows);
            jobs[nj++] = job(L.v, act.kv + kv_w, L.v.rows);
        }
        grouped(jobs, nj, hidden, L.attn_norm, false, "input norm + Q/gate + K/V");
    } else {
        const void* xb = f16_rows(act.norm, H, H, rows);
        proj(L.qgate, act.norm, act.normq, H, rows, act.wide, 2 * q_w, nullptr, 0, xb);
        if (L.fused_kv) {
            proj(L.k, act.norm, act.normq, H, rows, act.kv, 2 * kv_w, nullptr, 2 * kv_w, xb);
        } else {
            proj(L.k, act.norm, act.normq, H, rows, act.kv, 2 * kv_w, nullptr, 0, xb);
            proj(L.v, act.norm, act.normq, H, rows, act.kv + kv_w, 2 * kv_w, nullptr, 0, xb);  // after K in each row
        }
    }
    const float scale0 = 1.0f / std::sqrt(static_cast<float>(D));
    if (rows == 1 && hipllm::attn_decode_qgate_fits(dpos ? capacity : pos0 + 1, D)) {
        // One token: the Q / K head norms, RoPE, KV-cache write, attention
        // and output gate in one launch.
        launch_check(hipllm::launch_attn_decode_qgate(act.wide, act.kv, L.q_norm, L.k_norm, eps, rope_table,
                                                      config.rotary_dimension, L.kcache, L.vcache, act.gated,
                                                      act.gatedq, Hq, Hkv, D, pos0, scale0, stream, dpos, capacity),
                     "Q/K head norms + RoPE/KV write + attention + output gate");
        proj_out_norm(L.o, act.gated, act.gatedq, q_w, rows, next, hidden, L.post_norm, !grouped_moe(L, rows));
        return;
    }
    launch_check(hipllm::launch_split_qgate_norm(act.wide, 2 * q_w, act.kv, 2 * kv_w, L.q_norm, L.k_norm, act.wide2,
                                                 ldqkv, act.feat, q_w, rows, Hq, Hkv, D, eps, stream),
                 "Q/gate split + head norms");
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    if (rows == 1) {
        // RoPE of Q and K, the KV-cache write, the attention and its output
        // gate fused.
        launch_check(hipllm::launch_attn_decode_rope(act.wide2, rope_table, config.rotary_dimension, L.kcache,
                                                     L.vcache, act.gated, act.gatedq, act.attn_scratch, Hq, Hkv, D,
                                                     pos0, scale, stream, dpos, capacity, act.feat),
                     "RoPE/KV write + attention + output gate");
    } else {
        launch_check(hipllm::launch_rope_kv(act.wide2, rope_table, config.rotary_dimension, Hq, Hkv, D, pos0, rows,
                                            ldqkv, L.kcache, L.vcache, stream, dpos),
                     "RoPE/KV write");
        launch_check(hipllm::launch_attn_prefill(act.wide2, ldqkv, L.kcache, L.vcache, act.feat2, q_w, rows, Hq, Hkv,
                                                 D, pos0, scale, stream),
                     "prefill attention");
    }
    if (rows != 1) {
        launch_check(hipllm::launch_gate_mul(act.feat2, act.feat, act.gated, act.gatedq, rows * q_w, stream),
                     "attention output gate");
    }
    proj_out_norm(L.o, act.gated, act.gatedq, q_w, rows, next, hidden, L.post_norm, !grouped_moe(L, rows));
}

// Gated DeltaNet (moe_llm.mm:2436-2640); next = hidden + out_proj(...).
void HipMoeLLM::Impl::deltanet_layer(std::size_t li, std::size_t rows, float* hidden, float* next) {
    const MoeLayer& L = layers[li];
    const float eps = config.norm_epsilon;
    if (x16_deltanet(L, rows)) {
        launch_check(hipllm::launch_gemv_x16_pair(L.qkv.type, L.qkv.x16, qkv_w, act.wide, L.z.type, L.z.x16, inner,
                                                  act.feat, H, hidden, L.attn_norm, eps, L.conv, L.history,
                                                  config.ssm_conv_kernel, stream, in_norm ? act.inq : nullptr,
                                                  in_norm ? act.in_sumsq : nullptr),
                     "input norm + DeltaNet QKV (+ conv) / z");
        in_norm = false;
        launch_check(hipllm::launch_gdn_decode(act.wide, hidden, L.attn_norm,
                                               reinterpret_cast<const float*>(L.alpha.ptr), H, L.dt_bias, L.a,
                                               L.state, act.feat, L.ssm_norm, act.gated, act.gatedq, Hv, G, S, eps,
                                               stream),
                     "DeltaNet alpha / beta + L2 norms + scan + gated norm");
        proj_out_norm(L.ssm_out, act.gated, act.gatedq, inner, rows, next, hidden, L.post_norm,
                      !grouped_moe(L, rows));
        return;
    }
    if (grouped_mixer(L, rows)) {
        const hipllm::GemvJob jobs[3] = {job(L.qkv, act.wide, L.qkv.rows), job(L.z, act.feat, L.z.rows),
                                         job(L.alpha, act.ab, 2 * Hv)};
        grouped(jobs, 3, hidden, L.attn_norm, false, "input norm + DeltaNet QKV / z / alpha, beta");
    } else {
        const void* xb = f16_rows(act.norm, H, H, rows);
        proj(L.qkv, act.norm, act.normq, H, rows, act.wide, qkv_w, nullptr, 0, xb);
        proj(L.z, act.norm, act.normq, H, rows, act.feat, inner, nullptr, 0, xb);
        if (L.fused_ab) {
            proj(L.alpha, act.norm, act.normq, H, rows, act.ab, 2 * Hv, nullptr, 2 * Hv, xb);
        } else {
            proj(L.alpha, act.norm, act.normq, H, rows, act.ab, 2 * Hv, nullptr, 0, xb);
            proj(L.beta, act.norm, act.normq, H, rows, act.ab + Hv, 2 * Hv, nullptr, 0, xb);  // after alpha in each row
        }
    }
    if (rows <= kFusedDeltaNetRows) {
        // Decode: causal conv + SiLU with the Q and K heads (2 G vectors of
        // S per row, contiguous) L2-normalised in the same pass, then the
        // gates, recurrence and gated RMSNorm in one launch (block per value
        // head).
        launch_check(hipllm::launch_conv_l2norm(act.wide, qkv_w, L.history, L.conv, act.wide2, qkv_w, rows, qkv_w,
                                                config.ssm_conv_kernel, 2 * G * S, S, eps, stream),
                     "DeltaNet conv + L2 norm");
        launch_check(hipllm::launch_gdn_scan_gated(act.wide2, act.wide2 + G * S, qkv_w, act.wide2 + 2 * G * S, qkv_w,
                                                   act.ab, act.ab + Hv, 2 * Hv, L.dt_bias, L.a, L.state, act.feat,
                                                   inner, L.ssm_norm, act.gated, act.gatedq, inner, rows, Hv, G, S,
                                                   eps, stream),
                     "DeltaNet scan + gated norm");
    } else {
        // Many rows: the per-row steps that parallelise over rows run as
        // their own launches, and the scan runs one wave per four state
        // columns (each column's recurrence is independent).
        launch_check(hipllm::launch_gdn_gates(act.ab, act.ab + Hv, 2 * Hv, L.dt_bias, L.a, act.decay, act.beta, rows,
                                              Hv, stream),
                     "DeltaNet gates");
        launch_check(hipllm::launch_conv1d_silu(act.wide, qkv_w, L.history, L.conv, act.wide2, qkv_w, rows, qkv_w,
                                                config.ssm_conv_kernel, stream),
                     "DeltaNet conv");
        launch_check(hipllm::launch_l2norm_heads(act.wide2, qkv_w, rows, 2 * G, S, eps, stream), "DeltaNet L2 norm");
        launch_check(hipllm::launch_gdn_scan(act.wide2, act.wide2 + G * S, qkv_w, act.wide2 + 2 * G * S, qkv_w,
                                             act.decay, act.beta, L.state, act.feat2, inner, rows, Hv, G, S, stream),
                     "DeltaNet scan");
        launch_check(hipllm::launch_gated_rmsnorm(act.feat2, inner, L.ssm_norm, act.feat, inner, act.gated,
                                                  act.gatedq, inner, rows, Hv, S, eps, stream),
                     "DeltaNet gated norm");
    }
    proj_out_norm(L.ssm_out, act.gated, act.gatedq, inner, rows, next, hidden, L.post_norm, !grouped_moe(L, rows));
}

// MoE FFN (moe_llm.mm:2642-2843): `hidden` is the attention residual; the
// post-attention norm of it is in act.norm (or is made by the grouped router
// launch); next = hidden + routed + shared. next_gamma: the gain of the
// RMSNorm that follows (next layer's input norm or the output norm), applied
// to `next` into act.norm in the combine launch when next_norm (otherwise the
// next layer's grouped launch normalises in its prologue).
void HipMoeLLM::Impl::moe_layer(std::size_t li, std::size_t rows, float* hidden, float* next,
                                const float* next_gamma, bool next_norm) {
    const MoeLayer& L = layers[li];
    std::int32_t* ids = route_ids + li * act_rows * K;
    // Router logits and the shared-expert gate in one GEMV when packed.
    // The router logits stay FP32 (GEMV forms) in every path: top-k is
    // discontinuous, and fp16 rounding of the logits would flip near-tie
    // routes.
    const std::size_t ldr = E + 1;
    const bool grp = grouped_moe(L, rows);
    if (grp) {
        // Post-attention norm (stored for the expert projections), router,
        // shared-expert gate and shared gate/up + SwiGLU in one launch. The
        // SwiGLU output stays FP32 (4-row blocks, four times as many as the
        // 16-row blocks its XGroup form would need); the shared down
        // projection encodes it in its prologue.
        hipllm::GemvJob jobs[3];
        std::size_t nj = 0;
        if (L.fused_router) {
            jobs[nj++] = job(L.router, act.rlog, E + 1);
        } else {
            jobs[nj++] = job(L.router, act.rlog, E);
            jobs[nj++] = job(L.shexp_router, act.rlog + E, 1);
        }
        hipllm::GemvJob sh = job(L.sh_gate, act.sh_act, FFs);
        sh.mode = 1;
        sh.w2 = L.sh_up.ptr;
        jobs[nj++] = sh;
        grouped(jobs, nj, hidden, L.post_norm, true, "post-attention norm + router + shared gate/up");
    } else if (L.fused_router && rows >= kRouterMatmulRows && L.router.type == hipllm::kF32) {
        // A prompt: the router (and shared-expert gate) rows as an FP32 matmul.
        launch_check(hipllm::launch_matmul_f32(act.norm, H, reinterpret_cast<const float*>(L.router.ptr),
                                               L.router.row_bytes / 4, act.rlog, ldr, rows, E + 1, H, act.mm_scratch,
                                               act.mm_scratch_floats, stream),
                     "router (matmul)");
    } else if (L.fused_router) {
        proj(L.router, act.norm, act.normq, H, rows, act.rlog, ldr, nullptr, E + 1);
    } else {
        proj(L.router, act.norm, act.normq, H, rows, act.rlog, ldr);
        proj(L.shexp_router, act.norm, act.normq, H, rows, act.rlog + E, ldr);
    }
    if (probe_on) {
        hip_check(hipMemcpyAsync(probe + li * ldr, act.rlog + (rows - 1) * ldr, ldr * 4, hipMemcpyDeviceToDevice,
                                 stream),
                  "hipMemcpyAsync(route probe)");
    }
    // With the grouped launch, the expert gate/up picks the routes itself
    // (every block runs the top-k on the token's logits).
    const bool route_in_gemv = grp && E <= 256 && K <= 8 && groupable(L.gate_exps, true);
    if (!route_in_gemv) {
        launch_check(hipllm::launch_router_topk(act.rlog, ldr, rows, E, K, ids, act.rweight, stream),
                     "router top-k");
    }
    const void* xb = f16_rows(act.norm, H, H, rows);
    // Routed experts: gate/up + SwiGLU (and its XGroup form) for every
    // (row, route), then down.
    const bool x16_experts = rows == 1 && E <= 256 && K <= 8 && L.gate_exps.x16 && L.up_exps.x16 && L.down_exps.x16;
    // Prompts below the gathered-matmul threshold: the expert-grouped x16
    // products (the vector form reads an expert's weights once per vector).
    const bool x16_grouped = rows > 1 && !x16_experts && !route_in_gemv && !gathered_experts(L, rows, xb) &&
                             L.gate_exps.x16 && L.up_exps.x16 && L.down_exps.x16 && L.gate_exps.type == L.up_exps.type &&
                             FF % 16 == 0 && H % 16 == 0;
    const std::size_t x16_groups = hipllm::route_groups_max(rows * K, E, hipllm::kX16GroupRows);
    if (x16_experts) {
        // One token: the expert gate / up pair on the x16 copies, with the
        // top-k in the kernel when the grouped launch left it to the experts
        // (ids and weights stored for down and the combine).
        launch_check(hipllm::launch_gemv_x16_routed(L.gate_exps.type, L.gate_exps.x16, L.up_exps.x16, act.normq, H, 0,
                                                    act.act, act.actq, FF, FF, H, E, K, route_in_gemv ? nullptr : ids,
                                                    route_in_gemv ? act.rlog : nullptr, route_in_gemv ? ids : nullptr,
                                                    route_in_gemv ? act.rweight : nullptr, 0, stream),
                     "router top-k + expert gate/up");
    } else if (route_in_gemv) {
        launch_check(hipllm::launch_gemv_routed_swiglu(L.gate_exps.type, L.gate_exps.ptr, L.up_exps.ptr,
                                                       L.gate_exps.row_bytes, act.norm, act.normq, H, act.act,
                                                       act.actq, FF, H, rows, act.rlog, ldr, E, K,
                                                       L.gate_exps.expert_stride, ids, act.rweight, stream),
                     "router top-k + expert gate/up");
    } else if (gathered_experts(L, rows, xb)) {
        // A prompt: the routed vectors grouped by expert (up to 64 per group)
        // and each group multiplied as an fp16 MFMA matmul that reads its
        // expert's weights once, gate and up, SwiGLU, then down.
        const std::size_t nv = rows * K, mg = hipllm::route_groups_max(nv, E, hipllm::kGatherRows);
        launch_check(hipllm::launch_route_groups(ids, nv, E, hipllm::kGatherRows, act.route_order, act.route_groups,
                                                 act.route_ngroups, stream),
                     "route groups");
        auto gather = [&](const DevMatrix& w, const void* x, const float* xs, float* y, std::size_t n, std::size_t k,
                          int routed, const char* what) {
            launch_check(hipllm::launch_gemm_gather(w.type, w.ptr, w.row_bytes, x, xs, y, n, k, n, act.route_order,
                                                    act.route_groups, act.route_ngroups, mg, w.expert_stride, K,
                                                    routed, stream),
                         what);
        };
        gather(L.gate_exps, xb, act.xscale, act.gate_act, FF, H, 0, "expert gate (matmul)");
        gather(L.up_exps, xb, act.xscale, act.act, FF, H, 0, "expert up (matmul)");
        launch_check(hipllm::launch_swiglu(act.gate_act, act.act, act.act, act.actq, nv * FF, stream),
                     "expert SwiGLU");
        launch_check(hipllm::launch_to_f16(act.act, FF, act.act_b, act.act_bscale, nv, FF, stream),
                     "expert fp16 activations");
        gather(L.down_exps, act.act_b, act.act_bscale, act.down, H, FF, 1, "expert down (matmul)");
    } else if (x16_grouped) {
        // A short prompt: the routed vectors grouped by expert (at most four
        // per group) and each expert tile of the x16 copies read once per
        // group, gate / up with SwiGLU, then down.
        launch_check(hipllm::launch_route_groups(ids, rows * K, E, hipllm::kX16GroupRows, act.route_order,
                                                 act.route_groups, act.route_ngroups, stream),
                     "route groups");
        launch_check(hipllm::launch_x16_grouped(L.gate_exps.type, L.gate_exps.x16, L.up_exps.x16, act.normq, H, 0, K,
                                                act.act, act.actq, FF, FF, H, E, act.route_order, act.route_groups,
                                                act.route_ngroups, x16_groups, stream),
                     "expert gate/up (x16, grouped)");
    } else {
        launch_check(hipllm::launch_gemv_batched(L.gate_exps.type, L.gate_exps.ptr, L.up_exps.ptr,
                                                 L.gate_exps.row_bytes, act.norm, act.normq, nullptr, nullptr,
                                                 act.act, act.actq, FF, H, rows * K, ids, E, K,
                                                 L.gate_exps.expert_stride, 0, H, FF, stream),
                     "expert gate/up");
    }
    // One token after the grouped launch: the routed and shared down
    // projections and the combine as one launch on the x16 copies.
    const bool x16_down = x16_experts && grp && !next_norm && L.sh_down.x16 && FF % 256 == 0 && FFs <= 2048 &&
                          H % 16 == 0;
    if (x16_down) {
        // The next layer's x16 input projections take their norm from data
        // this launch leaves (the XGroup form of next * gamma, per-16 sums of
        // squares).
        const bool last = li + 1 == layers.size();
        const bool norm_out = !last && H % 16 == 0 &&
                              (x16_deltanet(layers[li + 1], rows) || x16_attention_in(layers[li + 1], rows));
        hipllm::X16Norm out{};
        out.gamma_out = next_gamma;
        out.yq_out = act.inq;
        out.sumsq_out = act.in_sumsq;
        launch_check(hipllm::launch_x16_moe_down(L.down_exps.type, L.down_exps.x16, ids, E, act.actq, FF, FF,
                                                 L.sh_down.type, L.sh_down.x16, act.sh_act, FFs, act.rweight,
                                                 act.rlog + E, hidden, next, H, K, stream, norm_out ? &out : nullptr),
                     "expert down + shared down + MoE combine");
        in_norm = norm_out;
        return;
    }
    if (x16_experts) {
        launch_check(hipllm::launch_gemv_x16_routed(L.down_exps.type, L.down_exps.x16, nullptr, act.actq, FF, 1,
                                                    act.down, nullptr, H, H, FF, E, K, ids, nullptr, nullptr, nullptr,
                                                    0, stream),
                     "expert down");
    } else if (x16_grouped) {
        launch_check(hipllm::launch_x16_grouped(L.down_exps.type, L.down_exps.x16, nullptr, act.actq, FF, 1, K,
                                                act.down, nullptr, H, H, FF, E, act.route_order, act.route_groups,
                                                act.route_ngroups, x16_groups, stream),
                     "expert down (x16, grouped)");
    } else if (!gathered_experts(L, rows, xb)) {
        launch_check(hipllm::launch_gemv_batched(L.down_exps.type, L.down_exps.ptr, nullptr, L.down_exps.row_bytes,
                                                 act.act, act.actq, nullptr, nullptr, act.down, nullptr, H, FF,
                                                 rows * K, ids, E, K, L.down_exps.expert_stride, 1, FF, H, stream),
                     "expert down");
    }
    // Shared expert (gate/up already in sh_act after a grouped launch).
    bool sh_f16 = false;  // the shared activations are already act.xb's fp16 rows
    if (!grp && xb && FFs % 128 == 0 && FFs <= 32768 && L.sh_gate.type == L.sh_up.type &&
        L.sh_gate.row_bytes == L.sh_up.row_bytes &&
        (L.sh_gate.type == hipllm::kQ4_K || L.sh_gate.type == hipllm::kQ6_K || L.sh_gate.type == hipllm::kQ8_0 ||
         L.sh_gate.type == hipllm::kQ5_0)) {
        // Gate and up keep their partial planes; one launch reduces both,
        // applies the SwiGLU and writes the down projection's fp16 rows into
        // act.xb (after the matmuls have read it; no FP32 or XGroup form).
        launch_check(hipllm::launch_gemm_mfma_swiglu(L.sh_gate.type, L.sh_gate.ptr, L.sh_up.ptr, L.sh_gate.row_bytes,
                                                     xb, act.xscale, nullptr, rows, FFs, H, FFs, act.split,
                                                     act.split_bytes, stream, act.xb, act.xscale),
                     "prefill shared gate / up + SwiGLU");
        sh_f16 = true;
    } else if (!grp && xb) {
        proj(L.sh_gate, act.norm, act.normq, H, rows, act.sh_gate, FFs, nullptr, 0, xb);
        proj(L.sh_up, act.norm, act.normq, H, rows, act.sh_act, FFs, nullptr, 0, xb);
        launch_check(hipllm::launch_swiglu(act.sh_gate, act.sh_act, act.sh_act, act.sh_actq, rows * FFs, stream),
                     "shared SwiGLU");
    } else if (!grp && L.sh_gate.type == L.sh_up.type) {
        launch_check(hipllm::launch_gemv_batched(L.sh_gate.type, L.sh_gate.ptr, L.sh_up.ptr, L.sh_gate.row_bytes,
                                                 act.norm, act.normq, nullptr, nullptr, act.sh_act, nullptr, FFs,
                                                 H, rows, nullptr, 1, 1, 0, 0, H, FFs, stream),
                     "shared gate/up");
        launch_check(hipllm::launch_prep_x(act.sh_act, act.sh_actq, rows * FFs, stream), "shared activations");
    } else if (!grp) {
        proj(L.sh_gate, act.norm, act.normq, H, rows, act.sh_down, FFs);
        proj(L.sh_up, act.norm, act.normq, H, rows, act.sh_act, FFs);
        launch_check(hipllm::launch_swiglu(act.sh_down, act.sh_act, act.sh_act, act.sh_actq, rows * FFs, stream),
                     "shared SwiGLU");
    }
    if (grp && !next_norm) {
        // The combine in the shared down projection's epilogue.
        launch_check(hipllm::launch_gemv_moe_combine(L.sh_down.type, L.sh_down.ptr, L.sh_down.row_bytes, act.sh_act,
                                                     hidden, act.down, act.rweight, act.rlog + E, K, next, H, FFs,
                                                     stream),
                     "shared down + MoE combine");
        return;
    }
    if (grp) {
        launch_check(hipllm::launch_gemv_norm(L.sh_down.type, L.sh_down.ptr, L.sh_down.row_bytes, act.sh_act, nullptr,
                                              0.0f, nullptr, nullptr, act.sh_down, H, FFs, 0, stream),
                     "shared down");
    } else {
        proj(L.sh_down, act.sh_act, act.sh_actq, FFs, rows, act.sh_down, H, nullptr, 0,
             sh_f16 ? act.xb : f16_rows(act.sh_act, FFs, FFs, rows));
    }
    if (next_norm) {
        launch_check(hipllm::launch_moe_combine_norm(hidden, act.down, act.rweight, act.sh_down, act.rlog + E, ldr,
                                                     next, next_gamma, act.norm, act.normq, rows, H, K,
                                                     config.norm_epsilon, stream),
                     "MoE combine + RMSNorm");
    } else {
        launch_check(hipllm::launch_moe_combine(hidden, act.down, act.rweight, act.sh_down, act.rlog + E, ldr, next,
                                                rows, H, K, stream),
                     "MoE combine");
    }
}

void HipMoeLLM::Impl::forward(std::size_t rows, std::size_t pos0, const std::int32_t* ids,
                              const std::uint32_t* dpos) {
    const float eps = config.norm_epsilon;
    float* h = act.hidden[0];
    float* tmp = act.hidden[1];
    in_norm = false;
    launch_check(hipllm::launch_embed(embedding.type, embedding.ptr, embedding.row_bytes, ids, rows,
                                      config.vocabulary_size, H, h, stream),
                 "embedding");
    // The MoE combine applies the next layer's input norm (the output norm
    // after the last layer) unless that layer's grouped launch normalises in
    // its prologue; the post-mixer norm runs after the output projection, or
    // inside the grouped router launch.
    if (!grouped_mixer(layers[0], rows)) {
        launch_check(hipllm::launch_rmsnorm(h, layers[0].attn_norm, act.norm, act.normq, rows, H, eps, stream),
                     "RMSNorm");
    }
    for (std::size_t l = 0; l < layers.size(); ++l) {
        const MoeLayer& L = layers[l];
        if (L.full) {
            attention_layer(l, rows, pos0, h, tmp, dpos);
        } else {
            deltanet_layer(l, rows, h, tmp);
        }
        const bool last = l + 1 == layers.size();
        moe_layer(l, rows, tmp, h, last ? output_norm : layers[l + 1].attn_norm,
                  last || !grouped_mixer(layers[l + 1], rows));
    }
    const float* last = act.norm + (rows - 1) * H;
    const hipllm::XGroup* lastq = act.normq + (rows - 1) * (H / 16);
    if (output.x16) {
        launch_check(hipllm::launch_gemv_x16(output.type, output.x16, lastq, nullptr, nullptr, act.logits,
                                             config.vocabulary_size, H, 0, stream),
                     "LM head");
    } else {
        launch_check(hipllm::launch_gemv_prepped(output.type, output.ptr, output.row_bytes, last, lastq, nullptr,
                                                 nullptr, act.logits, config.vocabulary_size, H, 0, stream),
                     "LM head");
    }
    launch_check(hipllm::launch_argmax(act.logits, config.vocabulary_size, act.token, act.argmax_scratch, stream),
                 "argmax");
    last_rows = rows;
}

// Records one decode step (token act.step[0] at position act.step[1]) as a
// graph: no allocation, copy or memset is recorded; the host writes act.step
// with an ordinary copy before each replay.
void HipMoeLLM::Impl::capture_decode() {
    hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
        forward(1, 0, reinterpret_cast<const std::int32_t*>(act.step), act.step + 1);
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

void HipMoeLLM::Impl::drop_decode_graph() {
    if (decode_exec) hipGraphExecDestroy(decode_exec);
    if (decode_graph) hipGraphDestroy(decode_graph);
    decode_exec = nullptr;
    decode_graph = nullptr;
}

std::int32_t HipMoeLLM::Impl::read_token() {
    hip_check(hipMemcpyAsync(host_token, act.token, 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(token)");
    hip_check(hipStreamSynchronize(stream), "HIP MoE forward");
    const std::uint32_t t = host_token[0];
    if (t > static_cast<std::uint32_t>(std::numeric_limits<std::int32_t>::max())) {
        throw std::overflow_error("generated token does not fit int32_t");
    }
    return static_cast<std::int32_t>(t);
}

HipMoeLLM::HipMoeLLM(const std::string& gguf_path, std::size_t max_sequence, const std::string& device,
                     std::size_t expert_cache_count)
    : impl_(std::make_unique<Impl>()) {
    impl_->load(gguf_path, max_sequence, parse_device_spec(device), expert_cache_count);
}

HipMoeLLM::~HipMoeLLM() = default;
HipMoeLLM::HipMoeLLM(HipMoeLLM&&) noexcept = default;
HipMoeLLM& HipMoeLLM::operator=(HipMoeLLM&&) noexcept = default;

void HipMoeLLM::reset() {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    hip_check(hipSetDevice(impl_->device), "hipSetDevice");
    impl_->zero_state();
    impl_->sequence_length = 0;
}

std::int32_t HipMoeLLM::prefill(const std::vector<std::int32_t>& ids) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    Impl& m = *impl_;
    if (ids.empty()) throw std::invalid_argument("MoE prefill requires at least one token");
    if (m.sequence_length != 0) throw std::invalid_argument("MoE prefill requires an empty state; call reset first");
    if (ids.size() > m.capacity) throw std::length_error("MoE prefill exceeds sequence capacity");
    for (std::int32_t id : ids) {
        if (id < 0 || static_cast<std::size_t>(id) >= m.config.vocabulary_size) {
            throw std::out_of_range("MoE prefill token is outside vocabulary");
        }
    }
    hip_check(hipSetDevice(m.device), "hipSetDevice");
    if (m.prof) m.prof->begin("prefill", ids.size(), "prefill.gpu_moe");
    m.ensure_rows(ids.size());
    std::memcpy(m.host_ids, ids.data(), ids.size() * 4);
    hip_check(hipMemcpyAsync(m.act.ids, m.host_ids, ids.size() * 4, hipMemcpyHostToDevice, m.stream),
              "hipMemcpy(ids)");
    m.forward(ids.size(), 0, m.act.ids);
    if (m.prof) m.prof->mark_gpu_end();
    const std::int32_t token = m.read_token();
    m.sequence_length = ids.size();
    m.expert_lookups += ids.size() * m.config.expert_used_count * m.layers.size();
    // The reference's MoE scopes carry no traffic estimate (moe_llm.mm:3083-3086).
    if (m.prof) m.prof->end(OpTraffic{});
    return token;
}

std::int32_t HipMoeLLM::decode(std::int32_t id) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    Impl& m = *impl_;
    if (m.sequence_length == 0) throw std::invalid_argument("MoE decode requires a completed prefill");
    if (m.sequence_length >= m.capacity) throw std::length_error("MoE decode exceeds sequence capacity");
    if (id < 0 || static_cast<std::size_t>(id) >= m.config.vocabulary_size) {
        throw std::out_of_range("MoE decode token is outside vocabulary");
    }
    hip_check(hipSetDevice(m.device), "hipSetDevice");
    const std::size_t pos = m.sequence_length;
    if (m.prof) m.prof->begin("decode", pos + 1, "decode.gpu_moe");
    m.host_step[0] = static_cast<std::uint32_t>(id);
    m.host_step[1] = static_cast<std::uint32_t>(pos);
    hip_check(hipMemcpyAsync(m.act.step, m.host_step, 8, hipMemcpyHostToDevice, m.stream), "hipMemcpy(step)");
    // Detailed profiling times every launch, so the step runs eagerly.
    const bool graph = m.decode_graphs && !(m.prof && m.prof->detailed());
    if (graph) {
        if (!m.decode_exec) m.capture_decode();
        hip_check(hipGraphLaunch(m.decode_exec, m.stream), "hipGraphLaunch(decode)");
        m.last_rows = 1;
    } else {
        m.forward(1, pos, reinterpret_cast<const std::int32_t*>(m.act.step));
    }
    if (m.prof) m.prof->mark_gpu_end();
    const std::int32_t token = m.read_token();
    m.sequence_length = pos + 1;
    m.expert_lookups += m.config.expert_used_count * m.layers.size();
    if (m.prof) m.prof->end(OpTraffic{}, graph ? &m.decode_graph_kernels : nullptr);
    return token;
}

void HipMoeLLM::set_decode_graphs(bool enabled) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    impl_->decode_graphs = enabled;
    if (!enabled) impl_->drop_decode_graph();
}

void HipMoeLLM::set_matmul_prefill(bool enabled) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    impl_->matmul_prefill = enabled;
}

void HipMoeLLM::set_route_probe(bool enabled) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    Impl& m = *impl_;
    hip_check(hipSetDevice(m.device), "hipSetDevice");
    hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    if (enabled && !m.probe) {
        hip_check(hipMalloc(reinterpret_cast<void**>(&m.probe), m.layers.size() * (m.E + 1) * 4),
                  "hipMalloc(route probe)");
    }
    m.drop_decode_graph();  // re-recorded with or without the probe copies
    m.probe_on = enabled;
}

void HipMoeLLM::copy_last_router_logits(float* dst, std::size_t count) const {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    const Impl& m = *impl_;
    if (!m.probe_on) throw std::invalid_argument("the route probe is off");
    if (count != m.layers.size() * (m.E + 1)) {
        throw std::invalid_argument("router logits buffer must hold layers x (experts + 1) floats");
    }
    if (m.last_rows == 0) throw std::invalid_argument("no forward has run");
    hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    hip_check(hipMemcpy(dst, m.probe, count * 4, hipMemcpyDeviceToHost), "hipMemcpy(route probe)");
}

void HipMoeLLM::enable_profiling(const std::string& csv_path, bool detailed_kernel_timestamps) {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    disable_profiling();
    hip_check(hipSetDevice(impl_->device), "hipSetDevice");
    impl_->prof = std::make_unique<RunProfiler>(csv_path, detailed_kernel_timestamps, impl_->stream);
}

void HipMoeLLM::disable_profiling() {
    if (impl_) impl_->prof.reset();
}

const GgufModelConfig& HipMoeLLM::config() const {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    return impl_->config;
}

std::size_t HipMoeLLM::position() const noexcept { return impl_ ? impl_->sequence_length : 0; }
std::size_t HipMoeLLM::max_sequence() const noexcept { return impl_ ? impl_->capacity : 0; }
bool HipMoeLLM::uses_gpu() const noexcept { return available(); }
bool HipMoeLLM::available() const noexcept { return impl_ && impl_->weights.base() && impl_->stream; }
std::size_t HipMoeLLM::expert_cache_count() const noexcept { return impl_ ? impl_->expert_cache : 0; }

HipExpertCacheStats HipMoeLLM::expert_cache_stats() const noexcept {
    HipExpertCacheStats s;
    if (impl_) s.hits = impl_->expert_lookups;
    return s;
}

const std::string& HipMoeLLM::device_name() const noexcept {
    static const std::string empty;
    return impl_ ? impl_->device_name : empty;
}

MemoryStats HipMoeLLM::memory_stats() const noexcept {
    if (!impl_) return {};
    MemoryStats s;
    s.weight_bytes = impl_->weight_bytes + impl_->x16_bytes;
    s.kv_cache_bytes = impl_->kv_cache_bytes;
    s.recurrent_state_bytes = impl_->recurrent_bytes;
    s.intermediate_bytes = impl_->act_bytes;
    s.intermediate_is_estimate = false;
    return s;
}

void HipMoeLLM::copy_last_logits(float* dst, std::size_t count) const {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    if (count != impl_->config.vocabulary_size) throw std::invalid_argument("logits buffer must hold the vocabulary");
    hip_check(hipStreamSynchronize(impl_->stream), "hipStreamSynchronize");
    hip_check(hipMemcpy(dst, impl_->act.logits, count * 4, hipMemcpyDeviceToHost), "hipMemcpy(logits)");
}

void HipMoeLLM::copy_last_routes(std::int32_t* dst, std::size_t count) const {
    if (!impl_) throw std::runtime_error("MoE model is not initialized");
    const Impl& m = *impl_;
    if (count != m.layers.size() * m.K) throw std::invalid_argument("routes buffer must hold layers x top-k ids");
    if (m.last_rows == 0) throw std::invalid_argument("no forward has run");
    hip_check(hipStreamSynchronize(m.stream), "hipStreamSynchronize");
    for (std::size_t l = 0; l < m.layers.size(); ++l) {
        hip_check(hipMemcpy(dst + l * m.K, m.route_ids + (l * m.act_rows + m.last_rows - 1) * m.K, m.K * 4,
                            hipMemcpyDeviceToHost),
                  "hipMemcpy(routes)");
    }
}

}  // namespace llm
