// Synthetic GGUF model writer (host only, no GPU).
//
// Emits the exact tensor schema the reference loaders accept for qwen2
// (model.cpp:861-919, metal_model.cpp:851-910: token_embd, output_norm,
// output and twelve tensors per block, nothing else) with GGUF v3 framing
// (magic, version, tensor/kv counts, metadata, tensor infos, data aligned to
// general.alignment = 32). Weights are N(0, stddev) values quantized per
// tensor role; norm gains are 1.0 F32; Q/K/V biases are N(0, bias_stddev) F32.
//
// Generation is deterministic for a given seed regardless of thread count:
// every value comes from a counter-based hash of (seed, tensor name, index).
#include "quants.h"
#include "synth_gguf.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <cmath>
#include <string>
#include <thread>
#include <vector>

namespace hipllm_tools {
namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;
constexpr uint32_t kKvU32 = 4;
constexpr uint32_t kKvF32 = 6;
constexpr uint32_t kKvString = 8;
constexpr size_t kAlignment = 32;

uint64_t fnv1a(const std::string& s) {
    uint64_t h = 1469598103934665603ULL;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ULL;
    }
    return h;
}

// Normal: N(0, stddev); Ones: 1.0; Bias: N(0, bias_stddev) (the second
// scale); Small: N(0, small_stddev); Conv: N(0, conv_stddev); NegDecay:
// -(0.25 + 0.5 |N(0, 1)|), a negative DeltaNet A per value head.
enum class Fill { Normal, Ones, Bias, Small, Conv, NegDecay };

struct Scales {
    float stddev = 0.02f;
    float bias = 0.02f;
    float small = 0.02f;
    float conv = 0.3f;
};

struct TensorPlan {
    std::string name;
    std::vector<uint64_t> dims;  // GGUF order: {cols, rows[, ...]}
    uint32_t type = kTypeF32;
    Fill fill = Fill::Normal;
    size_t rows = 0;
    size_t cols = 0;
    size_t bytes = 0;
    uint64_t offset = 0;
};

struct KvEntry {
    std::string key;
    uint32_t type = 0;
    uint32_t u32 = 0;
    float f32 = 0;
    std::string str;
};

class Writer {
public:
    explicit Writer(const std::string& path) : file_(std::fopen(path.c_str(), "wb")) {
        if (!file_) throw std::runtime_error("cannot create " + path);
    }
    ~Writer() {
        if (file_) std::fclose(file_);
    }
    void bytes(const void* data, size_t n) {
        if (n && std::fwrite(data, 1, n, file_) != n) throw std::runtime_error("short write");
        written_ += n;
    }
    void u32(uint32_t v) {
        uint8_t b[4] = {uint8_t(v), uint8_t(v >> 8), uint8_t(v >> 16), uint8_t(v >> 24)};
        bytes(b, 4);
    }
    void u64(uint64_t v) {
        uint8_t b[8];
        for (int i = 0; i < 8; ++i) b[i] = uint8_t(v >> (8 * i));
        bytes(b, 8);
    }
    void f32(float v) {
        uint32_t bits;
        std::memcpy(&bits, &v, 4);
        u32(bits);
    }
    void str(const std::string& s) {
        u64(s.size());
        bytes(s.data(), s.size());
    }
    void pad_to(size_t alignment) {
        static const uint8_t zeros[64] = {};
        while (written_ % alignment) bytes(zeros, std::min<size_t>(alignment - written_ % alignment, 64));
    }
    size_t written() const { return written_; }
    void close() {
        if (file_ && std::fclose(file_) != 0) {
            file_ = nullptr;
            throw std::runtime_error("close failed");
        }
        file_ = nullptr;
    }

private:
    FILE* file_;
    size_t written_ = 0;
};

void add_tensor(std::vector<TensorPlan>& plan, const std::string& name, size_t rows,
                size_t cols, uint32_t type, Fill fill, bool vector_shape, size_t experts = 0) {
    TensorPlan t;
    t.name = name;
    t.rows = experts ? rows * experts : rows;
    t.cols = cols;
    t.type = type;
    t.fill = fill;
    t.dims = vector_shape ? std::vector<uint64_t>{cols}
             : experts   ? std::vector<uint64_t>{cols, rows, experts}
                         : std::vector<uint64_t>{cols, rows};
    t.bytes = row_bytes(type, cols) * t.rows;
    if (t.bytes == 0) {
        throw std::runtime_error("tensor " + name + ": type " + std::to_string(type) +
                                 " cannot hold rows of " + std::to_string(cols));
    }
    plan.push_back(std::move(t));
}

void write_model(const std::string& path, const std::vector<KvEntry>& kvs,
                 std::vector<TensorPlan>& plan, uint64_t seed, const Scales& sc, unsigned threads) {
    uint64_t offset = 0;
    for (TensorPlan& t : plan) {
        offset = (offset + kAlignment - 1) / kAlignment * kAlignment;
        t.offset = offset;
        offset += t.bytes;
    }
    Writer w(path);
    w.u32(kGgufMagic);
    w.u32(3);
    w.u64(plan.size());
    w.u64(kvs.size());
    for (const KvEntry& kv : kvs) {
        w.str(kv.key);
        w.u32(kv.type);
        switch (kv.type) {
        case kKvU32: w.u32(kv.u32); break;
        case kKvF32: w.f32(kv.f32); break;
        case kKvString: w.str(kv.str); break;
        default: throw std::runtime_error("bad kv type");
        }
    }
    for (const TensorPlan& t : plan) {
        w.str(t.name);
        w.u32(static_cast<uint32_t>(t.dims.size()));
        for (uint64_t d : t.dims) w.u64(d);
        w.u32(t.type);
        w.u64(t.offset);
    }
    w.pad_to(kAlignment);
    const size_t data_start = w.written();

    if (threads == 0) threads = 1;
    std::vector<uint8_t> chunk;
    for (const TensorPlan& t : plan) {
        while (w.written() < data_start + t.offset) {
            const uint8_t zero = 0;
            w.bytes(&zero, 1);
        }
        const size_t rb = row_bytes(t.type, t.cols);
        const uint64_t stream = fnv1a(t.name);
        const size_t rows_per_chunk = std::max<size_t>(1, std::min<size_t>(t.rows, (64u << 20) / std::max<size_t>(rb, 1)));
        for (size_t r0 = 0; r0 < t.rows; r0 += rows_per_chunk) {
            const size_t nrows = std::min(rows_per_chunk, t.rows - r0);
            chunk.assign(nrows * rb, 0);
            auto work = [&](unsigned tid) {
                std::vector<float> row(t.cols);
                for (size_t r = tid; r < nrows; r += threads) {
                    const size_t global_row = r0 + r;
                    switch (t.fill) {
                    case Fill::Ones:
                        std::fill(row.begin(), row.end(), 1.0f);
                        break;
                    case Fill::Normal:
                        fill_normal(seed, stream, uint64_t(global_row) * t.cols, t.cols, sc.stddev, row.data());
                        break;
                    case Fill::Bias:
                        fill_normal(seed, stream, uint64_t(global_row) * t.cols, t.cols, sc.bias, row.data());
                        break;
                    case Fill::Small:
                        fill_normal(seed, stream, uint64_t(global_row) * t.cols, t.cols, sc.small, row.data());
                        break;
                    case Fill::Conv:
                        fill_normal(seed, stream, uint64_t(global_row) * t.cols, t.cols, sc.conv, row.data());
                        break;
                    case Fill::NegDecay:
                        fill_normal(seed, stream, uint64_t(global_row) * t.cols, t.cols, 1.0f, row.data());
                        for (float& v : row) v = -(0.25f + 0.5f * std::fabs(v));
                        break;
                    }
                    if (!quantize_row(t.type, row.data(), t.cols, chunk.data() + r * rb)) {
                        throw std::runtime_error("quantize failed for " + t.name);
                    }
                }
            };
            const unsigned used = static_cast<unsigned>(std::min<size_t>(threads, nrows));
            if (used <= 1) {
                work(0);
            } else {
                std::vector<std::thread> pool;
                std::vector<std::exception_ptr> errors(used);
                for (unsigned tid = 0; tid < used; ++tid) {
                    pool.emplace_back([&, tid] {
                        try {
                            work(tid);
                        } catch (...) {
                            errors[tid] = std::current_exception();
                        }
                    });
                }
                for (auto& th : pool) th.join();
                for (auto& e : errors) {
                    if (e) std::rethrow_exception(e);
                }
            }
            w.bytes(chunk.data(), chunk.size());
        }
    }
    w.close();
}

}  // namespace

void write_qwen2(const std::string& path, const Qwen2Spec& s) {
    if (s.layers == 0 || s.hidden == 0 || s.heads == 0 || s.kv_heads == 0 || s.ffn == 0 ||
        s.vocab == 0 || s.context == 0) {
        throw std::invalid_argument("qwen2 spec has a zero dimension");
    }
    if (s.hidden % s.heads != 0 || s.heads % s.kv_heads != 0) {
        throw std::invalid_argument("qwen2 head counts do not divide");
    }
    const size_t head = s.hidden / s.heads;
    const size_t kv = head * s.kv_heads;
    std::vector<KvEntry> kvs;
    auto kv_u32 = [&](const char* k, uint32_t v) { kvs.push_back({k, kKvU32, v, 0, {}}); };
    auto kv_f32 = [&](const char* k, float v) { kvs.push_back({k, kKvF32, 0, v, {}}); };
    kvs.push_back({"general.architecture", kKvString, 0, 0, "qwen2"});
    kv_u32("general.alignment", kAlignment);
    kv_u32("qwen2.block_count", s.layers);
    kv_u32("qwen2.embedding_length", s.hidden);
    kv_u32("qwen2.feed_forward_length", s.ffn);
    kv_u32("qwen2.attention.head_count", s.heads);
    kv_u32("qwen2.attention.head_count_kv", s.kv_heads);
    kv_u32("qwen2.context_length", s.context);
    kv_f32("qwen2.rope.freq_base", s.rope_theta);
    kv_f32("qwen2.attention.layer_norm_rms_epsilon", s.norm_eps);
    kv_u32("tokenizer.ggml.eos_token_id", s.eos_token_id);
    kv_u32("tokenizer.ggml.tokens_count", s.vocab);

    std::vector<TensorPlan> plan;
    add_tensor(plan, "token_embd.weight", s.vocab, s.hidden, s.type_embd, Fill::Normal, false);
    add_tensor(plan, "output_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
    add_tensor(plan, "output.weight", s.vocab, s.hidden, s.type_output, Fill::Normal, false);
    for (uint32_t i = 0; i < s.layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        add_tensor(plan, p + "attn_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
        add_tensor(plan, p + "attn_q.weight", s.hidden, s.hidden, s.type_attn_qkv, Fill::Normal, false);
        add_tensor(plan, p + "attn_q.bias", 1, s.hidden, kTypeF32, Fill::Bias, true);
        add_tensor(plan, p + "attn_k.weight", kv, s.hidden, s.type_attn_qkv, Fill::Normal, false);
        add_tensor(plan, p + "attn_k.bias", 1, kv, kTypeF32, Fill::Bias, true);
        add_tensor(plan, p + "attn_v.weight", kv, s.hidden, s.type_attn_qkv, Fill::Normal, false);
        add_tensor(plan, p + "attn_v.bias", 1, kv, kTypeF32, Fill::Bias, true);
        add_tensor(plan, p + "attn_output.weight", s.hidden, s.hidden, s.type_attn_out, Fill::Normal, false);
        add_tensor(plan, p + "ffn_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
        add_tensor(plan, p + "ffn_gate.weight", s.ffn, s.hidden, s.type_ffn_gate_up, Fill::Normal, false);
        add_tensor(plan, p + "ffn_up.weight", s.ffn, s.hidden, s.type_ffn_gate_up, Fill::Normal, false);
        add_tensor(plan, p + "ffn_down.weight", s.hidden, s.ffn, s.type_ffn_down, Fill::Normal, false);
    }
    Scales sc;
    sc.stddev = s.stddev;
    sc.bias = s.bias_stddev;
    write_model(path, kvs, plan, s.seed, sc, s.threads);
}

void write_qwen35moe(const std::string& path, const Qwen35MoeSpec& s) {
    if (s.layers == 0 || s.hidden == 0 || s.heads == 0 || s.kv_heads == 0 || s.head_dim == 0 || s.vocab == 0 ||
        s.context == 0 || s.experts == 0 || s.experts_used == 0 || s.experts_used > s.experts ||
        s.expert_ffn == 0 || s.shared_ffn == 0 || s.full_attention_interval == 0 || s.conv_kernel == 0 ||
        s.state_size == 0 || s.group_count == 0 || s.time_step_rank == 0) {
        throw std::invalid_argument("qwen35moe spec has a zero or inconsistent dimension");
    }
    if (s.heads % s.kv_heads != 0 || s.time_step_rank % s.group_count != 0 || s.rotary_dim > s.head_dim ||
        s.rotary_dim % 2 != 0) {
        throw std::invalid_argument("qwen35moe head counts do not divide");
    }
    const uint32_t inner = s.time_step_rank * s.state_size;
    const uint32_t qkv_w = 2 * s.group_count * s.state_size + inner;
    const uint32_t q_w = s.heads * s.head_dim;
    const uint32_t kv_w = s.kv_heads * s.head_dim;
    std::vector<KvEntry> kvs;
    auto kv_u32 = [&](const std::string& k, uint32_t v) { kvs.push_back({k, kKvU32, v, 0, {}}); };
    auto kv_f32 = [&](const std::string& k, float v) { kvs.push_back({k, kKvF32, 0, v, {}}); };
    const std::string a = "qwen35moe.";
    kvs.push_back({"general.architecture", kKvString, 0, 0, "qwen35moe"});
    kv_u32("general.alignment", kAlignment);
    kv_u32(a + "block_count", s.layers);
    kv_u32(a + "nextn_predict_layers", 0);
    kv_u32(a + "embedding_length", s.hidden);
    kv_u32(a + "attention.head_count", s.heads);
    kv_u32(a + "attention.head_count_kv", s.kv_heads);
    kv_u32(a + "attention.key_length", s.head_dim);
    kv_u32(a + "attention.value_length", s.head_dim);
    kv_u32(a + "context_length", s.context);
    kv_u32(a + "expert_count", s.experts);
    kv_u32(a + "expert_used_count", s.experts_used);
    kv_u32(a + "expert_feed_forward_length", s.expert_ffn);
    kv_u32(a + "expert_shared_feed_forward_length", s.shared_ffn);
    kv_u32(a + "full_attention_interval", s.full_attention_interval);
    kv_u32(a + "ssm.conv_kernel", s.conv_kernel);
    kv_u32(a + "ssm.state_size", s.state_size);
    kv_u32(a + "ssm.group_count", s.group_count);
    kv_u32(a + "ssm.time_step_rank", s.time_step_rank);
    kv_u32(a + "ssm.inner_size", inner);
    kv_u32(a + "rope.dimension_count", s.rotary_dim);
    kv_f32(a + "rope.freq_base", s.rope_theta);
    kv_f32(a + "attention.layer_norm_rms_epsilon", s.norm_eps);
    kv_u32("tokenizer.ggml.eos_token_id", s.eos_token_id);
    kv_u32("tokenizer.ggml.tokens_count", s.vocab);

    std::vector<TensorPlan> plan;
    add_tensor(plan, "token_embd.weight", s.vocab, s.hidden, s.type_embd, Fill::Normal, false);
    add_tensor(plan, "output_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
    add_tensor(plan, "output.weight", s.vocab, s.hidden, s.type_output, Fill::Normal, false);
    for (uint32_t i = 0; i < s.layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        add_tensor(plan, p + "attn_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
        add_tensor(plan, p + "post_attention_norm.weight", 1, s.hidden, kTypeF32, Fill::Ones, true);
        if ((i + 1) % s.full_attention_interval == 0) {
            add_tensor(plan, p + "attn_q.weight", 2 * q_w, s.hidden, s.type_attn_qgate, Fill::Normal, false);
            add_tensor(plan, p + "attn_k.weight", kv_w, s.hidden, s.type_attn_kv, Fill::Normal, false);
            add_tensor(plan, p + "attn_v.weight", kv_w, s.hidden, s.type_attn_kv, Fill::Normal, false);
            add_tensor(plan, p + "attn_q_norm.weight", 1, s.head_dim, kTypeF32, Fill::Ones, true);
            add_tensor(plan, p + "attn_k_norm.weight", 1, s.head_dim, kTypeF32, Fill::Ones, true);
            add_tensor(plan, p + "attn_output.weight", s.hidden, q_w, s.type_attn_out, Fill::Normal, false);
        } else {
            add_tensor(plan, p + "attn_qkv.weight", qkv_w, s.hidden, s.type_ssm_qkv, Fill::Normal, false);
            add_tensor(plan, p + "attn_gate.weight", inner, s.hidden, s.type_ssm_gate, Fill::Normal, false);
            add_tensor(plan, p + "ssm_alpha.weight", s.time_step_rank, s.hidden, kTypeF32, Fill::Small, false);
            add_tensor(plan, p + "ssm_beta.weight", s.time_step_rank, s.hidden, kTypeF32, Fill::Small, false);
            add_tensor(plan, p + "ssm_conv1d.weight", qkv_w, s.conv_kernel, kTypeF32, Fill::Conv, false);
            add_tensor(plan, p + "ssm_dt.bias", 1, s.time_step_rank, kTypeF32, Fill::Small, true);
            add_tensor(plan, p + "ssm_a", 1, s.time_step_rank, kTypeF32, Fill::NegDecay, true);
            add_tensor(plan, p + "ssm_norm.weight", 1, s.state_size, kTypeF32, Fill::Ones, true);
            add_tensor(plan, p + "ssm_out.weight", s.hidden, inner, s.type_ssm_out, Fill::Normal, false);
        }
        add_tensor(plan, p + "ffn_gate_inp.weight", s.experts, s.hidden, kTypeF32, Fill::Small, false);
        add_tensor(plan, p + "ffn_gate_exps.weight", s.expert_ffn, s.hidden, s.type_expert_gate_up, Fill::Normal,
                   false, s.experts);
        add_tensor(plan, p + "ffn_up_exps.weight", s.expert_ffn, s.hidden, s.type_expert_gate_up, Fill::Normal,
                   false, s.experts);
        add_tensor(plan, p + "ffn_down_exps.weight", s.hidden, s.expert_ffn, s.type_expert_down, Fill::Normal, false,
                   s.experts);
        add_tensor(plan, p + "ffn_gate_inp_shexp.weight", 1, s.hidden, kTypeF32, Fill::Small, true);
        add_tensor(plan, p + "ffn_gate_shexp.weight", s.shared_ffn, s.hidden, s.type_shared, Fill::Normal, false);
        add_tensor(plan, p + "ffn_up_shexp.weight", s.shared_ffn, s.hidden, s.type_shared, Fill::Normal, false);
        add_tensor(plan, p + "ffn_down_shexp.weight", s.hidden, s.shared_ffn, s.type_shared, Fill::Normal, false);
    }
    Scales sc;
    sc.stddev = s.stddev;
    sc.small = s.small_stddev;
    sc.conv = s.conv_stddev;
    write_model(path, kvs, plan, s.seed, sc, s.threads);
}

}  // namespace hipllm_tools
