// CPU oracle: restatement of the reference CPULLM path (see oracle.h for the
// file:line map). Test infrastructure only; never linked into the product.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

enum : uint32_t { kF32 = 0, kF16 = 1, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14 };

// ---------------------------------------------------------------- GGUF file
// model.cpp:49-140 (byte reader), 161-296 (metadata), 376-489 (file).
class Reader {
public:
    explicit Reader(const std::vector<uint8_t>& b) : b_(b) {}
    size_t pos() const { return p_; }
    uint8_t u8() { need(1); return b_[p_++]; }
    uint16_t u16() { need(2); uint16_t v = uint16_t(b_[p_] | (b_[p_ + 1] << 8)); p_ += 2; return v; }
    uint32_t u32() {
        need(4);
        uint32_t v = uint32_t(b_[p_]) | (uint32_t(b_[p_ + 1]) << 8) | (uint32_t(b_[p_ + 2]) << 16) |
                     (uint32_t(b_[p_ + 3]) << 24);
        p_ += 4;
        return v;
    }
    uint64_t u64() {
        need(8);
        uint64_t v = 0;
        for (int i = 0; i < 8; ++i) v |= uint64_t(b_[p_ + i]) << (8 * i);
        p_ += 8;
        return v;
    }
    float f32() { uint32_t u = u32(); float f; std::memcpy(&f, &u, 4); return f; }
    double f64() { uint64_t u = u64(); double d; std::memcpy(&d, &u, 8); return d; }
    std::string str() {
        uint64_t n = u64();
        if (n > b_.size() - p_) throw std::runtime_error("invalid GGUF string length");
        std::string s(reinterpret_cast<const char*>(b_.data() + p_), size_t(n));
        p_ += size_t(n);
        return s;
    }
    void skip(size_t n) { need(n); p_ += n; }

private:
    void need(size_t n) const {
        if (p_ > b_.size() || n > b_.size() - p_) throw std::runtime_error("truncated GGUF file");
    }
    const std::vector<uint8_t>& b_;
    size_t p_ = 0;
};

struct Metadata {
    std::unordered_map<std::string, uint64_t> ints;
    std::unordered_map<std::string, double> reals;
    std::unordered_map<std::string, std::string> texts;
    size_t vocabulary_entries = 0;
};

void skip_value(Reader& r, uint32_t type) {
    switch (type) {
    case 0: case 1: case 7: r.skip(1); break;
    case 2: case 3: r.skip(2); break;
    case 4: case 5: case 6: r.skip(4); break;
    case 10: case 11: case 12: r.skip(8); break;
    case 8: r.skip(size_t(r.u64())); break;
    case 9: {
        uint32_t et = r.u32();
        uint64_t n = r.u64();
        for (uint64_t i = 0; i < n; ++i) skip_value(r, et);
        break;
    }
    default: throw std::runtime_error("unsupported GGUF array element type " + std::to_string(type));
    }
}

void read_value(Reader& r, uint32_t type, const std::string& key, Metadata& m) {
    switch (type) {
    case 0: m.ints[key] = r.u8(); break;
    case 1: m.ints[key] = uint64_t(int8_t(r.u8())); break;
    case 2: m.ints[key] = r.u16(); break;
    case 3: m.ints[key] = uint64_t(int16_t(r.u16())); break;
    case 4: m.ints[key] = r.u32(); break;
    case 5: m.ints[key] = uint64_t(int32_t(r.u32())); break;
    case 6: m.reals[key] = r.f32(); break;
    case 7: m.ints[key] = r.u8() != 0 ? 1 : 0; break;
    case 8: m.texts[key] = r.str(); break;
    case 9: {
        uint32_t et = r.u32();
        uint64_t n = r.u64();
        if (key == "tokenizer.ggml.tokens" && et == 8) {
            m.vocabulary_entries = size_t(n);
            for (uint64_t i = 0; i < n; ++i) r.str();
        } else {
            for (uint64_t i = 0; i < n; ++i) skip_value(r, et);
        }
        break;
    }
    case 10: m.ints[key] = r.u64(); break;
    case 11: m.ints[key] = r.u64(); break;
    case 12: m.reals[key] = r.f64(); break;
    default: throw std::runtime_error("unsupported GGUF metadata type " + std::to_string(type));
    }
}

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t rel = 0;
    size_t offset = 0;
    size_t cols() const { return dims.empty() ? 1 : size_t(dims[0]); }
    size_t rows() const {
        size_t n = 1;
        for (size_t i = 1; i < dims.size(); ++i) n *= size_t(dims[i]);
        return n;
    }
};

size_t block_row_bytes(size_t cols, size_t block, size_t bytes, const char* name) {
    if (cols % block != 0) throw std::runtime_error(std::string(name) + " row is not block aligned");
    return cols / block * bytes;
}

size_t row_bytes(uint32_t type, size_t cols) {
    switch (type) {
    case kF32: return cols * 4;
    case kF16: return cols * 2;
    case kQ5_0: return block_row_bytes(cols, 32, 22, "Q5_0");
    case kQ8_0: return block_row_bytes(cols, 32, 34, "Q8_0");
    case kQ4_K: return block_row_bytes(cols, 256, 144, "Q4_K");
    case kQ6_K: return block_row_bytes(cols, 256, 210, "Q6_K");
    default: throw std::runtime_error("unsupported GGUF tensor type " + std::to_string(type));
    }
}

struct GgufFile {
    std::vector<uint8_t> bytes;
    Metadata meta;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> index;

    explicit GgufFile(const std::string& path) {
        std::ifstream in(path, std::ios::binary | std::ios::ate);
        if (!in) throw std::runtime_error("cannot open model: " + path);
        std::streamsize size = in.tellg();
        if (size <= 0) throw std::runtime_error("empty model file");
        in.seekg(0);
        bytes.resize(size_t(size));
        if (!in.read(reinterpret_cast<char*>(bytes.data()), size)) throw std::runtime_error("cannot read model: " + path);
        Reader r(bytes);
        if (r.u32() != 0x46554747u) throw std::runtime_error("not a GGUF file");
        uint32_t version = r.u32();
        if (version != 2 && version != 3) throw std::runtime_error("unsupported GGUF version");
        uint64_t tcount = r.u64();
        uint64_t kcount = r.u64();
        for (uint64_t i = 0; i < kcount; ++i) {
            std::string key = r.str();
            read_value(r, r.u32(), key, meta);
        }
        for (uint64_t i = 0; i < tcount; ++i) {
            TensorInfo t;
            t.name = r.str();
            uint32_t nd = r.u32();
            for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(r.u64());
            t.type = r.u32();
            t.rel = r.u64();
            tensors.push_back(t);
        }
        auto it = meta.ints.find("general.alignment");
        size_t align = it == meta.ints.end() ? 32 : size_t(it->second);
        if (align == 0 || (align & (align - 1))) throw std::runtime_error("invalid GGUF alignment");
        size_t start = (r.pos() + align - 1) & ~(align - 1);
        if (start > bytes.size()) throw std::runtime_error("GGUF tensor data starts past end of file");
        for (size_t i = 0; i < tensors.size(); ++i) {
            if (tensors[i].rel > bytes.size() - start) throw std::runtime_error("GGUF tensor offset is outside file");
            tensors[i].offset = start + size_t(tensors[i].rel);
            if (!index.emplace(tensors[i].name, i).second) throw std::runtime_error("duplicate GGUF tensor: " + tensors[i].name);
        }
    }

    const TensorInfo& require(const std::string& name) const {
        auto it = index.find(name);
        if (it == index.end()) throw std::runtime_error("missing tensor: " + name);
        return tensors[it->second];
    }

    const uint8_t* row_ptr(const TensorInfo& t, size_t row) const {
        size_t rb = row_bytes(t.type, t.cols());
        if (row >= t.rows()) throw std::runtime_error("tensor row is outside file: " + t.name);
        size_t off = t.offset + row * rb;
        if (off > bytes.size() || rb > bytes.size() - off) throw std::runtime_error("tensor row is outside file: " + t.name);
        return bytes.data() + off;
    }
};

// ------------------------------------------------------------- dequantizer
// model.cpp:500-683.
uint16_t load_u16(const uint8_t* d) { return uint16_t(d[0] | (d[1] << 8)); }

float half_to_float(uint16_t value) {
    const uint32_t sign = value >> 15;
    const uint32_t exponent = (value >> 10) & 0x1f;
    const uint32_t mantissa = value & 0x3ff;
    if (exponent == 0) {
        if (mantissa == 0) return sign ? -0.0f : 0.0f;
        const float result = std::ldexp(static_cast<float>(mantissa) / 1024.0f, -14);
        return sign ? -result : result;
    }
    if (exponent == 31) {
        if (mantissa == 0) return sign ? -INFINITY : INFINITY;
        return std::numeric_limits<float>::quiet_NaN();
    }
    const float result = std::ldexp(1.0f + static_cast<float>(mantissa) / 1024.0f,
                                    static_cast<int>(exponent) - 15);
    return sign ? -result : result;
}

void scale_min_k4(int j, const uint8_t* s, uint8_t& sc, uint8_t& m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = uint8_t((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        m = uint8_t((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

void dequant_row(uint32_t type, const uint8_t* data, size_t cols, float* out) {
    switch (type) {
    case kF32:
        for (size_t i = 0; i < cols; ++i) {
            uint32_t bits = uint32_t(data[4 * i]) | (uint32_t(data[4 * i + 1]) << 8) |
                            (uint32_t(data[4 * i + 2]) << 16) | (uint32_t(data[4 * i + 3]) << 24);
            std::memcpy(out + i, &bits, 4);
        }
        return;
    case kF16:
        for (size_t i = 0; i < cols; ++i) out[i] = half_to_float(load_u16(data + 2 * i));
        return;
    case kQ5_0:
        for (size_t b = 0; b < cols / 32; ++b) {
            const uint8_t* c = data + b * 22;
            const float d = half_to_float(load_u16(c));
            const uint32_t h = uint32_t(c[2]) | (uint32_t(c[3]) << 8) | (uint32_t(c[4]) << 16) | (uint32_t(c[5]) << 24);
            const uint8_t* q = c + 6;
            for (int j = 0; j < 16; ++j) {
                const int h0 = int(((h >> j) << 4) & 0x10);
                const int h1 = int((h >> (j + 12)) & 0x10);
                out[b * 32 + j] = (int(q[j] & 0x0f) | h0) * d - 16.0f * d;
                out[b * 32 + j + 16] = (int(q[j] >> 4) | h1) * d - 16.0f * d;
            }
        }
        return;
    case kQ8_0:
        for (size_t b = 0; b < cols / 32; ++b) {
            const uint8_t* c = data + b * 34;
            const float d = half_to_float(load_u16(c));
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = float(int8_t(c[2 + j])) * d;
        }
        return;
    case kQ4_K:
        for (size_t b = 0; b < cols / 256; ++b) {
            const uint8_t* c = data + b * 144;
            const float d = half_to_float(load_u16(c));
            const float dmin = half_to_float(load_u16(c + 2));
            const uint8_t* s = c + 4;
            const uint8_t* qs = c + 16;
            size_t o = b * 256;
            int is = 0;
            for (int j = 0; j < 256; j += 64) {
                uint8_t sc, m;
                scale_min_k4(is++, s, sc, m);
                const float d1 = d * sc;
                const float m1 = dmin * m;
                scale_min_k4(is++, s, sc, m);
                const float d2 = d * sc;
                const float m2 = dmin * m;
                const uint8_t* q = qs + j / 2;
                for (int l = 0; l < 32; ++l) {
                    out[o + l] = d1 * (q[l] & 0x0f) - m1;
                    out[o + 32 + l] = d2 * (q[l] >> 4) - m2;
                }
                o += 64;
            }
        }
        return;
    case kQ6_K:
        for (size_t b = 0; b < cols / 256; ++b) {
            const uint8_t* c = data + b * 210;
            const uint8_t* ql = c;
            const uint8_t* qh = c + 128;
            const int8_t* sc = reinterpret_cast<const int8_t*>(c + 192);
            const float d = half_to_float(load_u16(c + 208));
            size_t o = b * 256;
            int so = 0;
            for (int n = 0; n < 256; n += 128) {
                for (int l = 0; l < 32; ++l) {
                    const int q1 = int((ql[l] & 0x0f) | ((qh[l] & 0x03) << 4)) - 32;
                    const int q2 = int((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 0x03) << 4)) - 32;
                    const int q3 = int((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32;
                    const int q4 = int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32;
                    const int si = l / 16;
                    out[o + n + l] = d * sc[so + si + 0] * q1;
                    out[o + n + l + 32] = d * sc[so + si + 2] * q2;
                    out[o + n + l + 64] = d * sc[so + si + 4] * q3;
                    out[o + n + l + 96] = d * sc[so + si + 6] * q4;
                }
                ql += 64;
                qh += 32;
                so += 8;
            }
        }
        return;
    default:
        throw std::runtime_error("unsupported tensor type in dequantizer");
    }
}

// --------------------------------------------------------------- operators
// cpu_llm.cpp:143-235 and 453-665, on contiguous row-major storage.
void rmsnorm(float* x, const float* g, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += double(x[i]) * double(x[i]);
    const float ms = float(ss / double(n));
    const float inv = 1.0f / std::sqrt(ms + eps);
    for (size_t i = 0; i < n; ++i) x[i] *= inv * g[i];
}

void softmax(float* x, size_t n) {
    const float mx = *std::max_element(x, x + n);
    double den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        x[i] = std::exp(x[i] - mx);
        den += double(x[i]);
    }
    if (!std::isfinite(den) || den == 0.0) throw std::runtime_error("Softmax normalization is not finite");
    for (size_t i = 0; i < n; ++i) x[i] = float(double(x[i]) / den);
}

void swiglu(float* g, const float* u, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float gate = g[i];
        const float sig = gate >= 0.0f ? 1.0f / (1.0f + std::exp(-gate))
                                       : std::exp(gate) / (1.0f + std::exp(gate));
        g[i] = gate * sig * u[i];
    }
}

void rope(float* x, size_t len, size_t position, float theta, size_t rot) {
    if (rot == 0) rot = len;
    const size_t half = rot / 2;
    for (size_t p = 0; p < half; ++p) {
        const float freq = std::pow(theta, -2.0f * static_cast<float>(p) / static_cast<float>(rot));
        const float angle = static_cast<float>(position) * freq;
        const float c = std::cos(angle);
        const float s = std::sin(angle);
        const float a = x[p];
        const float b = x[p + half];
        x[p] = a * c - b * s;
        x[p + half] = a * s + b * c;
    }
}

// y[r] = sum_c x[c] * W[r][c] (+ bias[r] after the sum), cpu_llm.cpp:512-547.
void gevmt(const float* w, const float* x, const float* bias, size_t rows, size_t cols, float* y) {
    for (size_t r = 0; r < rows; ++r) {
        float acc = 0.0f;
        const float* wr = w + r * cols;
        for (size_t c = 0; c < cols; ++c) acc += x[c] * wr[c];
        if (bias) acc += bias[r];
        y[r] = acc;
    }
}

int32_t greedy(const float* x, size_t n) {
    return int32_t(std::max_element(x, x + n) - x);
}

struct Layer {
    std::vector<float> attn_norm, wq, bq, wk, bk, wv, bv, wo, ffn_norm, wg, wd, wu;
};

struct Status {
    int code;
    std::string message;
};

}  // namespace

struct OracleModel {
    OracleConfig cfg{};
    std::vector<float> embedding, output_norm, output;
    std::vector<Layer> layers;
    std::vector<std::vector<float>> kcache, vcache;  // [rows, kv_dim] per layer
    size_t max_sequence = 0;
    size_t sequence = 0;
    std::unordered_map<std::string, std::pair<std::vector<float>*, std::pair<size_t, size_t>>> named;
};

namespace {

size_t meta_size(const Metadata& m, const char* key) {
    auto it = m.ints.find(key);
    if (it == m.ints.end()) throw std::runtime_error(std::string("missing GGUF metadata: ") + key);
    if (it->second == 0) throw std::runtime_error(std::string("invalid GGUF metadata: ") + key);
    return size_t(it->second);
}

void load_model(OracleModel& M, const std::string& path, size_t max_sequence) {
    GgufFile f(path);
    auto arch = f.meta.texts.find("general.architecture");
    std::string a = arch == f.meta.texts.end() ? "" : arch->second;
    if (a != "qwen2") throw std::runtime_error("ModelFile currently supports qwen2 GGUF models, got " + a);
    OracleConfig& c = M.cfg;
    c.layer_count = meta_size(f.meta, "qwen2.block_count");
    c.embedding_size = meta_size(f.meta, "qwen2.embedding_length");
    c.feed_forward_size = meta_size(f.meta, "qwen2.feed_forward_length");
    c.attention_head_count = meta_size(f.meta, "qwen2.attention.head_count");
    c.kv_head_count = meta_size(f.meta, "qwen2.attention.head_count_kv");
    c.context_length = meta_size(f.meta, "qwen2.context_length");
    c.vocabulary_size = f.meta.vocabulary_entries;
    if (c.vocabulary_size == 0) c.vocabulary_size = meta_size(f.meta, "tokenizer.ggml.tokens_count");
    if (c.embedding_size % c.attention_head_count) throw std::runtime_error("embedding size must be divisible by attention head count");
    if (c.attention_head_count % c.kv_head_count) throw std::runtime_error("attention head count must be divisible by KV head count");
    c.head_size = c.embedding_size / c.attention_head_count;
    c.rotary_dimension = c.head_size;
    auto real = [&](const char* k, double fb) {
        auto it = f.meta.reals.find(k);
        return it == f.meta.reals.end() ? fb : it->second;
    };
    c.rope_theta = float(real("qwen2.rope.freq_base", 1000000.0));
    c.norm_epsilon = float(real("qwen2.attention.layer_norm_rms_epsilon", 1e-6));
    if (!std::isfinite(c.rope_theta) || c.rope_theta <= 0.0f) throw std::runtime_error("RoPE theta must be finite and positive");
    if (!std::isfinite(c.norm_epsilon) || c.norm_epsilon <= 0.0f) throw std::runtime_error("RMSNorm epsilon must be finite and positive");
    auto eos = f.meta.ints.find("tokenizer.ggml.eos_token_id");
    uint64_t e = eos == f.meta.ints.end() ? 151645 : eos->second;
    if (e > uint64_t(std::numeric_limits<int32_t>::max())) throw std::runtime_error("EOS token id does not fit in int32_t");
    c.eos_token_id = int32_t(e);
    for (const TensorInfo& t : f.tensors) c.parameter_count += t.rows() * t.cols();

    if (max_sequence == 0) max_sequence = c.context_length;
    if (max_sequence > c.context_length) throw std::invalid_argument("CPU maximum sequence must be within the model context length");

    std::unordered_set<std::string> loaded;
    auto matrix = [&](const std::string& name, size_t rows, size_t cols, std::vector<float>& dst) {
        const TensorInfo& t = f.require(name);
        if (t.rows() != rows || t.cols() != cols) {
            throw std::runtime_error("unexpected shape for tensor " + name + ": expected " + std::to_string(rows) + "x" +
                                     std::to_string(cols) + ", got " + std::to_string(t.rows()) + "x" + std::to_string(t.cols()));
        }
        dst.assign(rows * cols, 0.0f);
        for (size_t r = 0; r < rows; ++r) dequant_row(t.type, f.row_ptr(t, r), cols, dst.data() + r * cols);
        if (!loaded.insert(name).second) throw std::runtime_error("tensor loaded more than once: " + name);
        M.named[name] = {&dst, {rows, cols}};
    };
    const size_t H = c.embedding_size, F = c.feed_forward_size, V = c.vocabulary_size;
    const size_t KV = c.kv_head_count * c.head_size;
    matrix("token_embd.weight", V, H, M.embedding);
    matrix("output_norm.weight", 1, H, M.output_norm);
    matrix("output.weight", V, H, M.output);
    M.layers.resize(c.layer_count);
    for (size_t i = 0; i < c.layer_count; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        Layer& L = M.layers[i];
        matrix(p + "attn_norm.weight", 1, H, L.attn_norm);
        matrix(p + "attn_q.weight", H, H, L.wq);
        matrix(p + "attn_q.bias", 1, H, L.bq);
        matrix(p + "attn_k.weight", KV, H, L.wk);
        matrix(p + "attn_k.bias", 1, KV, L.bk);
        matrix(p + "attn_v.weight", KV, H, L.wv);
        matrix(p + "attn_v.bias", 1, KV, L.bv);
        matrix(p + "attn_output.weight", H, H, L.wo);
        matrix(p + "ffn_norm.weight", 1, H, L.ffn_norm);
        matrix(p + "ffn_gate.weight", F, H, L.wg);
        matrix(p + "ffn_down.weight", H, F, L.wd);
        matrix(p + "ffn_up.weight", F, H, L.wu);
    }
    if (loaded.size() != f.tensors.size()) {
        std::string msg = "GGUF contains tensors not mapped by ModelFile:";
        for (const TensorInfo& t : f.tensors) {
            if (!loaded.count(t.name)) msg += " " + t.name;
        }
        throw std::runtime_error(msg);
    }
    M.max_sequence = max_sequence;
    M.kcache.assign(c.layer_count, {});
    M.vcache.assign(c.layer_count, {});
}

// cpu_prefill_layer, cpu_llm.cpp:774-841. hidden is [N, H] row-major.
void prefill_layer(OracleModel& M, size_t li, std::vector<float>& hidden, size_t N) {
    const OracleConfig& c = M.cfg;
    const Layer& L = M.layers[li];
    const size_t H = c.embedding_size, D = c.head_size, Hq = c.attention_head_count, Hkv = c.kv_head_count;
    const size_t KV = Hkv * D, F = c.feed_forward_size, group = Hq / Hkv;

    std::vector<float> A = hidden;
    for (size_t r = 0; r < N; ++r) rmsnorm(&A[r * H], L.attn_norm.data(), H, c.norm_epsilon);

    // gemmtb: C[row][col] = sum_step A[row][step] * W[col][step], then + bias.
    auto gemmtb = [&](const std::vector<float>& in, size_t K, const std::vector<float>& W,
                      const float* bias, size_t Nout) {
        std::vector<float> out(N * Nout, 0.0f);
        for (size_t r = 0; r < N; ++r) {
            for (size_t col = 0; col < Nout; ++col) {
                float acc = 0.0f;
                const float* a = &in[r * K];
                const float* w = &W[col * K];
                for (size_t s = 0; s < K; ++s) acc += a[s] * w[s];
                if (bias) acc += bias[col];
                out[r * Nout + col] = acc;
            }
        }
        return out;
    };
    std::vector<float> Q = gemmtb(A, H, L.wq, L.bq.data(), H);
    std::vector<float> K = gemmtb(A, H, L.wk, L.bk.data(), KV);
    std::vector<float> Vv = gemmtb(A, H, L.wv, L.bv.data(), KV);
    for (size_t r = 0; r < N; ++r) {
        for (size_t h = 0; h < Hq; ++h) rope(&Q[r * H + h * D], D, r, c.rope_theta, c.rotary_dimension);
        for (size_t h = 0; h < Hkv; ++h) rope(&K[r * KV + h * D], D, r, c.rope_theta, c.rotary_dimension);
    }
    M.kcache[li] = K;
    M.vcache[li] = Vv;

    std::vector<float> C(N * H, 0.0f);
    std::vector<float> S(N * N);
    const float sq = std::sqrt(static_cast<float>(D));
    for (size_t h = 0; h < Hq; ++h) {
        const size_t g = h / group;
        // gemmts: scores = (q . k) / sqrt(D), cpu_llm.cpp:609-629.
        for (size_t i = 0; i < N; ++i) {
            for (size_t j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (size_t d = 0; d < D; ++d) acc += Q[i * H + h * D + d] * K[j * KV + g * D + d];
                acc /= sq;
                S[i * N + j] = acc;
            }
        }
        // causal_mask, cpu_llm.cpp:316-329.
        for (size_t i = 0; i < N; ++i) {
            for (size_t j = i + 1; j < N; ++j) S[i * N + j] = -std::numeric_limits<float>::infinity();
        }
        for (size_t i = 0; i < N; ++i) softmax(&S[i * N], N);
        // gemm: out[i][d] = sum_j S[i][j] * V[j][d], cpu_llm.cpp:549-565.
        for (size_t i = 0; i < N; ++i) {
            for (size_t d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (size_t j = 0; j < N; ++j) acc += S[i * N + j] * Vv[j * KV + g * D + d];
                C[i * H + h * D + d] = acc;
            }
        }
    }
    std::vector<float> O = gemmtb(C, H, L.wo, nullptr, H);
    std::vector<float> X(N * H);
    for (size_t i = 0; i < N * H; ++i) X[i] = hidden[i] + O[i];

    std::vector<float> Fn = X;
    for (size_t r = 0; r < N; ++r) rmsnorm(&Fn[r * H], L.ffn_norm.data(), H, c.norm_epsilon);
    std::vector<float> G = gemmtb(Fn, H, L.wg, nullptr, F);
    std::vector<float> U = gemmtb(Fn, H, L.wu, nullptr, F);
    for (size_t r = 0; r < N; ++r) swiglu(&G[r * F], &U[r * F], F);
    std::vector<float> Dn = gemmtb(G, F, L.wd, nullptr, H);
    for (size_t i = 0; i < N * H; ++i) hidden[i] = X[i] + Dn[i];
}

// cpu_decode_layer, cpu_llm.cpp:843-914.
// The decode FFN of cpu_decode_layer (cpu_llm.cpp:907-913): gate and up
// products of the normalised row, SwiGLU, down product.
void ffn_swiglu(const float* wg, const float* wu, const float* wd, const float* x, size_t H, size_t F, float* out) {
    std::vector<float> G(F), U(F);
    gevmt(wg, x, nullptr, F, H, G.data());
    gevmt(wu, x, nullptr, F, H, U.data());
    swiglu(G.data(), U.data(), F);
    gevmt(wd, G.data(), nullptr, H, F, out);
}

void decode_layer(OracleModel& M, size_t li, std::vector<float>& hidden) {
    const OracleConfig& c = M.cfg;
    const Layer& L = M.layers[li];
    const size_t H = c.embedding_size, D = c.head_size, Hq = c.attention_head_count, Hkv = c.kv_head_count;
    const size_t KV = Hkv * D, F = c.feed_forward_size, group = Hq / Hkv;
    std::vector<float>& kc = M.kcache[li];
    std::vector<float>& vc = M.vcache[li];
    const size_t position = kc.size() / KV;

    std::vector<float> A = hidden;
    rmsnorm(A.data(), L.attn_norm.data(), H, c.norm_epsilon);
    std::vector<float> Q(H), K(KV), Vv(KV);
    gevmt(L.wq.data(), A.data(), L.bq.data(), H, H, Q.data());
    gevmt(L.wk.data(), A.data(), L.bk.data(), KV, H, K.data());
    gevmt(L.wv.data(), A.data(), L.bv.data(), KV, H, Vv.data());
    for (size_t h = 0; h < Hq; ++h) rope(&Q[h * D], D, position, c.rope_theta, c.rotary_dimension);
    for (size_t h = 0; h < Hkv; ++h) rope(&K[h * D], D, position, c.rope_theta, c.rotary_dimension);
    kc.insert(kc.end(), K.begin(), K.end());
    vc.insert(vc.end(), Vv.begin(), Vv.end());
    const size_t rows = position + 1;

    std::vector<float> C(H);
    std::vector<float> s(rows);
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    for (size_t h = 0; h < Hq; ++h) {
        const size_t g = h / group;
        // gevmts: dot * (1 / sqrt(D)), cpu_llm.cpp:490-510.
        for (size_t r = 0; r < rows; ++r) {
            float dot = 0.0f;
            for (size_t d = 0; d < D; ++d) dot += kc[r * KV + g * D + d] * Q[h * D + d];
            s[r] = dot * scale;
        }
        softmax(s.data(), rows);
        // gevm: out[d] = sum_r p[r] * V[r][d], cpu_llm.cpp:453-467.
        for (size_t d = 0; d < D; ++d) {
            float acc = 0.0f;
            for (size_t r = 0; r < rows; ++r) acc += s[r] * vc[r * KV + g * D + d];
            C[h * D + d] = acc;
        }
    }
    std::vector<float> O(H);
    gevmt(L.wo.data(), C.data(), nullptr, H, H, O.data());
    std::vector<float> X(H);
    for (size_t i = 0; i < H; ++i) X[i] = hidden[i] + O[i];
    std::vector<float> Fn = X;
    rmsnorm(Fn.data(), L.ffn_norm.data(), H, c.norm_epsilon);
    std::vector<float> Dn(H);
    ffn_swiglu(L.wg.data(), L.wu.data(), L.wd.data(), Fn.data(), H, F, Dn.data());
    for (size_t i = 0; i < H; ++i) hidden[i] = X[i] + Dn[i];
}

int32_t lm_head(OracleModel& M, std::vector<float>& last, float* logits_out) {
    const OracleConfig& c = M.cfg;
    rmsnorm(last.data(), M.output_norm.data(), c.embedding_size, c.norm_epsilon);
    std::vector<float> logits(c.vocabulary_size);
    gevmt(M.output.data(), last.data(), nullptr, c.vocabulary_size, c.embedding_size, logits.data());
    if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * sizeof(float));
    return greedy(logits.data(), logits.size());
}

void set_err(char* err, size_t n, const std::string& m) {
    if (!err || !n) return;
    std::strncpy(err, m.c_str(), n - 1);
    err[n - 1] = 0;
}

template <typename Fn>
int guarded(char* err, size_t n, Fn fn) {
    try {
        fn();
        return 0;
    } catch (const std::invalid_argument& e) {
        set_err(err, n, e.what());
        return 1;
    } catch (const std::out_of_range& e) {
        set_err(err, n, e.what());
        return 2;
    } catch (const std::length_error& e) {
        set_err(err, n, e.what());
        return 3;
    } catch (const std::overflow_error& e) {
        set_err(err, n, e.what());
        return 5;
    } catch (const std::exception& e) {
        set_err(err, n, e.what());
        return 4;
    }
}

}  // namespace

extern "C" {

int oracle_open(const char* path, size_t max_sequence, OracleModel** out, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!path || !out) throw std::invalid_argument("null argument");
        auto m = std::make_unique<OracleModel>();
        load_model(*m, path, max_sequence);
        *out = m.release();
    });
}

void oracle_close(OracleModel* m) { delete m; }

int oracle_config(const OracleModel* m, OracleConfig* out) {
    if (!m || !out) return 1;
    *out = m->cfg;
    return 0;
}

size_t oracle_position(const OracleModel* m) { return m ? m->sequence : 0; }
size_t oracle_max_sequence(const OracleModel* m) { return m ? m->max_sequence : 0; }

int oracle_reset(OracleModel* m, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!m) throw std::runtime_error("CPU model is not initialized");
        m->sequence = 0;
        for (auto& k : m->kcache) k.clear();
        for (auto& v : m->vcache) v.clear();
    });
}

// CPULLM::prefill, cpu_llm.cpp:978-1023.
int oracle_prefill(OracleModel* m, const int32_t* ids, size_t n, int32_t* token, float* logits,
                   char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!m) throw std::runtime_error("CPU model is not initialized");
        if (n == 0 || !ids) throw std::invalid_argument("CPU prefill requires at least one token");
        if (m->sequence != 0) throw std::invalid_argument("CPU prefill requires an empty conversation; call reset first");
        if (n > m->max_sequence) throw std::length_error("CPU prefill exceeds sequence capacity");
        for (size_t i = 0; i < n; ++i) {
            if (ids[i] < 0 || uint64_t(ids[i]) >= m->cfg.vocabulary_size) {
                throw std::out_of_range("CPU prefill token id is outside the vocabulary");
            }
        }
        const size_t H = m->cfg.embedding_size;
        std::vector<float> hidden(n * H);
        for (size_t i = 0; i < n; ++i) std::memcpy(&hidden[i * H], &m->embedding[size_t(ids[i]) * H], H * 4);
        for (size_t l = 0; l < m->layers.size(); ++l) prefill_layer(*m, l, hidden, n);
        std::vector<float> last(hidden.end() - long(H), hidden.end());
        *token = lm_head(*m, last, logits);
        m->sequence = n;
    });
}

// CPULLM::decode, cpu_llm.cpp:1025-1073.
int oracle_decode(OracleModel* m, int32_t id, int32_t* token, float* logits, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        if (!m) throw std::runtime_error("CPU model is not initialized");
        if (m->sequence == 0) throw std::invalid_argument("CPU decode requires a completed prefill");
        if (id < 0 || uint64_t(id) >= m->cfg.vocabulary_size) throw std::out_of_range("CPU decode token id is outside the vocabulary");
        if (m->sequence >= m->max_sequence) throw std::length_error("CPU decode exceeds sequence capacity");
        const size_t H = m->cfg.embedding_size;
        std::vector<float> hidden(&m->embedding[size_t(id) * H], &m->embedding[size_t(id) * H] + H);
        for (size_t l = 0; l < m->layers.size(); ++l) decode_layer(*m, l, hidden);
        *token = lm_head(*m, hidden, logits);
        m->sequence += 1;
    });
}

int oracle_tensor_f32(const OracleModel* m, const char* name, float* out, size_t capacity, char* err, size_t errlen) {
    return guarded(err, errlen, [&] {
        auto it = m->named.find(name);
        if (it == m->named.end()) throw std::runtime_error(std::string("missing tensor: ") + name);
        const std::vector<float>& v = *it->second.first;
        if (capacity < v.size()) throw std::length_error("output buffer too small");
        std::memcpy(out, v.data(), v.size() * 4);
    });
}

int oracle_dequant_row(uint32_t type, const uint8_t* data, size_t cols, float* out) {
    try {
        row_bytes(type, cols);
        dequant_row(type, data, cols, out);
        return 0;
    } catch (...) {
        return 4;
    }
}

float oracle_half_to_float(uint16_t bits) { return half_to_float(bits); }

void oracle_gevmt(const float* w, const float* x, const float* bias, size_t rows, size_t cols, float* y) {
    gevmt(w, x, bias, rows, cols, y);
}
void oracle_rmsnorm(float* x, const float* g, size_t n, float eps) { rmsnorm(x, g, n, eps); }
void oracle_softmax(float* x, size_t n) { softmax(x, n); }
void oracle_swiglu(float* g, const float* u, size_t n) { swiglu(g, u, n); }
void oracle_ffn(const float* wg, const float* wu, const float* wd, const float* x, size_t h, size_t f, float* out) {
    ffn_swiglu(wg, wu, wd, x, h, f, out);
}
void oracle_rope(float* x, size_t len, size_t position, float theta, size_t rot) { rope(x, len, position, theta, rot); }
int32_t oracle_argmax(const float* x, size_t n) { return greedy(x, n); }

}  // extern "C"
