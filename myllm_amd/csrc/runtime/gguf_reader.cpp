// Streaming raw-tensor GGUF reader (see gguf_reader.h). Header parsing,
// validation and the error messages follow metal_model.cpp:394-976; the
// metadata is parsed from the read-only mapping instead of byte-by-byte
// stream reads.
#include "gguf_reader.h"

#include <cerrno>
#include <cmath>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace llm {
namespace {

constexpr std::uint32_t kGgufMagic = 0x46554747u;

std::size_t checked_size(std::uint64_t v, const std::string& what) {
    if (v > std::numeric_limits<std::size_t>::max()) throw std::runtime_error(what + " does not fit in size_t");
    return static_cast<std::size_t>(v);
}

std::size_t checked_mul(std::size_t a, std::size_t b, const std::string& what) {
    if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) throw std::runtime_error(what + " size overflows size_t");
    return a * b;
}

std::size_t checked_add(std::size_t a, std::size_t b, const std::string& what) {
    if (b > std::numeric_limits<std::size_t>::max() - a) throw std::runtime_error(what + " size overflows size_t");
    return a + b;
}

// Bounds-checked little-endian cursor over the header bytes.
class Cursor {
public:
    Cursor(const std::uint8_t* data, std::size_t size) : d_(data), n_(size) {}
    std::size_t pos() const { return p_; }
    void need(std::size_t k) const {
        if (p_ > n_ || k > n_ - p_) throw std::runtime_error("truncated GGUF file");
    }
    std::uint8_t u8() { need(1); return d_[p_++]; }
    std::uint16_t u16() { need(2); std::uint16_t v = static_cast<std::uint16_t>(d_[p_] | (d_[p_ + 1] << 8)); p_ += 2; return v; }
    std::uint32_t u32() {
        need(4);
        std::uint32_t v = 0;
        for (int i = 0; i < 4; ++i) v |= static_cast<std::uint32_t>(d_[p_ + i]) << (8 * i);
        p_ += 4;
        return v;
    }
    std::uint64_t u64() {
        need(8);
        std::uint64_t v = 0;
        for (int i = 0; i < 8; ++i) v |= static_cast<std::uint64_t>(d_[p_ + i]) << (8 * i);
        p_ += 8;
        return v;
    }
    float f32() { std::uint32_t b = u32(); float f; std::memcpy(&f, &b, 4); return f; }
    double f64() { std::uint64_t b = u64(); double f; std::memcpy(&f, &b, 8); return f; }
    std::string str() {
        const std::size_t len = checked_size(u64(), "GGUF string length");
        need(len);
        std::string s(reinterpret_cast<const char*>(d_ + p_), len);
        p_ += len;
        return s;
    }
    void skip(std::size_t k) { need(k); p_ += k; }

private:
    const std::uint8_t* d_;
    std::size_t n_;
    std::size_t p_ = 0;
};

struct Metadata {
    std::unordered_map<std::string, std::uint64_t> ints;
    std::unordered_map<std::string, double> reals;
    std::unordered_map<std::string, std::string> texts;
    std::vector<std::string> vocabulary;
    std::vector<std::string> merges;
};

void skip_value(Cursor& c, std::uint32_t type) {
    switch (type) {
    case 0: case 1: case 7: c.skip(1); break;
    case 2: case 3: c.skip(2); break;
    case 4: case 5: case 6: c.skip(4); break;
    case 10: case 11: case 12: c.skip(8); break;
    case 8: c.skip(checked_size(c.u64(), "GGUF string length")); break;
    case 9: {
        const std::uint32_t et = c.u32();
        const std::size_t n = checked_size(c.u64(), "GGUF nested array count");
        for (std::size_t i = 0; i < n; ++i) skip_value(c, et);
        break;
    }
    default: throw std::runtime_error("unsupported GGUF array element type " + std::to_string(type));
    }
}

void read_value(Cursor& c, std::uint32_t type, const std::string& key, Metadata& m) {
    switch (type) {
    case 0: m.ints[key] = c.u8(); break;
    case 1: m.ints[key] = static_cast<std::uint64_t>(static_cast<std::int8_t>(c.u8())); break;
    case 2: m.ints[key] = c.u16(); break;
    case 3: m.ints[key] = static_cast<std::uint64_t>(static_cast<std::int16_t>(c.u16())); break;
    case 4: m.ints[key] = c.u32(); break;
    case 5: m.ints[key] = static_cast<std::uint64_t>(static_cast<std::int32_t>(c.u32())); break;
    case 6: m.reals[key] = c.f32(); break;
    case 7: m.ints[key] = c.u8() != 0 ? 1 : 0; break;
    case 8: m.texts[key] = c.str(); break;
    case 9: {
        const std::uint32_t et = c.u32();
        const std::size_t n = checked_size(c.u64(), "GGUF metadata array count");
        if (key == "tokenizer.ggml.tokens" && et == 8) {
            m.vocabulary.clear();
            m.vocabulary.reserve(n);
            for (std::size_t i = 0; i < n; ++i) m.vocabulary.push_back(c.str());
        } else if (key == "tokenizer.ggml.merges" && et == 8) {
            m.merges.clear();
            m.merges.reserve(n);
            for (std::size_t i = 0; i < n; ++i) m.merges.push_back(c.str());
        } else {
            for (std::size_t i = 0; i < n; ++i) skip_value(c, et);
        }
        break;
    }
    case 10: m.ints[key] = c.u64(); break;
    case 11: m.ints[key] = c.u64(); break;
    case 12: m.reals[key] = c.f64(); break;
    default: throw std::runtime_error("unsupported GGUF metadata type " + std::to_string(type));
    }
}

bool known_type(std::uint32_t t) {
    switch (t) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9: case 10: case 11: case 12: case 13: case 14: case 30:
        return true;
    default:
        return false;
    }
}

std::size_t meta_size(const Metadata& m, const std::string& key) {
    const auto it = m.ints.find(key);
    if (it == m.ints.end() || it->second == 0 || it->second > std::numeric_limits<std::size_t>::max()) {
        throw std::runtime_error("missing or invalid GGUF metadata: " + key);
    }
    return static_cast<std::size_t>(it->second);
}

}  // namespace

const char* ggml_type_name(GgmlType type) noexcept {
    switch (type) {
    case GgmlType::F32: return "F32";
    case GgmlType::F16: return "F16";
    case GgmlType::Q4_0: return "Q4_0";
    case GgmlType::Q4_1: return "Q4_1";
    case GgmlType::Q5_0: return "Q5_0";
    case GgmlType::Q5_1: return "Q5_1";
    case GgmlType::Q8_0: return "Q8_0";
    case GgmlType::Q8_1: return "Q8_1";
    case GgmlType::Q2_K: return "Q2_K";
    case GgmlType::Q3_K: return "Q3_K";
    case GgmlType::Q4_K: return "Q4_K";
    case GgmlType::Q5_K: return "Q5_K";
    case GgmlType::Q6_K: return "Q6_K";
    case GgmlType::BF16: return "BF16";
    }
    return "UNKNOWN";
}

std::size_t ggml_block_size(GgmlType type) {
    switch (type) {
    case GgmlType::F32: case GgmlType::F16: case GgmlType::BF16: return 1;
    case GgmlType::Q4_0: case GgmlType::Q4_1: case GgmlType::Q5_0: case GgmlType::Q5_1:
    case GgmlType::Q8_0: case GgmlType::Q8_1: return 32;
    case GgmlType::Q2_K: case GgmlType::Q3_K: case GgmlType::Q4_K: case GgmlType::Q5_K: case GgmlType::Q6_K: return 256;
    }
    throw std::runtime_error("unsupported GGML tensor type");
}

std::size_t ggml_type_size(GgmlType type) {
    switch (type) {
    case GgmlType::F32: return 4;
    case GgmlType::F16: return 2;
    case GgmlType::Q4_0: return 18;
    case GgmlType::Q4_1: return 20;
    case GgmlType::Q5_0: return 22;
    case GgmlType::Q5_1: return 24;
    case GgmlType::Q8_0: return 34;
    case GgmlType::Q8_1: return 40;
    case GgmlType::Q2_K: return 84;
    case GgmlType::Q3_K: return 110;
    case GgmlType::Q4_K: return 144;
    case GgmlType::Q5_K: return 176;
    case GgmlType::Q6_K: return 210;
    case GgmlType::BF16: return 2;
    }
    throw std::runtime_error("unsupported GGML tensor type");
}

std::size_t ggml_row_bytes(GgmlType type, std::size_t columns) {
    const std::size_t bs = ggml_block_size(type);
    if (columns % bs != 0) throw std::runtime_error(std::string(ggml_type_name(type)) + " row is not block aligned");
    return checked_mul(columns / bs, ggml_type_size(type), std::string(ggml_type_name(type)) + " row");
}

struct GgufReader::Impl {
    std::string path;
    int fd = -1;
    std::size_t file_size = 0;
    const std::uint8_t* map = nullptr;
    Metadata meta;
    std::vector<TensorDescriptor> tensors;
    std::unordered_map<std::string, std::size_t> index;
    std::unordered_set<std::string> consumed;
    std::unordered_set<std::string> ignored;
    GgufModelConfig config;

    explicit Impl(const std::string& p) : path(p) {
        fd = ::open(p.c_str(), O_RDONLY);
        if (fd < 0) throw std::runtime_error("cannot open model: " + p);
        struct stat st;
        if (::fstat(fd, &st) != 0 || st.st_size <= 0) throw std::runtime_error("invalid or oversized GGUF model file");
        file_size = static_cast<std::size_t>(st.st_size);
        void* m = ::mmap(nullptr, file_size, PROT_READ, MAP_PRIVATE, fd, 0);
        std::vector<std::uint8_t> header_copy;
        const std::uint8_t* bytes = nullptr;
        if (m != MAP_FAILED) {
            map = static_cast<const std::uint8_t*>(m);
            bytes = map;
        } else {
            // Without a mapping the header is read into memory in full.
            header_copy.resize(file_size);
            std::size_t got = 0;
            while (got < file_size) {
                const ssize_t r = ::pread(fd, header_copy.data() + got, file_size - got, static_cast<off_t>(got));
                if (r <= 0) throw std::runtime_error("cannot read GGUF file");
                got += static_cast<std::size_t>(r);
            }
            bytes = header_copy.data();
        }
        Cursor c(bytes, file_size);
        if (c.u32() != kGgufMagic) throw std::runtime_error("not a GGUF file");
        const std::uint32_t version = c.u32();
        if (version != 2 && version != 3) throw std::runtime_error("unsupported GGUF version " + std::to_string(version));
        const std::size_t tcount = checked_size(c.u64(), "GGUF tensor count");
        const std::size_t kcount = checked_size(c.u64(), "GGUF metadata count");
        for (std::size_t i = 0; i < kcount; ++i) {
            const std::string key = c.str();
            read_value(c, c.u32(), key, meta);
        }
        tensors.reserve(tcount);
        std::vector<std::uint64_t> rel(tcount);
        for (std::size_t i = 0; i < tcount; ++i) {
            TensorDescriptor t;
            t.name = c.str();
            const std::uint32_t nd = c.u32();
            if (nd == 0) throw std::runtime_error("scalar GGUF tensors are unsupported: " + t.name);
            for (std::uint32_t d = 0; d < nd; ++d) t.dimensions.push_back(c.u64());
            const std::uint32_t type_id = c.u32();
            if (!known_type(type_id)) {
                throw std::runtime_error("unsupported GGUF tensor type " + std::to_string(type_id) + " for " + t.name);
            }
            t.type = static_cast<GgmlType>(type_id);
            rel[i] = c.u64();
            t.cols = checked_size(t.dimensions.front(), "GGUF tensor dimension");
            t.rows = 1;
            for (std::size_t d = 1; d < t.dimensions.size(); ++d) {
                t.rows = checked_mul(t.rows, checked_size(t.dimensions[d], "GGUF tensor dimension"), "GGUF tensor shape");
            }
            t.row_bytes = ggml_row_bytes(t.type, t.cols);
            t.byte_size = checked_mul(t.rows, t.row_bytes, "tensor " + t.name);
            tensors.push_back(std::move(t));
        }
        const auto al = meta.ints.find("general.alignment");
        const std::size_t alignment = al == meta.ints.end() ? 32 : checked_size(al->second, "GGUF alignment");
        if (alignment == 0 || (alignment & (alignment - 1)) != 0) throw std::runtime_error("invalid GGUF alignment");
        const std::size_t data_start = checked_add(c.pos(), (alignment - c.pos() % alignment) % alignment, "GGUF alignment");
        if (data_start > file_size) throw std::runtime_error("GGUF tensor data starts past end of file");
        for (std::size_t i = 0; i < tensors.size(); ++i) {
            TensorDescriptor& t = tensors[i];
            t.data_offset = checked_add(data_start, checked_size(rel[i], "GGUF tensor offset"), "GGUF tensor offset");
            if (t.data_offset > file_size || t.byte_size > file_size - t.data_offset) {
                throw std::runtime_error("tensor data is outside GGUF file: " + t.name);
            }
            if (!index.emplace(t.name, i).second) throw std::runtime_error("duplicate GGUF tensor: " + t.name);
        }
        derive_config();
    }

    ~Impl() {
        if (map) ::munmap(const_cast<std::uint8_t*>(map), file_size);
        if (fd >= 0) ::close(fd);
    }

    // metal_model.cpp:573-688.
    void derive_config() {
        auto at = meta.texts.find("general.architecture");
        config.architecture = at == meta.texts.end() ? "" : at->second;
        if (config.architecture != "qwen2" && config.architecture != "qwen35moe") {
            throw std::runtime_error("GGUF architecture is not supported: " + config.architecture);
        }
        config.tensor_count = tensors.size();
        const std::string p = config.architecture + ".";
        config.total_layer_count = meta_size(meta, p + "block_count");
        if (config.architecture == "qwen35moe") {
            const auto it = meta.ints.find(p + "nextn_predict_layers");
            config.nextn_layer_count = it == meta.ints.end() ? 0 : static_cast<std::size_t>(it->second);
        }
        if (config.nextn_layer_count >= config.total_layer_count) throw std::runtime_error("invalid optional NextN/MTP layer count");
        config.layer_count = config.total_layer_count - config.nextn_layer_count;
        config.embedding_size = meta_size(meta, p + "embedding_length");
        config.attention_head_count = meta_size(meta, p + "attention.head_count");
        config.kv_head_count = meta_size(meta, p + "attention.head_count_kv");
        config.context_length = meta_size(meta, p + "context_length");
        if (config.architecture == "qwen2") {
            config.feed_forward_size = meta_size(meta, "qwen2.feed_forward_length");
        } else {
            config.expert_count = meta_size(meta, p + "expert_count");
            config.expert_used_count = meta_size(meta, p + "expert_used_count");
            config.expert_feed_forward_size = meta_size(meta, p + "expert_feed_forward_length");
            config.shared_expert_feed_forward_size = meta_size(meta, p + "expert_shared_feed_forward_length");
            config.feed_forward_size = config.expert_feed_forward_size;
            config.full_attention_interval = meta_size(meta, p + "full_attention_interval");
            config.ssm_conv_kernel = meta_size(meta, p + "ssm.conv_kernel");
            config.ssm_state_size = meta_size(meta, p + "ssm.state_size");
            config.ssm_group_count = meta_size(meta, p + "ssm.group_count");
            config.ssm_time_step_rank = meta_size(meta, p + "ssm.time_step_rank");
            config.ssm_inner_size = meta_size(meta, p + "ssm.inner_size");
        }
        config.vocabulary_size = meta.vocabulary.size();
        if (config.vocabulary_size == 0) config.vocabulary_size = meta_size(meta, "tokenizer.ggml.tokens_count");
        config.vocabulary = meta.vocabulary;
        config.merges = meta.merges;
        const auto tp = meta.texts.find("tokenizer.ggml.pre");
        config.tokenizer_pre = tp == meta.texts.end() ? "" : tp->second;
        if (config.attention_head_count % config.kv_head_count != 0) {
            throw std::runtime_error("attention head count must be divisible by KV head count");
        }
        if (config.architecture == "qwen2") {
            if (config.embedding_size % config.attention_head_count != 0) {
                throw std::runtime_error("embedding size must be divisible by attention head count");
            }
            config.head_size = config.embedding_size / config.attention_head_count;
            config.rotary_dimension = config.head_size;
        } else {
            config.head_size = meta_size(meta, p + "attention.key_length");
            if (meta_size(meta, p + "attention.value_length") != config.head_size) {
                throw std::runtime_error("qwen35moe key/value head dimensions differ");
            }
            config.rotary_dimension = meta_size(meta, p + "rope.dimension_count");
        }
        const auto real = [&](const std::string& k, double fb) {
            const auto it = meta.reals.find(k);
            return it == meta.reals.end() ? fb : it->second;
        };
        config.rope_theta = static_cast<float>(real(p + "rope.freq_base", 1000000.0));
        config.norm_epsilon = static_cast<float>(real(p + "attention.layer_norm_rms_epsilon", 1e-6));
        if (!std::isfinite(config.rope_theta) || config.rope_theta <= 0.0f || !std::isfinite(config.norm_epsilon) ||
            config.norm_epsilon <= 0.0f) {
            throw std::runtime_error("invalid RoPE or RMSNorm metadata");
        }
        const auto eos = meta.ints.find("tokenizer.ggml.eos_token_id");
        const std::uint64_t e = eos == meta.ints.end() ? 151645 : eos->second;
        if (e > static_cast<std::uint64_t>(std::numeric_limits<std::int32_t>::max())) {
            throw std::runtime_error("EOS token id does not fit in int32_t");
        }
        config.eos_token_id = static_cast<std::int32_t>(e);
        for (const TensorDescriptor& t : tensors) {
            config.parameter_count = checked_add(config.parameter_count, checked_mul(t.rows, t.cols, "tensor " + t.name),
                                                 "model parameter count");
            config.stored_weight_bytes = checked_add(config.stored_weight_bytes, t.byte_size, "stored model weights");
        }
    }

    const TensorDescriptor& require(const std::string& name) const {
        const auto it = index.find(name);
        if (it == index.end()) throw std::runtime_error("missing tensor: " + name);
        return tensors[it->second];
    }
};

GgufReader::GgufReader(const std::string& path) : impl_(std::make_unique<Impl>(path)) {}
GgufReader::~GgufReader() = default;

const GgufModelConfig& GgufReader::config() const noexcept { return impl_->config; }

bool GgufReader::has_tensor(const std::string& name) const noexcept {
    return impl_->index.find(name) != impl_->index.end();
}

TensorDescriptor GgufReader::take(const std::string& name, std::size_t rows, std::size_t cols) {
    const TensorDescriptor& t = impl_->require(name);
    if (t.rows != rows || t.cols != cols) {
        throw std::runtime_error("unexpected shape for tensor " + name + ": expected " + std::to_string(rows) + "x" +
                                 std::to_string(cols) + ", got " + std::to_string(t.rows) + "x" + std::to_string(t.cols));
    }
    if (!impl_->consumed.insert(name).second) throw std::runtime_error("tensor consumed more than once: " + name);
    return t;
}

void GgufReader::read(const TensorDescriptor& t, std::size_t offset, void* dst, std::size_t bytes) const {
    const TensorDescriptor& known = impl_->require(t.name);
    if (known.data_offset != t.data_offset || known.byte_size != t.byte_size) {
        throw std::invalid_argument("tensor descriptor does not match GGUF index: " + t.name);
    }
    if (offset > t.byte_size || bytes > t.byte_size - offset) {
        throw std::out_of_range("tensor slice is outside GGUF tensor: " + t.name);
    }
    if (bytes == 0) return;
    if (dst == nullptr) throw std::invalid_argument("tensor slice destination is null: " + t.name);
    const std::size_t at = t.data_offset + offset;
    if (impl_->map) {
        std::memcpy(dst, impl_->map + at, bytes);
        return;
    }
    auto* out = static_cast<std::uint8_t*>(dst);
    std::size_t done = 0;
    while (done < bytes) {
        const ssize_t r = ::pread(impl_->fd, out + done, bytes - done, static_cast<off_t>(at + done));
        if (r < 0) throw std::runtime_error("cannot read GGUF tensor slice " + t.name + ": " + std::strerror(errno));
        if (r == 0) throw std::runtime_error("unexpected EOF while reading tensor slice: " + t.name);
        done += static_cast<std::size_t>(r);
    }
}

const std::uint8_t* GgufReader::mapped(const TensorDescriptor& t) const noexcept {
    return impl_->map ? impl_->map + t.data_offset : nullptr;
}

void GgufReader::ignore(const std::string& name) {
    if (!has_tensor(name)) throw std::runtime_error("cannot ignore missing tensor: " + name);
    if (impl_->consumed.count(name)) throw std::runtime_error("cannot ignore loaded tensor: " + name);
    impl_->ignored.insert(name);
}

void GgufReader::ignore_prefix(const std::string& prefix) {
    for (const TensorDescriptor& t : impl_->tensors) {
        if (t.name.compare(0, prefix.size(), prefix) == 0) {
            if (impl_->consumed.count(t.name)) throw std::runtime_error("cannot ignore loaded tensor: " + t.name);
            impl_->ignored.insert(t.name);
        }
    }
}

void GgufReader::validate_all_consumed() const {
    if (impl_->consumed.size() + impl_->ignored.size() == impl_->tensors.size()) return;
    std::string msg = "GGUF contains tensors not mapped by the loader:";
    for (const TensorDescriptor& t : impl_->tensors) {
        if (!impl_->consumed.count(t.name) && !impl_->ignored.count(t.name)) msg += " " + t.name;
    }
    throw std::runtime_error(msg);
}

}  // namespace llm
