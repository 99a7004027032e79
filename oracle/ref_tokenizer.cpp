// Harness around the reference's own tokenizer (QwenTokenizer and
// pretokenize, chat.cpp:207-529), compiled by oracle/Makefile from chat.cpp
// where it lies into oracle/_ref/. chat.cpp is included as a source file so
// that its anonymous-namespace classes are reachable; its main() is renamed
// and the unused backends drop out at link time (--gc-sections). Test
// infrastructure only: it writes golden vectors for the tokenizer tests.
//
//   ref_tokenizer IN OUT
//
// IN (little endian): u32 n + n strings (vocabulary), u32 m + m strings
// (merges), 1 string (tokenizer_pre), u32 t + t strings (texts); a string is
// u32 byte length + bytes.
// OUT: per text: i32 status (0 ok, 1 encode threw), u32 count + count i32 ids
// (0 ids on error), u32 pieces + 2 * pieces u64 byte offsets; then per
// vocabulary id: u8 is_special, u32 length + decode_piece bytes; then i32
// id("<|im_end|>"), i32 id("</s>").
#define main reference_chat_main
#include "chat.cpp"
#undef main

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>

namespace {

struct Reader {
    std::string data;
    size_t pos = 0;
    uint32_t u32() {
        if (pos + 4 > data.size()) throw std::runtime_error("truncated input");
        uint32_t v;
        std::memcpy(&v, data.data() + pos, 4);
        pos += 4;
        return v;
    }
    std::string str() {
        const uint32_t n = u32();
        if (pos + n > data.size()) throw std::runtime_error("truncated input");
        std::string s = data.substr(pos, n);
        pos += n;
        return s;
    }
    std::vector<std::string> list() {
        std::vector<std::string> v(u32());
        for (auto& s : v) s = str();
        return v;
    }
};

template <typename T>
void put(std::string& out, T v) {
    out.append(reinterpret_cast<const char*>(&v), sizeof(v));
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc != 3) throw std::invalid_argument("usage: ref_tokenizer IN OUT");
        std::ifstream in(argv[1], std::ios::binary);
        Reader r{std::string(std::istreambuf_iterator<char>(in), {})};
        const std::vector<std::string> vocabulary = r.list();
        const std::vector<std::string> merges = r.list();
        const std::string pre = r.str();
        const std::vector<std::string> texts = r.list();
        const chat::QwenTokenizer tok(vocabulary, merges, pre);
        std::string out;
        for (const std::string& text : texts) {
            std::vector<int32_t> ids;
            int32_t status = 0;
            try {
                ids = tok.encode(text);
            } catch (const std::exception&) {
                status = 1;
                ids.clear();
            }
            put(out, status);
            put(out, static_cast<uint32_t>(ids.size()));
            for (int32_t id : ids) put(out, id);
            const auto pieces = chat::pretokenize(text, pre == "qwen35");
            put(out, static_cast<uint32_t>(pieces.size()));
            for (const auto& p : pieces) {
                put(out, static_cast<uint64_t>(p.first));
                put(out, static_cast<uint64_t>(p.second));
            }
        }
        for (size_t i = 0; i < vocabulary.size(); ++i) {
            const int32_t id = static_cast<int32_t>(i);
            put(out, static_cast<uint8_t>(tok.is_special(id) ? 1 : 0));
            const std::string piece = tok.decode_piece(id);
            put(out, static_cast<uint32_t>(piece.size()));
            out += piece;
        }
        put(out, tok.id("<|im_end|>"));
        put(out, tok.id("</s>"));
        std::ofstream(argv[2], std::ios::binary).write(out.data(), static_cast<std::streamsize>(out.size()));
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_tokenizer: %s\n", e.what());
        return 1;
    }
}
