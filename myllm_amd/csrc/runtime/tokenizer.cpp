// Qwen byte-level BPE tokenizer (interface of chat.cpp:349-529).
#include "tokenizer.h"

#include <algorithm>
#include <cstring>
#include <queue>
#include <stdexcept>

namespace llm {
namespace {

// ---------------------------------------------------------------- UTF-8

struct Cp {
    std::uint32_t value;
    std::uint32_t length;  // bytes
};

// One codepoint at p (p < n). A lead byte whose continuation bytes are all
// present and well formed gives the decoded value (no overlong or range
// checks); anything else is one codepoint equal to the byte (chat.cpp:34-78).
inline Cp utf8_at(const unsigned char* s, std::size_t n, std::size_t p) {
    const std::uint32_t b0 = s[p];
    std::uint32_t need, value;
    if ((b0 & 0xe0u) == 0xc0u) {
        need = 1;
        value = b0 & 0x1fu;
    } else if ((b0 & 0xf0u) == 0xe0u) {
        need = 2;
        value = b0 & 0x0fu;
    } else if ((b0 & 0xf8u) == 0xf0u) {
        need = 3;
        value = b0 & 0x07u;
    } else {
        return {b0, 1};
    }
    if (p + need >= n) return {b0, 1};
    for (std::uint32_t i = 1; i <= need; ++i) {
        const std::uint32_t c = s[p + i];
        if ((c & 0xc0u) != 0x80u) return {b0, 1};
        value = (value << 6) | (c & 0x3fu);
    }
    return {value, need + 1};
}

// Encoder of chat.cpp:80-96: 1 to 4 bytes by value, no range checks.
inline void put_utf8(std::uint32_t v, std::string& out) {
    if (v < 0x80u) {
        out.push_back(static_cast<char>(v));
    } else if (v < 0x800u) {
        out.push_back(static_cast<char>(0xc0u | (v >> 6)));
        out.push_back(static_cast<char>(0x80u | (v & 0x3fu)));
    } else if (v < 0x10000u) {
        out.push_back(static_cast<char>(0xe0u | (v >> 12)));
        out.push_back(static_cast<char>(0x80u | ((v >> 6) & 0x3fu)));
        out.push_back(static_cast<char>(0x80u | (v & 0x3fu)));
    } else {
        out.push_back(static_cast<char>(0xf0u | (v >> 18)));
        out.push_back(static_cast<char>(0x80u | ((v >> 12) & 0x3fu)));
        out.push_back(static_cast<char>(0x80u | ((v >> 6) & 0x3fu)));
        out.push_back(static_cast<char>(0x80u | (v & 0x3fu)));
    }
}

// Decode and re-encode: the form in which merge operands are compared.
std::string canonical_utf8(const std::string& s) {
    const auto* b = reinterpret_cast<const unsigned char*>(s.data());
    std::string out;
    out.reserve(s.size() + 4);
    for (std::size_t p = 0; p < s.size();) {
        const Cp c = utf8_at(b, s.size(), p);
        put_utf8(c.value, out);
        p += c.length;
    }
    return out;
}

// ------------------------------------------------------ character classes
//
// Inclusive codepoint ranges of chat.cpp:101-172 (the Qwen chat demo's
// coarse stand-ins for \p{M}, \p{L}, \p{N} and \s).

struct Range {
    std::uint32_t lo, hi;
};

constexpr Range kMarks[] = {
    {0x0300, 0x036f}, {0x0483, 0x0489}, {0x0591, 0x05bd}, {0x05bf, 0x05bf}, {0x05c1, 0x05c2},
    {0x05c4, 0x05c5}, {0x05c7, 0x05c7}, {0x0610, 0x061a}, {0x064b, 0x065f}, {0x0670, 0x0670},
    {0x06d6, 0x06dc}, {0x06df, 0x06e4}, {0x06e7, 0x06e8}, {0x06ea, 0x06ed}, {0x0711, 0x0711},
    {0x0730, 0x074a}, {0x1ab0, 0x1aff}, {0x1dc0, 0x1dff}, {0x20d0, 0x20ff}, {0xfe00, 0xfe0f},
    {0xfe20, 0xfe2f}, {0xe0100, 0xe01ef},
};

constexpr Range kLetters[] = {
    {0x00c0, 0x02ff}, {0x0370, 0x052f}, {0x0530, 0x058f}, {0x0600, 0x06ff}, {0x0700, 0x074f},
    {0x0900, 0x0dff}, {0x0e00, 0x0e7f}, {0x10a0, 0x10ff}, {0x1100, 0x11ff}, {0x3040, 0x30ff},
    {0x3400, 0x9fff}, {0xac00, 0xd7af}, {0xf900, 0xfaff}, {0x20000, 0x323af},
};

constexpr Range kNumbers[] = {
    {'0', '9'}, {0x0660, 0x0669}, {0x06f0, 0x06f9}, {0x0966, 0x096f}, {0xff10, 0xff19},
};

constexpr Range kSpaces[] = {
    {'\t', '\r'},  // \t \n \v \f \r
    {' ', ' '},    {0x00a0, 0x00a0}, {0x1680, 0x1680}, {0x2000, 0x200a}, {0x2028, 0x2029},
    {0x202f, 0x202f}, {0x205f, 0x205f}, {0x3000, 0x3000},
};

template <std::size_t N>
constexpr bool in_ranges(const Range (&table)[N], std::uint32_t v) {
    for (const Range& r : table) {
        if (v < r.lo) return false;  // tables are sorted
        if (v <= r.hi) return true;
    }
    return false;
}

enum Class : std::uint8_t { kOther = 0, kLetter, kMark, kNumber, kSpace, kBreak };

Class classify(std::uint32_t v) {
    if (v < 0x80u) {
        if ((v | 0x20u) >= 'a' && (v | 0x20u) <= 'z') return kLetter;
        if (v >= '0' && v <= '9') return kNumber;
        if (v == '\n' || v == '\r') return kBreak;
        if (v == ' ' || (v >= '\t' && v <= '\r')) return kSpace;
        return kOther;
    }
    // Numbers and marks win over the letter ranges that contain them.
    if (in_ranges(kNumbers, v)) return kNumber;
    if (in_ranges(kMarks, v)) return kMark;
    if (in_ranges(kLetters, v)) return kLetter;
    if (in_ranges(kSpaces, v)) return kSpace;
    return kOther;
}

// ------------------------------------------------------- byte symbols

// GPT-2's reversible byte -> codepoint map: printable Latin-1 bytes
// (33-126, 161-172, 174-255) stand for themselves, the other 68 bytes take
// 256, 257, ... in byte order.
struct ByteMap {
    std::uint32_t to_cp[256];
    std::int16_t from_cp[512];  // -1: not a byte symbol
    ByteMap() {
        std::fill(std::begin(from_cp), std::end(from_cp), std::int16_t(-1));
        std::uint32_t next = 256;
        for (std::uint32_t b = 0; b < 256; ++b) {
            const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174);
            to_cp[b] = printable ? b : next++;
            from_cp[to_cp[b]] = static_cast<std::int16_t>(b);
        }
    }
};

const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

inline std::uint64_t pair_key(std::int32_t a, std::int32_t b) {
    return (static_cast<std::uint64_t>(static_cast<std::uint32_t>(a)) << 32) | static_cast<std::uint32_t>(b);
}

inline bool is_special_name(const std::string& s) {
    return s.size() >= 4 && s.compare(0, 2, "<|") == 0 && s.compare(s.size() - 2, 2, "|>") == 0;
}

}  // namespace

// ------------------------------------------------------------ construction

std::int32_t QwenTokenizer::find_symbol(const std::string& s) const {
    const auto it = symbols_.find(s);
    return it == symbols_.end() ? -1 : it->second;
}

std::int32_t QwenTokenizer::intern(const std::string& s) {
    const auto it = symbols_.find(s);
    if (it != symbols_.end()) return it->second;
    const auto sym = static_cast<std::int32_t>(vocabulary_.size() + extra_symbols_.size());
    extra_symbols_.push_back(s);
    symbols_.emplace(s, sym);
    return sym;
}

QwenTokenizer::QwenTokenizer(const std::vector<std::string>& vocabulary, const std::vector<std::string>& merges,
                             const std::string& tokenizer_pre)
    : vocabulary_(vocabulary), include_marks_(tokenizer_pre == "qwen35") {
    if (vocabulary_.size() >= 0x7fffffffu) throw std::invalid_argument("tokenizer vocabulary is too large");
    special_.assign(vocabulary_.size(), 0);
    symbols_.reserve(vocabulary_.size() * 2 + 512);
    for (std::size_t i = 0; i < vocabulary_.size(); ++i) {
        const std::string& s = vocabulary_[i];
        symbols_.emplace(s, static_cast<std::int32_t>(i));  // keeps the first id of a duplicate
        if (is_special_name(s)) {
            special_[i] = 1;
            special_ids_.emplace(s, static_cast<std::int32_t>(i));
            special_lengths_.push_back(s.size());
        }
    }
    std::sort(special_lengths_.begin(), special_lengths_.end(), std::greater<>());
    special_lengths_.erase(std::unique(special_lengths_.begin(), special_lengths_.end()), special_lengths_.end());

    const ByteMap& bm = byte_map();
    for (int b = 0; b < 256; ++b) {
        std::string one;
        put_utf8(bm.to_cp[b], one);
        byte_symbol_[b] = intern(one);
    }

    // "left right" with the separator at the first space past byte 0; lines
    // without one, or with an empty operand, are skipped; a repeated pair
    // keeps its first (lowest) rank (chat.cpp:364-373).
    merges_.reserve(merges.size() * 2);
    for (std::size_t rank = 0; rank < merges.size(); ++rank) {
        const std::string& line = merges[rank];
        const std::size_t sep = line.find(' ', 1);
        if (sep == std::string::npos || sep + 1 >= line.size()) continue;
        const std::string left = canonical_utf8(line.substr(0, sep));
        const std::string right = canonical_utf8(line.substr(sep + 1));
        const std::int32_t a = intern(left);
        const std::int32_t b = intern(right);
        const std::int32_t joined = intern(left + right);
        merges_.emplace(pair_key(a, b), Merge{static_cast<std::uint32_t>(rank), joined});
    }
}

// ------------------------------------------------------------ lookups

std::int32_t QwenTokenizer::id(const std::string& token) const {
    const std::int32_t s = find_symbol(token);
    return s >= 0 && static_cast<std::size_t>(s) < vocabulary_.size() ? s : -1;
}

bool QwenTokenizer::is_special(std::int32_t token) const {
    return token >= 0 && static_cast<std::size_t>(token) < special_.size() && special_[token] != 0;
}

std::string QwenTokenizer::decode_piece(std::int32_t token) const {
    if (token < 0 || static_cast<std::size_t>(token) >= vocabulary_.size() || is_special(token)) return {};
    const std::string& piece = vocabulary_[static_cast<std::size_t>(token)];
    const auto* b = reinterpret_cast<const unsigned char*>(piece.data());
    const ByteMap& bm = byte_map();
    std::string out;
    out.reserve(piece.size());
    for (std::size_t p = 0; p < piece.size();) {
        const Cp c = utf8_at(b, piece.size(), p);
        const int byte = c.value < 512 ? bm.from_cp[c.value] : -1;
        if (byte >= 0) {
            out.push_back(static_cast<char>(byte));
        } else {
            put_utf8(c.value, out);
        }
        p += c.length;
    }
    return out;
}

// ------------------------------------------------------------ special tokens

std::size_t QwenTokenizer::special_at(const std::string& text, std::size_t pos, std::int32_t* token) const {
    for (const std::size_t len : special_lengths_) {
        if (pos + len > text.size()) continue;
        const auto it = special_ids_.find(text.substr(pos, len));
        if (it != special_ids_.end()) {
            *token = it->second;
            return len;
        }
    }
    return 0;
}

// First position >= from where a special token starts (text.size() if none).
std::size_t QwenTokenizer::next_special(const std::string& text, std::size_t from) const {
    if (special_lengths_.empty()) return text.size();
    for (std::size_t p = text.find("<|", from); p != std::string::npos; p = text.find("<|", p + 1)) {
        std::int32_t tok;
        if (special_at(text, p, &tok) != 0) return p;
    }
    return text.size();
}

// ------------------------------------------------------------ pre-tokenizer

std::vector<std::pair<std::size_t, std::size_t>> QwenTokenizer::pieces(const std::string& text) const {
    const auto* s = reinterpret_cast<const unsigned char*>(text.data());
    const std::size_t nbytes = text.size();
    std::vector<std::uint32_t> cp, off;
    std::vector<Class> cls;
    cp.reserve(nbytes);
    off.reserve(nbytes + 1);
    for (std::size_t p = 0; p < nbytes;) {
        const Cp c = utf8_at(s, nbytes, p);
        cp.push_back(c.value);
        off.push_back(static_cast<std::uint32_t>(p));
        cls.push_back(classify(c.value));
        p += c.length;
    }
    off.push_back(static_cast<std::uint32_t>(nbytes));
    const std::size_t n = cp.size();
    const bool marks = include_marks_;
    auto word = [&](std::size_t i) { return cls[i] == kLetter || (marks && cls[i] == kMark); };
    auto space = [&](std::size_t i) { return cls[i] == kSpace || cls[i] == kBreak; };
    auto lower = [&](std::size_t i) { return cp[i] < 0x80u ? (cp[i] | ((cp[i] >= 'A' && cp[i] <= 'Z') ? 0x20u : 0u)) : cp[i]; };
    // Length of an English contraction at i: 's 't 'm 'd (2), 're 've 'll (3).
    auto contraction = [&](std::size_t i) -> std::size_t {
        if (cp[i] != '\'' || i + 1 >= n) return 0;
        const std::uint32_t c1 = lower(i + 1);
        if (c1 == 's' || c1 == 't' || c1 == 'm' || c1 == 'd') return 2;
        if (i + 2 >= n) return 0;
        const std::uint32_t c2 = lower(i + 2);
        if ((c1 == 'r' && c2 == 'e') || (c1 == 'v' && c2 == 'e') || (c1 == 'l' && c2 == 'l')) return 3;
        return 0;
    };

    std::vector<std::pair<std::size_t, std::size_t>> out;
    std::size_t i = 0;
    while (i < n) {
        std::size_t j;
        if (const std::size_t c = contraction(i)) {
            j = i + c;
        } else if (cls[i] != kBreak && cls[i] != kNumber && (word(i) || (i + 1 < n && word(i + 1)))) {
            // One optional non-letter prefix, then the letter run.
            j = i + 1;
            while (j < n && word(j)) ++j;
        } else if (cls[i] == kNumber) {
            j = i + 1;  // digits are single pieces
        } else {
            const std::size_t start = i + (cp[i] == ' ' ? 1 : 0);
            auto punct = [&](std::size_t k) { return !space(k) && !word(k) && cls[k] != kNumber; };
            if (start < n && punct(start)) {
                j = start;
                while (j < n && punct(j)) ++j;
                while (j < n && cls[j] == kBreak) ++j;
            } else {
                std::size_t run = 0, after_break = 0;
                while (i + run < n && space(i + run)) {
                    if (cls[i + run] == kBreak) after_break = i + run + 1;
                    ++run;
                }
                if (after_break != 0) {
                    j = after_break;  // up to and including the last line break
                } else if (run > 1 && i + run < n) {
                    j = i + run - 1;  // leave one space for the next word
                } else if (run > 0) {
                    j = i + run;
                } else {
                    j = i + 1;
                }
            }
        }
        out.emplace_back(off[i], off[j]);
        i = j;
    }
    return out;
}

// ------------------------------------------------------------ BPE

void QwenTokenizer::encode_piece(const unsigned char* bytes, std::size_t n, std::vector<std::int32_t>& out) const {
    if (n == 0) return;
    struct Node {
        std::int32_t sym;
        std::int32_t prev, next;  // -1 at the ends
        bool alive;
    };
    std::vector<Node> nodes(n);
    for (std::size_t i = 0; i < n; ++i) {
        nodes[i] = {byte_symbol_[bytes[i]], static_cast<std::int32_t>(i) - 1,
                    i + 1 < n ? static_cast<std::int32_t>(i + 1) : -1, true};
    }
    struct Candidate {
        std::uint32_t rank;
        std::int32_t left;  // node index = byte offset of the left chunk
        std::int32_t left_sym, right_sym;
        bool operator>(const Candidate& o) const { return rank != o.rank ? rank > o.rank : left > o.left; }
    };
    std::priority_queue<Candidate, std::vector<Candidate>, std::greater<Candidate>> heap;
    auto offer = [&](std::int32_t a) {
        if (a < 0) return;
        const std::int32_t b = nodes[a].next;
        if (b < 0) return;
        const auto it = merges_.find(pair_key(nodes[a].sym, nodes[b].sym));
        if (it != merges_.end()) heap.push({it->second.rank, a, nodes[a].sym, nodes[b].sym});
    };
    for (std::size_t i = 0; i + 1 < n; ++i) offer(static_cast<std::int32_t>(i));
    while (!heap.empty()) {
        const Candidate c = heap.top();
        heap.pop();
        Node& a = nodes[c.left];
        // A chunk's symbol only ever grows, so a candidate whose two symbols
        // still match the current neighbours is current.
        if (!a.alive || a.sym != c.left_sym || a.next < 0 || nodes[a.next].sym != c.right_sym) continue;
        Node& b = nodes[a.next];
        a.sym = merges_.find(pair_key(c.left_sym, c.right_sym))->second.result;
        b.alive = false;
        a.next = b.next;
        if (b.next >= 0) nodes[b.next].prev = c.left;
        offer(a.prev);
        offer(c.left);
    }
    const std::int32_t vocab = static_cast<std::int32_t>(vocabulary_.size());
    for (std::int32_t i = 0; i >= 0; i = nodes[i].next) {
        const std::int32_t sym = nodes[i].sym;
        if (sym < vocab) {
            out.push_back(sym);
            continue;
        }
        // Not a vocabulary string: one token per byte symbol, each of which
        // must be in the vocabulary.
        const std::string& str = extra_symbols_[static_cast<std::size_t>(sym - vocab)];
        const auto* b = reinterpret_cast<const unsigned char*>(str.data());
        for (std::size_t p = 0; p < str.size();) {
            const Cp c = utf8_at(b, str.size(), p);
            std::string one;
            put_utf8(c.value, one);
            const std::int32_t t = id(one);
            if (t < 0) throw std::runtime_error("tokenizer vocabulary is missing piece: " + str);
            out.push_back(t);
            p += c.length;
        }
    }
}

void QwenTokenizer::encode_ordinary(const std::string& text, std::size_t begin, std::size_t end,
                                    std::vector<std::int32_t>& out) const {
    const std::string part = text.substr(begin, end - begin);
    const auto* b = reinterpret_cast<const unsigned char*>(part.data());
    for (const auto& r : pieces(part)) encode_piece(b + r.first, r.second - r.first, out);
}

std::vector<std::int32_t> QwenTokenizer::encode(const std::string& text) const {
    std::vector<std::int32_t> out;
    std::size_t pos = 0;
    while (pos < text.size()) {
        std::int32_t tok;
        if (const std::size_t len = special_at(text, pos, &tok)) {
            out.push_back(tok);
            pos += len;
            continue;
        }
        const std::size_t stop = next_special(text, pos + 1);
        encode_ordinary(text, pos, stop, out);
        pos = stop;
    }
    return out;
}

std::string chat_prompt(const std::string& system, const std::string& user) {
    std::string p;
    p.reserve(system.size() + user.size() + 64);
    p += "<|im_start|>system\n";
    p += system;
    p += "<|im_end|>\n<|im_start|>user\n";
    p += user;
    p += "<|im_end|>\n<|im_start|>assistant\n";
    return p;
}

}  // namespace llm
