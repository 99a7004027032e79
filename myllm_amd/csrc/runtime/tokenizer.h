// Qwen byte-level BPE tokenizer over a GGUF vocabulary and merge table.
//
// Same interface and results as the reference's QwenTokenizer
// (chat.cpp:349-529): encode / id / decode_piece / is_special, built from
// tokenizer.ggml.tokens, tokenizer.ggml.merges and tokenizer.ggml.pre
// (include_marks for "qwen35", chat.cpp:355). What is kept identical, and
// why:
// * the lenient UTF-8 decoder (chat.cpp:34-78: a malformed byte is one
//   codepoint of its own value), because it decides piece boundaries;
// * the coarse letter / mark / number / space classes (chat.cpp:101-172),
//   which stand in for Unicode \p{L}, \p{M}, \p{N}, \s: the same ranges are
//   needed to produce the same pieces;
// * the pre-tokenizer rules (chat.cpp:207-298): contractions, an optional
//   non-letter prefix on a word run, single digits, an optionally
//   space-prefixed punctuation run with trailing line breaks, whitespace runs
//   split before the last line break or before a following word;
// * the GPT-2 byte-to-symbol map, and the merge order: always the adjacent
//   pair of lowest merge rank, leftmost first (chat.cpp:459-477);
// * special tokens: every vocabulary entry "<|...|>" of at least 4 bytes,
//   matched longest first, and split out of the text before pre-tokenizing.
//
// The implementation is its own: strings are interned to integer symbols so
// that a merge is one hash lookup on a 64-bit symbol pair, and each piece is
// merged with a binary heap over (rank, position) with lazy invalidation
// instead of rescanning every pair after each merge: O(n log n) per piece
// rather than O(n^2), with the same merge sequence.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace llm {

class QwenTokenizer {
public:
    // vocabulary: token strings by id; merges: "left right" by rank;
    // tokenizer_pre: "qwen35" attaches combining marks to letter runs.
    QwenTokenizer(const std::vector<std::string>& vocabulary, const std::vector<std::string>& merges,
                  const std::string& tokenizer_pre);

    // Token ids of text: special tokens first, then byte-level BPE of every
    // pre-tokenized piece. Throws std::runtime_error when the vocabulary lacks
    // a single-byte symbol the text needs (chat.cpp:509-518).
    std::vector<std::int32_t> encode(const std::string& text) const;

    // Id of a vocabulary string, -1 when absent (first id of a duplicate).
    std::int32_t id(const std::string& token) const;

    // Bytes of one token; "" for special tokens and ids out of range.
    std::string decode_piece(std::int32_t token) const;

    bool is_special(std::int32_t token) const;

    std::size_t vocabulary_size() const noexcept { return vocabulary_.size(); }
    bool include_marks() const noexcept { return include_marks_; }

    // Byte ranges [begin, end) of the pre-tokenized pieces of ordinary text
    // (no special-token split).
    std::vector<std::pair<std::size_t, std::size_t>> pieces(const std::string& text) const;

private:
    struct Merge {
        std::uint32_t rank;
        std::int32_t result;  // symbol of the concatenation
    };

    std::int32_t intern(const std::string& s);
    std::int32_t find_symbol(const std::string& s) const;
    void encode_ordinary(const std::string& text, std::size_t begin, std::size_t end,
                         std::vector<std::int32_t>& out) const;
    void encode_piece(const unsigned char* bytes, std::size_t n, std::vector<std::int32_t>& out) const;
    std::size_t special_at(const std::string& text, std::size_t pos, std::int32_t* token) const;
    std::size_t next_special(const std::string& text, std::size_t from) const;

    std::vector<std::string> vocabulary_;
    bool include_marks_ = false;
    // Symbol table: ids [0, vocabulary size) are vocabulary ids (a duplicate
    // string keeps its first id); strings met only in merges get later ids.
    std::unordered_map<std::string, std::int32_t> symbols_;
    std::vector<std::string> extra_symbols_;
    std::unordered_map<std::uint64_t, Merge> merges_;
    std::int32_t byte_symbol_[256];
    std::vector<std::uint8_t> special_;  // by vocabulary id
    std::unordered_map<std::string, std::int32_t> special_ids_;
    std::vector<std::size_t> special_lengths_;  // distinct lengths, longest first
};

// ChatML prompt of one user turn (chat.cpp:655-659).
std::string chat_prompt(const std::string& system, const std::string& user);

}  // namespace llm
