// Text side of the token loop: the PLaMo unigram tokenizer (Tokenizer.swift:11-282).
// Host C++ only (no device code).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace plamo {

class Tokenizer {
  public:
    static constexpr int VOCAB_SIZE = 107520;

    // Loads a tokenizer.jsonl vocabulary: one JSON array [piece, score, kind] per line
    // (Tokenizer.swift:12-23,59-106).  Throws Error(E_IO / E_FORMAT) with the reference's
    // messages for invalid byte tokens, scores and vocabularies.
    explicit Tokenizer(const std::string& path);

    // Unigram Viterbi over Unicode scalars with byte fallback (Tokenizer.swift:144-190).
    // `text` must be valid UTF-8.
    std::vector<int32_t> encode(const std::string& text, bool bos) const;

    // Raw bytes of one token (Tokenizer.swift:203-225); throws on an out-of-range id.
    void append_bytes(int32_t id, std::string& out) const;

    int size() const { return int(pieces_.size()); }

  private:
    std::vector<std::string> pieces_;                // UTF-8 piece of every id
    std::vector<int64_t> scores_;                    // round(score * 1e4), 0 for BYTE tokens
    std::vector<int32_t> byte_token_ = std::vector<int32_t>(256, -1);
    // Trie over Unicode scalars: child(node, scalar) in one hash map; token of each node
    std::unordered_map<uint64_t, int32_t> child_;
    std::vector<int32_t> token_ = std::vector<int32_t>(1, -1);  // node 0 is the root

    void add(const std::string& piece, double score, const std::string& kind, int line);
    int32_t child(int32_t node, uint32_t scalar) const {
        const auto it = child_.find((uint64_t(uint32_t(node)) << 32) | scalar);
        return it == child_.end() ? -1 : it->second;
    }
};

// Incremental decoding that holds back an unfinished trailing UTF-8 sequence
// (Tokenizer.swift:236-269): the concatenated outputs equal the decode of all ids.
class TokenStream {
  public:
    explicit TokenStream(const Tokenizer& t) : tok_(t) {}
    std::string push(int32_t id);
    std::string finish();

  private:
    const Tokenizer& tok_;
    std::string pending_;
};

// The translation prompt (Tokenizer.swift:272-281).
std::string translation_prompt(const std::string& text, const std::string& target);

// UTF-8 helpers shared with the C ABI: decode to scalars (false on invalid input) and encode.
bool utf8_scalars(const std::string& s, std::vector<uint32_t>& out);
void utf8_append(std::string& out, uint32_t cp);

}  // namespace plamo
