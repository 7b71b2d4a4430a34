// Text side of the token loop: the PLaMo unigram tokenizer (Tokenizer.swift:11-282).
// Host C++ only (no device code).
#pragma once

#include <cstdint>
#include <functional>
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
    // Bytes push(id) would return, without changing the stream (callers with a bounded
    // output buffer check the size first, so a failed call leaves the stream as it was).
    size_t push_size(int32_t id) const;
    size_t finish_size() const { return pending_.size(); }

  private:
    const Tokenizer& tok_;
    std::string pending_;
};

// Emits up to four documents' streamed tokens in document order (OrderedOutput.swift:24-67):
// the first unfinished document streams through; later ones buffer until every earlier one
// has stopped; a document ending on "length" closes the output (later documents and the
// tail are dropped).  Every emitted chunk is repaired UTF-8, as Swift's String(decoding:)
// does to each chunk.
class OrderedOutput {
  public:
    using Emit = std::function<void(const std::string&)>;
    OrderedOutput(const Tokenizer& t, std::vector<std::string> prefixes, std::string tail, Emit emit);
    void append(int lane, int32_t id);
    void finish(int lane, const std::string& reason);

  private:
    std::vector<std::string> prefixes_, buffers_, reasons_;
    std::string tail_;
    std::vector<TokenStream> streams_;
    Emit emit_;
    size_t first_ = 0;
    bool closed_ = false;
    void push(int lane, const std::string& text);
};

// One piece of a source document (Segments.swift:4-7): text to translate with its prompt
// tokens, or a whitespace run kept verbatim (no tokens).
struct Segment {
    std::string text;
    std::vector<int32_t> tokens;
};

// DocumentPlan (OrderedOutput.swift:3-21): the documents to translate (segments with tokens)
// and the text emitted before each of them: the whitespace runs since the previous document,
// or "\n" between two adjacent documents; the trailing run is the tail.  No document at all
// is an error ("No documents to translate").
struct DocumentPlan {
    std::vector<std::vector<int32_t>> inputs;
    std::vector<std::string> prefixes;
    std::string tail;
    explicit DocumentPlan(const std::vector<Segment>& parts);
};

// UTF-8 with every ill-formed sequence replaced by U+FFFD, one per maximal subpart.
std::string utf8_repair(const std::string& bytes);

// The translation prompt (Tokenizer.swift:272-281).
std::string translation_prompt(const std::string& text, const std::string& target);

// UTF-8 helpers shared with the C ABI: decode to scalars (false on invalid input) and encode.
bool utf8_scalars(const std::string& s, std::vector<uint32_t>& out);
void utf8_append(std::string& out, uint32_t cp);

}  // namespace plamo
