// PLaMo unigram tokenizer (Tokenizer.swift:11-282), host C++.
//
// Same vocabulary rules, segmentation and costs as the reference; the data structures are
// this file's own: the trie is one hash map from (node, scalar) to child, and the Viterbi
// costs live in a full array instead of a ring.  Neither changes which tokens are chosen.
#include "tokenizer.h"

#include <cmath>
#include <fstream>
#include <limits>
#include <set>
#include <sstream>

#include "common.h"
#include "json.h"

namespace plamo {

bool utf8_scalars(const std::string& s, std::vector<uint32_t>& out) {
    out.clear();
    out.reserve(s.size());
    const auto* p = reinterpret_cast<const unsigned char*>(s.data());
    const size_t n = s.size();
    for (size_t i = 0; i < n;) {
        const uint32_t c = p[i];
        uint32_t cp, need;
        if (c < 0x80) { cp = c; need = 0; }
        else if (c >= 0xC2 && c <= 0xDF) { cp = c & 0x1F; need = 1; }
        else if (c >= 0xE0 && c <= 0xEF) { cp = c & 0x0F; need = 2; }
        else if (c >= 0xF0 && c <= 0xF4) { cp = c & 0x07; need = 3; }
        else return false;
        if (need > 0 && i + need >= n) return false;  // truncated sequence
        for (uint32_t k = 1; k <= need; ++k) {
            const uint32_t d = p[i + k];
            if ((d & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (d & 0x3F);
        }
        // overlong forms, surrogates and values past U+10FFFF are not scalars
        if ((need == 2 && cp < 0x800) || (need == 3 && (cp < 0x10000 || cp > 0x10FFFF)) ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        out.push_back(cp);
        i += need + 1;
    }
    return true;
}

void utf8_append(std::string& out, uint32_t cp) {
    if (cp < 0x80) out += char(cp);
    else if (cp < 0x800) { out += char(0xC0 | (cp >> 6)); out += char(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) {
        out += char(0xE0 | (cp >> 12)); out += char(0x80 | ((cp >> 6) & 0x3F)); out += char(0x80 | (cp & 0x3F));
    } else {
        out += char(0xF0 | (cp >> 18)); out += char(0x80 | ((cp >> 12) & 0x3F));
        out += char(0x80 | ((cp >> 6) & 0x3F)); out += char(0x80 | (cp & 0x3F));
    }
}

namespace {

// "<0xNN>" with NN as Swift's Int(_:radix:16) reads it: an optional sign, then hex digits
// (Tokenizer.swift:100-101,216-217).  Returns the value or -1.
int byte_piece_value(const std::string& piece) {
    if (piece.size() != 6 || piece.compare(0, 3, "<0x") != 0 || piece[5] != '>') return -1;
    const char a = piece[3], b = piece[4];
    auto hex = [](char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    };
    if (a == '+' || a == '-') {
        const int v = hex(b);
        if (v < 0) return -1;
        return a == '-' ? (v == 0 ? 0 : -1) : v;  // negative values are out of range
    }
    const int hi = hex(a), lo = hex(b);
    return hi < 0 || lo < 0 ? -1 : hi * 16 + lo;
}

// ICU \s: [\t\n\f\r\p{Z}]
bool icu_space(uint32_t c) {
    return c == '\t' || c == '\n' || c == '\f' || c == '\r' || c == 0x20 || c == 0xA0 || c == 0x1680 ||
           (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 || c == 0x202F || c == 0x205F ||
           c == 0x3000;
}

// Length of a match of (<\|plamo:[^|\s\x1c-\x1f]{0,64}\|>)|(([^\n])\3{3,}| {2,}) at i, or 0
// (Tokenizer.swift:41-43): alternatives in order, quantifiers greedy.
size_t boundary_match(const std::vector<uint32_t>& s, size_t i) {
    const size_t n = s.size();
    static const char* open = "<|plamo:";
    size_t k = 0;
    while (k < 8 && i + k < n && s[i + k] == uint32_t(open[k])) ++k;
    if (k == 8) {
        size_t j = i + 8, run = 0;
        while (j < n && run <= 64 && s[j] != '|' && !icu_space(s[j]) && !(s[j] >= 0x1C && s[j] <= 0x1F)) ++j, ++run;
        // the class excludes '|', so fewer characters never put "|>" earlier
        if (run <= 64 && j + 1 < n && s[j] == '|' && s[j + 1] == '>') return j + 2 - i;
    }
    if (s[i] != '\n') {
        size_t j = i + 1;
        while (j < n && s[j] == s[i]) ++j;
        if (j - i >= 4) return j - i;
    }
    if (s[i] == ' ' && i + 1 < n && s[i + 1] == ' ') {
        size_t j = i;
        while (j < n && s[j] == ' ') ++j;
        return j - i;
    }
    return 0;
}

constexpr uint32_t MARK = 0xEE00;

}  // namespace

Tokenizer::Tokenizer(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error(E_IO, "Cannot read tokenizer " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    const std::string contents = ss.str();
    pieces_.reserve(VOCAB_SIZE);
    scores_.reserve(VOCAB_SIZE);
    // lines split on '\n' with empty lines skipped, as String.split does (Tokenizer.swift:85-88)
    int line = 0;
    for (size_t a = 0; a < contents.size();) {
        size_t b = contents.find('\n', a);
        if (b == std::string::npos) b = contents.size();
        ++line;
        if (b > a) {
            json::Value v;
            try {
                v = json::parse(contents.data() + a, b - a);
            } catch (const std::exception&) {
                throw Error(E_FORMAT, "Invalid tokenizer vocabulary line " + std::to_string(line));
            }
            if (v.kind != json::Value::Array || v.arr.size() < 3 || v.arr[0].kind != json::Value::String ||
                v.arr[1].kind != json::Value::Number || v.arr[2].kind != json::Value::String)
                throw Error(E_FORMAT, "Invalid tokenizer vocabulary line " + std::to_string(line));
            add(v.arr[0].str, v.arr[1].num, v.arr[2].str, line);
        }
        a = b + 1;
    }
    // Tokenizer.swift:90-95
    bool bytes_ok = true;
    for (int32_t t : byte_token_) bytes_ok = bytes_ok && t >= 0;
    if (int(pieces_.size()) != VOCAB_SIZE || !bytes_ok || pieces_[1] != "<|plamo:bos|>" || pieces_[16] != "<|plamo:tag|>")
        throw Error(E_FORMAT, "Expected the PLaMo 3 Translate 0.8B vocabulary");
}

// Tokenizer.swift:96-131
void Tokenizer::add(const std::string& piece, double score, const std::string& kind, int line) {
    const int32_t id = int32_t(pieces_.size());
    std::vector<uint32_t> scalars;
    if (!utf8_scalars(piece, scalars)) throw Error(E_FORMAT, "Invalid tokenizer vocabulary line " + std::to_string(line));
    pieces_.push_back(piece);
    if (kind == "BYTE") {
        const int byte = byte_piece_value(piece);
        if (byte < 0 || byte > 255) throw Error(E_FORMAT, "Invalid byte token");
        byte_token_[byte] = id;
        scores_.push_back(0);
        return;
    }
    const double scaled = std::nearbyint(score * 1e4);  // round half to even (default mode)
    if (!std::isfinite(scaled) || scaled < -9223372036854775808.0 || scaled >= 9223372036854775808.0)
        throw Error(E_FORMAT, "Invalid tokenizer score");
    scores_.push_back(int64_t(scaled));
    int32_t node = 0;
    for (uint32_t c : scalars) {
        int32_t next = child(node, c);
        if (next < 0) {
            next = int32_t(token_.size());
            token_.push_back(-1);
            child_.emplace((uint64_t(uint32_t(node)) << 32) | c, next);
        }
        node = next;
    }
    token_[node] = id;  // a repeated piece keeps its last id
}

// Tokenizer.swift:144-190
std::vector<int32_t> Tokenizer::encode(const std::string& text, bool bos) const {
    std::vector<uint32_t> s;
    if (!utf8_scalars(text, s)) throw Error(E_INVAL, "Invalid UTF-8 text");
    // wrap every boundary match in U+EE00, then split on U+EE00 (empty pieces dropped)
    std::vector<uint32_t> marked;
    marked.reserve(s.size() + 16);
    for (size_t i = 0; i < s.size();) {
        const size_t m = boundary_match(s, i);
        if (m) {
            marked.push_back(MARK);
            marked.insert(marked.end(), s.begin() + i, s.begin() + i + m);
            marked.push_back(MARK);
            i += m;
        } else {
            marked.push_back(s[i++]);
        }
    }
    std::vector<int32_t> out;
    if (bos) out.push_back(1);
    std::vector<int64_t> cost;
    std::vector<int32_t> len, tok;
    for (size_t a = 0; a < marked.size();) {
        if (marked[a] == MARK) { ++a; continue; }
        size_t b = a;
        while (b < marked.size() && marked[b] != MARK) ++b;
        const uint32_t* seg = marked.data() + a;
        const size_t n = b - a;
        cost.assign(n + 1, 0);
        len.assign(n, 1);
        tok.assign(n, -1);
        for (size_t i = n; i-- > 0;) {
            int64_t best = cost[i + 1] + 10000000;  // byte fallback of one scalar
            int32_t node = 0;
            for (size_t j = i; j < n; ++j) {
                node = child(node, seg[j]);
                if (node < 0) break;
                const int32_t t = token_[node];
                if (t >= 0) {
                    const int64_t c = cost[j + 1] - scores_[t];
                    if (c <= best) {  // ties go to the longer piece
                        best = c;
                        len[i] = int32_t(j - i + 1);
                        tok[i] = t;
                    }
                }
            }
            cost[i] = best;
        }
        for (size_t i = 0; i < n; i += size_t(len[i])) {
            if (tok[i] >= 0) {
                out.push_back(tok[i]);
            } else {
                std::string u;
                utf8_append(u, seg[i]);
                for (unsigned char c : u) out.push_back(byte_token_[c]);
            }
        }
        a = b;
    }
    return out;
}

// Tokenizer.swift:203-225 (vocabulary loaded from tokenizer.jsonl): a piece spelled "<0xNN>"
// is that byte, any other piece its UTF-8 text.
void Tokenizer::append_bytes(int32_t id, std::string& out) const {
    if (id < 0 || id >= int32_t(pieces_.size())) throw Error(E_INVAL, "Token ID out of range");
    const std::string& p = pieces_[size_t(id)];
    const int byte = byte_piece_value(p);
    if (byte >= 0 && byte <= 255) out += char(byte);
    else out += p;
}

namespace {
// Trailing bytes (0..3) that are a valid but unfinished UTF-8 sequence (Tokenizer.swift:257-268)
size_t incomplete_suffix(const std::string& b) {
    size_t trailer = 0, i = b.size();
    while (i > 0 && trailer < 3) {
        --i;
        const unsigned char c = (unsigned char)b[i];
        if ((c & 0xC0) == 0x80) { ++trailer; continue; }
        if (c < 0x80) return 0;
        const size_t needed = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : 2;
        return b.size() - i < needed ? b.size() - i : 0;
    }
    return 0;
}
}  // namespace

std::string TokenStream::push(int32_t id) {
    tok_.append_bytes(id, pending_);
    const size_t complete = pending_.size() - incomplete_suffix(pending_);
    std::string out = pending_.substr(0, complete);
    pending_.erase(0, complete);
    return out;
}

size_t TokenStream::push_size(int32_t id) const {
    std::string trial = pending_;
    tok_.append_bytes(id, trial);
    return trial.size() - incomplete_suffix(trial);
}

std::string TokenStream::finish() {
    std::string out;
    out.swap(pending_);
    return out;
}

std::string utf8_repair(const std::string& b) {
    std::string out;
    out.reserve(b.size());
    const size_t n = b.size();
    for (size_t i = 0; i < n;) {
        const unsigned char c = (unsigned char)b[i];
        if (c < 0x80) { out += char(c); ++i; continue; }
        size_t need = 0;
        unsigned char lo = 0x80, hi = 0xBF;  // allowed range of the second byte
        if (c >= 0xC2 && c <= 0xDF) need = 1;
        else if (c >= 0xE0 && c <= 0xEF) { need = 2; if (c == 0xE0) lo = 0xA0; if (c == 0xED) hi = 0x9F; }
        else if (c >= 0xF0 && c <= 0xF4) { need = 3; if (c == 0xF0) lo = 0x90; if (c == 0xF4) hi = 0x8F; }
        size_t k = 1;
        while (k <= need && i + k < n) {
            const unsigned char d = (unsigned char)b[i + k];
            if (k == 1 ? (d < lo || d > hi) : (d & 0xC0) != 0x80) break;
            ++k;
        }
        if (need && k == need + 1) out.append(b, i, k);
        else out += "\xEF\xBF\xBD";  // the maximal subpart (at least one byte) becomes U+FFFD
        i += need && k == need + 1 ? k : (k > 1 ? k : 1);
    }
    return out;
}

DocumentPlan::DocumentPlan(const std::vector<Segment>& parts) {
    std::string pending;
    for (const Segment& part : parts) {
        if (part.tokens.empty()) {
            pending += part.text;
            continue;
        }
        prefixes.push_back(!inputs.empty() && pending.empty() ? std::string("\n") : pending);
        inputs.push_back(part.tokens);
        pending.clear();
    }
    if (inputs.empty()) throw Error(E_INVAL, "No documents to translate");
    tail = pending;
}

OrderedOutput::OrderedOutput(const Tokenizer& t, std::vector<std::string> prefixes, std::string tail, Emit emit)
    : prefixes_(std::move(prefixes)), tail_(std::move(tail)), emit_(std::move(emit)) {
    if (prefixes_.empty() || prefixes_.size() > 4) throw Error(E_INVAL, "Expected one to four output prefixes");
    buffers_.assign(prefixes_.size(), std::string());
    reasons_.assign(prefixes_.size(), std::string());
    for (size_t i = 0; i < prefixes_.size(); ++i) streams_.emplace_back(t);
    if (!prefixes_[0].empty()) emit_(prefixes_[0]);
}

void OrderedOutput::push(int lane, const std::string& bytes) {
    if (bytes.empty()) return;
    const std::string text = utf8_repair(bytes);
    if (size_t(lane) == first_) emit_(text);
    else buffers_[size_t(lane)] += text;
}

void OrderedOutput::append(int lane, int32_t id) {
    if (lane < 0 || size_t(lane) >= reasons_.size() || !reasons_[size_t(lane)].empty() || closed_)
        throw Error(E_STATE, "Output after document finish");
    push(lane, streams_[size_t(lane)].push(id));
}

void OrderedOutput::finish(int lane, const std::string& reason) {
    if (lane < 0 || size_t(lane) >= reasons_.size() || !reasons_[size_t(lane)].empty() || closed_ ||
        (reason != "stop" && reason != "length"))
        throw Error(E_STATE, "Invalid document finish");
    push(lane, streams_[size_t(lane)].finish());
    reasons_[size_t(lane)] = reason;
    while (first_ < reasons_.size() && !reasons_[first_].empty()) {
        if (reasons_[first_] != "stop") { closed_ = true; return; }
        ++first_;
        if (first_ == reasons_.size()) {
            closed_ = true;
            if (!tail_.empty()) emit_(tail_);
            return;
        }
        if (!prefixes_[first_].empty()) emit_(prefixes_[first_]);
        if (!buffers_[first_].empty()) { emit_(buffers_[first_]); buffers_[first_].clear(); }
    }
}

std::string translation_prompt(const std::string& text, const std::string& target) {
    static const std::set<std::string> languages = {
        "ar", "az", "be", "bg", "bn", "ca", "ceb", "de", "en", "es", "et", "eu", "fa", "fr", "gu", "he",
        "hi", "hr", "hu", "hy", "id", "it", "ja", "jv", "ka", "kk", "km", "ko", "lt", "lv", "ml", "mr",
        "ms", "my", "ne", "nl", "pa", "pl", "ru", "si", "sk", "sl", "sr", "sw", "ta", "te", "th", "tl",
        "ur", "uz", "vi", "zh-hans", "zh-hant"};
    if (!languages.count(target)) throw Error(E_INVAL, "Unsupported target language");
    std::vector<uint32_t> s;
    bool reserved = !utf8_scalars(text, s) || text.empty() || text.find("<|plamo:") != std::string::npos;
    for (uint32_t c : s) reserved = reserved || c == MARK;
    if (reserved) throw Error(E_INVAL, "Source must be nonempty and contain no reserved PLaMo delimiters");
    return "<|plamo:tag|>dataset<|plamo:msg|>translation<|plamo:tag|>input<|plamo:msg|>" + text +
           "<|plamo:tag|>output<|plamo:key|>lang<|plamo:val|>" + target + "<|plamo:msg|>";
}

}  // namespace plamo
