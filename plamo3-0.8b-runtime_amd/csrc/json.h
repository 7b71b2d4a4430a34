// Minimal JSON reader for safetensors / .p12 headers and the model config files.
// Parses the full RFC 8259 grammar into a small value tree; numbers keep both the double
// value and whether the literal was an integer (config validation compares integers and
// doubles separately, as JSONSerialization does in Runtime.swift:184-188).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace plamo {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    bool integer = false;
    int64_t i = 0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;
    std::vector<std::string> keys;  // object keys in document order

    const Value* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(key);
        return it == obj.end() ? nullptr : &it->second;
    }
    bool is_int() const { return kind == Number && integer; }
};

class Parser {
  public:
    Parser(const char* p, size_t n) : p_(p), end_(p + n) {}
    Value parse() {
        Value v = value();
        ws();
        if (p_ != end_) fail();
        return v;
    }

  private:
    const char* p_;
    const char* end_;
    int depth_ = 0;
    [[noreturn]] void fail() { throw std::runtime_error("invalid JSON"); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool lit(const char* s) {
        const char* q = p_;
        for (; *s; ++s, ++q)
            if (q >= end_ || *q != *s) return false;
        p_ = q;
        return true;
    }
    Value value() {
        ws();
        if (p_ >= end_) fail();
        if (++depth_ > 64) fail();
        Value v;
        char c = *p_;
        if (c == '{') {
            v.kind = Value::Object;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; --depth_; return v; }
            for (;;) {
                ws();
                if (p_ >= end_ || *p_ != '"') fail();
                std::string k = string();
                ws();
                if (p_ >= end_ || *p_ != ':') fail();
                ++p_;
                if (!v.obj.count(k)) v.keys.push_back(k);
                v.obj[k] = value();
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; break; }
                fail();
            }
        } else if (c == '[') {
            v.kind = Value::Array;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; --depth_; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; break; }
                fail();
            }
        } else if (c == '"') {
            v.kind = Value::String;
            v.str = string();
        } else if (lit("true")) {
            v.kind = Value::Bool; v.b = true;
        } else if (lit("false")) {
            v.kind = Value::Bool; v.b = false;
        } else if (lit("null")) {
            v.kind = Value::Null;
        } else {
            number(v);
        }
        --depth_;
        return v;
    }
    void number(Value& v) {
        const char* s = p_;
        bool integer = true;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail();
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            integer = false;
            ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail();
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integer = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail();
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        std::string text(s, p_);
        v.kind = Value::Number;
        v.num = std::stod(text);
        v.integer = integer && text.size() < 19;
        if (v.integer) v.i = std::stoll(text);
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) out += char(cp);
        else if (cp < 0x800) { out += char(0xC0 | (cp >> 6)); out += char(0x80 | (cp & 63)); }
        else if (cp < 0x10000) {
            out += char(0xE0 | (cp >> 12)); out += char(0x80 | ((cp >> 6) & 63)); out += char(0x80 | (cp & 63));
        } else {
            out += char(0xF0 | (cp >> 18)); out += char(0x80 | ((cp >> 12) & 63));
            out += char(0x80 | ((cp >> 6) & 63)); out += char(0x80 | (cp & 63));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail();
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else fail();
        }
        return v;
    }
    std::string string() {
        ++p_;  // opening quote
        std::string out;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= end_) fail();
                char e = *p_++;
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        uint32_t cp = hex4();
                        if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                            p_ += 2;
                            uint32_t lo = hex4();
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        }
                        utf8(out, cp);
                        break;
                    }
                    default: fail();
                }
            } else {
                if ((unsigned char)c < 0x20) fail();
                out += c;
            }
        }
        if (p_ >= end_) fail();
        ++p_;
        return out;
    }
};

inline Value parse(const char* p, size_t n) { return Parser(p, n).parse(); }
inline Value parse(const std::string& s) { return parse(s.data(), s.size()); }

}  // namespace json
}  // namespace plamo
