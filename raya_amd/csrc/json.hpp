// Minimal JSON reader for the checkpoint configs and the safetensors header.
//
// Objects keep every key in file order, duplicates included, so a caller can
// report duplicate tensor names the way raya-weights does
// (crates/raya-weights/src/store.rs:239-281).  Numbers keep whether they were
// written as a non-negative integer (serde_json's is_u64) next to their value.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace raya {
namespace json {

struct Value;
using Object = std::vector<std::pair<std::string, Value>>;
using Array = std::vector<Value>;

struct Value {
    enum Kind { Null, Bool, Number, String, ArrayK, ObjectK } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_u64 = false;
    uint64_t u64 = 0;
    std::string str;  // String value, or the literal text of a Number
    std::shared_ptr<Array> arr;
    std::shared_ptr<Object> obj;

    bool is_null() const { return kind == Null; }
    bool is_number() const { return kind == Number; }
    bool is_string() const { return kind == String; }
    bool is_bool() const { return kind == Bool; }
    bool is_array() const { return kind == ArrayK; }
    bool is_object() const { return kind == ObjectK; }

    // Last value stored under `key` (serde_json keeps the last duplicate), or nullptr.
    const Value *get(const std::string &key) const {
        if (kind != ObjectK) return nullptr;
        const Value *found = nullptr;
        for (const auto &kv : *obj)
            if (kv.first == key) found = &kv.second;
        return found;
    }
    // Present and not null, as the reference's check_types reads a key.
    const Value *field(const std::string &key) const {
        const Value *v = get(key);
        return (v && !v->is_null()) ? v : nullptr;
    }
    std::string dump() const;
};

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n), begin_(p) {}

    Value parse_document() {
        Value v = parse_value(0);
        skip_ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

  private:
    const char *p_, *end_, *begin_;

    [[noreturn]] void fail(const char *what) {
        throw ParseError(std::string(what) + " at byte " + std::to_string(p_ - begin_));
    }
    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool literal(const char *word) {
        const char *q = p_;
        for (; *word; ++word, ++q)
            if (q >= end_ || *q != *word) return false;
        p_ = q;
        return true;
    }
    static void put_utf8(std::string &s, uint32_t c) {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("truncated \\u escape");
        uint32_t c = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            const char h = *p_;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= h - '0';
            else if (h >= 'a' && h <= 'f') c |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') c |= h - 'A' + 10;
            else fail("bad \\u escape");
        }
        return c;
    }
    std::string parse_string() {
        ++p_;  // opening quote
        std::string s;
        while (true) {
            if (p_ >= end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) fail("unterminated escape");
            const char e = *p_++;
            switch (e) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t c1 = hex4();
                if (c1 >= 0xD800 && c1 < 0xDC00) {
                    if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') fail("lone surrogate");
                    p_ += 2;
                    const uint32_t c2 = hex4();
                    if (c2 < 0xDC00 || c2 >= 0xE000) fail("bad surrogate pair");
                    c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                }
                put_utf8(s, c1);
                break;
            }
            default: fail("bad escape");
            }
        }
        return s;
    }
    Value parse_number() {
        const char *start = p_;
        bool integral = true, negative = false;
        if (*p_ == '-') {
            negative = true;
            ++p_;
        }
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad number");
        if (*p_ == '0') ++p_;
        else
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        Value v;
        v.kind = Value::Number;
        v.str.assign(start, p_);
        v.num = std::strtod(v.str.c_str(), nullptr);
        if (integral && !negative) {
            // serde_json: a non-negative integer literal that fits u64
            uint64_t acc = 0;
            bool fits = true;
            for (const char c : v.str) {
                const uint64_t d = (uint64_t)(c - '0');
                if (acc > (UINT64_MAX - d) / 10) {
                    fits = false;
                    break;
                }
                acc = acc * 10 + d;
            }
            v.is_u64 = fits;
            v.u64 = acc;
        }
        return v;
    }
    Value parse_value(int depth) {
        if (depth > 128) fail("nesting too deep");
        skip_ws();
        if (p_ >= end_) fail("unexpected end of input");
        Value v;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Value::ObjectK;
            v.obj = std::make_shared<Object>();
            skip_ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return v;
            }
            while (true) {
                skip_ws();
                if (p_ >= end_ || *p_ != '"') fail("expected a key");
                std::string key = parse_string();
                skip_ws();
                if (p_ >= end_ || *p_ != ':') fail("expected ':'");
                ++p_;
                Value item = parse_value(depth + 1);
                v.obj->emplace_back(std::move(key), std::move(item));
                skip_ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    break;
                }
                fail("expected ',' or '}'");
            }
        } else if (c == '[') {
            ++p_;
            v.kind = Value::ArrayK;
            v.arr = std::make_shared<Array>();
            skip_ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return v;
            }
            while (true) {
                v.arr->push_back(parse_value(depth + 1));
                skip_ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    break;
                }
                fail("expected ',' or ']'");
            }
        } else if (c == '"') {
            v.kind = Value::String;
            v.str = parse_string();
        } else if (c == 't') {
            if (!literal("true")) fail("bad literal");
            v.kind = Value::Bool;
            v.b = true;
        } else if (c == 'f') {
            if (!literal("false")) fail("bad literal");
            v.kind = Value::Bool;
        } else if (c == 'n') {
            if (!literal("null")) fail("bad literal");
        } else {
            v = parse_number();
        }
        return v;
    }
};

inline Value parse(const std::string &text) { return Parser(text.data(), text.size()).parse_document(); }
inline Value parse(const char *p, size_t n) { return Parser(p, n).parse_document(); }

inline std::string Value::dump() const {
    switch (kind) {
    case Null: return "null";
    case Bool: return b ? "true" : "false";
    case Number: return str;
    case String: return "\"" + str + "\"";
    case ArrayK: {
        std::string s = "[";
        for (size_t i = 0; i < arr->size(); ++i) s += (i ? "," : "") + (*arr)[i].dump();
        return s + "]";
    }
    default: {
        std::string s = "{";
        for (size_t i = 0; i < obj->size(); ++i)
            s += (i ? ",\"" : "\"") + (*obj)[i].first + "\":" + (*obj)[i].second.dump();
        return s + "}";
    }
    }
}

}  // namespace json
}  // namespace raya
