// exl3_json.hpp -- a small JSON reader for the model loader: the safetensors
// header and the deployment manifest.  Objects, arrays, strings with escapes
// (\uXXXX to UTF-8, surrogate pairs joined), integers (int64, kept apart from
// reals as JSON-for-Modern-C++ does: `128` is an integer, `128.0` and `1e2` are
// not), reals, true/false/null.  Nesting is limited to 64 levels; anything
// malformed throws std::runtime_error.  Repeated object keys keep the last value.
#pragma once

#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace exl3json {

struct Value {
    enum Kind { Null, Bool, Int, Real, String, Array, Object };
    Kind kind = Null;
    bool boolean = false;
    int64_t integer = 0;
    double real = 0.0;
    std::string text;
    std::vector<Value> items;                            // Array
    std::vector<std::pair<std::string, Value>> members;  // Object, in document order

    bool is_int() const { return kind == Int; }
    bool is_string() const { return kind == String; }
    bool is_array() const { return kind == Array; }
    bool is_object() const { return kind == Object; }
    const Value *find(const std::string &key) const {
        if (kind != Object) return nullptr;
        for (const auto &m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
    const Value &at(const std::string &key) const {
        const Value *v = find(key);
        if (!v) throw std::runtime_error("JSON key not found: " + key);
        return *v;
    }
    // value equality of a number or string with a literal
    bool equals(int64_t n) const { return (kind == Int && integer == n) || (kind == Real && real == (double)n); }
    bool equals(const char *s) const { return kind == String && text == s; }
};

class Parser {
public:
    Parser(const char *begin, const char *end) : p_(begin), end_(end) {}

    Value document() {
        Value v = value(0);
        skip_ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char *p_, *end_;

    [[noreturn]] static void fail(const char *what) { throw std::runtime_error(std::string("JSON parse error: ") + what); }

    void skip_ws() {
        while (p_ != end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    char peek() {
        skip_ws();
        if (p_ == end_) fail("unexpected end");
        return *p_;
    }
    void expect(const char *word) {
        for (const char *w = word; *w; ++w, ++p_)
            if (p_ == end_ || *p_ != *w) fail("bad literal");
    }

    Value value(int depth) {
        if (depth > 64) fail("nesting too deep");
        const char c = peek();
        Value v;
        if (c == '{') {
            ++p_;
            v.kind = Value::Object;
            if (peek() == '}') {
                ++p_;
                return v;
            }
            for (;;) {
                if (peek() != '"') fail("object key must be a string");
                std::string key = string_body();
                if (peek() != ':') fail("expected ':'");
                ++p_;
                Value item = value(depth + 1);
                bool replaced = false;
                for (auto &m : v.members)
                    if (m.first == key) {
                        m.second = std::move(item);
                        replaced = true;
                        break;
                    }
                if (!replaced) v.members.emplace_back(std::move(key), std::move(item));
                const char d = peek();
                ++p_;
                if (d == '}') return v;
                if (d != ',') fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Value::Array;
            if (peek() == ']') {
                ++p_;
                return v;
            }
            for (;;) {
                v.items.push_back(value(depth + 1));
                const char d = peek();
                ++p_;
                if (d == ']') return v;
                if (d != ',') fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Value::String;
            v.text = string_body();
            return v;
        }
        if (c == 't') {
            expect("true");
            v.kind = Value::Bool;
            v.boolean = true;
            return v;
        }
        if (c == 'f') {
            expect("false");
            v.kind = Value::Bool;
            return v;
        }
        if (c == 'n') {
            expect("null");
            return v;
        }
        return number();
    }

    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            if (p_ == end_) fail("short \\u escape");
            const char h = *p_;
            v <<= 4;
            if (h >= '0' && h <= '9') v |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') v |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') v |= (uint32_t)(h - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string_body() {  // at the opening quote
        ++p_;
        std::string out;
        for (;;) {
            if (p_ == end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') return out;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ == end_) fail("unterminated escape");
            const char e = *p_++;
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
                if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
                    if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') fail("lone surrogate");
                    p_ += 2;
                    const uint32_t lo = hex4();
                    if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    fail("lone surrogate");
                }
                put_utf8(out, cp);
                break;
            }
            default: fail("bad escape");
            }
        }
    }
    Value number() {
        const char *s = p_;
        if (p_ != end_ && *p_ == '-') ++p_;
        if (p_ == end_ || *p_ < '0' || *p_ > '9') fail("bad value");
        if (*p_ == '0') {
            ++p_;
        } else {
            while (p_ != end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        bool integral = true;
        if (p_ != end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') fail("bad fraction");
            while (p_ != end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ != end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ != end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ == end_ || *p_ < '0' || *p_ > '9') fail("bad exponent");
            while (p_ != end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string tok(s, p_);
        Value v;
        if (integral) {
            errno = 0;
            char *stop = nullptr;
            const long long n = std::strtoll(tok.c_str(), &stop, 10);
            if (errno == 0 && stop && *stop == '\0') {
                v.kind = Value::Int;
                v.integer = (int64_t)n;
                return v;
            }
            // beyond int64: kept as a real, like an unsigned 64-bit or larger literal
        }
        v.kind = Value::Real;
        v.real = std::strtod(tok.c_str(), nullptr);
        return v;
    }
};

inline Value parse(const char *begin, const char *end) { return Parser(begin, end).document(); }

}  // namespace exl3json
