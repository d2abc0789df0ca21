// json.hpp — minimal JSON value, parser and writer for the C ABI's parameter
// strings (CAPI.swift:9-37) and the model file (Booster.swift:2119-2162).
#pragma once
#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mbjson {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;                 // string value, or a number's source text
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    const Value *get(const std::string &key) const {
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class Parser {
  public:
    explicit Parser(const std::string &s) : s_(s) {}
    Value parse() {
        Value v = value();
        ws();
        if (p_ != s_.size()) fail("trailing characters");
        return v;
    }

  private:
    const std::string &s_;
    size_t p_ = 0;

    [[noreturn]] void fail(const char *what) {
        throw std::runtime_error(std::string("JSON parse error at offset ") + std::to_string(p_) +
                                 ": " + what);
    }
    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\n' || s_[p_] == '\t' || s_[p_] == '\r'))
            ++p_;
    }
    bool lit(const char *w) {
        size_t n = std::strlen(w);
        if (s_.compare(p_, n, w) == 0) { p_ += n; return true; }
        return false;
    }
    Value value() {
        ws();
        if (p_ >= s_.size()) fail("unexpected end");
        char c = s_[p_];
        Value v;
        if (c == '{') {
            v.kind = Value::Object;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == '}') { ++p_; return v; }
            for (;;) {
                ws();
                if (p_ >= s_.size() || s_[p_] != '"') fail("expected key");
                std::string k = string();
                ws();
                if (p_ >= s_.size() || s_[p_] != ':') fail("expected ':'");
                ++p_;
                Value item = value();
                v.obj.emplace_back(std::move(k), std::move(item));
                ws();
                if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
                if (p_ < s_.size() && s_[p_] == '}') { ++p_; break; }
                fail("expected ',' or '}'");
            }
        } else if (c == '[') {
            v.kind = Value::Array;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == ']') { ++p_; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
                if (p_ < s_.size() && s_[p_] == ']') { ++p_; break; }
                fail("expected ',' or ']'");
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
            v.kind = Value::Number;
            size_t start = p_;
            while (p_ < s_.size() && (std::isdigit((unsigned char)s_[p_]) || s_[p_] == '-' ||
                                      s_[p_] == '+' || s_[p_] == '.' || s_[p_] == 'e' || s_[p_] == 'E'))
                ++p_;
            if (start == p_) fail("unexpected character");
            double d = 0;
            auto r = std::from_chars(s_.data() + start, s_.data() + p_, d);
            if (r.ec != std::errc() || r.ptr != s_.data() + p_) fail("bad number");
            v.num = d;
            v.str.assign(s_.data() + start, p_ - start);
        }
        return v;
    }
    std::string string() {
        ++p_;   // opening quote
        std::string out;
        while (p_ < s_.size() && s_[p_] != '"') {
            char c = s_[p_++];
            if (c != '\\') { out.push_back(c); continue; }
            if (p_ >= s_.size()) fail("bad escape");
            char e = s_[p_++];
            switch (e) {
            case '"': out.push_back('"'); break;
            case '\\': out.push_back('\\'); break;
            case '/': out.push_back('/'); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                if (p_ + 4 > s_.size()) fail("bad \\u escape");
                unsigned cp = (unsigned)std::stoul(s_.substr(p_, 4), nullptr, 16);
                p_ += 4;
                if (cp >= 0xD800 && cp <= 0xDBFF && p_ + 6 <= s_.size() && s_[p_] == '\\' &&
                    s_[p_ + 1] == 'u') {
                    unsigned lo = (unsigned)std::stoul(s_.substr(p_ + 2, 4), nullptr, 16);
                    p_ += 6;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                if (cp < 0x80) out.push_back((char)cp);
                else if (cp < 0x800) { out.push_back((char)(0xC0 | (cp >> 6))); out.push_back((char)(0x80 | (cp & 0x3F))); }
                else if (cp < 0x10000) {
                    out.push_back((char)(0xE0 | (cp >> 12)));
                    out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                    out.push_back((char)(0x80 | (cp & 0x3F)));
                } else {
                    out.push_back((char)(0xF0 | (cp >> 18)));
                    out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
                    out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                    out.push_back((char)(0x80 | (cp & 0x3F)));
                }
                break;
            }
            default: fail("bad escape");
            }
        }
        if (p_ >= s_.size()) fail("unterminated string");
        ++p_;
        return out;
    }
};

inline Value parse(const std::string &s) { return Parser(s).parse(); }

// A number parsed straight from its text as f32 (no double rounding).
inline float as_float(const Value &v) {
    if (v.kind != Value::Number) throw std::runtime_error("expected a number");
    float f = 0;
    auto r = std::from_chars(v.str.data(), v.str.data() + v.str.size(), f);
    if (r.ec != std::errc()) return (float)v.num;
    return f;
}

// Shortest round-trip decimal for a float (what Swift's JSONEncoder emits).
inline void put_float(std::string &out, float f) {
    if (!std::isfinite(f)) throw std::runtime_error("non-finite float in model");
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof buf, f);
    out.append(buf, r.ptr);
}

inline void put_string(std::string &out, const std::string &s) {
    out.push_back('"');
    for (unsigned char c : s) {
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20) {
                char b[8];
                std::snprintf(b, sizeof b, "\\u%04x", c);
                out += b;
            } else {
                out.push_back((char)c);
            }
        }
    }
    out.push_back('"');
}

}  // namespace mbjson
