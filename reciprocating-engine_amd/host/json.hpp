// json.hpp - a small JSON reader (objects, arrays, strings, numbers, true,
// false, null) for the files this host layer reads: Hugging Face config.json,
// safetensors headers and the golden test fixture. Not a general-purpose
// library: numbers are kept as double plus the exact integer when they are
// written as one.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace reng_json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_int = false;
    int64_t i = 0;
    uint64_t u = 0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    bool has(const std::string &k) const { return kind == Object && obj.count(k) != 0; }
    const Value &operator[](const std::string &k) const {
        auto it = obj.find(k);
        if (kind != Object || it == obj.end()) throw std::runtime_error("json: missing key " + k);
        return it->second;
    }
    const Value &operator[](size_t idx) const {
        if (kind != Array || idx >= arr.size()) throw std::runtime_error("json: index out of range");
        return arr[idx];
    }
    size_t size() const { return kind == Array ? arr.size() : kind == Object ? obj.size() : 0; }
    const std::string &as_str() const {
        if (kind != String) throw std::runtime_error("json: not a string");
        return str;
    }
    double as_f64() const {
        if (kind != Number) throw std::runtime_error("json: not a number");
        return num;
    }
    uint64_t as_u64() const {
        if (kind != Number || !is_int || i < 0) throw std::runtime_error("json: not a non-negative integer");
        return u;
    }
    int64_t as_i64() const {
        if (kind != Number || !is_int) throw std::runtime_error("json: not an integer");
        return i;
    }
};

class Parser {
public:
    explicit Parser(const std::string &text) : s_(text) {}

    Value parse() {
        Value v = value();
        ws();
        if (p_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    const std::string &s_;
    size_t p_ = 0;

    [[noreturn]] void fail(const char *what) const {
        throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(p_));
    }
    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\n' || s_[p_] == '\r' || s_[p_] == '\t')) ++p_;
    }
    bool lit(const char *w) {
        size_t n = 0;
        while (w[n]) ++n;
        if (s_.compare(p_, n, w) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    Value value() {
        ws();
        if (p_ >= s_.size()) fail("unexpected end");
        const char c = s_[p_];
        Value v;
        if (c == '{') {
            v.kind = Value::Object;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == '}') {
                ++p_;
                return v;
            }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p_ >= s_.size() || s_[p_] != ':') fail("expected ':'");
                ++p_;
                v.obj.emplace(std::move(k), value());
                ws();
                if (p_ < s_.size() && s_[p_] == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < s_.size() && s_[p_] == '}') {
                    ++p_;
                    return v;
                }
                fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Value::Array;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == ']') {
                ++p_;
                return v;
            }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p_ < s_.size() && s_[p_] == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < s_.size() && s_[p_] == ']') {
                    ++p_;
                    return v;
                }
                fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Value::String;
            v.str = string();
            return v;
        }
        if (lit("true")) {
            v.kind = Value::Bool;
            v.b = true;
            return v;
        }
        if (lit("false")) {
            v.kind = Value::Bool;
            return v;
        }
        if (lit("null")) return v;
        return number();
    }
    std::string string() {
        if (p_ >= s_.size() || s_[p_] != '"') fail("expected a string");
        ++p_;
        std::string out;
        while (p_ < s_.size() && s_[p_] != '"') {
            char c = s_[p_++];
            if (c == '\\') {
                if (p_ >= s_.size()) fail("bad escape");
                const char e = s_[p_++];
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
                        if (p_ + 4 > s_.size()) fail("bad \\u escape");
                        const unsigned cp = (unsigned)std::stoul(s_.substr(p_, 4), nullptr, 16);
                        p_ += 4;
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xc0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3f));
                        } else {
                            out += (char)(0xe0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3f));
                            out += (char)(0x80 | (cp & 0x3f));
                        }
                        break;
                    }
                    default: fail("bad escape");
                }
            } else {
                out += c;
            }
        }
        if (p_ >= s_.size()) fail("unterminated string");
        ++p_;
        return out;
    }
    Value number() {
        const size_t start = p_;
        if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
        bool integral = true;
        while (p_ < s_.size()) {
            const char c = s_[p_];
            if (c >= '0' && c <= '9') {
                ++p_;
            } else if (c == '.' || c == 'e' || c == 'E' || c == '-' || c == '+') {
                integral = false;
                ++p_;
            } else {
                break;
            }
        }
        if (p_ == start) fail("unexpected character");
        const std::string t = s_.substr(start, p_ - start);
        Value v;
        v.kind = Value::Number;
        v.num = std::stod(t);
        if (integral) {
            v.is_int = true;
            if (t[0] == '-') {
                v.i = std::stoll(t);
                v.u = 0;
            } else {
                v.u = std::stoull(t);
                v.i = (int64_t)v.u;
            }
        }
        return v;
    }
};

inline Value parse(const std::string &text) { return Parser(text).parse(); }

}  // namespace reng_json
