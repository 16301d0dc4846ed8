// Minimal JSON reader for the CLI configs: objects, arrays, strings, numbers, true /
// false / null, with // and /* */ comments (the reference parses its stdin config with
// comments allowed, src/gpu_cli.cu:357).  Throws std::runtime_error on malformed input,
// including arrays and objects nested more than 256 deep (each level is a recursion).
#pragma once
#include <cctype>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace jsonl {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    bool has(const std::string& k) const { return kind == Object && obj.count(k) != 0; }
    const Value& at(const std::string& k) const {
        auto it = obj.find(k);
        if (kind != Object || it == obj.end()) throw std::runtime_error("missing key \"" + k + "\"");
        return it->second;
    }
    std::string as_string() const {
        if (kind != String) throw std::runtime_error("expected a string");
        return str;
    }
    double as_number() const {
        if (kind != Number) throw std::runtime_error("expected a number");
        return num;
    }
    // value(key, default) like nlohmann::json::value
    std::string value(const std::string& k, const std::string& d) const { return has(k) ? at(k).as_string() : d; }
    double value(const std::string& k, double d) const { return has(k) ? at(k).as_number() : d; }
};

class Parser {
public:
    explicit Parser(const std::string& s) : s_(s) {}
    Value parse() {
        Value v = value();
        ws();
        if (i_ != s_.size()) err("trailing characters");
        return v;
    }

private:
    const std::string& s_;
    size_t i_ = 0;
    int depth_ = 0;
    static constexpr int MAX_DEPTH = 256;
    struct Nest {  // one level of array / object nesting, for the depth limit
        Parser& p;
        explicit Nest(Parser& q) : p(q) {
            if (++p.depth_ > MAX_DEPTH) p.err("nesting deeper than 256 levels");
        }
        ~Nest() { --p.depth_; }
    };

    [[noreturn]] void err(const std::string& m) {
        throw std::runtime_error("JSON parse error at offset " + std::to_string(i_) + ": " + m);
    }
    void ws() {
        for (;;) {
            while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
            if (i_ + 1 < s_.size() && s_[i_] == '/' && s_[i_ + 1] == '/') {
                while (i_ < s_.size() && s_[i_] != '\n') ++i_;
            } else if (i_ + 1 < s_.size() && s_[i_] == '/' && s_[i_ + 1] == '*') {
                size_t e = s_.find("*/", i_ + 2);
                if (e == std::string::npos) err("unterminated comment");
                i_ = e + 2;
            } else {
                return;
            }
        }
    }
    Value value() {
        ws();
        if (i_ >= s_.size()) err("unexpected end");
        const char c = s_[i_];
        Value v;
        if (c == '{') {
            Nest nest(*this);
            v.kind = Value::Object;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == '}') {
                ++i_;
                return v;
            }
            for (;;) {
                ws();
                if (i_ >= s_.size() || s_[i_] != '"') err("expected a key");
                std::string k = string();
                ws();
                if (i_ >= s_.size() || s_[i_] != ':') err("expected ':'");
                ++i_;
                v.obj[k] = value();
                ws();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == '}') {
                    ++i_;
                    return v;
                }
                err("expected ',' or '}'");
            }
        }
        if (c == '[') {
            Nest nest(*this);
            v.kind = Value::Array;
            ++i_;
            ws();
            if (i_ < s_.size() && s_[i_] == ']') {
                ++i_;
                return v;
            }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == ']') {
                    ++i_;
                    return v;
                }
                err("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Value::String;
            v.str = string();
            return v;
        }
        if (s_.compare(i_, 4, "true") == 0) {
            i_ += 4;
            v.kind = Value::Bool;
            v.b = true;
            return v;
        }
        if (s_.compare(i_, 5, "false") == 0) {
            i_ += 5;
            v.kind = Value::Bool;
            return v;
        }
        if (s_.compare(i_, 4, "null") == 0) {
            i_ += 4;
            return v;
        }
        if (c == '-' || std::isdigit(static_cast<unsigned char>(c))) {
            const char* b = s_.c_str() + i_;
            char* e = nullptr;
            v.kind = Value::Number;
            v.num = std::strtod(b, &e);
            if (e == b) err("bad number");
            i_ += static_cast<size_t>(e - b);
            return v;
        }
        err(std::string("unexpected character '") + c + "'");
    }
    std::string string() {
        ++i_;  // opening quote
        std::string out;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) err("bad escape");
                char e = s_[i_++];
                switch (e) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'r': out += '\r'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u': {
                    if (i_ + 4 > s_.size()) err("bad \\u escape");
                    unsigned cp = static_cast<unsigned>(std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16));
                    i_ += 4;
                    if (cp < 0x80) out += static_cast<char>(cp);
                    else if (cp < 0x800) {
                        out += static_cast<char>(0xC0 | (cp >> 6));
                        out += static_cast<char>(0x80 | (cp & 0x3F));
                    } else {
                        out += static_cast<char>(0xE0 | (cp >> 12));
                        out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
                        out += static_cast<char>(0x80 | (cp & 0x3F));
                    }
                    break;
                }
                default: out += e;
                }
            } else {
                out += c;
            }
        }
        if (i_ >= s_.size()) err("unterminated string");
        ++i_;
        return out;
    }
};

inline Value parse(const std::string& s) { return Parser(s).parse(); }

}  // namespace jsonl
