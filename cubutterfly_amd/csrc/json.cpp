// Strict recursive-descent JSON reader (RFC 8259 grammar) and ordered writer.
#include "json.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <stdexcept>

namespace cbw::json {
namespace {

[[noreturn]] void fail(const std::string& what, std::size_t at) {
    throw std::invalid_argument("invalid JSON (" + what + ") at offset " + std::to_string(at));
}

class Parser {
  public:
    explicit Parser(const std::string& text) : s_(text) {}
    Value document() {
        skip();
        Value v = value(0);
        skip();
        if (i_ != s_.size()) fail("trailing data", i_);
        return v;
    }

  private:
    void skip() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    bool literal(const char* word) {
        std::size_t n = 0;
        while (word[n]) ++n;
        if (s_.compare(i_, n, word) == 0) {
            i_ += n;
            return true;
        }
        return false;
    }
    Value value(int depth) {
        if (depth > 64) fail("nesting too deep", i_);
        if (i_ >= s_.size()) fail("unexpected end", i_);
        Value v;
        const char c = s_[i_];
        if (c == '{') {
            v.kind = Value::Kind::Object;
            ++i_;
            skip();
            if (i_ < s_.size() && s_[i_] == '}') {
                ++i_;
                return v;
            }
            for (;;) {
                skip();
                if (i_ >= s_.size() || s_[i_] != '"') fail("expected key", i_);
                std::string k = string();
                for (const auto& m : v.members)
                    if (m.first == k) fail("duplicate key " + k, i_);
                skip();
                if (i_ >= s_.size() || s_[i_] != ':') fail("expected ':'", i_);
                ++i_;
                skip();
                v.members.emplace_back(std::move(k), value(depth + 1));
                skip();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == '}') {
                    ++i_;
                    return v;
                }
                fail("expected ',' or '}'", i_);
            }
        }
        if (c == '[') {
            v.kind = Value::Kind::Array;
            ++i_;
            skip();
            if (i_ < s_.size() && s_[i_] == ']') {
                ++i_;
                return v;
            }
            for (;;) {
                skip();
                v.items.push_back(value(depth + 1));
                skip();
                if (i_ < s_.size() && s_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < s_.size() && s_[i_] == ']') {
                    ++i_;
                    return v;
                }
                fail("expected ',' or ']'", i_);
            }
        }
        if (c == '"') {
            v.kind = Value::Kind::String;
            v.text = string();
            return v;
        }
        if (literal("true")) {
            v.kind = Value::Kind::Bool;
            v.boolean = true;
            return v;
        }
        if (literal("false")) {
            v.kind = Value::Kind::Bool;
            return v;
        }
        if (literal("null")) return v;
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        fail("unexpected character", i_);
    }
    std::string string() {
        ++i_;  // opening quote
        std::string out;
        while (i_ < s_.size()) {
            const char c = s_[i_++];
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in string", i_);
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (i_ >= s_.size()) break;
            const char e = s_[i_++];
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
                    if (i_ + 4 > s_.size()) fail("short \\u escape", i_);
                    unsigned code = 0;
                    for (int k = 0; k < 4; ++k) {
                        const char h = s_[i_++];
                        code <<= 4;
                        if (h >= '0' && h <= '9') code |= unsigned(h - '0');
                        else if (h >= 'a' && h <= 'f') code |= unsigned(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') code |= unsigned(h - 'A' + 10);
                        else fail("bad \\u escape", i_);
                    }
                    if (code >= 0xD800 && code <= 0xDFFF) fail("surrogate escapes unsupported", i_);
                    if (code < 0x80) out.push_back(char(code));
                    else if (code < 0x800) {
                        out.push_back(char(0xC0 | (code >> 6)));
                        out.push_back(char(0x80 | (code & 0x3F)));
                    } else {
                        out.push_back(char(0xE0 | (code >> 12)));
                        out.push_back(char(0x80 | ((code >> 6) & 0x3F)));
                        out.push_back(char(0x80 | (code & 0x3F)));
                    }
                    break;
                }
                default: fail("bad escape", i_);
            }
        }
        fail("unterminated string", i_);
    }
    Value number() {
        const std::size_t start = i_;
        Value v;
        v.kind = Value::Kind::Number;
        if (s_[i_] == '-') ++i_;
        if (i_ >= s_.size()) fail("bad number", i_);
        if (s_[i_] == '0') {
            ++i_;
        } else if (s_[i_] >= '1' && s_[i_] <= '9') {
            while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
        } else {
            fail("bad number", i_);
        }
        bool integral = true;
        if (i_ < s_.size() && s_[i_] == '.') {
            integral = false;
            ++i_;
            if (i_ >= s_.size() || s_[i_] < '0' || s_[i_] > '9') fail("bad fraction", i_);
            while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
        }
        if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
            integral = false;
            ++i_;
            if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
            if (i_ >= s_.size() || s_[i_] < '0' || s_[i_] > '9') fail("bad exponent", i_);
            while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
        }
        v.text = s_.substr(start, i_ - start);
        v.number = std::strtod(v.text.c_str(), nullptr);
        if (!std::isfinite(v.number)) fail("non-finite number", start);
        if (integral) {
            v.negative = v.text[0] == '-';
            std::uint64_t acc = 0;
            bool overflow = false;
            for (std::size_t k = v.negative ? 1 : 0; k < v.text.size(); ++k) {
                const unsigned d = unsigned(v.text[k] - '0');
                if (acc > (std::numeric_limits<std::uint64_t>::max() - d) / 10) overflow = true;
                acc = acc * 10 + d;
            }
            v.is_integer = !overflow;
            v.integer = acc;
        }
        return v;
    }
    const std::string& s_;
    std::size_t i_ = 0;
};

}  // namespace

Value parse(const std::string& text) { return Parser(text).document(); }

const Value* Value::find(const std::string& key) const {
    for (const auto& m : members)
        if (m.first == key) return &m.second;
    return nullptr;
}
const Value& Value::at(const std::string& key) const {
    if (kind != Kind::Object) throw std::invalid_argument("JSON value is not an object");
    const Value* v = find(key);
    if (!v) throw std::invalid_argument("missing JSON field: " + key);
    return *v;
}
std::uint64_t Value::as_u64(const char* field) const {
    if (kind != Kind::Number || !is_integer || (negative && integer != 0))
        throw std::invalid_argument(std::string("JSON field ") + field + " must be a nonnegative integer");
    return integer;
}
bool Value::as_bool(const char* field) const {
    if (kind != Kind::Bool) throw std::invalid_argument(std::string("JSON field ") + field + " must be boolean");
    return boolean;
}
const std::string& Value::as_string(const char* field) const {
    if (kind != Kind::String) throw std::invalid_argument(std::string("JSON field ") + field + " must be a string");
    return text;
}
double Value::as_double(const char* field) const {
    if (kind != Kind::Number) throw std::invalid_argument(std::string("JSON field ") + field + " must be a number");
    return number;
}

std::string quote(const std::string& text) {
    std::string out = "\"";
    for (const unsigned char c : text) {
        if (c == '"') out += "\\\"";
        else if (c == '\\') out += "\\\\";
        else if (c == '\n') out += "\\n";
        else if (c == '\t') out += "\\t";
        else if (c < 0x20) {
            char buffer[8];
            std::snprintf(buffer, sizeof buffer, "\\u%04x", c);
            out += buffer;
        } else {
            out.push_back(char(c));
        }
    }
    return out + "\"";
}

void Writer::separator() {
    if (after_key_) {
        after_key_ = false;
        return;
    }
    if (!first_.empty()) {
        if (!first_.back()) out_ += ",";
        first_.back() = false;
    }
}
Writer& Writer::begin_object() {
    separator();
    out_ += "{";
    first_.push_back(true);
    return *this;
}
Writer& Writer::end_object() {
    out_ += "}";
    first_.pop_back();
    return *this;
}
Writer& Writer::begin_array(const char* name) {
    if (name) key(name);
    separator();
    out_ += "[";
    first_.push_back(true);
    return *this;
}
Writer& Writer::end_array() {
    out_ += "]";
    first_.pop_back();
    return *this;
}
Writer& Writer::key(const char* name) {
    separator();
    out_ += quote(name) + ":";
    after_key_ = true;
    return *this;
}
Writer& Writer::value_raw(const std::string& raw) {
    separator();
    out_ += raw;
    return *this;
}
Writer& Writer::value(double v) {
    if (!std::isfinite(v)) throw std::invalid_argument("JSON cannot represent non-finite numbers");
    char buffer[40];
    std::snprintf(buffer, sizeof buffer, "%.17g", v);
    std::string text = buffer;
    if (text.find_first_of(".eE") == std::string::npos) text += ".0";
    return value_raw(text);
}

}  // namespace cbw::json
