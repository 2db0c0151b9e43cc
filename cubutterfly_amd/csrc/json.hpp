// Minimal strict JSON DOM for the C ABI's configuration strings (RNS plan
// config and mapping records, descriptor JSON). Integers keep full uint64
// precision; object member order is preserved; duplicate keys, trailing data
// and non-finite numbers are rejected with std::invalid_argument.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace cbw::json {

struct Value {
    enum class Kind { Null, Bool, Number, String, Array, Object } kind = Kind::Null;
    bool boolean = false;
    // Numbers: `text` is the literal; integral literals also set `is_integer`
    // and hold their value in `integer` (negative flag separate).
    std::string text;
    bool is_integer = false, negative = false;
    std::uint64_t integer = 0;
    double number = 0.0;
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;

    bool is_object() const { return kind == Kind::Object; }
    bool is_array() const { return kind == Kind::Array; }
    const Value* find(const std::string& key) const;
    const Value& at(const std::string& key) const;  // throws if absent
    std::uint64_t as_u64(const char* field) const;  // nonnegative integer
    bool as_bool(const char* field) const;
    const std::string& as_string(const char* field) const;
    double as_double(const char* field) const;
};

Value parse(const std::string& text);

// Serialisation helpers: a tiny ordered builder.
std::string quote(const std::string& text);

class Writer {
  public:
    Writer& begin_object();
    Writer& end_object();
    Writer& begin_array(const char* key = nullptr);
    Writer& end_array();
    Writer& key(const char* name);
    Writer& value_raw(const std::string& raw);
    Writer& value(const std::string& text) { return value_raw(quote(text)); }
    Writer& value(const char* text) { return value_raw(quote(text)); }
    Writer& value(std::uint64_t v) { return value_raw(std::to_string(v)); }
    Writer& value(std::int64_t v) { return value_raw(std::to_string(v)); }
    Writer& value(unsigned v) { return value_raw(std::to_string(v)); }
    Writer& value(int v) { return value_raw(std::to_string(v)); }
    Writer& value(bool v) { return value_raw(v ? "true" : "false"); }
    Writer& value(double v);
    template <class T>
    Writer& field(const char* name, const T& v) { return key(name).value(v); }
    const std::string& str() const { return out_; }

  private:
    void separator();
    std::string out_;
    std::vector<bool> first_;  // per open container: no element written yet
    bool after_key_ = false;
};

}  // namespace cbw::json
