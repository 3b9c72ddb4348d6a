// Minimal JSON document model for plan.json and target descriptions.
// Numbers keep whether they were written as integers (signed or unsigned) so the
// loader can reject "1.0" where the format requires an integer, as the reference
// loader does through nlohmann::json (tileinfer/src/runtime/plan.cpp:63-87).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace tiles {

class Json {
  public:
    enum class Kind { null, boolean, integer, unsigned_integer, real, string, array, object };

    Json() = default;
    static Json null() { return Json(); }
    static Json boolean(bool v) { Json j; j.kind_ = Kind::boolean; j.b_ = v; return j; }
    static Json integer(std::int64_t v);
    static Json uinteger(std::uint64_t v);
    static Json real(double v) { Json j; j.kind_ = Kind::real; j.d_ = v; return j; }
    static Json string(std::string v) { Json j; j.kind_ = Kind::string; j.s_ = std::move(v); return j; }
    static Json array() { Json j; j.kind_ = Kind::array; return j; }
    static Json object() { Json j; j.kind_ = Kind::object; return j; }

    static Json parse(std::string_view text);

    Kind kind() const { return kind_; }
    bool is_null() const { return kind_ == Kind::null; }
    bool is_bool() const { return kind_ == Kind::boolean; }
    bool is_integer() const { return kind_ == Kind::integer || kind_ == Kind::unsigned_integer; }
    bool is_unsigned() const { return kind_ == Kind::unsigned_integer || (kind_ == Kind::integer && i_ >= 0); }
    bool is_number() const { return is_integer() || kind_ == Kind::real; }
    bool is_string() const { return kind_ == Kind::string; }
    bool is_array() const { return kind_ == Kind::array; }
    bool is_object() const { return kind_ == Kind::object; }

    bool as_bool() const;
    std::int64_t as_int() const;     // integer that fits int64
    std::uint64_t as_uint() const;   // non-negative integer
    double as_double() const;        // any number
    const std::string& as_string() const;

    // Arrays
    std::size_t size() const;
    const Json& operator[](std::size_t index) const;
    Json& push_back(Json value);
    const std::vector<Json>& items() const;

    // Objects
    bool contains(const std::string& key) const;
    const Json& at(const std::string& key) const;  // throws "missing field <key>"
    Json& set(const std::string& key, Json value);
    const std::map<std::string, Json>& fields() const;

    bool operator==(const Json& other) const;
    bool operator!=(const Json& other) const { return !(*this == other); }

    // Serializes with sorted keys; indent < 0 gives compact output.
    std::string dump(int indent = -1) const;

  private:
    void dump_to(std::string& out, int indent, int depth) const;
    Kind kind_ = Kind::null;
    bool b_ = false;
    std::int64_t i_ = 0;
    std::uint64_t u_ = 0;
    double d_ = 0.0;
    std::string s_;
    std::vector<Json> a_;
    std::map<std::string, Json> o_;
};

} // namespace tiles
