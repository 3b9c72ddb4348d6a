#include "json.hpp"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <stdexcept>

namespace tiles {

Json Json::integer(std::int64_t v)
{
    Json j;
    j.kind_ = Kind::integer;
    j.i_ = v;
    return j;
}

Json Json::uinteger(std::uint64_t v)
{
    if (v <= static_cast<std::uint64_t>(std::numeric_limits<std::int64_t>::max()))
        return integer(static_cast<std::int64_t>(v));
    Json j;
    j.kind_ = Kind::unsigned_integer;
    j.u_ = v;
    return j;
}

namespace {
[[noreturn]] void fail(const std::string& message) { throw std::runtime_error(message); }

class Parser {
  public:
    explicit Parser(std::string_view text) : text_(text) {}

    Json document()
    {
        Json value = parse_value(0);
        skip();
        if (pos_ != text_.size())
            fail("invalid JSON: trailing characters");
        return value;
    }

  private:
    std::string_view text_;
    std::size_t pos_ = 0;

    void skip()
    {
        while (pos_ < text_.size() &&
               (text_[pos_] == ' ' || text_[pos_] == '\n' || text_[pos_] == '\r' || text_[pos_] == '\t'))
            ++pos_;
    }
    char peek()
    {
        skip();
        if (pos_ >= text_.size())
            fail("invalid JSON: unexpected end");
        return text_[pos_];
    }
    void expect(char c)
    {
        if (peek() != c)
            fail(std::string("invalid JSON: expected '") + c + "'");
        ++pos_;
    }
    bool literal(std::string_view word)
    {
        if (text_.substr(pos_, word.size()) == word) {
            pos_ += word.size();
            return true;
        }
        return false;
    }

    Json parse_value(int depth)
    {
        if (depth > 64)
            fail("invalid JSON: nesting too deep");
        const char c = peek();
        if (c == '{') {
            ++pos_;
            Json object = Json::object();
            if (peek() == '}') {
                ++pos_;
                return object;
            }
            while (true) {
                if (peek() != '"')
                    fail("invalid JSON: object key");
                std::string key = parse_string();
                expect(':');
                if (object.contains(key))
                    fail("invalid JSON: duplicate key " + key);
                object.set(key, parse_value(depth + 1));
                const char next = peek();
                ++pos_;
                if (next == '}')
                    return object;
                if (next != ',')
                    fail("invalid JSON: object separator");
            }
        }
        if (c == '[') {
            ++pos_;
            Json array = Json::array();
            if (peek() == ']') {
                ++pos_;
                return array;
            }
            while (true) {
                array.push_back(parse_value(depth + 1));
                const char next = peek();
                ++pos_;
                if (next == ']')
                    return array;
                if (next != ',')
                    fail("invalid JSON: array separator");
            }
        }
        if (c == '"')
            return Json::string(parse_string());
        if (literal("true"))
            return Json::boolean(true);
        if (literal("false"))
            return Json::boolean(false);
        if (literal("null"))
            return Json::null();
        return parse_number();
    }

    static void append_utf8(std::string& out, unsigned code)
    {
        if (code < 0x80) {
            out += static_cast<char>(code);
        } else if (code < 0x800) {
            out += static_cast<char>(0xC0 | (code >> 6));
            out += static_cast<char>(0x80 | (code & 0x3F));
        } else if (code < 0x10000) {
            out += static_cast<char>(0xE0 | (code >> 12));
            out += static_cast<char>(0x80 | ((code >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (code & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (code >> 18));
            out += static_cast<char>(0x80 | ((code >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((code >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (code & 0x3F));
        }
    }

    unsigned hex4()
    {
        if (pos_ + 4 > text_.size())
            fail("invalid JSON: escape");
        unsigned value = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = text_[pos_++];
            value <<= 4;
            if (h >= '0' && h <= '9') value |= h - '0';
            else if (h >= 'a' && h <= 'f') value |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') value |= h - 'A' + 10;
            else fail("invalid JSON: escape");
        }
        return value;
    }

    std::string parse_string()
    {
        expect('"');
        std::string out;
        while (true) {
            if (pos_ >= text_.size())
                fail("invalid JSON: unterminated string");
            const char c = text_[pos_++];
            if (c == '"')
                return out;
            if (static_cast<unsigned char>(c) < 0x20)
                fail("invalid JSON: control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (pos_ >= text_.size())
                fail("invalid JSON: escape");
            const char e = text_[pos_++];
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
                unsigned code = hex4();
                if (code >= 0xD800 && code < 0xDC00 && text_.substr(pos_, 2) == "\\u") {
                    pos_ += 2;
                    const unsigned low = hex4();
                    code = 0x10000 + ((code - 0xD800) << 10) + (low - 0xDC00);
                }
                append_utf8(out, code);
                break;
            }
            default: fail("invalid JSON: escape");
            }
        }
    }

    Json parse_number()
    {
        const std::size_t start = pos_;
        bool real = false;
        if (pos_ < text_.size() && text_[pos_] == '-')
            ++pos_;
        while (pos_ < text_.size()) {
            const char c = text_[pos_];
            if (c >= '0' && c <= '9') {
                ++pos_;
            } else if (c == '.' || c == 'e' || c == 'E' || c == '+' || c == '-') {
                real = true;
                ++pos_;
            } else {
                break;
            }
        }
        const std::string token(text_.substr(start, pos_ - start));
        if (token.empty() || token == "-")
            fail("invalid JSON: value");
        char* end = nullptr;
        if (!real) {
            errno = 0;
            if (token[0] == '-') {
                const long long v = std::strtoll(token.c_str(), &end, 10);
                if (errno == 0 && end && *end == '\0')
                    return Json::integer(v);
            } else {
                const unsigned long long v = std::strtoull(token.c_str(), &end, 10);
                if (errno == 0 && end && *end == '\0') {
                    if (v <= static_cast<unsigned long long>(std::numeric_limits<std::int64_t>::max()))
                        return Json::integer(static_cast<std::int64_t>(v));
                    return Json::uinteger(v);
                }
            }
        }
        const double v = std::strtod(token.c_str(), &end);
        if (!end || *end != '\0' || !std::isfinite(v))
            fail("invalid JSON: number");
        return Json::real(v);
    }

};
} // namespace

Json Json::parse(std::string_view text) { return Parser(text).document(); }

bool Json::as_bool() const
{
    if (kind_ != Kind::boolean)
        fail("JSON value is not a boolean");
    return b_;
}

std::int64_t Json::as_int() const
{
    if (kind_ != Kind::integer)
        fail("JSON value is not an integer");
    return i_;
}

std::uint64_t Json::as_uint() const
{
    if (kind_ == Kind::integer && i_ >= 0)
        return static_cast<std::uint64_t>(i_);
    if (kind_ == Kind::unsigned_integer)
        return u_;
    fail("JSON value is not a non-negative integer");
}

double Json::as_double() const
{
    switch (kind_) {
    case Kind::integer: return static_cast<double>(i_);
    case Kind::unsigned_integer: return static_cast<double>(u_);
    case Kind::real: return d_;
    default: fail("JSON value is not a number");
    }
}

const std::string& Json::as_string() const
{
    if (kind_ != Kind::string)
        fail("JSON value is not a string");
    return s_;
}

std::size_t Json::size() const
{
    if (kind_ == Kind::array) return a_.size();
    if (kind_ == Kind::object) return o_.size();
    fail("JSON value has no size");
}

const Json& Json::operator[](std::size_t index) const
{
    if (kind_ != Kind::array || index >= a_.size())
        fail("JSON array index outside range");
    return a_[index];
}

Json& Json::push_back(Json value)
{
    if (kind_ != Kind::array)
        fail("JSON value is not an array");
    a_.push_back(std::move(value));
    return a_.back();
}

const std::vector<Json>& Json::items() const
{
    if (kind_ != Kind::array)
        fail("JSON value is not an array");
    return a_;
}

bool Json::contains(const std::string& key) const { return kind_ == Kind::object && o_.count(key) != 0; }

const Json& Json::at(const std::string& key) const
{
    if (kind_ != Kind::object)
        fail("JSON value is not an object (looking up " + key + ")");
    const auto found = o_.find(key);
    if (found == o_.end())
        fail("missing field " + key);
    return found->second;
}

Json& Json::set(const std::string& key, Json value)
{
    if (kind_ != Kind::object)
        fail("JSON value is not an object");
    return o_[key] = std::move(value);
}

const std::map<std::string, Json>& Json::fields() const
{
    if (kind_ != Kind::object)
        fail("JSON value is not an object");
    return o_;
}

bool Json::operator==(const Json& other) const
{
    if (is_number() && other.is_number()) {
        if (is_integer() && other.is_integer()) {
            if (is_unsigned() != other.is_unsigned())
                return false;
            return is_unsigned() ? as_uint() == other.as_uint() : i_ == other.i_;
        }
        return as_double() == other.as_double();
    }
    if (kind_ != other.kind_)
        return false;
    switch (kind_) {
    case Kind::null: return true;
    case Kind::boolean: return b_ == other.b_;
    case Kind::string: return s_ == other.s_;
    case Kind::array: return a_ == other.a_;
    case Kind::object: return o_ == other.o_;
    default: return false;
    }
}

namespace {
void quote(std::string& out, const std::string& s)
{
    out += '"';
    for (const char c : s) {
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (static_cast<unsigned char>(c) < 0x20) {
                char buffer[8];
                std::snprintf(buffer, sizeof buffer, "\\u%04x", c);
                out += buffer;
            } else {
                out += c;
            }
        }
    }
    out += '"';
}
} // namespace

void Json::dump_to(std::string& out, int indent, int depth) const
{
    auto newline = [&](int level) {
        if (indent < 0)
            return;
        out += '\n';
        out.append(static_cast<std::size_t>(indent * level), ' ');
    };
    switch (kind_) {
    case Kind::null: out += "null"; break;
    case Kind::boolean: out += b_ ? "true" : "false"; break;
    case Kind::integer: out += std::to_string(i_); break;
    case Kind::unsigned_integer: out += std::to_string(u_); break;
    case Kind::real: {
        char buffer[32];
        std::snprintf(buffer, sizeof buffer, "%.17g", d_);
        out += buffer;
        break;
    }
    case Kind::string: quote(out, s_); break;
    case Kind::array:
        out += '[';
        for (std::size_t i = 0; i < a_.size(); ++i) {
            if (i) out += indent < 0 ? "," : ",";
            newline(depth + 1);
            a_[i].dump_to(out, indent, depth + 1);
        }
        if (!a_.empty()) newline(depth);
        out += ']';
        break;
    case Kind::object: {
        out += '{';
        bool first = true;
        for (const auto& [key, value] : o_) {
            if (!first) out += ",";
            first = false;
            newline(depth + 1);
            quote(out, key);
            out += indent < 0 ? ":" : ": ";
            value.dump_to(out, indent, depth + 1);
        }
        if (!o_.empty()) newline(depth);
        out += '}';
        break;
    }
    }
}

std::string Json::dump(int indent) const
{
    std::string out;
    dump_to(out, indent, 0);
    return out;
}

} // namespace tiles
