// Minimal JSON reader for compact MACE model files.
//
// Model files are tens to hundreds of MB, almost all of it flat arrays of
// numbers, so arrays whose elements are all numbers are stored as one
// std::vector<double> instead of a vector of values.  Parsing is a single
// recursive-descent pass with std::from_chars for numbers.
#pragma once

#include <charconv>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace sxl::json {

class Value {
public:
    enum class Kind { null, boolean, number, string, array, numbers, object };

    Kind kind = Kind::null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> items;                        // array
    std::vector<double> nums;                        // numbers (numeric array)
    std::vector<std::pair<std::string, Value>> obj;  // object, in file order

    bool is_object() const { return kind == Kind::object; }
    bool is_array() const { return kind == Kind::array || kind == Kind::numbers; }
    bool is_number() const { return kind == Kind::number; }

    std::size_t size() const
    {
        if (kind == Kind::numbers) return nums.size();
        if (kind == Kind::array) return items.size();
        if (kind == Kind::object) return obj.size();
        return 0;
    }
    const Value* find(std::string_view key) const
    {
        if (kind != Kind::object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    bool contains(std::string_view key) const { return find(key) != nullptr; }
    const Value& at(std::string_view key) const
    {
        const Value* v = find(key);
        if (!v) throw std::invalid_argument("model JSON is missing key '" + std::string(key) + "'");
        return *v;
    }
    double as_number(std::string_view what = "value") const
    {
        if (kind == Kind::number) return num;
        if (kind == Kind::boolean) return b ? 1.0 : 0.0;
        throw std::invalid_argument("model JSON " + std::string(what) + " is not a number");
    }
    int as_int(std::string_view what = "value") const
    {
        const double v = as_number(what);
        if (v != static_cast<double>(static_cast<long long>(v)) || v < -2147483648.0 || v > 2147483647.0)
            throw std::invalid_argument("model JSON " + std::string(what) + " is not an integer");
        return static_cast<int>(v);
    }
    bool as_bool(std::string_view what = "value") const
    {
        if (kind == Kind::boolean) return b;
        throw std::invalid_argument("model JSON " + std::string(what) + " is not a boolean");
    }
    const std::string& as_string(std::string_view what = "value") const
    {
        if (kind != Kind::string)
            throw std::invalid_argument("model JSON " + std::string(what) + " is not a string");
        return str;
    }
    // Flat numeric content of an array (nested arrays are flattened).
    std::vector<double> flat_numbers(std::string_view what = "array") const
    {
        std::vector<double> out;
        append_numbers(out, what);
        return out;
    }
    void append_numbers(std::vector<double>& out, std::string_view what) const
    {
        if (kind == Kind::numbers) {
            out.insert(out.end(), nums.begin(), nums.end());
        } else if (kind == Kind::array) {
            for (const auto& v : items) v.append_numbers(out, what);
        } else if (kind == Kind::number) {
            out.push_back(num);
        } else {
            throw std::invalid_argument("model JSON " + std::string(what) + " is not numeric");
        }
    }
    std::vector<int> ints(std::string_view what = "array") const
    {
        std::vector<double> v = flat_numbers(what);
        std::vector<int> out(v.size());
        for (std::size_t i = 0; i < v.size(); ++i) {
            if (v[i] != static_cast<double>(static_cast<long long>(v[i])))
                throw std::invalid_argument("model JSON " + std::string(what) + " holds a non-integer");
            out[i] = static_cast<int>(v[i]);
        }
        return out;
    }
    const Value& operator[](std::size_t i) const
    {
        if (kind != Kind::array || i >= items.size())
            throw std::out_of_range("model JSON array index out of range");
        return items[i];
    }
};

class Parser {
public:
    Parser(const char* begin, const char* end) : p_(begin), end_(end) {}

    Value parse_document()
    {
        Value v = parse_value();
        skip_ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;

    [[noreturn]] void fail(const char* what)
    {
        throw std::invalid_argument(std::string("model JSON parse error: ") + what);
    }
    void skip_ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool literal(const char* word)
    {
        const std::size_t n = std::strlen(word);
        if (static_cast<std::size_t>(end_ - p_) >= n && std::memcmp(p_, word, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    double parse_number()
    {
        double value = 0.0;
        const char* start = p_;
        if (p_ < end_ && *p_ == '+') fail("invalid number");
        auto res = std::from_chars(start, end_, value);
        if (res.ec == std::errc::result_out_of_range) {
            // keep the reference's behaviour of rejecting non-finite values later
            value = std::strtod(std::string(start, res.ptr).c_str(), nullptr);
        } else if (res.ec != std::errc()) {
            fail("invalid number");
        }
        p_ = res.ptr;
        return value;
    }
    std::string parse_string()
    {
        if (*p_ != '"') fail("expected string");
        ++p_;
        std::string out;
        while (true) {
            if (p_ >= end_) fail("unterminated string");
            char c = *p_++;
            if (c == '"') break;
            if (c == '\\') {
                if (p_ >= end_) fail("unterminated escape");
                char e = *p_++;
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
                    if (end_ - p_ < 4) fail("bad unicode escape");
                    unsigned code = 0;
                    for (int i = 0; i < 4; ++i) {
                        char h = *p_++;
                        code <<= 4;
                        if (h >= '0' && h <= '9') code |= h - '0';
                        else if (h >= 'a' && h <= 'f') code |= h - 'a' + 10;
                        else if (h >= 'A' && h <= 'F') code |= h - 'A' + 10;
                        else fail("bad unicode escape");
                    }
                    if (code < 0x80) {
                        out.push_back(static_cast<char>(code));
                    } else if (code < 0x800) {
                        out.push_back(static_cast<char>(0xC0 | (code >> 6)));
                        out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
                    } else {
                        out.push_back(static_cast<char>(0xE0 | (code >> 12)));
                        out.push_back(static_cast<char>(0x80 | ((code >> 6) & 0x3F)));
                        out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
                    }
                    break;
                }
                default: fail("bad escape");
                }
            } else {
                out.push_back(c);
            }
        }
        return out;
    }
    Value parse_value()
    {
        skip_ws();
        if (p_ >= end_) fail("unexpected end");
        Value v;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Value::Kind::object;
            skip_ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return v;
            }
            while (true) {
                skip_ws();
                std::string key = parse_string();
                skip_ws();
                if (p_ >= end_ || *p_ != ':') fail("expected ':'");
                ++p_;
                v.obj.emplace_back(std::move(key), parse_value());
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
            skip_ws();
            v.kind = Value::Kind::numbers;
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return v;
            }
            while (true) {
                skip_ws();
                if (p_ >= end_) fail("unexpected end");
                const char d = *p_;
                if (v.kind == Value::Kind::numbers && (d == '-' || (d >= '0' && d <= '9'))) {
                    v.nums.push_back(parse_number());
                } else {
                    if (v.kind == Value::Kind::numbers) {
                        v.kind = Value::Kind::array;
                        for (double x : v.nums) {
                            Value n;
                            n.kind = Value::Kind::number;
                            n.num = x;
                            v.items.push_back(std::move(n));
                        }
                        v.nums.clear();
                    }
                    v.items.push_back(parse_value());
                }
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
            v.kind = Value::Kind::string;
            v.str = parse_string();
        } else if (literal("true")) {
            v.kind = Value::Kind::boolean;
            v.b = true;
        } else if (literal("false")) {
            v.kind = Value::Kind::boolean;
            v.b = false;
        } else if (literal("null")) {
            v.kind = Value::Kind::null;
        } else {
            v.kind = Value::Kind::number;
            v.num = parse_number();
        }
        return v;
    }
};

Value parse_file(const std::string& path);

}  // namespace sxl::json
