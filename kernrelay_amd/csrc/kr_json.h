// Minimal JSON DOM: parse manifests / schedules, emit results.
// Plays the role of the reference's exec/runtime/json_min.hpp (Value :20,
// Parse :274, ParseFile :280, WriteFile :289); object key order is kept.
#pragma once

#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace kr {
namespace json {

class Value {
public:
    enum Kind { Null, Bool, Number, String, Array, Object };

    Value() = default;
    static Value MakeBool(bool b) { Value v; v.kind_ = Bool; v.b_ = b; return v; }
    static Value MakeNumber(double d) { Value v; v.kind_ = Number; v.n_ = d; return v; }
    static Value MakeString(std::string s) { Value v; v.kind_ = String; v.s_ = std::move(s); return v; }
    static Value MakeArray() { Value v; v.kind_ = Array; return v; }
    static Value MakeObject() { Value v; v.kind_ = Object; return v; }

    Kind kind() const { return kind_; }
    bool IsNull() const { return kind_ == Null; }
    bool IsObject() const { return kind_ == Object; }
    bool IsArray() const { return kind_ == Array; }
    bool IsNumber() const { return kind_ == Number; }
    bool IsString() const { return kind_ == String; }
    bool IsBool() const { return kind_ == Bool; }

    double AsNumber() const { Expect(Number, "number"); return n_; }
    bool AsBool() const { Expect(Bool, "bool"); return b_; }
    const std::string &AsString() const { Expect(String, "string"); return s_; }
    const std::vector<Value> &Items() const { Expect(Array, "array"); return arr_; }
    const std::vector<std::pair<std::string, Value>> &Members() const { Expect(Object, "object"); return obj_; }

    bool Has(const std::string &k) const
    {
        if (kind_ != Object) return false;
        for (const auto &kv : obj_)
            if (kv.first == k) return true;
        return false;
    }
    const Value &At(const std::string &k) const
    {
        Expect(Object, "object");
        for (const auto &kv : obj_)
            if (kv.first == k) return kv.second;
        throw std::runtime_error("json: missing key '" + k + "'");
    }
    const Value &At(size_t i) const
    {
        Expect(Array, "array");
        if (i >= arr_.size()) throw std::runtime_error("json: index out of range");
        return arr_[i];
    }
    double Num(const std::string &k, double dflt = 0.0) const
    {
        return Has(k) && At(k).IsNumber() ? At(k).n_ : dflt;
    }
    std::string Str(const std::string &k, const std::string &dflt = "") const
    {
        return Has(k) && At(k).IsString() ? At(k).s_ : dflt;
    }
    bool Flag(const std::string &k, bool dflt = false) const
    {
        return Has(k) && At(k).IsBool() ? At(k).b_ : dflt;
    }

    Value &Set(const std::string &k, Value v)
    {
        Expect(Object, "object");
        for (auto &kv : obj_)
            if (kv.first == k) { kv.second = std::move(v); return kv.second; }
        obj_.emplace_back(k, std::move(v));
        return obj_.back().second;
    }
    Value &Push(Value v) { Expect(Array, "array"); arr_.push_back(std::move(v)); return arr_.back(); }

    std::string Dump() const
    {
        std::ostringstream os;
        DumpTo(os);
        return os.str();
    }

    void DumpTo(std::ostringstream &os) const
    {
        switch (kind_) {
            case Null: os << "null"; break;
            case Bool: os << (b_ ? "true" : "false"); break;
            case Number: {
                if (!std::isfinite(n_)) { os << "null"; break; }
                char buf[40];
                if (n_ == std::floor(n_) && std::fabs(n_) < 1e15) {
                    std::snprintf(buf, sizeof buf, "%.0f", n_);
                } else {
                    std::snprintf(buf, sizeof buf, "%.9g", n_);
                }
                os << buf;
                break;
            }
            case String: Quote(os, s_); break;
            case Array: {
                os << '[';
                for (size_t i = 0; i < arr_.size(); ++i) {
                    if (i) os << ',';
                    arr_[i].DumpTo(os);
                }
                os << ']';
                break;
            }
            case Object: {
                os << '{';
                for (size_t i = 0; i < obj_.size(); ++i) {
                    if (i) os << ',';
                    Quote(os, obj_[i].first);
                    os << ':';
                    obj_[i].second.DumpTo(os);
                }
                os << '}';
                break;
            }
        }
    }

    static void Quote(std::ostringstream &os, const std::string &s)
    {
        os << '"';
        for (unsigned char c : s) {
            switch (c) {
                case '"': os << "\\\""; break;
                case '\\': os << "\\\\"; break;
                case '\n': os << "\\n"; break;
                case '\r': os << "\\r"; break;
                case '\t': os << "\\t"; break;
                default:
                    if (c < 0x20) {
                        char buf[8];
                        std::snprintf(buf, sizeof buf, "\\u%04x", c);
                        os << buf;
                    } else {
                        os << c;
                    }
            }
        }
        os << '"';
    }

private:
    void Expect(Kind k, const char *what) const
    {
        if (kind_ != k) throw std::runtime_error(std::string("json: expected ") + what);
    }

    Kind kind_ = Null;
    bool b_ = false;
    double n_ = 0.0;
    std::string s_;
    std::vector<Value> arr_;
    std::vector<std::pair<std::string, Value>> obj_;

    friend class Parser;
};

class Parser {
public:
    explicit Parser(const std::string &text) : t_(text) {}

    Value ParseDocument()
    {
        Value v = ParseValue(0);
        Skip();
        if (i_ != t_.size()) Fail("trailing characters");
        return v;
    }

private:
    [[noreturn]] void Fail(const std::string &m) const
    {
        throw std::runtime_error("json parse error at offset " + std::to_string(i_) + ": " + m);
    }
    void Skip()
    {
        while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\n' || t_[i_] == '\r' || t_[i_] == '\t')) ++i_;
    }
    bool Eat(char c)
    {
        Skip();
        if (i_ < t_.size() && t_[i_] == c) { ++i_; return true; }
        return false;
    }
    Value ParseValue(int depth)
    {
        if (depth > 256) Fail("nesting too deep");
        Skip();
        if (i_ >= t_.size()) Fail("unexpected end");
        const char c = t_[i_];
        if (c == '{') return ParseObject(depth);
        if (c == '[') return ParseArray(depth);
        if (c == '"') return Value::MakeString(ParseString());
        if (t_.compare(i_, 4, "true") == 0) { i_ += 4; return Value::MakeBool(true); }
        if (t_.compare(i_, 5, "false") == 0) { i_ += 5; return Value::MakeBool(false); }
        if (t_.compare(i_, 4, "null") == 0) { i_ += 4; return Value(); }
        return ParseNumber();
    }
    Value ParseObject(int depth)
    {
        ++i_;
        Value v = Value::MakeObject();
        if (Eat('}')) return v;
        do {
            Skip();
            if (i_ >= t_.size() || t_[i_] != '"') Fail("expected key");
            std::string k = ParseString();
            if (!Eat(':')) Fail("expected ':'");
            v.obj_.emplace_back(std::move(k), ParseValue(depth + 1));
        } while (Eat(','));
        if (!Eat('}')) Fail("expected '}'");
        return v;
    }
    Value ParseArray(int depth)
    {
        ++i_;
        Value v = Value::MakeArray();
        if (Eat(']')) return v;
        do {
            v.arr_.push_back(ParseValue(depth + 1));
        } while (Eat(','));
        if (!Eat(']')) Fail("expected ']'");
        return v;
    }
    static void PutUtf8(std::string &out, uint32_t cp)
    {
        if (cp < 0x80) {
            out += char(cp);
        } else if (cp < 0x800) {
            out += char(0xc0 | (cp >> 6));
            out += char(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += char(0xe0 | (cp >> 12));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        } else {
            out += char(0xf0 | (cp >> 18));
            out += char(0x80 | ((cp >> 12) & 0x3f));
            out += char(0x80 | ((cp >> 6) & 0x3f));
            out += char(0x80 | (cp & 0x3f));
        }
    }
    uint32_t Hex4()
    {
        if (i_ + 4 > t_.size()) Fail("bad \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= uint32_t(c - '0');
            else if (c >= 'a' && c <= 'f') v |= uint32_t(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= uint32_t(c - 'A' + 10);
            else Fail("bad hex digit");
        }
        return v;
    }
    std::string ParseString()
    {
        ++i_;
        std::string out;
        while (true) {
            if (i_ >= t_.size()) Fail("unterminated string");
            const char c = t_[i_++];
            if (c == '"') break;
            if (c != '\\') { out += c; continue; }
            if (i_ >= t_.size()) Fail("bad escape");
            const char e = t_[i_++];
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
                    uint32_t cp = Hex4();
                    if (cp >= 0xd800 && cp < 0xdc00 && i_ + 6 <= t_.size() && t_[i_] == '\\' && t_[i_ + 1] == 'u') {
                        i_ += 2;
                        const uint32_t lo = Hex4();
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    PutUtf8(out, cp);
                    break;
                }
                default: Fail("bad escape");
            }
        }
        return out;
    }
    Value ParseNumber()
    {
        const size_t start = i_;
        if (i_ < t_.size() && (t_[i_] == '-' || t_[i_] == '+')) ++i_;
        while (i_ < t_.size() && (std::isdigit(static_cast<unsigned char>(t_[i_])) || t_[i_] == '.' ||
                                  t_[i_] == 'e' || t_[i_] == 'E' || t_[i_] == '-' || t_[i_] == '+'))
            ++i_;
        if (start == i_) Fail("unexpected character");
        try {
            size_t used = 0;
            const double d = std::stod(t_.substr(start, i_ - start), &used);
            if (used != i_ - start) Fail("bad number");
            return Value::MakeNumber(d);
        } catch (const std::invalid_argument &) {
            Fail("bad number");
        } catch (const std::out_of_range &) {
            Fail("number out of range");
        }
    }

    const std::string &t_;
    size_t i_ = 0;
};

inline Value Parse(const std::string &text) { return Parser(text).ParseDocument(); }

inline Value ParseFile(const std::string &path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return Parse(ss.str());
}

inline void WriteFile(const std::string &path, const Value &v)
{
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f << v.Dump() << "\n";
}

}  // namespace json
}  // namespace kr
