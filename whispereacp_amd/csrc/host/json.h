// The JSON reader of the host code (safetensors headers, config.json,
// tokenizer.json): objects, arrays, strings (with \u escapes, written out as
// UTF-8), numbers, true/false/null, nested to a fixed depth, and whether a
// number was written as an integer, which the safetensors header's shapes and
// offsets must be. Errors are ModelErrors naming the document.
#pragma once

#include "../../../include/whispereacp/ModelError.h"

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace WSP
{
namespace
{
// ---------------------------------------------------------------------------
// JSON
// ---------------------------------------------------------------------------
struct Json
{
    enum class Kind
    {
        Null,
        Bool,
        Number,
        String,
        Array,
        Object
    };
    Kind kind = Kind::Null;
    bool boolean = false;
    double number = 0;
    bool integral = false; // written without fraction or exponent
    long long integer = 0; // its value, when integral and in range
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;

    const Json* member(const std::string& key) const
    {
        for (const auto& [k, v]: members)
            if (k == key)
                return &v;
        return nullptr;
    }
};

class JsonReader
{
public:
    JsonReader(const char* begin, const char* end, std::string what) : at(begin), stop(end), name(std::move(what)) {}

    Json document()
    {
        Json value = parseValue(0);
        skipSpace();
        if (at != stop)
            fail("trailing characters after the JSON value");
        return value;
    }

private:
    [[noreturn]] void fail(const std::string& why) const { throw ModelError(name + " is not valid JSON: " + why); }

    void skipSpace()
    {
        while (at != stop && (*at == ' ' || *at == '\t' || *at == '\n' || *at == '\r'))
            ++at;
    }

    Json parseValue(int depth)
    {
        if (depth > 64)
            fail("nesting is too deep");
        skipSpace();
        if (at == stop)
            fail("unexpected end");
        const char c = *at;
        if (c == '{')
            return parseObject(depth);
        if (c == '[')
            return parseArray(depth);
        if (c == '"')
        {
            Json v;
            v.kind = Json::Kind::String;
            v.text = parseString();
            return v;
        }
        if (c == '-' || (c >= '0' && c <= '9'))
            return parseNumber();
        if (literal("true"))
        {
            Json v;
            v.kind = Json::Kind::Bool;
            v.boolean = true;
            return v;
        }
        if (literal("false"))
        {
            Json v;
            v.kind = Json::Kind::Bool;
            return v;
        }
        if (literal("null"))
            return Json {};
        fail(std::string("unexpected character '") + c + "'");
    }

    bool literal(const char* word)
    {
        const std::size_t n = std::strlen(word);
        if ((std::size_t) (stop - at) >= n && std::memcmp(at, word, n) == 0)
        {
            at += n;
            return true;
        }
        return false;
    }

    Json parseObject(int depth)
    {
        Json v;
        v.kind = Json::Kind::Object;
        ++at;
        skipSpace();
        if (at != stop && *at == '}')
        {
            ++at;
            return v;
        }
        while (true)
        {
            skipSpace();
            if (at == stop || *at != '"')
                fail("an object key is not a string");
            std::string key = parseString();
            skipSpace();
            if (at == stop || *at != ':')
                fail("a key is not followed by ':'");
            ++at;
            v.members.emplace_back(std::move(key), parseValue(depth + 1));
            skipSpace();
            if (at != stop && *at == ',')
            {
                ++at;
                continue;
            }
            if (at != stop && *at == '}')
            {
                ++at;
                return v;
            }
            fail("an object is not closed");
        }
    }

    Json parseArray(int depth)
    {
        Json v;
        v.kind = Json::Kind::Array;
        ++at;
        skipSpace();
        if (at != stop && *at == ']')
        {
            ++at;
            return v;
        }
        while (true)
        {
            v.items.push_back(parseValue(depth + 1));
            skipSpace();
            if (at != stop && *at == ',')
            {
                ++at;
                continue;
            }
            if (at != stop && *at == ']')
            {
                ++at;
                return v;
            }
            fail("an array is not closed");
        }
    }

    static void appendUtf8(std::string& out, unsigned code)
    {
        if (code < 0x80)
            out += (char) code;
        else if (code < 0x800)
        {
            out += (char) (0xC0 | (code >> 6));
            out += (char) (0x80 | (code & 0x3F));
        }
        else if (code < 0x10000)
        {
            out += (char) (0xE0 | (code >> 12));
            out += (char) (0x80 | ((code >> 6) & 0x3F));
            out += (char) (0x80 | (code & 0x3F));
        }
        else
        {
            out += (char) (0xF0 | (code >> 18));
            out += (char) (0x80 | ((code >> 12) & 0x3F));
            out += (char) (0x80 | ((code >> 6) & 0x3F));
            out += (char) (0x80 | (code & 0x3F));
        }
    }

    unsigned hex4()
    {
        if (stop - at < 4)
            fail("a \\u escape is cut short");
        unsigned v = 0;
        for (int i = 0; i < 4; ++i)
        {
            const char c = *at++;
            v <<= 4;
            if (c >= '0' && c <= '9')
                v |= (unsigned) (c - '0');
            else if (c >= 'a' && c <= 'f')
                v |= (unsigned) (c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                v |= (unsigned) (c - 'A' + 10);
            else
                fail("a \\u escape has a non-hex digit");
        }
        return v;
    }

    std::string parseString()
    {
        ++at; // opening quote
        std::string out;
        while (true)
        {
            if (at == stop)
                fail("a string is not closed");
            const char c = *at++;
            if (c == '"')
                return out;
            if ((unsigned char) c < 0x20)
                fail("a string holds a control character");
            if (c != '\\')
            {
                out += c;
                continue;
            }
            if (at == stop)
                fail("a string ends in an escape");
            const char e = *at++;
            switch (e)
            {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u':
                {
                    unsigned code = hex4();
                    if (code >= 0xD800 && code < 0xDC00)
                    {
                        if (stop - at < 6 || at[0] != '\\' || at[1] != 'u')
                            fail("a surrogate pair is incomplete");
                        at += 2;
                        const unsigned low = hex4();
                        if (low < 0xDC00 || low > 0xDFFF)
                            fail("a surrogate pair is malformed");
                        code = 0x10000 + ((code - 0xD800) << 10) + (low - 0xDC00);
                    }
                    appendUtf8(out, code);
                    break;
                }
                default: fail(std::string("unknown escape \\") + e);
            }
        }
    }

    Json parseNumber()
    {
        const char* start = at;
        bool integral = true;
        if (*at == '-')
            ++at;
        if (at == stop || !(*at >= '0' && *at <= '9'))
            fail("a number has no digits");
        if (*at == '0')
            ++at;
        else
            while (at != stop && *at >= '0' && *at <= '9')
                ++at;
        if (at != stop && *at == '.')
        {
            integral = false;
            ++at;
            if (at == stop || !(*at >= '0' && *at <= '9'))
                fail("a fraction has no digits");
            while (at != stop && *at >= '0' && *at <= '9')
                ++at;
        }
        if (at != stop && (*at == 'e' || *at == 'E'))
        {
            integral = false;
            ++at;
            if (at != stop && (*at == '+' || *at == '-'))
                ++at;
            if (at == stop || !(*at >= '0' && *at <= '9'))
                fail("an exponent has no digits");
            while (at != stop && *at >= '0' && *at <= '9')
                ++at;
        }
        const std::string digits(start, at);
        Json v;
        v.kind = Json::Kind::Number;
        v.number = std::strtod(digits.c_str(), nullptr);
        if (integral)
        {
            errno = 0;
            const long long i = std::strtoll(digits.c_str(), nullptr, 10);
            v.integral = errno == 0;
            v.integer = i;
        }
        return v;
    }

    const char* at;
    const char* stop;
    std::string name;
};

} // namespace
} // namespace WSP
