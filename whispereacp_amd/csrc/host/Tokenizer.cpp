// Whisper's byte-level BPE tokenizer (Tokenizer/Tokenizer.cpp,
// Tokenizer/ByteEncoding.cpp, Tokenizer/PreTokenizer.cpp, Tokenizer/Unicode.cpp):
// host code, run once per transcript to turn the greedy tokens into text.
#include "../../../include/whispereacp/Tokenizer.h"
#include "json.h"
#include "unicode_table.h"

#include <algorithm>
#include <array>
#include <fstream>
#include <iterator>

namespace WSP
{
// ---------------------------------------------------------------------------
// Byte layer: the printable bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF stand
// for themselves; the other 68 are lifted to U+0100 onwards in byte order, so
// a space is U+0120 ('Ġ') and a newline U+010A ('Ċ').
// ---------------------------------------------------------------------------
namespace ByteEncoding
{
namespace
{
bool standsForItself(int byte)
{
    return (byte >= '!' && byte <= '~') || (byte >= 0xA1 && byte <= 0xAC) || (byte >= 0xAE && byte <= 0xFF);
}

struct Table
{
    std::array<char32_t, 256> forward {};
    Table()
    {
        int lifted = 0;
        for (int b = 0; b < 256; ++b)
            forward[b] = standsForItself(b) ? (char32_t) b : (char32_t) (0x100 + lifted++);
    }
};

const Table& table()
{
    static const Table t;
    return t;
}

void appendUtf8(std::string& out, char32_t c)
{
    if (c < 0x80)
        out += (char) c;
    else if (c < 0x800)
    {
        out += (char) (0xC0 | (c >> 6));
        out += (char) (0x80 | (c & 0x3F));
    }
    else if (c < 0x10000)
    {
        out += (char) (0xE0 | (c >> 12));
        out += (char) (0x80 | ((c >> 6) & 0x3F));
        out += (char) (0x80 | (c & 0x3F));
    }
    else
    {
        out += (char) (0xF0 | (c >> 18));
        out += (char) (0x80 | ((c >> 12) & 0x3F));
        out += (char) (0x80 | ((c >> 6) & 0x3F));
        out += (char) (0x80 | (c & 0x3F));
    }
}
} // namespace

char32_t codePointForByte(unsigned char byte)
{
    return table().forward[byte];
}

int byteForCodePoint(char32_t c)
{
    if (c < 0x100)
        return standsForItself((int) c) ? (int) c : -1;
    if (c < 0x100 + 68)
    {
        // the (c - 0x100)-th byte that does not stand for itself
        int lifted = (int) (c - 0x100);
        for (int b = 0; b < 256; ++b)
            if (!standsForItself(b) && lifted-- == 0)
                return b;
    }
    return -1;
}

std::string toPrintable(std::string_view bytes)
{
    std::string out;
    out.reserve(bytes.size() * 2);
    for (unsigned char b: bytes)
        appendUtf8(out, codePointForByte(b));
    return out;
}

std::string fromPrintable(std::string_view printable)
{
    std::string out;
    for (std::size_t at = 0; at < printable.size();)
    {
        const Unicode::CodePoint c = Unicode::readCodePoint(printable, at);
        at += (std::size_t) c.byteLength;
        const int b = byteForCodePoint(c.value);
        if (b >= 0)
            out += (char) b;
    }
    return out;
}
} // namespace ByteEncoding

// ---------------------------------------------------------------------------
// Unicode: UTF-8 decoding (strict: no overlongs, no surrogates, nothing past
// U+10FFFF) and the pre-tokenizer's three classes.
// ---------------------------------------------------------------------------
namespace Unicode
{
namespace
{
bool inRanges(char32_t c, const unicode_table::CodeRange* first, const unicode_table::CodeRange* last)
{
    const auto* it = std::upper_bound(first, last, c,
                                      [](char32_t v, const unicode_table::CodeRange& r) { return v < r.first; });
    return it != first && c <= (it - 1)->last;
}

// The White_Space property (Unicode PropList.txt), which \s matches.
bool isWhiteSpace(char32_t c)
{
    return (c >= 0x09 && c <= 0x0D) || c == 0x20 || c == 0x85 || c == 0xA0 || c == 0x1680
           || (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 || c == 0x202F || c == 0x205F
           || c == 0x3000;
}
} // namespace

Category categoryOf(char32_t c)
{
    if (isWhiteSpace(c))
        return Category::whitespace;
    if (inRanges(c, std::begin(unicode_table::kLetters), std::end(unicode_table::kLetters)))
        return Category::letter;
    if (inRanges(c, std::begin(unicode_table::kNumbers), std::end(unicode_table::kNumbers)))
        return Category::number;
    return Category::other;
}

CodePoint readCodePoint(std::string_view text, std::size_t at)
{
    const unsigned char lead = (unsigned char) text[at];
    CodePoint bad {lead, 1, Category::other};
    int length;
    char32_t value, minimum;
    if (lead < 0x80)
        return {lead, 1, categoryOf(lead)};
    if ((lead & 0xE0) == 0xC0)
        length = 2, value = lead & 0x1F, minimum = 0x80;
    else if ((lead & 0xF0) == 0xE0)
        length = 3, value = lead & 0x0F, minimum = 0x800;
    else if ((lead & 0xF8) == 0xF0)
        length = 4, value = lead & 0x07, minimum = 0x10000;
    else
        return bad;
    if (at + (std::size_t) length > text.size())
        return bad;
    for (int i = 1; i < length; ++i)
    {
        const unsigned char c = (unsigned char) text[at + i];
        if ((c & 0xC0) != 0x80)
            return bad;
        value = (value << 6) | (c & 0x3F);
    }
    if (value < minimum || value > 0x10FFFF || (value >= 0xD800 && value <= 0xDFFF))
        return bad;
    return {value, length, categoryOf(value)};
}
} // namespace Unicode

// ---------------------------------------------------------------------------
// The pre-tokenizer (Tokenizer/PreTokenizer.cpp): at each position the
// pattern's alternatives in order — a contraction, an optional literal space
// then a run of letters, of numbers, or of anything that is neither nor
// whitespace, then a whitespace run that leaves its last character to the
// piece after it (\s+(?!\S)), else the run to the end, else one character.
// ---------------------------------------------------------------------------
namespace
{
using Unicode::Category;

std::size_t contractionAt(std::string_view text, std::size_t at)
{
    static const std::string_view forms[] = {"'s", "'t", "'re", "'ve", "'m", "'ll", "'d"};
    for (std::string_view f: forms)
        if (text.substr(at, f.size()) == f)
            return f.size();
    return 0;
}

std::size_t runOf(std::string_view text, std::size_t at, Category want)
{
    const std::size_t start = text[at] == ' ' ? at + 1 : at;
    std::size_t end = start;
    while (end < text.size())
    {
        const Unicode::CodePoint c = Unicode::readCodePoint(text, end);
        if (c.category != want)
            break;
        end += (std::size_t) c.byteLength;
    }
    return end == start ? 0 : end - at;
}

std::size_t whitespaceAt(std::string_view text, std::size_t at)
{
    std::size_t end = at, lastStart = at;
    while (end < text.size())
    {
        const Unicode::CodePoint c = Unicode::readCodePoint(text, end);
        if (c.category != Category::whitespace)
            break;
        lastStart = end;
        end += (std::size_t) c.byteLength;
    }
    if (end == at)
        return 0;
    // followed by a non-space: leave the last character to the next piece
    if (end < text.size() && lastStart > at)
        return lastStart - at;
    return end - at;
}

std::size_t pieceAt(std::string_view text, std::size_t at)
{
    if (std::size_t n = contractionAt(text, at))
        return n;
    for (Category c: {Category::letter, Category::number, Category::other})
        if (std::size_t n = runOf(text, at, c))
            return n;
    if (std::size_t n = whitespaceAt(text, at))
        return n;
    return (std::size_t) Unicode::readCodePoint(text, at).byteLength;
}

std::uint64_t pairKey(int left, int right)
{
    return ((std::uint64_t) (std::uint32_t) left << 32) | (std::uint32_t) right;
}

std::string readAll(const std::string& path)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw TokenizerError("cannot open '" + path + "'");
    return std::string(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
}

int tokenId(const Json& v)
{
    if (v.kind != Json::Kind::Number || !v.integral || v.integer < 0 || v.integer > (1 << 28))
        throw TokenizerError("tokenizer.json holds a token id that is not a small non-negative integer");
    return (int) v.integer;
}

const Json& required(const Json& parent, const char* key)
{
    const Json* v = parent.kind == Json::Kind::Object ? parent.member(key) : nullptr;
    if (v == nullptr)
        throw TokenizerError(std::string("tokenizer.json has no '") + key + "'");
    return *v;
}
} // namespace

std::vector<std::string_view> preTokenize(std::string_view text)
{
    std::vector<std::string_view> pieces;
    for (std::size_t at = 0; at < text.size();)
    {
        const std::size_t n = pieceAt(text, at);
        pieces.push_back(text.substr(at, n));
        at += n;
    }
    return pieces;
}

// ---------------------------------------------------------------------------
// The tokenizer
// ---------------------------------------------------------------------------
Tokenizer Tokenizer::fromFile(const std::string& path)
{
    return fromJsonText(readAll(path));
}

Tokenizer Tokenizer::fromJsonText(std::string_view json)
{
    const Json root = JsonReader(json.data(), json.data() + json.size(), "tokenizer.json").document();
    const Json& model = required(root, "model");
    const Json& vocab = required(model, "vocab");
    const Json& rules = required(model, "merges");
    if (vocab.kind != Json::Kind::Object)
        throw TokenizerError("tokenizer.json model.vocab is not an object");
    if (rules.kind != Json::Kind::Array)
        throw TokenizerError("tokenizer.json model.merges is not a list");
    const Json* added = root.member("added_tokens");

    Tokenizer t;
    int highest = -1;
    for (const auto& [text, id]: vocab.members)
        highest = std::max(highest, tokenId(id));
    if (added != nullptr && added->kind == Json::Kind::Array)
        for (const Json& entry: added->items)
            highest = std::max(highest, tokenId(required(entry, "id")));
    t.texts.assign((std::size_t) highest + 1, std::string());
    t.specialFlags.assign((std::size_t) highest + 1, 0);
    for (const auto& [text, id]: vocab.members)
        t.texts[(std::size_t) tokenId(id)] = text;
    if (added != nullptr && added->kind == Json::Kind::Array)
        for (const Json& entry: added->items)
        {
            const int id = tokenId(required(entry, "id"));
            const Json& content = required(entry, "content");
            if (content.kind != Json::Kind::String)
                throw TokenizerError("tokenizer.json has an added token without its text");
            t.texts[(std::size_t) id] = content.text;
            t.specialFlags[(std::size_t) id] = 1;
        }
    for (int id = 0; id <= highest; ++id)
        if (!t.texts[(std::size_t) id].empty())
            t.ids.emplace(t.texts[(std::size_t) id], id);

    // A rule is "left right" or ["left", "right"]; a rank is its position,
    // and a rule over tokens the vocabulary lacks is never applicable.
    for (std::size_t rank = 0; rank < rules.items.size(); ++rank)
    {
        const Json& rule = rules.items[rank];
        std::string left, right;
        if (rule.kind == Json::Kind::String)
        {
            const std::size_t space = rule.text.find(' ');
            if (space == std::string::npos)
                throw TokenizerError("merge rule '" + rule.text + "' has no space");
            left = rule.text.substr(0, space);
            right = rule.text.substr(space + 1);
        }
        else if (rule.kind == Json::Kind::Array && rule.items.size() == 2
                 && rule.items[0].kind == Json::Kind::String && rule.items[1].kind == Json::Kind::String)
        {
            left = rule.items[0].text;
            right = rule.items[1].text;
        }
        else
            throw TokenizerError("a merge rule is neither a string nor a pair of strings");
        const int l = t.tokenForText(left), r = t.tokenForText(right), m = t.tokenForText(left + right);
        if (l != invalidTokenId && r != invalidTokenId && m != invalidTokenId)
            t.merges.emplace(pairKey(l, r), std::make_pair((int) rank, m));
    }
    t.special = specialTokensFromTokenizerJson(std::string(json));
    return t;
}

bool Tokenizer::isSpecial(int token) const
{
    return token >= 0 && token < size() && specialFlags[(std::size_t) token] != 0;
}

std::string_view Tokenizer::textForToken(int token) const
{
    return token >= 0 && token < size() ? std::string_view(texts[(std::size_t) token]) : std::string_view();
}

int Tokenizer::tokenForText(std::string_view text) const
{
    const auto it = ids.find(std::string(text));
    return it == ids.end() ? invalidTokenId : it->second;
}

// BPE over one piece: the piece's bytes in the printable alphabet, one symbol
// per code point; while some adjacent pair has a merge, the pair of lowest
// rank (the leftmost of equals) becomes its merged token. Symbols the
// vocabulary lacks are dropped.
void Tokenizer::encodePiece(std::string_view piece, std::vector<int>& out) const
{
    const std::string printable = ByteEncoding::toPrintable(piece);
    std::vector<int> symbols;
    for (std::size_t at = 0; at < printable.size();)
    {
        const int n = Unicode::readCodePoint(printable, at).byteLength;
        symbols.push_back(tokenForText(std::string_view(printable).substr(at, (std::size_t) n)));
        at += (std::size_t) n;
    }
    for (;;)
    {
        int bestRank = -1, bestAt = -1, bestToken = invalidTokenId;
        for (std::size_t i = 0; i + 1 < symbols.size(); ++i)
        {
            const auto it = merges.find(pairKey(symbols[i], symbols[i + 1]));
            if (it != merges.end() && (bestRank < 0 || it->second.first < bestRank))
            {
                bestRank = it->second.first;
                bestAt = (int) i;
                bestToken = it->second.second;
            }
        }
        if (bestAt < 0)
            break;
        symbols[(std::size_t) bestAt] = bestToken;
        symbols.erase(symbols.begin() + bestAt + 1);
    }
    for (int s: symbols)
        if (s != invalidTokenId)
            out.push_back(s);
}

// Special tokens written literally (`<|name|>`, an added token) are taken
// whole; the text between them goes through the pre-tokenizer and BPE.
std::vector<int> Tokenizer::encode(std::string_view text) const
{
    std::vector<int> out;
    std::size_t plain = 0, at = text.find("<|");
    auto flush = [&](std::size_t end) {
        for (std::string_view piece: preTokenize(text.substr(plain, end - plain)))
            encodePiece(piece, out);
    };
    while (at != std::string_view::npos)
    {
        const std::size_t close = text.find("|>", at + 2);
        const int token = close == std::string_view::npos ? invalidTokenId
                                                           : tokenForText(text.substr(at, close + 2 - at));
        if (!isSpecial(token))
        {
            at = text.find("<|", at + 1);
            continue;
        }
        flush(at);
        out.push_back(token);
        plain = close + 2;
        at = text.find("<|", plain);
    }
    flush(text.size());
    return out;
}

std::string Tokenizer::decodeAll(const int* tokens, int count, bool keepSpecial) const
{
    std::string text, printable;
    for (int i = 0; i < count; ++i)
    {
        const int token = tokens[i];
        if (token < 0 || token >= size())
            continue;
        if (isSpecial(token))
        {
            text += ByteEncoding::fromPrintable(printable);
            printable.clear();
            if (keepSpecial)
                text += texts[(std::size_t) token];
            continue;
        }
        printable += texts[(std::size_t) token];
    }
    return text + ByteEncoding::fromPrintable(printable);
}

std::string Tokenizer::decode(const int* tokens, int count) const
{
    return decodeAll(tokens, count, false);
}

std::string Tokenizer::decodeKeepingSpecialTokens(const int* tokens, int count) const
{
    return decodeAll(tokens, count, true);
}
} // namespace WSP
