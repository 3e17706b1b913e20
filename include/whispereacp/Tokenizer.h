// Whisper's byte-level BPE (Tokenizer/Tokenizer.h:20-80): the vocabulary and
// merges of a HuggingFace tokenizer.json, GPT-2's byte-to-printable layer,
// GPT-2's pre-tokenizer split, and the added tokens (every one of which is
// special: never produced by a merge, skipped by decode()).
#pragma once

#include "SafeTensors.h"

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace WSP
{
// Tokenizer/Tokenizer.h:20-24
class TokenizerError : public std::runtime_error
{
    using std::runtime_error::runtime_error;
};

constexpr int invalidTokenId = -1;

// GPT-2's byte-level layer (Tokenizer/ByteEncoding.h): every byte maps to a
// printable code point and back, a bijection, so any byte string round-trips.
namespace ByteEncoding
{
char32_t codePointForByte(unsigned char byte);
int byteForCodePoint(char32_t codePoint); // -1 outside the table
std::string toPrintable(std::string_view bytes);
std::string fromPrintable(std::string_view printable);
} // namespace ByteEncoding

// The three classes the pre-tokenizer's pattern names (\p{L}, \p{N}, \s)
// and everything else (Tokenizer/Unicode.h).
namespace Unicode
{
enum class Category
{
    other,
    letter,
    number,
    whitespace
};

struct CodePoint
{
    char32_t value = 0;
    int byteLength = 1;
    Category category = Category::other;
};

Category categoryOf(char32_t codePoint);
// A byte that starts no valid UTF-8 sequence reads as one byte of `other`.
CodePoint readCodePoint(std::string_view text, std::size_t position);
} // namespace Unicode

// GPT-2's pattern 's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
// (Tokenizer/PreTokenizer.h): the pieces BPE runs on, in order.
std::vector<std::string_view> preTokenize(std::string_view text);

class Tokenizer
{
public:
    static Tokenizer fromJsonText(std::string_view json);
    static Tokenizer fromFile(const std::string& path);

    std::vector<int> encode(std::string_view text) const;
    std::string decode(const int* tokens, int count) const;
    std::string decodeKeepingSpecialTokens(const int* tokens, int count) const;

    int size() const { return (int) texts.size(); }
    bool isSpecial(int token) const;
    std::string_view textForToken(int token) const; // in the printable alphabet
    int tokenForText(std::string_view text) const;  // invalidTokenId when absent
    const SpecialTokens& specials() const { return special; }

private:
    void encodePiece(std::string_view piece, std::vector<int>& out) const;
    std::string decodeAll(const int* tokens, int count, bool keepSpecial) const;

    std::vector<std::string> texts;
    std::vector<char> specialFlags;
    std::unordered_map<std::string, int> ids;
    std::unordered_map<std::uint64_t, std::pair<int, int>> merges; // (left, right) -> (rank, merged)
    SpecialTokens special;
};
} // namespace WSP
