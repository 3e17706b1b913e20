// The tokenizer's building blocks (host/Tokenizer.cpp) checked case by case,
// in a build with AddressSanitizer and UndefinedBehaviorSanitizer: the byte
// layer, the Unicode classes, UTF-8 decoding edges and the pre-tokenizer
// split, as Tests/Tokenizer/TokenizerTests.cpp:147-330 checks the reference's.
// Then every file named on the command line goes through
// Tokenizer::fromFile and encode/decode round trips. Test infrastructure
// (tests/test_tokenizer.py runs it). Prints one line per failed check and
// "checks: <n> failed: <m>"; exits 1 when a check failed.
#include "../../include/whispereacp/ModelError.h"
#include "../../include/whispereacp/Tokenizer.h"

#include <cstdio>
#include <string>
#include <vector>

namespace
{
int checks = 0, failures = 0;

void check(bool ok, const char* what, int line)
{
    ++checks;
    if (!ok)
    {
        ++failures;
        std::printf("failed: %s (line %d)\n", what, line);
    }
}
#define CHECK(x) check((x), #x, __LINE__)

bool splitsInto(std::string_view text, const std::vector<std::string>& expected)
{
    const auto pieces = WSP::preTokenize(text);
    if (pieces.size() != expected.size())
        return false;
    for (std::size_t i = 0; i < pieces.size(); ++i)
        if (pieces[i] != expected[i])
            return false;
    return true;
}

void byteLayer()
{
    using namespace WSP::ByteEncoding;
    bool bijection = true;
    for (int b = 0; b < 256; ++b)
        bijection = bijection && byteForCodePoint(codePointForByte((unsigned char) b)) == b;
    CHECK(bijection);
    CHECK(codePointForByte(' ') == 0x120);
    CHECK(codePointForByte('\n') == 0x10A);
    CHECK(codePointForByte(0) == 0x100);
    CHECK(codePointForByte(0x7F) == 0x121);
    CHECK(codePointForByte(0xAD) == 0x143);
    CHECK(codePointForByte('a') == U'a');
    CHECK(codePointForByte(0xFF) == 0xFF);
    std::string all;
    for (int b = 0; b < 256; ++b)
        all += (char) b;
    CHECK(fromPrintable(toPrintable(all)) == all);
    CHECK(toPrintable(" the") == "\xc4\xa0the");
    CHECK(toPrintable("Hello!") == "Hello!");
}

void unicodeClasses()
{
    using WSP::Unicode::Category;
    using WSP::Unicode::categoryOf;
    CHECK(categoryOf(U'a') == Category::letter);
    CHECK(categoryOf(U'7') == Category::number);
    CHECK(categoryOf(U'!') == Category::other);
    CHECK(categoryOf(U' ') == Category::whitespace);
    CHECK(categoryOf(U'\n') == Category::whitespace);
    CHECK(categoryOf(0x00E9) == Category::letter);
    CHECK(categoryOf(0x4F60) == Category::letter);
    CHECK(categoryOf(0x0301) == Category::other);
    CHECK(categoryOf(0x1F600) == Category::other);
    CHECK(categoryOf(0x3002) == Category::other);
    CHECK(categoryOf(0x00B2) == Category::number);
    CHECK(categoryOf(0x0663) == Category::number);
    CHECK(categoryOf(0x00A0) == Category::whitespace);
    CHECK(categoryOf(0x3000) == Category::whitespace);
    CHECK(categoryOf(0x200B) == Category::other);
    CHECK(categoryOf(0xFEFF) == Category::other);
}

void utf8Edges()
{
    using WSP::Unicode::readCodePoint;
    CHECK(readCodePoint("\x80", 0).byteLength == 1);
    CHECK(readCodePoint("\x80", 0).category == WSP::Unicode::Category::other);
    CHECK(readCodePoint(std::string_view("\xe4\xbd", 2), 0).byteLength == 1);
    CHECK(readCodePoint("\xc0\xaf", 0).byteLength == 1);               // overlong
    CHECK(readCodePoint("\xed\xa0\x80", 0).byteLength == 1);           // a surrogate
    CHECK(readCodePoint("\xf4\x90\x80\x80", 0).byteLength == 1);       // past U+10FFFF
    CHECK(readCodePoint("\xc3", 0).category == WSP::Unicode::Category::other);
    CHECK(readCodePoint("\xe4\xbd\xa0", 0).value == 0x4F60 && readCodePoint("\xe4\xbd\xa0", 0).byteLength == 3);
    CHECK(readCodePoint("\xf0\x9f\x98\x80", 0).value == 0x1F600);
    CHECK(readCodePoint("ab\xe4\xbd\xa0z", 2).category == WSP::Unicode::Category::letter);
}

void preTokenizer()
{
    CHECK(splitsInto("Hello world", {"Hello", " world"}));
    CHECK(splitsInto(" Hello, world!", {" Hello", ",", " world", "!"}));
    CHECK(splitsInto("Don't stop", {"Don", "'t", " stop"}));
    CHECK(splitsInto("It's", {"It", "'s"}));
    CHECK(splitsInto("1234 567.89", {"1234", " 567", ".", "89"}));
    CHECK(splitsInto("", {}));
    CHECK(splitsInto("  double  spaces", {" ", " double", " ", " spaces"}));
    CHECK(splitsInto("x  ", {"x", "  "}));
    CHECK(splitsInto("a\tb", {"a", "\t", "b"}));
    CHECK(splitsInto("\n\nx", {"\n", "\n", "x"}));
    CHECK(splitsInto("caf\xc3\xa9 \xe4\xbd\xa0\xe5\xa5\xbd", {"caf\xc3\xa9", " \xe4\xbd\xa0\xe5\xa5\xbd"}));
    CHECK(splitsInto("a\x80z", {"a", "\x80", "z"}));
}

void file(const char* path)
{
    try
    {
        const WSP::Tokenizer t = WSP::Tokenizer::fromFile(path);
        std::string every;
        for (int b = 1; b < 256; ++b)
            every += (char) b;
        for (const std::string& text: {std::string("the quick brown fox"), std::string("caf\xc3\xa9 x"), every})
        {
            const std::vector<int> ids = t.encode(text);
            CHECK(t.decode(ids.data(), (int) ids.size()) == text);
        }
        std::printf("read: %s, %d tokens\n", path, t.size());
    }
    catch (const std::exception& e)
    {
        std::printf("refused: %s\n", e.what());
    }
}
} // namespace

int main(int argc, char** argv)
{
    byteLayer();
    unicodeClasses();
    utf8Edges();
    preTokenizer();
    for (int i = 1; i < argc; ++i)
        file(argv[i]);
    std::printf("checks: %d failed: %d\n", checks, failures);
    return failures == 0 ? 0 : 1;
}
