// The host-side file readers (host/SafeTensors.cpp, with host/Half.cpp for
// the widening) driven over files named on the command line, for a build with
// AddressSanitizer and UndefinedBehaviorSanitizer: each malformed file must be
// refused with a ModelError and every well-formed one read in full, with no
// sanitizer report. Test infrastructure (tests/test_safetensors.py runs it).
//
//   safetensors_check open FILE...     SafeTensors::fromFile, then readFloats
//                                       of every floating tensor
//   safetensors_check config FILE...   decoderShapeFromConfigFile and
//                                       decodingConfigFromConfigFile (with masks)
//   safetensors_check tokenizer FILE... specialTokensFromTokenizerFile
//
// Prints one line per file: "refused: <message>", "read: <n> tensors, <m>
// floats" or "config: <width> <heads> ..."; exits 0 unless something other
// than a ModelError escaped.
#include "../../include/whispereacp/ModelError.h"
#include "../../include/whispereacp/SafeTensors.h"

#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace
{
void openFile(const char* path)
{
    const WSP::SafeTensors file = WSP::SafeTensors::fromFile(path);
    std::size_t floats = 0;
    for (const WSP::TensorInfo& t : file.tensors())
    {
        if (t.type != WSP::TensorType::F32 && t.type != WSP::TensorType::F16 && t.type != WSP::TensorType::BF16
            && t.type != WSP::TensorType::F64)
            continue;
        const std::vector<float> values = file.readFloats(t.name);
        floats += values.size();
    }
    std::size_t metadataBytes = 0;
    for (const auto& [key, value] : file.metadata())
        metadataBytes += key.size() + value.size();
    std::printf("read: %zu tensors, %zu floats, %zu metadata bytes\n", file.tensors().size(), floats, metadataBytes);
}

void readConfig(const char* path)
{
    const WSP::DecoderShape s = WSP::decoderShapeFromConfigFile(path);
    const WSP::DecodingConfig d = WSP::decodingConfigFromConfigFile(path);
    WSP::DecodingConfig masked = d;
    masked.vocabularySize = s.vocabularySize;
    std::vector<float> first, later;
    masked.suppressionMasks(first, later);
    std::printf("config: %d %d %d %d %d %d %d, %zu + %zu suppressed\n", s.width, s.heads, s.layers,
                s.feedForwardWidth, s.vocabularySize, s.maxPositions, s.crossPositions, d.suppressedTokens.size(),
                d.initiallySuppressedTokens.size());
}
void readTokenizer(const char* path)
{
    const WSP::SpecialTokens t = WSP::specialTokensFromTokenizerFile(path);
    std::printf("tokenizer: %d %d %d, %zu languages, %d timestamps\n", t.endOfText, t.startOfTranscript,
                t.noTimestamps, t.languages.size(), t.timestampCount);
}
} // namespace

int main(int argc, char** argv)
{
    if (argc < 3
        || (std::strcmp(argv[1], "open") != 0 && std::strcmp(argv[1], "config") != 0
            && std::strcmp(argv[1], "tokenizer") != 0))
    {
        std::fprintf(stderr, "usage: %s open|config|tokenizer FILE...\n", argv[0]);
        return 2;
    }
    const bool config = std::strcmp(argv[1], "config") == 0;
    const bool tokenizer = std::strcmp(argv[1], "tokenizer") == 0;
    for (int i = 2; i < argc; ++i)
    {
        try
        {
            if (tokenizer)
                readTokenizer(argv[i]);
            else if (config)
                readConfig(argv[i]);
            else
                openFile(argv[i]);
        }
        catch (const WSP::ModelError& e)
        {
            std::printf("refused: %s\n", e.what());
        }
        catch (const std::exception& e)
        {
            std::printf("escaped: %s\n", e.what());
            return 1;
        }
    }
    return 0;
}
