// Model/SafeTensors.h — a safetensors file: an 8-byte little-endian header
// length, a JSON header naming each tensor's dtype, shape and byte range, then
// the data blob. The file is mapped, not read; a header that does not describe
// the blob exactly is a ModelError naming the problem, raised when the file is
// opened (Tests/Model/SafeTensorsTests.cpp:212-397 lists the cases).
//
// A SafeTensors is a TensorSource, so DecoderWeights loads straight from one;
// decoderShapeFromConfig reads the HuggingFace config.json the same
// checkpoint ships with (Model/ModelConfig.cpp:58-120, Decoder/DecoderShape.cpp:7-17).
#pragma once

#include "DecoderShape.h"
#include "DecoderWeights.h"

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace WSP
{
// The dtypes a safetensors header may name (Model/TensorType.h:12-27).
enum class TensorType
{
    Bool,
    U8,
    I8,
    U16,
    I16,
    F16,
    BF16,
    U32,
    I32,
    F32,
    U64,
    I64,
    F64
};

const char* tensorTypeName(TensorType type);
int tensorTypeBytes(TensorType type);

struct TensorInfo
{
    std::string name;
    TensorType type = TensorType::F32;
    std::vector<long long> shape;
    std::uint64_t begin = 0, end = 0; // byte range within the blob
    std::uint64_t byteCount = 0;

    int rank() const { return (int) shape.size(); }
    long long dimension(int index) const { return shape.at((std::size_t) index); }
    long long elementCount() const;
};

class SafeTensors final : public TensorSource
{
public:
    // Maps the file; ModelError when it is missing, unmappable or malformed.
    static SafeTensors fromFile(const std::string& path);
    // Parses a copy of these bytes.
    static SafeTensors fromBytes(const void* bytes, std::size_t size);

    SafeTensors(SafeTensors&&) noexcept;
    SafeTensors& operator=(SafeTensors&&) noexcept;
    ~SafeTensors() override;

    const std::vector<TensorInfo>& tensors() const { return entries; } // sorted by name
    std::vector<std::string> names() const;
    const std::map<std::string, std::string>& metadata() const { return meta; }

    bool contains(const std::string& name) const { return findInfo(name) != nullptr; }
    const TensorInfo* findInfo(const std::string& name) const;
    const TensorInfo& info(const std::string& name) const; // ModelError when absent

    // The tensor's bytes within the mapped blob.
    const std::uint8_t* rawBytes(const TensorInfo& tensor) const { return blob + tensor.begin; }
    const std::uint8_t* rawBytes(const std::string& name) const { return rawBytes(info(name)); }

    // F32, F16, BF16 and F64 tensors as floats (F16 and BF16 widened exactly,
    // F64 rounded); any other dtype is a ModelError.
    std::vector<float> readFloats(const std::string& name) const;
    void readFloats(const std::string& name, float* destination, std::size_t capacity) const;

    // TensorSource: the file's tensors as HostTensors pointing into the map.
    const HostTensor* find(const std::string& name) const override;

private:
    SafeTensors() = default;
    void parse(const std::uint8_t* bytes, std::size_t size);

    struct Storage;
    std::unique_ptr<Storage> storage;
    const std::uint8_t* blob = nullptr;
    std::uint64_t blobBytes = 0;
    std::vector<TensorInfo> entries;
    std::map<std::string, std::string> meta;
    std::map<std::string, HostTensor> hostTensors;
};

// A HuggingFace Whisper config.json's decoder extents: d_model,
// decoder_attention_heads, decoder_layers, decoder_ffn_dim, vocab_size,
// max_target_positions; crossPositionCount zero takes max_source_positions.
DecoderShape decoderShapeFromConfig(const std::string& json, int crossPositionCount = 0);
DecoderShape decoderShapeFromConfigFile(const std::string& path, int crossPositionCount = 0);

// The greedy loop's inputs a config.json carries (Model/ModelConfig.cpp:85-101,
// Whisper/Whisper.cpp:202-254): the tokens every step suppresses
// (suppress_tokens), those only the first step also suppresses
// (begin_suppress_tokens), and the start / end-of-text ids (-1 when absent).
struct DecodingConfig
{
    std::vector<int> suppressedTokens;
    std::vector<int> initiallySuppressedTokens;
    int decoderStartToken = -1;
    int endOfTextToken = -1;
    int vocabularySize = 0;

    // Whisper::buildSuppressionMasks: float masks over the vocabulary (1 =
    // suppressed); the first step's adds begin_suppress_tokens. An id outside
    // the vocabulary is a ModelError.
    void suppressionMasks(std::vector<float>& firstStep, std::vector<float>& laterSteps) const;
};

DecodingConfig decodingConfigFromConfig(const std::string& json);
DecodingConfig decodingConfigFromConfigFile(const std::string& path);

// The tokens that steer decoding, by name, out of a HuggingFace
// tokenizer.json's added_tokens (Tokenizer/SpecialTokens.h:16-44,
// Tokenizer/Tokenizer.cpp:102-138): an entry `<|name|>` fills the field of
// that name, a two- or three-letter lowercase name is a language, and
// `<|12.34|>` is a timestamp (the lowest id and its seconds start the run, the
// interval is the seconds spanned over the ids spanned). -1: absent.
struct SpecialTokens
{
    int endOfText = -1;
    int startOfTranscript = -1;
    int startOfPrevious = -1;
    int startOfLanguageModel = -1;
    int translate = -1;
    int transcribe = -1;
    int noTimestamps = -1;
    int noSpeech = -1; // <|nospeech|>, or <|nocaptions|> in older vocabularies
    int firstTimestamp = -1;
    int timestampCount = 0;
    float timestampInterval = 0.0f;
    std::map<std::string, int> languages;

    bool isTimestamp(int token) const;
    int timestampForSeconds(float seconds) const; // -1 outside the run
    float secondsForTimestamp(int token) const;   // -1 for a token outside the run
    int forLanguage(const std::string& code) const;
};

SpecialTokens specialTokensFromTokenizerJson(const std::string& json);
SpecialTokens specialTokensFromTokenizerFile(const std::string& path);

// Whisper::buildPrompt (Whisper/Whisper.cpp:202-225): the English-only prompt
// [start, <|notimestamps|>], the start being config.json's
// decoder_start_token_id when it names one, else the vocabulary's
// <|startoftranscript|>. A ModelError when either is missing.
std::vector<int> transcriptPrompt(const DecodingConfig& config, const SpecialTokens& specials);
} // namespace WSP
