// Whisper end to end on gfx950 (Whisper/Whisper.h:144-560, the kernels
// backend): the four files of a HuggingFace Whisper repo in, the samples of
// one 30 s window through the mel front end, the encoder and the greedy
// decoder, the transcript's tokens and text out.
//
// load() parses config.json, preprocessor_config.json, tokenizer.json and
// maps model.safetensors; it builds the prompt [decoder_start_token_id or
// <|startoftranscript|>, <|notimestamps|>] and the two suppression masks
// (suppress_tokens at every step, begin_suppress_tokens added at the first),
// and touches no GPU. prepare() uploads the weights, the filterbank and the
// masks and sizes every intermediate; transcribe() allocates nothing.
#pragma once

#include "Decoder.h"
#include "DecoderWeights.h"
#include "Encoder.h"
#include "GreedyDecoder.h"
#include "SafeTensors.h"
#include "Tokenizer.h"

#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace WSP
{
// preprocessor_config.json (Model/PreprocessorConfig.h:21-48): the audio
// contract and the mel filterbank, held mel-major ([melBins, fftSize / 2 + 1])
// whichever way round the file serialises it.
struct PreprocessorConfig
{
    int sampleRate = 0;
    int fftSize = 0;
    int hopSize = 0;
    int melBins = 0;
    int chunkSeconds = 0;
    int windowSamples = 0;
    int maxFrames = 0;
    std::vector<float> melFilters;

    int melFilterColumns() const { return fftSize / 2 + 1; }

    static PreprocessorConfig fromJson(const std::string& text);
    static PreprocessorConfig fromFile(const std::string& path);
};

// The same four files as text plus a weights file path
// (Model/ModelFiles.h), for a caller that holds them already.
struct ModelFiles
{
    std::string config;
    std::string preprocessorConfig;
    std::string tokenizer;
    std::string weightsPath;
};

class Whisper
{
public:
    // Whisper/Whisper.h:411-447: positions per second of audio are
    // sampleRate / (hop * 2); a context is rounded up to whole tiles and held
    // between the floor and the window.
    static constexpr int audioContextTile = 64;
    static constexpr int audioContextFloor = 448;
    static constexpr double defaultAudioContextMargin = 2.5;

    Whisper();
    ~Whisper();
    Whisper(const Whisper&) = delete;
    Whisper& operator=(const Whisper&) = delete;

    // A missing file is a ModelError naming it (Whisper/Whisper.cpp:43-51).
    void load(const std::string& modelDirectory);
    void load(const ModelFiles& files);
    bool isLoaded() const { return weightsFile.has_value(); }

    // Set before prepare(): fp16 wherever narrowing is exact, for the
    // projections and the logits' copy of embed_tokens.
    bool packsWeights() const { return packedWeights; }
    void setPacksWeights(bool shouldPack);

    void prepare(const Device& device = Device::shared(), void* hipStream = nullptr);
    bool isPrepared() const { return decoder != nullptr; }

    const DecoderShape& decoderShape() const;
    const EncoderShape& encoderShape() const;
    const PreprocessorConfig& preprocessor() const;
    const Tokenizer& tokenizer() const;

    const std::vector<int>& prompt() const { return promptTokens; }
    const std::vector<float>& firstStepMask() const { return firstStepSuppression; }
    const std::vector<float>& laterStepMask() const { return laterStepSuppression; }
    int endOfTextToken() const;

    int maximumTokens() const { return maximumTokenCount; }
    void setMaximumTokens(int count);

    int audioContext() const { return audioContextPositions; }
    void setAudioContext(int positions);
    int encodedPositions() const;
    int audioContextForSamples(int sampleCount, double marginSeconds = defaultAudioContextMargin) const;

    // At most one window of samples (host memory), zero-padded to the window.
    std::vector<int> transcribe(const float* samples, std::size_t count);
    std::string transcribeText(const float* samples, std::size_t count);
    std::string textForTokens(const std::vector<int>& tokens) const;

    // The last run: mel + encoder (upload to encoded rows, host clock), the
    // decode (first submit to the last token read) and the steps read.
    double lastEncodeSeconds() const { return encodeSeconds; }
    double lastDecodeSeconds() const { return decodeSeconds; }
    int lastStepCount() const { return stepCount; }

    // The encoded rows of the last run (device, [encodedPositions(), width]).
    const float* encodedRows() const;

private:
    struct Mel;

    void buildGenerationConfig();
    void requireLoaded() const;
    void requirePrepared() const;
    void requireWhisperShapes() const;
    void unprepare();

    std::string configText;
    std::optional<DecoderShape> decoderExtents;
    std::optional<EncoderShape> encoderExtents;
    DecodingConfig decoding;
    PreprocessorConfig preprocessing;
    std::optional<Tokenizer> vocabulary;
    std::optional<SafeTensors> weightsFile;

    bool packedWeights = true;
    std::vector<int> promptTokens;
    std::vector<float> firstStepSuppression;
    std::vector<float> laterStepSuppression;
    int maximumTokenCount = 0;
    int audioContextPositions = 0;

    Device device;
    void* stream = nullptr;
    std::unique_ptr<EncoderWeights> encoderWeights;
    std::unique_ptr<Encoder> encoder;
    std::unique_ptr<Mel> mel;
    std::unique_ptr<DecoderWeights> decoderWeights;
    std::unique_ptr<Decoder> decoder;
    std::unique_ptr<GreedyDecoder> greedy;
    DeviceBuffer sampleBuffer, filterBuffer, melBuffer, encodedBuffer, firstMaskBuffer, laterMaskBuffer;
    float* stagedSamples = nullptr; // pinned, one window

    double encodeSeconds = 0.0;
    double decodeSeconds = 0.0;
    int stepCount = 0;
};
} // namespace WSP
