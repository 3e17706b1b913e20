// Whisper end to end on gfx950 (Whisper/Whisper.cpp:121-254, 415-460,
// 583-596, 1336-1443, 1497-1507), the kernels backend: the four files parsed at
// load, the device side built at prepare, and a run that uploads one window of
// samples, records the mel and the encoder on the decoder's stream and hands
// the encoded rows to the greedy loop.
#include "../../../include/whispereacp/Whisper.h"
#include "../../../include/whispereacp/ModelError.h"
#include "host_common.h"
#include "json.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <fstream>
#include <limits>
#include <sstream>
#include <sys/stat.h>

namespace WSP
{
namespace
{
const char* const configFile = "config.json";
const char* const preprocessorFile = "preprocessor_config.json";
const char* const tokenizerFile = "tokenizer.json";
const char* const weightsFileName = "model.safetensors";

std::string requireFile(const std::string& directory, const char* name)
{
    const std::string path = directory + "/" + name;
    struct stat info {};
    if (::stat(path.c_str(), &info) != 0 || !S_ISREG(info.st_mode))
        throw ModelError("the model directory " + directory + " has no " + name);
    return path;
}

std::string readText(const std::string& path)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw ModelError("cannot open '" + path + "'");
    std::ostringstream text;
    text << in.rdbuf();
    return text.str();
}

int intField(const Json& object, const char* key)
{
    const Json* v = object.member(key);
    if (v == nullptr)
        throw ModelError(std::string("preprocessor_config.json has no '") + key + "'");
    if (v->kind != Json::Kind::Number || !v->integral || v->integer < std::numeric_limits<int>::min()
        || v->integer > std::numeric_limits<int>::max())
        throw ModelError(std::string("preprocessor_config.json '") + key + "' is not a whole number that fits an int");
    return (int) v->integer;
}

using Clock = std::chrono::steady_clock;

double secondsSince(Clock::time_point start)
{
    return std::chrono::duration<double>(Clock::now() - start).count();
}
} // namespace

// ---------------------------------------------------------------------------
// preprocessor_config.json (Model/PreprocessorConfig.cpp:20-136)
// ---------------------------------------------------------------------------
PreprocessorConfig PreprocessorConfig::fromJson(const std::string& text)
{
    const Json root = JsonReader(text.data(), text.data() + text.size(), "preprocessor_config.json").document();
    if (root.kind != Json::Kind::Object)
        throw ModelError("preprocessor_config.json is not a JSON object");
    PreprocessorConfig c;
    c.sampleRate = intField(root, "sampling_rate");
    c.fftSize = intField(root, "n_fft");
    c.hopSize = intField(root, "hop_length");
    c.melBins = intField(root, "feature_size");
    c.chunkSeconds = intField(root, "chunk_length");
    c.windowSamples = intField(root, "n_samples");
    c.maxFrames = intField(root, "nb_max_frames");
    if (c.sampleRate <= 0 || c.hopSize <= 0 || c.melBins <= 0)
        throw ModelError("preprocessor_config.json has a non-positive rate, hop or mel bin count");
    if (c.fftSize <= 0 || c.fftSize % 2 != 0)
        throw ModelError("preprocessor_config.json n_fft is not a positive even number");

    const Json* filters = root.member("mel_filters");
    if (filters == nullptr)
        throw ModelError("preprocessor_config.json has no 'mel_filters'");
    if (filters->kind != Json::Kind::Array)
        throw ModelError("preprocessor_config.json mel_filters is not an array");
    const int rows = (int) filters->items.size();
    int columns = 0;
    std::vector<float> values;
    for (const Json& row : filters->items)
    {
        if (row.kind != Json::Kind::Array)
            throw ModelError("preprocessor_config.json mel_filters has a row that is not an array");
        if (columns == 0)
            columns = (int) row.items.size();
        else if ((int) row.items.size() != columns)
            throw ModelError("preprocessor_config.json mel_filters is ragged");
        for (const Json& entry : row.items)
        {
            if (entry.kind != Json::Kind::Number)
                throw ModelError("preprocessor_config.json mel_filters is not a number");
            values.push_back((float) entry.number);
        }
    }
    // HF has written the matrix both ways round; hold it mel-major.
    const int bins = c.melBins, wanted = c.melFilterColumns();
    if (rows == bins && columns == wanted)
        c.melFilters = std::move(values);
    else if (rows == wanted && columns == bins)
    {
        c.melFilters.resize(values.size());
        for (int r = 0; r < rows; ++r)
            for (int k = 0; k < columns; ++k)
                c.melFilters[(std::size_t) k * rows + r] = values[(std::size_t) r * columns + k];
    }
    else
        throw ModelError("preprocessor_config.json mel_filters is not " + std::to_string(bins) + " x "
                         + std::to_string(wanted));
    return c;
}

PreprocessorConfig PreprocessorConfig::fromFile(const std::string& path)
{
    return fromJson(readText(path));
}

// ---------------------------------------------------------------------------
// The mel front end's handle (Mel/MelSpectrogram.h:12-25)
// ---------------------------------------------------------------------------
struct Whisper::Mel
{
    wsp_mel* handle = nullptr;

    Mel(const PreprocessorConfig& p, const Device& device, void* stream)
    {
        const wsp_mel_shape s {p.windowSamples, p.fftSize, p.hopSize, p.maxFrames, p.melBins};
        const int status = wsp_mel_create(&s, device.index, stream, &handle);
        if (status == WSP_ERR_SHAPE || status == WSP_ERR_ARGUMENT)
            throw ModelError("preprocessor_config.json's window of " + std::to_string(p.windowSamples)
                             + " samples cannot hold " + std::to_string(p.maxFrames) + " frames of hop "
                             + std::to_string(p.hopSize) + " and an n_fft of " + std::to_string(p.fftSize));
        if (status != WSP_OK)
            throwForStatus(status, "wsp_mel_create failed");
    }
    ~Mel()
    {
        if (handle != nullptr)
            wsp_mel_destroy(handle);
    }
    Mel(const Mel&) = delete;
    Mel& operator=(const Mel&) = delete;
};

// ---------------------------------------------------------------------------
// Whisper
// ---------------------------------------------------------------------------
Whisper::Whisper() = default;

Whisper::~Whisper()
{
    unprepare();
}

void Whisper::load(const std::string& modelDirectory)
{
    ModelFiles files;
    files.config = readText(requireFile(modelDirectory, configFile));
    files.preprocessorConfig = readText(requireFile(modelDirectory, preprocessorFile));
    files.tokenizer = readText(requireFile(modelDirectory, tokenizerFile));
    files.weightsPath = requireFile(modelDirectory, weightsFileName);
    load(files);
}

// The same parses in the same order, whichever way the files arrive; a load
// that throws leaves this unloaded.
void Whisper::load(const ModelFiles& files)
{
    unprepare();
    weightsFile.reset();
    vocabulary.reset();
    decoderExtents.reset();
    encoderExtents.reset();

    configText = files.config;
    decoderExtents = decoderShapeFromConfig(files.config);
    encoderExtents = encoderShapeFromConfig(files.config);
    decoding = decodingConfigFromConfig(files.config);
    preprocessing = PreprocessorConfig::fromJson(files.preprocessorConfig);
    vocabulary.emplace(Tokenizer::fromJsonText(files.tokenizer));
    try
    {
        weightsFile.emplace(SafeTensors::fromFile(files.weightsPath));
        buildGenerationConfig();
    }
    catch (...)
    {
        weightsFile.reset();
        throw;
    }
}

// Whisper/Whisper.cpp:148-254.
void Whisper::buildGenerationConfig()
{
    promptTokens = transcriptPrompt(decoding, vocabulary->specials());
    decoding.suppressionMasks(firstStepSuppression, laterStepSuppression);
    maximumTokenCount = decoderExtents->maxPositions - (int) promptTokens.size();
    audioContextPositions = 0;
}

void Whisper::requireLoaded() const
{
    if (!isLoaded())
        throw ModelError("this Whisper has not loaded a model yet");
}

void Whisper::requirePrepared() const
{
    if (!isPrepared())
        throw ModelError("this Whisper has not been prepared on a device yet");
}

// Whisper/Whisper.cpp:174-200, against this build's shape-generic front end:
// the filterbank, the frame count and the widths must agree between the files.
void Whisper::requireWhisperShapes() const
{
    const EncoderShape& e = *encoderExtents;
    const DecoderShape& d = *decoderExtents;
    if (preprocessing.melBins != e.melBins)
        throw ModelError("this model wants " + std::to_string(e.melBins) + " mel bins and the front-end produces "
                         + std::to_string(preprocessing.melBins));
    if (preprocessing.maxFrames != e.inputFrames)
        throw ModelError("this model wants " + std::to_string(e.inputFrames) + " mel frames and the front-end produces "
                         + std::to_string(preprocessing.maxFrames));
    if (d.width != e.width)
        throw ModelError("config.json's decoder and encoder widths differ");
    if (d.crossPositions != e.positions())
        throw ModelError("config.json max_source_positions is " + std::to_string(d.crossPositions)
                         + " and the encoder's window makes " + std::to_string(e.positions()));
}

void Whisper::setPacksWeights(bool shouldPack)
{
    if (isPrepared())
        throw std::logic_error("weight packing is chosen before prepare()");
    packedWeights = shouldPack;
}

void Whisper::unprepare()
{
    greedy.reset();
    decoder.reset();
    decoderWeights.reset();
    mel.reset();
    encoder.reset();
    encoderWeights.reset();
    sampleBuffer = DeviceBuffer();
    filterBuffer = DeviceBuffer();
    melBuffer = DeviceBuffer();
    encodedBuffer = DeviceBuffer();
    firstMaskBuffer = DeviceBuffer();
    laterMaskBuffer = DeviceBuffer();
    if (stagedSamples != nullptr)
    {
        (void) hipHostFree(stagedSamples);
        stagedSamples = nullptr;
    }
}

// Whisper/Whisper.cpp:462-581: every weight, the filterbank and the masks
// uploaded and every intermediate sized, on `device`, ordered on `hipStream`.
// A prepare that throws leaves this unprepared.
void Whisper::prepare(const Device& deviceToUse, void* hipStream)
{
    unprepare();
    requireLoaded();
    requireWhisperShapes();
    try
    {
        device = deviceToUse;
        stream = hipStream;
        checkHip(hipSetDevice(device.index), "hipSetDevice");
        const WeightPacking packing = packedWeights ? WeightPacking::ExactHalf : WeightPacking::Float;
        const EncoderShape& e = *encoderExtents;
        const DecoderShape& d = *decoderExtents;

        encoderWeights = std::make_unique<EncoderWeights>(*weightsFile, e, packing, device);
        encoder = std::make_unique<Encoder>(e, device, stream);
        mel = std::make_unique<Mel>(preprocessing, device, stream);
        decoderWeights = std::make_unique<DecoderWeights>(*weightsFile, d, packing, device);
        auto built = std::make_unique<Decoder>(d);
        built->prepare(device, stream);
        greedy = std::make_unique<GreedyDecoder>(*built, *decoderWeights, device);

        const std::size_t window = (std::size_t) preprocessing.windowSamples;
        sampleBuffer = DeviceBuffer(device, window * sizeof(float));
        filterBuffer = DeviceBuffer(device, preprocessing.melFilters.data(), preprocessing.melFilters.size() * sizeof(float));
        melBuffer = DeviceBuffer(device, (std::size_t) e.melBins * e.inputFrames * sizeof(float));
        encodedBuffer = DeviceBuffer(device, (std::size_t) e.positions() * e.width * sizeof(float));
        firstMaskBuffer = DeviceBuffer(device, firstStepSuppression.data(), firstStepSuppression.size() * sizeof(float));
        laterMaskBuffer = DeviceBuffer(device, laterStepSuppression.data(), laterStepSuppression.size() * sizeof(float));
        checkHip(hipHostMalloc(reinterpret_cast<void**>(&stagedSamples), window * sizeof(float), 0), "hipHostMalloc");
        decoder = std::move(built);
    }
    catch (...)
    {
        unprepare();
        throw;
    }
}

const DecoderShape& Whisper::decoderShape() const
{
    requireLoaded();
    return *decoderExtents;
}

const EncoderShape& Whisper::encoderShape() const
{
    requireLoaded();
    return *encoderExtents;
}

const PreprocessorConfig& Whisper::preprocessor() const
{
    requireLoaded();
    return preprocessing;
}

const Tokenizer& Whisper::tokenizer() const
{
    requireLoaded();
    return *vocabulary;
}

int Whisper::endOfTextToken() const
{
    requireLoaded();
    return decoding.endOfTextToken >= 0 ? decoding.endOfTextToken : vocabulary->specials().endOfText;
}

void Whisper::setMaximumTokens(int count)
{
    if (count <= 0)
        throw ModelError("a transcript has to be allowed at least one token");
    maximumTokenCount = count;
}

// Whisper/Whisper.cpp:415-428.
void Whisper::setAudioContext(int positions)
{
    requireLoaded();
    const int window = encoderExtents->positions();
    if (positions < 0 || positions > window)
        throw ModelError("an audio context is between 1 and " + std::to_string(window)
                         + " encoder positions, or zero for the whole window, and this one is "
                         + std::to_string(positions));
    audioContextPositions = positions;
}

int Whisper::encodedPositions() const
{
    requireLoaded();
    return audioContextPositions == 0 ? encoderExtents->positions() : audioContextPositions;
}

// Whisper/Whisper.cpp:450-460 with this model's hop and window.
int Whisper::audioContextForSamples(int sampleCount, double marginSeconds) const
{
    requireLoaded();
    const long long samplesPerPosition = (long long) preprocessing.hopSize * EncoderShape::secondConvolutionStride;
    const long long margin = (long long) std::ceil(marginSeconds * preprocessing.sampleRate);
    const long long wanted = std::max(0, sampleCount) + std::max(0LL, margin);
    const long long positions = (wanted + samplesPerPosition - 1) / samplesPerPosition;
    const long long tiles = (positions + audioContextTile - 1) / audioContextTile;
    const int window = encoderExtents->positions();
    return (int) std::clamp<long long>(tiles * audioContextTile, std::min(audioContextFloor, window), window);
}

// Whisper/Whisper.cpp:1336-1351 and 598-680: the samples zero-padded to the
// window and uploaded, the mel and the encoder recorded on the decoder's
// stream, then the greedy loop of Whisper::decodeTranscript.
std::vector<int> Whisper::transcribe(const float* samples, std::size_t count)
{
    requirePrepared();
    const std::size_t window = (std::size_t) preprocessing.windowSamples;
    if (count > window)
        throw ModelError("this run holds " + std::to_string(count) + " samples and one window is "
                         + std::to_string(window) + "; chunking a longer recording is a layer that does not exist");
    if (count > 0 && samples == nullptr)
        throw std::invalid_argument("transcribe: null samples");

    const auto hip = static_cast<hipStream_t>(stream);
    const auto encodeStart = Clock::now();
    checkHip(hipStreamSynchronize(hip), "hipStreamSynchronize"); // the staging buffer is free
    std::copy(samples, samples + count, stagedSamples);
    std::fill(stagedSamples + count, stagedSamples + window, 0.0f);
    checkHip(hipMemcpyAsync(sampleBuffer.data(), stagedSamples, window * sizeof(float), hipMemcpyHostToDevice, hip),
             "upload samples");
    const int melStatus = wsp_mel_encode(mel->handle, static_cast<const float*>(sampleBuffer.data()),
                                         static_cast<const float*>(filterBuffer.data()),
                                         static_cast<float*>(melBuffer.data()));
    if (melStatus != WSP_OK)
        throwForStatus(melStatus, wsp_mel_last_error(mel->handle));
    const int positions = encodedPositions();
    encoder->encode(*encoderWeights, static_cast<const float*>(melBuffer.data()),
                    static_cast<float*>(encodedBuffer.data()), audioContextPositions);
    checkHip(hipStreamSynchronize(hip), "hipStreamSynchronize");
    encodeSeconds = secondsSince(encodeStart);

    Pass pass(stream);
    const GreedyRun run = greedy->decode(pass, BufferRange::of(encodedBuffer), positions, promptTokens,
                                         maximumTokenCount, endOfTextToken(),
                                         static_cast<const float*>(firstMaskBuffer.data()),
                                         static_cast<const float*>(laterMaskBuffer.data()));
    decodeSeconds = run.decodeSeconds;
    stepCount = run.steps;
    return run.tokens;
}

std::string Whisper::transcribeText(const float* samples, std::size_t count)
{
    const std::vector<int> tokens = transcribe(samples, count);
    return textForTokens(tokens);
}

std::string Whisper::textForTokens(const std::vector<int>& tokens) const
{
    requireLoaded();
    return vocabulary->decode(tokens.data(), (int) tokens.size());
}

const float* Whisper::encodedRows() const
{
    requirePrepared();
    return static_cast<const float*>(encodedBuffer.data());
}
} // namespace WSP
