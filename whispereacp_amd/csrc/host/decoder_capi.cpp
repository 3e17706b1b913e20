// The C binding of the C++ decoder surface (include/wsp_decoder.h): every
// exception the reference would throw is caught here and returned as a status
// plus its kind and message.
#include "../../../include/wsp_decoder.h"
#include "../../../include/whispereacp/Argmax.h"
#include "../../../include/whispereacp/BatchedDecoder.h"
#include "../../../include/whispereacp/Decoder.h"
#include "../../../include/whispereacp/GreedyDecoder.h"
#include "../../../include/whispereacp/SafeTensors.h"
#include "../../../include/whispereacp/Tokenizer.h"
#include "../../../include/whispereacp/Whisper.h"

#include <algorithm>
#include <climits>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>

struct wsp_decoder
{
    WSP::DecoderShape shape;
    WSP::Device device;
    void* stream = nullptr;
    std::unique_ptr<WSP::DecoderWeights> weights;
    std::unique_ptr<WSP::Decoder> decoder;
    std::unique_ptr<WSP::Argmax> selection;
    std::unique_ptr<WSP::GreedyDecoder> greedy;
    std::string error;
    int errorKind = WSP_KIND_NONE;
};

struct wsp_safetensors
{
    std::unique_ptr<WSP::SafeTensors> file;
    std::string error;
    int errorKind = WSP_KIND_NONE;
};

struct wsp_whisper
{
    WSP::Whisper whisper;
    std::string error;
    int errorKind = WSP_KIND_NONE;
};

struct wsp_batch_decoder
{
    WSP::DecoderShape shape;
    WSP::Device device;
    std::unique_ptr<WSP::DecoderWeights> weights;
    std::unique_ptr<WSP::BatchedDecoder> decoder;
    std::string error;
    int errorKind = WSP_KIND_NONE;
};

namespace
{
template <typename Handle, typename Body>
int guarded(Handle* d, Body body)
{
    if (d == nullptr)
        return WSP_ERR_ARGUMENT;
    d->error.clear();
    d->errorKind = WSP_KIND_NONE;
    try
    {
        body();
        return WSP_OK;
    }
    catch (const WSP::ModelError& e)
    {
        d->error = e.what();
        d->errorKind = WSP_KIND_MODEL_ERROR;
        return WSP_ERR_SHAPE;
    }
    catch (const std::invalid_argument& e)
    {
        d->error = e.what();
        d->errorKind = WSP_KIND_INVALID_ARGUMENT;
        return WSP_ERR_CAPACITY;
    }
    catch (const std::logic_error& e)
    {
        d->error = e.what();
        d->errorKind = WSP_KIND_LOGIC_ERROR;
        return WSP_ERR_LOGIC;
    }
    catch (const std::exception& e)
    {
        d->error = e.what();
        d->errorKind = WSP_KIND_RUNTIME_ERROR;
        return WSP_ERR_HIP;
    }
}

WSP::BufferRange range(const void* p, std::size_t bytes)
{
    return {const_cast<void*>(p), 0, bytes};
}

WSP::DecoderShape checkedShape(const wsp_decoder_shape* shape)
{
    WSP::DecoderShape s {shape->width,           shape->heads,         shape->layers,       shape->feed_forward_width,
                         shape->vocabulary_size, shape->max_positions, shape->cross_positions};
    if (s.width <= 0 || s.heads <= 0 || s.width % s.heads != 0 || s.layers <= 0 || s.feedForwardWidth <= 0
        || s.vocabularySize <= 0 || s.maxPositions <= 0 || s.crossPositions <= 0)
        throw WSP::ModelError("a decoder shape needs positive extents and a width divisible by its heads");
    return s;
}

WSP::MapTensorSource sourceOf(const wsp_tensor_entry* tensors, int count)
{
    WSP::MapTensorSource source;
    for (int i = 0; i < count; ++i)
    {
        const wsp_tensor_entry& e = tensors[i];
        if (e.name == nullptr || e.dtype == nullptr || e.rank < 0 || (e.rank > 0 && e.extents == nullptr))
            throw std::invalid_argument("tensor entry " + std::to_string(i) + " is incomplete");
        WSP::HostTensor t;
        t.dtype = e.dtype;
        t.extents.assign(e.extents, e.extents + e.rank);
        t.data = e.data;
        source.add(e.name, std::move(t));
    }
    return source;
}

WSP::WeightPacking packingOf(int packing)
{
    return packing == 1 ? WSP::WeightPacking::ExactHalf : WSP::WeightPacking::Float;
}

// DecoderWeights + Decoder + Argmax + the greedy loop's buffers, every buffer
// sized once, so no later call allocates.
void buildDecoder(wsp_decoder* d, const WSP::TensorSource& source, int packing, void* stream)
{
    d->weights = std::make_unique<WSP::DecoderWeights>(source, d->shape, packingOf(packing), d->device);
    d->decoder = std::make_unique<WSP::Decoder>(d->shape);
    d->decoder->prepare(d->device, stream);
    d->selection = std::make_unique<WSP::Argmax>();
    d->selection->prepare(d->device, d->shape.maxPositions, d->shape.vocabularySize, stream);
    d->greedy = std::make_unique<WSP::GreedyDecoder>(*d->decoder, *d->weights, d->device);
}

void buildBatch(wsp_batch_decoder* d, const WSP::TensorSource& source, int packing, int streams, int maxStepTokens,
                void* stream)
{
    d->weights = std::make_unique<WSP::DecoderWeights>(source, d->shape, packingOf(packing), d->device);
    d->decoder = std::make_unique<WSP::BatchedDecoder>(d->shape, streams, maxStepTokens);
    d->decoder->prepare(*d->weights, d->device, stream);
}
} // namespace

extern "C" {

int wsp_decoder_create(const wsp_decoder_shape* shape, const wsp_tensor_entry* tensors, int count, int packing,
                       int device, void* stream, wsp_decoder** out)
{
    if (shape == nullptr || out == nullptr || (count > 0 && tensors == nullptr))
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    auto* d = new (std::nothrow) wsp_decoder {};
    if (d == nullptr)
        return WSP_ERR_CAPACITY;
    const int status = guarded(d, [&] {
        d->shape = checkedShape(shape);
        d->device = WSP::Device {device};
        d->stream = stream;
        const WSP::MapTensorSource source = sourceOf(tensors, count);
        buildDecoder(d, source, packing, stream);
    });
    if (status != WSP_OK)
    {
        // Keep the object so the caller can read why; it is unusable otherwise.
        d->greedy.reset();
        d->decoder.reset();
        d->weights.reset();
        *out = d;
        return status;
    }
    *out = d;
    return WSP_OK;
}

int wsp_decoder_create_from_file(const char* path, const wsp_decoder_shape* shape, int packing, int device,
                                 void* stream, wsp_decoder** out)
{
    if (path == nullptr || shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    auto* d = new (std::nothrow) wsp_decoder {};
    if (d == nullptr)
        return WSP_ERR_CAPACITY;
    const int status = guarded(d, [&] {
        d->shape = checkedShape(shape);
        d->device = WSP::Device {device};
        d->stream = stream;
        const WSP::SafeTensors file = WSP::SafeTensors::fromFile(path);
        buildDecoder(d, file, packing, stream);
    });
    if (status != WSP_OK)
    {
        d->greedy.reset();
        d->decoder.reset();
        d->weights.reset();
    }
    *out = d;
    return status;
}

void wsp_decoder_destroy(wsp_decoder* d)
{
    delete d;
}

const char* wsp_decoder_last_error(const wsp_decoder* d)
{
    return d == nullptr ? "no decoder" : d->error.c_str();
}

int wsp_decoder_last_error_kind(const wsp_decoder* d)
{
    return d == nullptr ? WSP_KIND_INVALID_ARGUMENT : d->errorKind;
}

int wsp_decoder_begin_sequence(wsp_decoder* d, const float* encoder_rows, int cross_position_count)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("the decoder was not created");
        WSP::Pass pass(d->stream);
        d->decoder->beginSequence(pass, range(encoder_rows, (std::size_t) d->shape.crossElementCount() * 4),
                                  *d->weights, cross_position_count);
    });
}

int wsp_decoder_step(wsp_decoder* d, const uint32_t* tokens, int count, float* logits)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("the decoder was not created");
        WSP::Pass pass(d->stream);
        d->decoder->step(pass, range(tokens, (std::size_t) (count > 0 ? count : 0) * 4), count, *d->weights,
                         range(logits, (std::size_t) (count > 0 ? count : 0) * d->shape.vocabularySize * 4));
    });
}

int wsp_decoder_step_and_sample(wsp_decoder* d, const uint32_t* token, float* logits, const float* mask,
                                uint32_t* argmax_slot)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("the decoder was not created");
        WSP::Pass pass(d->stream);
        d->decoder->stepAndSample(pass, range(token, 4), *d->weights,
                                  range(logits, (std::size_t) d->shape.vocabularySize * 4), mask,
                                  range(argmax_slot, 4));
    });
}

int wsp_decoder_position(const wsp_decoder* d)
{
    return d != nullptr && d->decoder ? d->decoder->position() : -1;
}

int wsp_decoder_cross_positions(const wsp_decoder* d)
{
    return d != nullptr && d->decoder ? d->decoder->crossPositions() : -1;
}

const float* wsp_decoder_hidden_states(const wsp_decoder* d)
{
    return d != nullptr && d->decoder ? static_cast<const float*>(d->decoder->hiddenStates().data()) : nullptr;
}

int wsp_decoder_set_fused(wsp_decoder* d, int enabled)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("the decoder was not created");
        d->decoder->setFusedSteps(enabled != 0);
    });
}

int wsp_decoder_uses_fused(const wsp_decoder* d)
{
    return d != nullptr && d->decoder && d->decoder->usesFusedStep(*d->weights, 1) ? 1 : 0;
}

int wsp_decoder_step_persistent(const wsp_decoder* d)
{
    return d != nullptr && d->decoder ? wsp_hip_step_persistent(d->decoder->net().context()) : 0;
}

int wsp_decoder_device_status(wsp_decoder* d, int* status, int clear)
{
    if (d == nullptr || !d->decoder || status == nullptr)
        return WSP_ERR_ARGUMENT;
    return wsp_hip_device_status(d->decoder->net().context(), status, clear);
}

int wsp_decoder_raise_device_status(wsp_decoder* d)
{
    if (d == nullptr || !d->decoder)
        return WSP_ERR_ARGUMENT;
    return wsp_hip_raise_device_status(d->decoder->net().context());
}

int wsp_decoder_argmax(wsp_decoder* d, const float* logits, int rows, int row_length, const float* mask,
                       uint32_t* out)
{
    return guarded(d, [&] {
        if (!d->selection)
            throw std::logic_error("the decoder was not created");
        WSP::Pass pass(d->stream);
        d->selection->encode(pass, range(logits, (std::size_t) rows * row_length * 4), mask,
                             range(out, (std::size_t) rows * 4), rows, row_length);
    });
}

int wsp_decoder_greedy(wsp_decoder* d, const float* encoder_rows, int cross_position_count, const int* prompt,
                       int prompt_count, int maximum_tokens, int end_of_text, const float* first_mask,
                       const float* later_mask, int* tokens_out, int capacity, int* count_out,
                       double* decode_seconds)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("the decoder was not created");
        if (prompt == nullptr || prompt_count <= 0 || tokens_out == nullptr || count_out == nullptr)
            throw std::invalid_argument("greedy decode needs a prompt and somewhere to put the tokens");
        if (!d->greedy)
            throw std::logic_error("the decoder was not created");
        WSP::Pass pass(d->stream);
        const std::vector<int> promptTokens(prompt, prompt + prompt_count);
        const WSP::GreedyRun run = d->greedy->decode(
            pass, range(encoder_rows, (std::size_t) d->shape.crossElementCount() * 4), cross_position_count,
            promptTokens, maximum_tokens, end_of_text, first_mask, later_mask);
        const int total = (int) run.tokens.size();
        const int n = std::min(total, std::max(capacity, 0));
        for (int i = 0; i < n; ++i)
            tokens_out[i] = run.tokens[(std::size_t) i];
        *count_out = total;
        if (decode_seconds != nullptr)
            *decode_seconds = run.decodeSeconds;
        if (total > n)
            throw std::invalid_argument("greedy decode: " + std::to_string(total) + " tokens, room for "
                                        + std::to_string(n) + " (the first " + std::to_string(n)
                                        + " were written)");
    });
}

int wsp_batch_decoder_create(const wsp_decoder_shape* shape, const wsp_tensor_entry* tensors, int count,
                             int packing, int streams, int max_step_tokens, int device, void* stream,
                             wsp_batch_decoder** out)
{
    if (shape == nullptr || out == nullptr || (count > 0 && tensors == nullptr))
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    auto* d = new (std::nothrow) wsp_batch_decoder {};
    if (d == nullptr)
        return WSP_ERR_CAPACITY;
    const int status = guarded(d, [&] {
        d->shape = checkedShape(shape);
        d->device = WSP::Device {device};
        const WSP::MapTensorSource source = sourceOf(tensors, count);
        buildBatch(d, source, packing, streams, max_step_tokens, stream);
    });
    if (status != WSP_OK)
    {
        d->decoder.reset();
        d->weights.reset();
    }
    *out = d;
    return status;
}

void wsp_batch_decoder_destroy(wsp_batch_decoder* d)
{
    delete d;
}

const char* wsp_batch_decoder_last_error(const wsp_batch_decoder* d)
{
    return d == nullptr ? "no decoder" : d->error.c_str();
}

int wsp_batch_decoder_last_error_kind(const wsp_batch_decoder* d)
{
    return d == nullptr ? WSP_KIND_INVALID_ARGUMENT : d->errorKind;
}

int wsp_batch_decoder_begin(wsp_batch_decoder* d, const float* encoder_rows, int cross_position_count)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("this batched decoder failed to build");
        const int rows = cross_position_count == 0 ? d->shape.crossPositions : cross_position_count;
        const std::size_t bytes = sizeof(float) * (std::size_t) d->decoder->streams() * (std::size_t) std::max(rows, 0)
                                  * d->shape.width;
        WSP::Pass pass(d->decoder->hipStream());
        d->decoder->beginSequences(pass, range(encoder_rows, bytes), *d->weights, cross_position_count);
    });
}

int wsp_batch_decoder_step(wsp_batch_decoder* d, const uint32_t* tokens, int count, float* logits, const float* mask,
                           uint32_t* argmax_slots)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("this batched decoder failed to build");
        const std::size_t rows = (std::size_t) d->decoder->streams() * (std::size_t) std::max(count, 0);
        WSP::Pass pass(d->decoder->hipStream());
        const auto t = range(tokens, rows * sizeof(uint32_t));
        const auto l = range(logits, rows * d->shape.vocabularySize * sizeof(float));
        if (argmax_slots == nullptr)
            d->decoder->step(pass, t, count, *d->weights, l);
        else
            d->decoder->stepAndSample(pass, t, count, *d->weights, l, mask,
                                      range(argmax_slots, (std::size_t) d->decoder->streams() * sizeof(uint32_t)));
    });
}

int wsp_batch_decoder_ring_step(wsp_batch_decoder* d, uint32_t* ring, float* logits, const float* mask)
{
    return guarded(d, [&] {
        if (!d->decoder)
            throw std::logic_error("this batched decoder failed to build");
        const std::size_t streams = (std::size_t) d->decoder->streams();
        WSP::Pass pass(d->decoder->hipStream());
        d->decoder->ringStep(pass, range(ring, (std::size_t) (d->shape.maxPositions + 1) * streams * sizeof(uint32_t)),
                             *d->weights, range(logits, streams * d->shape.vocabularySize * sizeof(float)), mask);
    });
}

int wsp_batch_decoder_position(const wsp_batch_decoder* d)
{
    return d == nullptr || !d->decoder ? -1 : d->decoder->position();
}

int wsp_batch_decoder_product_storage(const wsp_batch_decoder* d)
{
    return d == nullptr || !d->decoder ? 0 : d->decoder->productStorage();
}

const float* wsp_batch_decoder_hidden_states(const wsp_batch_decoder* d)
{
    return d == nullptr || !d->decoder ? nullptr : static_cast<const float*>(d->decoder->hiddenStates().data());
}

int wsp_batch_decoder_create_from_file(const char* path, const wsp_decoder_shape* shape, int packing, int streams,
                                       int max_step_tokens, int device, void* stream, wsp_batch_decoder** out)
{
    if (path == nullptr || shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    auto* d = new (std::nothrow) wsp_batch_decoder {};
    if (d == nullptr)
        return WSP_ERR_CAPACITY;
    const int status = guarded(d, [&] {
        d->shape = checkedShape(shape);
        d->device = WSP::Device {device};
        const WSP::SafeTensors file = WSP::SafeTensors::fromFile(path);
        buildBatch(d, file, packing, streams, max_step_tokens, stream);
    });
    if (status != WSP_OK)
    {
        d->decoder.reset();
        d->weights.reset();
    }
    *out = d;
    return status;
}

int wsp_safetensors_open(const char* path, wsp_safetensors** out)
{
    if (path == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    auto* f = new (std::nothrow) wsp_safetensors {};
    if (f == nullptr)
        return WSP_ERR_CAPACITY;
    *out = f;
    return guarded(f, [&] { f->file = std::make_unique<WSP::SafeTensors>(WSP::SafeTensors::fromFile(path)); });
}

int wsp_safetensors_open_bytes(const void* bytes, size_t size, wsp_safetensors** out)
{
    if ((bytes == nullptr && size > 0) || out == nullptr)
        return WSP_ERR_ARGUMENT;
    auto* f = new (std::nothrow) wsp_safetensors {};
    if (f == nullptr)
        return WSP_ERR_CAPACITY;
    *out = f;
    return guarded(f, [&] { f->file = std::make_unique<WSP::SafeTensors>(WSP::SafeTensors::fromBytes(bytes, size)); });
}

void wsp_safetensors_close(wsp_safetensors* f)
{
    delete f;
}

const char* wsp_safetensors_last_error(const wsp_safetensors* f)
{
    return f == nullptr ? "no file" : f->error.c_str();
}

int wsp_safetensors_count(const wsp_safetensors* f)
{
    return f == nullptr || !f->file ? -1 : (int) f->file->tensors().size();
}

int wsp_safetensors_tensor(const wsp_safetensors* f, int index, const char** name, const char** dtype, int* rank,
                           long long* extents, int capacity, long long* byte_count)
{
    if (f == nullptr || !f->file || index < 0 || index >= (int) f->file->tensors().size())
        return WSP_ERR_ARGUMENT;
    const WSP::TensorInfo& t = f->file->tensors()[(std::size_t) index];
    if (name != nullptr)
        *name = t.name.c_str();
    if (dtype != nullptr)
        *dtype = WSP::tensorTypeName(t.type);
    if (rank != nullptr)
        *rank = t.rank();
    if (extents != nullptr)
        for (int i = 0; i < t.rank() && i < capacity; ++i)
            extents[i] = t.shape[(std::size_t) i];
    if (byte_count != nullptr)
        *byte_count = (long long) t.byteCount;
    return WSP_OK;
}

int wsp_safetensors_read_floats(wsp_safetensors* f, const char* name, float* out, long long capacity)
{
    return guarded(f, [&] {
        if (!f->file)
            throw std::logic_error("this safetensors file failed to open");
        if (name == nullptr || (out == nullptr && capacity > 0) || capacity < 0)
            throw std::invalid_argument("wsp_safetensors_read_floats: null name or destination");
        f->file->readFloats(name, out, (std::size_t) capacity);
    });
}

const char* wsp_safetensors_metadata(const wsp_safetensors* f, const char* key)
{
    if (f == nullptr || !f->file || key == nullptr)
        return nullptr;
    const auto it = f->file->metadata().find(key);
    return it == f->file->metadata().end() ? nullptr : it->second.c_str();
}

int wsp_decoding_from_config(const char* config_path, float* first_mask, float* later_mask, int capacity,
                             int* start_token, int* end_token, char* error, int error_capacity)
{
    if (config_path == nullptr)
        return WSP_ERR_ARGUMENT;
    try
    {
        const WSP::DecodingConfig config = WSP::decodingConfigFromConfigFile(config_path);
        if (first_mask != nullptr || later_mask != nullptr)
        {
            if (capacity < config.vocabularySize)
                throw WSP::ModelError("the masks hold fewer floats than config.json's vocab_size");
            std::vector<float> first, later;
            config.suppressionMasks(first, later);
            if (first_mask != nullptr)
                std::memcpy(first_mask, first.data(), first.size() * sizeof(float));
            if (later_mask != nullptr)
                std::memcpy(later_mask, later.data(), later.size() * sizeof(float));
        }
        if (start_token != nullptr)
            *start_token = config.decoderStartToken;
        if (end_token != nullptr)
            *end_token = config.endOfTextToken;
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        if (error != nullptr && error_capacity > 0)
        {
            std::strncpy(error, e.what(), (std::size_t) error_capacity - 1);
            error[error_capacity - 1] = 0;
        }
        return WSP_ERR_SHAPE;
    }
}

namespace
{
int reportModelError(const std::exception& e, char* error, int error_capacity)
{
    if (error != nullptr && error_capacity > 0)
    {
        std::strncpy(error, e.what(), (std::size_t) error_capacity - 1);
        error[error_capacity - 1] = 0;
    }
    return WSP_ERR_SHAPE;
}
} // namespace

int wsp_special_tokens_from_file(const char* tokenizer_path, wsp_special_tokens* out, char* error,
                                 int error_capacity)
{
    if (tokenizer_path == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    try
    {
        const WSP::SpecialTokens t = WSP::specialTokensFromTokenizerFile(tokenizer_path);
        *out = wsp_special_tokens {t.endOfText,     t.startOfTranscript,
                                   t.startOfPrevious, t.startOfLanguageModel,
                                   t.translate,     t.transcribe,
                                   t.noTimestamps,  t.noSpeech,
                                   t.firstTimestamp, t.timestampCount,
                                   t.timestampInterval, (int) t.languages.size(),
                                   t.forLanguage("en")};
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        return reportModelError(e, error, error_capacity);
    }
}

int wsp_prompt_from_files(const char* config_path, const char* tokenizer_path, int* prompt_out, int capacity,
                          int* count_out, char* error, int error_capacity)
{
    if (config_path == nullptr || tokenizer_path == nullptr || prompt_out == nullptr || count_out == nullptr)
        return WSP_ERR_ARGUMENT;
    try
    {
        const std::vector<int> prompt = WSP::transcriptPrompt(WSP::decodingConfigFromConfigFile(config_path),
                                                              WSP::specialTokensFromTokenizerFile(tokenizer_path));
        *count_out = (int) prompt.size();
        if ((int) prompt.size() > capacity)
            throw WSP::ModelError("the prompt holds " + std::to_string(prompt.size()) + " tokens, more than the "
                                  + std::to_string(capacity) + " the buffer takes");
        std::copy(prompt.begin(), prompt.end(), prompt_out);
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        return reportModelError(e, error, error_capacity);
    }
}

int wsp_shape_from_config(const char* config_path, int cross_positions, wsp_decoder_shape* out, char* error,
                          int error_capacity)
{
    if (config_path == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    try
    {
        *out = WSP::decoderShapeFromConfigFile(config_path, cross_positions).toC();
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        if (error != nullptr && error_capacity > 0)
        {
            std::strncpy(error, e.what(), (std::size_t) error_capacity - 1);
            error[error_capacity - 1] = 0;
        }
        return WSP_ERR_SHAPE;
    }
}

} // extern "C"

// ---------------------------------------------------------------------------
// The tokenizer
// ---------------------------------------------------------------------------
struct wsp_tokenizer
{
    WSP::Tokenizer tokenizer;
};

extern "C" {

int wsp_tokenizer_open_bytes(const char* json, size_t length, wsp_tokenizer** out, char* error, int error_capacity)
{
    if (json == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    try
    {
        *out = new wsp_tokenizer {WSP::Tokenizer::fromJsonText(std::string_view(json, length))};
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        return reportModelError(e, error, error_capacity);
    }
}

int wsp_tokenizer_open(const char* path, wsp_tokenizer** out, char* error, int error_capacity)
{
    if (path == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    try
    {
        *out = new wsp_tokenizer {WSP::Tokenizer::fromFile(path)};
        return WSP_OK;
    }
    catch (const std::exception& e)
    {
        return reportModelError(e, error, error_capacity);
    }
}

void wsp_tokenizer_close(wsp_tokenizer* t)
{
    delete t;
}

int wsp_tokenizer_size(const wsp_tokenizer* t)
{
    return t == nullptr ? WSP_ERR_ARGUMENT : t->tokenizer.size();
}

int wsp_tokenizer_is_special(const wsp_tokenizer* t, int token)
{
    return t != nullptr && t->tokenizer.isSpecial(token) ? 1 : 0;
}

int wsp_tokenizer_token_for_text(const wsp_tokenizer* t, const char* text, size_t length)
{
    if (t == nullptr || text == nullptr)
        return WSP::invalidTokenId;
    return t->tokenizer.tokenForText(std::string_view(text, length));
}

int wsp_tokenizer_encode(const wsp_tokenizer* t, const char* text, size_t length, int* ids_out, int capacity,
                         int* count_out)
{
    if (t == nullptr || (text == nullptr && length > 0) || count_out == nullptr || capacity < 0
        || (ids_out == nullptr && capacity > 0))
        return WSP_ERR_ARGUMENT;
    try
    {
        const std::vector<int> ids = t->tokenizer.encode(std::string_view(text == nullptr ? "" : text, length));
        if (ids.size() > (size_t) INT_MAX)
            return WSP_ERR_CAPACITY;
        *count_out = (int) ids.size();
        if ((int) ids.size() > capacity)
            return WSP_ERR_CAPACITY;
        std::copy(ids.begin(), ids.end(), ids_out);
        return WSP_OK;
    }
    catch (const std::bad_alloc&)
    {
        return WSP_ERR_CAPACITY;
    }
    catch (const std::exception&)
    {
        return WSP_ERR_ARGUMENT;
    }
}

int wsp_tokenizer_decode(const wsp_tokenizer* t, const int* ids, int count, int keep_special, char* text_out,
                         int capacity, int* length_out)
{
    if (t == nullptr || (ids == nullptr && count > 0) || count < 0 || length_out == nullptr || text_out == nullptr
        || capacity <= 0)
        return WSP_ERR_ARGUMENT;
    try
    {
        const std::string text = keep_special ? t->tokenizer.decodeKeepingSpecialTokens(ids, count)
                                              : t->tokenizer.decode(ids, count);
        if (text.size() >= (size_t) INT_MAX)
            return WSP_ERR_CAPACITY;
        *length_out = (int) text.size();
        if ((int) text.size() >= capacity)
            return WSP_ERR_CAPACITY;
        std::memcpy(text_out, text.data(), text.size());
        text_out[text.size()] = 0;
        return WSP_OK;
    }
    catch (const std::bad_alloc&)
    {
        return WSP_ERR_CAPACITY;
    }
    catch (const std::exception&)
    {
        return WSP_ERR_ARGUMENT;
    }
}

} // extern "C"

// ---- Whisper end to end ---------------------------------------------------
namespace
{
// A tokenizer.json the tokenizer refuses is a model file the load refuses.
template <typename Body>
int whisperGuarded(wsp_whisper* w, Body body)
{
    return guarded(w, [&] {
        try
        {
            body();
        }
        catch (const WSP::TokenizerError& e)
        {
            throw WSP::ModelError(e.what());
        }
    });
}
} // namespace

extern "C" {

int wsp_whisper_create(wsp_whisper** out)
{
    if (out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = new (std::nothrow) wsp_whisper {};
    return *out == nullptr ? WSP_ERR_CAPACITY : WSP_OK;
}

void wsp_whisper_destroy(wsp_whisper* w)
{
    delete w;
}

const char* wsp_whisper_last_error(const wsp_whisper* w)
{
    return w == nullptr ? "null whisper" : w->error.c_str();
}

int wsp_whisper_last_error_kind(const wsp_whisper* w)
{
    return w == nullptr ? WSP_KIND_NONE : w->errorKind;
}

int wsp_whisper_load(wsp_whisper* w, const char* model_directory)
{
    return whisperGuarded(w, [&] {
        if (model_directory == nullptr)
            throw std::invalid_argument("wsp_whisper_load: null directory");
        w->whisper.load(std::string(model_directory));
    });
}

int wsp_whisper_load_files(wsp_whisper* w, const char* config_json, const char* preprocessor_json,
                           const char* tokenizer_json, const char* weights_path)
{
    return whisperGuarded(w, [&] {
        if (config_json == nullptr || preprocessor_json == nullptr || tokenizer_json == nullptr
            || weights_path == nullptr)
            throw std::invalid_argument("wsp_whisper_load_files: a null file");
        WSP::ModelFiles files;
        files.config = config_json;
        files.preprocessorConfig = preprocessor_json;
        files.tokenizer = tokenizer_json;
        files.weightsPath = weights_path;
        w->whisper.load(files);
    });
}

int wsp_whisper_set_packs_weights(wsp_whisper* w, int pack)
{
    return guarded(w, [&] { w->whisper.setPacksWeights(pack != 0); });
}

int wsp_whisper_prepare(wsp_whisper* w, int device, void* stream)
{
    return guarded(w, [&] { w->whisper.prepare(WSP::Device {device}, stream); });
}

int wsp_whisper_prompt(wsp_whisper* w, int* tokens_out, int capacity, int* count_out)
{
    return guarded(w, [&] {
        if (count_out == nullptr || capacity < 0 || (tokens_out == nullptr && capacity > 0))
            throw std::invalid_argument("wsp_whisper_prompt: no room described");
        if (!w->whisper.isLoaded())
            throw WSP::ModelError("this Whisper has not loaded a model yet");
        const std::vector<int>& p = w->whisper.prompt();
        *count_out = (int) p.size();
        if ((int) p.size() > capacity)
            throw std::invalid_argument("wsp_whisper_prompt: " + std::to_string(p.size()) + " tokens, room for "
                                        + std::to_string(capacity));
        std::copy(p.begin(), p.end(), tokens_out);
    });
}

int wsp_whisper_masks(wsp_whisper* w, float* first_mask, float* later_mask, int capacity)
{
    return guarded(w, [&] {
        if (!w->whisper.isLoaded())
            throw WSP::ModelError("this Whisper has not loaded a model yet");
        const auto& first = w->whisper.firstStepMask();
        const auto& later = w->whisper.laterStepMask();
        if ((first_mask != nullptr || later_mask != nullptr) && capacity < (int) first.size())
            throw std::invalid_argument("wsp_whisper_masks: the masks are " + std::to_string(first.size())
                                        + " floats long");
        if (first_mask != nullptr)
            std::copy(first.begin(), first.end(), first_mask);
        if (later_mask != nullptr)
            std::copy(later.begin(), later.end(), later_mask);
    });
}

int wsp_whisper_end_of_text(wsp_whisper* w, int* token_out)
{
    return guarded(w, [&] {
        if (token_out == nullptr)
            throw std::invalid_argument("wsp_whisper_end_of_text: null output");
        *token_out = w->whisper.endOfTextToken();
    });
}

int wsp_whisper_set_maximum_tokens(wsp_whisper* w, int count)
{
    return guarded(w, [&] { w->whisper.setMaximumTokens(count); });
}

int wsp_whisper_maximum_tokens(wsp_whisper* w, int* count_out)
{
    return guarded(w, [&] {
        if (count_out == nullptr)
            throw std::invalid_argument("wsp_whisper_maximum_tokens: null output");
        *count_out = w->whisper.maximumTokens();
    });
}

int wsp_whisper_set_audio_context(wsp_whisper* w, int positions)
{
    return guarded(w, [&] { w->whisper.setAudioContext(positions); });
}

int wsp_whisper_audio_context_for_samples(wsp_whisper* w, int sample_count, double margin_seconds,
                                          int* positions_out)
{
    return guarded(w, [&] {
        if (positions_out == nullptr)
            throw std::invalid_argument("wsp_whisper_audio_context_for_samples: null output");
        *positions_out = w->whisper.audioContextForSamples(sample_count, margin_seconds);
    });
}

int wsp_whisper_transcribe(wsp_whisper* w, const float* samples, int sample_count, int* tokens_out, int capacity,
                           int* count_out)
{
    return guarded(w, [&] {
        if (sample_count < 0 || count_out == nullptr || capacity < 0 || (tokens_out == nullptr && capacity > 0))
            throw std::invalid_argument("wsp_whisper_transcribe: bad sample count or output");
        const std::vector<int> tokens = w->whisper.transcribe(samples, (std::size_t) sample_count);
        *count_out = (int) tokens.size();
        const int n = std::min((int) tokens.size(), capacity);
        std::copy(tokens.begin(), tokens.begin() + n, tokens_out);
        if ((int) tokens.size() > capacity)
            throw std::invalid_argument("wsp_whisper_transcribe: " + std::to_string(tokens.size())
                                        + " tokens, room for " + std::to_string(capacity) + " (the first "
                                        + std::to_string(n) + " were written)");
    });
}

int wsp_whisper_text_for_tokens(wsp_whisper* w, const int* tokens, int count, char* text_out, int capacity,
                                int* length_out)
{
    return guarded(w, [&] {
        if (count < 0 || (tokens == nullptr && count > 0) || length_out == nullptr || text_out == nullptr
            || capacity <= 0)
            throw std::invalid_argument("wsp_whisper_text_for_tokens: bad tokens or output");
        const std::string text = w->whisper.textForTokens(std::vector<int>(tokens, tokens + count));
        *length_out = (int) text.size();
        if ((int) text.size() >= capacity)
            throw std::invalid_argument("wsp_whisper_text_for_tokens: " + std::to_string(text.size())
                                        + " bytes and a NUL, room for " + std::to_string(capacity));
        std::memcpy(text_out, text.data(), text.size());
        text_out[text.size()] = 0;
    });
}

int wsp_whisper_timing(wsp_whisper* w, double* encode_seconds, double* decode_seconds, int* steps)
{
    return guarded(w, [&] {
        if (encode_seconds != nullptr)
            *encode_seconds = w->whisper.lastEncodeSeconds();
        if (decode_seconds != nullptr)
            *decode_seconds = w->whisper.lastDecodeSeconds();
        if (steps != nullptr)
            *steps = w->whisper.lastStepCount();
    });
}

int wsp_whisper_encoded_rows(wsp_whisper* w, const float** rows_out, int* positions_out, int* width_out)
{
    return guarded(w, [&] {
        if (rows_out == nullptr || positions_out == nullptr || width_out == nullptr)
            throw std::invalid_argument("wsp_whisper_encoded_rows: null output");
        *rows_out = w->whisper.encodedRows();
        *positions_out = w->whisper.encodedPositions();
        *width_out = w->whisper.encoderShape().width;
    });
}

} // extern "C"
