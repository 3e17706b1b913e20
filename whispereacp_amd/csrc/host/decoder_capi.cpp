// The C binding of the C++ decoder surface (include/wsp_decoder.h): every
// exception the reference would throw is caught here and returned as a status
// plus its kind and message.
#include "../../../include/wsp_decoder.h"
#include "../../../include/whispereacp/Argmax.h"
#include "../../../include/whispereacp/Decoder.h"
#include "../../../include/whispereacp/GreedyDecoder.h"

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

namespace
{
template <typename Body>
int guarded(wsp_decoder* d, Body body)
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
        d->shape = {shape->width,           shape->heads,         shape->layers,       shape->feed_forward_width,
                    shape->vocabulary_size, shape->max_positions, shape->cross_positions};
        if (d->shape.width <= 0 || d->shape.heads <= 0 || d->shape.width % d->shape.heads != 0 || d->shape.layers <= 0
            || d->shape.feedForwardWidth <= 0 || d->shape.vocabularySize <= 0 || d->shape.maxPositions <= 0
            || d->shape.crossPositions <= 0)
            throw WSP::ModelError("a decoder shape needs positive extents and a width divisible by its heads");
        d->device = WSP::Device {device};
        d->stream = stream;
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
        d->weights = std::make_unique<WSP::DecoderWeights>(
            source, d->shape, packing == 1 ? WSP::WeightPacking::ExactHalf : WSP::WeightPacking::Float, d->device);
        d->decoder = std::make_unique<WSP::Decoder>(d->shape);
        d->decoder->prepare(d->device, stream);
        d->selection = std::make_unique<WSP::Argmax>();
        d->selection->prepare(d->device, d->shape.maxPositions, d->shape.vocabularySize, stream);
    });
    if (status != WSP_OK)
    {
        // Keep the object so the caller can read why; it is unusable otherwise.
        d->decoder.reset();
        d->weights.reset();
        *out = d;
        return status;
    }
    *out = d;
    return WSP_OK;
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
            d->greedy = std::make_unique<WSP::GreedyDecoder>(*d->decoder, *d->weights, d->device);
        WSP::Pass pass(d->stream);
        const std::vector<int> promptTokens(prompt, prompt + prompt_count);
        const WSP::GreedyRun run = d->greedy->decode(
            pass, range(encoder_rows, (std::size_t) d->shape.crossElementCount() * 4), cross_position_count,
            promptTokens, maximum_tokens, end_of_text, first_mask, later_mask);
        const int n = std::min<int>((int) run.tokens.size(), capacity);
        for (int i = 0; i < n; ++i)
            tokens_out[i] = run.tokens[(std::size_t) i];
        *count_out = n;
        if (decode_seconds != nullptr)
            *decode_seconds = run.decodeSeconds;
    });
}

} // extern "C"
