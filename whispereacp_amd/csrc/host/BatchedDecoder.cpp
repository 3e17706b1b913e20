// WSP::BatchedDecoder over the wsp_batch C ABI.
#include "../../../include/whispereacp/BatchedDecoder.h"
#include "host_common.h"

#include <stdexcept>
#include <string>

namespace WSP
{
BatchedDecoder::BatchedDecoder(const DecoderShape& shapeToUse, int streamCountToUse, int maxStepTokensToUse)
    : decoderShape(shapeToUse), streamCount(streamCountToUse), maxStepTokens(maxStepTokensToUse)
{
    if (streamCount <= 0 || maxStepTokens <= 0)
        throw std::invalid_argument("a batched decoder needs at least one stream and one token per step");
}

BatchedDecoder::~BatchedDecoder()
{
    wsp_batch_destroy(batch);
}

void BatchedDecoder::prepare(const DecoderWeights& weights, const Device& device, void* hipStream)
{
    requireMatchingWeights(weights);
    if (batch != nullptr)
        throw std::logic_error("a batched decoder is prepared once");
    const auto storage = weights.uniformProjectionStorage();
    if (!storage || (*storage != WeightStorage::PackedHalf && *storage != WeightStorage::PackedBFloat16))
        throw std::logic_error("batched decoding needs every projection stored as F16 or BF16");
    const wsp_decoder_shape c = decoderShape.toC();
    const int status = wsp_batch_create(&c, streamCount, maxStepTokens, wsp_dtype_of(*storage), device.index,
                                        hipStream, &batch);
    if (status != WSP_OK)
        throwForStatus(status, "wsp_batch_create failed for this shape and stream count");
    stream = hipStream;
    hidden = DeviceBuffer(device, sizeof(float) * (std::size_t) streamCount * maxStepTokens * decoderShape.width);
    layerTables.clear();
    for (const auto& layer : weights.layers)
        layerTables.push_back(layerTable(layer));
}

// The table of the weights this step is given (Decoder::step's weights
// argument, Decoder/Decoder.h:49-148): every layer's entries are taken from
// them, not from the weights the batch was prepared with. The batch packs its
// own copy again when the table's pointers change.
wsp_decoder_tensors BatchedDecoder::tablesFor(const DecoderWeights& weights)
{
    layerTables.resize(weights.layers.size());
    for (std::size_t i = 0; i < weights.layers.size(); ++i)
        layerTables[i] = layerTable(weights.layers[i]);
    return decoderTable(weights, layerTables);
}

void BatchedDecoder::requireMatchingWeights(const DecoderWeights& weights) const
{
    if (!(weights.shape == decoderShape))
        throw ModelError("these weights were loaded for another decoder shape");
}

int BatchedDecoder::position() const
{
    return batch == nullptr ? 0 : wsp_batch_position(batch);
}

int BatchedDecoder::productStorage() const
{
    return batch == nullptr ? 0 : wsp_batch_product_storage(batch);
}

int BatchedDecoder::crossPositions() const
{
    return batch == nullptr ? 0 : wsp_batch_cross_rows(batch);
}

void BatchedDecoder::beginSequences(Pass& pass, const BufferRange& encoderRows, const DecoderWeights& weights,
                                    int crossPositionCount)
{
    requireMatchingWeights(weights);
    if (batch == nullptr)
        throw std::logic_error("beginSequences before prepare");
    if (pass.hipStream() != stream)
        throw std::logic_error("a batched decoder records into the stream it was prepared with");
    if (crossPositionCount < 0 || crossPositionCount > decoderShape.crossPositions)
        throw ModelError("the encoder output has " + std::to_string(crossPositionCount)
                         + " rows, and this decoder was built for at most "
                         + std::to_string(decoderShape.crossPositions));
    const int rows = crossPositionCount == 0 ? decoderShape.crossPositions : crossPositionCount;
    const std::size_t needed = sizeof(float) * (std::size_t) streamCount * rows * decoderShape.width;
    if (encoderRows.size < needed)
        throw ModelError("the encoder rows hold fewer than streams x " + std::to_string(rows) + " rows");

    std::vector<wsp_cross_tensors> cross;
    cross.reserve(weights.layers.size());
    for (const auto& layer : weights.layers)
        cross.push_back({layer.crossKeyWeight.data(), layer.crossValueWeight.data(),
                         static_cast<const float*>(layer.crossValueBias.data())});
    const int status = wsp_batch_begin(batch, cross.data(), wsp_dtype_of(weights.layers.front().crossKeyWeight.type),
                                       static_cast<const float*>(encoderRows.data()), rows);
    if (status != WSP_OK)
        throwForStatus(status, wsp_batch_last_error(batch));
}

void BatchedDecoder::record(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                            const BufferRange& logits, const float* mask, const BufferRange* argmaxSlots)
{
    requireMatchingWeights(weights);
    if (batch == nullptr)
        throw std::logic_error("step before prepare");
    if (pass.hipStream() != stream)
        throw std::logic_error("a batched decoder records into the stream it was prepared with");
    if (tokenCount <= 0 || tokenCount > maxStepTokens)
        throw std::invalid_argument("a batched step takes 1.." + std::to_string(maxStepTokens) + " tokens per stream");
    if (position() + tokenCount > decoderShape.maxPositions)
        throw ModelError("decoding " + std::to_string(tokenCount) + " more tokens would pass the "
                         + std::to_string(decoderShape.maxPositions) + "-position context");
    if (crossPositions() <= 0)
        throw std::logic_error("step before beginSequences");
    const std::size_t rows = (std::size_t) streamCount * tokenCount;
    if (tokens.size < rows * sizeof(uint32_t) || logits.size < rows * decoderShape.vocabularySize * sizeof(float))
        throw ModelError("the token or logits range is smaller than streams x tokens rows");
    if (argmaxSlots != nullptr && argmaxSlots->size < (std::size_t) streamCount * sizeof(uint32_t))
        throw ModelError("the argmax range holds fewer slots than streams");

    const wsp_decoder_tensors tensors = tablesFor(weights);
    const int status = wsp_batch_step(batch, &tensors, static_cast<const uint32_t*>(tokens.data()), tokenCount,
                                      static_cast<float*>(hidden.data()), static_cast<float*>(logits.data()), mask,
                                      argmaxSlots != nullptr ? static_cast<uint32_t*>(argmaxSlots->data()) : nullptr);
    if (status != WSP_OK)
        throwForStatus(status, wsp_batch_last_error(batch));
}

void BatchedDecoder::ringStep(Pass& pass, const BufferRange& ring, const DecoderWeights& weights,
                              const BufferRange& logits, const float* mask)
{
    requireMatchingWeights(weights);
    if (batch == nullptr)
        throw std::logic_error("step before prepare");
    if (pass.hipStream() != stream)
        throw std::logic_error("a batched decoder records into the stream it was prepared with");
    if (crossPositions() <= 0)
        throw std::logic_error("step before beginSequences");
    if (position() < 1)
        throw std::logic_error("a ring step follows the prompt step");
    if (position() + 1 > decoderShape.maxPositions)
        throw ModelError("decoding one more token would pass the " + std::to_string(decoderShape.maxPositions)
                         + "-position context");
    const std::size_t slots = (std::size_t) (decoderShape.maxPositions + 1) * streamCount;
    if (ring.size < slots * sizeof(uint32_t))
        throw ModelError("the token ring holds fewer than (maxPositions + 1) x streams slots");
    if (logits.size < (std::size_t) streamCount * decoderShape.vocabularySize * sizeof(float))
        throw ModelError("the logits range is smaller than streams rows");
    const wsp_decoder_tensors tensors = tablesFor(weights);
    const int status = wsp_batch_ring_step(batch, &tensors, static_cast<uint32_t*>(ring.data()),
                                           static_cast<float*>(logits.data()), mask);
    if (status != WSP_OK)
        throwForStatus(status, wsp_batch_last_error(batch));
}

void BatchedDecoder::step(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                          const BufferRange& logits)
{
    record(pass, tokens, tokenCount, weights, logits, nullptr, nullptr);
}

void BatchedDecoder::stepAndSample(Pass& pass, const BufferRange& tokens, int tokenCount,
                                   const DecoderWeights& weights, const BufferRange& logits, const float* mask,
                                   const BufferRange& argmaxSlots)
{
    record(pass, tokens, tokenCount, weights, logits, mask, &argmaxSlots);
}
} // namespace WSP
