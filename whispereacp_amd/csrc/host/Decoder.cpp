// The Decoder class around the decoder body (Decoder/Decoder.cpp:113-308):
// caches and scratch sized once, the recorded steps on HipNet
// (DecoderRecording.cpp), and the fused single-token path.
#include "../../../include/whispereacp/Decoder.h"
#include "host_common.h"

#include <functional>
#include <string>
#include <utility>

namespace WSP
{
namespace
{
void addCaches(std::vector<Cache>& caches, Net& net, int layers, int rows, int width)
{
    caches.clear();
    for (int i = 0; i < layers; ++i)
        caches.push_back(net.makeCache(rows, width));
}
} // namespace

Decoder::Decoder(const DecoderShape& shapeToUse) : decoderShape(shapeToUse) {}

void Decoder::prepare(const Device& device, void* hipStream)
{
    HipNetLayout layout;
    layout.shape = decoderShape;
    layout.scratch = {{decoderShape.stepElementCount(), 4}, {decoderShape.stepFeedForwardElementCount(), 1}};
    hipNet.prepare(device, layout, hipStream);

    const int layers = decoderShape.layers, width = decoderShape.width;
    addCaches(caches.selfKeys, hipNet, layers, decoderShape.maxPositions, width);
    addCaches(caches.selfValues, hipNet, layers, decoderShape.maxPositions, width);
    addCaches(caches.crossKeys, hipNet, layers, decoderShape.crossPositions, width);
    addCaches(caches.crossValues, hipNet, layers, decoderShape.crossPositions, width);

    normalisedRows.emplace(device, (std::size_t) decoderShape.stepElementCount() * sizeof(float));
    decodedPositions = 0;
    activeCrossPositions = decoderShape.crossPositions;
}

void Decoder::prepare()
{
    prepare(Device::shared());
}

void Decoder::requireMatchingWeights(const DecoderWeights& weights) const
{
    if (!(weights.shape == decoderShape))
        throw ModelError("the weights were loaded against a different decoder shape than this decoder was built for");
    if (!normalisedRows)
        throw std::logic_error("a decoder records once it is prepared");
}

void Decoder::requireRoomFor(int tokenCount) const
{
    if (tokenCount <= 0)
        throw ModelError("a decoder step needs at least one token");
    if (decodedPositions + tokenCount > decoderShape.maxPositions)
        throw ModelError("this step would carry the sequence to " + std::to_string(decodedPositions + tokenCount)
                         + " tokens, past the " + std::to_string(decoderShape.maxPositions)
                         + " this decoder was built for");
}

void Decoder::beginSequence(Pass& pass, const DeviceBuffer& encoderOutput, const DecoderWeights& weights,
                            int crossPositionCount)
{
    beginSequence(pass, BufferRange::of(encoderOutput), weights, crossPositionCount);
}

void Decoder::beginSequence(Pass& pass, const BufferRange& encoderOutput, const DecoderWeights& weights,
                            int crossPositionCount)
{
    requireMatchingWeights(weights);
    if (crossPositionCount < 0 || crossPositionCount > decoderShape.crossPositions)
        throw ModelError("a decoder built for " + std::to_string(decoderShape.crossPositions)
                         + " encoder rows was asked to attend to " + std::to_string(crossPositionCount));
    const int rows = crossPositionCount == 0 ? decoderShape.crossPositions : crossPositionCount;
    const Binding encoderRows {encoderOutput, Shape {decoderShape.crossPositions, decoderShape.width}, "encoder_rows"};

    hipNet.begin(pass);
    recordSequenceStart(hipNet, decoderShape, weights, caches, encoderRows, rows);
    hipNet.end();

    decodedPositions = 0;
    activeCrossPositions = rows;
}

bool Decoder::usesFusedStep(const DecoderWeights& weights, int tokenCount) const
{
    const int headWidth = decoderShape.headWidth();
    return fusedSteps && tokenCount >= 1 && tokenCount <= fusedPromptTokens
           && weights.uniformProjectionStorage().has_value() && headWidth % 4 == 0 && headWidth <= 64;
}

void Decoder::step(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                   const BufferRange& logits)
{
    requireMatchingWeights(weights);
    requireRoomFor(tokenCount);

    if (usesFusedStep(weights, tokenCount))
    {
        // Token i at position + i sees the keys of every token before it, as
        // the causal recorded step would (Kernels/Attention.h:34-47).
        fusedStep(pass, tokens, tokenCount, weights, logits, nullptr, nullptr);
        return;
    }

    const Binding tokenSlots {tokens, Shape {decoderShape.maxPositions}, "tokens"};
    hipNet.begin(pass);
    recordDecoderStep(hipNet, decoderShape, weights, caches, tokenSlots, tokenCount, decodedPositions,
                      Binding {BufferRange::of(*normalisedRows), {}, "hidden_states"},
                      Binding {logits, {}, "logits"});
    hipNet.end();
    decodedPositions += tokenCount;
}

void Decoder::stepAndSample(Pass& pass, const BufferRange& tokens, const DecoderWeights& weights,
                            const BufferRange& logits, const float* mask, const BufferRange& argmaxSlot)
{
    requireMatchingWeights(weights);
    requireRoomFor(1);
    if (usesFusedStep(weights, 1))
    {
        fusedStep(pass, tokens, 1, weights, logits, mask, &argmaxSlot);
        return;
    }
    step(pass, tokens, 1, weights, logits);
    const int status = wsp_hip_argmax(hipNet.context(), static_cast<const float*>(logits.data()), 1,
                                      decoderShape.vocabularySize, mask, static_cast<uint32_t*>(argmaxSlot.data()));
    if (status != WSP_OK)
        throwForStatus(status, wsp_hip_last_error(hipNet.context()));
}

void Decoder::fusedStep(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                        const BufferRange& logits, const float* mask, const BufferRange* argmaxSlot)
{
    if (pass.hipStream() != wsp_hip_stream(hipNet.context()))
        throw std::logic_error("a decoder records into the stream it was prepared with");

    fusedLayers.resize((std::size_t) decoderShape.layers);
    for (int l = 0; l < decoderShape.layers; ++l)
    {
        const auto i = (std::size_t) l;
        wsp_layer_tensors& L = fusedLayers[i];
        L = layerTable(weights.layers[i]);
        L.self_keys = hipNet.cacheData(caches.selfKeys[i]);
        L.self_values = hipNet.cacheData(caches.selfValues[i]);
        L.cross_keys = hipNet.cacheData(caches.crossKeys[i]);
        L.cross_values = hipNet.cacheData(caches.crossValues[i]);
    }
    const wsp_decoder_tensors tensors = decoderTable(weights, fusedLayers);

    const int status = wsp_hip_decoder_step_tokens(
        hipNet.context(), &tensors, static_cast<const uint32_t*>(tokens.data()), tokenCount, decodedPositions,
        activeCrossPositions, static_cast<float*>(normalisedRows->data()), static_cast<float*>(logits.data()), mask,
        argmaxSlot != nullptr ? static_cast<uint32_t*>(argmaxSlot->data()) : nullptr);
    if (status != WSP_OK)
        throwForStatus(status, wsp_hip_last_error(hipNet.context()));

    // The self caches now hold the new rows; their Cache records follow.
    for (int l = 0; l < decoderShape.layers; ++l)
    {
        caches.selfKeys[(std::size_t) l].rows = decodedPositions + tokenCount;
        caches.selfValues[(std::size_t) l].rows = decodedPositions + tokenCount;
    }
    decodedPositions += tokenCount;
}
} // namespace WSP
