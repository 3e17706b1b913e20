// The decoder body written once against Net (Decoder/Decoder.cpp:73-177):
// recordSequenceStart projects the cross keys and values, recordDecoderStep
// embeds, runs the pre-norm layers and writes the final rows and the tied
// logits. HipNet runs it on gfx950; any other Net (a host one in the tests)
// runs the same recording.
//
// WSP_MUTATION (0 in every product build) selects one deliberate mistake for
// the host-side mutation check (tests/test_decoder_on_host.py), which builds
// this file alone with each value on the CPU:
//   1  cross-attention before self-attention
//   2  self keys and values projected from the unnormalised rows
//   3  every step embedded at position zero
//   4  the causal flag dropped
//   5  fc2 without its residual
//   6  the final LayerNorm skipped before the logits
//   7  the cross values' bias dropped
#include "../../../include/whispereacp/Decoder.h"

#include <functional>
#include <utility>

#ifndef WSP_MUTATION
#define WSP_MUTATION 0
#endif

namespace WSP
{
namespace
{
// One pre-norm attention sublayer: normalise, project the queries (and, for
// self-attention, append this step's keys and values from the same
// normalised rows), attend, and add the output projection into the stream.
Tensor attentionSublayer(Net& net, const DecoderShape& shape, const TensorBuffer& normWeight,
                         const TensorBuffer& normBias, const TensorBuffer& queryWeight,
                         const TensorBuffer& queryBias, const TensorBuffer& outputWeight,
                         const TensorBuffer& outputBias, const Tensor& stream, bool causal,
                         const std::function<std::pair<Tensor, Tensor>(const Tensor&)>& keysAndValues)
{
    const Tensor normalised = net.layerNorm(stream, normWeight, normBias);
    const Tensor queries = net.linear(normalised, queryWeight, &queryBias, Activation::none);
    const auto [keys, values] = keysAndValues(normalised);
    const Tensor attended = net.attention(queries, keys, values, shape.heads, causal);
    return net.linearAdd(attended, outputWeight, &outputBias, stream);
}

Tensor selfAttention(Net& net, const DecoderShape& shape, const DecoderLayerWeights& w, DecoderCaches& caches,
                     int layer, const Tensor& stream)
{
    // Keys and values come from this step's normalised rows, appended to the
    // cache; the causal mask keeps each row out of its future.
    return attentionSublayer(
        net, shape, w.selfAttentionNormWeight, w.selfAttentionNormBias, w.selfQueryWeight, w.selfQueryBias,
        w.selfAttentionOutputWeight, w.selfAttentionOutputBias, stream, WSP_MUTATION != 4,
        [&](const Tensor& normalised) {
            const Tensor& source = WSP_MUTATION == 2 ? stream : normalised;
            Tensor keys = net.appendLinear(caches.selfKeys[(std::size_t) layer], source, w.selfKeyWeight, nullptr);
            Tensor values = net.appendLinear(caches.selfValues[(std::size_t) layer], source, w.selfValueWeight,
                                             &w.selfValueBias);
            return std::make_pair(keys, values);
        });
}

Tensor crossAttention(Net& net, const DecoderShape& shape, const DecoderLayerWeights& w, DecoderCaches& caches,
                      int layer, const Tensor& stream)
{
    // The keys and values were projected when the sequence opened; nothing
    // is masked.
    return attentionSublayer(
        net, shape, w.crossAttentionNormWeight, w.crossAttentionNormBias, w.crossQueryWeight, w.crossQueryBias,
        w.crossAttentionOutputWeight, w.crossAttentionOutputBias, stream, false, [&](const Tensor&) {
            return std::make_pair(net.cached(caches.crossKeys[(std::size_t) layer]),
                                  net.cached(caches.crossValues[(std::size_t) layer]));
        });
}

Tensor layerBody(Net& net, const DecoderShape& shape, const DecoderLayerWeights& w, DecoderCaches& caches,
                 int layer, const Tensor& hidden)
{
    const Tensor afterCross = WSP_MUTATION == 1
                                  ? selfAttention(net, shape, w, caches, layer,
                                                  crossAttention(net, shape, w, caches, layer, hidden))
                                  : crossAttention(net, shape, w, caches, layer,
                                                   selfAttention(net, shape, w, caches, layer, hidden));
    const Tensor inner = net.linear(net.layerNorm(afterCross, w.finalNormWeight, w.finalNormBias),
                                    w.feedForwardWeight, &w.feedForwardBias, Activation::gelu);
    if (WSP_MUTATION == 5)
        return net.linear(inner, w.feedForwardOutputWeight, &w.feedForwardOutputBias, Activation::none);
    return net.linearAdd(inner, w.feedForwardOutputWeight, &w.feedForwardOutputBias, afterCross);
}
} // namespace

void recordSequenceStart(Net& net, const DecoderShape& shape, const DecoderWeights& weights, DecoderCaches& caches,
                         const Binding& encoderRows, int rows)
{
    const Tensor encoded = net.input(encoderRows, {rows, shape.width}, DType::float32);
    for (int layer = 0; layer < shape.layers; ++layer)
    {
        const auto& w = weights.layers[(std::size_t) layer];
        const auto i = (std::size_t) layer;
        caches.selfKeys[i].clear();
        caches.selfValues[i].clear();
        caches.crossKeys[i].clear();
        caches.crossValues[i].clear();
        net.appendLinear(caches.crossKeys[i], encoded, w.crossKeyWeight, nullptr);
        net.appendLinear(caches.crossValues[i], encoded, w.crossValueWeight,
                         WSP_MUTATION == 7 ? nullptr : &w.crossValueBias);
    }
}

void recordDecoderStep(Net& net, const DecoderShape& shape, const DecoderWeights& weights, DecoderCaches& caches,
                       const Binding& tokens, int tokenCount, int firstPosition, const Binding& hiddenStates,
                       const Binding& logits)
{
    Tensor hidden = net.embed(net.input(tokens, {tokenCount}, DType::int32), weights.tokenEmbedding,
                              weights.positionalEmbedding, WSP_MUTATION == 3 ? 0 : firstPosition);
    for (int layer = 0; layer < shape.layers; ++layer)
        hidden = layerBody(net, shape, weights.layers[(std::size_t) layer], caches, layer, hidden);

    const Tensor normalised =
        WSP_MUTATION == 6 ? hidden : net.layerNorm(hidden, weights.finalNormWeight, weights.finalNormBias);
    net.output(normalised, hiddenStates);
    // Tied logits: embed_tokens itself, no bias (Decoder/DecoderWeights.h:66-79).
    net.output(net.linear(normalised, weights.logitsWeight(), nullptr, Activation::none), logits);
}

} // namespace WSP
