// Decoder/Decoder.h:1-148 — HuggingFace's WhisperDecoder.forward with a KV
// cache, on gfx950:
//
//   h = embed_tokens[token] + embed_positions[position + t]
//   per layer: h += self_attn.out_proj(attention(self_attn_layer_norm(h)))
//              h += encoder_attn.out_proj(attention(encoder_attn_layer_norm(h), encoder rows))
//              h += fc2(gelu(fc1(final_layer_norm(h))))
//   h = layer_norm(h);  logits = h · embed_tokensᵀ
//
// The body is recordSequenceStart / recordDecoderStep written once against
// Net, run by HipNet. A single-token step may instead take the fused path
// (wsp_hip_decoder_step), which computes the same step in one launch; both
// write the same caches, hidden rows and logits, so steps may alternate.
#pragma once

#include "DecoderWeights.h"
#include "HipNet.h"
#include "ModelError.h"

#include <optional>

namespace WSP
{
struct DecoderCaches
{
    std::vector<Cache> selfKeys;
    std::vector<Cache> selfValues;
    std::vector<Cache> crossKeys;
    std::vector<Cache> crossValues;
};

class Decoder
{
public:
    explicit Decoder(const DecoderShape& shapeToUse);

    // Sizes every intermediate and cache once (Decoder/Decoder.cpp:194-227).
    // hipStream is the stream every pass given to this decoder wraps.
    void prepare(const Device& device, void* hipStream = nullptr);
    void prepare();

    const DecoderShape& shape() const { return decoderShape; }

    // Projects the cross keys and values of the first crossPositionCount
    // encoder rows (zero: all of them) and resets the position
    // (Decoder/Decoder.cpp:241-268). ModelError past the capacity.
    void beginSequence(Pass& pass, const DeviceBuffer& encoderOutput, const DecoderWeights& weights,
                       int crossPositionCount = 0);
    void beginSequence(Pass& pass, const BufferRange& encoderOutput, const DecoderWeights& weights,
                       int crossPositionCount = 0);

    // Appends tokenCount tokens read from `tokens` (uint32 ids on the device)
    // and writes their logits [tokenCount, vocabularySize]. A step past
    // maxPositions is a ModelError thrown before anything is recorded
    // (Decoder/Decoder.cpp:270-308). When argmaxSlot is valid and the step
    // takes the fused path, the greedy token of the last row (under mask, which
    // may be null) is written there as part of the same launch.
    void step(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
              const BufferRange& logits);

    // The fused path: on by default when the weights allow it. A step of up
    // to fusedPromptTokens tokens runs as persistent launches of up to four
    // tokens each (wsp_hip_decoder_step_tokens), whose rows share every
    // weight read; longer steps run the recorded sequence.
    static constexpr int fusedPromptTokens = 16;
    void setFusedSteps(bool enabled) { fusedSteps = enabled; }
    bool usesFusedStep(const DecoderWeights& weights, int tokenCount) const;

    // One single-token step and its masked argmax in one fused launch; the
    // token lands in argmaxSlot (a uint32 on the device).
    void stepAndSample(Pass& pass, const BufferRange& tokens, const DecoderWeights& weights,
                       const BufferRange& logits, const float* mask, const BufferRange& argmaxSlot);

    int position() const { return decodedPositions; }
    int crossPositions() const { return activeCrossPositions; }

    // The last step's rows after the final layer norm, [tokenCount, width].
    const DeviceBuffer& hiddenStates() const { return *normalisedRows; }

    HipNet& net() { return hipNet; }

private:
    void requireMatchingWeights(const DecoderWeights& weights) const;
    void requireRoomFor(int tokenCount) const;
    // tokenCount fused tokens: their logits and hidden rows out, the argmax of
    // the last row into argmaxSlot when given.
    void fusedStep(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                   const BufferRange& logits, const float* mask, const BufferRange* argmaxSlot);

    DecoderShape decoderShape;
    int decodedPositions = 0;
    int activeCrossPositions = 0;
    bool fusedSteps = true;

    HipNet hipNet;
    DecoderCaches caches;
    std::optional<DeviceBuffer> normalisedRows;
    std::vector<wsp_layer_tensors> fusedLayers;
};

// Empties every cache and projects the cross keys and values out of the first
// `rows` encoder rows (Decoder/Decoder.cpp:121-146).
void recordSequenceStart(Net& net, const DecoderShape& shape, const DecoderWeights& weights,
                         DecoderCaches& caches, const Binding& encoderRows, int rows);

// Appends tokenCount tokens to the self caches and writes their final hidden
// rows and logits (Decoder/Decoder.cpp:151-177).
void recordDecoderStep(Net& net, const DecoderShape& shape, const DecoderWeights& weights,
                       DecoderCaches& caches, const Binding& tokens, int tokenCount, int firstPosition,
                       const Binding& hiddenStates, const Binding& logits);
} // namespace WSP
