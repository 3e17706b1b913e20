// Decoder/DecoderShape.h:20-83 — every extent one decoder is built against.
#pragma once

#include "../wsp_hip.h"

namespace WSP
{
struct DecoderShape
{
    int width = 0;
    int heads = 0;
    int layers = 0;
    int feedForwardWidth = 0;
    int vocabularySize = 0;
    int maxPositions = 0;
    int crossPositions = 0;

    friend bool operator==(const DecoderShape&, const DecoderShape&) = default;

    int headWidth() const { return width / heads; }
    int rowElementCount() const { return width; }
    int feedForwardElementCount() const { return feedForwardWidth; }
    int logitElementCount() const { return vocabularySize; }
    int stepElementCount() const { return maxPositions * width; }
    int stepFeedForwardElementCount() const { return maxPositions * feedForwardWidth; }
    int cacheElementCount() const { return maxPositions * width; }
    int crossElementCount() const { return crossPositions * width; }

    // D^-0.5 in float, applied to the scores (Decoder/DecoderShape.cpp:23-26).
    float attentionScale() const;

    wsp_decoder_shape toC() const
    {
        return {width, heads, layers, feedForwardWidth, vocabularySize, maxPositions, crossPositions};
    }
};
} // namespace WSP
