// The greedy token loop above the decoder, in the shape of
// Whisper::decodeTranscript / encodeStep (Whisper/Whisper.cpp:1164-1224,
// 1361-1443): a prompt step, then single-token steps whose input is the slot
// the previous step's argmax wrote on the device, with stepsInFlight steps
// submitted ahead of the host's reads; the run stops at end-of-text or the
// token limit.
#pragma once

#include "Argmax.h"
#include "Decoder.h"

#include <vector>

namespace WSP
{
struct GreedyRun
{
    std::vector<int> tokens;  // sampled tokens, end-of-text excluded
    int steps = 0;            // steps whose token was read
    double decodeSeconds = 0; // first submit to the last token read
};

class GreedyDecoder
{
public:
    static constexpr int stepsInFlight = 2; // Whisper/Whisper.h:585-591

    GreedyDecoder(Decoder& decoder, const DecoderWeights& weights, const Device& device = Device::shared());
    ~GreedyDecoder();
    GreedyDecoder(const GreedyDecoder&) = delete;
    GreedyDecoder& operator=(const GreedyDecoder&) = delete;

    // firstMask / laterMask: device float [vocabularySize] suppression masks
    // (nonzero = suppressed), or null. endOfText < 0 never stops early.
    GreedyRun decode(Pass& pass, const BufferRange& encoderRows, int crossPositionCount,
                     const std::vector<int>& prompt, int maximumTokens, int endOfText,
                     const float* firstMask, const float* laterMask);

private:
    Decoder& decoder;
    const DecoderWeights& weights;
    DeviceBuffer sequenceTokens; // uint32 [maxPositions + 1]
    DeviceBuffer logitRows;      // float [maxPositions, vocabularySize]
    int* hostReports = nullptr; // pinned (token, watchdog word) pairs, one per step in flight
    std::vector<void*> events;
};
} // namespace WSP
