// Independent streams decoded together: the Decoder surface
// (Decoder/Decoder.h:49-127) over `streams` sequences that share one weight
// read per step. No reference counterpart — the reference runs one Decoder
// per sequence; every stream's rows equal what Decoder::step computes for it
// alone. Built on the wsp_batch C ABI (include/wsp_hip.h); needs a file whose
// projections and tied logits share one 16-bit storage (F16 or BF16, with
// WeightPacking::ExactHalf for the logits' packed copy).
#pragma once

#include "DecoderWeights.h"
#include "ModelError.h"

#include <vector>

namespace WSP
{
class BatchedDecoder
{
public:
    BatchedDecoder(const DecoderShape& shapeToUse, int streamCount, int maxStepTokens = 4);
    ~BatchedDecoder();
    BatchedDecoder(const BatchedDecoder&) = delete;
    BatchedDecoder& operator=(const BatchedDecoder&) = delete;

    // Every stream's caches and the step buffers, once (Decoder/Decoder.cpp:194-227).
    void prepare(const DecoderWeights& weights, const Device& device, void* hipStream = nullptr);

    // Decoder::beginSequence for every stream: encoderRows holds
    // [streams][crossPositionCount][width] f32 (zero: the shape's capacity).
    void beginSequences(Pass& pass, const BufferRange& encoderRows, const DecoderWeights& weights,
                        int crossPositionCount = 0);

    // Decoder::step for every stream: tokens [streams][tokenCount] uint32
    // (stream-major), logits [streams·tokenCount][vocabularySize]. A step
    // past maxPositions is a ModelError thrown before anything is recorded.
    void step(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
              const BufferRange& logits);

    // A step followed by each stream's masked argmax of its last row, written
    // to argmaxSlots [streams] (the next step's tokens).
    void stepAndSample(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                       const BufferRange& logits, const float* mask, const BufferRange& argmaxSlots);

    // One single-token step per stream driven by a token ring [maxPositions +
    // 1][streams] (position-major): each stream's token at the current
    // position p is read from ring[p] and its masked greedy successor written
    // to ring[p + 1], logits [streams][vocabularySize] too. Replayed from a
    // captured HIP graph (wsp_batch_ring_step); needs p >= 1.
    void ringStep(Pass& pass, const BufferRange& ring, const DecoderWeights& weights, const BufferRange& logits,
                  const float* mask);

    const DecoderShape& shape() const { return decoderShape; }
    int streams() const { return streamCount; }
    int position() const;
    // The storage the step's products read the weights in (wsp_batch_product_storage).
    int productStorage() const;
    int crossPositions() const;
    void* hipStream() const { return stream; }

    // The last step's rows after the final layer norm, [streams·tokenCount, width].
    const DeviceBuffer& hiddenStates() const { return hidden; }

private:
    void record(Pass& pass, const BufferRange& tokens, int tokenCount, const DecoderWeights& weights,
                const BufferRange& logits, const float* mask, const BufferRange* argmaxSlots);
    void requireMatchingWeights(const DecoderWeights& weights) const;
    wsp_decoder_tensors tablesFor(const DecoderWeights& weights);

    DecoderShape decoderShape;
    int streamCount = 0;
    int maxStepTokens = 0;
    wsp_batch* batch = nullptr;
    void* stream = nullptr;
    DeviceBuffer hidden;
    std::vector<wsp_layer_tensors> layerTables;
};
} // namespace WSP
