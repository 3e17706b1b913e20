// Decoder/DecoderWeights.h:25-161 — every decoder tensor of a Whisper file,
// uploaded and checked against the shape it is supposed to have.
//
// The source is any TensorSource (a name -> host tensor lookup), so the same
// loader serves synthetic weights and a safetensors file. A missing name, a
// wrong rank or a dimension that disagrees with the shape is a ModelError
// naming the tensor (Decoder/DecoderWeights.cpp:17-74).
//
// Storage follows the reference's policy: projection weights stay packed
// (F16 or BF16) when the file holds them packed, every other tensor is widened
// to float, and the token embedding is always float for the gather. Under
// WeightPacking::ExactHalf every F32 projection that survives narrowing to
// fp16 bit-exactly is packed, and the logits read a packed copy of
// embed_tokens when one exists (Decoder/DecoderWeights.h:104-123).
//
// Layout: each attention's q, k and v weights share one [3·width, width]
// allocation (q rows, then k, then v) and the self-attention biases one
// [3·width] buffer [q | 0 | v], so the fused step can stream the three as one
// matrix; the per-projection TensorBuffers view into them.
#pragma once

#include "DecoderShape.h"
#include "Net.h"

#include <map>
#include <optional>
#include <string>
#include <vector>

namespace WSP
{
enum class WeightPacking
{
    Float,
    ExactHalf
};

// A tensor as a file holds it: "F32", "F16" or "BF16" little-endian, row-major.
struct HostTensor
{
    std::string dtype;
    std::vector<long long> extents;
    const void* data = nullptr;
};

class TensorSource
{
public:
    virtual ~TensorSource() = default;
    virtual const HostTensor* find(const std::string& name) const = 0;
};

class MapTensorSource final : public TensorSource
{
public:
    void add(const std::string& name, HostTensor tensor) { tensors[name] = std::move(tensor); }
    const HostTensor* find(const std::string& name) const override;

private:
    std::map<std::string, HostTensor> tensors;
};

struct DecoderLayerWeights
{
    TensorBuffer selfAttentionNormWeight;
    TensorBuffer selfAttentionNormBias;
    TensorBuffer selfQueryWeight;
    TensorBuffer selfQueryBias;
    TensorBuffer selfKeyWeight;
    TensorBuffer selfValueWeight;
    TensorBuffer selfValueBias;
    TensorBuffer selfAttentionOutputWeight;
    TensorBuffer selfAttentionOutputBias;

    TensorBuffer crossAttentionNormWeight;
    TensorBuffer crossAttentionNormBias;
    TensorBuffer crossQueryWeight;
    TensorBuffer crossQueryBias;
    TensorBuffer crossKeyWeight;
    TensorBuffer crossValueWeight;
    TensorBuffer crossValueBias;
    TensorBuffer crossAttentionOutputWeight;
    TensorBuffer crossAttentionOutputBias;

    TensorBuffer finalNormWeight;
    TensorBuffer finalNormBias;
    TensorBuffer feedForwardWeight;
    TensorBuffer feedForwardBias;
    TensorBuffer feedForwardOutputWeight;
    TensorBuffer feedForwardOutputBias;

    // The [q | 0 | v] bias block the self q/v biases view into.
    TensorBuffer selfQkvBias;
};

struct DecoderWeights
{
    DecoderWeights(const TensorSource& file, const DecoderShape& shapeToUse,
                   WeightPacking packing = WeightPacking::Float,
                   const Device& device = Device::shared());

    DecoderShape shape;

    TensorBuffer tokenEmbedding;                      // always float: the gather's table
    std::optional<TensorBuffer> packedTokenEmbedding; // the logits' packed copy
    const TensorBuffer& logitsWeight() const
    {
        return packedTokenEmbedding ? *packedTokenEmbedding : tokenEmbedding;
    }

    TensorBuffer positionalEmbedding;
    TensorBuffer finalNormWeight;
    TensorBuffer finalNormBias;

    std::vector<DecoderLayerWeights> layers;

    // The one storage every projection weight shares, when they share one —
    // what the fused step needs. Empty for a mixed file.
    std::optional<WeightStorage> uniformProjectionStorage() const;
};

// The device pointers of one layer's weights in the C ABI's layout, cache
// pointers left null, and the whole decoder's table over `layers` (which must
// outlive it). Needs a uniform projection storage.
wsp_layer_tensors layerTable(const DecoderLayerWeights& w);
wsp_decoder_tensors decoderTable(const DecoderWeights& weights, const std::vector<wsp_layer_tensors>& layers);
} // namespace WSP
