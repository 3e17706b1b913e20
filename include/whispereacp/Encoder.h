// The encoder's C++ surface (Encoder/EncoderShape.h:25-67,
// Encoder/EncoderWeights.h:19-93, Encoder/Encoder.h:8-71) over the gfx950
// encoder of include/wsp_hip.h: a shape read from config.json, the weights of
// a Whisper file checked and uploaded, and an Encoder that owns the
// intermediates of one window.
//
// Storage follows the reference's loader: every projection weight stays as
// the file holds it (F16 or BF16) or is packed to fp16 where narrowing is
// exact under WeightPacking::ExactHalf; everything else is widened to float.
// BF16 projections are held as exact fp16 multiples w·2^k with their scales
// (wsp_encoder_scaled_halves) when every one of them narrows exactly and the
// shape's products run over pre-split inputs.
// The gfx950 encoder reads one projection storage for the whole model, so a
// file whose projections would end up in different storages is uploaded with
// every projection widened to float.
#pragma once

#include "DecoderWeights.h"
#include "Gpu.h"

#include "../wsp_hip.h"

#include <string>
#include <vector>

namespace WSP
{
struct EncoderShape
{
    static constexpr int convolutionKernelSize = 3;
    static constexpr int secondConvolutionStride = 2;

    int melBins = 0;
    int width = 0;
    int heads = 0;
    int layers = 0;
    int feedForwardWidth = 0;
    int inputFrames = 0;

    int headWidth() const { return width / heads; }
    // Frames after the stride-1 convolution, and positions after the stride-2
    // one (kernel 3, padding 1: (n + 2 - 3) / stride + 1).
    int convolutionFrames() const { return inputFrames; }
    int positions() const { return (inputFrames - 1) / secondConvolutionStride + 1; }

    wsp_encoder_shape cShape() const { return {melBins, width, heads, layers, feedForwardWidth, inputFrames}; }
};

// config.json's encoder extents: num_mel_bins, d_model,
// encoder_attention_heads, encoder_layers, encoder_ffn_dim, and the input
// frames 2 * max_source_positions (Model/ModelConfig.h:50-53).
EncoderShape encoderShapeFromConfig(const std::string& json);

struct EncoderWeights
{
    EncoderWeights(const TensorSource& file, const EncoderShape& shapeToUse,
                   WeightPacking packing = WeightPacking::Float, const Device& device = Device::shared());

    EncoderShape shape;
    int projectionType = WSP_F32; // the storage every projection weight shares

    // The device pointers in the C ABI's layout; `layerTable` holds the
    // per-layer entries the returned table points at.
    wsp_encoder_tensors table() const;

private:
    std::vector<DeviceBuffer> buffers;
    std::vector<wsp_encoder_layer_tensors> layerTable;
    wsp_encoder_tensors model {};
};

class Encoder
{
public:
    Encoder(const EncoderShape& shape, const Device& device, void* hipStream);
    ~Encoder();
    Encoder(const Encoder&) = delete;
    Encoder& operator=(const Encoder&) = delete;

    const EncoderShape& shape() const { return encoderShape; }

    // mel: device [melBins, inputFrames]; output: device, positionCount rows
    // of width floats (0 = the whole window). A count past the window is a
    // ModelError (Encoder/Encoder.cpp:159-163).
    void encode(const EncoderWeights& weights, const float* mel, float* output, int positionCount = 0);

private:
    EncoderShape encoderShape;
    wsp_encoder* handle = nullptr;
};
} // namespace WSP
