// DecoderWeights: the decoder tensors of a Whisper file, checked and uploaded
// (Decoder/DecoderWeights.cpp:1-178, Model/TensorLoader.cpp:54-88,
// Model/SafeTensors.cpp:554-592 for the exact-half packing rule).
#include "../../../include/whispereacp/DecoderWeights.h"
#include "../../../include/whispereacp/ModelError.h"
#include "host_common.h"

#include <cstring>
#include <stdexcept>
#include <sstream>

namespace WSP
{
namespace
{
const std::string decoderPrefix = "model.decoder.";

std::string layerName(int index, const std::string& suffix)
{
    return decoderPrefix + "layers." + std::to_string(index) + "." + suffix;
}

std::string describe(const std::vector<long long>& extents)
{
    std::ostringstream s;
    s << "[";
    for (std::size_t i = 0; i < extents.size(); ++i)
        s << (i ? ", " : "") << extents[i];
    s << "]";
    return s.str();
}

std::size_t countOf(const std::vector<long long>& extents)
{
    std::size_t n = 1;
    for (long long e : extents)
        n *= (std::size_t) e;
    return n;
}

// What the file holds, checked before anything is uploaded.
struct Loader
{
    const TensorSource& file;
    const Device& device;

    const HostTensor& require(const std::string& name) const
    {
        const HostTensor* t = file.find(name);
        if (t == nullptr)
            throw ModelError("tensor '" + name + "' is missing from the decoder file");
        if (t->dtype != "F32" && t->dtype != "F16" && t->dtype != "BF16")
            throw ModelError("tensor '" + name + "' is stored as " + t->dtype
                             + ", and the decoder reads F32, F16 and BF16");
        if (t->data == nullptr)
            throw ModelError("tensor '" + name + "' carries no data");
        return *t;
    }

    const HostTensor& requireShape(const std::string& name, const std::vector<long long>& expected) const
    {
        const HostTensor& t = require(name);
        if (t.extents != expected)
            throw ModelError("tensor '" + name + "' has shape " + describe(t.extents) + ", and this decoder expects "
                             + describe(expected));
        return t;
    }

    static std::vector<float> widen(const HostTensor& t)
    {
        const std::size_t n = countOf(t.extents);
        std::vector<float> out(n);
        if (t.dtype == "F32")
            std::memcpy(out.data(), t.data, n * sizeof(float));
        else
        {
            const auto* bits = static_cast<const std::uint16_t*>(t.data);
            for (std::size_t i = 0; i < n; ++i)
                out[i] = t.dtype == "F16" ? halfToFloat(bits[i]) : bfloat16ToFloat(bits[i]);
        }
        return out;
    }

    TensorBuffer floats(const std::string& name, const std::vector<long long>& extents) const
    {
        const auto values = widen(requireShape(name, extents));
        TensorBuffer b;
        b.storage = std::make_shared<DeviceBuffer>(device, values.data(), values.size() * sizeof(float));
        for (long long e : extents)
            b.extents.push_back((int) e);
        b.type = WeightStorage::Float;
        return b;
    }
};

WeightStorage storageOfFile(const std::string& dtype)
{
    return dtype == "F16" ? WeightStorage::PackedHalf
           : dtype == "BF16" ? WeightStorage::PackedBFloat16
                             : WeightStorage::Float;
}

// The halves of `values` if narrowing changes none of them, else nothing
// (Model/SafeTensors.cpp:554-592).
bool exactHalves(const std::vector<float>& values, std::vector<std::uint16_t>& halves)
{
    halves.resize(values.size());
    for (std::size_t i = 0; i < values.size(); ++i)
    {
        halves[i] = floatToHalf(values[i]);
        const float back = halfToFloat(halves[i]);
        if (std::memcmp(&back, &values[i], sizeof(float)) != 0)
            return false;
    }
    return true;
}

// The bytes one projection weight is uploaded with: the file's own halves for
// a packed file, an exact fp16 narrowing under ExactHalf, floats otherwise.
struct ProjectionBytes
{
    WeightStorage type = WeightStorage::Float;
    std::vector<unsigned char> bytes;
};

ProjectionBytes projectionBytes(const HostTensor& t, WeightPacking packing)
{
    ProjectionBytes out;
    const std::size_t n = countOf(t.extents);
    if (t.dtype != "F32")
    {
        out.type = storageOfFile(t.dtype);
        out.bytes.resize(n * 2);
        std::memcpy(out.bytes.data(), t.data, n * 2);
        return out;
    }
    const auto values = Loader::widen(t);
    std::vector<std::uint16_t> halves;
    if (packing == WeightPacking::ExactHalf && exactHalves(values, halves))
    {
        out.type = WeightStorage::PackedHalf;
        out.bytes.resize(n * 2);
        std::memcpy(out.bytes.data(), halves.data(), n * 2);
        return out;
    }
    out.bytes.resize(n * 4);
    std::memcpy(out.bytes.data(), values.data(), n * 4);
    return out;
}

// Widens a packed projection to float bytes (used when q, k and v disagree
// on storage and have to share the float block).
ProjectionBytes asFloats(const ProjectionBytes& p, std::size_t n)
{
    if (p.type == WeightStorage::Float)
        return p;
    ProjectionBytes out;
    out.bytes.resize(n * 4);
    const auto* bits = reinterpret_cast<const std::uint16_t*>(p.bytes.data());
    auto* f = reinterpret_cast<float*>(out.bytes.data());
    for (std::size_t i = 0; i < n; ++i)
        f[i] = p.type == WeightStorage::PackedHalf ? halfToFloat(bits[i]) : bfloat16ToFloat(bits[i]);
    return out;
}

TensorBuffer upload(const Device& device, const ProjectionBytes& p, std::vector<int> extents)
{
    TensorBuffer b;
    b.storage = std::make_shared<DeviceBuffer>(device, p.bytes.data(), p.bytes.size());
    b.extents = std::move(extents);
    b.type = p.type;
    return b;
}

TensorBuffer viewOf(const TensorBuffer& block, std::size_t byteOffset, std::vector<int> extents)
{
    TensorBuffer v;
    v.storage = block.storage;
    v.byteOffset = block.byteOffset + byteOffset;
    v.extents = std::move(extents);
    v.type = block.type;
    return v;
}
} // namespace

const HostTensor* MapTensorSource::find(const std::string& name) const
{
    const auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
}

DecoderWeights::DecoderWeights(const TensorSource& file, const DecoderShape& shapeToUse, WeightPacking packing,
                               const Device& device)
    : shape(shapeToUse)
{
    const Loader load {file, device};
    const long long d = shape.width, f = shape.feedForwardWidth, v = shape.vocabularySize;

    // embed_tokens: always float for the gather; the logits may get a packed
    // copy (Decoder/DecoderWeights.cpp:24-41, 151-178).
    const std::string tokenName = decoderPrefix + "embed_tokens.weight";
    const HostTensor& tokens = load.requireShape(tokenName, {v, d});
    tokenEmbedding = load.floats(tokenName, {v, d});
    if (packing == WeightPacking::ExactHalf)
    {
        if (tokens.dtype != "F32")
            packedTokenEmbedding = upload(device, projectionBytes(tokens, WeightPacking::Float), {(int) v, (int) d});
        else
        {
            const auto p = projectionBytes(tokens, WeightPacking::ExactHalf);
            if (p.type == WeightStorage::PackedHalf)
                packedTokenEmbedding = upload(device, p, {(int) v, (int) d});
        }
    }

    // embed_positions: more rows than maxPositions is fine, fewer is not
    // (Decoder/DecoderWeights.cpp:43-69).
    const std::string positionName = decoderPrefix + "embed_positions.weight";
    const HostTensor& positions = load.require(positionName);
    if (positions.extents.size() != 2 || positions.extents[1] != d)
        throw ModelError("tensor '" + positionName + "' has shape " + describe(positions.extents)
                         + ", and this decoder expects rows of " + std::to_string(d));
    if (positions.extents[0] < shape.maxPositions)
        throw ModelError("tensor '" + positionName + "' carries " + std::to_string(positions.extents[0])
                         + " positions, and this decoder was built for " + std::to_string(shape.maxPositions));
    positionalEmbedding = load.floats(positionName, positions.extents);

    finalNormWeight = load.floats(decoderPrefix + "layer_norm.weight", {d});
    finalNormBias = load.floats(decoderPrefix + "layer_norm.bias", {d});

    layers.reserve((std::size_t) shape.layers);
    for (int i = 0; i < shape.layers; ++i)
    {
        DecoderLayerWeights w;
        auto vec = [&](const std::string& suffix, long long n) { return load.floats(layerName(i, suffix), {n}); };
        auto projection = [&](const std::string& suffix, long long rows, long long cols) {
            return projectionBytes(load.requireShape(layerName(i, suffix), {rows, cols}), packing);
        };

        w.selfAttentionNormWeight = vec("self_attn_layer_norm.weight", d);
        w.selfAttentionNormBias = vec("self_attn_layer_norm.bias", d);

        // q, k and v share one [3d, d] block in one storage.
        ProjectionBytes q = projection("self_attn.q_proj.weight", d, d);
        ProjectionBytes k = projection("self_attn.k_proj.weight", d, d);
        ProjectionBytes vv = projection("self_attn.v_proj.weight", d, d);
        if (q.type != k.type || q.type != vv.type)
        {
            q = asFloats(q, (std::size_t) (d * d));
            k = asFloats(k, (std::size_t) (d * d));
            vv = asFloats(vv, (std::size_t) (d * d));
        }
        ProjectionBytes block;
        block.type = q.type;
        block.bytes = q.bytes;
        block.bytes.insert(block.bytes.end(), k.bytes.begin(), k.bytes.end());
        block.bytes.insert(block.bytes.end(), vv.bytes.begin(), vv.bytes.end());
        const TensorBuffer qkv = upload(device, block, {(int) (3 * d), (int) d});
        const std::size_t matrixBytes = q.bytes.size();
        w.selfQueryWeight = viewOf(qkv, 0, {(int) d, (int) d});
        w.selfKeyWeight = viewOf(qkv, matrixBytes, {(int) d, (int) d});
        w.selfValueWeight = viewOf(qkv, 2 * matrixBytes, {(int) d, (int) d});

        // [q_bias | 0 | v_bias]: k_proj has no bias (Decoder/DecoderWeights.h:19-23).
        std::vector<float> biases((std::size_t) (3 * d), 0.f);
        const auto qb = Loader::widen(load.requireShape(layerName(i, "self_attn.q_proj.bias"), {d}));
        const auto vb = Loader::widen(load.requireShape(layerName(i, "self_attn.v_proj.bias"), {d}));
        std::copy(qb.begin(), qb.end(), biases.begin());
        std::copy(vb.begin(), vb.end(), biases.begin() + 2 * d);
        w.selfQkvBias.storage = std::make_shared<DeviceBuffer>(device, biases.data(), biases.size() * sizeof(float));
        w.selfQkvBias.extents = {(int) (3 * d)};
        w.selfQueryBias = viewOf(w.selfQkvBias, 0, {(int) d});
        w.selfValueBias = viewOf(w.selfQkvBias, (std::size_t) (2 * d) * sizeof(float), {(int) d});

        w.selfAttentionOutputWeight = upload(device, projection("self_attn.out_proj.weight", d, d), {(int) d, (int) d});
        w.selfAttentionOutputBias = vec("self_attn.out_proj.bias", d);

        w.crossAttentionNormWeight = vec("encoder_attn_layer_norm.weight", d);
        w.crossAttentionNormBias = vec("encoder_attn_layer_norm.bias", d);
        w.crossQueryWeight = upload(device, projection("encoder_attn.q_proj.weight", d, d), {(int) d, (int) d});
        w.crossQueryBias = vec("encoder_attn.q_proj.bias", d);
        w.crossKeyWeight = upload(device, projection("encoder_attn.k_proj.weight", d, d), {(int) d, (int) d});
        w.crossValueWeight = upload(device, projection("encoder_attn.v_proj.weight", d, d), {(int) d, (int) d});
        w.crossValueBias = vec("encoder_attn.v_proj.bias", d);
        w.crossAttentionOutputWeight =
            upload(device, projection("encoder_attn.out_proj.weight", d, d), {(int) d, (int) d});
        w.crossAttentionOutputBias = vec("encoder_attn.out_proj.bias", d);

        w.finalNormWeight = vec("final_layer_norm.weight", d);
        w.finalNormBias = vec("final_layer_norm.bias", d);
        w.feedForwardWeight = upload(device, projection("fc1.weight", f, d), {(int) f, (int) d});
        w.feedForwardBias = vec("fc1.bias", f);
        w.feedForwardOutputWeight = upload(device, projection("fc2.weight", d, f), {(int) d, (int) f});
        w.feedForwardOutputBias = vec("fc2.bias", d);

        layers.push_back(std::move(w));
    }
}

std::optional<WeightStorage> DecoderWeights::uniformProjectionStorage() const
{
    if (layers.empty())
        return std::nullopt;
    const WeightStorage first = layers[0].selfQueryWeight.type;
    for (const auto& w : layers)
    {
        const TensorBuffer* all[] = {&w.selfQueryWeight, &w.selfAttentionOutputWeight, &w.crossQueryWeight,
                                     &w.crossAttentionOutputWeight, &w.feedForwardWeight,
                                     &w.feedForwardOutputWeight};
        for (const TensorBuffer* t : all)
            if (t->type != first)
                return std::nullopt;
    }
    return first;
}

wsp_layer_tensors layerTable(const DecoderLayerWeights& w)
{
    auto f = [](const TensorBuffer& t) { return static_cast<const float*>(t.data()); };
    wsp_layer_tensors L {};
    L.self_norm_w = f(w.selfAttentionNormWeight);
    L.self_norm_b = f(w.selfAttentionNormBias);
    L.self_qkv_w = w.selfQueryWeight.data();
    L.self_qkv_b = f(w.selfQkvBias);
    L.self_out_w = w.selfAttentionOutputWeight.data();
    L.self_out_b = f(w.selfAttentionOutputBias);
    L.cross_norm_w = f(w.crossAttentionNormWeight);
    L.cross_norm_b = f(w.crossAttentionNormBias);
    L.cross_q_w = w.crossQueryWeight.data();
    L.cross_q_b = f(w.crossQueryBias);
    L.cross_out_w = w.crossAttentionOutputWeight.data();
    L.cross_out_b = f(w.crossAttentionOutputBias);
    L.final_norm_w = f(w.finalNormWeight);
    L.final_norm_b = f(w.finalNormBias);
    L.fc1_w = w.feedForwardWeight.data();
    L.fc1_b = f(w.feedForwardBias);
    L.fc2_w = w.feedForwardOutputWeight.data();
    L.fc2_b = f(w.feedForwardOutputBias);
    return L;
}

wsp_decoder_tensors decoderTable(const DecoderWeights& weights, const std::vector<wsp_layer_tensors>& layers)
{
    const auto storage = weights.uniformProjectionStorage();
    if (!storage)
        throw std::logic_error("the fused and batched steps need one storage for every projection weight");
    wsp_decoder_tensors tensors {};
    tensors.wdtype = wsp_dtype_of(*storage);
    tensors.token_embedding = static_cast<const float*>(weights.tokenEmbedding.data());
    tensors.logits_weight = weights.logitsWeight().data();
    tensors.logits_wdtype = wsp_dtype_of(weights.logitsWeight().type);
    tensors.position_embedding = static_cast<const float*>(weights.positionalEmbedding.data());
    tensors.final_norm_w = static_cast<const float*>(weights.finalNormWeight.data());
    tensors.final_norm_b = static_cast<const float*>(weights.finalNormBias.data());
    tensors.layers = layers.data();
    return tensors;
}
} // namespace WSP
