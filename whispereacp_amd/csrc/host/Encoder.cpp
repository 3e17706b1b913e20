// EncoderShape from config.json, EncoderWeights and the Encoder wrapper
// (Encoder/EncoderShape.h:25-67, Encoder/EncoderWeights.cpp:1-200,
// Encoder/Encoder.cpp:113-174) over the gfx950 encoder's C ABI.
#include "../../../include/whispereacp/Encoder.h"
#include "../../../include/whispereacp/ModelError.h"
#include "host_common.h"
#include "json.h"

#include <cstring>
#include <limits>
#include <sstream>

namespace WSP
{
namespace
{
int positiveField(const Json& config, const char* key)
{
    const Json* v = config.member(key);
    if (v == nullptr)
        throw ModelError(std::string("config.json has no '") + key + "'");
    if (v->kind != Json::Kind::Number || !v->integral || v->integer <= 0 || v->integer > std::numeric_limits<int>::max())
        throw ModelError(std::string("config.json '") + key + "' is not a positive integer");
    return (int) v->integer;
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

std::vector<float> widened(const HostTensor& t)
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

const std::string encoderPrefix = "model.encoder.";

std::string layerName(int index, const char* suffix)
{
    return encoderPrefix + "layers." + std::to_string(index) + "." + suffix;
}

// A tensor checked against the extents this encoder expects; the first axis
// of embed_positions is a capacity (Encoder/EncoderWeights.cpp:24-45).
const HostTensor& require(const TensorSource& file, const std::string& name, const std::vector<long long>& expected,
                          bool capacityFirst = false)
{
    const HostTensor* t = file.find(name);
    if (t == nullptr)
        throw ModelError("tensor '" + name + "' is missing from the encoder file");
    if (t->dtype != "F32" && t->dtype != "F16" && t->dtype != "BF16")
        throw ModelError("tensor '" + name + "' is stored as " + t->dtype + ", and the encoder reads F32, F16 and BF16");
    if (t->data == nullptr)
        throw ModelError("tensor '" + name + "' carries no data");
    if (capacityFirst)
    {
        if (t->extents.size() != 2 || t->extents[1] != expected[1])
            throw ModelError("tensor '" + name + "' has shape " + describe(t->extents)
                             + ", and this encoder expects [positions, " + std::to_string(expected[1]) + "]");
        if (t->extents[0] < expected[0])
            throw ModelError("tensor '" + name + "' carries " + std::to_string(t->extents[0])
                             + " positions, and this run needs " + std::to_string(expected[0]));
    }
    else if (t->extents != expected)
        throw ModelError("tensor '" + name + "' has shape " + describe(t->extents) + ", and this encoder expects "
                         + describe(expected));
    return *t;
}

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

int storageOf(const std::string& dtype)
{
    return dtype == "F16" ? WSP_F16 : dtype == "BF16" ? WSP_BF16 : WSP_F32;
}
} // namespace

EncoderShape encoderShapeFromConfig(const std::string& json)
{
    const Json config = JsonReader(json.data(), json.data() + json.size(), "config.json").document();
    if (config.kind != Json::Kind::Object)
        throw ModelError("config.json is not a JSON object");
    EncoderShape s;
    s.melBins = positiveField(config, "num_mel_bins");
    s.width = positiveField(config, "d_model");
    s.heads = positiveField(config, "encoder_attention_heads");
    s.layers = positiveField(config, "encoder_layers");
    s.feedForwardWidth = positiveField(config, "encoder_ffn_dim");
    const int source = positiveField(config, "max_source_positions");
    if (source > std::numeric_limits<int>::max() / 2)
        throw ModelError("config.json 'max_source_positions' is too large");
    s.inputFrames = 2 * source;
    if (s.width % s.heads != 0)
        throw ModelError("config.json d_model does not divide into the encoder head count");
    return s;
}

EncoderWeights::EncoderWeights(const TensorSource& file, const EncoderShape& shapeToUse, WeightPacking packing,
                               const Device& device)
    : shape(shapeToUse)
{
    const long long d = shape.width, f = shape.feedForwardWidth, k = EncoderShape::convolutionKernelSize;

    // Every check first, so a bad file uploads nothing.
    struct Entry
    {
        std::string name;
        const HostTensor* tensor;
        bool projection;
    };
    std::vector<Entry> entries;
    auto add = [&](const std::string& name, std::vector<long long> extents, bool projection = false,
                   bool capacityFirst = false) {
        entries.push_back({name, &require(file, name, extents, capacityFirst), projection});
    };
    add(encoderPrefix + "conv1.weight", {d, shape.melBins, k});
    add(encoderPrefix + "conv1.bias", {d});
    add(encoderPrefix + "conv2.weight", {d, d, k});
    add(encoderPrefix + "conv2.bias", {d});
    add(encoderPrefix + "embed_positions.weight", {shape.positions(), d}, false, true);
    add(encoderPrefix + "layer_norm.weight", {d});
    add(encoderPrefix + "layer_norm.bias", {d});
    for (int i = 0; i < shape.layers; ++i)
    {
        add(layerName(i, "self_attn_layer_norm.weight"), {d});
        add(layerName(i, "self_attn_layer_norm.bias"), {d});
        add(layerName(i, "self_attn.q_proj.weight"), {d, d}, true);
        add(layerName(i, "self_attn.q_proj.bias"), {d});
        add(layerName(i, "self_attn.k_proj.weight"), {d, d}, true);
        add(layerName(i, "self_attn.v_proj.weight"), {d, d}, true);
        add(layerName(i, "self_attn.v_proj.bias"), {d});
        add(layerName(i, "self_attn.out_proj.weight"), {d, d}, true);
        add(layerName(i, "self_attn.out_proj.bias"), {d});
        add(layerName(i, "final_layer_norm.weight"), {d});
        add(layerName(i, "final_layer_norm.bias"), {d});
        add(layerName(i, "fc1.weight"), {f, d}, true);
        add(layerName(i, "fc1.bias"), {f});
        add(layerName(i, "fc2.weight"), {d, f}, true);
        add(layerName(i, "fc2.bias"), {d});
    }

    // The projections' one storage: the file's when every projection shares a
    // packed dtype; fp16 when every F32 projection narrows exactly under
    // ExactHalf (Model/SafeTensors.cpp:554-592); float otherwise.
    int storage = -1;
    bool uniform = true;
    for (const Entry& e : entries)
        if (e.projection)
        {
            const int s = storageOf(e.tensor->dtype);
            if (storage >= 0 && s != storage)
                uniform = false;
            storage = s;
        }
    if (storage < 0 || !uniform)
        storage = WSP_F32;
    std::vector<std::vector<std::uint16_t>> packedHalves;
    if (storage == WSP_F32 && uniform && packing == WeightPacking::ExactHalf)
    {
        bool exact = true;
        for (const Entry& e : entries)
            if (e.projection && exact)
            {
                packedHalves.emplace_back();
                exact = e.tensor->dtype == "F32" && exactHalves(widened(*e.tensor), packedHalves.back());
            }
        if (exact)
            storage = WSP_F16;
        else
            packedHalves.clear();
    }
    // BF16 projections as exact fp16 multiples w·2^k (wsp_encoder_scaled_halves),
    // all or none: the products then read two fp16 parts of their input
    // instead of three bf16 ones.
    std::vector<float> scales;
    if (storage == WSP_BF16 && shape.layers > 0)
    {
        const wsp_encoder_shape cs = shape.cShape();
        for (const Entry& e : entries)
            if (e.projection)
            {
                const std::size_t n = countOf(e.tensor->extents);
                packedHalves.emplace_back(n);
                float scale = 1.f;
                const int status = wsp_encoder_scaled_halves(&cs, e.tensor->data, n, packedHalves.back().data(), &scale);
                if (status == WSP_ERR_LOGIC || status == WSP_ERR_SHAPE)
                {
                    packedHalves.clear();
                    scales.clear();
                    break;
                }
                if (status != WSP_OK)
                    throwForStatus(status, "wsp_encoder_scaled_halves failed");
                scales.push_back(scale);
            }
        if (!packedHalves.empty())
            storage = WSP_F16;
    }
    projectionType = storage;

    buffers.reserve(entries.size());
    std::size_t packedIndex = 0;
    std::vector<const void*> pointers;
    std::vector<float> entryScales; // per entry: its projection's scale (1 for the rest)
    for (const Entry& e : entries)
    {
        entryScales.push_back(e.projection && !scales.empty() ? scales[packedIndex] : 1.f);
        if (e.projection && storage == WSP_F16 && !packedHalves.empty())
        {
            const auto& h = packedHalves[packedIndex++];
            buffers.emplace_back(device, h.data(), h.size() * sizeof(std::uint16_t));
        }
        else if (e.projection && storage != WSP_F32)
            buffers.emplace_back(device, e.tensor->data, countOf(e.tensor->extents) * sizeof(std::uint16_t));
        else
        {
            const auto values = widened(*e.tensor);
            buffers.emplace_back(device, values.data(), values.size() * sizeof(float));
        }
        pointers.push_back(buffers.back().data());
    }

    auto f32 = [&](std::size_t i) { return static_cast<const float*>(pointers[i]); };
    model.wdtype = storage;
    model.conv1_w = f32(0);
    model.conv1_b = f32(1);
    model.conv2_w = f32(2);
    model.conv2_b = f32(3);
    model.positions = f32(4);
    model.final_norm_w = f32(5);
    model.final_norm_b = f32(6);
    layerTable.resize((std::size_t) shape.layers);
    for (int i = 0; i < shape.layers; ++i)
    {
        const std::size_t b = 7 + (std::size_t) i * 15;
        wsp_encoder_layer_tensors& L = layerTable[(std::size_t) i];
        L.attention_norm_w = f32(b + 0);
        L.attention_norm_b = f32(b + 1);
        L.q_w = pointers[b + 2];
        L.q_b = f32(b + 3);
        L.k_w = pointers[b + 4];
        L.v_w = pointers[b + 5];
        L.v_b = f32(b + 6);
        L.out_w = pointers[b + 7];
        L.out_b = f32(b + 8);
        L.final_norm_w = f32(b + 9);
        L.final_norm_b = f32(b + 10);
        L.fc1_w = pointers[b + 11];
        L.fc1_b = f32(b + 12);
        L.fc2_w = pointers[b + 13];
        L.fc2_b = f32(b + 14);
        L.q_scale = entryScales[b + 2];
        L.k_scale = entryScales[b + 4];
        L.v_scale = entryScales[b + 5];
        L.out_scale = entryScales[b + 7];
        L.fc1_scale = entryScales[b + 11];
        L.fc2_scale = entryScales[b + 13];
    }
}

wsp_encoder_tensors EncoderWeights::table() const
{
    wsp_encoder_tensors t = model;
    t.layers = layerTable.empty() ? nullptr : layerTable.data();
    return t;
}

Encoder::Encoder(const EncoderShape& shape, const Device& device, void* hipStream) : encoderShape(shape)
{
    const wsp_encoder_shape s = shape.cShape();
    const int status = wsp_encoder_create(&s, device.index, hipStream, &handle);
    if (status == WSP_ERR_SHAPE)
        throw ModelError("the gfx950 encoder takes head widths that are multiples of 4, at most 64");
    if (status != WSP_OK)
        throwForStatus(status, "wsp_encoder_create failed");
}

Encoder::~Encoder()
{
    if (handle != nullptr)
        wsp_encoder_destroy(handle);
}

void Encoder::encode(const EncoderWeights& weights, const float* mel, float* output, int positionCount)
{
    if (weights.shape.melBins != encoderShape.melBins || weights.shape.width != encoderShape.width
        || weights.shape.layers != encoderShape.layers || weights.shape.feedForwardWidth != encoderShape.feedForwardWidth)
        throw ModelError("the weights were loaded against a different encoder shape than this encoder was built for");
    const wsp_encoder_tensors t = weights.table();
    const int status = wsp_encoder_encode(handle, &t, mel, output, positionCount);
    if (status == WSP_ERR_SHAPE)
        throw ModelError(wsp_encoder_last_error(handle));
    if (status != WSP_OK)
        throwForStatus(status, wsp_encoder_last_error(handle));
}
} // namespace WSP
