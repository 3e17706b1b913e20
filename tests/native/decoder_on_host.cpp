// The decoder body (DecoderRecording.cpp) recorded against the host Net —
// TEST INFRASTRUCTURE, no GPU. Weights come from a safetensors file placed
// in host memory (Device::host()); the run opens the sequence over the
// encoder rows, decodes the prompt in one step and then `steps` single-token
// steps, each fed the argmax of the row before, and writes every logits row
// (float32, prompt rows first) to the output file.
//
//   decoder_on_host <model.safetensors> <width heads layers ffn vocab max_positions cross_positions>
//                   <encoder rows f32 file> <steps> <output file> <prompt ids...>
//
// Built once per WSP_MUTATION value by tests/native/Makefile; the mutants must
// fail the comparison with the oracle that the unmutated build passes.
#include "host_net.h"

#include <whispereacp/Decoder.h>
#include <whispereacp/SafeTensors.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <vector>

using namespace WSP;

namespace
{
std::vector<char> readAll(const char* path)
{
    std::ifstream in(path, std::ios::binary);
    return std::vector<char>((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
}

Binding bind(void* data, std::size_t bytes, Shape capacity, const char* name)
{
    return Binding {BufferRange {data, 0, bytes}, capacity, name};
}
} // namespace

int main(int argc, char** argv)
{
    if (argc < 15)
    {
        std::fprintf(stderr, "usage: decoder_on_host model shape(7) encoder steps output prompt...\n");
        return 2;
    }
    try
    {
        DecoderShape shape {std::atoi(argv[2]), std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]),
                            std::atoi(argv[6]), std::atoi(argv[7]), std::atoi(argv[8])};
        std::vector<char> encoder = readAll(argv[9]);
        const int steps = std::atoi(argv[10]);
        const char* output = argv[11];
        std::vector<std::int32_t> prompt;
        for (int i = 12; i < argc; ++i)
            prompt.push_back(std::atoi(argv[i]));
        if (encoder.size() != (std::size_t) shape.crossPositions * shape.width * 4)
            throw std::runtime_error("the encoder rows file does not hold cross_positions x width floats");

        const SafeTensors file = SafeTensors::fromFile(argv[1]);
        const DecoderWeights weights(file, shape, WeightPacking::Float, Device::host());

        Testing::HostNet net;
        DecoderCaches caches;
        for (int i = 0; i < shape.layers; ++i)
        {
            caches.selfKeys.push_back(net.makeCache(shape.maxPositions, shape.width));
            caches.selfValues.push_back(net.makeCache(shape.maxPositions, shape.width));
            caches.crossKeys.push_back(net.makeCache(shape.crossPositions, shape.width));
            caches.crossValues.push_back(net.makeCache(shape.crossPositions, shape.width));
        }
        recordSequenceStart(net, shape, weights, caches,
                            bind(encoder.data(), encoder.size(), {shape.crossPositions, shape.width}, "encoder"),
                            shape.crossPositions);

        const int V = shape.vocabularySize;
        std::vector<float> rows;
        std::vector<float> hidden((std::size_t) prompt.size() * shape.width);
        std::vector<float> logits((std::size_t) prompt.size() * V);
        recordDecoderStep(net, shape, weights, caches,
                          bind(prompt.data(), prompt.size() * 4, {(int) prompt.size()}, "tokens"), (int) prompt.size(),
                          0, bind(hidden.data(), hidden.size() * 4, {(int) prompt.size(), shape.width}, "hidden"),
                          bind(logits.data(), logits.size() * 4, {(int) prompt.size(), V}, "logits"));
        rows.insert(rows.end(), logits.begin(), logits.end());
        int position = (int) prompt.size();
        auto argmaxOfLast = [&](const std::vector<float>& r, int count) {
            const float* last = r.data() + (std::size_t) (count - 1) * V;
            int best = 0;
            for (int i = 1; i < V; ++i)
                if (last[i] > last[best])
                    best = i;
            return (std::int32_t) best;
        };
        std::int32_t token = argmaxOfLast(logits, (int) prompt.size());
        for (int s = 0; s < steps; ++s)
        {
            std::vector<float> row((std::size_t) V), h((std::size_t) shape.width);
            recordDecoderStep(net, shape, weights, caches, bind(&token, 4, {1}, "tokens"), 1, position,
                              bind(h.data(), h.size() * 4, {1, shape.width}, "hidden"),
                              bind(row.data(), row.size() * 4, {1, V}, "logits"));
            rows.insert(rows.end(), row.begin(), row.end());
            ++position;
            token = argmaxOfLast(row, 1);
        }
        std::ofstream out(output, std::ios::binary);
        out.write(reinterpret_cast<const char*>(rows.data()), (std::streamsize) (rows.size() * 4));
        return out ? 0 : 1;
    }
    catch (const std::exception& e)
    {
        std::fprintf(stderr, "decoder_on_host: %s\n", e.what());
        return 1;
    }
}
