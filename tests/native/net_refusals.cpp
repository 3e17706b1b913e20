// The misuse refusals of WSP::HipNet, the gfx950 Net backend. HipNet records a
// program and places every value when the recording ends, so a misuse is
// refused either at the op (no recording open, a stale or foreign handle, a
// cache overflow, a bad output()) or at end() before the first launch (a value
// with nowhere to live, scratch buffers too few for the values live at once).
// Each case misuses a fresh net and must get std::logic_error naming the
// problem. One proper recording runs on the device, and a chain of LayerNorms
// whose handles all stay held shows buffers shared by liveness. Test
// infrastructure (tests/test_gpu_net.py and tests/test_abi.py run it).
//
//   net_refusals host      the cases that need no device (nothing prepared)
//   net_refusals device    the cases on a prepared net (device 0)
//
// Prints "ok <case>" or "FAIL <case>: <why>" per case; the exit status is the
// number of failures.
#include "../../include/whispereacp/HipNet.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

using namespace WSP;

namespace
{
int failures = 0;

void expectRefusal(const char* name, const char* fragment, const std::function<void()>& misuse)
{
    try
    {
        misuse();
        std::printf("FAIL %s: no exception\n", name);
        ++failures;
    }
    catch (const std::logic_error& e)
    {
        if (std::strstr(e.what(), fragment) == nullptr)
        {
            std::printf("FAIL %s: logic_error \"%s\" does not say \"%s\"\n", name, e.what(), fragment);
            ++failures;
        }
        else
            std::printf("ok %s\n", name);
    }
    catch (const std::exception& e)
    {
        std::printf("FAIL %s: %s instead of a logic_error\n", name, e.what());
        ++failures;
    }
}

void expectNoRefusal(const char* name, const std::function<void()>& use)
{
    try
    {
        use();
        std::printf("ok %s\n", name);
    }
    catch (const std::exception& e)
    {
        std::printf("FAIL %s: %s\n", name, e.what());
        ++failures;
    }
}

constexpr int kWidth = 64;

DecoderShape tinyShape()
{
    DecoderShape s;
    s.width = kWidth;
    s.heads = 4;
    s.layers = 1;
    s.feedForwardWidth = 4 * kWidth;
    s.vocabularySize = 97;
    s.maxPositions = 8;
    s.crossPositions = 8;
    return s;
}

HipNetLayout layout(int slots, int values = 4096)
{
    HipNetLayout l;
    l.shape = tinyShape();
    l.scratch = {{kWidth, slots}};
    l.valueCapacity = values;
    return l;
}

// LayerNorm of one row, gamma 1 and beta 0, in double (the oracle's formula).
std::vector<double> hostLayerNorm(const std::vector<double>& x)
{
    double mean = 0;
    for (double v : x)
        mean += v;
    mean /= (double) x.size();
    double var = 0;
    for (double v : x)
        var += (v - mean) * (v - mean);
    var /= (double) x.size();
    std::vector<double> y(x.size());
    for (std::size_t i = 0; i < x.size(); ++i)
        y[i] = (x[i] - mean) / std::sqrt(var + 1e-5);
    return y;
}

// A device vector of `count` floats, all `value`.
Weight vectorOf(const Device& device, int count, float value)
{
    std::vector<float> host((std::size_t) count, value);
    Weight w;
    w.storage = std::make_shared<DeviceBuffer>(device, host.data(), host.size() * sizeof(float));
    w.extents = {count};
    return w;
}

Weight matrixOf(const Device& device, int rows, int columns, float value)
{
    Weight w = vectorOf(device, rows * columns, value);
    w.extents = {rows, columns};
    return w;
}

Binding bindingOf(const Weight& w, int rows, int columns)
{
    return Binding {BufferRange {w.storage->data(), 0, w.storage->size()}, Shape {rows, columns}, "x"};
}

void hostCases()
{
    expectRefusal("begin before prepare", "not prepared", [] {
        HipNet net;
        Pass pass;
        net.begin(pass);
    });
    expectRefusal("cache before prepare", "not prepared", [] {
        HipNet net;
        (void) net.makeCache(4, kWidth);
    });
    expectRefusal("an op before prepare", "no recording is open", [] {
        HipNet net;
        (void) net.input(Binding {}, Shape {1, kWidth}, DType::float32);
    });
    expectRefusal("transpose is an encoder op", "encoder op", [] {
        HipNet net;
        (void) net.transpose(Tensor {});
    });
    expectRefusal("conv1d is an encoder op", "encoder op", [] {
        HipNet net;
        Weight w;
        (void) net.conv1d(Tensor {}, w, w, 1, 1, Activation::none);
    });
    expectRefusal("add is an encoder op", "encoder op", [] {
        HipNet net;
        (void) net.add(Tensor {}, Tensor {});
    });
    expectRefusal("a shape of five extents", "at most four extents", [] { (void) Shape {1, 2, 3, 4, 5}; });
}

void deviceCases()
{
    const Device device {0};
    const Weight x = matrixOf(device, 1, kWidth, 0.5f);
    const Weight gamma = vectorOf(device, kWidth, 1.0f);
    const Weight beta = vectorOf(device, kWidth, 0.0f);
    const Weight square = matrixOf(device, kWidth, kWidth, 0.01f);
    const Weight out = matrixOf(device, 1, kWidth, 0.0f);

    expectRefusal("an op with no recording open", "no recording is open", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        (void) net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
    });
    expectRefusal("a pass on another stream", "another stream", [&] {
        hipStream_t other = nullptr;
        if (hipStreamCreate(&other) != hipSuccess)
            throw std::runtime_error("hipStreamCreate");
        struct Destroy
        {
            hipStream_t s;
            ~Destroy() { (void) hipStreamDestroy(s); }
        } destroy {other};
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass(other);
        net.begin(pass);
    });
    expectRefusal("a second begin", "already open", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        net.begin(pass);
    });
    expectRefusal("a handle kept past its recording", "recording that has ended", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor kept = net.layerNorm(in, gamma, beta);
        net.output(kept, bindingOf(out, 1, kWidth));
        net.end();
        pass.synchronize();
        net.begin(pass);
        (void) net.layerNorm(kept, gamma, beta);
    });
    expectRefusal("more values live than scratch buffers", "are live than the 2 scratch buffers", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor a = net.layerNorm(in, gamma, beta);
        Tensor b = net.layerNorm(in, gamma, beta);
        Tensor c = net.layerNorm(in, gamma, beta); // a and b are read later: three live here
        (void) net.linearAdd(a, square, nullptr, c);
        net.output(net.layerNorm(b, gamma, beta), bindingOf(out, 1, kWidth));
        net.end();
    });
    expectRefusal("more values than the table holds", "already holds 8 values", [&] {
        HipNet net;
        net.prepare(device, layout(2, 8), nullptr);
        Pass pass;
        net.begin(pass);
        for (int i = 0; i < 9; ++i)
            (void) net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
    });
    expectRefusal("a tensor of another net", "not a value of this net", [&] {
        HipNet first, second;
        first.prepare(device, layout(2), nullptr);
        second.prepare(device, layout(2), nullptr);
        Pass pass;
        first.begin(pass);
        second.begin(pass);
        Tensor in = first.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        (void) second.layerNorm(in, gamma, beta);
    });
    expectRefusal("a value with nowhere to live", "no scratch buffers of that capacity", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        const Weight rows = matrixOf(device, 2, kWidth, 0.25f);
        Tensor in = net.input(bindingOf(rows, 2, kWidth), Shape {2, kWidth}, DType::float32);
        (void) net.layerNorm(in, gamma, beta); // 128 floats: no class, never bound
        net.end();
    });
    expectRefusal("a cache appended past its capacity", "would overflow a cache", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Cache cache = net.makeCache(2, kWidth);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor r1 = net.appendLinear(cache, in, square, nullptr);
        Tensor r2 = net.appendLinear(cache, in, square, nullptr);
        Tensor r3 = net.appendLinear(cache, in, square, nullptr); // the cache holds two rows
    });
    expectRefusal("output() of a view", "view of storage", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        net.output(in, bindingOf(out, 1, kWidth));
    });
    // The same ops used as the net intends pass, so the refusals above are the
    // misuse and not the setup.
    expectNoRefusal("a proper recording", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Cache cache = net.makeCache(2, kWidth);
        Pass pass;
        net.begin(pass);
        {
            Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
            Tensor a = net.layerNorm(in, gamma, beta);
            Tensor r = net.appendLinear(cache, a, square, nullptr);
            net.output(net.linear(a, square, nullptr, Activation::none), bindingOf(out, 1, kWidth));
        }
        net.end();
        pass.synchronize();
    });
    // Four chained LayerNorms whose handles all stay held: their spans meet
    // pairwise only, so two buffers carry them, and the bound result matches
    // four LayerNorms on the host.
    expectNoRefusal("a chain sharing two buffers", [&] {
        std::vector<float> row(kWidth);
        for (int i = 0; i < kWidth; ++i)
            row[(std::size_t) i] = (float) (i % 7) - 2.5f + 0.01f * (float) i;
        Weight input;
        input.storage = std::make_shared<DeviceBuffer>(device, row.data(), row.size() * sizeof(float));
        input.extents = {1, kWidth};
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(input, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor a = net.layerNorm(in, gamma, beta);
        Tensor b = net.layerNorm(a, gamma, beta);
        Tensor c = net.layerNorm(b, gamma, beta);
        Tensor d = net.layerNorm(c, gamma, beta);
        Tensor e = net.layerNorm(d, gamma, beta);
        net.output(e, bindingOf(out, 1, kWidth));
        net.end();
        pass.synchronize();
        if (net.scratchHighWater().at(0) != 2)
            throw std::runtime_error("the chain used " + std::to_string(net.scratchHighWater().at(0))
                                     + " buffers, not 2");
        std::vector<float> got(kWidth);
        out.storage->read(got.data(), got.size() * sizeof(float));
        std::vector<double> want(row.begin(), row.end());
        for (int k = 0; k < 5; ++k)
            want = hostLayerNorm(want);
        for (int i = 0; i < kWidth; ++i)
            if (std::fabs(got[(std::size_t) i] - want[(std::size_t) i]) > 1e-4)
                throw std::runtime_error("element " + std::to_string(i) + ": " + std::to_string(got[(std::size_t) i])
                                         + " against " + std::to_string(want[(std::size_t) i]));
    });
}
} // namespace

int main(int argc, char** argv)
{
    const bool device = argc > 1 && std::strcmp(argv[1], "device") == 0;
    if (argc < 2 || (!device && std::strcmp(argv[1], "host") != 0))
    {
        std::fprintf(stderr, "usage: %s host|device\n", argv[0]);
        return 2;
    }
    if (device)
        deviceCases();
    else
        hostCases();
    return failures;
}
