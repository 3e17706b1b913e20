// The misuse refusals of WSP::HipNet, the gfx950 Net backend, in the manner of
// the reference's KernelNet (Net/KernelNet.cpp:228-244, 274-288, 313-335): each
// case misuses a fresh net and must get std::logic_error with the reference's
// message, before anything wrong reaches the device. Test infrastructure
// (tests/test_gpu_net.py and tests/test_abi.py run it).
//
//   net_refusals host      the cases that need no device (nothing prepared)
//   net_refusals device    the cases on a prepared net (device 0)
//
// Prints "ok <case>" or "FAIL <case>: <why>" per case; the exit status is the
// number of failures.
#include "../../include/whispereacp/HipNet.h"

#include <hip/hip_runtime_api.h>

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

HipNetLayout layout(int slots)
{
    HipNetLayout l;
    l.shape = tinyShape();
    l.scratch = {{kWidth, slots}};
    return l;
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
    expectRefusal("begin before prepare", "records once it is prepared", [] {
        HipNet net;
        Pass pass;
        net.begin(pass);
    });
    expectRefusal("cache before prepare", "makes a cache once it is prepared", [] {
        HipNet net;
        (void) net.makeCache(4, kWidth);
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

    expectRefusal("an op outside begin and end", "records between begin() and end()", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor a = net.layerNorm(in, gamma, beta);
        Tensor b = net.layerNorm(a, gamma, beta); // dispatches the first: no pass is open
    });
    expectRefusal("a pass on another stream", "the stream it was prepared with", [&] {
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
    expectRefusal("a value outliving its recording", "outlived the recording", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        Tensor kept;
        net.begin(pass);
        {
            Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
            kept = net.layerNorm(in, gamma, beta);
        }
        net.end(); // kept still holds a scratch buffer
    });
    expectRefusal("every scratch buffer held", "every scratch buffer of 64 elements is holding a value", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        Tensor in = net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        Tensor a = net.layerNorm(in, gamma, beta);
        Tensor b = net.layerNorm(in, gamma, beta);
        Tensor c = net.layerNorm(in, gamma, beta); // two buffers of this capacity were reserved
    });
    expectRefusal("more live values than records", "more values at once than it has records for", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        std::vector<Tensor> held;
        for (int i = 0; i < 65; ++i)
            held.push_back(net.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32));
    });
    expectRefusal("a tensor of another net", "holds no value of this net", [&] {
        HipNet first, second;
        first.prepare(device, layout(2), nullptr);
        second.prepare(device, layout(2), nullptr);
        Tensor in = first.input(bindingOf(x, 1, kWidth), Shape {1, kWidth}, DType::float32);
        (void) second.layerNorm(in, gamma, beta);
    });
    expectRefusal("a value with no buffer of its capacity", "has to be placed by output()", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Pass pass;
        net.begin(pass);
        const Weight rows = matrixOf(device, 2, kWidth, 0.25f);
        Tensor in = net.input(bindingOf(rows, 2, kWidth), Shape {2, kWidth}, DType::float32);
        Tensor a = net.layerNorm(in, gamma, beta); // 128 elements: nothing was reserved at that capacity
        Tensor b = net.layerNorm(in, gamma, beta);
    });
    expectRefusal("a cache appended past its capacity", "appended to past its capacity", [&] {
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
    // The same recording used as the net intends passes, so the refusals above
    // are the misuse and not the setup.
    expectNoRefusal("a proper recording", [&] {
        HipNet net;
        net.prepare(device, layout(2), nullptr);
        Cache cache = net.makeCache(2, kWidth);
        const Weight out = matrixOf(device, 1, kWidth, 0.0f);
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
