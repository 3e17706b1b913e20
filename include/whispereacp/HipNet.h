// HipNet: the gfx950 backend of Net (Net/Net.h:110-171), run as a recorded
// program over the C ABI in wsp_hip.h.
//
// begin() opens a recording. Each op appends one instruction and returns a
// handle to the value that instruction writes; nothing reaches the device
// while the recording is open. end() then works in two passes:
//
//   1. placement. Every value gets its home before anything runs:
//      - a value given to output() lives in the caller's binding, so the
//        instruction that writes it writes there (the meaning
//        Net/KernelNet.cpp:487-513 gives output());
//      - inputs, weight rows and cache views live where their storage is;
//      - every other value needs a scratch buffer of its capacity class for
//        the span from the instruction that first writes it to the last one
//        that touches it. Spans are walked in program order and each takes
//        the lowest free buffer of its class, so values whose spans do not
//        meet share one buffer; the buffers an instruction writes are never
//        the ones it reads.
//      A misplaced value (no class and no binding, or more values of a class
//      live at one instruction than buffers were reserved) fails the whole
//      recording before the first launch.
//   2. issue. The instructions go to the pass's stream in order. Stream order
//      is the only ordering the device needs, so no hazards are tracked.
//
// Values live for their recording. A handle carries the recording's
// generation, so a handle kept past end() is refused when a later recording
// is given it. Buffers are reserved once, at prepare(); the value and
// instruction tables are sized there too, so a recording allocates nothing.
#pragma once

#include "DecoderShape.h"
#include "Net.h"

#include <cstdint>
#include <vector>

namespace WSP
{
// `count` scratch buffers of `elements` floats: one capacity class.
struct ScratchReservation
{
    int elements = 0;
    int count = 0;
};

struct HipNetLayout
{
    DecoderShape shape;
    std::vector<ScratchReservation> scratch;
    int valueCapacity = 4096;       // values one recording may hold
    int instructionCapacity = 2048; // instructions one recording may hold
};

class HipNet final : public Net
{
public:
    HipNet() = default;
    ~HipNet() override;

    HipNet(const HipNet&) = delete;
    HipNet& operator=(const HipNet&) = delete;

    void prepare(const Device& device, const HipNetLayout& layout, void* hipStream);

    void begin(Pass& pass);
    void end();

    Tensor input(const Binding& source, const Shape& shape, DType type) override;
    void output(const Tensor& value, const Binding& target) override;

    Tensor rows(const Weight& table, int first, int count) override;
    Tensor transpose(const Tensor& matrix) override;
    Tensor cached(const Cache& cache) override;

    Tensor conv1d(const Tensor& frames, const Weight& weight, const Weight& bias, int stride,
                  int padding, Activation activation) override;

    Tensor linear(const Tensor& input, const Weight& weight, const Weight* bias,
                  Activation activation) override;
    Tensor linearAdd(const Tensor& input, const Weight& weight, const Weight* bias,
                     const Tensor& stream) override;
    Tensor add(const Tensor& stream, const Tensor& addend) override;
    Tensor layerNorm(const Tensor& input, const Weight& weight, const Weight& bias) override;
    Tensor attention(const Tensor& queries, const Tensor& keys, const Tensor& values, int heads,
                     bool causal) override;
    Tensor embed(const Tensor& tokens, const Weight& tokenTable, const Weight& positionTable,
                 int firstPosition) override;
    Tensor appendLinear(Cache& cache, const Tensor& input, const Weight& weight,
                        const Weight* bias) override;

    Cache makeCache(int capacityRows, int width) override;

    // The storage of a cache, for the fused step, which reads and appends to
    // the caches directly.
    float* cacheData(const Cache& cache) const;

    // The C-ABI context every launch goes through.
    wsp_hip_ctx* context() const { return ctx; }

    // Scratch buffers the last placed recording used of each class, in the
    // order of the layout's reservations (a diagnostic for sizing layouts).
    const std::vector<int>& scratchHighWater() const { return highWater; }

protected:
    // Handles do not decide lifetimes here (a value lives for its recording),
    // so these only accept the handles of the open recording.
    void retain(int handle) override;
    void release(int handle) override;

private:
    // Where a value lives.
    enum class Home : std::uint8_t
    {
        fixed,   // storage given to the recording: an input, weight rows, a cache view
        scratch, // a buffer of its capacity class, chosen at placement
        bound    // a caller's binding, set by output()
    };

    struct Value
    {
        Home home = Home::fixed;
        BufferRange range;   // fixed and bound: the storage; scratch: set at placement
        Shape shape;
        int elements = 0;    // capacity, in floats
        int writer = -1;     // first instruction writing it; -1: written outside the recording
        int lastTouch = -1;  // last instruction reading or writing it
        int cls = -1;        // scratch: its capacity class (-1: none reserved)
        int buffer = -1;     // scratch: the buffer placement gave it
        int nextStarting = -1, nextEnding = -1; // placement's per-instruction lists
    };

    enum class Opcode : std::uint8_t
    {
        project,   // rows of in0 · weightᵀ (+ bias) (+ GELU), into dst at dstRow
        accumulate,// the same added into dst (in1 is dst)
        normalize, // LayerNorm of in0's rows
        attend,    // attention of queries in0 over keys in1 and values in2
        embedRows  // token rows of the table at in0's ids, plus position rows
    };

    struct Instruction
    {
        Opcode code = Opcode::project;
        int dst = -1;
        int in[3] = {-1, -1, -1};
        int dstRow = 0;            // project into a cache: the first row written
        const Weight* weight = nullptr;
        const Weight* bias = nullptr;
        const Weight* positions = nullptr;
        int heads = 0;
        int firstPosition = 0;
        bool gelu = false;
        bool causal = false;
    };

    struct ScratchClass
    {
        int elements = 0;
        int first = 0; // its first buffer's index in `held`
        std::vector<DeviceBuffer> buffers;
    };

    struct CacheBlock
    {
        DeviceBuffer buffer;
        int capacity = 0;
        int width = 0;
    };

    void requireRecording(const char* op) const;
    int newValue(Home home, const BufferRange& range, const Shape& shape, int elements);
    int valueOf(const Tensor& handle, const char* op) const;
    Tensor handleTo(int value);
    int scratchClassOf(int elements) const;
    int emit(const Instruction& instruction);
    void touch(int value, int instruction);

    void place();
    void issue(const Instruction& instruction);
    void check(int status) const;
    void closeRecording();

    Device device;
    wsp_hip_ctx* ctx = nullptr;
    int valueCapacity = 0;
    int instructionCapacity = 0;

    std::vector<ScratchClass> scratchClasses;
    std::vector<CacheBlock> caches;
    std::vector<int> highWater;

    // The open recording.
    Pass* pass = nullptr;
    std::uint32_t generation = 1;
    std::vector<Value> values;
    std::vector<Instruction> program;
    // Placement's work arrays, sized at prepare: per instruction the first
    // value whose span starts / ends there, and per buffer (classes in order)
    // whether a value holds it.
    std::vector<int> starting, ending;
    std::vector<char> held;
};
} // namespace WSP
