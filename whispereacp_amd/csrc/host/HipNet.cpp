// HipNet: Net on gfx950 as a recorded program (include/whispereacp/HipNet.h).
// Ops append instructions; end() places every value (bindings, fixed views,
// scratch buffers shared by liveness) and then issues the instructions in
// order, each one or two C-ABI calls on the context's stream.
#include "../../../include/whispereacp/HipNet.h"
#include "host_common.h"

#include <cmath>

#include <stdexcept>
#include <string>

namespace WSP
{
namespace
{
constexpr int kIndexBits = 16;
constexpr int kIndexMask = (1 << kIndexBits) - 1;
constexpr std::uint32_t kGenerationMask = 0x7FFF; // handles stay non-negative ints

std::size_t floatBytes(long long elements)
{
    return (std::size_t) elements * sizeof(float);
}

std::string floats(int elements)
{
    return std::to_string(elements) + " floats";
}
} // namespace

void throwForStatus(int status, const std::string& message)
{
    switch (status)
    {
        case WSP_OK: return;
        case WSP_ERR_LOGIC: throw std::logic_error(message);
        case WSP_ERR_HIP:
        case WSP_ERR_DEVICE: throw std::runtime_error(message);
        default: throw std::invalid_argument(message);
    }
}

HipNet::~HipNet()
{
    wsp_hip_ctx_destroy(ctx);
}

void HipNet::prepare(const Device& deviceToUse, const HipNetLayout& layout, void* hipStream)
{
    if (layout.valueCapacity <= 0 || layout.valueCapacity > kIndexMask + 1 || layout.instructionCapacity <= 0)
        throw std::invalid_argument("HipNet::prepare: the value and instruction tables need a size in [1, 65536]");
    device = deviceToUse;
    wsp_hip_ctx_destroy(ctx);
    ctx = nullptr;
    const wsp_decoder_shape shape = layout.shape.toC();
    const int status = wsp_hip_ctx_create(&shape, device.index, hipStream, &ctx);
    if (status != WSP_OK)
        throwForStatus(status, "HipNet::prepare: the kernel context could not be created");

    // Reservations of one capacity join one class, so a layout may list a
    // capacity twice.
    scratchClasses.clear();
    int total = 0;
    for (const auto& reservation : layout.scratch)
    {
        int c = scratchClassOf(reservation.elements);
        if (c < 0)
        {
            scratchClasses.push_back(ScratchClass {reservation.elements, 0, {}});
            c = (int) scratchClasses.size() - 1;
        }
        for (int i = 0; i < reservation.count; ++i)
            scratchClasses[(std::size_t) c].buffers.emplace_back(device, floatBytes(reservation.elements));
        total += reservation.count;
    }
    for (std::size_t c = 0, first = 0; c < scratchClasses.size(); ++c)
    {
        scratchClasses[c].first = (int) first;
        first += scratchClasses[c].buffers.size();
    }
    highWater.assign(scratchClasses.size(), 0);
    held.assign((std::size_t) total, 0);

    caches.clear();
    valueCapacity = layout.valueCapacity;
    instructionCapacity = layout.instructionCapacity;
    values.clear();
    values.reserve((std::size_t) valueCapacity);
    program.clear();
    program.reserve((std::size_t) instructionCapacity);
    starting.assign((std::size_t) instructionCapacity, -1);
    ending.assign((std::size_t) instructionCapacity, -1);
    pass = nullptr;
    ++generation;
}

void HipNet::check(int status) const
{
    if (status != WSP_OK)
        throwForStatus(status, wsp_hip_last_error(ctx));
}

Cache HipNet::makeCache(int capacityRows, int width)
{
    if (ctx == nullptr)
        throw std::logic_error("HipNet::makeCache: the net is not prepared yet, so it has no device to hold a cache");
    caches.push_back(CacheBlock {DeviceBuffer(device, floatBytes((long long) capacityRows * width)), capacityRows,
                                 width});
    return {(int) caches.size() - 1, 0};
}

float* HipNet::cacheData(const Cache& cache) const
{
    return static_cast<float*>(caches.at((std::size_t) cache.id).buffer.data());
}

// ---------------------------------------------------------------------------
// Recording
// ---------------------------------------------------------------------------
void HipNet::begin(Pass& passToUse)
{
    if (ctx == nullptr)
        throw std::logic_error("HipNet::begin: the net is not prepared yet");
    if (pass != nullptr)
        throw std::logic_error("HipNet::begin: a recording is already open; end() it first");
    if (passToUse.hipStream() != wsp_hip_stream(ctx))
        throw std::logic_error("HipNet::begin: the pass wraps another stream than the one the net was prepared with");
    pass = &passToUse;
    values.clear();
    program.clear();
}

void HipNet::requireRecording(const char* op) const
{
    if (pass == nullptr)
        throw std::logic_error(std::string("HipNet::") + op + ": no recording is open (ops go between begin() and end())");
}

void HipNet::closeRecording()
{
    pass = nullptr;
    values.clear();
    program.clear();
    generation = (generation + 1) & kGenerationMask;
    if (generation == 0)
        generation = 1;
}

int HipNet::scratchClassOf(int elements) const
{
    for (std::size_t c = 0; c < scratchClasses.size(); ++c)
        if (scratchClasses[c].elements == elements)
            return (int) c;
    return -1;
}

int HipNet::newValue(Home home, const BufferRange& range, const Shape& shape, int elements)
{
    if ((int) values.size() >= valueCapacity)
        throw std::logic_error("HipNet: this recording already holds " + std::to_string(valueCapacity)
                               + " values, the most the net was prepared for");
    Value v;
    v.home = home;
    v.range = range;
    v.shape = shape;
    v.elements = elements;
    if (home == Home::scratch)
        v.cls = scratchClassOf(elements);
    values.push_back(v);
    return (int) values.size() - 1;
}

Tensor HipNet::handleTo(int value)
{
    return {*this, (int) ((generation & kGenerationMask) << kIndexBits) | value};
}

int HipNet::valueOf(const Tensor& handle, const char* op) const
{
    requireRecording(op);
    if (!handle.isValid() || !handle.isOwnedBy(*this))
        throw std::logic_error(std::string("HipNet::") + op + ": the tensor is not a value of this net");
    const int id = handle.index();
    const int index = id & kIndexMask;
    if ((std::uint32_t) (id >> kIndexBits) != (generation & kGenerationMask) || index >= (int) values.size())
        throw std::logic_error(std::string("HipNet::") + op
                               + ": the tensor belongs to a recording that has ended; values live for one recording");
    return index;
}

void HipNet::retain(int) {}

void HipNet::release(int) {}

void HipNet::touch(int value, int instruction)
{
    Value& v = values[(std::size_t) value];
    if (v.writer < 0 && v.home == Home::scratch)
        v.writer = instruction;
    if (instruction > v.lastTouch)
        v.lastTouch = instruction;
}

int HipNet::emit(const Instruction& instruction)
{
    if ((int) program.size() >= instructionCapacity)
        throw std::logic_error("HipNet: this recording already holds " + std::to_string(instructionCapacity)
                               + " instructions, the most the net was prepared for");
    const int at = (int) program.size();
    program.push_back(instruction);
    // The written value first: its span starts here even when it is also read.
    touch(instruction.dst, at);
    for (int source : instruction.in)
        if (source >= 0)
            touch(source, at);
    return at;
}

Tensor HipNet::input(const Binding& source, const Shape& shape, DType)
{
    requireRecording("input");
    const Shape capacity = source.capacity.rank() == 0 ? shape : source.capacity;
    return handleTo(newValue(Home::fixed, source.range, shape, capacity.elementCount()));
}

Tensor HipNet::rows(const Weight& table, int first, int count)
{
    requireRecording("rows");
    const int width = table.dimension(1);
    const std::size_t skip = floatBytes((long long) first * width);
    const BufferRange range {const_cast<void*>(table.data()), skip, table.storage->size() - table.byteOffset - skip};
    return handleTo(newValue(Home::fixed, range, Shape {count, width}, count * width));
}

Tensor HipNet::cached(const Cache& cache)
{
    requireRecording("cached");
    const CacheBlock& block = caches.at((std::size_t) cache.id);
    return handleTo(newValue(Home::fixed, BufferRange::of(block.buffer), Shape {cache.rows, block.width},
                             block.capacity * block.width));
}

Tensor HipNet::transpose(const Tensor&)
{
    throw std::logic_error("HipNet::transpose: an encoder op; this backend runs the decoder");
}

Tensor HipNet::conv1d(const Tensor&, const Weight&, const Weight&, int, int, Activation)
{
    throw std::logic_error("HipNet::conv1d: an encoder op; this backend runs the decoder");
}

Tensor HipNet::add(const Tensor&, const Tensor&)
{
    throw std::logic_error("HipNet::add: an encoder op; the decoder's residuals go through linearAdd");
}

Tensor HipNet::linear(const Tensor& input, const Weight& weight, const Weight* bias, Activation activation)
{
    const int source = valueOf(input, "linear");
    const Value& in = values[(std::size_t) source];
    const int outputs = weight.dimension(0);
    const int capacityRows = in.elements / in.shape.columns();
    const int dst = newValue(Home::scratch, {}, Shape {in.shape.rows(), outputs}, capacityRows * outputs);
    Instruction op;
    op.code = Opcode::project;
    op.dst = dst;
    op.in[0] = source;
    op.weight = &weight;
    op.bias = bias;
    op.gelu = activation == Activation::gelu;
    emit(op);
    return handleTo(dst);
}

Tensor HipNet::linearAdd(const Tensor& input, const Weight& weight, const Weight* bias, const Tensor& stream)
{
    const int source = valueOf(input, "linearAdd");
    const int into = valueOf(stream, "linearAdd");
    Instruction op;
    op.code = Opcode::accumulate;
    op.dst = into;
    op.in[0] = source;
    op.in[1] = into;
    op.weight = &weight;
    op.bias = bias;
    emit(op);
    return handleTo(into);
}

Tensor HipNet::layerNorm(const Tensor& input, const Weight& weight, const Weight& bias)
{
    const int source = valueOf(input, "layerNorm");
    const Value& in = values[(std::size_t) source];
    const int dst = newValue(Home::scratch, {}, in.shape, in.elements);
    Instruction op;
    op.code = Opcode::normalize;
    op.dst = dst;
    op.in[0] = source;
    op.weight = &weight;
    op.bias = &bias;
    emit(op);
    return handleTo(dst);
}

Tensor HipNet::attention(const Tensor& queries, const Tensor& keys, const Tensor& values_, int heads, bool causal)
{
    const int q = valueOf(queries, "attention");
    const int k = valueOf(keys, "attention");
    const int v = valueOf(values_, "attention");
    const Value& in = values[(std::size_t) q];
    const int dst = newValue(Home::scratch, {}, in.shape, in.elements);
    Instruction op;
    op.code = Opcode::attend;
    op.dst = dst;
    op.in[0] = q;
    op.in[1] = k;
    op.in[2] = v;
    op.heads = heads;
    op.causal = causal;
    emit(op);
    return handleTo(dst);
}

Tensor HipNet::embed(const Tensor& tokens, const Weight& tokenTable, const Weight& positionTable, int firstPosition)
{
    const int ids = valueOf(tokens, "embed");
    const Value& in = values[(std::size_t) ids];
    const int width = tokenTable.dimension(1);
    const int dst = newValue(Home::scratch, {}, Shape {in.shape[0], width}, in.elements * width);
    Instruction op;
    op.code = Opcode::embedRows;
    op.dst = dst;
    op.in[0] = ids;
    op.weight = &tokenTable;
    op.positions = &positionTable;
    op.firstPosition = firstPosition;
    emit(op);
    return handleTo(dst);
}

// The projection lands in the rows the cache holds next (Net/KernelNet.cpp
// :724-758 gives appendLinear that meaning); the value returned is the whole
// cache as it stands after them.
Tensor HipNet::appendLinear(Cache& cache, const Tensor& input, const Weight& weight, const Weight* bias)
{
    const int source = valueOf(input, "appendLinear");
    const CacheBlock& block = caches.at((std::size_t) cache.id);
    const int count = values[(std::size_t) source].shape.rows();
    if (cache.rows + count > block.capacity)
        throw std::logic_error("HipNet::appendLinear: " + std::to_string(count) + " more rows would overflow a cache of "
                               + std::to_string(block.capacity) + " rows holding " + std::to_string(cache.rows));
    const int dst = newValue(Home::fixed, BufferRange::of(block.buffer), Shape {cache.rows + count, block.width},
                             block.capacity * block.width);
    Instruction op;
    op.code = Opcode::project;
    op.dst = dst;
    op.dstRow = cache.rows;
    op.in[0] = source;
    op.weight = &weight;
    op.bias = bias;
    emit(op);
    cache.rows += count;
    return handleTo(dst);
}

void HipNet::output(const Tensor& handle, const Binding& target)
{
    const int index = valueOf(handle, "output");
    Value& v = values[(std::size_t) index];
    switch (v.home)
    {
        case Home::scratch:
            if (target.range.size != 0 && target.range.size < floatBytes((long long) v.shape.elementCount()))
                throw std::logic_error("HipNet::output: the binding '" + target.name + "' holds "
                                       + std::to_string(target.range.size) + " bytes, less than the value's "
                                       + std::to_string(floatBytes((long long) v.shape.elementCount())));
            v.home = Home::bound;
            v.range = target.range;
            return;
        case Home::bound:
        case Home::fixed:
            if (v.range.sameStart(target.range))
                return; // already there
            throw std::logic_error(v.home == Home::bound
                                       ? "HipNet::output: the value is already bound to other storage"
                                       : "HipNet::output: the value is a view of storage the recording was given; "
                                         "output() binds values the recording computes");
    }
}

// ---------------------------------------------------------------------------
// end(): placement, then issue
// ---------------------------------------------------------------------------
void HipNet::end()
{
    requireRecording("end");
    try
    {
        place();
        for (const Instruction& instruction : program)
            issue(instruction);
    }
    catch (...)
    {
        closeRecording();
        throw;
    }
    closeRecording();
}

// Walks the program once. At instruction i, first every scratch value whose
// span starts at i takes the lowest free buffer of its class, then every one
// whose span ends at i gives its buffer back: an instruction never writes a
// buffer it reads, and a buffer returns to use at the first instruction after
// its value's last touch. The spans are threaded into per-instruction lists
// through the values themselves, so nothing is allocated.
void HipNet::place()
{
    const int instructions = (int) program.size();
    std::fill(starting.begin(), starting.begin() + instructions, -1);
    std::fill(ending.begin(), ending.begin() + instructions, -1);
    for (int n = (int) values.size() - 1; n >= 0; --n)
    {
        Value& v = values[(std::size_t) n];
        if (v.home != Home::scratch)
            continue;
        if (v.cls < 0)
            throw std::logic_error("HipNet: instruction " + std::to_string(v.writer) + " writes a value of "
                                   + floats(v.elements)
                                   + " capacity; no scratch buffers of that capacity were reserved and output() "
                                     "did not bind it");
        v.nextStarting = starting[(std::size_t) v.writer];
        starting[(std::size_t) v.writer] = n;
        v.nextEnding = ending[(std::size_t) v.lastTouch];
        ending[(std::size_t) v.lastTouch] = n;
    }

    std::fill(held.begin(), held.end(), 0);
    std::fill(highWater.begin(), highWater.end(), 0);
    for (int i = 0; i < instructions; ++i)
    {
        for (int n = starting[(std::size_t) i]; n >= 0; n = values[(std::size_t) n].nextStarting)
        {
            Value& v = values[(std::size_t) n];
            ScratchClass& cls = scratchClasses[(std::size_t) v.cls];
            const int count = (int) cls.buffers.size();
            int b = 0;
            while (b < count && held[(std::size_t) (cls.first + b)])
                ++b;
            if (b == count)
                throw std::logic_error("HipNet: at instruction " + std::to_string(i) + " more values of "
                                       + floats(cls.elements) + " capacity are live than the "
                                       + std::to_string(count) + " scratch buffers reserved for it");
            held[(std::size_t) (cls.first + b)] = 1;
            v.buffer = b;
            v.range = BufferRange::of(cls.buffers[(std::size_t) b]);
            if (b + 1 > highWater[(std::size_t) v.cls])
                highWater[(std::size_t) v.cls] = b + 1;
        }
        for (int n = ending[(std::size_t) i]; n >= 0; n = values[(std::size_t) n].nextEnding)
        {
            const Value& v = values[(std::size_t) n];
            held[(std::size_t) (scratchClasses[(std::size_t) v.cls].first + v.buffer)] = 0;
        }
    }
}

void HipNet::issue(const Instruction& op)
{
    auto at = [&](int value) { return values[(std::size_t) value].range.data(); };
    const Value& dst = values[(std::size_t) op.dst];
    switch (op.code)
    {
        case Opcode::project:
        case Opcode::accumulate:
        {
            const Value& in = values[(std::size_t) op.in[0]];
            const int outputs = op.weight->dimension(0);
            int flags = op.gelu ? WSP_LINEAR_GELU : 0;
            if (op.code == Opcode::accumulate)
                flags |= WSP_LINEAR_RESIDUAL;
            float* target = static_cast<float*>(at(op.dst)) + (std::size_t) op.dstRow * (std::size_t) outputs;
            const float* bias = op.bias != nullptr ? static_cast<const float*>(op.bias->data()) : nullptr;
            check(wsp_hip_linear(ctx, static_cast<const float*>(at(op.in[0])), in.shape.rows(), in.shape.columns(),
                                 op.weight->data(), wsp_dtype_of(op.weight->type), bias, target, outputs, flags));
            return;
        }
        case Opcode::normalize:
        {
            const Value& in = values[(std::size_t) op.in[0]];
            check(wsp_hip_layernorm(ctx, static_cast<const float*>(at(op.in[0])),
                                    static_cast<const float*>(op.weight->data()),
                                    static_cast<const float*>(op.bias->data()), static_cast<float*>(at(op.dst)),
                                    in.shape.rows(), in.shape.columns(), 1e-5f));
            return;
        }
        case Opcode::attend:
        {
            const Value& q = values[(std::size_t) op.in[0]];
            const Value& k = values[(std::size_t) op.in[1]];
            const int width = q.shape.columns();
            const float scale = 1.f / std::sqrt((float) (width / op.heads));
            check(wsp_hip_attention(ctx, static_cast<const float*>(at(op.in[0])), q.shape.rows(),
                                    static_cast<const float*>(at(op.in[1])), static_cast<const float*>(at(op.in[2])),
                                    k.shape.rows(), width, op.heads, op.causal ? 1 : 0, scale,
                                    static_cast<float*>(at(op.dst))));
            return;
        }
        case Opcode::embedRows:
        {
            const Value& ids = values[(std::size_t) op.in[0]];
            check(wsp_hip_embed(ctx, static_cast<const uint32_t*>(at(op.in[0])), ids.shape[0],
                                static_cast<const float*>(op.weight->data()),
                                static_cast<const float*>(op.positions->data()), op.firstPosition,
                                static_cast<float*>(at(op.dst)), dst.shape.columns()));
            return;
        }
    }
}
} // namespace WSP
