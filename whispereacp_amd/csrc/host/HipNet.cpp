// HipNet: the decoder profile of Net on gfx950 (include/whispereacp/HipNet.h).
// The value bookkeeping follows Net/KernelNet.cpp:220-513; each op is one or
// two C-ABI calls on the context's stream.
#include "../../../include/whispereacp/HipNet.h"
#include "host_common.h"

#include <cmath>

#include <stdexcept>
#include <string>

namespace WSP
{
namespace
{
std::size_t floatBytes(int elements)
{
    return (std::size_t) elements * sizeof(float);
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

void HipNet::prepare(const Device& deviceToUse, const HipNetLayout& layoutToUse, void* hipStream)
{
    layout = layoutToUse;
    device = deviceToUse;
    wsp_hip_ctx_destroy(ctx);
    ctx = nullptr;
    const wsp_decoder_shape shape = layout.shape.toC();
    const int status = wsp_hip_ctx_create(&shape, device.index, hipStream, &ctx);
    if (status != WSP_OK)
        throwForStatus(status, "HipNet::prepare: the kernel context could not be created");

    records.assign(maxRecords, Record {});
    slots.clear();
    for (const auto& reservation : layout.scratch)
        for (int i = 0; i < reservation.count; ++i)
            slots.push_back(ScratchSlot {DeviceBuffer(device, floatBytes(reservation.elements)),
                                         reservation.elements, -1});
    caches.clear();
    pending = {};
}

void HipNet::check(int status) const
{
    if (status != WSP_OK)
        throwForStatus(status, wsp_hip_last_error(ctx));
}

Cache HipNet::makeCache(int capacityRows, int width)
{
    if (ctx == nullptr)
        throw std::logic_error("a net makes a cache once it is prepared");
    caches.push_back(CacheStorage {DeviceBuffer(device, floatBytes(capacityRows * width)), capacityRows, width});
    return {(int) caches.size() - 1, 0};
}

float* HipNet::cacheData(const Cache& cache) const
{
    return static_cast<float*>(caches.at((std::size_t) cache.id).buffer.data());
}

void HipNet::begin(Pass& pass)
{
    if (ctx == nullptr)
        throw std::logic_error("a net records once it is prepared");
    if (pass.hipStream() != wsp_hip_stream(ctx))
        throw std::logic_error("a net records into the stream it was prepared with");
    recordingPass = &pass;
    pending = {};
}

void HipNet::end()
{
    flush();
    recordingPass = nullptr;
    for (const auto& slot : slots)
        if (slot.holder >= 0)
            throw std::logic_error("a value outlived the recording that made it");
}

void HipNet::retain(int index)
{
    ++records[(std::size_t) index].references;
}

void HipNet::release(int index)
{
    auto& record = records[(std::size_t) index];
    if (--record.references > 0)
        return;
    record.live = false;
    if (record.slot >= 0)
    {
        slots[(std::size_t) record.slot].holder = -1;
        record.slot = -1;
    }
    if (record.base >= 0)
    {
        const int base = record.base;
        record.base = -1;
        release(base);
    }
}

int HipNet::makeRecord()
{
    flush();
    for (std::size_t i = 0; i < records.size(); ++i)
        if (!records[i].live)
        {
            records[i] = Record {};
            records[i].live = true;
            return (int) i;
        }
    throw std::logic_error("a net recording holds more values at once than it has records for");
}

HipNet::Record& HipNet::recordOf(const Tensor& value)
{
    if (!value.isValid() || !value.isOwnedBy(*this))
        throw std::logic_error("an op was given a tensor that holds no value of this net");
    return records[(std::size_t) value.index()];
}

Tensor HipNet::view(const Record& source)
{
    const int index = makeRecord();
    records[(std::size_t) index] = source;
    records[(std::size_t) index].live = true;
    records[(std::size_t) index].references = 0;
    return {*this, index};
}

int HipNet::takeSlot(int elements)
{
    flush();
    bool reserved = false;
    for (std::size_t i = 0; i < slots.size(); ++i)
    {
        if (slots[i].elements != elements)
            continue;
        reserved = true;
        if (slots[i].holder < 0)
            return (int) i;
    }
    if (reserved)
        throw std::logic_error("every scratch buffer of " + std::to_string(elements)
                               + " elements is holding a value");
    return -1;
}

Tensor HipNet::fresh(const Shape& shape, const Shape& capacity)
{
    const int slot = takeSlot(capacity.elementCount());
    Record record;
    record.shape = shape;
    record.capacity = capacity;
    record.slot = slot;
    if (slot >= 0)
        record.storage = BufferRange::of(slots[(std::size_t) slot].buffer);
    Tensor value = view(record);
    if (slot >= 0)
        slots[(std::size_t) slot].holder = value.index();
    return value;
}

bool HipNet::makesNewValue(OpKind kind)
{
    return kind == OpKind::linear || kind == OpKind::layerNorm || kind == OpKind::attention
           || kind == OpKind::embed;
}

void HipNet::flush()
{
    if (pending.kind == OpKind::none)
        return;
    const PendingOp op = pending;
    pending = {};
    if (makesNewValue(op.kind) && !records[(std::size_t) op.result].storage.isValid())
        throw std::logic_error("a value with no scratch buffer of its capacity has to be placed by output()");
    run(op);
}

void HipNet::run(const PendingOp& op)
{
    if (recordingPass == nullptr)
        throw std::logic_error("a net records between begin() and end()");
    switch (op.kind)
    {
        case OpKind::linear:
        case OpKind::linearAdd:
        case OpKind::append: runProjection(op); break;
        case OpKind::add: runAdd(op); break;
        case OpKind::layerNorm: runLayerNorm(op); break;
        case OpKind::attention: runAttention(op); break;
        case OpKind::embed: runEmbed(op); break;
        case OpKind::none: break;
    }
}

Tensor HipNet::input(const Binding& source, const Shape& shape, DType)
{
    flush();
    Record record;
    record.storage = source.range;
    record.shape = shape;
    record.capacity = source.capacity.rank() == 0 ? shape : source.capacity;
    return view(record);
}

void HipNet::output(const Tensor& value, const Binding& target)
{
    auto& record = recordOf(value);
    const bool madeByPending = pending.result == value.index() && makesNewValue(pending.kind);
    if (madeByPending)
    {
        if (record.slot >= 0)
            slots[(std::size_t) record.slot].holder = -1;
        record.slot = -1;
        record.storage = target.range;
        flush();
        return;
    }
    if (!record.storage.sameStart(target.range))
        throw std::logic_error("the backend places an output by pointing the op just before it at the target");
    flush();
}

Tensor HipNet::rows(const Weight& table, int first, int count)
{
    flush();
    const int width = table.dimension(1);
    Record record;
    record.storage = {const_cast<void*>(table.data()), floatBytes(first * width),
                      table.storage->size() - table.byteOffset - floatBytes(first * width)};
    record.shape = {count, width};
    record.capacity = record.shape;
    return view(record);
}

Tensor HipNet::transpose(const Tensor&)
{
    throw std::logic_error("transpose is an encoder op; the decoder backend does not run it");
}

Tensor HipNet::conv1d(const Tensor&, const Weight&, const Weight&, int, int, Activation)
{
    throw std::logic_error("conv1d is an encoder op; the decoder backend does not run it");
}

Tensor HipNet::add(const Tensor&, const Tensor&)
{
    throw std::logic_error("add is an encoder op; the decoder folds its residuals into linearAdd");
}

Tensor HipNet::cached(const Cache& cache)
{
    flush();
    const auto& storage = caches.at((std::size_t) cache.id);
    Record record;
    record.storage = BufferRange::of(storage.buffer);
    record.shape = {cache.rows, storage.width};
    record.capacity = {storage.capacity, storage.width};
    return view(record);
}

Tensor HipNet::linear(const Tensor& input, const Weight& weight, const Weight* bias, Activation activation)
{
    flush();
    const auto source = recordOf(input);
    const int outputs = weight.dimension(0);
    Tensor result = fresh({source.shape.rows(), outputs}, {source.capacity.rows(), outputs});
    PendingOp op;
    op.kind = OpKind::linear;
    op.result = result.index();
    op.first = input.index();
    op.weight = &weight;
    op.bias = bias;
    op.activation = activation;
    pending = op;
    return result;
}

Tensor HipNet::linearAdd(const Tensor& input, const Weight& weight, const Weight* bias, const Tensor& stream)
{
    flush();
    PendingOp op;
    op.kind = OpKind::linearAdd;
    op.result = stream.index();
    op.first = input.index();
    op.weight = &weight;
    op.bias = bias;
    pending = op;
    return stream;
}

Tensor HipNet::layerNorm(const Tensor& input, const Weight& weight, const Weight& bias)
{
    flush();
    const auto source = recordOf(input);
    Tensor result = fresh(source.shape, source.capacity);
    PendingOp op;
    op.kind = OpKind::layerNorm;
    op.result = result.index();
    op.first = input.index();
    op.weight = &weight;
    op.bias = &bias;
    pending = op;
    return result;
}

Tensor HipNet::attention(const Tensor& queries, const Tensor& keys, const Tensor& values, int heads, bool causal)
{
    flush();
    const auto source = recordOf(queries);
    Tensor result = fresh(source.shape, source.capacity);
    PendingOp op;
    op.kind = OpKind::attention;
    op.result = result.index();
    op.first = queries.index();
    op.second = keys.index();
    op.third = values.index();
    op.heads = heads;
    op.causal = causal;
    pending = op;
    return result;
}

Tensor HipNet::embed(const Tensor& tokens, const Weight& tokenTable, const Weight& positionTable, int firstPosition)
{
    flush();
    const auto source = recordOf(tokens);
    const int width = tokenTable.dimension(1);
    Tensor result = fresh({source.shape[0], width}, {source.capacity[0], width});
    PendingOp op;
    op.kind = OpKind::embed;
    op.result = result.index();
    op.first = tokens.index();
    op.weight = &tokenTable;
    op.positionTable = &positionTable;
    op.position = firstPosition;
    pending = op;
    return result;
}

// Net/KernelNet.cpp:724-758: the projection writes straight into the rows the
// cache holds next.
Tensor HipNet::appendLinear(Cache& cache, const Tensor& input, const Weight& weight, const Weight* bias)
{
    flush();
    const auto& storage = caches.at((std::size_t) cache.id);
    const int width = storage.width;
    const int count = recordOf(input).shape.rows();
    if (cache.rows + count > storage.capacity)
        throw std::logic_error("a cache was appended to past its capacity");
    PendingOp op;
    op.kind = OpKind::append;
    op.first = input.index();
    op.weight = &weight;
    op.bias = bias;
    op.target = {storage.buffer.data(), floatBytes(cache.rows * width), floatBytes(count * width)};
    cache.rows += count;
    Tensor result = cached(cache);
    op.result = result.index();
    pending = op;
    return result;
}

void HipNet::runProjection(const PendingOp& op)
{
    const auto& input = records[(std::size_t) op.first];
    const BufferRange target = op.kind == OpKind::append ? op.target : records[(std::size_t) op.result].storage;
    int flags = 0;
    if (op.activation == Activation::gelu)
        flags |= WSP_LINEAR_GELU;
    if (op.kind == OpKind::linearAdd)
        flags |= WSP_LINEAR_RESIDUAL;
    const float* bias = op.bias != nullptr ? static_cast<const float*>(op.bias->data()) : nullptr;
    check(wsp_hip_linear(ctx, static_cast<const float*>(input.storage.data()), input.shape.rows(),
                         input.shape.columns(), op.weight->data(), wsp_dtype_of(op.weight->type), bias,
                         static_cast<float*>(target.data()), op.weight->dimension(0), flags));
}

void HipNet::runAdd(const PendingOp&)
{
    throw std::logic_error("add is an encoder op");
}

void HipNet::runLayerNorm(const PendingOp& op)
{
    const auto& input = records[(std::size_t) op.first];
    const auto& output = records[(std::size_t) op.result];
    check(wsp_hip_layernorm(ctx, static_cast<const float*>(input.storage.data()),
                            static_cast<const float*>(op.weight->data()),
                            static_cast<const float*>(op.bias->data()), static_cast<float*>(output.storage.data()),
                            input.shape.rows(), input.shape.columns(), 1e-5f));
}

void HipNet::runAttention(const PendingOp& op)
{
    const auto& queries = records[(std::size_t) op.first];
    const auto& keys = records[(std::size_t) op.second];
    const auto& values = records[(std::size_t) op.third];
    const auto& output = records[(std::size_t) op.result];
    const int width = queries.shape.columns();
    const float scale = 1.f / std::sqrt((float) (width / op.heads));
    check(wsp_hip_attention(ctx, static_cast<const float*>(queries.storage.data()), queries.shape.rows(),
                            static_cast<const float*>(keys.storage.data()),
                            static_cast<const float*>(values.storage.data()), keys.shape.rows(), width, op.heads,
                            op.causal ? 1 : 0, scale, static_cast<float*>(output.storage.data())));
}

void HipNet::runEmbed(const PendingOp& op)
{
    const auto& tokens = records[(std::size_t) op.first];
    const auto& output = records[(std::size_t) op.result];
    check(wsp_hip_embed(ctx, static_cast<const uint32_t*>(tokens.storage.data()), tokens.shape[0],
                        static_cast<const float*>(op.weight->data()),
                        static_cast<const float*>(op.positionTable->data()), op.position,
                        static_cast<float*>(output.storage.data()), output.shape.columns()));
}
} // namespace WSP
