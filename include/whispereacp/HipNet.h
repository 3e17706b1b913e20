// The gfx950 backend of Net — the decoder profile of the reference's KernelNet
// (Net/KernelNet.h:63-306) over the C ABI in wsp_hip.h.
//
// A value lives in a scratch buffer of the capacity it could reach, taken
// from those reserved at prepare(), and goes back when its last Tensor does.
// An op is dispatched when the next op is called, or at end(), so output()
// can still point the op that made a value at the caller's buffer
// (Net/KernelNet.cpp:487-513). Work is ordered by the stream the pass wraps,
// so no barriers are derived. Nothing is allocated after prepare().
#pragma once

#include "DecoderShape.h"
#include "Net.h"

#include <vector>

namespace WSP
{
struct ScratchReservation
{
    int elements = 0;
    int count = 0;
};

struct HipNetLayout
{
    DecoderShape shape;
    std::vector<ScratchReservation> scratch;
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

    // The C-ABI context every dispatch goes through.
    wsp_hip_ctx* context() const { return ctx; }

protected:
    void retain(int index) override;
    void release(int index) override;

private:
    struct Record
    {
        BufferRange storage;
        Shape shape;
        Shape capacity;
        int slot = -1;
        int base = -1;
        int references = 0;
        bool live = false;
    };

    enum class OpKind
    {
        none,
        linear,
        linearAdd,
        add,
        layerNorm,
        attention,
        embed,
        append
    };

    struct PendingOp
    {
        OpKind kind = OpKind::none;
        int result = -1;
        int first = -1;
        int second = -1;
        int third = -1;
        const Weight* weight = nullptr;
        const Weight* bias = nullptr;
        const Weight* positionTable = nullptr;
        int heads = 0;
        int position = 0;
        Activation activation = Activation::none;
        bool causal = false;
        BufferRange target;
    };

    struct ScratchSlot
    {
        DeviceBuffer buffer;
        int elements = 0;
        int holder = -1;
    };

    struct CacheStorage
    {
        DeviceBuffer buffer;
        int capacity = 0;
        int width = 0;
    };

    static constexpr int maxRecords = 64;

    int makeRecord();
    Tensor view(const Record& source);
    Tensor fresh(const Shape& shape, const Shape& capacity);
    int takeSlot(int elements);
    Record& recordOf(const Tensor& value);

    void flush();
    void run(const PendingOp& op);
    static bool makesNewValue(OpKind kind);
    void check(int status) const;

    void runProjection(const PendingOp& op);
    void runAdd(const PendingOp& op);
    void runLayerNorm(const PendingOp& op);
    void runAttention(const PendingOp& op);
    void runEmbed(const PendingOp& op);

    HipNetLayout layout;
    Device device;
    wsp_hip_ctx* ctx = nullptr;
    Pass* recordingPass = nullptr;

    std::vector<Record> records;
    PendingOp pending;
    std::vector<ScratchSlot> slots;
    std::vector<CacheStorage> caches;
};
} // namespace WSP
