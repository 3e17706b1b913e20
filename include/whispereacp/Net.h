// Net/Net.h:1-171 — the backend-neutral op list the decoder body is written
// against, with eacp's buffer types replaced by the HIP ones in Gpu.h. The
// decoder body (Decoder.cpp) calls these; HipNet runs them on gfx950.
#pragma once

#include "Gpu.h"

#include <array>
#include <initializer_list>
#include <memory>
#include <string>
#include <vector>

namespace WSP
{
enum class Activation
{
    none,
    gelu
};

enum class DType
{
    float32,
    float16,
    int32
};

// How a tensor is stored on the device (Model/TensorType.h). Projection
// weights may stay packed; everything else is widened to float.
enum class WeightStorage
{
    Float,
    PackedHalf,
    PackedBFloat16
};

int wsp_dtype_of(WeightStorage storage);

// A weight on the device (Model/TensorLoader.h TensorBuffer): a byte range of
// a shared allocation, its extents and its storage. Several tensors may view
// one allocation (the fused q/k/v block).
struct TensorBuffer
{
    std::shared_ptr<DeviceBuffer> storage;
    std::size_t byteOffset = 0;
    std::vector<int> extents;
    WeightStorage type = WeightStorage::Float;

    const void* data() const
    {
        return static_cast<const char*>(storage->data()) + byteOffset;
    }
    int dimension(int axis) const { return extents[(std::size_t) axis]; }
    bool isPackedHalf() const { return type != WeightStorage::Float; }
    std::size_t elementCount() const;
};

using Weight = TensorBuffer;

class Shape
{
public:
    static constexpr auto maxRank = 4;

    Shape() = default;
    Shape(std::initializer_list<int> extentsToUse);

    int rank() const { return count; }
    int operator[](int axis) const { return extents[(std::size_t) axis]; }

    int rows() const;
    int columns() const;
    int elementCount() const;

    friend bool operator==(const Shape&, const Shape&) = default;

private:
    std::array<int, maxRank> extents {};
    int count = 0;
};

// Storage outside the net (Net/Net.h:64-69).
struct Binding
{
    BufferRange range;
    Shape capacity;
    std::string name;
};

// Rows a sequence keeps between recordings (Net/Net.h:73-79).
struct Cache
{
    int id = -1;
    int rows = 0;

    void clear() { rows = 0; }
};

class Net;

// A value inside one recording; copies share it (Net/Net.h:86-108).
class Tensor
{
public:
    Tensor() = default;
    Tensor(Net& ownerToUse, int indexToUse);

    Tensor(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(const Tensor& other);
    Tensor& operator=(Tensor&& other) noexcept;
    ~Tensor();

    bool isValid() const { return owner != nullptr; }
    bool isOwnedBy(const Net& net) const { return owner == &net; }
    int index() const { return id; }

private:
    void retain() const;
    void release() const;

    Net* owner = nullptr;
    int id = -1;
};

class Net
{
public:
    virtual ~Net() = default;

    virtual Tensor input(const Binding& source, const Shape& shape, DType type) = 0;
    virtual void output(const Tensor& value, const Binding& target) = 0;

    virtual Tensor rows(const Weight& table, int first, int count) = 0;
    virtual Tensor transpose(const Tensor& matrix) = 0;
    virtual Tensor cached(const Cache& cache) = 0;

    virtual Tensor conv1d(const Tensor& frames, const Weight& weight, const Weight& bias, int stride,
                          int padding, Activation activation) = 0;

    virtual Tensor linear(const Tensor& input, const Weight& weight, const Weight* bias,
                          Activation activation) = 0;

    // The projection of input added into stream, which is consumed.
    virtual Tensor linearAdd(const Tensor& input, const Weight& weight, const Weight* bias,
                             const Tensor& stream) = 0;

    virtual Tensor add(const Tensor& stream, const Tensor& addend) = 0;

    virtual Tensor layerNorm(const Tensor& input, const Weight& weight, const Weight& bias) = 0;

    virtual Tensor attention(const Tensor& queries, const Tensor& keys, const Tensor& values, int heads,
                             bool causal) = 0;

    virtual Tensor embed(const Tensor& tokens, const Weight& tokenTable, const Weight& positionTable,
                         int firstPosition) = 0;

    // A projection written into the rows the cache holds next.
    virtual Tensor appendLinear(Cache& cache, const Tensor& input, const Weight& weight,
                                const Weight* bias) = 0;

    virtual Cache makeCache(int capacityRows, int width) = 0;

protected:
    friend class Tensor;

    virtual void retain(int index) = 0;
    virtual void release(int index) = 0;
};
} // namespace WSP
