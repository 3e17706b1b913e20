// Shape, Tensor reference counting and the small value types of Net
// (Net/Net.cpp), plus DecoderShape::attentionScale.
#include "../../../include/whispereacp/DecoderShape.h"
#include "../../../include/whispereacp/Net.h"

#include <cmath>
#include <stdexcept>

namespace WSP
{
float DecoderShape::attentionScale() const
{
    return 1.f / std::sqrt((float) headWidth());
}

int wsp_dtype_of(WeightStorage storage)
{
    switch (storage)
    {
        case WeightStorage::PackedHalf: return WSP_F16;
        case WeightStorage::PackedBFloat16: return WSP_BF16;
        default: return WSP_F32;
    }
}

std::size_t TensorBuffer::elementCount() const
{
    std::size_t count = 1;
    for (int e : extents)
        count *= (std::size_t) e;
    return count;
}

Shape::Shape(std::initializer_list<int> extentsToUse)
{
    if ((int) extentsToUse.size() > maxRank)
        throw std::logic_error("a shape holds at most four extents");
    for (int e : extentsToUse)
        extents[(std::size_t) count++] = e;
}

int Shape::rows() const
{
    return count <= 1 ? 1 : elementCount() / columns();
}

int Shape::columns() const
{
    return count == 0 ? 1 : extents[(std::size_t) count - 1];
}

int Shape::elementCount() const
{
    int total = 1;
    for (int i = 0; i < count; ++i)
        total *= extents[(std::size_t) i];
    return total;
}

Tensor::Tensor(Net& ownerToUse, int indexToUse) : owner(&ownerToUse), id(indexToUse)
{
    retain();
}

Tensor::Tensor(const Tensor& other) : owner(other.owner), id(other.id)
{
    retain();
}

Tensor::Tensor(Tensor&& other) noexcept : owner(other.owner), id(other.id)
{
    other.owner = nullptr;
    other.id = -1;
}

Tensor& Tensor::operator=(const Tensor& other)
{
    if (this != &other)
    {
        other.retain();
        release();
        owner = other.owner;
        id = other.id;
    }
    return *this;
}

Tensor& Tensor::operator=(Tensor&& other) noexcept
{
    if (this != &other)
    {
        release();
        owner = other.owner;
        id = other.id;
        other.owner = nullptr;
        other.id = -1;
    }
    return *this;
}

Tensor::~Tensor()
{
    release();
}

void Tensor::retain() const
{
    if (owner != nullptr)
        owner->retain(id);
}

void Tensor::release() const
{
    if (owner != nullptr)
        owner->release(id);
}
} // namespace WSP
