// HIP stand-ins for the eacp GPU types (include/whispereacp/Gpu.h).
#include "../../../include/whispereacp/Gpu.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <cstring>
#include <new>

namespace WSP
{
Device& Device::shared()
{
    static Device device {0};
    return device;
}

void checkHip(int status, const char* what)
{
    if (status != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString((hipError_t) status));
}

DeviceBuffer::DeviceBuffer(const Device& deviceToUse, std::size_t byteCount)
    : bytes(byteCount), device(deviceToUse.index)
{
    if (device == Device::hostIndex)
    {
        pointer = std::malloc(bytes > 0 ? bytes : 1);
        if (pointer == nullptr)
            throw std::bad_alloc();
        return;
    }
    checkHip(hipSetDevice(device), "hipSetDevice");
    checkHip(hipMalloc(&pointer, bytes > 0 ? bytes : 1), "hipMalloc");
}

DeviceBuffer::DeviceBuffer(const Device& deviceToUse, const void* host, std::size_t byteCount)
    : DeviceBuffer(deviceToUse, byteCount)
{
    upload(host, byteCount);
}

namespace
{
void release(void* pointer, int device)
{
    if (pointer == nullptr)
        return;
    if (device == Device::hostIndex)
        std::free(pointer);
    else
        (void) hipFree(pointer);
}
} // namespace

DeviceBuffer::~DeviceBuffer()
{
    release(pointer, device);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : pointer(other.pointer), bytes(other.bytes), device(other.device)
{
    other.pointer = nullptr;
    other.bytes = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept
{
    if (this != &other)
    {
        release(pointer, device);
        pointer = other.pointer;
        bytes = other.bytes;
        device = other.device;
        other.pointer = nullptr;
        other.bytes = 0;
    }
    return *this;
}

void DeviceBuffer::upload(const void* host, std::size_t count, std::size_t offset) const
{
    if (offset + count > bytes)
        throw std::out_of_range("upload past the end of a device buffer");
    if (device == Device::hostIndex)
    {
        std::memcpy(static_cast<char*>(pointer) + offset, host, count);
        return;
    }
    checkHip(hipMemcpy(static_cast<char*>(pointer) + offset, host, count, hipMemcpyHostToDevice),
             "hipMemcpy host to device");
}

void DeviceBuffer::read(void* host, std::size_t count, std::size_t offset) const
{
    if (offset + count > bytes)
        throw std::out_of_range("read past the end of a device buffer");
    if (device == Device::hostIndex)
    {
        std::memcpy(host, static_cast<char*>(pointer) + offset, count);
        return;
    }
    checkHip(hipMemcpy(host, static_cast<char*>(pointer) + offset, count, hipMemcpyDeviceToHost),
             "hipMemcpy device to host");
}

void Pass::synchronize() const
{
    checkHip(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}
} // namespace WSP
