// HIP stand-ins for the eacp GPU types the reference's decoder surface names
// (Kernels/KernelTypes.h:11-24): a device, an owning buffer, a byte range of
// one, and a pass, which here is a HIP stream (work is ordered by the stream,
// so nothing records barriers).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

namespace WSP
{
// The device a decoder runs on. One GPU per process is the supported model.
// Device::host() places buffers in host memory instead (the reference's
// WeightPlacement::Host, Model/TensorLoader.h:40-44): weights loaded there
// serve a Net that runs on the host, and nothing touches a GPU.
struct Device
{
    static constexpr int hostIndex = -1;

    int index = 0;

    static Device& shared();
    static Device host() { return Device {hostIndex}; }
    bool isHost() const { return index == hostIndex; }
};

// Device memory (host memory on Device::host()), allocated on construction
// and freed on destruction.
class DeviceBuffer
{
public:
    DeviceBuffer() = default;
    DeviceBuffer(const Device& device, std::size_t bytes);
    DeviceBuffer(const Device& device, const void* host, std::size_t bytes);
    ~DeviceBuffer();

    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    void* data() const { return pointer; }
    std::size_t size() const { return bytes; }
    bool isValid() const { return pointer != nullptr; }

    void upload(const void* host, std::size_t count, std::size_t offset = 0) const;
    void read(void* host, std::size_t count, std::size_t offset = 0) const;

private:
    void* pointer = nullptr;
    std::size_t bytes = 0;
    int device = 0;
};

// A byte range of device memory (eacp::GPU::BufferRange). Views are not
// owning: the buffer outlives the range.
struct BufferRange
{
    void* base = nullptr;
    std::size_t offset = 0;
    std::size_t size = 0;

    static BufferRange of(const DeviceBuffer& buffer) { return {buffer.data(), 0, buffer.size()}; }

    void* data() const { return static_cast<char*>(base) + offset; }
    bool isValid() const { return base != nullptr; }
    bool sameStart(const BufferRange& other) const { return data() == other.data(); }
};

// The recording target of a step (eacp::GPU::ComputePass): a HIP stream.
class Pass
{
public:
    explicit Pass(void* hipStream = nullptr) : stream(hipStream) {}

    void* hipStream() const { return stream; }
    void synchronize() const;

private:
    void* stream = nullptr;
};

// Throws std::runtime_error naming `what` when status is a HIP error.
void checkHip(int status, const char* what);
} // namespace WSP
