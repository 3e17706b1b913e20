// Kernels/Argmax.h:221-248 — greedy sampling's masked argmax, sized once by
// prepare() and recorded into a pass by encode().
#pragma once

#include "Gpu.h"
#include "../wsp_hip.h"

namespace WSP
{
class Argmax
{
public:
    Argmax() = default;
    ~Argmax();
    Argmax(const Argmax&) = delete;
    Argmax& operator=(const Argmax&) = delete;

    void prepare(const Device& device, int rowCount, int rowLength, void* hipStream = nullptr);

    // indices[r] = the first j maximising logits[r * rowLength + j] over the j
    // with mask[j] == 0 (mask null: none suppressed). std::invalid_argument
    // beyond the prepared capacity (Kernels/Argmax.cpp:47-58).
    void encode(Pass& pass, const BufferRange& logits, const float* mask, const BufferRange& indices,
                int rowCount, int rowLength);

private:
    wsp_hip_ctx* ctx = nullptr;
    int rowCapacity = 0;
    int lengthCapacity = 0;
};
} // namespace WSP
