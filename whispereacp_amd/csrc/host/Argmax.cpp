// Argmax (Kernels/Argmax.cpp:17-81): a context sized for the rows and the row
// length once, then the two-stage masked argmax per encode().
#include "../../../include/whispereacp/Argmax.h"
#include "host_common.h"

#include <stdexcept>
#include <string>

namespace WSP
{
Argmax::~Argmax()
{
    wsp_hip_ctx_destroy(ctx);
}

void Argmax::prepare(const Device& device, int rowCount, int rowLength, void* hipStream)
{
    if (rowCount <= 0 || rowLength <= 0)
        throw std::invalid_argument("Argmax is prepared for at least one row of one element");
    wsp_hip_ctx_destroy(ctx);
    ctx = nullptr;
    // A context whose argmax workspace covers rowCount rows of rowLength.
    const wsp_decoder_shape shape {4, 1, 1, 4, rowLength, rowCount, 1};
    const int status = wsp_hip_ctx_create(&shape, device.index, hipStream, &ctx);
    if (status != WSP_OK)
        throwForStatus(status, "Argmax::prepare: the kernel context could not be created");
    rowCapacity = rowCount;
    lengthCapacity = rowLength;
}

void Argmax::encode(Pass& pass, const BufferRange& logits, const float* mask, const BufferRange& indices,
                    int rowCount, int rowLength)
{
    if (ctx == nullptr)
        throw std::logic_error("Argmax encodes once it is prepared");
    if (rowCount > rowCapacity || rowLength > lengthCapacity)
        throw std::invalid_argument("Argmax was prepared for " + std::to_string(rowCapacity) + " rows of "
                                    + std::to_string(lengthCapacity) + " and asked to scan "
                                    + std::to_string(rowCount) + " of " + std::to_string(rowLength));
    if (pass.hipStream() != wsp_hip_stream(ctx))
        throw std::logic_error("Argmax encodes into the stream it was prepared with");
    const int status = wsp_hip_argmax(ctx, static_cast<const float*>(logits.data()), rowCount, rowLength, mask,
                                      static_cast<uint32_t*>(indices.data()));
    if (status != WSP_OK)
        throwForStatus(status, wsp_hip_last_error(ctx));
}
} // namespace WSP
