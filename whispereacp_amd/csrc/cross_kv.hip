// The once-per-sequence cross-attention key/value projection
// (Decoder/Decoder.cpp:121-146): out = X·Wᵀ (+ bias) over the encoder rows,
// fp32 accumulation.
#include "capi_internal.h"
#include "ops.h"

namespace wsp
{
int cross_kv_projection(Context* ctx, const float* x, int rows, int width, const void* weight,
                        const float* bias, int wdtype, float* out)
{
    return context_hip(ctx, ops::linear(ctx->stream, x, rows, width, weight, wdtype, bias, out, width, 0),
                       "cross K/V projection");
}
} // namespace wsp
