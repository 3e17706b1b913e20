// The once-per-sequence cross-attention key/value projection
// (Decoder/Decoder.cpp:121-146): K = X·Wkᵀ, V = X·Wvᵀ + bv over the encoder
// rows with fp32 accumulation — one matrix-core launch for both when the
// weights are 16-bit, else the fp32 tiled product twice.
#include "capi_internal.h"
#include "ops.h"

namespace wsp
{
int cross_kv_projection(Context* ctx, const float* x, int rows, int width, const void* wk, const void* wv,
                        const float* bv, int wdtype, float* k_out, float* v_out)
{
    if (ops::tile_product_fits(wdtype, width, 2 * width, width, x))
    {
        ops::TileProduct p {};
        p.x = x;
        p.rows = rows;
        p.inner = width;
        p.w0 = wk;
        p.w1 = wv;
        p.split = width;
        p.out = 2 * width;
        p.bias0 = nullptr;
        p.bias1 = bv;
        p.y0 = k_out;
        p.y1 = v_out;
        p.ldy = width;
        p.rows_per_group = rows;
        p.group_stride = 0;
        p.flags = 0;
        p.wdtype = wdtype;
        return context_hip(ctx, ops::tile_product(ctx->stream, p), "cross K/V projection");
    }
    hipError_t e = ops::linear(ctx->stream, x, rows, width, wk, wdtype, nullptr, k_out, width, 0);
    if (e == hipSuccess)
        e = ops::linear(ctx->stream, x, rows, width, wv, wdtype, bv, v_out, width, 0);
    return context_hip(ctx, e, "cross K/V projection");
}
} // namespace wsp
