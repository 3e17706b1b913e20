// The C ABI (include/wsp_hip.h): argument checks, per-context workspaces and
// error strings around the per-op kernels in ops.hip and the fused step in
// fused_step.hip. No call here allocates after wsp_hip_ctx_create.
#include "capi_internal.h"
#include "ops.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>

using wsp::Context;

namespace
{
int fail(Context* ctx, int code, const char* format, ...)
{
    if (ctx != nullptr)
    {
        va_list args;
        va_start(args, format);
        std::vsnprintf(ctx->error, sizeof(ctx->error), format, args);
        va_end(args);
    }
    return code;
}

int hip_status(Context* ctx, hipError_t e, const char* what)
{
    if (e == hipSuccess)
        return WSP_OK;
    return fail(ctx, WSP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool valid_dtype(int wdtype)
{
    return wdtype == WSP_F32 || wdtype == WSP_F16 || wdtype == WSP_BF16;
}
} // namespace

namespace wsp
{
int context_fail(Context* ctx, int code, const char* message)
{
    return fail(ctx, code, "%s", message);
}

int context_hip(Context* ctx, hipError_t e, const char* what)
{
    return hip_status(ctx, e, what);
}
} // namespace wsp

extern "C" {

int wsp_hip_ctx_create(const wsp_decoder_shape* shape, int device, void* stream, wsp_hip_ctx** out)
{
    if (shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    if (shape->width <= 0 || shape->heads <= 0 || shape->layers <= 0 || shape->feed_forward_width <= 0
        || shape->vocabulary_size <= 0 || shape->max_positions <= 0 || shape->cross_positions <= 0
        || shape->width % shape->heads != 0)
        return WSP_ERR_SHAPE;

    auto* ctx = new (std::nothrow) Context {};
    if (ctx == nullptr)
        return WSP_ERR_CAPACITY;
    ctx->shape = *shape;
    ctx->device = device;
    ctx->stream = static_cast<hipStream_t>(stream);

    int status = hip_status(ctx, hipSetDevice(device), "hipSetDevice");
    if (status == WSP_OK)
    {
        const int head_width = shape->width / shape->heads;
        const int longest = std::max(shape->max_positions, shape->cross_positions);
        size_t floats = 0;
        for (int q = 1; q <= shape->max_positions; ++q)
            floats = std::max(floats, wsp::ops::attention_workspace_floats(shape->heads, q, longest,
                                                                           head_width));
        ctx->attention_floats = std::max<size_t>(floats, 1);
        status = hip_status(ctx, hipMalloc(&ctx->attention_workspace, ctx->attention_floats * sizeof(float)),
                            "attention workspace");
        // The prompt attention's per-head counters start at zero (each launch
        // leaves them zero again).
        if (status == WSP_OK)
            status = hip_status(ctx, hipMemset(ctx->attention_workspace, 0,
                                               wsp::ops::kAttentionCounters * sizeof(unsigned int)),
                                "attention workspace");
    }
    if (status == WSP_OK)
    {
        ctx->argmax_candidates =
            (size_t) shape->max_positions * wsp::ops::argmax_groups(shape->vocabulary_size);
        status = hip_status(ctx, hipMalloc(&ctx->argmax_values, ctx->argmax_candidates * sizeof(float)),
                            "argmax workspace");
        if (status == WSP_OK)
            status = hip_status(ctx,
                                hipMalloc(&ctx->argmax_indices, ctx->argmax_candidates * sizeof(uint32_t)),
                                "argmax workspace");
    }
    if (status == WSP_OK)
        status = wsp::fused_prepare(ctx);
    if (status != WSP_OK)
    {
        wsp_hip_ctx_destroy(ctx);
        return status;
    }
    *out = ctx;
    return WSP_OK;
}

void wsp_hip_ctx_destroy(wsp_hip_ctx* ctx)
{
    if (ctx == nullptr)
        return;
    hipSetDevice(ctx->device);
    wsp::fused_release(ctx);
    hipFree(ctx->attention_workspace);
    hipFree(ctx->argmax_values);
    hipFree(ctx->argmax_indices);
    delete ctx;
}

const char* wsp_hip_last_error(const wsp_hip_ctx* ctx)
{
    return ctx == nullptr ? "no context" : ctx->error;
}

void* wsp_hip_stream(const wsp_hip_ctx* ctx)
{
    return ctx == nullptr ? nullptr : static_cast<void*>(ctx->stream);
}

int wsp_hip_linear(wsp_hip_ctx* ctx, const float* x, int rows, int inner, const void* weight,
                   int wdtype, const float* bias, float* y, int out, int flags)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (x == nullptr || weight == nullptr || y == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "linear: null input, weight or output");
    if (rows <= 0 || inner <= 0 || out <= 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "linear: extents %d x %d -> %d must be positive", rows,
                    inner, out);
    if (!valid_dtype(wdtype) || (flags & ~(WSP_LINEAR_GELU | WSP_LINEAR_RESIDUAL)) != 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "linear: unknown weight storage %d or flags %d", wdtype,
                    flags);
    return hip_status(ctx, wsp::ops::linear(ctx->stream, x, rows, inner, weight, wdtype, bias, y, out, flags),
                      "linear");
}

int wsp_hip_layernorm(wsp_hip_ctx* ctx, const float* x, const float* gamma, const float* beta,
                      float* y, int rows, int width, float eps)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (x == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "layernorm: null pointer");
    if (rows <= 0 || width <= 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "layernorm: %d rows of %d", rows, width);
    return hip_status(ctx, wsp::ops::layernorm(ctx->stream, x, gamma, beta, y, rows, width, eps),
                      "layernorm");
}

int wsp_hip_embed(wsp_hip_ctx* ctx, const uint32_t* tokens, int count, const float* token_table,
                  const float* position_table, int first_position, float* y, int width)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (tokens == nullptr || token_table == nullptr || position_table == nullptr || y == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "embed: null pointer");
    if (count <= 0 || width <= 0 || first_position < 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "embed: %d tokens of width %d from %d", count, width,
                    first_position);
    if (first_position + count > ctx->shape.max_positions)
        return fail(ctx, WSP_ERR_CAPACITY, "embed: positions %d..%d past the %d-row table",
                    first_position, first_position + count - 1, ctx->shape.max_positions);
    return hip_status(ctx,
                      wsp::ops::embed(ctx->stream, tokens, count, token_table, position_table,
                                      first_position, y, width, ctx->shape.vocabulary_size),
                      "embed");
}

int wsp_hip_attention(wsp_hip_ctx* ctx, const float* q, int q_count, const float* keys,
                      const float* values, int k_count, int width, int heads, int causal,
                      float scale, float* out)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (q == nullptr || keys == nullptr || values == nullptr || out == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "attention: null pointer");
    if (q_count <= 0 || k_count <= 0 || width <= 0 || heads <= 0 || width % heads != 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "attention: %d queries, %d keys, width %d, %d heads",
                    q_count, k_count, width, heads);
    const int head_width = width / heads;
    if (head_width % 4 != 0 || head_width > wsp::ops::kMaxHeadWidth)
        return fail(ctx, WSP_ERR_LOGIC,
                    "attention holds heads up to %d wide in quads and was asked for %d",
                    wsp::ops::kMaxHeadWidth, head_width);
    if (causal && q_count > k_count)
        return fail(ctx, WSP_ERR_SHAPE, "attention: %d causal queries over only %d keys", q_count,
                    k_count);
    if (wsp::ops::attention_workspace_floats(heads, q_count, k_count, head_width) > ctx->attention_floats)
        return fail(ctx, WSP_ERR_CAPACITY,
                    "attention was sized for this context's shape and asked for %d queries over %d keys",
                    q_count, k_count);
    return hip_status(ctx,
                      wsp::ops::attention(ctx->stream, q, q_count, keys, values, k_count, width, heads,
                                          causal, scale, out, ctx->attention_workspace),
                      "attention");
}

int wsp_hip_argmax(wsp_hip_ctx* ctx, const float* logits, int rows, int row_length,
                   const float* mask, uint32_t* out)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (logits == nullptr || out == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "argmax: null pointer");
    if (rows <= 0 || row_length <= 0)
        return fail(ctx, WSP_ERR_ARGUMENT, "argmax: %d rows of %d", rows, row_length);
    if ((size_t) rows * wsp::ops::argmax_groups(row_length) > ctx->argmax_candidates)
        return fail(ctx, WSP_ERR_CAPACITY,
                    "Argmax was prepared for %d rows of %d and asked to scan %d of %d",
                    ctx->shape.max_positions, ctx->shape.vocabulary_size, rows, row_length);
    return hip_status(ctx,
                      wsp::ops::argmax(ctx->stream, logits, rows, row_length, mask, out,
                                       ctx->argmax_values, ctx->argmax_indices),
                      "argmax");
}

int wsp_hip_project_cross_kv(wsp_hip_ctx* ctx, const float* x, int rows, int width, const void* wk,
                             const void* wv, const float* bv, int wdtype, float* k_out, float* v_out)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (x == nullptr || wk == nullptr || wv == nullptr || k_out == nullptr || v_out == nullptr)
        return fail(ctx, WSP_ERR_ARGUMENT, "cross K/V: null pointer");
    if (rows <= 0 || width <= 0 || !valid_dtype(wdtype))
        return fail(ctx, WSP_ERR_ARGUMENT, "cross K/V: %d rows of %d, storage %d", rows, width, wdtype);
    if (rows > ctx->shape.cross_positions)
        return fail(ctx, WSP_ERR_CAPACITY, "cross K/V: %d rows past the %d cross positions", rows,
                    ctx->shape.cross_positions);
    return wsp::cross_kv_projection(ctx, x, rows, width, wk, wv, bv, wdtype, k_out, v_out);
}

} // extern "C"
