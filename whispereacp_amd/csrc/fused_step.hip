// wsp_hip_decoder_step: one single-token decoder step plus its greedy argmax
// (Decoder/Decoder.cpp:151-177 followed by Whisper/Whisper.cpp:1164-1184).
// This version records the step as the per-op kernel sequence on the
// context's stream.
#include "capi_internal.h"
#include "ops.h"

#include <new>

namespace wsp
{
namespace
{
struct FusedState
{
    float* hidden = nullptr;     // residual stream [width]
    float* normalised = nullptr; // [width]
    float* query = nullptr;      // [width]
    float* attended = nullptr;   // [width]
    float* inner = nullptr;      // [feed_forward_width]
};

size_t element_bytes(int wdtype)
{
    return wdtype == WSP_F32 ? 4 : 2;
}

const void* offset(const void* base, size_t elements, int wdtype)
{
    return static_cast<const char*>(base) + elements * element_bytes(wdtype);
}
} // namespace

int fused_prepare(Context* ctx)
{
    auto* state = new (std::nothrow) FusedState {};
    if (state == nullptr)
        return context_fail(ctx, WSP_ERR_CAPACITY, "fused step state");
    ctx->fused = state;
    const size_t d = ctx->shape.width, f = ctx->shape.feed_forward_width;
    float** buffers[] = {&state->hidden, &state->normalised, &state->query, &state->attended};
    for (float** b : buffers)
    {
        const int status = context_hip(ctx, hipMalloc(b, d * sizeof(float)), "fused step scratch");
        if (status != WSP_OK)
            return status;
    }
    return context_hip(ctx, hipMalloc(&state->inner, f * sizeof(float)), "fused step scratch");
}

void fused_release(Context* ctx)
{
    auto* state = static_cast<FusedState*>(ctx->fused);
    if (state == nullptr)
        return;
    hipFree(state->hidden);
    hipFree(state->normalised);
    hipFree(state->query);
    hipFree(state->attended);
    hipFree(state->inner);
    delete state;
    ctx->fused = nullptr;
}
} // namespace wsp

extern "C" int wsp_hip_decoder_step(wsp_hip_ctx* ctx, const wsp_decoder_tensors* tensors,
                                    const uint32_t* tokens, int position, int cross_rows,
                                    float* hidden, float* logits, const float* mask,
                                    uint32_t* argmax_out)
{
    using namespace wsp;
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (tensors == nullptr || tensors->layers == nullptr || tokens == nullptr || hidden == nullptr
        || logits == nullptr)
        return context_fail(ctx, WSP_ERR_ARGUMENT, "decoder step: null pointer");
    const wsp_decoder_shape& s = ctx->shape;
    if (position < 0 || position + 1 > s.max_positions)
        return context_fail(ctx, WSP_ERR_CAPACITY, "decoder step: position past the window");
    if (cross_rows <= 0 || cross_rows > s.cross_positions)
        return context_fail(ctx, WSP_ERR_CAPACITY, "decoder step: cross rows outside the encoder output");
    const int head_width = s.width / s.heads;
    if (head_width % 4 != 0 || head_width > ops::kMaxHeadWidth)
        return context_fail(ctx, WSP_ERR_LOGIC, "decoder step: unsupported head width");

    auto* st = static_cast<FusedState*>(ctx->fused);
    const hipStream_t stream = ctx->stream;
    const int d = s.width, f = s.feed_forward_width;
    const int wt = tensors->wdtype;
    const float scale = 1.f / sqrtf((float) head_width);
    const float eps = 1e-5f;
    hipError_t e = hipSuccess;
#define WSP_TRY(call)                                                                              \
    do                                                                                             \
    {                                                                                              \
        e = (call);                                                                                \
        if (e != hipSuccess)                                                                       \
            return context_hip(ctx, e, "decoder step");                                            \
    } while (0)

    WSP_TRY(ops::embed(stream, tokens, 1, tensors->token_embedding, tensors->position_embedding, position,
                       st->hidden, d, s.vocabulary_size));

    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = tensors->layers[l];
        float* krow = L.self_keys + (size_t) position * d;
        float* vrow = L.self_values + (size_t) position * d;

        WSP_TRY(ops::layernorm(stream, st->hidden, L.self_norm_w, L.self_norm_b, st->normalised, 1, d, eps));
        WSP_TRY(ops::linear(stream, st->normalised, 1, d, L.self_qkv_w, wt, L.self_qkv_b, st->query, d, 0));
        WSP_TRY(ops::linear(stream, st->normalised, 1, d, offset(L.self_qkv_w, (size_t) d * d, wt), wt,
                            nullptr, krow, d, 0));
        WSP_TRY(ops::linear(stream, st->normalised, 1, d, offset(L.self_qkv_w, (size_t) 2 * d * d, wt), wt,
                            L.self_qkv_b + 2 * d, vrow, d, 0));
        WSP_TRY(ops::attention(stream, st->query, 1, L.self_keys, L.self_values, position + 1, d, s.heads, 1,
                               scale, st->attended, ctx->attention_workspace));
        WSP_TRY(ops::linear(stream, st->attended, 1, d, L.self_out_w, wt, L.self_out_b, st->hidden, d,
                            WSP_LINEAR_RESIDUAL));

        WSP_TRY(ops::layernorm(stream, st->hidden, L.cross_norm_w, L.cross_norm_b, st->normalised, 1, d, eps));
        WSP_TRY(ops::linear(stream, st->normalised, 1, d, L.cross_q_w, wt, L.cross_q_b, st->query, d, 0));
        WSP_TRY(ops::attention(stream, st->query, 1, L.cross_keys, L.cross_values, cross_rows, d, s.heads, 0,
                               scale, st->attended, ctx->attention_workspace));
        WSP_TRY(ops::linear(stream, st->attended, 1, d, L.cross_out_w, wt, L.cross_out_b, st->hidden, d,
                            WSP_LINEAR_RESIDUAL));

        WSP_TRY(ops::layernorm(stream, st->hidden, L.final_norm_w, L.final_norm_b, st->normalised, 1, d, eps));
        WSP_TRY(ops::linear(stream, st->normalised, 1, d, L.fc1_w, wt, L.fc1_b, st->inner, f, WSP_LINEAR_GELU));
        WSP_TRY(ops::linear(stream, st->inner, 1, f, L.fc2_w, wt, L.fc2_b, st->hidden, d, WSP_LINEAR_RESIDUAL));
    }

    WSP_TRY(ops::layernorm(stream, st->hidden, tensors->final_norm_w, tensors->final_norm_b, hidden, 1, d, eps));
    WSP_TRY(ops::linear(stream, hidden, 1, d, tensors->logits_weight, tensors->logits_wdtype, nullptr, logits,
                        s.vocabulary_size, 0));
    if (argmax_out != nullptr)
        WSP_TRY(ops::argmax(stream, logits, 1, s.vocabulary_size, mask, argmax_out, ctx->argmax_values,
                            ctx->argmax_indices));
#undef WSP_TRY
    return WSP_OK;
}
