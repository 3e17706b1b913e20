// The Whisper encoder (Encoder/Encoder.cpp:82-111) on gfx950: the step before
// the decode path, producing the [positions, width] rows the decoder's cross
// keys and values are projected from.
//
//   x = gelu(conv1(mel))   stride 1, kernel 3, padding 1
//   x = gelu(conv2(x))     stride 2: the frames halve into positions
//   h = x + embed_positions
//   per layer: h += out_proj(attention(LN(h)));  h += fc2(gelu(fc1(LN(h))))
//   rows = LN(h)
//
// Both convolutions are products: a column kernel gathers, for every output
// frame, the three taps of every input channel into one row (index
// channel * 3 + tap, the order of a [out, in, 3] weight row), with zero past
// the frames the run was given (Encoder/Encoder.h:46-56), and the product
// adds the bias, applies GELU and — for conv2 — adds the positional rows the
// output buffer was filled with. The projections, LayerNorms and attention
// are the library's per-op kernels; their 16-bit-weight products run on the
// matrix cores (tile_product_kernel) over 1500-row operands.
#include "../../include/wsp_hip.h"
#include "device_common.h"
#include "ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <new>
#include <vector>

namespace wsp::encoder
{
namespace
{
constexpr int kColumnThreads = 256;

// Kernels/Conv1d.h:121-124 with kernel 3 and padding 1.
int conv_length(int length, int stride)
{
    return (length + 2 - 3) / stride + 1;
}

// Row t of the first convolution's columns: mel[s][t + tap - 1] at
// s * 3 + tap. The mel is band-major with `stride` frames a band, of which
// the run reads the first `frames`.
__global__ void __launch_bounds__(kColumnThreads) mel_columns_kernel(const float* __restrict__ mel, int bins,
                                                                     int stride, int frames,
                                                                     float* __restrict__ columns)
{
    const int t = blockIdx.x;
    const int inner = bins * 3;
    for (int i = threadIdx.x; i < inner; i += kColumnThreads)
    {
        const int s = i / 3, at = t + i % 3 - 1;
        columns[(size_t) t * inner + i] = at >= 0 && at < frames ? mel[(size_t) s * stride + at] : 0.f;
    }
}

// Row p of the second convolution's columns over frame-major rows x
// [frames, channels]: x[2p + tap - 1][s] at s * 3 + tap.
__global__ void __launch_bounds__(kColumnThreads) frame_columns_kernel(const float* __restrict__ x, int channels,
                                                                       int frames, float* __restrict__ columns)
{
    const int p = blockIdx.x;
    const int inner = channels * 3;
    for (int i = threadIdx.x; i < inner; i += kColumnThreads)
    {
        const int s = i / 3, at = 2 * p + i % 3 - 1;
        columns[(size_t) p * inner + i] = at >= 0 && at < frames ? x[(size_t) at * channels + s] : 0.f;
    }
}
} // namespace
} // namespace wsp::encoder

struct wsp_encoder
{
    wsp_encoder_shape shape {};
    int device = 0;
    hipStream_t stream = nullptr;
    float* columns = nullptr; // both convolutions' gathered rows
    float* conv = nullptr;    // [conv frames, width] frame-major
    float* hidden = nullptr;  // [positions, width]
    float* normed = nullptr;
    float* q = nullptr;
    float* k = nullptr;
    float* v = nullptr;
    float* att = nullptr;
    float* ff = nullptr;      // [positions, feed_forward_width]
    float* workspace = nullptr;
    std::vector<void*> owned;
    char error[512] = {0};
};

namespace
{
int encoder_fail(wsp_encoder* e, int code, const char* message)
{
    std::snprintf(e->error, sizeof e->error, "%s", message);
    return code;
}

int encoder_hip(wsp_encoder* e, hipError_t status, const char* what)
{
    if (status == hipSuccess)
        return WSP_OK;
    std::snprintf(e->error, sizeof e->error, "%s: %s", what, hipGetErrorString(status));
    return WSP_ERR_HIP;
}

hipError_t encoder_allocate(wsp_encoder* e, float** out, size_t floats)
{
    void* p = nullptr;
    const hipError_t status = hipMalloc(&p, std::max<size_t>(floats, 1) * sizeof(float));
    if (status == hipSuccess)
    {
        e->owned.push_back(p);
        *out = static_cast<float*>(p);
    }
    return status;
}
} // namespace

extern "C" {

int wsp_encoder_create(const wsp_encoder_shape* shape, int device, void* stream, wsp_encoder** out)
{
    using wsp::encoder::conv_length;
    if (shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    const wsp_encoder_shape& s = *shape;
    if (s.mel_bins <= 0 || s.width <= 0 || s.heads <= 0 || s.layers < 0 || s.feed_forward_width <= 0
        || s.input_frames <= 0)
        return WSP_ERR_ARGUMENT;
    if (s.width % s.heads != 0 || (s.width / s.heads) % 4 != 0 || s.width / s.heads > wsp::ops::kMaxHeadWidth)
        return WSP_ERR_SHAPE;

    wsp_encoder* e = new (std::nothrow) wsp_encoder;
    if (e == nullptr)
        return WSP_ERR_HIP;
    e->shape = s;
    e->device = device;
    e->stream = static_cast<hipStream_t>(stream);
    const size_t frames = (size_t) conv_length(s.input_frames, 1);
    const size_t positions = (size_t) conv_length((int) frames, 2);
    const size_t d = (size_t) s.width;
    hipError_t status = hipSetDevice(device);
    if (status == hipSuccess)
        status = encoder_allocate(e, &e->columns, std::max(frames * s.mel_bins * 3, positions * d * 3));
    if (status == hipSuccess)
        status = encoder_allocate(e, &e->conv, frames * d);
    float** rows[] = {&e->hidden, &e->normed, &e->q, &e->k, &e->v, &e->att};
    for (float** r : rows)
        if (status == hipSuccess)
            status = encoder_allocate(e, r, positions * d);
    if (status == hipSuccess)
        status = encoder_allocate(e, &e->ff, positions * s.feed_forward_width);
    if (status == hipSuccess)
        status = encoder_allocate(e, &e->workspace,
                                  wsp::ops::attention_workspace_floats(s.heads, (int) positions, (int) positions,
                                                                       s.width / s.heads));
    // The attention workspace's counters start at zero.
    if (status == hipSuccess)
        status = hipMemsetAsync(e->workspace, 0, wsp::ops::kAttentionCounters * sizeof(unsigned), e->stream);
    if (status == hipSuccess)
        status = hipStreamSynchronize(e->stream);
    if (status != hipSuccess)
    {
        for (void* p : e->owned)
            (void) hipFree(p);
        delete e;
        return WSP_ERR_HIP;
    }
    *out = e;
    return WSP_OK;
}

void wsp_encoder_destroy(wsp_encoder* e)
{
    if (e == nullptr)
        return;
    (void) hipSetDevice(e->device);
    (void) hipStreamSynchronize(e->stream);
    for (void* p : e->owned)
        (void) hipFree(p);
    delete e;
}

const char* wsp_encoder_last_error(const wsp_encoder* e)
{
    return e == nullptr ? "null encoder" : e->error;
}

int wsp_encoder_encode(wsp_encoder* e, const wsp_encoder_tensors* T, const float* mel, float* output,
                       int position_count)
{
    using namespace wsp::encoder;
    namespace ops = wsp::ops;
    if (e == nullptr)
        return WSP_ERR_ARGUMENT;
    e->error[0] = 0;
    if (T == nullptr || mel == nullptr || output == nullptr || (e->shape.layers > 0 && T->layers == nullptr))
        return encoder_fail(e, WSP_ERR_ARGUMENT, "wsp_encoder_encode: null tensors, mel or output");
    const wsp_encoder_shape& s = e->shape;
    const int window_positions = conv_length(conv_length(s.input_frames, 1), 2);
    if (position_count < 0 || position_count > window_positions)
        return encoder_fail(e, WSP_ERR_SHAPE, "wsp_encoder_encode: more positions than the window holds");
    if (T->wdtype != WSP_F32 && T->wdtype != WSP_F16 && T->wdtype != WSP_BF16)
        return encoder_fail(e, WSP_ERR_LOGIC, "wsp_encoder_encode: unknown projection storage");
    const int frames = position_count == 0 ? s.input_frames : std::min(2 * position_count, s.input_frames);
    const int conv_frames = conv_length(frames, 1);
    const int positions = conv_length(conv_frames, 2);
    const int d = s.width, f = s.feed_forward_width, heads = s.heads;
    const float scale = 1.f / std::sqrt((float) (d / heads));
    const float eps = 1e-5f;
    hipStream_t st = e->stream;
    (void) hipSetDevice(e->device);
    hipError_t status;

    hipLaunchKernelGGL(mel_columns_kernel, dim3(conv_frames), dim3(kColumnThreads), 0, st, mel, s.mel_bins,
                       s.input_frames, frames, e->columns);
    if ((status = hipGetLastError()) != hipSuccess)
        return encoder_hip(e, status, "conv1 columns");
    if ((status = ops::linear(st, e->columns, conv_frames, 3 * s.mel_bins, T->conv1_w, WSP_F32, T->conv1_b, e->conv,
                              d, 1)) != hipSuccess)
        return encoder_hip(e, status, "conv1");
    hipLaunchKernelGGL(frame_columns_kernel, dim3(positions), dim3(kColumnThreads), 0, st, e->conv, d, conv_frames,
                       e->columns);
    if ((status = hipGetLastError()) != hipSuccess)
        return encoder_hip(e, status, "conv2 columns");
    // h = gelu(conv2) + embed_positions: the rows start as the positional
    // table's first rows and the product adds to them (bias, GELU, residual).
    if ((status = hipMemcpyAsync(e->hidden, T->positions, (size_t) positions * d * sizeof(float),
                                 hipMemcpyDeviceToDevice, st)) != hipSuccess)
        return encoder_hip(e, status, "positional rows");
    if ((status = ops::linear(st, e->columns, positions, 3 * d, T->conv2_w, WSP_F32, T->conv2_b, e->hidden, d, 3))
        != hipSuccess)
        return encoder_hip(e, status, "conv2");

    const int wt = T->wdtype;
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_encoder_layer_tensors& L = T->layers[l];
        if ((status = ops::layernorm(st, e->hidden, L.attention_norm_w, L.attention_norm_b, e->normed, positions, d,
                                     eps)) != hipSuccess
            || (status = ops::linear(st, e->normed, positions, d, L.q_w, wt, L.q_b, e->q, d, 0)) != hipSuccess
            || (status = ops::linear(st, e->normed, positions, d, L.k_w, wt, nullptr, e->k, d, 0)) != hipSuccess
            || (status = ops::linear(st, e->normed, positions, d, L.v_w, wt, L.v_b, e->v, d, 0)) != hipSuccess)
            return encoder_hip(e, status, "self-attention projections");
        if ((status = ops::attention(st, e->q, positions, e->k, e->v, positions, d, heads, 0, scale, e->att,
                                     e->workspace)) != hipSuccess)
            return encoder_hip(e, status, "self attention");
        if ((status = ops::linear(st, e->att, positions, d, L.out_w, wt, L.out_b, e->hidden, d, 2)) != hipSuccess)
            return encoder_hip(e, status, "attention output");
        if ((status = ops::layernorm(st, e->hidden, L.final_norm_w, L.final_norm_b, e->normed, positions, d, eps))
                != hipSuccess
            || (status = ops::linear(st, e->normed, positions, d, L.fc1_w, wt, L.fc1_b, e->ff, f, 1)) != hipSuccess
            || (status = ops::linear(st, e->ff, positions, f, L.fc2_w, wt, L.fc2_b, e->hidden, d, 2)) != hipSuccess)
            return encoder_hip(e, status, "feed-forward");
    }
    if ((status = ops::layernorm(st, e->hidden, T->final_norm_w, T->final_norm_b, output, positions, d, eps))
        != hipSuccess)
        return encoder_hip(e, status, "final norm");
    return WSP_OK;
}

} // extern "C"
