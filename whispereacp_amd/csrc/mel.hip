// The mel front end (Mel/MelSpectrogram.cpp) on gfx950: 16 kHz samples in,
// the normalised log-mel the encoder's first convolution reads out.
//
//   frames[f][t] = reflect-padded samples[f·hop + t - fft/2] · hann[t]
//   spectrum     = frames · basis^T          basis rows cos / -sin per bin
//   power[f][b]  = re^2 + im^2               (the non-redundant half)
//   mel[f][m]    = power · filters^T         the published filterbank
//   out[m][f]    = (max(log10 max(mel, 1e-10), peak - 8) + 4) / 4
//
// The transform is a product against a DFT basis built once in double on the
// host (as the reference's SpectrumProduct is), so it runs through the
// library's tiled product; the window is the periodic Hann
// (Tests/Mel/ScalarMel.h:20-28) and the padding numpy's "reflect" folded into
// the frame index (Tests/Mel/ScalarMel.h:32-49).
#include "../../include/wsp_hip.h"
#include "device_common.h"
#include "ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <new>
#include <vector>

namespace wsp::mel
{
namespace
{
constexpr int kThreads = 256;
constexpr int kLogBlocks = 512; // blocks of the log pass, each leaving one maximum

__global__ void __launch_bounds__(kThreads) frames_kernel(const float* __restrict__ samples, int count,
                                                          const float* __restrict__ window, int fft, int hop,
                                                          float* __restrict__ frames)
{
    const int f = blockIdx.x;
    for (int t = threadIdx.x; t < fft; t += kThreads)
    {
        int x = f * hop + t - fft / 2;
        if (x < 0)
            x = -x;
        if (x >= count)
            x = 2 * (count - 1) - x;
        frames[(size_t) f * fft + t] = samples[x] * window[t];
    }
}

// power rows have a stride of `padded` (bins rounded up to a multiple of 4,
// the padding left at zero) so the filterbank product takes vector loads.
__global__ void __launch_bounds__(kThreads) power_kernel(const float* __restrict__ spectrum, int bins, int padded,
                                                         int total, float* __restrict__ power)
{
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= total)
        return;
    const int f = i / bins, b = i % bins;
    const float re = spectrum[(size_t) f * 2 * bins + 2 * b], im = spectrum[(size_t) f * 2 * bins + 2 * b + 1];
    power[(size_t) f * padded + b] = re * re + im * im;
}

// log10 of the [frames, mels] products into the band-major output, and each
// block's largest value into peaks[block].
__global__ void __launch_bounds__(kThreads) log_kernel(const float* __restrict__ rows, int frames, int mels,
                                                       float* __restrict__ out, float* __restrict__ peaks)
{
    __shared__ float scratch[kThreads / kWave];
    const int total = frames * mels;
    float best = -INFINITY;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads)
    {
        const int m = i / frames, f = i % frames; // band-major index, so stores coalesce
        const float v = log10f(fmaxf(rows[(size_t) f * mels + m], 1e-10f));
        out[i] = v;
        best = fmaxf(best, v);
    }
    best = block_max(best, scratch);
    if (threadIdx.x == 0)
        peaks[blockIdx.x] = best;
}

__global__ void __launch_bounds__(kThreads) normalise_kernel(float* __restrict__ out, int total,
                                                             const float* __restrict__ peaks, int blocks)
{
    __shared__ float scratch[kThreads / kWave];
    float best = -INFINITY;
    for (int i = threadIdx.x; i < blocks; i += kThreads)
        best = fmaxf(best, peaks[i]);
    const float floor = block_max(best, scratch) - 8.f;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads)
        out[i] = (fmaxf(out[i], floor) + 4.f) / 4.f;
}
} // namespace
} // namespace wsp::mel

struct wsp_mel
{
    wsp_mel_shape shape {};
    int device = 0;
    hipStream_t stream = nullptr;
    float* window = nullptr;   // [fft]
    float* basis = nullptr;    // [2 bins][fft]: cos, -sin
    float* frames = nullptr;   // [frames][fft]
    float* spectrum = nullptr; // [frames][2 bins]
    float* power = nullptr;    // [frames][padded bins], the padding zero
    float* filters = nullptr;  // [mels][padded bins]: the call's filterbank, the padding zero
    float* rows = nullptr;     // [frames][mels]
    float* peaks = nullptr;    // [kLogBlocks]
    std::vector<void*> owned;
    char error[512] = {0};
};

namespace
{
hipError_t mel_allocate(wsp_mel* m, float** out, size_t floats)
{
    void* p = nullptr;
    const hipError_t status = hipMalloc(&p, std::max<size_t>(floats, 1) * sizeof(float));
    if (status == hipSuccess)
    {
        m->owned.push_back(p);
        *out = static_cast<float*>(p);
    }
    return status;
}

int mel_hip(wsp_mel* m, hipError_t status, const char* what)
{
    if (status == hipSuccess)
        return WSP_OK;
    std::snprintf(m->error, sizeof m->error, "%s: %s", what, hipGetErrorString(status));
    return WSP_ERR_HIP;
}
} // namespace

extern "C" {

int wsp_mel_create(const wsp_mel_shape* shape, int device, void* stream, wsp_mel** out)
{
    if (shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    const wsp_mel_shape& s = *shape;
    if (s.sample_count <= 0 || s.fft_length < 2 || s.hop_length <= 0 || s.frame_count <= 0 || s.mel_count <= 0)
        return WSP_ERR_ARGUMENT;
    // Reflect padding mirrors fft / 2 samples about each end, and the last
    // frame must start inside the padded signal.
    if (s.sample_count <= s.fft_length / 2 || (long long) (s.frame_count - 1) * s.hop_length > s.sample_count)
        return WSP_ERR_SHAPE;
    wsp_mel* m = new (std::nothrow) wsp_mel;
    if (m == nullptr)
        return WSP_ERR_HIP;
    m->shape = s;
    m->device = device;
    m->stream = static_cast<hipStream_t>(stream);
    const int fft = s.fft_length, bins = fft / 2 + 1;
    std::vector<float> window(fft), basis((size_t) 2 * bins * fft);
    const double two_pi = 2.0 * 3.14159265358979323846;
    for (int n = 0; n < fft; ++n)
        window[n] = (float) (0.5 * (1.0 - std::cos(two_pi * n / fft)));
    for (int b = 0; b < bins; ++b)
        for (int t = 0; t < fft; ++t)
        {
            // the angle reduced modulo the period first, so it stays exact in double
            const double angle = two_pi * (double) (((long long) b * t) % fft) / fft;
            basis[(size_t) 2 * b * fft + t] = (float) std::cos(angle);
            basis[(size_t) (2 * b + 1) * fft + t] = (float) -std::sin(angle);
        }
    hipError_t status = hipSetDevice(device);
    if (status == hipSuccess)
        status = mel_allocate(m, &m->window, fft);
    if (status == hipSuccess)
        status = mel_allocate(m, &m->basis, basis.size());
    if (status == hipSuccess)
        status = mel_allocate(m, &m->frames, (size_t) s.frame_count * fft);
    if (status == hipSuccess)
        status = mel_allocate(m, &m->spectrum, (size_t) s.frame_count * 2 * bins);
    const int padded = (bins + 3) / 4 * 4;
    if (status == hipSuccess)
        status = mel_allocate(m, &m->power, (size_t) s.frame_count * padded);
    if (status == hipSuccess)
        status = mel_allocate(m, &m->filters, (size_t) s.mel_count * padded);
    if (status == hipSuccess)
        status = hipMemset(m->power, 0, (size_t) s.frame_count * padded * sizeof(float));
    if (status == hipSuccess)
        status = hipMemset(m->filters, 0, (size_t) s.mel_count * padded * sizeof(float));
    if (status == hipSuccess)
        status = mel_allocate(m, &m->rows, (size_t) s.frame_count * s.mel_count);
    if (status == hipSuccess)
        status = mel_allocate(m, &m->peaks, wsp::mel::kLogBlocks);
    if (status == hipSuccess)
        status = hipMemcpy(m->window, window.data(), window.size() * sizeof(float), hipMemcpyHostToDevice);
    if (status == hipSuccess)
        status = hipMemcpy(m->basis, basis.data(), basis.size() * sizeof(float), hipMemcpyHostToDevice);
    if (status != hipSuccess)
    {
        for (void* p : m->owned)
            (void) hipFree(p);
        delete m;
        return WSP_ERR_HIP;
    }
    *out = m;
    return WSP_OK;
}

void wsp_mel_destroy(wsp_mel* m)
{
    if (m == nullptr)
        return;
    (void) hipSetDevice(m->device);
    (void) hipStreamSynchronize(m->stream);
    for (void* p : m->owned)
        (void) hipFree(p);
    delete m;
}

const char* wsp_mel_last_error(const wsp_mel* m)
{
    return m == nullptr ? "null mel front end" : m->error;
}

int wsp_mel_encode(wsp_mel* m, const float* samples, const float* filters, float* output)
{
    using namespace wsp::mel;
    if (m == nullptr)
        return WSP_ERR_ARGUMENT;
    m->error[0] = 0;
    if (samples == nullptr || filters == nullptr || output == nullptr)
    {
        std::snprintf(m->error, sizeof m->error, "wsp_mel_encode: null samples, filters or output");
        return WSP_ERR_ARGUMENT;
    }
    const wsp_mel_shape& s = m->shape;
    const int fft = s.fft_length, bins = fft / 2 + 1, frames = s.frame_count, mels = s.mel_count;
    hipStream_t st = m->stream;
    (void) hipSetDevice(m->device);
    hipError_t status;
    hipLaunchKernelGGL(frames_kernel, dim3(frames), dim3(kThreads), 0, st, samples, s.sample_count, m->window, fft,
                       s.hop_length, m->frames);
    if ((status = hipGetLastError()) != hipSuccess)
        return mel_hip(m, status, "framing");
    if ((status = wsp::ops::linear(st, m->frames, frames, fft, m->basis, WSP_F32, nullptr, m->spectrum, 2 * bins, 0))
        != hipSuccess)
        return mel_hip(m, status, "spectrum");
    const int cells = frames * bins, padded = (bins + 3) / 4 * 4;
    hipLaunchKernelGGL(power_kernel, dim3((cells + kThreads - 1) / kThreads), dim3(kThreads), 0, st, m->spectrum,
                       bins, padded, cells, m->power);
    if ((status = hipGetLastError()) != hipSuccess)
        return mel_hip(m, status, "power");
    // The filterbank into rows of the padded stride (the padding stays zero):
    // the product then sums the same terms in the same order, plus zeros.
    if ((status = hipMemcpy2DAsync(m->filters, (size_t) padded * sizeof(float), filters, (size_t) bins * sizeof(float),
                                   (size_t) bins * sizeof(float), mels, hipMemcpyDeviceToDevice, st))
        != hipSuccess)
        return mel_hip(m, status, "filterbank copy");
    if ((status = wsp::ops::linear(st, m->power, frames, padded, m->filters, WSP_F32, nullptr, m->rows, mels, 0))
        != hipSuccess)
        return mel_hip(m, status, "filterbank");
    const int total = frames * mels;
    const int blocks = std::min(kLogBlocks, (total + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(log_kernel, dim3(blocks), dim3(kThreads), 0, st, m->rows, frames, mels, output, m->peaks);
    if ((status = hipGetLastError()) != hipSuccess)
        return mel_hip(m, status, "log");
    hipLaunchKernelGGL(normalise_kernel, dim3(blocks), dim3(kThreads), 0, st, output, total, m->peaks, blocks);
    if ((status = hipGetLastError()) != hipSuccess)
        return mel_hip(m, status, "normalise");
    return WSP_OK;
}

} // extern "C"
