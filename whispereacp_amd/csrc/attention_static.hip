// wsp_hip_attention_static: wsp_hip_attention without a context, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc). It runs the same kernels
// (ops.hip: prompt_attention_kernel for 2 to 16 queries, else
// attention_chunk_kernel and attention_combine_kernel); their split-key
// partials, which the context-bound entry point keeps in a workspace allocated
// at wsp_hip_ctx_create, live here in one file-scope device array per GPU.
//
// The array is fixed in size (kStaticAttentionFloats floats, 4 MiB) and held
// by every GPU the library runs on until the process ends. Every call on a GPU
// shares that GPU's array, so calls that overlap on one GPU (two streams, two
// threads) race on it; calls ordered on one stream do not. The partials are
// written in full before they are read. The first kAttentionCounters words are
// the prompt attention's per-head counters: zero when the array is loaded, and
// every launch leaves them zero again, so nothing needs clearing between
// calls.
#include "ops.h"
#include "../../include/wsp_hip.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

namespace
{
constexpr size_t kStaticAttentionFloats = size_t(1) << 20;
constexpr int kMaxDevices = 64;

// On the host this name is a stand-in, not a device address: only the
// pointer hipGetSymbolAddress returns for the current device may reach a
// kernel or a copy.
static __device__ __align__(256) float scratch[kStaticAttentionFloats];

std::mutex scratch_mutex;
float* scratch_address[kMaxDevices] = {};

int report(char* error, int capacity, int code, const char* format, ...)
{
    if (error != nullptr && capacity > 0)
    {
        va_list args;
        va_start(args, format);
        std::vsnprintf(error, (size_t) capacity, format, args);
        va_end(args);
    }
    return code;
}

// This device's copy of the array, looked up once per device with that device
// current (the caller's current device is the one the kernels run on). The
// address is kept for the life of the process: hipDeviceReset unloads the
// code object that holds the array, so a process that resets a device must
// not call this entry point on that device afterwards.
hipError_t device_scratch(float** out)
{
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        return e;
    if (device < 0 || device >= kMaxDevices)
        return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_address[device] == nullptr)
    {
        void* address = nullptr;
        e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return e;
        scratch_address[device] = static_cast<float*>(address);
    }
    *out = scratch_address[device];
    return hipSuccess;
}
} // namespace

extern "C" int wsp_hip_attention_static(const float* q, int q_count, const float* keys, const float* values,
                                        int k_count, int width, int heads, int causal, float scale, float* out,
                                        void* stream, char* error, int error_capacity)
{
    if (q == nullptr || keys == nullptr || values == nullptr || out == nullptr)
        return report(error, error_capacity, WSP_ERR_ARGUMENT, "attention: null pointer");
    if (q_count <= 0 || k_count <= 0 || width <= 0 || heads <= 0 || width % heads != 0)
        return report(error, error_capacity, WSP_ERR_ARGUMENT, "attention: %d queries, %d keys, width %d, %d heads",
                      q_count, k_count, width, heads);
    const int head_width = width / heads;
    if (head_width % 4 != 0 || head_width > wsp::ops::kMaxHeadWidth)
        return report(error, error_capacity, WSP_ERR_LOGIC,
                      "attention holds heads up to %d wide in quads and was asked for %d", wsp::ops::kMaxHeadWidth,
                      head_width);
    if (causal && q_count > k_count)
        return report(error, error_capacity, WSP_ERR_SHAPE, "attention: %d causal queries over only %d keys", q_count,
                      k_count);
    const size_t needed = wsp::ops::attention_workspace_floats(heads, q_count, k_count, head_width);
    if (needed > kStaticAttentionFloats)
        return report(error, error_capacity, WSP_ERR_CAPACITY,
                      "attention without allocation holds %zu partial floats and %d queries over %d keys in %d "
                      "heads need %zu",
                      kStaticAttentionFloats, q_count, k_count, heads, needed);
    float* workspace = nullptr;
    hipError_t e = device_scratch(&workspace);
    if (e == hipSuccess)
        e = wsp::ops::attention(static_cast<hipStream_t>(stream), q, q_count, keys, values, k_count, width, heads,
                                causal, scale, out, workspace);
    if (e != hipSuccess)
        return report(error, error_capacity, WSP_ERR_HIP, "attention: %s", hipGetErrorString(e));
    return WSP_OK;
}
