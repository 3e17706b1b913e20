// The context behind wsp_hip_ctx and the internal entry points the C ABI
// shares between its translation units.
#pragma once

#include "../../include/wsp_hip.h"

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct wsp_hip_ctx
{
    wsp_decoder_shape shape {};
    int device = 0;
    hipStream_t stream = nullptr;

    float* attention_workspace = nullptr;
    size_t attention_floats = 0;

    float* argmax_values = nullptr;
    uint32_t* argmax_indices = nullptr;
    size_t argmax_candidates = 0;

    void* fused = nullptr; // fused-step state (fused_step.hip)

    // wsp_hip_step_report_next: the host pair the next sampling step writes
    // (armed), and the one the last persistent step took over (reported).
    int* armed_report = nullptr;
    int* reported = nullptr;

    char error[512] = {0};
};

namespace wsp
{
using Context = wsp_hip_ctx;

int context_fail(Context* ctx, int code, const char* message);
int context_hip(Context* ctx, hipError_t e, const char* what);

// fused_step.hip
int fused_prepare(Context* ctx);
void fused_release(Context* ctx);
bool fused_persistent(const Context* ctx);
int fused_status(Context* ctx, int* status, int clear);
int fused_status_copy(Context* ctx, int* dst);
int fused_raise_status(Context* ctx);
int fused_report(Context* ctx, const uint32_t* slot, int* host_pair);

// cross_kv.hip: K = X·Wkᵀ and V = X·Wvᵀ + bv for `rows` rows of `width`.
int cross_kv_projection(Context* ctx, const float* x, int rows, int width, const void* wk, const void* wv,
                        const float* bv, int wdtype, float* k_out, float* v_out);
} // namespace wsp
