// Host-side launchers of the per-op gfx950 kernels. Each returns the launch's
// hipError_t; argument checking is the C ABI's job (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wsp::ops
{
// Rows up to this count take the split GEMV; more take the tiled product
// (the reference's splitRowLimit, Net/KernelNet.h:144-149).
constexpr int kSplitRowLimit = 16;
constexpr int kMaxHeadWidth = 64;
constexpr int kAttentionChunkKeys = 1024; // longest key chunk one workgroup scores

hipError_t linear(hipStream_t stream, const float* x, int rows, int inner, const void* weight,
                  int wdtype, const float* bias, float* y, int out, int flags);

hipError_t layernorm(hipStream_t stream, const float* x, const float* gamma, const float* beta,
                     float* y, int rows, int width, float eps);

// Token ids at or past `vocabulary` poison their row with NaN.
hipError_t embed(hipStream_t stream, const uint32_t* tokens, int count, const float* token_table,
                 const float* position_table, int first_position, float* y, int width,
                 int vocabulary);

// How many key chunks the split-key attention uses for this shape, and the
// workspace (floats) it needs: chunks * (head_width + 2) per (head, query).
int attention_chunks(int heads, int q_count, int k_count);
size_t attention_workspace_floats(int heads, int q_count, int k_count, int head_width);

hipError_t attention(hipStream_t stream, const float* q, int q_count, const float* keys,
                     const float* values, int k_count, int width, int heads, int causal,
                     float scale, float* out, float* workspace);

int argmax_groups(int row_length);
hipError_t argmax(hipStream_t stream, const float* logits, int rows, int row_length,
                  const float* mask, uint32_t* out, float* partial_values,
                  uint32_t* partial_indices);
} // namespace wsp::ops
