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

// The matrix-core tall product (mfma_product.hip): y = X·Wᵀ (+ bias, GELU,
// residual as in `flags`) for fp32 X [rows, inner] and 16-bit W. Output
// columns n < split read W rows from w0 and write y0 (bias0); the rest read
// w1 row n - split and write y1 (bias1) — the key and value projections in one
// launch. Output row r of column c lands at
// (r / rows_per_group)·group_stride + (r % rows_per_group)·ldy + c.
struct TileProduct
{
    const float* x;
    int rows, inner;
    // Up to three weight matrices side by side: columns [0, split) read w0,
    // [split, split2) w1 and [split2, out) w2, each with its bias and output
    // (split2 0: two matrices, w1 running to out).
    const void* w0;
    const void* w1;
    int split, out;
    const float* bias0;
    const float* bias1;
    float* y0;
    float* y1;
    int ldy;
    int rows_per_group;
    size_t group_stride;
    int flags;
    int wdtype;
    const void* w2;
    const float* bias2;
    float* y2;
    int split2;
};

// 16-bit weights, inner % 32 == 0, out and split (and split2) multiples of
// 128, X 16-byte aligned.
bool tile_product_fits(int wdtype, int inner, int out, int split, const void* x);
hipError_t tile_product(hipStream_t stream, const TileProduct& product);

hipError_t layernorm(hipStream_t stream, const float* x, const float* gamma, const float* beta,
                     float* y, int rows, int width, float eps);

// The encoder's products over pre-split activations (split_product.hip):
// y = X·Wᵀ where X [rows, inner] is held as exact 16-bit parts (three bf16
// parts for bf16 W, fp16 hi + lo for fp16 W), part p at
// parts + p·part_stride + r·inner. Columns [0, split) read w0 (bias0, y0),
// [split, split2) w1 and [split2, out) w2, each matrix's own column index c;
// row r of a column lands at y·[r·ldy + c] (+= with kProductResidual, after
// GELU with kProductGelu), or, with out_parts set, as the parts of the value
// (one matrix only, rows of `out` values, part p at out_parts + p·out_part_stride).
constexpr int kProductGelu = 1;
constexpr int kProductResidual = 2;
struct SplitProduct
{
    const void* parts;
    size_t part_stride;
    int rows, inner;
    const void* w0;
    const void* w1;
    const void* w2;
    int split, split2, out;
    const float* bias0;
    const float* bias1;
    const float* bias2;
    float* y0;
    float* y1;
    float* y2;
    int ldy;
    int flags;
    void* out_parts;
    size_t out_part_stride;
    int wdtype;
    // Columns [split, split2) (y1_halves) and [split2, out) (y2_halves_t), when
    // set, go out as fp16 hi = fp16(v) and lo = fp16(v - hi) instead of fp32:
    // hi of row r, column c at y1_halves[r·width + c], lo halves_pitch·width
    // further; y2_halves_t transposed, hi at [c·halves_pitch + r]. (The
    // encoder's keys and values for its attention.)
    void* y1_halves;
    void* y2_halves_t;
    int halves_pitch;
    // Each matrix's sums are multiplied by its factor before the bias: the
    // reciprocal of the power of two its stored weights carry (exact), 1 for
    // weights stored as they are.
    float scale0 = 1.f, scale1 = 1.f, scale2 = 1.f;
};

// 16-bit weights, inner % 32 == 0, out, split and split2 multiples of 128.
bool split_product_fits(int wdtype, int inner, int out, int split, int split2);
hipError_t split_product(hipStream_t stream, const SplitProduct& product);
// LayerNorm rows (as layernorm) written as the parts of split_product's input;
// widths that are multiples of 4 up to 2048 (layernorm_parts_fits).
bool layernorm_parts_fits(int width);
hipError_t layernorm_parts(hipStream_t stream, const float* x, const float* gamma, const float* beta, void* parts,
                           size_t part_stride, int rows, int width, float eps, int wdtype);
// count fp32 values (a multiple of 8) as parts for 16-bit weights of wdtype.
hipError_t split_rows(hipStream_t stream, const float* x, size_t count, int wdtype, void* parts,
                      size_t part_stride);

// Token ids at or past `vocabulary` poison their row with NaN.
hipError_t embed(hipStream_t stream, const uint32_t* tokens, int count, const float* token_table,
                 const float* position_table, int first_position, float* y, int width,
                 int vocabulary);

// Queries a prompt step's attention takes in one launch (prompt_attention).
constexpr int kMaxPromptQueries = 16;
// The attention workspace starts with this many per-head counters (the
// prompt attention's last-block election); they are zero between launches,
// and whoever provides a workspace zeroes them once before its first use.
constexpr int kAttentionCounters = 256;

// How many key chunks the split-key attention uses for this shape, and the
// workspace (floats) it needs: the counters, then the partials —
// chunks * (head_width + 2) per (head, query) for one query or more than
// kMaxPromptQueries, splits * kMaxPromptQueries * (kMaxHeadWidth + 2) per head
// for a prompt step.
int attention_chunks(int heads, int q_count, int k_count);
int prompt_attention_splits(int heads, int k_count);
size_t attention_workspace_floats(int heads, int q_count, int k_count, int head_width);

hipError_t attention(hipStream_t stream, const float* q, int q_count, const float* keys,
                     const float* values, int k_count, int width, int heads, int causal,
                     float scale, float* out, float* workspace);

int argmax_groups(int row_length);
hipError_t argmax(hipStream_t stream, const float* logits, int rows, int row_length,
                  const float* mask, uint32_t* out, float* partial_values,
                  uint32_t* partial_indices);

// The same over rows `row_stride` floats apart.
hipError_t argmax_rows(hipStream_t stream, const float* logits, int rows, size_t row_stride,
                       int row_length, const float* mask, uint32_t* out, float* partial_values,
                       uint32_t* partial_indices);
} // namespace wsp::ops
