// The persistent single-token step kernel (step_kernel.hip): its capacities and
// its argument block. The host side (fused_step.hip) sizes the exchange area,
// picks the work split and launches it cooperatively.
#pragma once

#include "../../include/wsp_hip.h"

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wsp::step
{
constexpr int kThreads = 512;          // one workgroup per CU, 8 waves
constexpr int kMaxWidth = 1280;        // d_model
constexpr int kMaxFeedForward = 5120;  // fc1 width
constexpr int kMaxHeadWidth = 64;
constexpr int kMaxCombine = 4096;      // attention partial floats one workgroup combines
constexpr int kSelfKeys = 256;         // self-attention keys one head group holds
constexpr int kCrossKeys = 128;        // cross-attention keys one row group holds
constexpr int kMaxLayers = 32;         // layer table entries held in LDS
constexpr int kPollThreads = kThreads - 64; // threads that poll exchange words (waves 1-7)
constexpr int kPollBlocked = 2;        // slots per polling thread for a width-long vector, per chunk
constexpr int kPollBlockedFF = 8;      // ... for the feed-forward vector
constexpr int kFoldChunks = 2;         // chunks of kPollBlocked * kPollThreads slots a LayerNorm's input may span
constexpr int kMaxTokens = 4;          // tokens one multi-token launch carries (their rows share each weight load)

// Exchange words per token and layer, in this order (offsets in StepArgs; a
// layer holds kMaxTokens such blocks, token_words apart):
//   qkv [row_groups << log2_qkv] | self partials [self_split_max][heads][hd + 2]
//   | h2 [row_groups << log2_d] | xq [row_groups << log2_d]
//   | cross partials [heads][cross_split_max][hd + 2] | xattn [d]
//   | h3 [row_groups << log2_d] | ff [row_groups << log2_f] | h4 [row_groups << log2_d]
// followed by one argmax block [16 * workgroups] after the last layer (its
// first 2 * workgroups words: a (value, index) candidate per workgroup). A
// row-group vector keeps each producing workgroup's rows in a block of its own
// (2^log2 words: the workgroup's rows-per-phase rounded up to a power of two).
struct StepArgs
{
    const wsp_layer_tensors* layers; // device copy of the per-layer table
    const float* token_embedding;
    const void* logits_weight;
    const float* position_embedding;
    const float* final_norm_w;
    const float* final_norm_b;
    const uint32_t* tokens;
    float* hidden;
    float* logits;
    const float* mask;
    uint32_t* argmax_out;
    int* host_pair;     // with argmax_out: the token and the watchdog word, written to pinned host memory, or null
    uint64_t* exchange;
    int* status;

    int width, heads, layer_count, feed_forward, vocabulary, logits_wdtype;
    int position, cross_rows;
    int token_count;    // tokens of this launch (1 for the single-token kernel, else 1..kMaxTokens)
    int row_groups;     // workgroups [0, row_groups) run projections and cross chunks
    int self_splits;    // key splits per head for this position (<= self_split_max)
    int self_chunk;     // keys per split (<= kSelfKeys); split s holds keys [s * self_chunk, ...)
    int cross_splits;   // key chunks per head
    int cross_chunk;    // keys per chunk (<= kCrossKeys)
    uint32_t epoch;
    float scale, eps;
    float inv_width; // 1 / width, the LayerNorm mean factor

    int off_qkv, off_self, off_h2, off_xq, off_xpart, off_xattn, off_h3, off_ff, off_h4;
    int token_words, layer_words, off_argmax;
    int log2_qkv, log2_d, log2_f; // producer block sizes of the row-group vectors
    uint64_t* timeline; // per-workgroup timestamps of a WSP_STEP_TIMELINE build (else unused)

    // The folded LayerNorms' per-row terms (fold_terms_kernel): per layer
    // terms_stride floats, holding for the q/k/v, cross-query and fc1 rows
    // gain_r = sum_i W_ri gamma_i and bias_r = b_r + sum_i W_ri beta_i of the
    // LayerNorm each consumes, at these offsets.
    const float* fold_terms;
    int terms_stride;
    int terms_qkv_gain, terms_qkv_bias, terms_xq_gain, terms_xq_bias, terms_fc1_gain, terms_fc1_bias;
};

// The folded terms' layout for a shape (floats; see StepArgs::fold_terms).
struct FoldTermsLayout
{
    int stride, qkv_gain, qkv_bias, xq_gain, xq_bias, fc1_gain, fc1_bias;
};

inline FoldTermsLayout fold_terms_layout(int width, int feed_forward)
{
    FoldTermsLayout t {};
    t.qkv_gain = 0;
    t.qkv_bias = 3 * width;
    t.xq_gain = 6 * width;
    t.xq_bias = 7 * width;
    t.fc1_gain = 8 * width;
    t.fc1_bias = 8 * width + feed_forward;
    t.stride = 8 * width + 2 * feed_forward;
    return t;
}

// Longest projection row, in 16-byte chunks: 16 slices of 3 chunks per lane.
constexpr int kMaxRowChunks = 16 * 32 * 3;

// The kernel for this projection storage (the logits storage is an argument),
// carrying one token or up to kMaxTokens.
const void* kernel_for(int wdtype, bool multi_token);
} // namespace wsp::step
