// wsp_hip_decoder_step: one single-token decoder step plus its greedy argmax
// (Decoder/Decoder.cpp:151-177 followed by Whisper/Whisper.cpp:1164-1184).
//
// The step runs as one persistent cooperative launch (step_kernel.hip) when
// the shape fits its capacities; otherwise it is recorded as the per-op
// kernel sequence on the context's stream. This file sizes the persistent
// kernel's exchange area, chooses its work split per call and launches it.
#include "capi_internal.h"
#include "ops.h"
#include "step_kernel.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

namespace wsp
{
namespace
{
// Where a WSP_STEP_TIMELINE build writes each launch's timestamps (set with
// wsp_step_timeline; null otherwise).
uint64_t* step_timeline = nullptr;
} // namespace
} // namespace wsp

#ifdef WSP_STEP_TIMELINE
extern "C" void wsp_step_timeline(uint64_t* buffer)
{
    wsp::step_timeline = buffer;
}
#endif

namespace wsp
{
namespace
{
// Exchange areas live in uncached device memory: the device-scope stores and
// polls of a hand-over then skip the L2, and a width-long all-to-all among 224
// workgroups takes about 2.0 us instead of 2.3. Uncached memory that a kernel
// has read is never handed back to the HIP allocator (memory allocated after
// such a free has held wrong values on this platform): a released area waits
// in this process-wide pool, per device, for the next context's.
struct PooledArea
{
    int device;
    size_t bytes;
    void* memory;
};

std::mutex area_pool_mutex;
std::vector<PooledArea>& area_pool()
{
    static std::vector<PooledArea> pool;
    return pool;
}

// The smallest pooled area of this device holding `bytes`, else a new one.
// Sets *held to the area's size.
hipError_t acquire_area(int device, size_t bytes, void** out, size_t* held)
{
    {
        std::lock_guard<std::mutex> lock(area_pool_mutex);
        auto& pool = area_pool();
        auto best = pool.end();
        for (auto it = pool.begin(); it != pool.end(); ++it)
            if (it->device == device && it->bytes >= bytes && (best == pool.end() || it->bytes < best->bytes))
                best = it;
        if (best != pool.end())
        {
            *out = best->memory;
            *held = best->bytes;
            pool.erase(best);
            return hipSuccess;
        }
    }
    *held = bytes;
    if (hipExtMallocWithFlags(out, bytes, hipDeviceMallocUncached) == hipSuccess)
        return hipSuccess;
    // A device without uncached allocations: default memory, whose
    // device-scope accesses are coherent too, only slower to hand over.
    (void) hipGetLastError();
    return hipMalloc(out, bytes);
}

void release_area(int device, size_t bytes, void* memory)
{
    if (memory == nullptr)
        return;
    std::lock_guard<std::mutex> lock(area_pool_mutex);
    area_pool().push_back({device, bytes, memory});
}

struct FusedState
{
    // Per-op sequence scratch.
    float* hidden = nullptr;     // residual stream [width]
    float* normalised = nullptr; // [width]
    float* query = nullptr;      // [width]
    float* attended = nullptr;   // [width]
    float* inner = nullptr;      // [feed_forward_width]

    // Persistent kernel.
    bool persistent = false;
    char why_not[160] = {0};
    int workgroups = 0;
    int row_groups = 0;
    int self_split_max = 0;
    int cross_split_max = 0;
    int max_tokens = 1; // tokens one launch may carry (head groups for every (token, head) pair)
    int token_words = 0, layer_words = 0;
    int off_qkv = 0, off_self = 0, off_h2 = 0, off_xq = 0, off_xpart = 0, off_xattn = 0, off_h3 = 0, off_ff = 0,
        off_h4 = 0, off_argmax = 0;
    int log2_qkv = 0, log2_d = 0, log2_f = 0;
    uint64_t* exchange = nullptr; // uncached, from the area pool
    size_t exchange_words = 0;
    size_t exchange_held = 0; // bytes of the pooled area
    int* status = nullptr;
    wsp_layer_tensors* table = nullptr; // device copy
    std::vector<wsp_layer_tensors> table_host;
    bool table_valid = false;
    int table_wdtype = -1;
    float* fold_terms = nullptr; // the folded LayerNorms' per-row terms, layers x FoldTermsLayout::stride
    uint32_t epoch = 0;
};

// Per-row terms of a LayerNorm folded into the projection that consumes it
// (step_kernel.hip): gain_r = sum_i W_ri gamma_i and bias_r = b_r + sum_i
// W_ri beta_i, accumulated in double over the stored weights widened to
// float, and rounded once. One wave per row; a null bias counts as zero.
template <int WT>
__global__ void __launch_bounds__(256) fold_terms_kernel(const void* weight, const float* bias, const float* gamma,
                                                        const float* beta, int rows, int inner, float* gain_out,
                                                        float* bias_out)
{
    const int row = blockIdx.x * 4 + (int) (threadIdx.x / 64);
    const int lane = threadIdx.x & 63;
    if (row >= rows) // uniform over the wave
        return;
    double g = 0.0, c = 0.0;
    for (int i = lane; i < inner; i += 64)
    {
        const size_t at = (size_t) row * inner + i;
        float w;
        if constexpr (WT == WSP_F32)
            w = static_cast<const float*>(weight)[at];
        else if constexpr (WT == WSP_F16)
            w = (float) static_cast<const _Float16*>(weight)[at];
        else
            w = __uint_as_float((uint32_t) static_cast<const uint16_t*>(weight)[at] << 16);
        g += (double) w * (double) gamma[i];
        c += (double) w * (double) beta[i];
    }
    for (int offset = 32; offset > 0; offset >>= 1)
    {
        g += __shfl_xor(g, offset);
        c += __shfl_xor(c, offset);
    }
    if (lane == 0)
    {
        gain_out[row] = (float) g;
        bias_out[row] = (float) ((bias != nullptr ? (double) bias[row] : 0.0) + c);
    }
}

// Every layer's folded terms for this table, on the context's stream.
hipError_t compute_fold_terms(const wsp_decoder_shape& s, const wsp_layer_tensors* layers, int wdtype, float* terms,
                              hipStream_t stream)
{
    const int d = s.width, f = s.feed_forward_width;
    const step::FoldTermsLayout t = step::fold_terms_layout(d, f);
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = layers[l];
        float* T = terms + (size_t) l * t.stride;
        struct Job
        {
            const void* w;
            const float* b;
            const float* gamma;
            const float* beta;
            int rows;
            int gain, bias;
        } jobs[] = {{L.self_qkv_w, L.self_qkv_b, L.self_norm_w, L.self_norm_b, 3 * d, t.qkv_gain, t.qkv_bias},
                    {L.cross_q_w, L.cross_q_b, L.cross_norm_w, L.cross_norm_b, d, t.xq_gain, t.xq_bias},
                    {L.fc1_w, L.fc1_b, L.final_norm_w, L.final_norm_b, f, t.fc1_gain, t.fc1_bias}};
        for (const Job& j : jobs)
        {
            const dim3 grid((unsigned) ((j.rows + 3) / 4));
            switch (wdtype)
            {
                case WSP_F32:
                    hipLaunchKernelGGL(fold_terms_kernel<WSP_F32>, grid, dim3(256), 0, stream, j.w, j.b, j.gamma,
                                       j.beta, j.rows, d, T + j.gain, T + j.bias);
                    break;
                case WSP_F16:
                    hipLaunchKernelGGL(fold_terms_kernel<WSP_F16>, grid, dim3(256), 0, stream, j.w, j.b, j.gamma,
                                       j.beta, j.rows, d, T + j.gain, T + j.bias);
                    break;
                default:
                    hipLaunchKernelGGL(fold_terms_kernel<WSP_BF16>, grid, dim3(256), 0, stream, j.w, j.b, j.gamma,
                                       j.beta, j.rows, d, T + j.gain, T + j.bias);
                    break;
            }
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess)
                return e;
        }
    }
    return hipSuccess;
}

size_t element_bytes(int wdtype)
{
    return wdtype == WSP_F32 ? 4 : 2;
}

const void* offset(const void* base, size_t elements, int wdtype)
{
    return static_cast<const char*>(base) + elements * element_bytes(wdtype);
}

int ceil_div(int a, int b)
{
    return (a + b - 1) / b;
}

// Whether the persistent kernel can run this shape on this device, and its
// fixed layout. Leaves state->persistent false with the reason otherwise.
void plan_persistent(Context* ctx, FusedState* st)
{
    const wsp_decoder_shape& s = ctx->shape;
    const int d = s.width, f = s.feed_forward_width, H = s.heads, hd = d / H;
    auto refuse = [&](const char* why) {
        std::snprintf(st->why_not, sizeof(st->why_not), "%s", why);
        st->persistent = false;
    };
    if (d > step::kMaxWidth || f > step::kMaxFeedForward)
        return refuse("width or feed-forward width past the persistent kernel's capacity");
    if (d % 8 != 0 || f % 8 != 0)
        return refuse("widths must be multiples of 8");
    if (f / 4 > step::kMaxRowChunks)
        return refuse("feed-forward rows past the persistent kernel's capacity");
    if (hd % 4 != 0 || hd > step::kMaxHeadWidth)
        return refuse("head width must be a multiple of 4, at most 64");
    if (s.layers > step::kMaxLayers)
        return refuse("more layers than the persistent kernel's table holds");

    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, ctx->device) != hipSuccess)
        return refuse("device properties unavailable");
    int cooperative = 0;
    hipDeviceGetAttribute(&cooperative, hipDeviceAttributeCooperativeLaunch, ctx->device);
    if (!cooperative)
        return refuse("device has no cooperative launch");
    const int G = prop.multiProcessorCount;
    const int key_blocks = ceil_div(s.max_positions, step::kSelfKeys); // splits the longest sequence needs
    const int head_groups = H * key_blocks;
    // Row groups: the fewest in the top eighth of the CUs not holding a head
    // group whose width-long vectors' producer blocks fit two words per
    // polling thread (each poll round tests every slot a thread holds, so
    // rounds of two slots are the shortest). Fewer consumers make each
    // all-to-all hand-over cheaper; a projection's rows per workgroup grow by
    // at most an eighth (at the small shape 203 row groups ran 268.5 us/step
    // against 270.0 for 224). Spare workgroups run as idle head groups and
    // join the tied logits.
    int row_groups = G - head_groups;
    for (int rg = row_groups - row_groups / 8; rg <= row_groups && rg > 0; ++rg)
    {
        int block = 1;
        while (block < ceil_div(d, rg))
            block <<= 1;
        if (rg * block <= step::kPollBlocked * step::kPollThreads)
        {
            row_groups = rg;
            break;
        }
    }
    if (row_groups < H)
        return refuse("too few CUs for the head groups");
    {
        // A LayerNorm's input vector spans at most kFoldChunks poll chunks
        // (the polling threads hold gamma at that many slots).
        int block = 1;
        while (block < ceil_div(d, row_groups))
            block <<= 1;
        if (row_groups * block > step::kFoldChunks * step::kPollBlocked * step::kPollThreads)
            return refuse("width past the folded LayerNorm's poll capacity");
    }
    // The spare workgroups past the row groups split each head's keys further
    // when a position's keys allow (splits of at least kSelfSplitKeys keys).
    const int self_split_max =
        std::max(key_blocks, std::min((G - row_groups) / H, step::kMaxCombine / (H * (hd + 2))));
    if (self_split_max * H * (hd + 2) > step::kMaxCombine || 2 * G > step::kMaxCombine || G > 256)
        return refuse("attention partials past the combine capacity");
    const int cross_needed = ceil_div(s.cross_positions, step::kCrossKeys);
    const int cross_cap = std::min(step::kMaxCombine / (hd + 2), 64); // one wave folds the partials
    if (cross_needed > cross_cap)
        return refuse("cross positions past the persistent kernel's capacity");
    const int cross_split_max = std::min(cross_cap, std::max(cross_needed, row_groups / H));

    // Every kernel variant must fit one workgroup per CU.
    for (int wt : {WSP_F32, WSP_F16, WSP_BF16})
        for (bool multi : {false, true})
        {
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, step::kernel_for(wt, multi), step::kThreads,
                                                             0)
                    != hipSuccess
                || blocks < 1)
                return refuse("the persistent kernel does not fit a CU");
        }

    // Producer blocks: a row group's rows of a phase, rounded up to a power of two.
    auto block_log2 = [&](int rows) {
        const int per = ceil_div(rows, row_groups);
        int log2 = 0;
        while ((1 << log2) < per)
            ++log2;
        return log2;
    };
    st->log2_qkv = block_log2(3 * d);
    st->log2_d = block_log2(d);
    st->log2_f = block_log2(f);
    st->workgroups = G;
    st->row_groups = row_groups;
    st->self_split_max = self_split_max;
    st->cross_split_max = cross_split_max;
    int at = 0;
    const int block_d = row_groups << st->log2_d;
    st->off_qkv = at, at += row_groups << st->log2_qkv;
    st->off_self = at, at += self_split_max * H * (hd + 2);
    st->off_h2 = at, at += block_d;
    st->off_xq = at, at += block_d;
    st->off_xpart = at, at += H * cross_split_max * (hd + 2);
    st->off_xattn = at, at += d;
    st->off_h3 = at, at += block_d;
    st->off_ff = at, at += row_groups << st->log2_f;
    st->off_h4 = at, at += block_d;
    // Every layer holds kMaxTokens token blocks, so a multi-token launch
    // writes each token's words where a single-token launch writes token 0's.
    st->token_words = at;
    st->layer_words = step::kMaxTokens * at;
    st->off_argmax = st->layer_words * s.layers;
    st->exchange_words = (size_t) st->layer_words * s.layers + 16 * G;
    st->max_tokens = std::max(1, std::min(step::kMaxTokens, (G - row_groups) / H));
    st->persistent = true;
}

int per_op_step(Context* ctx, FusedState* st, const wsp_decoder_tensors* tensors, const uint32_t* tokens,
                int position, int cross_rows, float* hidden, float* logits, const float* mask,
                uint32_t* argmax_out)
{
    const wsp_decoder_shape& s = ctx->shape;
    const hipStream_t stream = ctx->stream;
    const int d = s.width, f = s.feed_forward_width;
    const int wt = tensors->wdtype;
    const float scale = 1.f / sqrtf((float) (s.width / s.heads));
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

bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// The fewest keys a self-attention split takes when spare head groups could
// split a head's keys further. One full block: at the small shape, splits of
// 128 keys ran 269 us/step and of 64 keys 276, against 261 unsplit (the row
// groups' combine of the partials costs more than the shorter chains save).
constexpr int kSelfSplitKeys = step::kSelfKeys;

// `count` tokens (1, or up to st->max_tokens with the multi-token kernel) at
// position .. position + count - 1.
int persistent_step(Context* ctx, FusedState* st, const wsp_decoder_tensors* tensors, const uint32_t* tokens,
                    int count, int position, int cross_rows, float* hidden, float* logits, const float* mask,
                    uint32_t* argmax_out)
{
    const wsp_decoder_shape& s = ctx->shape;
    const int d = s.width, H = s.heads, hd = d / H;

    // Every row the kernel streams in 16-byte chunks must start 16-byte aligned.
    if (!aligned16(tensors->logits_weight) || !aligned16(tensors->token_embedding))
        return context_fail(ctx, WSP_ERR_ARGUMENT, "decoder step: weights must be 16-byte aligned");
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = tensors->layers[l];
        const void* rows[] = {L.self_qkv_w, L.self_out_w, L.cross_q_w, L.cross_out_w, L.fc1_w, L.fc2_w,
                              L.self_keys, L.self_values, L.cross_keys, L.cross_values};
        for (const void* p : rows)
            if (p == nullptr || !aligned16(p))
                return context_fail(ctx, WSP_ERR_ARGUMENT, "decoder step: layer tensors must be 16-byte aligned");
    }

    // The per-layer table lives on the device; it is uploaded when it changes.
    const size_t table_bytes = sizeof(wsp_layer_tensors) * (size_t) s.layers;
    if (!st->table_valid || st->table_wdtype != tensors->wdtype
        || std::memcmp(st->table_host.data(), tensors->layers, table_bytes) != 0)
    {
        // A table with the same pointers is taken to hold the same weights, so
        // the folded LayerNorms' terms are computed when the table changes.
        st->table_valid = false;
        st->table_host.assign(tensors->layers, tensors->layers + s.layers);
        hipError_t e = hipMemcpyAsync(st->table, st->table_host.data(), table_bytes, hipMemcpyHostToDevice,
                                      ctx->stream);
        if (e == hipSuccess)
            e = compute_fold_terms(s, st->table_host.data(), tensors->wdtype, st->fold_terms, ctx->stream);
        if (e != hipSuccess)
            return context_hip(ctx, e, "decoder step: layer table upload");
        st->table_wdtype = tensors->wdtype;
        const hipError_t w = hipStreamSynchronize(ctx->stream);
        if (w != hipSuccess)
            return context_hip(ctx, w, "decoder step: layer table upload");
        st->table_valid = true;
    }

    // The work split of this call.
    // Self-attention key splits: as many blocks of kSelfKeys as the keys
    // need, more (down to kSelfSplitKeys keys each) where head groups allow;
    // a multi-token launch keeps one.
    int self_splits = ceil_div(position + 1, step::kSelfKeys);
    if (count == 1)
        self_splits = std::min(st->self_split_max, std::max(self_splits, ceil_div(position + 1, kSelfSplitKeys)));
    const int self_chunk = ceil_div(position + 1, self_splits);
    // As few cross-attention chunks as the per-task key capacity allows: the
    // head's combine then polls the fewest partials (at 1500 keys, 12 chunks of
    // 125 ran 269 us/step against 273 for 18 chunks of 84).
    int cross_splits = std::max(1, ceil_div(cross_rows, step::kCrossKeys));
    cross_splits = std::min(cross_splits, st->cross_split_max);
    const int cross_chunk = ceil_div(cross_rows, cross_splits);
    cross_splits = ceil_div(cross_rows, cross_chunk);
    if (cross_chunk > step::kCrossKeys || self_splits > st->self_split_max)
        return context_fail(ctx, WSP_ERR_CAPACITY, "decoder step: attention split past the planned capacity");
    if (count > 1
        && (count > st->max_tokens || position + count > step::kSelfKeys
            || count * cross_splits * (hd + 2) > step::kMaxCombine))
        return context_fail(ctx, WSP_ERR_LOGIC, "decoder step: tokens past the multi-token kernel's capacity");

    step::StepArgs a {};
    a.layers = st->table;
    a.token_embedding = tensors->token_embedding;
    a.logits_weight = tensors->logits_weight;
    a.position_embedding = tensors->position_embedding;
    a.final_norm_w = tensors->final_norm_w;
    a.final_norm_b = tensors->final_norm_b;
    a.tokens = tokens;
    a.hidden = hidden;
    a.logits = logits;
    a.mask = mask;
    a.argmax_out = argmax_out;
    a.host_pair = argmax_out != nullptr ? ctx->armed_report : nullptr;
    a.exchange = st->exchange;
    a.status = st->status;
    a.width = d;
    a.heads = H;
    a.layer_count = s.layers;
    a.feed_forward = s.feed_forward_width;
    a.vocabulary = s.vocabulary_size;
    a.logits_wdtype = tensors->logits_wdtype;
    a.position = position;
    a.cross_rows = cross_rows;
    a.token_count = count;
    a.row_groups = st->row_groups;
    a.self_splits = self_splits;
    a.self_chunk = self_chunk;
    a.cross_splits = cross_splits;
    a.cross_chunk = cross_chunk;
    a.epoch = ++st->epoch;
    a.scale = 1.f / sqrtf((float) hd);
    a.eps = 1e-5f;
    a.inv_width = 1.f / (float) s.width;
    a.off_qkv = st->off_qkv;
    a.off_self = st->off_self;
    a.off_h2 = st->off_h2;
    a.off_xq = st->off_xq;
    a.off_xpart = st->off_xpart;
    a.off_xattn = st->off_xattn;
    a.off_h3 = st->off_h3;
    a.off_ff = st->off_ff;
    a.off_h4 = st->off_h4;
    a.token_words = st->token_words;
    a.layer_words = st->layer_words;
    a.off_argmax = st->off_argmax;
    a.log2_qkv = st->log2_qkv;
    a.log2_d = st->log2_d;
    a.log2_f = st->log2_f;
    a.timeline = step_timeline;
    const step::FoldTermsLayout terms = step::fold_terms_layout(d, s.feed_forward_width);
    a.fold_terms = st->fold_terms;
    a.terms_stride = terms.stride;
    a.terms_qkv_gain = terms.qkv_gain;
    a.terms_qkv_bias = terms.qkv_bias;
    a.terms_xq_gain = terms.xq_gain;
    a.terms_xq_bias = terms.xq_bias;
    a.terms_fc1_gain = terms.fc1_gain;
    a.terms_fc1_bias = terms.fc1_bias;

    // A plain launch: the grid is one workgroup per CU, a CU holds only one of
    // these workgroups (registers), and the stream runs kernels one after
    // another, so every workgroup is resident at once on a GPU this process
    // has to itself. A cooperative launch guarantees the same but adds about
    // 20 us per step; WSP_STEP_LAUNCH=cooperative asks for it (a GPU shared
    // with other work). Either way every wait in the kernel is bounded.
    void* args[] = {&a};
    static const bool cooperative =
        getenv("WSP_STEP_LAUNCH") != nullptr && strcmp(getenv("WSP_STEP_LAUNCH"), "cooperative") == 0;
    const hipError_t e = cooperative
                             ? hipLaunchCooperativeKernel(step::kernel_for(tensors->wdtype, count > 1),
                                                          dim3(st->workgroups), dim3(step::kThreads), args, 0,
                                                          ctx->stream)
                             : hipLaunchKernel(step::kernel_for(tensors->wdtype, count > 1), dim3(st->workgroups),
                                               dim3(step::kThreads), args, 0, ctx->stream);
    if (e == hipSuccess && a.host_pair != nullptr)
    {
        ctx->reported = a.host_pair;
        ctx->armed_report = nullptr;
    }
    return context_hip(ctx, e, "decoder step launch");
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
    int status = context_hip(ctx, hipMalloc(&state->inner, f * sizeof(float)), "fused step scratch");
    if (status != WSP_OK)
        return status;

    plan_persistent(ctx, state);
    if (!state->persistent)
        return WSP_OK;
    void* area = nullptr;
    status = context_hip(ctx, acquire_area(ctx->device, state->exchange_words * sizeof(uint64_t), &area,
                                           &state->exchange_held),
                         "step exchange area");
    state->exchange = static_cast<uint64_t*>(area);
    if (status == WSP_OK)
        status = context_hip(ctx, hipMalloc(&state->status, sizeof(int)), "step status word");
    if (status == WSP_OK)
        status = context_hip(ctx,
                             hipMalloc(&state->table, sizeof(wsp_layer_tensors) * (size_t) ctx->shape.layers),
                             "step layer table");
    if (status == WSP_OK)
        status = context_hip(ctx,
                             hipMalloc(&state->fold_terms,
                                       sizeof(float) * (size_t) ctx->shape.layers
                                           * (size_t) step::fold_terms_layout(ctx->shape.width,
                                                                              ctx->shape.feed_forward_width)
                                                 .stride),
                             "step folded LayerNorm terms");
    // Epoch 0 is never used, so zeroed words never pass for a step's output
    // (a pooled area also holds a previous context's epochs until cleared).
    if (status == WSP_OK)
        status = context_hip(ctx, hipMemset(state->exchange, 0, state->exchange_words * sizeof(uint64_t)),
                             "step exchange area");
    if (status == WSP_OK)
        status = context_hip(ctx, hipMemset(state->status, 0, sizeof(int)), "step status word");
    return status;
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
    release_area(ctx->device, state->exchange_held, state->exchange);
    hipFree(state->status);
    hipFree(state->table);
    hipFree(state->fold_terms);
    delete state;
    ctx->fused = nullptr;
}

bool fused_persistent(const Context* ctx)
{
    const auto* state = static_cast<const FusedState*>(ctx->fused);
    return state != nullptr && state->persistent;
}

int fused_status(Context* ctx, int* status, int clear)
{
    auto* state = static_cast<FusedState*>(ctx->fused);
    *status = 0;
    if (state == nullptr || state->status == nullptr)
        return WSP_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpy(status, state->status, sizeof(int), hipMemcpyDeviceToHost);
    if (e == hipSuccess && clear && *status != 0)
        e = hipMemset(state->status, 0, sizeof(int));
    return context_hip(ctx, e, "step status word");
}

int fused_status_copy(Context* ctx, int* dst)
{
    auto* state = static_cast<FusedState*>(ctx->fused);
    if (state == nullptr || state->status == nullptr)
    {
        *dst = 0;
        return WSP_OK;
    }
    return context_hip(ctx, hipMemcpyAsync(dst, state->status, sizeof(int), hipMemcpyDeviceToHost, ctx->stream),
                       "step status word");
}

// A sampled token and the watchdog word into pinned host memory: one thread,
// system-scope stores, so the host reads both behind one event.
__global__ void report_kernel(const uint32_t* slot, const int* status, int* host_pair)
{
    const int token = (int) __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int word = status != nullptr ? __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    __hip_atomic_store(host_pair, token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(host_pair + 1, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

int fused_report(Context* ctx, const uint32_t* slot, int* host_pair)
{
    ctx->armed_report = nullptr;
    if (ctx->reported == host_pair) // the persistent step wrote it when it ended
    {
        ctx->reported = nullptr;
        return WSP_OK;
    }
    auto* state = static_cast<FusedState*>(ctx->fused);
    const int* status = state != nullptr ? state->status : nullptr;
    hipLaunchKernelGGL(report_kernel, dim3(1), dim3(1), 0, ctx->stream, slot, status, host_pair);
    return context_hip(ctx, hipGetLastError(), "step report");
}

int fused_raise_status(Context* ctx)
{
    auto* state = static_cast<FusedState*>(ctx->fused);
    if (state == nullptr || state->status == nullptr)
        return context_fail(ctx, WSP_ERR_LOGIC, "the context runs no persistent step");
    static const int tripped = 1;
    hipError_t e = hipMemcpyAsync(state->status, &tripped, sizeof(int), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    return context_hip(ctx, e, "step status word");
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
    if (st->persistent)
        return persistent_step(ctx, st, tensors, tokens, 1, position, cross_rows, hidden, logits, mask, argmax_out);
    return per_op_step(ctx, st, tensors, tokens, position, cross_rows, hidden, logits, mask, argmax_out);
}

extern "C" int wsp_hip_decoder_step_tokens(wsp_hip_ctx* ctx, const wsp_decoder_tensors* tensors,
                                           const uint32_t* tokens, int token_count, int position, int cross_rows,
                                           float* hidden, float* logits, const float* mask, uint32_t* argmax_out)
{
    using namespace wsp;
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    if (tensors == nullptr || tensors->layers == nullptr || tokens == nullptr || hidden == nullptr
        || logits == nullptr || token_count <= 0)
        return context_fail(ctx, WSP_ERR_ARGUMENT, "decoder step: null pointer or no tokens");
    const wsp_decoder_shape& s = ctx->shape;
    if (position < 0 || position + token_count > s.max_positions)
        return context_fail(ctx, WSP_ERR_CAPACITY, "decoder step: position past the window");
    if (cross_rows <= 0 || cross_rows > s.cross_positions)
        return context_fail(ctx, WSP_ERR_CAPACITY, "decoder step: cross rows outside the encoder output");
    const int head_width = s.width / s.heads;
    if (head_width % 4 != 0 || head_width > ops::kMaxHeadWidth)
        return context_fail(ctx, WSP_ERR_LOGIC, "decoder step: unsupported head width");

    // Launches of as many tokens as the multi-token kernel takes at their
    // position (one where the self keys would leave its key block, or the
    // cross partials its combine capacity); each sees the keys the ones
    // before it appended. Only the last launch writes the argmax.
    auto* st = static_cast<FusedState*>(ctx->fused);
    const size_t d = (size_t) s.width, V = (size_t) s.vocabulary_size;
    int cross_splits = std::max(1, ceil_div(cross_rows, step::kCrossKeys));
    if (st->persistent)
        cross_splits = std::min(cross_splits, st->cross_split_max);
    for (int done = 0; done < token_count;)
    {
        const int at = position + done;
        int n = 1;
        if (st->persistent)
        {
            n = std::min(token_count - done, st->max_tokens);
            n = std::min(n, step::kMaxCombine / (cross_splits * (head_width + 2)));
            if (at + n > step::kSelfKeys || (head_width & (head_width - 1)) != 0)
                n = 1;
            n = std::max(n, 1);
        }
        const bool last = done + n == token_count;
        const int status =
            st->persistent
                ? persistent_step(ctx, st, tensors, tokens + done, n, at, cross_rows, hidden + done * d,
                                  logits + done * V, last ? mask : nullptr, last ? argmax_out : nullptr)
                : per_op_step(ctx, st, tensors, tokens + done, at, cross_rows, hidden + done * d, logits + done * V,
                              last ? mask : nullptr, last ? argmax_out : nullptr);
        if (status != WSP_OK)
            return status;
        done += n;
    }
    return WSP_OK;
}

extern "C" int wsp_hip_step_persistent(const wsp_hip_ctx* ctx)
{
    return ctx != nullptr && wsp::fused_persistent(ctx) ? 1 : 0;
}

extern "C" int wsp_hip_device_status(wsp_hip_ctx* ctx, int* status, int clear)
{
    if (ctx == nullptr || status == nullptr)
        return WSP_ERR_ARGUMENT;
    return wsp::fused_status(ctx, status, clear);
}

extern "C" int wsp_hip_device_status_copy(wsp_hip_ctx* ctx, int* dst)
{
    if (ctx == nullptr || dst == nullptr)
        return WSP_ERR_ARGUMENT;
    return wsp::fused_status_copy(ctx, dst);
}

extern "C" int wsp_hip_step_report(wsp_hip_ctx* ctx, const uint32_t* slot, int* host_pair)
{
    if (ctx == nullptr || slot == nullptr || host_pair == nullptr)
        return WSP_ERR_ARGUMENT;
    return wsp::fused_report(ctx, slot, host_pair);
}

extern "C" int wsp_hip_step_report_next(wsp_hip_ctx* ctx, int* host_pair)
{
    if (ctx == nullptr || host_pair == nullptr)
        return WSP_ERR_ARGUMENT;
    ctx->armed_report = host_pair;
    ctx->reported = nullptr;
    return WSP_OK;
}

extern "C" int wsp_hip_raise_device_status(wsp_hip_ctx* ctx)
{
    if (ctx == nullptr)
        return WSP_ERR_ARGUMENT;
    return wsp::fused_raise_status(ctx);
}
