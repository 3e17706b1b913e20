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
#include <climits>
#include <cmath>
#include <cstdio>
#include <new>
#include <vector>

namespace wsp::encoder
{
namespace
{
constexpr int kColumnThreads = 256;
constexpr int kFlashWaves = 4;     // queries per attention block: 16 per wave
constexpr int kFlashWideWaves = 8; // the same with twice the queries per K/V tile, when the blocks still fill the chip
constexpr int kMaxFlashSplits = 4; // key splits of the attention when its 64-query blocks leave CUs idle

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

// ---------------------------------------------------------------------------
// Self attention of the encoder (Tests/Encoder/Common.h:547-594: every query
// sees every key, softmax(scale q.k) v per head) for head width 64, on the
// matrix cores, one pass over the keys with an online softmax.
//
// A block takes 16 queries per wave of one head; key tiles of 64 rows of K
// and V go through LDS once for all its waves (a large-v3 window took 12.19
// ms with 64-key tiles, 12.33 with 32, 12.30 with 128: half the barriers and
// softmax passes of 32, fewer registers than 128).
// Every fp32 operand is cut into fp16 parts, hi = fp16(x) and
// lo = fp16(x - hi), and a product takes
// the three terms hi·hi + hi·lo + lo·hi (v_mfma_f32_16x16x32_f16, fp32
// accumulation): what is dropped, lo·lo, is about 2^-22 of the product, so
// the sums stay at fp32 rather than fp16 accuracy.
//
// Layout: the wave computes S^T = K·Q^T, so lane (g, l) holds the scores of
// keys 4g..4g+3 and 16+4g..16+4g+3 of each 32-key block of the tile for
// query l — exactly the B operand of O^T = V^T·P^T once the key order
// inside each 32-key block is taken as (4g..4g+3, 16+4g..16+4g+3) for both
// operands, so P
// never leaves its registers. V is staged transposed for that A operand.
// Scores are in base-2 units (scale·log2 e folded in); each new tile
// rescales the running row by exp2(m_old - m_new) (exact online softmax).
// ---------------------------------------------------------------------------
constexpr int kFlashKeys = 64;
constexpr int kFlashWidth = 64;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ _Float16 half_hi(float x)
{
    return (_Float16) x;
}

__device__ __forceinline__ _Float16 half_lo(float x)
{
    return (_Float16) (x - (float) (_Float16) x);
}

__device__ __forceinline__ f32x4 mfma3(const f16x8& ah, const f16x8& al, const f16x8& bh, const f16x8& bl, f32x4 c)
{
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
}

int compute_units()
{
    static const int units = [] {
        int device = 0, count = 0;
        if (hipGetDevice(&device) == hipSuccess
            && hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && count > 0)
            return count;
        return 256;
    }();
    return units;
}

// Key splits: blockIdx.z takes keys [z·span, min((z + 1)·span, count)); with
// one split the block writes the normalised rows to out (OUT = kF32) or as
// the exact 16-bit parts of the output product's input (OUT = kF16, kBF16:
// part p at out_parts + p·out_part_stride), with several it writes (max, sum,
// row) partials [split][head][query][66] for flash_combine_kernel.
// With PRESPLIT, K and V arrive already cut into fp16 hi and lo by the q/k/v
// product (k_halves [2][pitch][width], vt_halves transposed [2][width][pitch],
// pitch a multiple of the key tile and zero past count), so a tile's staging
// is a copy; otherwise the fp32 k and v are cut here.
template <int WAVES, bool PRESPLIT = false, int OUT = kF32>
__global__ void __launch_bounds__(WAVES * 64) flash_attention_kernel(const float* __restrict__ q,
                                                                    const float* __restrict__ k,
                                                                    const float* __restrict__ v, int count,
                                                                    int width, float scale2, float* __restrict__ out,
                                                                    int span, float* __restrict__ partials,
                                                                    const uint16_t* __restrict__ k_halves,
                                                                    const uint16_t* __restrict__ vt_halves, int pitch,
                                                                    uint16_t* __restrict__ out_parts,
                                                                    size_t out_part_stride)
{
    constexpr int kThreadsHere = WAVES * 64;
    constexpr int kUnits = kFlashKeys * kFlashWidth / 4; // float4 runs of a K (or V) tile
    constexpr int kPerThread = (kUnits + kThreadsHere - 1) / kThreadsHere;
    constexpr int kHalfChunks = 2 * kFlashKeys * kFlashWidth / 8; // 16-byte runs of a tile's K (or V) halves
    constexpr int KB = kFlashKeys / 32;                           // 32-key blocks of a tile (P·V k-steps)
    constexpr int kHalfPerThread = kHalfChunks / kThreadsHere;
    static_assert(kHalfChunks % kThreadsHere == 0, "whole half runs per thread");
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][kFlashKeys][kFlashWidth + 8];
    // V^T rows padded by four halves (a pitch of 34 words): the 8-byte operand
    // reads of 16 lanes (rows li) then land on 16 distinct bank pairs; K's
    // 16-byte reads of 8 lanes need a pitch of 4 words mod 32 (72 halves).
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][kFlashWidth][kFlashKeys + 4];

    const int head = blockIdx.y;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, li = lane % 16, g = lane / 16;
    const int column = head * kFlashWidth;
    const int query = blockIdx.x * 16 * WAVES + 16 * wave + li;
    const bool query_in = query < count;
    const int k_begin = (int) blockIdx.z * span, k_end = min(count, k_begin + span);

    // This lane's B fragments of Q^T: query `query`, dims 32 s + 8 g .. + 7.
    f16x8 qh[2], ql[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
    {
        const float* src = q + (size_t) min(query, count - 1) * width + column + 32 * s + 8 * g;
        const f32x4 a = *reinterpret_cast<const f32x4*>(src);
        const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            qh[s][e] = half_hi(a[e]);
            ql[s][e] = half_lo(a[e]);
            qh[s][4 + e] = half_hi(b[e]);
            ql[s][4 + e] = half_lo(b[e]);
        }
    }

    float m = -INFINITY, l = 0.f;
    f32x4 o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        o[t] = f32x4 {0.f, 0.f, 0.f, 0.f};

    // K and V runs of a tile, loaded two tiles ahead of its use into one of
    // two register stages (a tile past the end reloads the last keys, unused).
    struct Stage
    {
        f32x4 k[kPerThread], v[kPerThread];
        u32x4 kh[kHalfPerThread], vh[kHalfPerThread];
    };
    // Run i of this thread in a tile of halves: part, then K row and 8-column
    // block, or V^T row (channel) and 8-key block.
    auto half_run = [&](int i, int& part, int& a, int& b, int& c, int& kb) {
        const int unit = (int) threadIdx.x + i * kThreadsHere;
        const int rest = unit % (kHalfChunks / 2);
        part = unit / (kHalfChunks / 2);
        a = rest / (kFlashWidth / 8);
        b = rest % (kFlashWidth / 8);
        c = rest / (kFlashKeys / 8);
        kb = rest % (kFlashKeys / 8);
    };
    const int last_first = k_begin + (max(k_end - k_begin, 1) - 1) / kFlashKeys * kFlashKeys;
    const size_t halves_part = (size_t) pitch * width;
    auto load_tile = [&](Stage& st, int first) {
        if constexpr (PRESPLIT)
        {
            const int f = min(first, last_first);
#pragma unroll
            for (int i = 0; i < kHalfPerThread; ++i)
            {
                int part, row, cb, c, kb;
                half_run(i, part, row, cb, c, kb);
                st.kh[i] = *reinterpret_cast<const u32x4*>(k_halves + part * halves_part + (size_t) (f + row) * width
                                                           + column + 8 * cb);
                st.vh[i] = *reinterpret_cast<const u32x4*>(vt_halves + part * halves_part
                                                           + (size_t) (column + c) * pitch + f + 8 * kb);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < kPerThread; ++i)
        {
            const int unit = (int) threadIdx.x + i * kThreadsHere;
            const int key = first + (unit % kUnits) / 16, d4 = 4 * (unit % 16);
            const size_t at = (size_t) min(key, k_end - 1) * width + column + d4;
            st.k[i] = *reinterpret_cast<const f32x4*>(k + at);
            st.v[i] = *reinterpret_cast<const f32x4*>(v + at);
        }
    };

    // One tile: its stage into LDS (as fp16 parts), the stage refilled with
    // the tile two ahead, then the scores, the online softmax and P·V.
    auto tile = [&](int first, Stage& st) {
        __syncthreads(); // the previous tile has been read
        if constexpr (PRESPLIT)
        {
#pragma unroll
            for (int i = 0; i < kHalfPerThread; ++i)
            {
                int part, row, cb, c, kb;
                half_run(i, part, row, cb, c, kb);
                *reinterpret_cast<u32x4*>(&ks[part][row][8 * cb]) = st.kh[i];
                // (8-byte aligned rows: two 8-byte stores)
                uint2* v2 = reinterpret_cast<uint2*>(&vt[part][c][8 * kb]);
                v2[0] = uint2 {st.vh[i][0], st.vh[i][1]};
                v2[1] = uint2 {st.vh[i][2], st.vh[i][3]};
            }
        }
        else
        {
#pragma unroll
            for (int i = 0; i < kPerThread; ++i)
            {
                const int unit = (int) threadIdx.x + i * kThreadsHere;
                if (unit < kUnits)
                {
                    const int row = unit / 16, d4 = 4 * (unit % 16);
                    const bool in = first + row < k_end;
                    f16x4 kh, kl;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        const float kv = in ? st.k[i][e] : 0.f, vv = in ? st.v[i][e] : 0.f;
                        kh[e] = half_hi(kv);
                        kl[e] = half_lo(kv);
                        vt[0][d4 + e][row] = half_hi(vv);
                        vt[1][d4 + e][row] = half_lo(vv);
                    }
                    *reinterpret_cast<f16x4*>(&ks[0][row][d4]) = kh;
                    *reinterpret_cast<f16x4*>(&ks[1][row][d4]) = kl;
                }
            }
        }
        __syncthreads();
        if (k_begin < k_end)
            load_tile(st, first + 2 * kFlashKeys);

        // S^T for keys 16 mt + 4 g + r of the tile, query li.
        f32x4 st_[2 * KB];
#pragma unroll
        for (int mt = 0; mt < 2 * KB; ++mt)
        {
            st_[mt] = f32x4 {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; ++s)
            {
                const f16x8 kh = *reinterpret_cast<const f16x8*>(&ks[0][16 * mt + li][32 * s + 8 * g]);
                const f16x8 kl = *reinterpret_cast<const f16x8*>(&ks[1][16 * mt + li][32 * s + 8 * g]);
                st_[mt] = mfma3(kh, kl, qh[s], ql[s], st_[mt]);
            }
        }
        float x[8 * KB];
        float tile_max = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2 * KB; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const int key = first + 16 * mt + 4 * g + r;
                x[4 * mt + r] = key < k_end ? st_[mt][r] * scale2 : -INFINITY;
                tile_max = fmaxf(tile_max, x[4 * mt + r]);
            }
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
        const float m_new = fmaxf(m, tile_max);
        const float alpha = exp2f(m - m_new);
        float p[8 * KB], own = 0.f;
#pragma unroll
        for (int j = 0; j < 8 * KB; ++j)
        {
            p[j] = exp2f(x[j] - m_new);
            own += p[j];
        }
        l = l * alpha + own;
        m = m_new;
        // Key block b (keys 32 b .. 32 b + 31 of the tile) takes p[8 b .. 8 b + 7].
        f16x8 ph[KB], pl[KB];
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int j = 0; j < 8; ++j)
            {
                ph[b][j] = half_hi(p[8 * b + j]);
                pl[b][j] = half_lo(p[8 * b + j]);
            }
#pragma unroll
        for (int t = 0; t < 4; ++t)
        {
            o[t] *= alpha;
#pragma unroll
            for (int b = 0; b < KB; ++b)
            {
                const f16x4 a0 = *reinterpret_cast<const f16x4*>(&vt[0][16 * t + li][32 * b + 4 * g]);
                const f16x4 a1 = *reinterpret_cast<const f16x4*>(&vt[0][16 * t + li][32 * b + 16 + 4 * g]);
                const f16x4 b0 = *reinterpret_cast<const f16x4*>(&vt[1][16 * t + li][32 * b + 4 * g]);
                const f16x4 b1 = *reinterpret_cast<const f16x4*>(&vt[1][16 * t + li][32 * b + 16 + 4 * g]);
                const f16x8 vh = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                const f16x8 vl = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
                o[t] = mfma3(vh, vl, ph[b], pl[b], o[t]);
            }
        }
    };

    // Pairs of tiles, then an odd last one outside the loop, so the loop's
    // back edge always follows the second tile of a pair.
    Stage s0, s1;
    if (k_begin < k_end)
    {
        load_tile(s0, k_begin);
        load_tile(s1, k_begin + kFlashKeys);
    }
    int first = k_begin;
    for (; first + kFlashKeys < k_end; first += 2 * kFlashKeys)
    {
        tile(first, s0);
        tile(first + kFlashKeys, s1);
    }
    if (first < k_end)
        tile(first, s0);
    // The row sum over the four lanes of query li, then O = O^T / l.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (partials != nullptr)
    {
        if (query_in)
        {
            const int heads = gridDim.y;
            float* part = partials + (((size_t) blockIdx.z * heads + head) * count + query) * (kFlashWidth + 2);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    part[2 + 16 * t + 4 * g + r] = o[t][r];
            if (g == 0)
            {
                part[0] = m;
                part[1] = l;
            }
        }
        return;
    }
    if (query_in)
    {
        const float inv = 1.f / l;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const size_t at = (size_t) query * width + column + 16 * t + 4 * g + r;
                if constexpr (OUT == kF32)
                    out[at] = o[t][r] * inv;
                else
                {
                    uint32_t bits[3];
                    exact_parts<OUT>(o[t][r] * inv, bits);
#pragma unroll
                    for (int p = 0; p < (OUT == kF16 ? 2 : 3); ++p)
                        out_parts[p * out_part_stride + at] = (uint16_t) bits[p];
                }
            }
    }
}

// The key splits of every (query, head) combined in split order, in base-2
// units: out = Σ 2^(m_s - m)·row_s / Σ 2^(m_s - m)·l_s. One 64-lane wave per
// (query, head), a lane per channel.
__global__ void __launch_bounds__(kFlashWidth) flash_combine_kernel(const float* __restrict__ partials, int count,
                                                                    int heads, int splits, int width,
                                                                    float* __restrict__ out)
{
    const int query = blockIdx.x, head = blockIdx.y, c = threadIdx.x;
    const size_t stride = (size_t) heads * count * (kFlashWidth + 2);
    const float* base = partials + ((size_t) head * count + query) * (kFlashWidth + 2);
    float largest = -INFINITY;
    for (int s = 0; s < splits; ++s)
        largest = fmaxf(largest, base[s * stride]);
    float numerator = 0.f, denominator = 0.f;
    for (int s = 0; s < splits; ++s)
    {
        const float* part = base + s * stride;
        if (part[1] == 0.f) // a split with no key
            continue;
        const float f = exp2f(part[0] - largest);
        numerator += f * part[2 + c];
        denominator += f * part[1];
    }
    out[(size_t) query * width + head * kFlashWidth + c] = numerator / denominator;
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
    // 16-bit weights: a product's input as exact 16-bit parts (split_product):
    // up to three [positions, width] parts, and fc2's [positions, feed_forward_width].
    void* parts = nullptr;
    void* ff_parts = nullptr;
    // The attention's keys and values as fp16 hi and lo halves, written by the
    // q/k/v product: [2][pitch][width] and transposed [2][width][pitch], pitch
    // the positions rounded up to the key tile, zero past the positions.
    uint16_t* k_halves = nullptr;
    uint16_t* vt_halves = nullptr;
    int pitch = 0;
    float* workspace = nullptr;
    float* flash_partials = nullptr; // [kMaxFlashSplits][heads][positions][66], split-key attention
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

// The products run over pre-split inputs (split_product) for 16-bit weights
// when every product's extents and the LayerNorm's width fit them.
bool pre_split_shape(int wdtype, int d, int f)
{
    namespace ops = wsp::ops;
    return d % 8 == 0 && ops::layernorm_parts_fits(d) && ops::split_product_fits(wdtype, d, 3 * d, d, 2 * d)
           && ops::split_product_fits(wdtype, d, f, f, f) && ops::split_product_fits(wdtype, f, d, d, d);
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
    // Three 16-bit parts take 1.5 floats a value.
    if (status == hipSuccess)
        status = encoder_allocate(e, reinterpret_cast<float**>(&e->parts), (positions * d * 3 + 1) / 2);
    if (status == hipSuccess)
        status = encoder_allocate(e, reinterpret_cast<float**>(&e->ff_parts),
                                  (positions * s.feed_forward_width * 3 + 1) / 2);
    e->pitch = (int) ((positions + wsp::encoder::kFlashKeys - 1) / wsp::encoder::kFlashKeys
                      * wsp::encoder::kFlashKeys);
    const size_t halves = (size_t) 2 * e->pitch * d; // two parts of 16 bits
    if (status == hipSuccess)
        status = encoder_allocate(e, reinterpret_cast<float**>(&e->k_halves), halves / 2);
    if (status == hipSuccess)
        status = encoder_allocate(e, reinterpret_cast<float**>(&e->vt_halves), halves / 2);
    if (status == hipSuccess)
        status = hipMemsetAsync(e->k_halves, 0, halves * sizeof(uint16_t), e->stream);
    if (status == hipSuccess)
        status = hipMemsetAsync(e->vt_halves, 0, halves * sizeof(uint16_t), e->stream);
    if (status == hipSuccess && s.heads > 0 && s.width == s.heads * wsp::encoder::kFlashWidth)
        status = encoder_allocate(e, &e->flash_partials,
                                  (size_t) wsp::encoder::kMaxFlashSplits * s.heads * positions
                                      * (wsp::encoder::kFlashWidth + 2));
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

    // Stored projection scales (powers of two in [2^-126, 2^126], so their
    // reciprocals are normal floats; 0 reads as 1) and whether any
    // projection carries one: those take the pre-split products at every
    // position count, the only products that divide a scale out.
    bool scaled = false;
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_encoder_layer_tensors& L = T->layers[l];
        for (const float c : {L.q_scale, L.k_scale, L.v_scale, L.out_scale, L.fc1_scale, L.fc2_scale})
        {
            int exponent = 0;
            if (c != 0.f && !(std::isfinite(c) && c > 0.f && std::frexp(c, &exponent) == 0.5f && exponent >= -125
                               && exponent <= 127))
                return encoder_fail(e, WSP_ERR_ARGUMENT,
                                    "wsp_encoder_encode: a projection scale is not a power of two in [2^-126, 2^126]");
            scaled = scaled || (c != 0.f && c != 1.f);
        }
    }
    if (scaled && !pre_split_shape(T->wdtype, d, f))
        return encoder_fail(e, WSP_ERR_SHAPE,
                            "wsp_encoder_encode: scaled projections need 16-bit storage and the pre-split products' "
                            "shapes");
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
    auto unscale = [](float c) { return c == 0.f ? 1.f : 1.f / c; };
    // 16-bit weights take the products over pre-split inputs: each product's
    // input is stored once as its 16-bit parts (fc1 writes fc2's itself):
    // three exact bf16 parts, or fp16 hi + lo for fp16 and scaled weights.
    const size_t part_stride = (size_t) positions * d, ff_part_stride = (size_t) positions * f;
    const bool split = (positions > 16 || scaled) && part_stride % 8 == 0 && pre_split_shape(wt, d, f);
    auto split_product = [&](const void* parts, size_t stride, int inner, const void* w, const float* bias, float* y,
                             int out, int flags, void* out_parts, float stored_scale) {
        ops::SplitProduct p {};
        p.parts = parts;
        p.part_stride = stride;
        p.rows = positions;
        p.inner = inner;
        p.w0 = w;
        p.out = out;
        p.bias0 = bias;
        p.y0 = y;
        p.ldy = out;
        p.flags = flags;
        p.out_parts = out_parts;
        p.out_part_stride = ff_part_stride;
        p.wdtype = wt;
        p.scale0 = unscale(stored_scale);
        return ops::split_product(st, p);
    };
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_encoder_layer_tensors& L = T->layers[l];
        bool att_parts = false; // the attention wrote its rows as the output product's parts
        status = split ? ops::layernorm_parts(st, e->hidden, L.attention_norm_w, L.attention_norm_b, e->parts,
                                              part_stride, positions, d, eps, wt)
                       : ops::layernorm(st, e->hidden, L.attention_norm_w, L.attention_norm_b, e->normed, positions,
                                        d, eps);
        if (status != hipSuccess)
            return encoder_hip(e, status, "self-attention norm");
        if (split)
        {
            // q, k and v side by side in one launch.
            ops::SplitProduct p {};
            p.parts = e->parts;
            p.part_stride = part_stride;
            p.rows = positions;
            p.inner = d;
            p.w0 = L.q_w;
            p.w1 = L.k_w;
            p.w2 = L.v_w;
            p.split = d;
            p.split2 = 2 * d;
            p.out = 3 * d;
            p.bias0 = L.q_b;
            p.bias2 = L.v_b;
            p.y0 = e->q;
            p.y1 = e->k;
            p.y2 = e->v;
            p.ldy = d;
            p.wdtype = wt;
            p.scale0 = unscale(L.q_scale);
            p.scale1 = unscale(L.k_scale);
            p.scale2 = unscale(L.v_scale);
            if (d / heads == kFlashWidth)
            {
                // The attention takes k and v as fp16 halves.
                p.y1_halves = e->k_halves;
                p.y2_halves_t = e->vt_halves;
                p.halves_pitch = e->pitch;
            }
            status = ops::split_product(st, p);
        }
        else if (positions > 16 && ops::tile_product_fits(wt, d, 3 * d, d, e->normed) && d % 128 == 0)
        {
            // q, k and v side by side in one launch: three times the blocks of one.
            ops::TileProduct p {};
            p.x = e->normed;
            p.rows = positions;
            p.inner = d;
            p.w0 = L.q_w;
            p.w1 = L.k_w;
            p.w2 = L.v_w;
            p.split = d;
            p.split2 = 2 * d;
            p.out = 3 * d;
            p.bias0 = L.q_b;
            p.bias2 = L.v_b;
            p.y0 = e->q;
            p.y1 = e->k;
            p.y2 = e->v;
            p.ldy = d;
            p.rows_per_group = positions;
            p.wdtype = wt;
            status = ops::tile_product(st, p);
        }
        else if ((status = ops::linear(st, e->normed, positions, d, L.q_w, wt, L.q_b, e->q, d, 0)) == hipSuccess
                 && (status = ops::linear(st, e->normed, positions, d, L.k_w, wt, nullptr, e->k, d, 0)) == hipSuccess)
            status = ops::linear(st, e->normed, positions, d, L.v_w, wt, L.v_b, e->v, d, 0);
        if (status != hipSuccess)
            return encoder_hip(e, status, "self-attention projections");
        if (d / heads == kFlashWidth && d % 4 == 0)
        {
            // 128 queries a block share each K/V tile when that still leaves
            // at most an eighth of the CUs idle (large-v3: 240 blocks,
            // 14.2 -> 13.4 ms a window); else 64 (tiny.en's 72 blocks of 128
            // queries measured slower than 144 of 64).
            const int wide_blocks = (positions + 16 * kFlashWideWaves - 1) / (16 * kFlashWideWaves) * heads;
            const float scale2 = scale * 1.44269504088896340736f;
            // Fewer 64-query blocks than CUs (tiny.en: 144): the keys are
            // split over up to four blocks per query tile, at least 64 keys
            // each, and the splits combined after.
            const int narrow_blocks = (positions + 16 * kFlashWaves - 1) / (16 * kFlashWaves) * heads;
            int splits = 1;
            if (narrow_blocks < compute_units() && e->flash_partials != nullptr)
                splits = std::max(1, std::min({kMaxFlashSplits, (compute_units() + narrow_blocks - 1) / narrow_blocks,
                                               positions / 64}));
            const int span = ((positions + splits - 1) / splits + kFlashKeys - 1) / kFlashKeys * kFlashKeys;
            float* partials = splits > 1 ? e->flash_partials : nullptr;
            const bool wide = 8 * wide_blocks >= 7 * compute_units();
            // With the pre-split products, one split writes its rows straight
            // as the output product's input parts.
            att_parts = split && (wide || splits == 1);
            const dim3 grid = wide ? dim3((positions + 16 * kFlashWideWaves - 1) / (16 * kFlashWideWaves), heads)
                                   : dim3((positions + 16 * kFlashWaves - 1) / (16 * kFlashWaves), heads, splits);
            const int key_span = wide ? positions : span;
            uint16_t* const out_parts = static_cast<uint16_t*>(e->parts);
            auto launch = [&](auto kernel, int waves) {
                hipLaunchKernelGGL(kernel, grid, dim3(64 * waves), 0, st, e->q, e->k, e->v, positions, d, scale2,
                                   e->att, key_span, wide ? nullptr : partials, e->k_halves, e->vt_halves, e->pitch,
                                   out_parts, part_stride);
            };
            if (!split)
            {
                if (wide)
                    launch(flash_attention_kernel<kFlashWideWaves>, kFlashWideWaves);
                else
                    launch(flash_attention_kernel<kFlashWaves>, kFlashWaves);
            }
            else if (!att_parts)
                launch(flash_attention_kernel<kFlashWaves, true>, kFlashWaves);
            else if (wt == WSP_F16)
            {
                if (wide)
                    launch(flash_attention_kernel<kFlashWideWaves, true, wsp::kF16>, kFlashWideWaves);
                else
                    launch(flash_attention_kernel<kFlashWaves, true, wsp::kF16>, kFlashWaves);
            }
            else if (wide)
                launch(flash_attention_kernel<kFlashWideWaves, true, wsp::kBF16>, kFlashWideWaves);
            else
                launch(flash_attention_kernel<kFlashWaves, true, wsp::kBF16>, kFlashWaves);
            status = hipGetLastError();
            if (status == hipSuccess && splits > 1)
            {
                hipLaunchKernelGGL(flash_combine_kernel, dim3(positions, heads), dim3(kFlashWidth), 0, st,
                                   e->flash_partials, positions, heads, splits, d, e->att);
                status = hipGetLastError();
            }
        }
        else
            status = ops::attention(st, e->q, positions, e->k, e->v, positions, d, heads, 0, scale, e->att,
                                    e->workspace);
        if (status != hipSuccess)
            return encoder_hip(e, status, "self attention");
        if (split)
        {
            if (att_parts || (status = ops::split_rows(st, e->att, part_stride, wt, e->parts, part_stride))
                                 == hipSuccess)
                status = split_product(e->parts, part_stride, d, L.out_w, L.out_b, e->hidden, d,
                                       ops::kProductResidual, nullptr, L.out_scale);
        }
        else
            status = ops::linear(st, e->att, positions, d, L.out_w, wt, L.out_b, e->hidden, d, 2);
        if (status != hipSuccess)
            return encoder_hip(e, status, "attention output");
        status = split ? ops::layernorm_parts(st, e->hidden, L.final_norm_w, L.final_norm_b, e->parts, part_stride,
                                              positions, d, eps, wt)
                       : ops::layernorm(st, e->hidden, L.final_norm_w, L.final_norm_b, e->normed, positions, d, eps);
        if (status != hipSuccess)
            return encoder_hip(e, status, "feed-forward norm");
        if (split)
        {
            if ((status = split_product(e->parts, part_stride, d, L.fc1_w, L.fc1_b, nullptr, f, ops::kProductGelu,
                                        e->ff_parts, L.fc1_scale))
                == hipSuccess)
                status = split_product(e->ff_parts, ff_part_stride, f, L.fc2_w, L.fc2_b, e->hidden, d,
                                       ops::kProductResidual, nullptr, L.fc2_scale);
        }
        else if ((status = ops::linear(st, e->normed, positions, d, L.fc1_w, wt, L.fc1_b, e->ff, f, 1)) == hipSuccess)
            status = ops::linear(st, e->ff, positions, f, L.fc2_w, wt, L.fc2_b, e->hidden, d, 2);
        if (status != hipSuccess)
            return encoder_hip(e, status, "feed-forward");
    }
    if ((status = ops::layernorm(st, e->hidden, T->final_norm_w, T->final_norm_b, output, positions, d, eps))
        != hipSuccess)
        return encoder_hip(e, status, "final norm");
    return WSP_OK;
}

int wsp_encoder_scaled_halves(const wsp_encoder_shape* shape, const void* bf16, size_t count, void* halves,
                              float* scale)
{
    if (shape == nullptr || scale == nullptr || (count > 0 && (bf16 == nullptr || halves == nullptr)))
        return WSP_ERR_ARGUMENT;
    if (!pre_split_shape(WSP_F16, shape->width, shape->feed_forward_width))
        return WSP_ERR_SHAPE;
    const uint16_t* in = static_cast<const uint16_t*>(bf16);
    uint16_t* out = static_cast<uint16_t*>(halves);
    auto widen = [](uint16_t bits) { return __builtin_bit_cast(float, (uint32_t) bits << 16); };
    // The shift puts the largest magnitude's binade at 2^15 (fp16's top one:
    // an 8-bit significand there is at most 65280 < 65504).
    int top = INT_MIN;
    for (size_t i = 0; i < count; ++i)
    {
        const float v = widen(in[i]);
        if (!std::isfinite(v))
            return WSP_ERR_LOGIC;
        if (v != 0.f)
            top = std::max(top, std::ilogb(v));
    }
    // (At most 126, so the scale stays a finite float and its reciprocal a normal one.)
    const int shift = top == INT_MIN ? 0 : std::min(15 - top, 126);
    for (size_t i = 0; i < count; ++i)
    {
        const float v = widen(in[i]);
        const _Float16 h = (_Float16) std::ldexp(v, shift);
        if (__builtin_bit_cast(uint32_t, std::ldexp((float) h, -shift)) != __builtin_bit_cast(uint32_t, v))
            return WSP_ERR_LOGIC;
        out[i] = __builtin_bit_cast(uint16_t, h);
    }
    *scale = std::ldexp(1.f, shift);
    return WSP_OK;
}

} // extern "C"
