// Batched decode of independent streams on gfx950. B sequences, each with its
// own self and cross caches and all at the same position, share one read of
// every weight per step; the step of one token per stream is the
// medium/large-configuration decode loop.
//
// Projections run on the matrix cores. An fp32 activation x is carried as a
// sum of 16-bit parts: hi = fp16(x), lo = fp16(x - hi) for fp16 weights, or
// three bf16 parts (each the rounded remainder of the last) for bf16 weights.
// Every part times a 16-bit weight is exact in fp32, so W·hi + W·lo (+ W·lo2)
// accumulated in fp32 reproduces the fp32 product the reference computes with
// widened weights (Kernels/Linear.h:229-246) to fp32 rounding, not to 16-bit
// rounding. The fp16 form needs |x| < 65504.
//
// Kernels per layer: LayerNorm + split, the q/k/v product (k and v rows land
// in the self caches), split-key attention (+ combine), the output product
// with its residual, and the same for cross attention and the feed-forward
// pair. Every reduction runs in a fixed order.
#include "../../include/wsp_hip.h"
#include "batch_plan.h"
#include "device_common.h"
#include "ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

namespace wsp::batch
{
namespace
{
typedef uint16_t u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kProductThreads = 512; // 8 waves split the inner dimension of a 16-column tile
constexpr int kProductWaves = kProductThreads / kWave;
constexpr int kAttendThreads = 256;  // 16 key groups x 16 lanes of four channels
constexpr int kTileKeys = 128;       // keys an attention block holds per pass
constexpr int kNormThreads = 256;
constexpr int kMaxRowTiles = 8;      // 16-row tiles per product: 128 rows

template <int WT>
constexpr int parts_of()
{
    return WT == kF16 ? 2 : 3;
}

// x as 16-bit parts at out[p * part_stride + index].
template <int WT>
__device__ __forceinline__ void store_split(u16* out, size_t part_stride, size_t index, float x)
{
    if constexpr (WT == kF16)
    {
        const _Float16 hi = (_Float16) x;
        const _Float16 lo = (_Float16) (x - (float) hi);
        out[index] = __builtin_bit_cast(u16, hi);
        out[part_stride + index] = __builtin_bit_cast(u16, lo);
    }
    else
    {
        float rest = x;
#pragma unroll
        for (int p = 0; p < 3; ++p)
        {
            const __bf16 b = (__bf16) rest;
            out[(size_t) p * part_stride + index] = __builtin_bit_cast(u16, b);
            rest -= (float) b;
        }
    }
}

// Split activations ([parts][rows_padded][width]) are stored fragment-major:
// the 16 rows x 32 inner values one v_mfma_f32_16x16x32 A-operand load covers
// are 64 lanes x 16 contiguous bytes in lane order (lane 16g + r holds row r,
// values 8g..8g+7), so a wave reads each fragment as one contiguous kilobyte.
// Read row by row (16 rows x 64 bytes a load) the same activations took 6.5
// of an 80-block product's 9.6 us; fragment-major, 1.9.
__device__ __forceinline__ size_t fragment_index(int row, int col, int width)
{
    const int t = row / 16, r = row % 16, kb = col / 32, g = (col % 32) / 8, e = col % 8;
    return (((size_t) t * (width / 32) + kb) * 64 + g * 16 + r) * 8 + e;
}

// The fp32 residual stream h ([rows_padded][width]) is stored fragment-major
// as well: fragment (t, kb) holds rows 16t.. and inner values 32kb.. as two
// 1 KB halves, half j holding values 8g + 4j .. 8g + 4j + 3 of row r at lane
// 16g + r, so each of a wave's two fragment loads is one contiguous kilobyte
// and four consecutive values of a row stay contiguous.
__device__ __forceinline__ size_t residual_index(int row, int col, int width)
{
    const int t = row / 16, r = row % 16, kb = col / 32, g = (col % 32) / 8, e = col % 8;
    return (((size_t) t * (width / 32) + kb) * 2 + e / 4) * 256 + (g * 16 + r) * 4 + e % 4;
}

// Projection weights W [n][k] (16-bit) are read from a fragment-major copy
// made once per weight table: the 16 rows x 32 inner values one
// v_mfma_f32_16x16x32 B-operand load covers are 64 lanes x 16 contiguous
// bytes, lane 16g + r holding row r's values 8g..8g+7, tiles of 16 rows in
// order and k-blocks in order within a tile (rows past the last padded with
// zeros). Read from the row-major weights, each load touched 16 rows x 64
// bytes; fragment-major, an 80-block product launch took 4.4 us instead of
// 5.1. Element (tile, kb) starts at (tile * (k / 32) + kb) * 512.
constexpr int kFragment = 512; // 16-bit values per fragment

__global__ void __launch_bounds__(256) pack_fragments_kernel(const u16* __restrict__ w, int rows, int inner,
                                                             u16* __restrict__ out, size_t chunks)
{
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; // 16-byte chunk of the output
    if (i >= chunks)
        return;
    const int lane = (int) (i % 64), kbs = inner / 32;
    const size_t fragment = i / 64;
    const int kb = (int) (fragment % kbs), tile = (int) (fragment / kbs);
    const int n = tile * 16 + lane % 16, k = kb * 32 + 8 * (lane / 16);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (n < rows)
        v = *reinterpret_cast<const u32x4*>(w + (size_t) n * inner + k);
    *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

// bf16 weights held as exact fp16 multiples w·2^shift (the products then
// take two fp16 parts of their input instead of three bf16 ones, and divide
// 2^shift out of each sum). bf16_range_kernel leaves the largest magnitude's
// bits (sign dropped) of n values in range[0] and sets range[1] if a value is
// not finite; pack_scaled_kernel is pack_fragments_kernel narrowing each
// value, and sets *inexact if one does not come back bit for bit.
__global__ void __launch_bounds__(256) bf16_range_kernel(const u16* __restrict__ w, size_t n,
                                                         unsigned* __restrict__ range)
{
    unsigned top = 0, bad = 0;
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t) gridDim.x * 256)
    {
        const unsigned m = w[i] & 0x7FFFu;
        if (m >= 0x7F80u)
            bad = 1u;
        else
            top = max(top, m);
    }
    for (int offset = 32; offset > 0; offset >>= 1)
    {
        top = max(top, (unsigned) __shfl_xor((int) top, offset));
        bad |= (unsigned) __shfl_xor((int) bad, offset);
    }
    if (threadIdx.x % 64 == 0)
    {
        if (top != 0)
            atomicMax(range, top);
        if (bad != 0)
            atomicOr(range + 1, 1u);
    }
}

__global__ void __launch_bounds__(256) pack_scaled_kernel(const u16* __restrict__ w, int rows, int inner,
                                                          u16* __restrict__ out, size_t chunks, int shift,
                                                          unsigned* __restrict__ inexact)
{
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks)
        return;
    const int lane = (int) (i % 64), kbs = inner / 32;
    const size_t fragment = i / 64;
    const int kb = (int) (fragment % kbs), tile = (int) (fragment / kbs);
    const int n = tile * 16 + lane % 16, k = kb * 32 + 8 * (lane / 16);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (n < rows)
    {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(w + (size_t) n * inner + k);
        bool exact = true;
#pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            const uint32_t bits = (raw[j / 2] >> (16 * (j % 2))) & 0xFFFFu;
            const float x = __uint_as_float(bits << 16);
            const _Float16 y = (_Float16) ldexpf(x, shift);
            exact = exact && __float_as_uint(ldexpf((float) y, -shift)) == __float_as_uint(x);
            v[j / 2] |= (uint32_t) __builtin_bit_cast(u16, y) << (16 * (j % 2));
        }
        if (!exact)
            atomicOr(inexact, 1u);
    }
    *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

// 16-bit values of the fragment-major copy of a [rows][inner] weight.
size_t packed_size(int rows, int inner)
{
    return (size_t) ((rows + 15) / 16) * 16 * inner;
}

// The same parts as register values.
template <int WT>
__device__ __forceinline__ void split_value(float x, u16 (&out)[parts_of<WT>()])
{
    if constexpr (WT == kF16)
    {
        const _Float16 hi = (_Float16) x;
        const _Float16 lo = (_Float16) (x - (float) hi);
        out[0] = __builtin_bit_cast(u16, hi);
        out[1] = __builtin_bit_cast(u16, lo);
    }
    else
    {
        float rest = x;
#pragma unroll
        for (int p = 0; p < 3; ++p)
        {
            const __bf16 b = (__bf16) rest;
            out[p] = __builtin_bit_cast(u16, b);
            rest -= (float) b;
        }
    }
}

template <int WT>
__device__ __forceinline__ float4v mfma16(u32x4 a, u32x4 b, float4v c)
{
    if constexpr (WT == kF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// LayerNorm of one row into its split parts (Kernels/LayerNorm.h:44-89:
// mean, centred biased variance, rsqrt(var + eps)); with EMBED the row is
// first built as token_table[token] + position_table[position]
// (Kernels/Embed.h:38-62) and kept as the residual stream.
// ---------------------------------------------------------------------------
struct Norm
{
    float* h;             // [rows_padded, width] residual stream (residual_index layout)
    int width;
    const float* gamma;
    const float* beta;
    float eps;
    u16* xs;              // split output [parts][rows_padded][width], fragment-major
    size_t xs_part;
    float* y;             // optional f32 copy of the normalised rows
    const uint32_t* tokens; // [streams][step_tokens], or null with a ring
    const uint32_t* ring;   // position-major [max_positions + 1][streams] (one token per stream)
    const int* state;       // device word: the position of the step's first token
    const float* token_table;
    const float* position_table;
    int streams, step_tokens, vocabulary;
};

template <int WT, bool EMBED>
__global__ void __launch_bounds__(kNormThreads) norm_kernel(Norm a)
{
    __shared__ float scratch[kNormThreads / kWave];
    const int row = blockIdx.x;
    float* h = a.h;
    const auto at = [&](int c) { return residual_index(row, c, a.width); };
    if constexpr (EMBED)
    {
        const int first = *a.state;
        const uint32_t token = a.ring != nullptr ? a.ring[(size_t) first * a.streams + row] : a.tokens[row];
        const int position = first + row % a.step_tokens;
        for (int c = threadIdx.x; c < a.width; c += kNormThreads)
            h[at(c)] = token < (uint32_t) a.vocabulary
                           ? a.token_table[(size_t) token * a.width + c]
                                 + a.position_table[(size_t) position * a.width + c]
                           : __builtin_nanf("");
        if (a.xs == nullptr) // the embedding only: the next product normalises
            return;
    }
    float total = 0.f;
    for (int c = threadIdx.x; c < a.width; c += kNormThreads)
        total += h[at(c)];
    const float mean = block_sum(total, scratch) / (float) a.width;
    float squares = 0.f;
    for (int c = threadIdx.x; c < a.width; c += kNormThreads)
    {
        const float centred = h[at(c)] - mean;
        squares += centred * centred;
    }
    const float scale = rsqrtf(block_sum(squares, scratch) / (float) a.width + a.eps);
    for (int c = threadIdx.x; c < a.width; c += kNormThreads)
    {
        const float v = (h[at(c)] - mean) * scale * a.gamma[c] + a.beta[c];
        store_split<WT>(a.xs, a.xs_part, fragment_index(row, c, a.width), v);
        if (a.y != nullptr)
            a.y[(size_t) row * a.width + c] = v;
    }
}

// ---------------------------------------------------------------------------
// Skinny product y[m, n] = Σ_k x[m, k]·W[n, k] for up to 128 rows. A block
// owns 16 output columns for every row tile; its 8 waves split the inner
// dimension into contiguous runs of 32-wide k-blocks, each lane loading 16
// bytes of one weight row and of each split activation fragment per k-block
// (v_mfma_f32_16x16x32: A = activations, lane l row l % 16; B = weights,
// lane l column l % 16; both with k = 8(l / 16) + j). KB k-blocks are loaded
// before their products, the next batch's weights ahead of them. The 8 run
// partials are summed in run order.
// ---------------------------------------------------------------------------
enum Epilogue : int
{
    kStore = 0,     // y = acc + bias
    kResidual = 1,  // y += acc + bias
    kQkv = 3,       // q | self key row | self value row
    kGelu = 4       // y = gelu(acc + bias), fp32
};

struct Product
{
    const u16* x;     // [parts][rows_padded][inner]
    size_t x_part;
    int rows, inner, out;
    const void* w;    // [out][inner]
    const float* bias;
    int epilogue;
    float* y;
    int ldy;
    float* q;
    float* keys;      // stream 0's cache of this layer
    float* values;
    size_t stream_stride;
    const int* state; // device word: the position of the step's first token
    int step_tokens, width;
    // normed_product_kernel: x = LayerNorm(h) computed in the product
    const float* h;   // [rows_padded][inner] residual stream (residual_index layout)
    const float* gamma;
    const float* beta;
    float eps;
    float scale = 1.f; // each sum's factor before the bias: 2^-shift of weights held scaled
};

// `prior` is y[m][n] read before the product (kResidual; unused otherwise).
template <int WT>
__device__ __forceinline__ void finish(const Product& a, int m, int n, float acc, float prior = 0.f)
{
    const float v = acc * a.scale + (a.bias != nullptr ? a.bias[n] : 0.f);
    switch (a.epilogue)
    {
        case kStore: a.y[(size_t) m * a.ldy + n] = v; break;
        case kResidual: a.y[residual_index(m, n, a.ldy)] = prior + v; break; // y is h
        case kGelu: a.y[(size_t) m * a.ldy + n] = exact_gelu(v); break;
        default:
        {
            const int d = a.width;
            const int stream = m / a.step_tokens, i = m % a.step_tokens;
            const size_t row = (size_t) stream * a.stream_stride + (size_t) (*a.state + i) * d;
            if (n < d)
                a.q[(size_t) m * d + n] = v;
            else if (n < 2 * d)
                a.keys[row + (n - d)] = v;
            else
                a.values[row + (n - 2 * d)] = v;
        }
    }
}

// The run of the inner dimension wave `wave` of this block takes. Every block
// reads all of the activations, and the blocks of one XCD (every eighth
// block) would otherwise read them in the same order at the same time, all
// on the same few L2 channels: rotating the runs by the block's place on its
// XCD spreads them (measured: the activation reads of an 80-block product
// took 6.5 of its 9.6 us unrotated). Partials are kept by run and summed in
// run order, so the arithmetic is the same for every rotation.
__device__ __forceinline__ int inner_run(int wave)
{
    return (wave + (int) blockIdx.x / 8) % kProductWaves;
}

// k-blocks a wave loads at once: as many as about 160 registers of weight
// and activation fragments hold (4 + 4·P·MT per k-block), at most 8.
template <int P, int MT>
constexpr int kblocks_per_load()
{
    constexpr int kb = 160 / (4 + 4 * P * MT);
    return kb < 1 ? 1 : (kb > 8 ? 8 : kb);
}

template <int WT, int MT, bool PREFETCH>
__global__ void __launch_bounds__(kProductThreads) product_kernel(Product a)
{
    constexpr int P = parts_of<WT>();
    constexpr int KB = kblocks_per_load<P, MT>();
    constexpr int OUTS = (MT * 256 + kProductThreads - 1) / kProductThreads; // outputs a thread finishes
    __shared__ float partial[kProductWaves][MT * 256];

    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int li = lane % 16, g = lane / 16;
    const int n0 = blockIdx.x * 16;
    const int kblocks = a.inner / 32;
    const int run = inner_run(wave);
    const int kb_begin = run * kblocks / kProductWaves;
    const int kb_end = (run + 1) * kblocks / kProductWaves;
    // This block's weight tile, fragment-major (padding rows are zero).
    const u16* wfrag = static_cast<const u16*>(a.w) + (size_t) blockIdx.x * kblocks * kFragment + lane * 8;

    float4v acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        acc[t] = float4v {0.f, 0.f, 0.f, 0.f};

    // The weights of the next batch of k-blocks are requested before the
    // products of the current one, so HBM latency overlaps the matrix work;
    // activations (L2-resident) are loaded per batch.
    // A wave may own no k-block (inner < 256): its loads then re-read its
    // first block index, which is always < inner / 32, and are never used.
    const int kb_last = max(kb_end - 1, kb_begin);
    u32x4 wv[KB];
#pragma unroll
    for (int u = 0; u < KB; ++u)
        wv[u] = *reinterpret_cast<const u32x4*>(wfrag + (size_t) min(kb_begin + u, kb_last) * kFragment);
    // The epilogue's outputs: output o of this thread is C[16 t + row][col]
    // with t·256 + row·16 + col = threadIdx.x + o·512. A residual product
    // reads their y values now, behind the first weight loads (ahead of them
    // they would delay the weights), so its epilogue waits for no load.
    float prior[OUTS];
#pragma unroll
    for (int o = 0; o < OUTS; ++o)
    {
        const int i = (int) threadIdx.x + o * kProductThreads;
        const int m = min((i / 256) * 16 + (i % 256) / 16, a.rows - 1), n = min(n0 + i % 16, a.out - 1);
        prior[o] = a.epilogue == kResidual ? a.y[residual_index(m, n, a.ldy)] : 0.f;
    }
    for (int kb = kb_begin; kb < kb_end; kb += KB)
    {
        u32x4 xv[KB][P][MT];
#pragma unroll
        for (int u = 0; u < KB; ++u)
        {
            const int k = min(kb + u, kb_end - 1) * 32;
#pragma unroll
            for (int p = 0; p < P; ++p)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    xv[u][p][t] = *reinterpret_cast<const u32x4*>(
                        a.x + p * a.x_part + (((size_t) t * kblocks + k / 32) * 64 + lane) * 8);
        }
        u32x4 wn[KB];
        if constexpr (PREFETCH)
        {
#pragma unroll
            for (int u = 0; u < KB; ++u)
                wn[u] = *reinterpret_cast<const u32x4*>(wfrag + (size_t) min(kb + KB + u, kb_end - 1) * kFragment);
        }
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (kb + u < kb_end)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int p = 0; p < P; ++p)
                        acc[t] = mfma16<WT>(xv[u][p][t], wv[u], acc[t]);
        if constexpr (PREFETCH)
        {
#pragma unroll
            for (int u = 0; u < KB; ++u)
                wv[u] = wn[u];
        }
        else if (kb + KB < kb_end)
        {
#pragma unroll
            for (int u = 0; u < KB; ++u)
                wv[u] = *reinterpret_cast<const u32x4*>(wfrag + (size_t) min(kb + KB + u, kb_end - 1) * kFragment);
        }
    }

    // acc[t][r] of lane (g, li) is C[4g + r][li] of row tile t. Every tile
    // goes to LDS at once; each output is then the 8 waves' sum in order.
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            partial[run][t * 256 + lane * 4 + r] = acc[t][r];
    __syncthreads();
#pragma unroll
    for (int o = 0; o < OUTS; ++o)
    {
        const int i = (int) threadIdx.x + o * kProductThreads;
        if (i >= MT * 256)
            break;
        const int t = i / 256, row = (i % 256) / 16, col = i % 16;
        const int src = t * 256 + ((row / 4) * 16 + col) * 4 + row % 4;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kProductWaves; ++w)
            v += partial[w][src];
        const int m = t * 16 + row, n = n0 + col;
        if (m < a.rows && n < a.out)
            finish<WT>(a, m, n, v, prior[o]);
    }
}

// The same product with a LayerNorm in front (Kernels/LayerNorm.h:44-89):
// x = (h - mean)·rsqrt(var + eps)·gamma + beta of the fp32 residual rows, for
// up to 32 rows and inner ≤ 2048. Every wave holds the h values of its whole
// k-range in registers, so the row statistics are two fixed-order sums of
// per-wave partials through LDS — mean first, then the centred squares — and
// the normalised values are split into their 16-bit parts in registers. No
// separate LayerNorm launch, and no split activations written or read.
constexpr int kNormedBlocks = 5;   // k-blocks per wave: inner <= 8 waves * 5 * 32 = 1280
constexpr int kNormedWidth = kProductWaves * kNormedBlocks * 32;

// NT column tiles of 16 per block: 2 when one tile a block would give more
// blocks than CUs, so every block still has a CU of its own and the h rows are
// loaded and normalised once for both tiles.
template <int WT, int MT, int NT>
__global__ void __launch_bounds__(kProductThreads) normed_product_kernel(Product a)
{
    constexpr int P = parts_of<WT>();
    constexpr int TILES = NT * MT;
    constexpr int OUTS = (TILES * 256 + kProductThreads - 1) / kProductThreads; // outputs a thread finishes
    __shared__ float partial[kProductWaves][TILES * 256];
    __shared__ float stats[2][kProductWaves][MT * 16];
    __shared__ float4v sh_gamma[kNormedWidth / 4], sh_beta[kNormedWidth / 4];

    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int li = lane % 16, g = lane / 16;
    const int n0 = blockIdx.x * 16 * NT;
    const int kblocks = a.inner / 32;
    const int run = inner_run(wave);
    const int kb_begin = run * kblocks / kProductWaves;
    const int kb_end = (run + 1) * kblocks / kProductWaves;
    const int nkb = kb_end - kb_begin;
    // The block's weight tiles, fragment-major; a second tile past the last
    // (an odd tile count) re-reads the last one and is never stored.
    const u16* wfrag[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
        wfrag[nt] = static_cast<const u16*>(a.w)
                    + (size_t) min((int) blockIdx.x * NT + nt, (a.out + 15) / 16 - 1) * kblocks * kFragment + lane * 8;

    u32x4 wv[kNormedBlocks][NT];
    float4v hv[kNormedBlocks][MT][2];
#pragma unroll
    for (int u = 0; u < kNormedBlocks; ++u)
        if (u < nkb)
        {
            const int k = (kb_begin + u) * 32;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                wv[u][nt] = *reinterpret_cast<const u32x4*>(wfrag[nt] + (size_t) (kb_begin + u) * kFragment);
#pragma unroll
            for (int t = 0; t < MT; ++t)
            {
                const float* half0 = a.h + ((size_t) t * kblocks + k / 32) * 512 + lane * 4;
                hv[u][t][0] = *reinterpret_cast<const float4v*>(half0);
                hv[u][t][1] = *reinterpret_cast<const float4v*>(half0 + 256);
            }
        }
    for (int i = threadIdx.x; i < a.inner / 4; i += kProductThreads)
    {
        sh_gamma[i] = reinterpret_cast<const float4v*>(a.gamma)[i];
        sh_beta[i] = reinterpret_cast<const float4v*>(a.beta)[i];
    }

    // Row t*16 + li: this lane's 8·nkb values, summed over the four lanes of
    // the row (l ^ 16, l ^ 32), then over the 8 waves in order.
    float mean[MT], scale[MT];
#pragma unroll
    for (int pass = 0; pass < 2; ++pass)
    {
#pragma unroll
        for (int t = 0; t < MT; ++t)
        {
            float s = 0.f;
#pragma unroll
            for (int u = 0; u < kNormedBlocks; ++u)
                if (u < nkb)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                        {
                            const float v = hv[u][t][j][e];
                            s += pass == 0 ? v : (v - mean[t]) * (v - mean[t]);
                        }
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            if (g == 0)
                stats[pass][run][t * 16 + li] = s;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < MT; ++t)
        {
            float total = 0.f;
#pragma unroll
            for (int w = 0; w < kProductWaves; ++w)
                total += stats[pass][w][t * 16 + li];
            if (pass == 0)
                mean[t] = total / (float) a.inner;
            else
                scale[t] = rsqrtf(total / (float) a.inner + a.eps);
        }
    }

    float4v acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int t = 0; t < MT; ++t)
            acc[nt][t] = float4v {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kNormedBlocks; ++u)
        if (u < nkb)
#pragma unroll
            for (int t = 0; t < MT; ++t)
            {
                uint32_t packed[P][4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2)
                {
                    uint32_t lo16[P], hi16[P];
#pragma unroll
                    for (int half = 0; half < 2; ++half)
                    {
                        const int e = 2 * e2 + half;
                        const int q4 = ((kb_begin + u) * 32 + 8 * g) / 4 + e / 4;
                        const float v = (hv[u][t][e / 4][e % 4] - mean[t]) * scale[t] * sh_gamma[q4][e % 4]
                                        + sh_beta[q4][e % 4];
                        u16 parts[P];
                        split_value<WT>(v, parts);
#pragma unroll
                        for (int p = 0; p < P; ++p)
                            (half == 0 ? lo16 : hi16)[p] = parts[p];
                    }
#pragma unroll
                    for (int p = 0; p < P; ++p)
                        packed[p][e2] = lo16[p] | (hi16[p] << 16);
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int p = 0; p < P; ++p)
                        acc[nt][t] = mfma16<WT>(u32x4 {packed[p][0], packed[p][1], packed[p][2], packed[p][3]},
                                                wv[u][nt], acc[nt][t]);
            }

    // Every tile goes to LDS at once (tile nt·MT + t); each output is then
    // the 8 waves' sum in order. (No residual epilogue here.)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                partial[run][(nt * MT + t) * 256 + lane * 4 + r] = acc[nt][t][r];
    __syncthreads();
#pragma unroll
    for (int o = 0; o < OUTS; ++o)
    {
        const int i = (int) threadIdx.x + o * kProductThreads;
        if (i >= TILES * 256)
            break;
        const int tile = i / 256, row = (i % 256) / 16, col = i % 16;
        const int nt = tile / MT, t = tile % MT;
        const int src = tile * 256 + ((row / 4) * 16 + col) * 4 + row % 4;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kProductWaves; ++w)
            v += partial[w][src];
        const int m = t * 16 + row, n = n0 + nt * 16 + col;
        if (m < a.rows && n < a.out)
            finish<WT>(a, m, n, v);
    }
}

// ---------------------------------------------------------------------------
// LayerNorm statistics of h from 64-column groups: a residual tile product's
// epilogue writes, for every 64-column group of a row, the group's mean and
// its centred sum of squares. A consumer combines the groups in order with
// Chan's pairwise update (exact algebra, stable in fp32), which gives the
// row's mean and centred biased variance (Kernels/LayerNorm.h:44-89) without
// reading the whole row.
// ---------------------------------------------------------------------------
constexpr int kGroupColumns = 64;

__device__ __forceinline__ void row_statistics(const float* stats, int groups, int width, float eps, float& mean,
                                               float& scale)
{
    float m = 0.f, m2 = 0.f, count = 0.f;
    for (int c = 0; c < groups; ++c)
    {
        const float nb = (float) min(kGroupColumns, width - c * kGroupColumns);
        const float mb = stats[2 * c], qb = stats[2 * c + 1];
        const float total = count + nb;
        const float delta = mb - m;
        m += delta * (nb / total);
        m2 += qb + delta * delta * (count * nb / total);
        count = total;
    }
    mean = m;
    scale = rsqrtf(m2 / (float) width + eps);
}

// The final LayerNorm written out as the step's hidden rows (Decoder/
// Decoder.cpp:174, readable until the next step, Decoder/Decoder.h:111-115).
__global__ void __launch_bounds__(kNormThreads) hidden_kernel(const float* h, const float* stats, int groups,
                                                              int width, const float* gamma, const float* beta,
                                                              float eps, float* out)
{
    const int row = blockIdx.x;
    float mean, scale;
    row_statistics(stats + (size_t) row * groups * 2, groups, width, eps, mean, scale);
    for (int c = threadIdx.x; c < width; c += kNormThreads)
        out[(size_t) row * width + c] = (h[residual_index(row, c, width)] - mean) * scale * gamma[c] + beta[c];
}

// ---------------------------------------------------------------------------
// Skinny products y[m, n] = Σ_k x[m, k]·W[n, k] + b[n] for up to 128 rows, on
// the matrix cores (v_mfma_f32_16x16x32: A = activations, lane l row l % 16;
// B = weights, lane l column l % 16; both with k = 8(l / 16) + j).
//
// A block owns 64 output columns (one 16-column tile per wave) and a run of
// the inner dimension (a split). It stages its rows' fp32 activations for
// the run into LDS once — LayerNorm applied on the way in when the product
// has one, each value cut into its exact 16-bit parts — and every wave reads
// its A fragments from there, so the activations are fetched once per block
// instead of once per 16 columns. Weight fragments for a batch of k-blocks
// are loaded before the batch's activations.
//
// Splits: when 64-column groups alone leave the chip idle, the inner
// dimension is cut into `splits` runs. Each block writes its partial tile
// with device-scope stores, waits for them, and counts itself in on the
// group's counter; the block that counts last sums the partials in split
// order (so the result does not depend on which block finishes last), runs
// the epilogue and sets the counter back to zero for the next launch.
// ---------------------------------------------------------------------------
constexpr int kTileThreads = 256; // (kTileColumns and kMaxSplits: batch_plan.h)
constexpr int kStageBytes = 64 * 1024; // LDS for a block's split activations

struct Tile
{
    const float* x;        // [rows][ldx] fp32 activations (the residual stream's layout when x_residual)
    int ldx;
    int x_residual;
    int short_batches;     // stage two k-blocks a batch (see stage_kblocks)
    int rows, inner, out;
    const void* w;         // [out][inner], 16-bit
    const float* bias;
    const float* gamma;    // LayerNorm on the way in when non-null
    const float* beta;
    const float* stats_in; // [rows][stat_groups][2]
    int stat_groups;
    float eps;
    int epilogue;
    float* y;
    int ldy;
    float* stats_out;      // kResidual: [rows][out / 64][2]
    float* q;              // kQkv
    float* keys;           // stream 0's cache of this layer
    float* values;
    size_t stream_stride;
    const int* state;      // device word: the position of the step's first token
    int step_tokens, width;
    int splits, kb_per_split;
    float* partials;       // [blocks][kTileThreads][columns per thread]
    unsigned* counters;    // [column groups], zero between launches
    size_t partials_capacity, counters_capacity; // floats and counters the buffers hold
    float scale = 1.f;     // each sum's factor before the bias (as Product::scale)
};

// k-blocks (32 inner values) a block stages per batch: what the LDS holds,
// at most 10 float4 activation runs per thread in registers, and at most
// CAP. Long batches suit a launch of fewer blocks than CUs (fc2's splits:
// fewer dependent batches); a launch of several blocks a CU (the logits,
// 811 blocks) runs faster with batches of two k-blocks, whose smaller LDS
// and register footprint lets more blocks share a CU: measured 38.0 -> 23.7
// us at the medium shape and 69.6 -> 49.0 at large-v3 against batches of 10.
template <int P, int MT, int CAP>
constexpr int stage_kblocks()
{
    constexpr int fit = (kStageBytes - P * MT * 16 * 16) / (P * MT * 16 * 64);
    constexpr int runs = 20 / MT;
    constexpr int kb = fit < runs ? fit : runs;
    return kb < 1 ? 1 : (kb > CAP ? CAP : kb);
}

template <int WT, int MT, int CAP>
__global__ void __launch_bounds__(kTileThreads) tile_kernel(Tile a)
{
    constexpr int P = parts_of<WT>();
    constexpr int R = MT * 16;                // rows held (padding rows are zero)
    constexpr int KB = stage_kblocks<P, MT, CAP>();
    constexpr int RS = KB * 32 + 8;           // LDS row stride in 16-bit values (16 bytes of padding)
    constexpr int RUNS = R * KB * 8 / kTileThreads; // float4 runs a thread stages per batch
    constexpr int TPR = kTileThreads / R;     // epilogue threads per row
    constexpr int CPT = kTileColumns / TPR;   // columns per epilogue thread
    static_assert(R * KB * 8 % kTileThreads == 0, "whole runs per thread");
    __shared__ __attribute__((aligned(16))) u16 xs[P][R][RS];
    __shared__ float tile[R][kTileColumns + 1];
    __shared__ float row_mean[R], row_scale[R];
    __shared__ int last_block;

    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int li = lane % 16, g = lane / 16;
    const int cg = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
    const int n0 = cg * kTileColumns;
    // The epilogue's row and columns; a residual product reads its h values
    // now, so the epilogue's read-modify-write waits for nothing.
    const int m = threadIdx.x / TPR, c0 = (threadIdx.x % TPR) * CPT;
    const bool row_in = m < a.rows;
    float resid[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c)
    {
        const int n = min(n0 + c0 + c, a.out - 1);
        resid[c] = a.epilogue == kResidual ? a.y[residual_index(min(m, a.rows - 1), n, a.ldy)] : 0.f; // y is h
    }
    const int kblocks = a.inner / 32;
    const int kb_begin = split * a.kb_per_split;
    const int kb_end = min(kb_begin + a.kb_per_split, kblocks);
    // This wave's weight tile, fragment-major; tiles past the last (the last
    // group of a vocabulary) re-read the last tile and are never stored.
    const u16* wfrag = static_cast<const u16*>(a.w)
                       + (size_t) min(n0 / 16 + wave, (a.out + 15) / 16 - 1) * kblocks * kFragment + lane * 8;

    if (a.gamma != nullptr)
    {
        if (threadIdx.x < R)
        {
            float mean = 0.f, scale = 0.f;
            if ((int) threadIdx.x < a.rows)
                row_statistics(a.stats_in + (size_t) threadIdx.x * a.stat_groups * 2, a.stat_groups, a.inner, a.eps,
                               mean, scale);
            row_mean[threadIdx.x] = mean;
            row_scale[threadIdx.x] = scale;
        }
        __syncthreads();
    }

    float4v acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        acc[t] = float4v {0.f, 0.f, 0.f, 0.f};

    u32x4 wv[KB];
    for (int kb0 = kb_begin; kb0 < kb_end; kb0 += KB)
    {
        const int nkb = min(KB, kb_end - kb0);
#pragma unroll
        for (int u = 0; u < KB; ++u)
            wv[u] = *reinterpret_cast<const u32x4*>(wfrag + (size_t) (kb0 + min(u, nkb - 1)) * kFragment);
        // Stage rows [0, R) x inner [32 kb0, 32 (kb0 + nkb)) as float4 runs
        // (row m, values 4j .. 4j + 3 of the batch), taken in the source's
        // order so that a wave's loads are contiguous: row-major runs for a
        // row-major x; for the residual stream, its fragment-major order
        // (fragment (t, kb), half, lane slot 16g + r).
        const auto run_at = [&](int i, int& m, int& j) {
            if (a.x_residual)
            {
                const int t = i / (KB * 128), rest = i % (KB * 128), slot = rest % 64;
                m = t * 16 + slot % 16;
                j = (rest / 128) * 8 + (slot / 16) * 2 + (rest / 64) % 2;
            }
            else
            {
                m = i / (KB * 8);
                j = i % (KB * 8);
            }
        };
        float4v xv[RUNS];
#pragma unroll
        for (int r = 0; r < RUNS; ++r)
        {
            int m, j;
            run_at((int) threadIdx.x + r * kTileThreads, m, j);
            xv[r] = float4v {0.f, 0.f, 0.f, 0.f};
            if (m < a.rows && j < nkb * 8)
                xv[r] = *reinterpret_cast<const float4v*>(
                    a.x + (a.x_residual ? residual_index(m, kb0 * 32 + 4 * j, a.ldx) : (size_t) m * a.ldx + kb0 * 32 + 4 * j));
        }
#pragma unroll
        for (int r = 0; r < RUNS; ++r)
        {
            int m, j;
            run_at((int) threadIdx.x + r * kTileThreads, m, j);
            float4v v = xv[r];
            if (a.gamma != nullptr && m < a.rows && j < nkb * 8)
            {
                const int k = kb0 * 32 + 4 * j;
                const float4v gm = *reinterpret_cast<const float4v*>(a.gamma + k);
                const float4v bt = *reinterpret_cast<const float4v*>(a.beta + k);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (v[e] - row_mean[m]) * row_scale[m] * gm[e] + bt[e];
            }
            uint32_t lo[P], hi[P];
#pragma unroll
            for (int half = 0; half < 2; ++half)
            {
                u16 pa[P], pb[P];
                split_value<WT>(v[2 * half], pa);
                split_value<WT>(v[2 * half + 1], pb);
#pragma unroll
                for (int p = 0; p < P; ++p)
                    (half == 0 ? lo : hi)[p] = (uint32_t) pa[p] | ((uint32_t) pb[p] << 16);
            }
#pragma unroll
            for (int p = 0; p < P; ++p)
                *reinterpret_cast<uint2*>(&xs[p][m][4 * j]) = uint2 {lo[p], hi[p]};
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (u < nkb)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int p = 0; p < P; ++p)
                        acc[t] = mfma16<WT>(*reinterpret_cast<const u32x4*>(&xs[p][t * 16 + li][u * 32 + 8 * g]),
                                            wv[u], acc[t]);
        __syncthreads();
    }

    // acc[t][r] of lane (g, li) in wave w is C[16 t + 4 g + r][16 w + li].
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            tile[t * 16 + 4 * g + r][16 * wave + li] = acc[t][r];
    __syncthreads();
    float v[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c)
        v[c] = tile[m][c0 + c];

    if (a.splits > 1)
    {
        // This split's partial, in the order the reducing thread reads it.
        uint64_t* mine = reinterpret_cast<uint64_t*>(a.partials + ((size_t) blockIdx.x * kTileThreads + threadIdx.x) * CPT);
#pragma unroll
        for (int c = 0; c < CPT; c += 2)
            __hip_atomic_store(mine + c / 2,
                               (uint64_t) __float_as_uint(v[c]) | ((uint64_t) __float_as_uint(v[c + 1]) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The barrier orders every thread's partial stores before thread 0's
        // count (workgroup scope); the count is an agent-scope release, so
        // the partials are visible device-wide before it is, and an acquire,
        // so the last block reads every other block's partials after it.
        __syncthreads();
        if (threadIdx.x == 0)
        {
            const unsigned before = __hip_atomic_fetch_add(a.counters + cg, 1u, __ATOMIC_ACQ_REL,
                                                           __HIP_MEMORY_SCOPE_AGENT);
            const bool last = before == (unsigned) a.splits - 1;
            if (last)
                __hip_atomic_store(a.counters + cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_block = last;
        }
        __syncthreads();
        if (!last_block)
            return;
#pragma unroll
        for (int c = 0; c < CPT; ++c)
            v[c] = 0.f;
        for (int s0 = 0; s0 < a.splits; s0 += 4)
        {
            uint64_t part[4][CPT / 2];
#pragma unroll
            for (int s = 0; s < 4; ++s)
                if (s0 + s < a.splits)
                {
                    const uint64_t* theirs = reinterpret_cast<const uint64_t*>(
                        a.partials + (((size_t) cg * a.splits + s0 + s) * kTileThreads + threadIdx.x) * CPT);
#pragma unroll
                    for (int c = 0; c < CPT / 2; ++c)
                        part[s][c] = __hip_atomic_load(const_cast<uint64_t*>(theirs) + c, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
            for (int s = 0; s < 4; ++s)
                if (s0 + s < a.splits)
#pragma unroll
                    for (int c = 0; c < CPT / 2; ++c)
                    {
                        v[2 * c] += __uint_as_float((uint32_t) part[s][c]);
                        v[2 * c + 1] += __uint_as_float((uint32_t) (part[s][c] >> 32));
                    }
        }
    }

    // Epilogue: row m, columns n0 + c0 .. + CPT.
#pragma unroll
    for (int c = 0; c < CPT; ++c)
    {
        const int n = n0 + c0 + c;
        if (n < a.out)
            v[c] = v[c] * a.scale + (a.bias != nullptr ? a.bias[n] : 0.f);
    }
    switch (a.epilogue)
    {
        case kStore:
        case kGelu:
            if (row_in)
#pragma unroll
                for (int c = 0; c < CPT; ++c)
                {
                    const int n = n0 + c0 + c;
                    if (n < a.out)
                        a.y[(size_t) m * a.ldy + n] = a.epilogue == kGelu ? exact_gelu(v[c]) : v[c];
                }
            break;
        case kResidual:
        {
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < CPT; ++c)
            {
                const int n = n0 + c0 + c;
                if (row_in && n < a.out)
                {
                    v[c] += resid[c];
                    a.y[residual_index(m, n, a.ldy)] = v[c];
                    sum += v[c];
                }
            }
            // The group's statistics over the TPR threads of the row (lanes
            // next to each other), every pair added symmetrically.
#pragma unroll
            for (int offset = 1; offset < TPR; offset <<= 1)
                sum += __shfl_xor(sum, offset, TPR);
            const float count = (float) min(kGroupColumns, a.out - n0);
            const float mean = sum / count;
            float m2 = 0.f;
#pragma unroll
            for (int c = 0; c < CPT; ++c)
            {
                const int n = n0 + c0 + c;
                if (row_in && n < a.out)
                    m2 += (v[c] - mean) * (v[c] - mean);
            }
#pragma unroll
            for (int offset = 1; offset < TPR; offset <<= 1)
                m2 += __shfl_xor(m2, offset, TPR);
            const int groups = (a.out + kGroupColumns - 1) / kGroupColumns;
            if (row_in && threadIdx.x % TPR == 0)
            {
                a.stats_out[((size_t) m * groups + cg) * 2] = mean;
                a.stats_out[((size_t) m * groups + cg) * 2 + 1] = m2;
            }
            break;
        }
        default:
            if (row_in)
            {
                const int d = a.width;
                const int stream = m / a.step_tokens, i = m % a.step_tokens;
                const size_t row = (size_t) stream * a.stream_stride + (size_t) (*a.state + i) * d;
#pragma unroll
                for (int c = 0; c < CPT; ++c)
                {
                    const int n = n0 + c0 + c;
                    if (n < d)
                        a.q[(size_t) m * d + n] = v[c];
                    else if (n < 2 * d)
                        a.keys[row + (n - d)] = v[c];
                    else if (n < 3 * d)
                        a.values[row + (n - 2 * d)] = v[c];
                }
            }
    }
}

// ---------------------------------------------------------------------------
// Split-key attention for (row, head, chunk): the row's query against keys
// [chunk·len, min((chunk + 1)·len, visible)) of its stream's cache, visible
// being the causal limit position + i + 1 for self attention (the query at
// position + i sees every key up to itself, Kernels/Attention.h:34-47) and
// k_count for cross attention. Keys are taken
// 128 at a time; lane (group, sub) holds channels 4·sub.. of keys group + 16u
// and all its key and value loads are issued together. Tiles fold into a
// running (max, sum, row) with exact exp(m_old - m_new) rescaling; one chunk
// writes the normalised split row, several write (max, sum, row) for the
// combine (Kernels/SingleQueryAttention.h:27-37).
// ---------------------------------------------------------------------------
struct Attend
{
    const float* q;       // [rows][width]
    const float* keys;    // stream 0's cache of this layer, [capacity][width]
    const float* values;
    size_t stream_stride; // elements between streams' first keys
    size_t key_stride;    // elements between one stream's consecutive keys
    const int* state;     // device word: the position of the step's first token
    int k_count, step_tokens, causal, heads, head_width, width; // k_count: cross rows (causal: unused)
    float scale;
    int chunks, chunk_len;
    u16* xs;              // split output [parts][rows_padded][width] (fragment-major) when chunks == 1
    size_t xs_part;
    float* partials;      // [rows][heads][chunks][head_width + 2]
};

template <int WT>
__global__ void __launch_bounds__(kAttendThreads) attend_kernel(Attend a)
{
    __shared__ float wave_max[2][4];
    __shared__ float wave_sum[4];
    __shared__ float4v wave_row[4][16];

    const int chunk = blockIdx.x % a.chunks;
    const int head = (blockIdx.x / a.chunks) % a.heads;
    const int row = blockIdx.x / (a.chunks * a.heads);
    const int stream = row / a.step_tokens, i = row % a.step_tokens;
    const int sub = threadIdx.x % 16, group = threadIdx.x / 16;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int quads = a.head_width / 4;
    const int column = head * a.head_width + 4 * min(sub, quads - 1);

    float4v qv = {0.f, 0.f, 0.f, 0.f};
    if (sub < quads)
        qv = *reinterpret_cast<const float4v*>(a.q + (size_t) row * a.width + column);
    const int visible = a.causal ? *a.state + i + 1 : a.k_count;
    const int first = chunk * a.chunk_len;
    const int last = min(first + a.chunk_len, visible);
    const float* kbase = a.keys + (size_t) stream * a.stream_stride + column;
    const float* vbase = a.values + (size_t) stream * a.stream_stride + column;

    float run_max = -INFINITY, run_sum = 0.f;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    int flip = 0;
    for (int ts = first; ts < last; ts += kTileKeys)
    {
        float4v kv[8], vv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            const size_t key = (size_t) min(ts + group + 16 * u, last - 1);
            kv[u] = *reinterpret_cast<const float4v*>(kbase + key * a.key_stride);
            vv[u] = *reinterpret_cast<const float4v*>(vbase + key * a.key_stride);
        }
        float s[8];
        float tile_max = -INFINITY;
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            float part = qv[0] * kv[u][0] + qv[1] * kv[u][1] + qv[2] * kv[u][2] + qv[3] * kv[u][3];
#pragma unroll
            for (int offset = 1; offset < 16; offset <<= 1)
                part += __shfl_xor(part, offset, 16);
            s[u] = ts + group + 16 * u < last ? a.scale * part : -INFINITY;
            tile_max = fmaxf(tile_max, s[u]);
        }
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
        if (lane == 0)
            wave_max[flip][wave] = tile_max;
        __syncthreads();
        tile_max = fmaxf(fmaxf(wave_max[flip][0], wave_max[flip][1]), fmaxf(wave_max[flip][2], wave_max[flip][3]));
        flip ^= 1;

        const float new_max = fmaxf(run_max, tile_max);
        const float factor = expf(run_max - new_max);
        float psum = 0.f;
        float4v pv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            const float p = expf(s[u] - new_max);
            psum += p;
            pv += p * vv[u];
        }
        run_sum = run_sum * factor + psum;
        acc = acc * factor + pv;
        run_max = new_max;
    }

    // Sum the 16 key groups: the four of a wave by lane exchange, then the
    // four waves in order.
    run_sum += __shfl_xor(run_sum, 16);
    run_sum += __shfl_xor(run_sum, 32);
#pragma unroll
    for (int r = 0; r < 4; ++r)
    {
        acc[r] += __shfl_xor(acc[r], 16);
        acc[r] += __shfl_xor(acc[r], 32);
    }
    if (lane < 16)
    {
        wave_row[wave][lane] = acc;
        if (lane == 0)
            wave_sum[wave] = run_sum;
    }
    __syncthreads();
    if (threadIdx.x < a.head_width)
    {
        const int c = threadIdx.x, q4 = c / 4, r = c % 4;
        const float total = (wave_sum[0] + wave_sum[1]) + (wave_sum[2] + wave_sum[3]);
        const float value = (wave_row[0][q4][r] + wave_row[1][q4][r]) + (wave_row[2][q4][r] + wave_row[3][q4][r]);
        if (a.chunks == 1)
            store_split<WT>(a.xs, a.xs_part, fragment_index(row, head * a.head_width + c, a.width), value / total);
        else
        {
            float* part = a.partials + (((size_t) row * a.heads + head) * a.chunks + chunk) * (a.head_width + 2);
            part[2 + c] = value;
            if (c == 0)
            {
                part[0] = last > first ? run_max : -INFINITY;
                part[1] = total;
            }
        }
    }
}

// The chunks of one (row, head) combined in chunk order: every chunk's
// maximum is read at once (one chunk a lane) and reduced, then the factors
// exp(m_k - m) of a run of up to 64 chunks go through LDS, so the row's loads
// for the whole run are independent of each other.
template <int WT>
__global__ void __launch_bounds__(kWave) combine_kernel(const float* __restrict__ partials, int heads,
                                                        int head_width, int chunks, int width, u16* xs,
                                                        size_t xs_part)
{
    __shared__ float factor[kWave], weight[kWave];
    const int head = blockIdx.x % heads, row = blockIdx.x / heads;
    const int lane = threadIdx.x;
    const size_t stride = (size_t) head_width + 2;
    const float* base = partials + ((size_t) row * heads + head) * chunks * stride;
    float largest = -INFINITY;
    for (int k = lane; k < chunks; k += kWave)
        largest = fmaxf(largest, base[k * stride]);
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1)
        largest = fmaxf(largest, __shfl_xor(largest, offset));
    float numerator = 0.f, denominator = 0.f;
    for (int k0 = 0; k0 < chunks; k0 += kWave)
    {
        float f = 0.f, sum = 0.f;
        if (k0 + lane < chunks)
        {
            sum = base[(k0 + lane) * stride + 1];
            if (sum != 0.f) // an empty chunk (no visible key) adds nothing
                f = expf(base[(k0 + lane) * stride] - largest);
        }
        __syncthreads();
        factor[lane] = f;
        weight[lane] = f * sum;
        __syncthreads();
        const int run = min(kWave, chunks - k0);
        if (lane < head_width)
        {
            const float* column = base + (size_t) k0 * stride + 2 + lane;
#pragma unroll 8
            for (int i = 0; i < run; ++i)
            {
                numerator += factor[i] * column[i * stride];
                denominator += weight[i];
            }
        }
    }
    if (lane < head_width)
        store_split<WT>(xs, xs_part, fragment_index(row, head * head_width + lane, width), numerator / denominator);
}

// ---------------------------------------------------------------------------
// Cross attention of one query row per stream by key sweep. The cross caches
// are key-major ([key][stream][width]), and block (stream, j) takes every head
// of its stream over the key passes j, j + G, j + 2G, ... of KR·8 keys each
// (G blocks a stream, blocks of one key range adjacent), so at any time the
// chip reads one front of whole rows moving through memory instead of one
// short strided run per (head, chunk). One block a CU with nontemporal loads
// keeps about 80-128 KB of loads in flight per CU, which streams faster than
// more blocks with more loads in flight. Thread (kr, quad) holds channels
// 4·quad.. (head quad / 16) of keys first + kr + KR·u; each 16-lane row keeps
// its own running (max, sum, row) over its keys, so the loop has no barrier.
// The KR key lanes are folded in order through LDS at the end; the block then
// writes one (max, sum, row) partial per head for combine_kernel
// (Kernels/SingleQueryAttention.h:27-37), or with G = 1 the normalised row
// itself. Head width 64.
// ---------------------------------------------------------------------------
constexpr int kSweepKeys = 8;       // keys per lane per pass
constexpr int kSweepBlocksPerCU = 1;
constexpr int kSweepThreads = 512;  // most threads a sweep block takes
constexpr int kMaxSweepGroups = 32; // most blocks per stream

template <int WT>
__global__ void __launch_bounds__(kSweepThreads) sweep_attend_kernel(Attend a, int key_lanes, int groups)
{
    extern __shared__ float4v fold[]; // [key_lanes][quads] rows, then [key_lanes][heads] maxima and sums
    const int quads = a.width / 4;
    const int quad = threadIdx.x % quads, kr = threadIdx.x / quads;
    const int streams = gridDim.x / groups;
    const int stream = blockIdx.x % streams, j = blockIdx.x / streams; // blocks of one key range adjacent
    const int head = quad / 16, lane16 = quad % 16;
    const float4v qv = *reinterpret_cast<const float4v*>(a.q + (size_t) stream * a.width + 4 * quad);
    const float* kbase = a.keys + (size_t) stream * a.stream_stride + 4 * quad;
    const float* vbase = a.values + (size_t) stream * a.stream_stride + 4 * quad;
    const int pass_keys = key_lanes * kSweepKeys;

    float run_max = -INFINITY, run_sum = 0.f;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    for (int first = j * pass_keys; first < a.k_count; first += groups * pass_keys)
    {
        float4v kv[kSweepKeys], vv[kSweepKeys];
#pragma unroll
        for (int u = 0; u < kSweepKeys; ++u)
        {
            const size_t key = (size_t) min(first + kr + key_lanes * u, a.k_count - 1);
            kv[u] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(kbase + key * a.key_stride));
            vv[u] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(vbase + key * a.key_stride));
        }
        float s[kSweepKeys];
        float tile_max = -INFINITY;
#pragma unroll
        for (int u = 0; u < kSweepKeys; ++u)
        {
            const float part = sum16(qv[0] * kv[u][0] + qv[1] * kv[u][1] + qv[2] * kv[u][2] + qv[3] * kv[u][3]);
            s[u] = first + kr + key_lanes * u < a.k_count ? a.scale * part : -INFINITY;
            tile_max = fmaxf(tile_max, s[u]);
        }
        const float new_max = fmaxf(run_max, tile_max);
        if (new_max != -INFINITY) // every key of this lane's pass past the end: nothing to fold
        {
            const float factor = expf(run_max - new_max);
            float psum = 0.f;
            float4v pv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < kSweepKeys; ++u)
            {
                const float p = expf(s[u] - new_max);
                psum += p;
                pv += p * vv[u];
            }
            run_sum = run_sum * factor + psum;
            acc = acc * factor + pv;
            run_max = new_max;
        }
    }

    if (key_lanes > 1)
    {
        const int heads = quads / 16;
        float* maxima = reinterpret_cast<float*>(fold + key_lanes * quads);
        float* sums = maxima + key_lanes * heads;
        fold[kr * quads + quad] = acc;
        if (lane16 == 0)
        {
            maxima[kr * heads + head] = run_max;
            sums[kr * heads + head] = run_sum;
        }
        __syncthreads();
        if (kr != 0)
            return;
        float largest = -INFINITY;
        for (int k = 0; k < key_lanes; ++k)
            largest = fmaxf(largest, maxima[k * heads + head]);
        run_sum = 0.f;
        acc = float4v {0.f, 0.f, 0.f, 0.f};
        if (largest != -INFINITY)
            for (int k = 0; k < key_lanes; ++k)
            {
                const float factor = expf(maxima[k * heads + head] - largest);
                run_sum += factor * sums[k * heads + head];
                acc += factor * fold[k * quads + quad];
            }
        run_max = largest;
    }

    if (groups == 1)
    {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            store_split<WT>(a.xs, a.xs_part, fragment_index(stream, 4 * quad + r, a.width), acc[r] / run_sum);
        return;
    }
    float* part = a.partials + (((size_t) stream * a.heads + head) * groups + j) * (a.head_width + 2);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        part[2 + 4 * lane16 + r] = acc[r];
    if (lane16 == 0)
    {
        part[0] = run_max;
        part[1] = run_sum;
    }
}

// The step's last launch: with a ring, each stream's greedy token goes to the
// ring row of the next position; then the position word advances. One block,
// so every thread has read the position before thread 0 moves it.
__global__ void __launch_bounds__(128) advance_kernel(int* state, uint32_t* ring, const uint32_t* next, int streams,
                                                      int count)
{
    const int position = *state;
    if (ring != nullptr)
        for (int s = threadIdx.x; s < streams; s += blockDim.x)
            ring[(size_t) (position + count) * streams + s] = next[s];
    __syncthreads();
    if (threadIdx.x == 0)
        *state = position + count;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

template <int WT, int MT>
void launch_product_tiles(hipStream_t stream, const Product& a)
{
    // Prefetch the next batch's weights only when a wave has more than one
    // batch (the inner dimension is split over the block's 8 waves).
    constexpr int KB = kblocks_per_load<parts_of<WT>(), MT>();
    const int per_wave = (a.inner / 32 + kProductWaves - 1) / kProductWaves;
    const dim3 grid((a.out + 15) / 16);
    if (per_wave > KB)
        hipLaunchKernelGGL((product_kernel<WT, MT, true>), grid, dim3(kProductThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((product_kernel<WT, MT, false>), grid, dim3(kProductThreads), 0, stream, a);
}

template <int WT>
hipError_t launch_product(hipStream_t stream, const Product& a)
{
    switch (row_tiles(a.rows))
    {
        case 1: launch_product_tiles<WT, 1>(stream, a); break;
        case 2: launch_product_tiles<WT, 2>(stream, a); break;
        case 4: launch_product_tiles<WT, 4>(stream, a); break;
        default: launch_product_tiles<WT, 8>(stream, a); break;
    }
    return hipGetLastError();
}

// Decode steps (at most 32 rows, inner at most 2048) take the product with the
// LayerNorm folded in.
bool normed_fits(int rows, int inner)
{
    return row_tiles(rows) <= 2 && inner <= kNormedWidth && inner % 32 == 0;
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

template <int WT>
hipError_t launch_normed_product(hipStream_t stream, const Product& a)
{
    const int tiles = (a.out + 15) / 16;
    const bool pair = tiles > compute_units();
    const dim3 grid(pair ? (tiles + 1) / 2 : tiles);
    const bool two_rows = row_tiles(a.rows) != 1;
    if (!pair && !two_rows)
        hipLaunchKernelGGL((normed_product_kernel<WT, 1, 1>), grid, dim3(kProductThreads), 0, stream, a);
    else if (!pair)
        hipLaunchKernelGGL((normed_product_kernel<WT, 2, 1>), grid, dim3(kProductThreads), 0, stream, a);
    else if (!two_rows)
        hipLaunchKernelGGL((normed_product_kernel<WT, 1, 2>), grid, dim3(kProductThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((normed_product_kernel<WT, 2, 2>), grid, dim3(kProductThreads), 0, stream, a);
    return hipGetLastError();
}

template <int WT>
hipError_t launch_norm(hipStream_t stream, const Norm& a, int rows, bool embed)
{
    if (embed)
        hipLaunchKernelGGL((norm_kernel<WT, true>), dim3(rows), dim3(kNormThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((norm_kernel<WT, false>), dim3(rows), dim3(kNormThreads), 0, stream, a);
    return hipGetLastError();
}

// Splits of the inner dimension for a tile product: eight runs (as measured
// best for fc2 at the medium and large-v3 shapes), whole k-blocks each.
void plan_splits(Tile& a, bool can_split)
{
    plan_split_runs(a.inner, can_split, a.kb_per_split, a.splits);
}

template <int WT, int MT>
void launch_tile_rows(hipStream_t stream, const Tile& a)
{
    const int groups = (a.out + kTileColumns - 1) / kTileColumns;
    if (a.short_batches)
        hipLaunchKernelGGL((tile_kernel<WT, MT, 2>), dim3(groups * a.splits), dim3(kTileThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((tile_kernel<WT, MT, 10>), dim3(groups * a.splits), dim3(kTileThreads), 0, stream, a);
}

template <int WT>
hipError_t launch_tile(hipStream_t stream, const Tile& a)
{
    // A split launch writes 64 x (16 row tiles) partial floats per block and
    // counts on one counter per column group: refuse it when the buffers are
    // smaller than that.
    if (!split_launch_fits(a.out, a.rows, a.splits, a.partials_capacity, a.counters_capacity))
        return hipErrorInvalidValue;
    switch (row_tiles(a.rows))
    {
        case 1: launch_tile_rows<WT, 1>(stream, a); break;
        case 2: launch_tile_rows<WT, 2>(stream, a); break;
        case 4: launch_tile_rows<WT, 4>(stream, a); break;
        default: launch_tile_rows<WT, 8>(stream, a); break;
    }
    return hipGetLastError();
}

// Key chunks for `units` (row, head) pairs over k_count keys: about `target`
// blocks in all, no chunk shorter than one 128-key tile. Cross attention
// (1500 keys a stream) aims at one full round of resident blocks (blocks per
// CU x CUs: 1536 on MI355X, which measured faster than 1024, 2048, 3072 or
// 4096); self attention at 256, so a large batch covers the chip without the
// combine launch.
int attend_chunks(int units, int k_count, int target)
{
    const int most = std::max(1, (k_count + kTileKeys - 1) / kTileKeys);
    return std::max(1, std::min(most, (target + units - 1) / units));
}

// Attention of `rows` query rows whose keys number at most `span`; a.chunks
// and a.chunk_len are planned here for that span (chunks past the visible keys
// come out empty, which the combine skips).
template <int WT>
hipError_t launch_attend(hipStream_t stream, Attend a, int rows, int span, int cross_target)
{
    a.chunks = attend_chunks(rows * a.heads, span, a.causal ? 256 : cross_target);
    a.chunk_len = (span + a.chunks - 1) / a.chunks;
    a.chunks = (span + a.chunk_len - 1) / a.chunk_len;
    hipLaunchKernelGGL((attend_kernel<WT>), dim3(rows * a.heads * a.chunks), dim3(kAttendThreads), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.chunks == 1)
        return e;
    hipLaunchKernelGGL((combine_kernel<WT>), dim3(rows * a.heads), dim3(kWave), 0, stream, a.partials, a.heads,
                       a.head_width, a.chunks, a.width, a.xs, a.xs_part);
    return hipGetLastError();
}

// Key lanes of a sweep block for this width: the fewest that make whole
// waves (medium: one lane of 256 threads measured as fast as two of 512, or
// two blocks a CU); 0 when the shape does not fit (head width other than 64,
// or one key lane already too wide).
int sweep_key_lanes(int width, int heads)
{
    if (heads <= 0 || width != heads * 64)
        return 0;
    const int quads = width / 4;
    int lanes = 1;
    while ((quads * lanes) % kWave != 0)
        lanes *= 2;
    if (quads * lanes > kSweepThreads)
        return 0;
    return lanes;
}

// Cross attention of one row per stream by key sweep: about `target` blocks
// (a whole number per stream, at most kMaxSweepGroups and at most one per key
// pass), then the combine of each (stream, head)'s partials.
template <int WT>
hipError_t launch_sweep_attend(hipStream_t stream, Attend a, int streams, int lanes, int target)
{
    const int quads = a.width / 4;
    const int pass_keys = lanes * kSweepKeys;
    const int passes = (a.k_count + pass_keys - 1) / pass_keys;
    const int groups = std::max(1, std::min({kMaxSweepGroups, passes, (target + streams / 2) / streams}));
    const size_t lds = lanes > 1 ? (size_t) lanes * quads * sizeof(float4v) + 2 * (size_t) lanes * a.heads * sizeof(float)
                                 : 0;
    hipLaunchKernelGGL((sweep_attend_kernel<WT>), dim3(streams * groups), dim3(quads * lanes), lds, stream, a, lanes,
                       groups);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || groups == 1)
        return e;
    hipLaunchKernelGGL((combine_kernel<WT>), dim3(streams * a.heads), dim3(kWave), 0, stream, a.partials, a.heads,
                       a.head_width, groups, a.width, a.xs, a.xs_part);
    return hipGetLastError();
}
} // namespace
} // namespace wsp::batch

// ---------------------------------------------------------------------------
// The batch context and its C ABI
// ---------------------------------------------------------------------------
struct wsp_batch
{
    wsp_decoder_shape shape {};
    int streams = 0, max_step_tokens = 0, wdtype = 0, device = 0;
    hipStream_t stream = nullptr;
    int rows_cap = 0, rows_padded = 0;
    int position = 0, cross_rows = 0;
    int cross_target = 1536; // cross-attention blocks per launch: one round of resident blocks
    int sweep_target = 512;  // key-sweep cross-attention blocks per launch

    float* self_keys = nullptr;   // [layers][streams][max_positions][width]
    float* self_values = nullptr;
    float* cross_keys = nullptr;  // [layers][cross_positions][streams][width]
    float* cross_values = nullptr;
    float* cross_scratch = nullptr; // [cross_positions][width], made by the first begin that needs it
    float* h = nullptr;           // [rows_padded][width] residual stream, fragment-major (residual_index)
    float* q = nullptr;           // [rows_padded][width] queries
    uint16_t* xs = nullptr;       // [parts][rows_padded][width]
    float* ff = nullptr;          // [rows_padded][feed_forward] gelu(fc1) rows
    float* stats = nullptr;       // [rows_padded][width / 64][2] LayerNorm statistics of h after fc2
    float* partials = nullptr;    // attention chunk partials
    float* tile_partials = nullptr; // split products' partial tiles
    unsigned* counters = nullptr; // split products' per-group counters (zero between launches)
    size_t tile_partials_capacity = 0, counters_capacity = 0; // floats, counters
    float* argmax_values = nullptr;
    uint32_t* argmax_indices = nullptr;
    int* state = nullptr;         // device word: the position of the next step's first token
    uint32_t* next = nullptr;     // [streams] greedy tokens of a ring step
    std::vector<void*> owned;

    // Fragment-major copies of the projection and tied logits weights the
    // step's products read, packed from the caller's table when a table is
    // first seen (packed_table: the table they came from).
    uint16_t* packed = nullptr;
    std::vector<char> packed_table;
    std::vector<wsp_layer_tensors> packed_layers;
    wsp_decoder_tensors packed_tensors {};
    // bf16 tables: the copies hold exact fp16 multiples w·2^k when every
    // matrix narrows exactly (compute WSP_F16, scales[i] = 2^-k of matrix i:
    // per layer q/k/v, out, cross q, cross out, fc1, fc2, then the logits);
    // else bf16 as given (compute WSP_BF16, scales 1). `range` is device
    // scratch for the check, three words a matrix.
    int compute = 0;
    std::vector<float> scales;
    unsigned* range = nullptr;

    // The single-token ring step, captured once as a HIP graph on a private
    // stream and replayed on `stream`; re-captured when anything it bakes in
    // (ring, logits, mask, cross rows, the weight table) changes.
    hipStream_t capture = nullptr;
    hipGraphExec_t graph = nullptr;
    const void* graph_ring = nullptr;
    const void* graph_logits = nullptr;
    const void* graph_mask = nullptr;
    int graph_cross_rows = -1;
    std::vector<char> graph_table;

    char error[512] = {0};
};

namespace
{
using wsp::batch::u16;

int fail(wsp_batch* b, int code, const char* message)
{
    std::snprintf(b->error, sizeof b->error, "%s", message);
    return code;
}

int hip_fail(wsp_batch* b, hipError_t e, const char* what)
{
    if (e == hipSuccess)
        return WSP_OK;
    std::snprintf(b->error, sizeof b->error, "%s: %s", what, hipGetErrorString(e));
    return WSP_ERR_HIP;
}

int parts_for(int wdtype)
{
    return wdtype == WSP_F16 ? 2 : 3;
}

size_t self_layer_stride(const wsp_batch* b)
{
    return (size_t) b->streams * b->shape.max_positions * b->shape.width;
}

size_t cross_layer_stride(const wsp_batch* b)
{
    return (size_t) b->streams * b->shape.cross_positions * b->shape.width;
}

// Cross caches are key-major, [cross_positions][streams][width]: key k of
// every stream is one contiguous run, so the blocks of a key sweep that take
// the same keys of all streams read one front of memory together.
size_t cross_stream_stride(const wsp_batch* b)
{
    return (size_t) b->shape.width;
}

size_t cross_key_stride(const wsp_batch* b)
{
    return (size_t) b->streams * b->shape.width;
}

void release(wsp_batch* b)
{
    for (void* p : b->owned)
        (void) hipFree(p);
    b->owned.clear();
}

template <typename T>
hipError_t allocate(wsp_batch* b, T** out, size_t elements)
{
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, std::max<size_t>(elements, 1) * sizeof(T));
    if (e == hipSuccess)
    {
        b->owned.push_back(p);
        *out = static_cast<T*>(p);
    }
    return e;
}

// What one step reads and writes. Either `tokens` ([streams][count]) and an
// optional `argmax_out` ([streams]), or — one token per stream — a `ring`
// read at the device position and written at the next (fixed_grid then plans
// the self attention for max_positions keys, so nothing in the launches
// depends on the position and the step can be replayed from a graph).
struct StepIo
{
    const uint32_t* tokens;
    uint32_t* ring;
    int count;
    float* hidden;
    float* logits;
    const float* mask;
    uint32_t* argmax_out;
    bool fixed_grid;
};

template <int WT>
int run_step(wsp_batch* b, const wsp_decoder_tensors* T, const StepIo& io, hipStream_t st)
{
    const int count = io.count;
    float* const hidden = io.hidden;
    float* const logits = io.logits;
    const float* const mask = io.mask;
    using namespace wsp::batch;
    const wsp_decoder_shape& s = b->shape;
    const int d = s.width, f = s.feed_forward_width, H = s.heads, hd = d / H;
    const int rows = b->streams * count;
    const size_t xs_part = (size_t) b->rows_padded * d;
    const int groups = (d + kGroupColumns - 1) / kGroupColumns;
    const float eps = 1e-5f;
    const float scale = 1.f / std::sqrt((float) hd);
    hipError_t e = hipSuccess;

    Norm n {};
    n.h = b->h;
    n.width = d;
    n.eps = eps;
    n.xs = b->xs;
    n.xs_part = xs_part;
    n.tokens = io.tokens;
    n.ring = io.ring;
    n.state = b->state;
    n.streams = b->streams;
    n.token_table = T->token_embedding;
    n.position_table = T->position_embedding;
    n.step_tokens = count;
    n.vocabulary = s.vocabulary_size;

    Product p {};
    p.x = b->xs;
    p.x_part = xs_part;
    p.rows = rows;
    p.inner = d;

    Tile tile {};
    tile.rows = rows;
    tile.stats_in = b->stats;
    tile.stat_groups = groups;
    tile.eps = eps;
    tile.stats_out = b->stats;
    tile.partials = b->tile_partials;
    tile.counters = b->counters;
    tile.partials_capacity = b->tile_partials_capacity;
    tile.counters_capacity = b->counters_capacity;

    Attend at {};
    at.q = b->q;
    at.step_tokens = count;
    at.heads = H;
    at.head_width = hd;
    at.width = d;
    at.scale = scale;
    at.xs = b->xs;
    at.xs_part = xs_part;
    at.partials = b->partials;
    at.state = b->state;
    const int self_span = io.fixed_grid ? s.max_positions : b->position + count;
    // One query row per stream: the cross attention sweeps each stream's keys.
    const int sweep_lanes = count == 1 ? wsp::batch::sweep_key_lanes(d, H) : 0;

    // Decode steps fold each LayerNorm into the product that consumes it.
    const bool normed = wsp::batch::normed_fits(rows, d);
    p.h = b->h;
    p.eps = eps;
    auto product_after_norm = [&](const float* gamma, const float* beta) -> hipError_t {
        if (!normed)
            return launch_product<WT>(st, p);
        Product q = p;
        q.gamma = gamma;
        q.beta = beta;
        return wsp::batch::launch_normed_product<WT>(st, q);
    };

    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = T->layers[l];
        float* self_k = b->self_keys + (size_t) l * self_layer_stride(b);
        float* self_v = b->self_values + (size_t) l * self_layer_stride(b);
        const float* cross_k = b->cross_keys + (size_t) l * cross_layer_stride(b);
        const float* cross_v = b->cross_values + (size_t) l * cross_layer_stride(b);

        // self attention
        n.gamma = L.self_norm_w;
        n.beta = L.self_norm_b;
        n.y = nullptr;
        n.xs = normed ? nullptr : b->xs;
        if ((l == 0 || !normed) && (e = launch_norm<WT>(st, n, rows, l == 0)) != hipSuccess)
            return hip_fail(b, e, "self-attention norm");
        n.xs = b->xs;

        p.x = b->xs;
        p.x_part = xs_part;
        p.inner = d;
        p.out = 3 * d;
        const float* const scales = b->scales.data() + (size_t) 6 * l;
        p.w = L.self_qkv_w;
        p.scale = scales[0];
        p.bias = L.self_qkv_b;
        p.epilogue = kQkv;
        p.q = b->q;
        p.keys = self_k;
        p.values = self_v;
        p.stream_stride = (size_t) s.max_positions * d;
        p.state = b->state;
        p.step_tokens = count;
        p.width = d;
        if ((e = product_after_norm(L.self_norm_w, L.self_norm_b)) != hipSuccess)
            return hip_fail(b, e, "q/k/v product");

        at.keys = self_k;
        at.values = self_v;
        at.stream_stride = (size_t) s.max_positions * d;
        at.key_stride = d;
        at.k_count = 0;
        at.causal = 1;
        if ((e = launch_attend<WT>(st, at, rows, self_span, b->cross_target)) != hipSuccess)
            return hip_fail(b, e, "self attention");

        p.out = d;
        p.w = L.self_out_w;
        p.scale = scales[1];
        p.bias = L.self_out_b;
        p.epilogue = kResidual;
        p.y = b->h;
        p.ldy = d;
        if ((e = launch_product<WT>(st, p)) != hipSuccess)
            return hip_fail(b, e, "self-attention output product");

        // cross attention
        n.gamma = L.cross_norm_w;
        n.beta = L.cross_norm_b;
        if (!normed && (e = launch_norm<WT>(st, n, rows, false)) != hipSuccess)
            return hip_fail(b, e, "cross-attention norm");
        p.w = L.cross_q_w;
        p.scale = scales[2];
        p.bias = L.cross_q_b;
        p.epilogue = kStore;
        p.y = b->q;
        if ((e = product_after_norm(L.cross_norm_w, L.cross_norm_b)) != hipSuccess)
            return hip_fail(b, e, "cross query product");

        at.keys = cross_k;
        at.values = cross_v;
        at.stream_stride = cross_stream_stride(b);
        at.key_stride = cross_key_stride(b);
        at.k_count = b->cross_rows;
        at.causal = 0;
        e = sweep_lanes > 0 ? launch_sweep_attend<WT>(st, at, rows, sweep_lanes, b->sweep_target)
                            : launch_attend<WT>(st, at, rows, b->cross_rows, b->cross_target);
        if (e != hipSuccess)
            return hip_fail(b, e, "cross attention");

        p.w = L.cross_out_w;
        p.scale = scales[3];
        p.bias = L.cross_out_b;
        p.epilogue = kResidual;
        p.y = b->h;
        if ((e = launch_product<WT>(st, p)) != hipSuccess)
            return hip_fail(b, e, "cross-attention output product");

        // feed-forward
        n.gamma = L.final_norm_w;
        n.beta = L.final_norm_b;
        if (!normed && (e = launch_norm<WT>(st, n, rows, false)) != hipSuccess)
            return hip_fail(b, e, "feed-forward norm");
        p.out = f;
        p.w = L.fc1_w;
        p.scale = scales[4];
        p.bias = L.fc1_b;
        p.epilogue = kGelu;
        p.y = b->ff;
        p.ldy = f;
        if ((e = product_after_norm(L.final_norm_w, L.final_norm_b)) != hipSuccess)
            return hip_fail(b, e, "fc1 product");

        // fc2 (inner 4d) as a split tile product: its epilogue also leaves
        // the LayerNorm statistics of h for the final norm and the logits.
        Tile t = tile;
        t.x = b->ff;
        t.ldx = f;
        t.inner = f;
        t.out = d;
        t.w = L.fc2_w;
        t.scale = scales[5];
        t.bias = L.fc2_b;
        t.epilogue = kResidual;
        t.y = b->h;
        t.ldy = d;
        plan_splits(t, true);
        if ((e = launch_tile<WT>(st, t)) != hipSuccess)
            return hip_fail(b, e, "fc2 product");
    }

    if (hidden != nullptr)
    {
        hipLaunchKernelGGL(hidden_kernel, dim3(rows), dim3(kNormThreads), 0, st, b->h, b->stats, groups, d,
                           T->final_norm_w, T->final_norm_b, eps, hidden);
        if ((e = hipGetLastError()) != hipSuccess)
            return hip_fail(b, e, "final norm");
    }
    {
        // The tied logits over the final LayerNorm of h, folded into the tile
        // product (64 vocabulary rows a block).
        Tile t = tile;
        t.x = b->h;
        t.x_residual = 1;
        t.short_batches = 1;
        t.ldx = d;
        t.inner = d;
        t.out = s.vocabulary_size;
        t.w = T->logits_weight;
        t.scale = b->scales[(size_t) 6 * s.layers];
        t.gamma = T->final_norm_w;
        t.beta = T->final_norm_b;
        t.epilogue = kStore;
        t.y = logits;
        t.ldy = s.vocabulary_size;
        plan_splits(t, false);
        if ((e = launch_tile<WT>(st, t)) != hipSuccess)
            return hip_fail(b, e, "logits product");
    }

    uint32_t* const argmax_out = io.ring != nullptr ? b->next : io.argmax_out;
    if (argmax_out != nullptr)
    {
        const size_t V = (size_t) s.vocabulary_size;
        e = wsp::ops::argmax_rows(st, logits + (size_t) (count - 1) * V, b->streams, (size_t) count * V,
                                  s.vocabulary_size, mask, argmax_out, b->argmax_values, b->argmax_indices);
        if (e != hipSuccess)
            return hip_fail(b, e, "argmax");
    }
    hipLaunchKernelGGL(wsp::batch::advance_kernel, dim3(1), dim3(128), 0, st, b->state, io.ring, b->next, b->streams,
                       count);
    if ((e = hipGetLastError()) != hipSuccess)
        return hip_fail(b, e, "position advance");
    return WSP_OK;
}

bool same_table(const wsp_batch* b, const std::vector<char>& table)
{
    return b->graph_table.size() == table.size() && std::memcmp(b->graph_table.data(), table.data(), table.size()) == 0;
}

// The bytes the captured step bakes in from the weight table.
std::vector<char> table_bytes(const wsp_decoder_tensors* T, int layers)
{
    std::vector<char> bytes(sizeof(wsp_decoder_tensors) + sizeof(wsp_layer_tensors) * (size_t) layers);
    wsp_decoder_tensors top = *T;
    top.layers = nullptr;
    std::memcpy(bytes.data(), &top, sizeof top);
    std::memcpy(bytes.data() + sizeof top, T->layers, sizeof(wsp_layer_tensors) * (size_t) layers);
    return bytes;
}

// 16-bit values of every fragment-major weight copy of one batch.
size_t packed_capacity(const wsp_decoder_shape& s)
{
    using wsp::batch::packed_size;
    const int d = s.width, f = s.feed_forward_width;
    return (size_t) s.layers * (packed_size(3 * d, d) + 3 * packed_size(d, d) + packed_size(f, d) + packed_size(d, f))
           + packed_size(s.vocabulary_size, d);
}

// The caller's table with every projection and the logits weight replaced by
// its fragment-major copy, packed (on the batch's stream) when this table has
// not been seen before. A table with the same pointers is taken to hold the
// same weights. Null on failure, with the status in `status`.
const wsp_decoder_tensors* packed_weights(wsp_batch* b, const wsp_decoder_tensors* T, int& status)
{
    std::vector<char> table = table_bytes(T, b->shape.layers);
    if (b->packed_table.size() == table.size() && std::memcmp(b->packed_table.data(), table.data(), table.size()) == 0)
        return &b->packed_tensors;
    const wsp_decoder_shape& s = b->shape;
    const int d = s.width, f = s.feed_forward_width;
    if (T->logits_weight == nullptr)
    {
        status = fail(b, WSP_ERR_ARGUMENT, "batch step: null logits weight");
        return nullptr;
    }
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = T->layers[l];
        if (L.self_qkv_w == nullptr || L.self_out_w == nullptr || L.cross_q_w == nullptr || L.cross_out_w == nullptr
            || L.fc1_w == nullptr || L.fc2_w == nullptr)
        {
            status = fail(b, WSP_ERR_ARGUMENT, "batch step: a layer without projection weights");
            return nullptr;
        }
    }
    b->packed_table.clear();
    hipError_t e = hipSuccess;
    // Every matrix in packing order: per layer q/k/v, out, cross q, cross
    // out, fc1, fc2, then the logits weight.
    struct Matrix
    {
        const void* w;
        int rows, inner;
    };
    std::vector<Matrix> matrices;
    for (int l = 0; l < s.layers; ++l)
    {
        const wsp_layer_tensors& L = T->layers[l];
        matrices.push_back({L.self_qkv_w, 3 * d, d});
        matrices.push_back({L.self_out_w, d, d});
        matrices.push_back({L.cross_q_w, d, d});
        matrices.push_back({L.cross_out_w, d, d});
        matrices.push_back({L.fc1_w, f, d});
        matrices.push_back({L.fc2_w, d, f});
    }
    matrices.push_back({T->logits_weight, s.vocabulary_size, d});
    const size_t M = matrices.size();
    b->compute = b->wdtype;
    b->scales.assign(M, 1.f);
    std::vector<int> shifts(M, 0);
    if (b->wdtype == WSP_BF16 && b->range != nullptr)
    {
        // The shift puts each matrix's largest magnitude in fp16's top binade
        // [2^15, 2^16) (an 8-bit significand there is at most 65280); at most
        // 126, so 2^-shift stays a normal float.
        std::vector<unsigned> words(3 * M);
        e = hipMemsetAsync(b->range, 0, words.size() * sizeof(unsigned), b->stream);
        for (size_t i = 0; i < M && e == hipSuccess; ++i)
        {
            const size_t n = (size_t) matrices[i].rows * matrices[i].inner;
            const unsigned blocks = (unsigned) std::min<size_t>((n + 255) / 256, 1024);
            hipLaunchKernelGGL(wsp::batch::bf16_range_kernel, dim3(blocks), dim3(256), 0, b->stream,
                               static_cast<const uint16_t*>(matrices[i].w), n, b->range + 3 * i);
            e = hipGetLastError();
        }
        if (e == hipSuccess)
            e = hipMemcpyAsync(words.data(), b->range, words.size() * sizeof(unsigned), hipMemcpyDeviceToHost,
                               b->stream);
        if (e == hipSuccess)
            e = hipStreamSynchronize(b->stream);
        bool finite = e == hipSuccess;
        for (size_t i = 0; i < M && finite; ++i)
        {
            finite = words[3 * i + 1] == 0;
            const unsigned top = words[3 * i];
            const int exponent = top == 0 ? 0 : std::ilogb(__builtin_bit_cast(float, top << 16));
            shifts[i] = top == 0 ? 0 : std::min(15 - exponent, 126);
        }
        if (finite)
        {
            uint16_t* at = b->packed;
            for (size_t i = 0; i < M && e == hipSuccess; ++i)
            {
                const Matrix& m = matrices[i];
                const size_t values = wsp::batch::packed_size(m.rows, m.inner), chunks = values / 8;
                hipLaunchKernelGGL(wsp::batch::pack_scaled_kernel, dim3((unsigned) ((chunks + 255) / 256)), dim3(256),
                                   0, b->stream, static_cast<const uint16_t*>(m.w), m.rows, m.inner, at, chunks,
                                   shifts[i], b->range + 3 * i + 2);
                e = hipGetLastError();
                at += values;
            }
            if (e == hipSuccess)
                e = hipMemcpyAsync(words.data(), b->range, words.size() * sizeof(unsigned), hipMemcpyDeviceToHost,
                                   b->stream);
            if (e == hipSuccess)
                e = hipStreamSynchronize(b->stream);
            bool exact = e == hipSuccess;
            for (size_t i = 0; i < M && exact; ++i)
                exact = words[3 * i + 2] == 0;
            if (exact)
            {
                b->compute = WSP_F16;
                for (size_t i = 0; i < M; ++i)
                    b->scales[i] = std::ldexp(1.f, -shifts[i]);
            }
        }
        if (e != hipSuccess)
        {
            status = hip_fail(b, e, "weight range check");
            return nullptr;
        }
    }
    uint16_t* at = b->packed;
    auto pack = [&](const void* w, int rows, int inner) -> const void* {
        const size_t values = wsp::batch::packed_size(rows, inner), chunks = values / 8;
        if (e == hipSuccess && b->compute == b->wdtype)
        {
            hipLaunchKernelGGL(wsp::batch::pack_fragments_kernel, dim3((unsigned) ((chunks + 255) / 256)), dim3(256),
                               0, b->stream, static_cast<const uint16_t*>(w), rows, inner, at, chunks);
            e = hipGetLastError();
        }
        const void* out = at;
        at += values;
        return out;
    };
    b->packed_layers.assign(T->layers, T->layers + s.layers);
    for (int l = 0; l < s.layers; ++l)
    {
        wsp_layer_tensors& L = b->packed_layers[l];
        L.self_qkv_w = pack(L.self_qkv_w, 3 * d, d);
        L.self_out_w = pack(L.self_out_w, d, d);
        L.cross_q_w = pack(L.cross_q_w, d, d);
        L.cross_out_w = pack(L.cross_out_w, d, d);
        L.fc1_w = pack(L.fc1_w, f, d);
        L.fc2_w = pack(L.fc2_w, d, f);
    }
    b->packed_tensors = *T;
    b->packed_tensors.layers = b->packed_layers.data();
    b->packed_tensors.logits_weight = pack(T->logits_weight, s.vocabulary_size, d);
    if (e != hipSuccess)
    {
        status = hip_fail(b, e, "weight packing");
        return nullptr;
    }
    b->packed_table = std::move(table);
    return &b->packed_tensors;
}

void drop_graph(wsp_batch* b)
{
    if (b->graph != nullptr)
        (void) hipGraphExecDestroy(b->graph);
    b->graph = nullptr;
    b->graph_table.clear();
}

template <int WT>
int capture_ring_step(wsp_batch* b, const wsp_decoder_tensors* T, uint32_t* ring, float* logits, const float* mask)
{
    drop_graph(b);
    hipError_t e = hipStreamBeginCapture(b->capture, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess)
        return hip_fail(b, e, "graph capture");
    StepIo io {nullptr, ring, 1, nullptr, logits, mask, nullptr, true};
    const int status = run_step<WT>(b, T, io, b->capture);
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(b->capture, &graph);
    if (status != WSP_OK)
    {
        if (graph != nullptr)
            (void) hipGraphDestroy(graph);
        return status;
    }
    if (e != hipSuccess)
        return hip_fail(b, e, "graph capture");
    e = hipGraphInstantiate(&b->graph, graph, nullptr, nullptr, 0);
    (void) hipGraphDestroy(graph);
    if (e != hipSuccess)
    {
        b->graph = nullptr;
        return hip_fail(b, e, "graph instantiate");
    }
    b->graph_ring = ring;
    b->graph_logits = logits;
    b->graph_mask = mask;
    b->graph_cross_rows = b->cross_rows;
    b->graph_table = table_bytes(T, b->shape.layers);
    return WSP_OK;
}
} // namespace

extern "C" {

int wsp_batch_create(const wsp_decoder_shape* shape, int streams, int max_step_tokens, int wdtype, int device,
                     void* stream, wsp_batch** out)
{
    if (shape == nullptr || out == nullptr)
        return WSP_ERR_ARGUMENT;
    *out = nullptr;
    const wsp_decoder_shape& s = *shape;
    if (s.width <= 0 || s.heads <= 0 || s.layers <= 0 || s.feed_forward_width <= 0 || s.vocabulary_size <= 0
        || s.max_positions <= 0 || s.cross_positions <= 0 || streams <= 0 || max_step_tokens <= 0)
        return WSP_ERR_ARGUMENT;
    if (wdtype != WSP_F16 && wdtype != WSP_BF16)
        return WSP_ERR_LOGIC;
    if (s.width % s.heads != 0 || (s.width / s.heads) % 4 != 0 || s.width / s.heads > 64 || s.width % 32 != 0
        || s.feed_forward_width % 32 != 0)
        return WSP_ERR_SHAPE;
    if ((long long) streams * max_step_tokens > 16 * wsp::batch::kMaxRowTiles)
        return WSP_ERR_CAPACITY;

    wsp_batch* b = new (std::nothrow) wsp_batch;
    if (b == nullptr)
        return WSP_ERR_HIP;
    b->shape = s;
    b->streams = streams;
    b->max_step_tokens = max_step_tokens;
    b->wdtype = wdtype;
    b->device = device;
    b->stream = static_cast<hipStream_t>(stream);
    b->rows_cap = streams * max_step_tokens;
    b->rows_padded = 16 * wsp::batch::row_tiles(b->rows_cap);

    const int P = parts_for(wdtype);
    const size_t d = (size_t) s.width, H = (size_t) s.heads, hd = d / H;
    const size_t stat_groups = (d + wsp::batch::kGroupColumns - 1) / wsp::batch::kGroupColumns;
    const size_t split_groups = (d + wsp::batch::kTileColumns - 1) / wsp::batch::kTileColumns; // fc2
    const int most_chunks = std::max({(s.cross_positions + wsp::batch::kTileKeys - 1) / wsp::batch::kTileKeys,
                                      (s.max_positions + wsp::batch::kTileKeys - 1) / wsp::batch::kTileKeys,
                                      wsp::batch::kMaxSweepGroups});
    const int groups = wsp::ops::argmax_groups(s.vocabulary_size);
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess)
        e = allocate(b, &b->self_keys, (size_t) s.layers * self_layer_stride(b));
    if (e == hipSuccess)
        e = allocate(b, &b->self_values, (size_t) s.layers * self_layer_stride(b));
    if (e == hipSuccess)
        e = allocate(b, &b->cross_keys, (size_t) s.layers * cross_layer_stride(b));
    if (e == hipSuccess)
        e = allocate(b, &b->cross_values, (size_t) s.layers * cross_layer_stride(b));
    if (e == hipSuccess)
        e = allocate(b, &b->h, (size_t) b->rows_padded * d);
    if (e == hipSuccess)
        e = allocate(b, &b->q, (size_t) b->rows_padded * d);
    if (e == hipSuccess)
        e = allocate(b, &b->xs, (size_t) P * b->rows_padded * d);
    if (e == hipSuccess)
        e = allocate(b, &b->ff, (size_t) b->rows_padded * s.feed_forward_width);
    if (e == hipSuccess)
        e = allocate(b, &b->packed, packed_capacity(s));
    if (e == hipSuccess)
        e = allocate(b, &b->stats, (size_t) b->rows_padded * stat_groups * 2);
    b->tile_partials_capacity = wsp::batch::split_partials_capacity(split_groups, b->rows_padded);
    b->counters_capacity = split_groups;
    if (e == hipSuccess)
        e = allocate(b, &b->tile_partials, b->tile_partials_capacity);
    if (e == hipSuccess)
        e = allocate(b, &b->counters, split_groups);
    if (e == hipSuccess)
        e = hipMemsetAsync(b->counters, 0, split_groups * sizeof(unsigned), b->stream);
    if (e == hipSuccess)
        e = allocate(b, &b->partials, (size_t) b->rows_cap * H * most_chunks * (hd + 2));
    if (e == hipSuccess)
        e = allocate(b, &b->argmax_values, (size_t) streams * groups);
    if (e == hipSuccess)
        e = allocate(b, &b->argmax_indices, (size_t) streams * groups);
    if (e == hipSuccess)
        e = allocate(b, &b->state, 4);
    if (e == hipSuccess)
        e = allocate(b, &b->next, (size_t) streams);
    if (e == hipSuccess && wdtype == WSP_BF16)
        e = allocate(b, &b->range, (size_t) 3 * (6 * s.layers + 1));
    if (e == hipSuccess)
        e = hipMemsetAsync(b->state, 0, 4 * sizeof(int), b->stream);
    if (e == hipSuccess)
        e = hipStreamCreateWithFlags(&b->capture, hipStreamNonBlocking);
    if (e == hipSuccess)
    {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess
            && hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu,
                                                            wdtype == WSP_F16
                                                                ? (const void*) wsp::batch::attend_kernel<wsp::kF16>
                                                                : (const void*) wsp::batch::attend_kernel<wsp::kBF16>,
                                                            wsp::batch::kAttendThreads, 0) == hipSuccess
            && cus > 0 && per_cu > 0)
            b->cross_target = cus * per_cu;
        if (cus > 0)
            b->sweep_target = wsp::batch::kSweepBlocksPerCU * cus;
    }
    // Padding rows of the split buffer are read by the products (their sums
    // are discarded); zero them once so they hold finite values.
    if (e == hipSuccess)
        e = hipMemsetAsync(b->xs, 0, (size_t) P * b->rows_padded * d * sizeof(u16), b->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(b->stream);
    if (e != hipSuccess)
    {
        if (b->capture != nullptr)
            (void) hipStreamDestroy(b->capture);
        release(b);
        delete b;
        return WSP_ERR_HIP;
    }
    *out = b;
    return WSP_OK;
}

void wsp_batch_destroy(wsp_batch* b)
{
    if (b == nullptr)
        return;
    (void) hipSetDevice(b->device);
    (void) hipStreamSynchronize(b->stream);
    drop_graph(b);
    if (b->capture != nullptr)
        (void) hipStreamDestroy(b->capture);
    release(b);
    delete b;
}

const char* wsp_batch_last_error(const wsp_batch* b)
{
    return b == nullptr ? "null batch" : b->error;
}

int wsp_batch_product_storage(const wsp_batch* b)
{
    return b == nullptr || b->packed_table.empty() ? 0 : b->compute;
}

int wsp_batch_position(const wsp_batch* b)
{
    return b == nullptr ? -1 : b->position;
}

int wsp_batch_cross_rows(const wsp_batch* b)
{
    return b == nullptr ? -1 : b->cross_rows;
}

int wsp_batch_begin(wsp_batch* b, const wsp_cross_tensors* layers, int wdtype, const float* encoder_rows,
                    int cross_rows)
{
    if (b == nullptr)
        return WSP_ERR_ARGUMENT;
    b->error[0] = 0;
    if (layers == nullptr || encoder_rows == nullptr)
        return fail(b, WSP_ERR_ARGUMENT, "wsp_batch_begin: null layer table or encoder rows");
    if (cross_rows == 0)
        cross_rows = b->shape.cross_positions;
    if (cross_rows < 0 || cross_rows > b->shape.cross_positions)
        return fail(b, WSP_ERR_SHAPE, "wsp_batch_begin: more cross rows than the batch was sized for");
    const int d = b->shape.width;
    for (int l = 0; l < b->shape.layers; ++l)
    {
        const wsp_cross_tensors& L = layers[l];
        if (L.key_w == nullptr || L.value_w == nullptr)
            return fail(b, WSP_ERR_ARGUMENT, "wsp_batch_begin: a layer without cross key/value weights");
        float* keys = b->cross_keys + (size_t) l * cross_layer_stride(b);
        float* values = b->cross_values + (size_t) l * cross_layer_stride(b);
        hipError_t e = hipSuccess;
        if (wsp::ops::tile_product_fits(wdtype, d, 2 * d, d, encoder_rows))
        {
            // Every stream's rows in one launch: row r of the encoder block is
            // row r % cross_rows of stream r / cross_rows.
            wsp::ops::TileProduct p {};
            p.x = encoder_rows;
            p.rows = b->streams * cross_rows;
            p.inner = d;
            p.w0 = L.key_w;
            p.w1 = L.value_w;
            p.split = d;
            p.out = 2 * d;
            p.bias1 = L.value_b;
            p.y0 = keys;
            p.y1 = values;
            p.ldy = (int) cross_key_stride(b);
            p.rows_per_group = cross_rows;
            p.group_stride = cross_stream_stride(b);
            p.wdtype = wdtype;
            e = wsp::ops::tile_product(b->stream, p);
        }
        else
            for (int c = 0; c < b->streams && e == hipSuccess; ++c)
            {
                const float* x = encoder_rows + (size_t) c * cross_rows * d;
                // Dense rows into the scratch block, then strided into the
                // key-major cache.
                const size_t at = (size_t) c * cross_stream_stride(b);
                const size_t pitch = cross_key_stride(b) * sizeof(float), row = (size_t) d * sizeof(float);
                if (b->cross_scratch == nullptr)
                    e = allocate(b, &b->cross_scratch, (size_t) b->shape.cross_positions * d);
                if (e == hipSuccess)
                    e = wsp::ops::linear(b->stream, x, cross_rows, d, L.key_w, wdtype, nullptr, b->cross_scratch, d, 0);
                if (e == hipSuccess)
                    e = hipMemcpy2DAsync(keys + at, pitch, b->cross_scratch, row, row, cross_rows,
                                         hipMemcpyDeviceToDevice, b->stream);
                if (e == hipSuccess)
                    e = wsp::ops::linear(b->stream, x, cross_rows, d, L.value_w, wdtype, L.value_b, b->cross_scratch,
                                         d, 0);
                if (e == hipSuccess)
                    e = hipMemcpy2DAsync(values + at, pitch, b->cross_scratch, row, row, cross_rows,
                                         hipMemcpyDeviceToDevice, b->stream);
            }
        if (e != hipSuccess)
            return hip_fail(b, e, "cross key/value projection");
    }
    const hipError_t e = hipMemsetAsync(b->state, 0, sizeof(int), b->stream);
    if (e != hipSuccess)
        return hip_fail(b, e, "position reset");
    b->cross_rows = cross_rows;
    b->position = 0;
    return WSP_OK;
}

int wsp_batch_step(wsp_batch* b, const wsp_decoder_tensors* tensors, const uint32_t* tokens, int count,
                   float* hidden, float* logits, const float* mask, uint32_t* argmax_out)
{
    if (b == nullptr)
        return WSP_ERR_ARGUMENT;
    b->error[0] = 0;
    if (tensors == nullptr || tensors->layers == nullptr || tokens == nullptr || logits == nullptr)
        return fail(b, WSP_ERR_ARGUMENT, "wsp_batch_step: null tensors, tokens or logits");
    if (count <= 0 || count > b->max_step_tokens)
        return fail(b, WSP_ERR_CAPACITY, "wsp_batch_step: more tokens per stream than the batch was sized for");
    if (b->cross_rows <= 0)
        return fail(b, WSP_ERR_LOGIC, "wsp_batch_step: no sequence begun");
    if (b->position + count > b->shape.max_positions)
        return fail(b, WSP_ERR_SHAPE, "wsp_batch_step: the step runs past max_positions");
    if (tensors->wdtype != b->wdtype || tensors->logits_wdtype != b->wdtype)
        return fail(b, WSP_ERR_LOGIC, "wsp_batch_step: projections and logits must share the batch's 16-bit storage");
    (void) hipSetDevice(b->device);
    int status = WSP_OK;
    const wsp_decoder_tensors* packed = packed_weights(b, tensors, status);
    if (packed == nullptr)
        return status;
    const StepIo io {tokens, nullptr, count, hidden, logits, mask, argmax_out, false};
    status = b->compute == WSP_F16 ? run_step<wsp::kF16>(b, packed, io, b->stream)
                                   : run_step<wsp::kBF16>(b, packed, io, b->stream);
    if (status == WSP_OK)
        b->position += count;
    return status;
}

int wsp_batch_ring_step(wsp_batch* b, const wsp_decoder_tensors* tensors, uint32_t* ring, float* logits,
                        const float* mask)
{
    if (b == nullptr)
        return WSP_ERR_ARGUMENT;
    b->error[0] = 0;
    if (tensors == nullptr || tensors->layers == nullptr || ring == nullptr || logits == nullptr)
        return fail(b, WSP_ERR_ARGUMENT, "wsp_batch_ring_step: null tensors, ring or logits");
    if (b->cross_rows <= 0)
        return fail(b, WSP_ERR_LOGIC, "wsp_batch_ring_step: no sequence begun");
    if (b->position < 1 || b->position + 1 > b->shape.max_positions)
        return fail(b, WSP_ERR_SHAPE, "wsp_batch_ring_step: the ring step needs a position in [1, max_positions)");
    if (tensors->wdtype != b->wdtype || tensors->logits_wdtype != b->wdtype)
        return fail(b, WSP_ERR_LOGIC, "wsp_batch_ring_step: projections and logits must share the batch's 16-bit storage");
    (void) hipSetDevice(b->device);
    int packing = WSP_OK;
    const wsp_decoder_tensors* packed = packed_weights(b, tensors, packing);
    if (packed == nullptr)
        return packing;
    if (b->graph == nullptr || b->graph_ring != ring || b->graph_logits != logits || b->graph_mask != mask
        || b->graph_cross_rows != b->cross_rows || !same_table(b, table_bytes(packed, b->shape.layers)))
    {
        const int status = b->compute == WSP_F16 ? capture_ring_step<wsp::kF16>(b, packed, ring, logits, mask)
                                                 : capture_ring_step<wsp::kBF16>(b, packed, ring, logits, mask);
        if (status != WSP_OK)
            return status;
    }
    const hipError_t e = hipGraphLaunch(b->graph, b->stream);
    if (e != hipSuccess)
        return hip_fail(b, e, "graph launch");
    b->position += 1;
    return WSP_OK;
}

int wsp_batch_self_cache(const wsp_batch* b, int layer, const float** keys, const float** values)
{
    if (b == nullptr || keys == nullptr || values == nullptr || layer < 0 || layer >= b->shape.layers)
        return WSP_ERR_ARGUMENT;
    *keys = b->self_keys + (size_t) layer * self_layer_stride(b);
    *values = b->self_values + (size_t) layer * self_layer_stride(b);
    return WSP_OK;
}

int wsp_batch_cross_cache(const wsp_batch* b, int layer, const float** keys, const float** values)
{
    if (b == nullptr || keys == nullptr || values == nullptr || layer < 0 || layer >= b->shape.layers)
        return WSP_ERR_ARGUMENT;
    *keys = b->cross_keys + (size_t) layer * cross_layer_stride(b);
    *values = b->cross_values + (size_t) layer * cross_layer_stride(b);
    return WSP_OK;
}

} // extern "C"
