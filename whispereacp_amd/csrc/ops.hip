// Per-op gfx950 kernels behind the C ABI: the split GEMV and tiled product
// (Kernels/Linear.h), LayerNorm (Kernels/LayerNorm.h), Embed
// (Kernels/Embed.h), split-key attention with its combine
// (Kernels/SingleQueryAttention.h, Kernels/Attention.h) and the two-stage
// argmax (Kernels/Argmax.h). Written for wave64 CDNA4; every reduction runs in
// a fixed order, so results are deterministic run to run.
#include "device_common.h"
#include "ops.h"

#include <algorithm>
#include <cmath>

namespace wsp::ops
{
namespace
{
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// ---------------------------------------------------------------------------
// Split GEMV: each wave owns OPW output columns for up to RMAX rows. Lane l
// walks the inner dimension in runs of 8 (one 16-byte weight load for F16 and
// BF16, two for F32) at k = 8l, 8l + 512, ...; the 64 lane partials are then
// summed by a fixed xor-butterfly. The epilogue is the reference's store
// (Kernels/Linear.h:213-227): bias, then GELU, then the residual.
// ---------------------------------------------------------------------------
template <int WT, int RMAX, int OPW>
__global__ void __launch_bounds__(kBlock) gemv_kernel(const float* __restrict__ x, int rows,
                                                      int inner, const void* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int out, int flags,
                                                      int vectorised)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    const int o0 = wave * OPW;

    if (o0 >= out)
        return;

    float acc[RMAX][OPW];
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
#pragma unroll
        for (int j = 0; j < OPW; ++j)
            acc[r][j] = 0.f;

    if (vectorised)
    {
        for (int k = lane * 8; k < inner; k += kWave * 8)
        {
            float wv[OPW][8];
#pragma unroll
            for (int j = 0; j < OPW; ++j)
            {
                const int o = min(o0 + j, out - 1);
                load8<WT>(w, (size_t) o * inner + k, wv[j]);
            }
#pragma unroll
            for (int r = 0; r < RMAX; ++r)
            {
                if (r >= rows)
                    break;
                const float4v* xp = reinterpret_cast<const float4v*>(x + (size_t) r * inner + k);
                const float4v a = xp[0], b = xp[1];
                const float xv[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
                for (int j = 0; j < OPW; ++j)
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        acc[r][j] += xv[i] * wv[j][i];
            }
        }
    }
    else
    {
        for (int k = lane; k < inner; k += kWave)
        {
            float wv[OPW];
#pragma unroll
            for (int j = 0; j < OPW; ++j)
                wv[j] = load1<WT>(w, (size_t) min(o0 + j, out - 1) * inner + k);
#pragma unroll
            for (int r = 0; r < RMAX; ++r)
            {
                if (r >= rows)
                    break;
                const float xv = x[(size_t) r * inner + k];
#pragma unroll
                for (int j = 0; j < OPW; ++j)
                    acc[r][j] += xv * wv[j];
            }
        }
    }

#pragma unroll
    for (int r = 0; r < RMAX; ++r)
#pragma unroll
        for (int j = 0; j < OPW; ++j)
            acc[r][j] = wave_sum(acc[r][j]);

#pragma unroll
    for (int r = 0; r < RMAX; ++r)
#pragma unroll
        for (int j = 0; j < OPW; ++j)
        {
            const int o = o0 + j;
            if (r < rows && o < out && lane == ((r * OPW + j) & (kWave - 1)))
            {
                float v = acc[r][j] + (bias != nullptr ? bias[o] : 0.f);
                if (flags & 1)
                    v = exact_gelu(v);
                float* dst = y + (size_t) r * out + o;
                if (flags & 2)
                    v += *dst;
                *dst = v;
            }
        }
}

// ---------------------------------------------------------------------------
// Tiled product for many rows: 64x64 output tiles, 16-deep K slices staged in
// LDS (weights widened to float on the way in), 4x4 outputs per thread, k
// ascending within each thread's sum. Same epilogue as the GEMV. With VEC
// (inner a multiple of 4, rows 16-byte aligned) each thread moves one row's
// four consecutive k per operand per slice as one vector load, the next
// slice's loads are in flight while the current one is multiplied, and the
// fragments come out of LDS as float4 reads.
// ---------------------------------------------------------------------------
constexpr int kTile = 64;
constexpr int kTileK = 16;

// Four consecutive weights widened to float (VEC loads: 16 bytes for F32,
// 8 for F16 and BF16).
template <int WT>
__device__ __forceinline__ float4v load4(const void* w, size_t index)
{
    if constexpr (WT == kF32)
        return *reinterpret_cast<const float4v*>(static_cast<const float*>(w) + index);
    else
    {
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + index);
        const uint16_t h[4] = {(uint16_t) u.x, (uint16_t) (u.x >> 16), (uint16_t) u.y, (uint16_t) (u.y >> 16)};
        float4v v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            if constexpr (WT == kF16)
                v[i] = (float) __builtin_bit_cast(_Float16, h[i]);
            else
                v[i] = bf16_to_float(h[i]);
        }
        return v;
    }
}

// TM rows by 64 columns a block: RT = TM / 16 rows by 4 columns a thread
// (TM 32, VEC only, when 64-row blocks leave CUs idle).
template <int WT, bool VEC, int TM>
__global__ void __launch_bounds__(kBlock) gemm_kernel(const float* __restrict__ x, int rows,
                                                      int inner, const void* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int out, int flags)
{
    constexpr int RT = TM / 16;
    static_assert(TM == kTile || (VEC && TM == 32), "32-row blocks take vector loads");
    __shared__ __attribute__((aligned(16))) float xs[kTileK][kTile + 4];
    __shared__ __attribute__((aligned(16))) float ws[kTileK][kTile + 4];

    const int row0 = blockIdx.y * TM;
    const int col0 = blockIdx.x * kTile;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;

    float acc[RT][4] = {};

    if constexpr (VEC)
    {
        // Thread t stages row (or weight row) t / 4, k = 4 (t % 4) .. + 3 of
        // the slice.
        const int sr = threadIdx.x / 4, sq = (threadIdx.x % 4) * 4;
        const int gr = row0 + sr, gc = col0 + sr;
        float4v xa = {0.f, 0.f, 0.f, 0.f}, wa = {0.f, 0.f, 0.f, 0.f};
        auto fetch = [&](int k0) {
            const int gk = k0 + sq;
            xa = float4v {0.f, 0.f, 0.f, 0.f};
            wa = float4v {0.f, 0.f, 0.f, 0.f};
            if (sr < TM && gr < rows && gk < inner)
                xa = *reinterpret_cast<const float4v*>(x + (size_t) gr * inner + gk);
            if (gc < out && gk < inner)
                wa = load4<WT>(w, (size_t) gc * inner + gk);
        };
        fetch(0);
        for (int k0 = 0; k0 < inner; k0 += kTileK)
        {
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                if (sr < TM)
                    xs[sq + i][sr] = xa[i];
                ws[sq + i][sr] = wa[i];
            }
            __syncthreads();
            if (k0 + kTileK < inner)
                fetch(k0 + kTileK);
#pragma unroll
            for (int kk = 0; kk < kTileK; ++kk)
            {
                float a[RT];
                if constexpr (RT == 4)
                {
                    const float4v v = *reinterpret_cast<const float4v*>(&xs[kk][ty * 4]);
                    a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
                }
                else
                {
                    const float2 v = *reinterpret_cast<const float2*>(&xs[kk][ty * 2]);
                    a[0] = v.x; a[1] = v.y;
                }
                const float4v b = *reinterpret_cast<const float4v*>(&ws[kk][tx * 4]);
#pragma unroll
                for (int i = 0; i < RT; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] += a[i] * b[j];
            }
            __syncthreads();
        }
    }
    else if constexpr (TM == kTile)
        for (int k0 = 0; k0 < inner; k0 += kTileK)
        {
            // 64 x 16 of each operand: 1024 elements, 4 per thread.
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int e = threadIdx.x + i * kBlock;
                const int r = e / kTileK, kk = e % kTileK;
                const int gk = k0 + kk;
                const int gr = row0 + r, gc = col0 + r;
                xs[kk][r] = (gr < rows && gk < inner) ? x[(size_t) gr * inner + gk] : 0.f;
                ws[kk][r] = (gc < out && gk < inner) ? load1<WT>(w, (size_t) gc * inner + gk) : 0.f;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < kTileK; ++kk)
            {
                float a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    a[i] = xs[kk][ty * 4 + i];
                    b[i] = ws[kk][tx * 4 + i];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] += a[i] * b[j];
            }
            __syncthreads();
        }

#pragma unroll
    for (int i = 0; i < RT; ++i)
    {
        const int r = row0 + ty * RT + i;
        if (r >= rows)
            continue;
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int c = col0 + tx * 4 + j;
            if (c >= out)
                continue;
            float v = acc[i][j] + (bias != nullptr ? bias[c] : 0.f);
            if (flags & 1)
                v = exact_gelu(v);
            float* dst = y + (size_t) r * out + c;
            if (flags & 2)
                v += *dst;
            *dst = v;
        }
    }
}

// ---------------------------------------------------------------------------
// LayerNorm: one block per row; mean, then the centred variance, then
// (x - mean) * rsqrt(var + eps) * gamma + beta (Kernels/LayerNorm.h:44-89).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) layernorm_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta,
                                                           float* __restrict__ y, int width,
                                                           float eps)
{
    __shared__ float scratch[kWavesPerBlock];
    const float* row = x + (size_t) blockIdx.x * width;
    float* dst = y + (size_t) blockIdx.x * width;

    float total = 0.f;
    for (int c = threadIdx.x; c < width; c += kBlock)
        total += row[c];
    const float mean = block_sum(total, scratch) / (float) width;

    float squares = 0.f;
    for (int c = threadIdx.x; c < width; c += kBlock)
    {
        const float centred = row[c] - mean;
        squares += centred * centred;
    }
    const float scale = rsqrtf(block_sum(squares, scratch) / (float) width + eps);

    for (int c = threadIdx.x; c < width; c += kBlock)
        dst[c] = (row[c] - mean) * scale * gamma[c] + beta[c];
}

// ---------------------------------------------------------------------------
// Embed: out[t, c] = tokens table row + position table row (Kernels/Embed.h).
// ---------------------------------------------------------------------------
// A token id outside the vocabulary (it arrives from device memory, so the host
// cannot check it) poisons its row with NaN rather than reading past the table.
__global__ void embed_kernel(const uint32_t* __restrict__ tokens,
                             const float* __restrict__ token_table,
                             const float* __restrict__ position_table, int first_position,
                             float* __restrict__ y, int width, int vocabulary)
{
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= width)
        return;
    const uint32_t token = tokens[t];
    y[(size_t) t * width + c] = token < (uint32_t) vocabulary
                                    ? token_table[(size_t) token * width + c]
                                          + position_table[(size_t) (first_position + t) * width + c]
                                    : __builtin_nanf("");
}

// ---------------------------------------------------------------------------
// Split-key attention. Block (head h, query i, chunk c) scores its chunk of
// the keys query i can see (the last q_count of k_count positions when
// causal, Kernels/Attention.h:34-47), takes the chunk maximum, exponentiates
// and sums, and walks the value rows. One chunk writes the normalised row;
// several write (max, sum, unnormalised row) for the combine, which rescales
// each chunk by exp(max_c - max) exactly as Kernels/SingleQueryAttention.h
// :27-37 describes.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) attention_chunk_kernel(
    const float* __restrict__ q, int q_count, const float* __restrict__ keys,
    const float* __restrict__ values, int k_count, int width, int head_width, int causal,
    float scale, int chunks, int chunk_length, float* __restrict__ out,
    float* __restrict__ partials)
{
    __shared__ float scores[kAttentionChunkKeys];
    __shared__ float scratch[kWavesPerBlock];
    __shared__ float rows_sum[4][kMaxHeadWidth];

    const int chunk = blockIdx.x % chunks;
    const int query = (blockIdx.x / chunks) % q_count;
    const int head = blockIdx.x / (chunks * q_count);
    const int column = head * head_width;

    const int visible = causal ? k_count - q_count + query + 1 : k_count;
    const int first = chunk * chunk_length;
    const int last = min(first + chunk_length, visible);
    const int count = max(0, last - first);

    // Scores: 16 lanes per key, each lane a run of four channels.
    const int sub = threadIdx.x % 16, group = threadIdx.x / 16;
    const float* qrow = q + (size_t) query * width + column;
    float4v qv = {0.f, 0.f, 0.f, 0.f};
    if (4 * sub < head_width)
        qv = *reinterpret_cast<const float4v*>(qrow + 4 * sub);

    float local_max = -INFINITY;
    for (int j = group; j < count; j += 16)
    {
        float part = 0.f;
        if (4 * sub < head_width)
        {
            const float4v kv =
                *reinterpret_cast<const float4v*>(keys + (size_t) (first + j) * width + column + 4 * sub);
            part = qv[0] * kv[0] + qv[1] * kv[1] + qv[2] * kv[2] + qv[3] * kv[3];
        }
#pragma unroll
        for (int offset = 8; offset > 0; offset >>= 1)
            part += __shfl_xor(part, offset, 16);
        const float s = scale * part;
        if (sub == 0)
            scores[j] = s;
        local_max = fmaxf(local_max, s);
    }
    const float chunk_max = block_max(local_max, scratch);

    float local_sum = 0.f;
    for (int j = threadIdx.x; j < count; j += kBlock)
    {
        const float p = expf(scores[j] - chunk_max);
        scores[j] = p;
        local_sum += p;
    }
    const float chunk_sum = block_sum(local_sum, scratch);

    // Values: channel c = t % 64, keys j = t / 64 (mod 4).
    const int c = threadIdx.x % kMaxHeadWidth, kg = threadIdx.x / kMaxHeadWidth;
    float acc = 0.f;
    if (c < head_width)
        for (int j = kg; j < count; j += 4)
            acc += scores[j] * values[(size_t) (first + j) * width + column + c];
    rows_sum[kg][c] = acc;
    __syncthreads();

    if (threadIdx.x < head_width)
    {
        const float row = (rows_sum[0][c] + rows_sum[1][c]) + (rows_sum[2][c] + rows_sum[3][c]);
        if (chunks == 1)
            out[(size_t) query * width + column + c] = row / chunk_sum;
        else
        {
            float* part = partials + ((size_t) (head * q_count + query) * chunks + chunk) * (head_width + 2);
            part[2 + c] = row;
            if (c == 0)
            {
                part[0] = count > 0 ? chunk_max : -INFINITY;
                part[1] = chunk_sum;
            }
        }
    }
}

__global__ void attention_combine_kernel(const float* __restrict__ partials, int q_count,
                                         int width, int head_width, int chunks,
                                         float* __restrict__ out)
{
    const int query = blockIdx.x % q_count;
    const int head = blockIdx.x / q_count;
    const int c = threadIdx.x;
    if (c >= head_width)
        return;
    const float* base = partials + (size_t) (head * q_count + query) * chunks * (head_width + 2);

    float largest = -INFINITY;
    for (int k = 0; k < chunks; ++k)
        largest = fmaxf(largest, base[(size_t) k * (head_width + 2)]);

    float numerator = 0.f, denominator = 0.f;
    for (int k = 0; k < chunks; ++k)
    {
        const float* part = base + (size_t) k * (head_width + 2);
        if (part[1] == 0.f)
            continue;
        const float factor = expf(part[0] - largest);
        numerator += factor * part[2 + c];
        denominator += factor * part[1];
    }
    out[(size_t) query * width + head * head_width + c] = numerator / denominator;
}

// ---------------------------------------------------------------------------
// Multi-query attention of a prompt step (2..16 queries): the scores, the
// softmax and the weighted value sum of Kernels/Attention.h:75-209, with its
// causal rule (query i of q stands at absolute position k - q + i and sees the
// keys up to it, Kernels/Attention.h:34-47), in one launch. Block (head,
// split) takes every query of its head over keys [split·span, +span) in tiles
// of 64 keys staged in LDS, and keeps per query an online (max, sum, row) with
// exact exp(m_old - m_new) rescaling: masked keys get weight exactly 0. Wave w
// owns queries 4w .. 4w + 3 in every phase (lane = key for the scores, lane =
// channel for the values), so a query's statistics never leave its wave. With
// several splits each block writes its (max, sum, row) per query, and the last
// block of the head to finish (a per-head counter it resets to zero) combines
// them in split order, so the result does not depend on which block is last.
// ---------------------------------------------------------------------------
constexpr int kPromptTile = 64;
constexpr int kPromptKeyStride = kMaxHeadWidth + 4; // padded rows: lanes reading key rows spread over the banks
constexpr int kPromptPartial = kMaxHeadWidth + 2;
static_assert(kMaxPromptQueries == 4 * kWavesPerBlock, "four queries per wave");

__global__ void __launch_bounds__(kBlock) prompt_attention_kernel(
    const float* __restrict__ q, int q_count, const float* __restrict__ keys, const float* __restrict__ values,
    int k_count, int width, int head_width, int causal, float scale, int splits, int span, float* __restrict__ out,
    float* __restrict__ partials, unsigned int* __restrict__ counters)
{
    __shared__ __attribute__((aligned(16))) float qs[kMaxPromptQueries][kMaxHeadWidth];
    __shared__ __attribute__((aligned(16))) float ks[kPromptTile][kPromptKeyStride];
    __shared__ float vs[kPromptTile][kMaxHeadWidth];
    __shared__ float ps[kMaxPromptQueries][kPromptTile];
    __shared__ int last_block;

    const int split = blockIdx.x % splits, head = blockIdx.x / splits;
    const int column = head * head_width;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int first = split * span, end = min(first + span, k_count);

    for (int i = threadIdx.x; i < kMaxPromptQueries * kMaxHeadWidth; i += kBlock)
    {
        const int r = i / kMaxHeadWidth, c = i % kMaxHeadWidth;
        qs[r][c] = r < q_count && c < head_width ? q[(size_t) r * width + column + c] : 0.f;
    }

    float m[4], l[4], acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        m[k] = -INFINITY;
        l[k] = 0.f;
        acc[k] = 0.f;
    }
    for (int t0 = first; t0 < end; t0 += kPromptTile)
    {
        const int n = min(kPromptTile, end - t0);
        __syncthreads(); // the previous tile's readers are done (and the queries are in)
        for (int i = threadIdx.x; i < kPromptTile * kMaxHeadWidth / 4; i += kBlock)
        {
            const int j = i / (kMaxHeadWidth / 4), c4 = 4 * (i % (kMaxHeadWidth / 4));
            float4v kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
            if (j < n && c4 < head_width)
            {
                const size_t at = (size_t) (t0 + j) * width + column + c4;
                kv = *reinterpret_cast<const float4v*>(keys + at);
                vv = *reinterpret_cast<const float4v*>(values + at);
            }
            *reinterpret_cast<float4v*>(&ks[j][c4]) = kv;
            *reinterpret_cast<float4v*>(&vs[j][c4]) = vv;
        }
        __syncthreads();

        // Scores of key t0 + lane against this wave's four queries.
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < head_width; c += 4)
        {
            const float4v kv = *reinterpret_cast<const float4v*>(&ks[lane][c]);
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const float4v qv = *reinterpret_cast<const float4v*>(&qs[4 * wave + k][c]);
                s[k] += (qv[0] * kv[0] + qv[1] * kv[1]) + (qv[2] * kv[2] + qv[3] * kv[3]);
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const int query = 4 * wave + k;
            const int key = t0 + lane;
            const bool seen = query < q_count && lane < n && (!causal || key <= k_count - q_count + query);
            const float score = seen ? scale * s[k] : -INFINITY;
            const float m_new = fmaxf(m[k], wave_max(score));
            const float alpha = m_new == -INFINITY ? 1.f : expf(m[k] - m_new);
            const float p = seen ? expf(score - m_new) : 0.f;
            l[k] = l[k] * alpha + wave_sum(p);
            acc[k] *= alpha;
            m[k] = m_new;
            ps[query][lane] = p;
        }
        __syncthreads();

        // Values: lane = channel.
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            float sum = 0.f;
            for (int j = 0; j < n; ++j)
                sum += ps[4 * wave + k][j] * vs[j][lane];
            acc[k] += sum;
        }
    }

    if (splits == 1)
    {
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const int query = 4 * wave + k;
            if (query < q_count && lane < head_width)
                out[(size_t) query * width + column + lane] = acc[k] / l[k];
        }
        return;
    }

    float* const head_parts = partials + (size_t) head * splits * kMaxPromptQueries * kPromptPartial;
#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        const int query = 4 * wave + k;
        float* part = head_parts + ((size_t) split * kMaxPromptQueries + query) * kPromptPartial;
        if (query < q_count)
        {
            if (lane < head_width)
                part[2 + lane] = acc[k];
            if (lane == 0)
            {
                part[0] = m[k];
                part[1] = l[k];
            }
        }
    }
    __threadfence(); // the partial is visible device-wide before the count says so
    __syncthreads();
    if (threadIdx.x == 0)
        last_block = atomicAdd(&counters[head], 1u) == (unsigned) (splits - 1);
    __syncthreads();
    if (!last_block)
        return;
    __threadfence(); // every other block's partial is visible from here on

#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        const int query = 4 * wave + k;
        if (query >= q_count)
            continue;
        float largest = -INFINITY;
        for (int sp = 0; sp < splits; ++sp)
        {
            const float* part = head_parts + ((size_t) sp * kMaxPromptQueries + query) * kPromptPartial;
            if (part[1] != 0.f)
                largest = fmaxf(largest, part[0]);
        }
        float numerator = 0.f, denominator = 0.f;
        for (int sp = 0; sp < splits; ++sp)
        {
            const float* part = head_parts + ((size_t) sp * kMaxPromptQueries + query) * kPromptPartial;
            if (part[1] == 0.f)
                continue;
            const float factor = expf(part[0] - largest);
            numerator += factor * (lane < head_width ? part[2 + lane] : 0.f);
            denominator += factor * part[1];
        }
        if (lane < head_width)
            out[(size_t) query * width + column + lane] = numerator / denominator;
    }
    if (threadIdx.x == 0)
        counters[head] = 0u; // zero again for the next launch
}

// ---------------------------------------------------------------------------
// Argmax (Kernels/Argmax.h:46-262): candidates are (value, index) pairs; a
// larger value wins and equal values keep the lower index, so the fold ends on
// the index a left-to-right scan stops at. Suppressed entries never compete;
// a row with none allowed yields 0.
// ---------------------------------------------------------------------------
constexpr uint32_t kUnchosen = 0xFFFFFFFFu;
constexpr int kArgmaxPerThread = 8;

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi)
{
    if (i == kUnchosen)
        return false;
    if (bi == kUnchosen)
        return true;
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void block_argmax(float& v, uint32_t& i)
{
    __shared__ float sv[kWavesPerBlock];
    __shared__ uint32_t si[kWavesPerBlock];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
    {
        const float ov = __shfl_xor(v, offset, kWave);
        const uint32_t oi = __shfl_xor(i, offset, kWave);
        if (better(ov, oi, v, i))
        {
            v = ov;
            i = oi;
        }
    }
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    if (lane == 0)
    {
        sv[wave] = v;
        si[wave] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int k = 1; k < (int) (blockDim.x / kWave); ++k)
        if (better(sv[k], si[k], v, i))
        {
            v = sv[k];
            i = si[k];
        }
}

__global__ void __launch_bounds__(kBlock) argmax_partial_kernel(const float* __restrict__ logits,
                                                                size_t row_stride, int row_length,
                                                                const float* __restrict__ mask,
                                                                int groups,
                                                                float* __restrict__ pv,
                                                                uint32_t* __restrict__ pi)
{
    const int row = blockIdx.x / groups, part = blockIdx.x % groups;
    const float* values = logits + (size_t) row * row_stride;
    float bv = 0.f;
    uint32_t bi = kUnchosen;
    for (int j = part * kBlock + threadIdx.x; j < row_length; j += groups * kBlock)
    {
        if (mask != nullptr && mask[j] != 0.f)
            continue;
        const float v = values[j];
        if (bi == kUnchosen || v > bv)
        {
            bv = v;
            bi = (uint32_t) j;
        }
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0)
    {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ void __launch_bounds__(kWave) argmax_final_kernel(const float* __restrict__ pv,
                                                             const uint32_t* __restrict__ pi,
                                                             int groups, uint32_t* __restrict__ out)
{
    const int row = blockIdx.x;
    float bv = 0.f;
    uint32_t bi = kUnchosen;
    for (int k = threadIdx.x; k < groups; k += kWave)
        if (better(pv[row * groups + k], pi[row * groups + k], bv, bi))
        {
            bv = pv[row * groups + k];
            bi = pi[row * groups + k];
        }
    block_argmax(bv, bi);
    if (threadIdx.x == 0)
        out[row] = bi == kUnchosen ? 0u : bi;
}

template <int WT>
hipError_t launch_gemv(hipStream_t stream, const float* x, int rows, int inner, const void* w,
                       const float* bias, float* y, int out, int flags)
{
    const bool vectorised = inner % 8 == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0
                            && (reinterpret_cast<uintptr_t>(w) % 16) == 0;
    // Enough waves to cover the chip at one output per wave; several outputs
    // per wave only once there are plenty of waves.
    const int opw = out >= 8192 ? 4 : 1;
    for (int r0 = 0; r0 < rows; r0 += 4)
    {
        const int rr = std::min(4, rows - r0);
        const float* xr = x + (size_t) r0 * inner;
        float* yr = y + (size_t) r0 * out;
        const int waves = (out + opw - 1) / opw;
        const dim3 grid((waves + kWavesPerBlock - 1) / kWavesPerBlock);
        if (rr == 1 && opw == 1)
            hipLaunchKernelGGL((gemv_kernel<WT, 1, 1>), grid, dim3(kBlock), 0, stream, xr, rr, inner, w, bias, yr, out, flags, (int) vectorised);
        else if (rr == 1)
            hipLaunchKernelGGL((gemv_kernel<WT, 1, 4>), grid, dim3(kBlock), 0, stream, xr, rr, inner, w, bias, yr, out, flags, (int) vectorised);
        else if (opw == 1)
            hipLaunchKernelGGL((gemv_kernel<WT, 4, 1>), grid, dim3(kBlock), 0, stream, xr, rr, inner, w, bias, yr, out, flags, (int) vectorised);
        else
            hipLaunchKernelGGL((gemv_kernel<WT, 4, 4>), grid, dim3(kBlock), 0, stream, xr, rr, inner, w, bias, yr, out, flags, (int) vectorised);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

template <int WT>
hipError_t launch_gemm(hipStream_t stream, const float* x, int rows, int inner, const void* w,
                       const float* bias, float* y, int out, int flags)
{
    const dim3 grid((out + kTile - 1) / kTile, (rows + kTile - 1) / kTile);
    const size_t w_align = WT == kF32 ? 16 : 8;
    const bool vec = inner % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0
                     && reinterpret_cast<uintptr_t>(w) % w_align == 0;
    static const int units = [] {
        int device = 0, count = 0;
        if (hipGetDevice(&device) == hipSuccess
            && hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && count > 0)
            return count;
        return 256;
    }();
    if (vec && (long long) grid.x * grid.y < units) // 32-row blocks: twice the blocks
        hipLaunchKernelGGL((gemm_kernel<WT, true, 32>), dim3(grid.x, (rows + 31) / 32), dim3(kBlock), 0, stream, x,
                           rows, inner, w, bias, y, out, flags);
    else if (vec)
        hipLaunchKernelGGL((gemm_kernel<WT, true, kTile>), grid, dim3(kBlock), 0, stream, x, rows, inner, w, bias, y,
                           out, flags);
    else
        hipLaunchKernelGGL((gemm_kernel<WT, false, kTile>), grid, dim3(kBlock), 0, stream, x, rows, inner, w, bias, y,
                           out, flags);
    return hipGetLastError();
}
} // namespace

hipError_t linear(hipStream_t stream, const float* x, int rows, int inner, const void* weight,
                  int wdtype, const float* bias, float* y, int out, int flags)
{
    if (rows <= kSplitRowLimit)
    {
        switch (wdtype)
        {
            case kF32: return launch_gemv<kF32>(stream, x, rows, inner, weight, bias, y, out, flags);
            case kF16: return launch_gemv<kF16>(stream, x, rows, inner, weight, bias, y, out, flags);
            default: return launch_gemv<kBF16>(stream, x, rows, inner, weight, bias, y, out, flags);
        }
    }
    if (tile_product_fits(wdtype, inner, out, out, x))
    {
        TileProduct p {};
        p.x = x;
        p.rows = rows;
        p.inner = inner;
        p.w0 = p.w1 = weight;
        p.split = p.out = out;
        p.bias0 = p.bias1 = bias;
        p.y0 = p.y1 = y;
        p.ldy = out;
        p.rows_per_group = rows;
        p.group_stride = 0;
        p.flags = flags;
        p.wdtype = wdtype;
        return tile_product(stream, p);
    }
    switch (wdtype)
    {
        case kF32: return launch_gemm<kF32>(stream, x, rows, inner, weight, bias, y, out, flags);
        case kF16: return launch_gemm<kF16>(stream, x, rows, inner, weight, bias, y, out, flags);
        default: return launch_gemm<kBF16>(stream, x, rows, inner, weight, bias, y, out, flags);
    }
}

hipError_t layernorm(hipStream_t stream, const float* x, const float* gamma, const float* beta,
                     float* y, int rows, int width, float eps)
{
    hipLaunchKernelGGL(layernorm_kernel, dim3(rows), dim3(kBlock), 0, stream, x, gamma, beta, y, width, eps);
    return hipGetLastError();
}

hipError_t embed(hipStream_t stream, const uint32_t* tokens, int count, const float* token_table,
                 const float* position_table, int first_position, float* y, int width,
                 int vocabulary)
{
    const dim3 grid((width + kBlock - 1) / kBlock, count);
    hipLaunchKernelGGL(embed_kernel, grid, dim3(kBlock), 0, stream, tokens, token_table, position_table, first_position, y, width, vocabulary);
    return hipGetLastError();
}

int attention_chunks(int heads, int q_count, int k_count)
{
    // Enough blocks to cover the chip (about 256), at least 32 keys a chunk,
    // and no chunk longer than the shared score array.
    const int units = heads * q_count;
    int chunks = std::max(1, std::min((k_count + 31) / 32, (256 + units - 1) / units));
    while ((k_count + chunks - 1) / chunks > kAttentionChunkKeys)
        ++chunks;
    return chunks;
}

// Keys per split of a prompt step's attention: a whole number of 64-key tiles,
// as few as give about one round of blocks over the chip (256).
int prompt_attention_span(int heads, int k_count)
{
    const int tiles = std::max(1, (k_count + kPromptTile - 1) / kPromptTile);
    const int wanted = std::max(1, std::min(tiles, (256 + heads - 1) / heads));
    return (tiles + wanted - 1) / wanted * kPromptTile;
}

int prompt_attention_splits(int heads, int k_count)
{
    const int span = prompt_attention_span(heads, k_count);
    return std::max(1, (k_count + span - 1) / span);
}

bool takes_prompt_attention(int q_count, int heads)
{
    return q_count >= 2 && q_count <= kMaxPromptQueries && heads <= kAttentionCounters;
}

size_t attention_workspace_floats(int heads, int q_count, int k_count, int head_width)
{
    if (takes_prompt_attention(q_count, heads))
    {
        const int splits = prompt_attention_splits(heads, k_count);
        return kAttentionCounters
               + (splits > 1 ? (size_t) heads * splits * kMaxPromptQueries * kPromptPartial : 0);
    }
    const int chunks = attention_chunks(heads, q_count, k_count);
    return kAttentionCounters + (chunks > 1 ? (size_t) heads * q_count * chunks * (head_width + 2) : 0);
}

hipError_t attention(hipStream_t stream, const float* q, int q_count, const float* keys,
                     const float* values, int k_count, int width, int heads, int causal,
                     float scale, float* out, float* workspace)
{
    const int head_width = width / heads;
    unsigned int* const counters = reinterpret_cast<unsigned int*>(workspace);
    float* const partials = workspace + kAttentionCounters;
    if (takes_prompt_attention(q_count, heads))
    {
        const int splits = prompt_attention_splits(heads, k_count);
        hipLaunchKernelGGL(prompt_attention_kernel, dim3(heads * splits), dim3(kBlock), 0, stream, q, q_count, keys,
                           values, k_count, width, head_width, causal, scale, splits,
                           prompt_attention_span(heads, k_count), out, partials, counters);
        return hipGetLastError();
    }
    workspace = partials;
    const int chunks = attention_chunks(heads, q_count, k_count);
    const int chunk_length = (k_count + chunks - 1) / chunks;
    hipLaunchKernelGGL(attention_chunk_kernel, dim3(heads * q_count * chunks), dim3(kBlock), 0, stream,
                       q, q_count, keys, values, k_count, width, head_width, causal, scale, chunks,
                       chunk_length, out, workspace);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || chunks == 1)
        return e;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(heads * q_count), dim3(kMaxHeadWidth), 0, stream,
                       workspace, q_count, width, head_width, chunks, out);
    return hipGetLastError();
}

int argmax_groups(int row_length)
{
    const int per_group = kBlock * kArgmaxPerThread;
    return std::max(1, (row_length + per_group - 1) / per_group);
}

hipError_t argmax(hipStream_t stream, const float* logits, int rows, int row_length,
                  const float* mask, uint32_t* out, float* partial_values,
                  uint32_t* partial_indices)
{
    return argmax_rows(stream, logits, rows, (size_t) row_length, row_length, mask, out, partial_values,
                       partial_indices);
}

hipError_t argmax_rows(hipStream_t stream, const float* logits, int rows, size_t row_stride,
                       int row_length, const float* mask, uint32_t* out, float* partial_values,
                       uint32_t* partial_indices)
{
    const int groups = argmax_groups(row_length);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(rows * groups), dim3(kBlock), 0, stream, logits,
                       row_stride, row_length, mask, groups, partial_values, partial_indices);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(kWave), 0, stream, partial_values,
                       partial_indices, groups, out);
    return hipGetLastError();
}
} // namespace wsp::ops
