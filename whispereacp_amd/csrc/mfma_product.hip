// The tall product on gfx950 matrix cores: y = X·Wᵀ for many rows of fp32 X
// and a 16-bit W — the cross-attention key/value projection of the encoder
// rows (Decoder/Decoder.cpp:121-146, LinearProduct in the reference) and any
// linear of more than 16 rows.
//
// X is split on its way into LDS into exact 16-bit parts (fp16 hi + lo for
// fp16 weights, three bf16 parts for bf16 weights), so every matrix-core
// product is exact and the fp32 sums match an fp32 product with widened
// weights to fp32 rounding (the fp16 split needs |x| < 65504).
//
// A 256-thread block computes a 128 x 128 tile in 32-wide k-steps; each of its
// four waves owns 64 x 64 (4 x 4 MFMA tiles of 16 x 16). The next k-step's
// global loads are issued before the current step's products. LDS rows are
// padded to 80 bytes, which keeps each 16-lane fragment read on distinct
// banks.
#include "device_common.h"
#include "ops.h"

namespace wsp::ops
{
namespace
{
typedef uint16_t u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTile = 128;
constexpr int kStep = 32;
constexpr int kRow = kStep + 8; // halves per LDS row

template <int WT>
constexpr int parts_of()
{
    return WT == kF16 ? 2 : 3;
}

template <int WT>
__device__ __forceinline__ float4v mfma16(u32x4 a, u32x4 b, float4v c)
{
    if constexpr (WT == kF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The 16-bit parts of x, part p in bits[p].
template <int WT>
__device__ __forceinline__ void split(float x, uint32_t (&bits)[3])
{
    if constexpr (WT == kF16)
    {
        const _Float16 hi = (_Float16) x;
        const _Float16 lo = (_Float16) (x - (float) hi);
        bits[0] = __builtin_bit_cast(u16, hi);
        bits[1] = __builtin_bit_cast(u16, lo);
        bits[2] = 0;
    }
    else
    {
        float rest = x;
#pragma unroll
        for (int p = 0; p < 3; ++p)
        {
            const __bf16 b = (__bf16) rest;
            bits[p] = __builtin_bit_cast(u16, b);
            rest -= (float) b;
        }
    }
}

template <int WT>
__global__ void __launch_bounds__(kThreads) tile_product_kernel(TileProduct a)
{
    constexpr int P = parts_of<WT>();
    __shared__ __attribute__((aligned(16))) u16 sa[P][kTile][kRow];
    __shared__ __attribute__((aligned(16))) u16 sb[kTile][kRow];

    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int li = lane % 16, g = lane / 16;
    const int wm = wave / 2, wn = wave % 2;
    const int n_block = blockIdx.x * kTile, m_block = blockIdx.y * kTile;

    // Staging: thread (row sr, half sh) moves 16 consecutive k of one X row
    // and one W row per k-step. Rows past the end re-read the last row.
    const int sr = tid / 2, sh = (tid % 2) * 16;
    const float* ap = a.x + (size_t) min(m_block + sr, a.rows - 1) * a.inner + sh;
    const int nrow = n_block + sr;
    const u16* bp = (nrow < a.split ? static_cast<const u16*>(a.w0) + (size_t) nrow * a.inner
                                    : static_cast<const u16*>(a.w1) + (size_t) (nrow - a.split) * a.inner)
                    + sh;

    float4v ar[4];
    u32x4 br[2];
#define WSP_TILE_LOAD(k0)                                                            \
    do                                                                               \
    {                                                                                \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) ar[j] =                        \
            *reinterpret_cast<const float4v*>(ap + (k0) + 4 * j);                    \
        br[0] = *reinterpret_cast<const u32x4*>(bp + (k0));                          \
        br[1] = *reinterpret_cast<const u32x4*>(bp + (k0) + 8);                      \
    } while (0)

    float4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = float4v {0.f, 0.f, 0.f, 0.f};

    const int steps = a.inner / kStep;
    WSP_TILE_LOAD(0);
    for (int s = 0; s < steps; ++s)
    {
        __syncthreads(); // the previous step's fragments are read
#pragma unroll
        for (int h = 0; h < 2; ++h)
        {
            uint32_t packed[P][4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const float4v v = ar[2 * h + j / 2];
                uint32_t b0[3], b1[3];
                split<WT>(v[(j % 2) * 2], b0);
                split<WT>(v[(j % 2) * 2 + 1], b1);
#pragma unroll
                for (int p = 0; p < P; ++p)
                    packed[p][j] = b0[p] | (b1[p] << 16);
            }
#pragma unroll
            for (int p = 0; p < P; ++p)
                *reinterpret_cast<u32x4*>(&sa[p][sr][sh + 8 * h]) = u32x4 {packed[p][0], packed[p][1], packed[p][2], packed[p][3]};
        }
        *reinterpret_cast<u32x4*>(&sb[sr][sh]) = br[0];
        *reinterpret_cast<u32x4*>(&sb[sr][sh + 8]) = br[1];
        __syncthreads();
        if (s + 1 < steps)
            WSP_TILE_LOAD((s + 1) * kStep);

        u32x4 af[4][P], bf[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int p = 0; p < P; ++p)
                af[mt][p] = *reinterpret_cast<const u32x4*>(&sa[p][wm * 64 + mt * 16 + li][8 * g]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
            bf[nt] = *reinterpret_cast<const u32x4*>(&sb[wn * 64 + nt * 16 + li][8 * g]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                for (int p = 0; p < P; ++p)
                    acc[mt][nt] = mfma16<WT>(af[mt][p], bf[nt], acc[mt][nt]);
    }
#undef WSP_TILE_LOAD

    // acc[mt][nt][r] of lane (g, li) is C[4g + r][li] of that 16 x 16 tile.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
        {
            const int row = m_block + wm * 64 + mt * 16 + 4 * g + r;
            if (row >= a.rows)
                continue;
            const size_t base = (size_t) (row / a.rows_per_group) * a.group_stride
                                + (size_t) (row % a.rows_per_group) * a.ldy;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
            {
                const int n = n_block + wn * 64 + nt * 16 + li;
                const bool first = n < a.split;
                const int c = first ? n : n - a.split;
                const float* bias = first ? a.bias0 : a.bias1;
                float* y = first ? a.y0 : a.y1;
                float v = acc[mt][nt][r];
                if (bias != nullptr)
                    v += bias[c];
                if (a.flags & 1)
                    v = exact_gelu(v);
                if (a.flags & 2)
                    y[base + c] += v;
                else
                    y[base + c] = v;
            }
        }
}
} // namespace

bool tile_product_fits(int wdtype, int inner, int out, int split, const void* x)
{
    return (wdtype == kF16 || wdtype == kBF16) && inner % kStep == 0 && out % kTile == 0 && split % kTile == 0
           && split <= out && (reinterpret_cast<uintptr_t>(x) % 16) == 0;
}

hipError_t tile_product(hipStream_t stream, const TileProduct& a)
{
    const dim3 grid(a.out / kTile, (a.rows + kTile - 1) / kTile);
    if (a.wdtype == kF16)
        hipLaunchKernelGGL((tile_product_kernel<kF16>), grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((tile_product_kernel<kBF16>), grid, dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}
} // namespace wsp::ops
