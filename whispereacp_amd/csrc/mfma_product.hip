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
// A 256-thread block computes a 128 x 128 tile (or 64 x 128 when 128-row tiles
// would give fewer than four blocks per CU) in 32-wide k-steps; each of its four waves owns a
// quarter (4 x 4 or 2 x 4 MFMA tiles of 16 x 16). The next k-step's global
// loads are issued before the current step's products. LDS rows are padded to
// 96 bytes: against 80-byte rows that halves the bank-conflict cycles
// (SQ_LDS_BANK_CONFLICT) of the large-v3 fc1 product. Up to
// three weight matrices share one launch side by side (the encoder's q, k and
// v; the cross keys and values).
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
constexpr int kRow = kStep + 16; // halves per LDS row (96 bytes)

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

// TM rows by 128 columns per block: four waves as 2 x 2, each TM/2 x 64.
template <int WT, int TM>
__global__ void __launch_bounds__(kThreads) tile_product_kernel(TileProduct a)
{
    constexpr int P = parts_of<WT>();
    constexpr int MW = TM / 32;              // 16-row tiles per wave
    constexpr int XPER = TM * kStep / kThreads; // X floats one thread stages per k-step (16 or 8)
    constexpr int XTPR = kStep / XPER;       // threads per X row
    __shared__ __attribute__((aligned(16))) u16 sa[P][TM][kRow];
    __shared__ __attribute__((aligned(16))) u16 sb[kTile][kRow];

    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int li = lane % 16, g = lane / 16;
    const int wm = wave / 2, wn = wave % 2;
    const int n_block = blockIdx.x * kTile, m_block = blockIdx.y * TM;

    // Staging: thread (row sr, offset sh) moves XPER consecutive k of one X
    // row; thread (row br, half bh) moves 16 k of one W row. Rows past the end
    // re-read the last row.
    const int sr = tid / XTPR, sh = (tid % XTPR) * XPER;
    const float* ap = a.x + (size_t) min(m_block + sr, a.rows - 1) * a.inner + sh;
    const int br = tid / 2, bh = (tid % 2) * 16;
    const int nrow = n_block + br;
    const void* wbase = nrow < a.split ? a.w0 : nrow < a.split2 ? a.w1 : a.w2;
    const int wrow = nrow < a.split ? nrow : nrow < a.split2 ? nrow - a.split : nrow - a.split2;
    const u16* bp = static_cast<const u16*>(wbase) + (size_t) wrow * a.inner + bh;

    float4v ar[XPER / 4];
    u32x4 br2[2];
#define WSP_TILE_LOAD(k0)                                                            \
    do                                                                               \
    {                                                                                \
        _Pragma("unroll") for (int j = 0; j < XPER / 4; ++j) ar[j] =                 \
            *reinterpret_cast<const float4v*>(ap + (k0) + 4 * j);                    \
        br2[0] = *reinterpret_cast<const u32x4*>(bp + (k0));                         \
        br2[1] = *reinterpret_cast<const u32x4*>(bp + (k0) + 8);                     \
    } while (0)

    float4v acc[MW][4];
#pragma unroll
    for (int i = 0; i < MW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = float4v {0.f, 0.f, 0.f, 0.f};

    const int steps = a.inner / kStep;
    WSP_TILE_LOAD(0);
    for (int s = 0; s < steps; ++s)
    {
        __syncthreads(); // the previous step's fragments are read
        if constexpr (XPER == 4) // 32-row tiles: one float4 of a row per thread
        {
            uint32_t packed[P][2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
            {
                uint32_t b0[3], b1[3];
                split<WT>(ar[0][2 * j], b0);
                split<WT>(ar[0][2 * j + 1], b1);
#pragma unroll
                for (int p = 0; p < P; ++p)
                    packed[p][j] = b0[p] | (b1[p] << 16);
            }
#pragma unroll
            for (int p = 0; p < P; ++p)
                *reinterpret_cast<uint2*>(&sa[p][sr][sh]) = uint2 {packed[p][0], packed[p][1]};
        }
#pragma unroll
        for (int h = 0; h < XPER / 8; ++h)
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
        *reinterpret_cast<u32x4*>(&sb[br][bh]) = br2[0];
        *reinterpret_cast<u32x4*>(&sb[br][bh + 8]) = br2[1];
        __syncthreads();
        if (s + 1 < steps)
            WSP_TILE_LOAD((s + 1) * kStep);

        u32x4 af[MW][P], bf[4];
#pragma unroll
        for (int mt = 0; mt < MW; ++mt)
#pragma unroll
            for (int p = 0; p < P; ++p)
                af[mt][p] = *reinterpret_cast<const u32x4*>(&sa[p][wm * (TM / 2) + mt * 16 + li][8 * g]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
            bf[nt] = *reinterpret_cast<const u32x4*>(&sb[wn * 64 + nt * 16 + li][8 * g]);
#pragma unroll
        for (int mt = 0; mt < MW; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                for (int p = 0; p < P; ++p)
                    acc[mt][nt] = mfma16<WT>(af[mt][p], bf[nt], acc[mt][nt]);
    }
#undef WSP_TILE_LOAD

    // acc[mt][nt][r] of lane (g, li) is C[4g + r][li] of that 16 x 16 tile.
#pragma unroll
    for (int mt = 0; mt < MW; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
        {
            const int row = m_block + wm * (TM / 2) + mt * 16 + 4 * g + r;
            if (row >= a.rows)
                continue;
            const size_t base = (size_t) (row / a.rows_per_group) * a.group_stride
                                + (size_t) (row % a.rows_per_group) * a.ldy;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
            {
                const int n = n_block + wn * 64 + nt * 16 + li;
                const int seg = n < a.split ? 0 : n < a.split2 ? 1 : 2;
                const int c = seg == 0 ? n : seg == 1 ? n - a.split : n - a.split2;
                const float* bias = seg == 0 ? a.bias0 : seg == 1 ? a.bias1 : a.bias2;
                float* y = seg == 0 ? a.y0 : seg == 1 ? a.y1 : a.y2;
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

// 128-row tiles unless that leaves most of the chip idle: a grid of fewer
// blocks than CUs takes 64-row tiles (twice the blocks, each half the work).
hipError_t tile_product(hipStream_t stream, const TileProduct& product)
{
    TileProduct a = product;
    if (a.split2 <= 0 || a.split2 > a.out)
        a.split2 = a.out;
    if (a.split2 < a.split || a.split2 % kTile != 0)
        return hipErrorInvalidValue;
    static const int units = [] {
        int device = 0, count = 0;
        if (hipGetDevice(&device) == hipSuccess
            && hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && count > 0)
            return count;
        return 256;
    }();
    const int columns = a.out / kTile;
    const bool narrow = (long long) columns * ((a.rows + kTile - 1) / kTile) < 4LL * units;
    // 32-row tiles when even 64-row tiles give fewer blocks than CUs (the
    // tiny.en encoder's 384-column products: 72 blocks of 64 rows).
    const bool narrowest = narrow && (long long) columns * ((a.rows + 63) / 64) < units;
    const int tm = narrowest ? 32 : narrow ? 64 : kTile;
    const dim3 grid(columns, (a.rows + tm - 1) / tm);
    if (a.wdtype == kF16)
    {
        if (narrowest)
            hipLaunchKernelGGL((tile_product_kernel<kF16, 32>), grid, dim3(kThreads), 0, stream, a);
        else if (narrow)
            hipLaunchKernelGGL((tile_product_kernel<kF16, 64>), grid, dim3(kThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((tile_product_kernel<kF16, kTile>), grid, dim3(kThreads), 0, stream, a);
    }
    else
    {
        if (narrowest)
            hipLaunchKernelGGL((tile_product_kernel<kBF16, 32>), grid, dim3(kThreads), 0, stream, a);
        else if (narrow)
            hipLaunchKernelGGL((tile_product_kernel<kBF16, 64>), grid, dim3(kThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((tile_product_kernel<kBF16, kTile>), grid, dim3(kThreads), 0, stream, a);
    }
    return hipGetLastError();
}
} // namespace wsp::ops
