// The encoder's products on gfx950 matrix cores with pre-split activations:
// y = X·Wᵀ for fp32 X of 1500 rows and a 16-bit W (Encoder/Encoder.cpp:82-174:
// the q/k/v, attention-output, fc1 and fc2 products of every layer).
//
// X is stored once in exact 16-bit parts (three bf16 parts for bf16 weights,
// fp16 hi + lo for fp16 weights, |x| < 65504), part-major: part p of row r at
// parts + p·part_stride + r·inner. Every matrix-core product of a part with W
// is exact, and the fp32 sums match an fp32 product with widened weights to
// fp32 rounding. The parts are written by split_rows (from fp32 rows) or by a
// product's own epilogue (fc1 writes its GELU output as parts for fc2), so
// the products' inner loops carry no conversion work.
//
// A 256-thread block computes a 128 x TN tile (TN 128, or 64 where 128-column
// tiles would leave most CUs idle) in 32-wide k-steps. Both operands go
// straight from memory into LDS with direct-to-LDS loads (each lane's 16 bytes
// land at the wave's slot + 16·lane), into one of kStages stage buffers, so a
// step's loads are issued kStages - 1 steps before its products and hold no
// registers meanwhile. A 16-byte chunk c (8 k values) of tile row r sits at
// slot 4r + (c ^ ((r >> 1) & 3)): a 16-byte operand read serves eight lanes
// (128 bytes, the 32 banks) at a time, and the matrix-core operand reads (rows
// li of a 16-row tile, chunk g, for lanes (li, g)) then give each eight lanes
// eight different bank groups. The
// loads are issued from inline assembly with explicit waits: the compiler's
// own wait insertion would drain every load in flight before each LDS read.
// The four waves form a 2 x 2 grid of 64 x TN/2 sub-tiles.
#include "device_common.h"
#include "ops.h"

namespace wsp::ops
{
namespace
{
typedef uint16_t u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kThreads = 256;
constexpr int kTileRows = 128;
constexpr int kStep = 32;       // k per step: four 16-byte chunks of 16-bit values per row
// Stage buffers: 128-column tiles keep two (64 KB, two blocks a CU), 64-column
// tiles four (112 KB for bf16, one block a CU): at 1500 rows the 128-column
// products ran 70 us a launch with two stages against 96 with four, the
// 64-column ones 72 with four against 84 with two.
template <int TN>
constexpr int kStages = TN == 128 ? 2 : 4;
constexpr int kSplitThreads = 256;
constexpr int kWaveRows = 4; // waves along the tile's rows (the rest along its columns)

template <int WT>
constexpr int parts_of()
{
    return WT == kF16 ? 2 : 3;
}

template <int WT>
__device__ __forceinline__ float4v mfma16(u32x4 a, u32x4 b, float4v c)
{
    if constexpr (WT == kF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                       0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                        0, 0, 0);
}

template <int WT>
__device__ __forceinline__ void split(float x, uint32_t (&bits)[3])
{
    exact_parts<WT>(x, bits);
}

// Eight consecutive values of a row as parts: part p's eight 16-bit values in
// out[p] (the first value in the low half of the first word).
template <int WT>
__device__ __forceinline__ void split8(const float (&v)[8], u32x4 (&out)[3])
{
#pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        uint32_t b0[3], b1[3];
        split<WT>(v[2 * j], b0);
        split<WT>(v[2 * j + 1], b1);
#pragma unroll
        for (int p = 0; p < 3; ++p)
            out[p][j] = b0[p] | (b1[p] << 16);
    }
}

// fp32 rows [rows][width] -> parts; one thread converts eight values.
template <int WT>
__global__ void __launch_bounds__(kSplitThreads) split_rows_kernel(const float* __restrict__ x, size_t count,
                                                                   u16* __restrict__ parts, size_t part_stride)
{
    constexpr int P = parts_of<WT>();
    const size_t i = ((size_t) blockIdx.x * kSplitThreads + threadIdx.x) * 8;
    if (i >= count)
        return;
    const float4v a = *reinterpret_cast<const float4v*>(x + i);
    const float4v b = *reinterpret_cast<const float4v*>(x + i + 4);
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    u32x4 out[3];
    split8<WT>(v, out);
#pragma unroll
    for (int p = 0; p < P; ++p)
        *reinterpret_cast<u32x4*>(parts + p * part_stride + i) = out[p];
}

// LayerNorm of one row per wave (ops::layernorm's arithmetic: the mean, the
// centred squares' mean, then (x - mean)·rstd·gamma + beta), written as the
// parts of split_product's input. A lane holds float4 runs lane, lane + 64,
// ... of the row in registers (at most kNormRuns of them), so the row is read
// once; each part's four values of a run go out as one 8-byte store.
constexpr int kNormRowsPerBlock = 4;
constexpr int kNormRuns = 8; // widths up to 2048

template <int WT>
__global__ void __launch_bounds__(kNormRowsPerBlock * kWave) layernorm_parts_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta, int rows,
    int width, float eps, u16* __restrict__ parts, size_t part_stride)
{
    constexpr int P = parts_of<WT>();
    const int row = blockIdx.x * kNormRowsPerBlock + (int) threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (row >= rows)
        return;
    const int runs = width / 4;
    const float* src = x + (size_t) row * width;
    float4v v[kNormRuns];
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < kNormRuns; ++i)
    {
        const int r = lane + kWave * i;
        v[i] = r < runs ? *reinterpret_cast<const float4v*>(src + 4 * r) : float4v {0.f, 0.f, 0.f, 0.f};
        total += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
    }
    const float mean = wave_sum(total) / (float) width;
    float squares = 0.f;
#pragma unroll
    for (int i = 0; i < kNormRuns; ++i)
        if (lane + kWave * i < runs)
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const float c = v[i][e] - mean;
                squares += c * c;
            }
    const float scale = rsqrtf(wave_sum(squares) / (float) width + eps);
#pragma unroll
    for (int i = 0; i < kNormRuns; ++i)
    {
        const int r = lane + kWave * i;
        if (r >= runs)
            continue;
        uint32_t bits[4][3];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            split<WT>((v[i][e] - mean) * scale * gamma[4 * r + e] + beta[4 * r + e], bits[e]);
#pragma unroll
        for (int p = 0; p < P; ++p)
            *reinterpret_cast<uint2*>(parts + p * part_stride + (size_t) row * width + 4 * r)
                = uint2 {bits[0][p] | (bits[1][p] << 16), bits[2][p] | (bits[3][p] << 16)};
    }
}

// The LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_address(const void* p)
{
    return (uint32_t) (uintptr_t) (lds_char*) (p);
}

// One direct-to-LDS load: this lane's 16 bytes at base + offset land at LDS
// address lds + 16·lane (lds uniform over the wave).
__device__ __forceinline__ void load_lds16(const void* base, uint32_t offset, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(offset), "s"(base)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_loads()
{
    static_assert(N >= 0 && N < 64, "vmcnt holds 0..63");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Slot of chunk c of tile row r (16-byte slots).
__device__ __forceinline__ int slot(int r, int c)
{
    return 4 * r + (c ^ ((r >> 1) & 3));
}

template <int WT, int TN>
struct Layout
{
    static constexpr int P = parts_of<WT>();
    static constexpr int kABytes = kTileRows * kStep * 2;          // one part's tile
    static constexpr int kStageBytes = P * kABytes + TN * kStep * 2;
    static constexpr int kLoads = (P * kTileRows + TN) / 16;       // wave loads (1 KB each) per stage
    static_assert(kLoads % 4 == 0, "whole loads per wave");
    static constexpr int kPerWave = kLoads / 4;
    static constexpr int kStages = wsp::ops::kStages<TN>;
};

template <int WT, int TN>
__global__ void __launch_bounds__(kThreads) split_product_kernel(SplitProduct a)
{
    using L = Layout<WT, TN>;
    constexpr int P = L::P;
    constexpr int WM = kWaveRows, WN = 4 / WM;   // the waves' grid over the tile
    constexpr int MT = kTileRows / 16 / WM;     // 16-row tiles per wave
    constexpr int NT = TN / 16 / WN;            // 16-column tiles per wave
    extern __shared__ __attribute__((aligned(16))) unsigned char stage_mem[];

    const int tid = threadIdx.x, lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave); // uniform, so the load bases are scalar
    const int li = lane % 16, g = lane / 16;
    const int wm = wave / WN, wn = wave % WN;
    const int n_block = blockIdx.x * TN, m_block = blockIdx.y * kTileRows;
    const int steps = a.inner / kStep;
    // The block's columns lie in one of the (up to three) matrices.
    const int seg = n_block < a.split ? 0 : n_block < a.split2 ? 1 : 2;
    const int seg_first = seg == 0 ? 0 : seg == 1 ? a.split : a.split2;
    const void* w = seg == 0 ? a.w0 : seg == 1 ? a.w1 : a.w2;

    // This wave's loads: load q = wave + 4 t of a stage covers 16 tile rows
    // (parts' rows first, then W's); lane i moves row 16 q' + i / 4, chunk
    // (i % 4) ^ ((row >> 1) & 3), so it lands in that chunk's slot.
    const void* src[L::kPerWave];
    uint32_t offset[L::kPerWave];
    uint32_t dst[L::kPerWave]; // byte offset in the stage
#pragma unroll
    for (int t = 0; t < L::kPerWave; ++t)
    {
        const int q = wave + 4 * t;
        const int r = 16 * (q % (kTileRows / 16)) + lane / 4; // row within its tile (parts: 128 rows)
        if (q < P * (kTileRows / 16))
        {
            const int p = q / (kTileRows / 16);
            const int row = min(m_block + r, a.rows - 1);
            const int c = (lane % 4) ^ ((r >> 1) & 3);
            src[t] = a.parts;
            offset[t] = (uint32_t) (((size_t) p * a.part_stride + (size_t) row * a.inner + 8 * c) * 2);
            dst[t] = p * L::kABytes + 1024 * (q % (kTileRows / 16));
        }
        else
        {
            const int wq = q - P * (kTileRows / 16);
            const int col = 16 * wq + lane / 4;
            const int c = (lane % 4) ^ ((col >> 1) & 3);
            src[t] = w;
            offset[t] = (uint32_t) (((size_t) (n_block - seg_first + col) * a.inner + 8 * c) * 2);
            dst[t] = P * L::kABytes + 1024 * wq;
        }
    }
    const uint32_t stage0 = lds_address(stage_mem);
    // Issues step `step`'s loads into stage buffer `buf` (a step past the end
    // reloads the last one into a buffer no one reads again).
    auto issue = [&](int step, int buf) {
        const uint32_t k_bytes = (uint32_t) min(step, steps - 1) * (kStep * 2);
#pragma unroll
        for (int t = 0; t < L::kPerWave; ++t)
            load_lds16(src[t], offset[t] + k_bytes,
                       __builtin_amdgcn_readfirstlane(stage0 + buf * L::kStageBytes + dst[t]));
    };

    float4v acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
            acc[i][j] = float4v {0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < L::kStages - 1; ++s)
        issue(s, s);
    int buf = 0;
    for (int s = 0; s < steps; ++s)
    {
        // This wave's loads of step s are done once at most the later
        // kStages - 2 steps' loads are in flight; the barrier then makes every
        // wave's loads visible and ends every read of the buffer refilled next.
        wait_loads<(L::kStages - 2) * L::kPerWave>();
        __syncthreads();
        issue(s + L::kStages - 1, buf == 0 ? L::kStages - 1 : buf - 1);
        const unsigned char* st = stage_mem + buf * L::kStageBytes;
        u32x4 af[MT][P], bf[NT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int p = 0; p < P; ++p)
                af[mt][p] = reinterpret_cast<const u32x4*>(st + p * L::kABytes)[slot(16 * (MT * wm + mt) + li, g)];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            bf[nt] = reinterpret_cast<const u32x4*>(st + P * L::kABytes)[slot(16 * (NT * wn + nt) + li, g)];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int p = 0; p < P; ++p)
                    acc[mt][nt] = mfma16<WT>(af[mt][p], bf[nt], acc[mt][nt]);
        buf = buf == L::kStages - 1 ? 0 : buf + 1;
    }
    wait_loads<0>();

    // acc[mt][nt][r] of lane (g, li) is C[4g + r][li] of that 16 x 16 tile.
    float* y = seg == 0 ? a.y0 : seg == 1 ? a.y1 : a.y2;
    const float* bias = seg == 0 ? a.bias0 : seg == 1 ? a.bias1 : a.bias2;
    const float scale = seg == 0 ? a.scale0 : seg == 1 ? a.scale1 : a.scale2;
    const int width = seg == 0 ? a.split : seg == 1 ? a.split2 - a.split : a.out - a.split2;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
    {
        const int c = n_block - seg_first + 16 * (NT * wn + nt) + li;
        const float b = bias != nullptr ? bias[c] : 0.f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const int row = m_block + 16 * (MT * wm + mt) + 4 * g + r;
                if (row >= a.rows)
                    continue;
                float v = acc[mt][nt][r] * scale + b;
                if (a.flags & kProductGelu)
                    v = exact_gelu(v);
                if (a.out_parts != nullptr)
                {
                    uint32_t bits[3];
                    split<WT>(v, bits);
                    u16* o = static_cast<u16*>(a.out_parts) + (size_t) row * width + c;
#pragma unroll
                    for (int p = 0; p < P; ++p)
                        o[p * a.out_part_stride] = (u16) bits[p];
                }
                else if ((seg == 1 && a.y1_halves != nullptr) || (seg == 2 && a.y2_halves_t != nullptr))
                {
                    const _Float16 hi = (_Float16) v;
                    const _Float16 lo = (_Float16) (v - (float) hi);
                    u16* o = seg == 1 ? static_cast<u16*>(a.y1_halves) + (size_t) row * width + c
                                      : static_cast<u16*>(a.y2_halves_t) + (size_t) c * a.halves_pitch + row;
                    o[0] = __builtin_bit_cast(u16, hi);
                    o[(size_t) a.halves_pitch * width] = __builtin_bit_cast(u16, lo);
                }
                else if (a.flags & kProductResidual)
                    y[(size_t) row * a.ldy + c] += v;
                else
                    y[(size_t) row * a.ldy + c] = v;
            }
    }
}

template <int WT>
hipError_t launch(hipStream_t stream, const SplitProduct& a, bool wide)
{
    const dim3 grid(a.out / (wide ? 128 : 64), (a.rows + kTileRows - 1) / kTileRows);
    constexpr size_t wide_bytes = kStages<128> * Layout<WT, 128>::kStageBytes;
    constexpr size_t narrow_bytes = kStages<64> * Layout<WT, 64>::kStageBytes;
    if (wide)
        hipLaunchKernelGGL((split_product_kernel<WT, 128>), grid, dim3(kThreads), wide_bytes, stream, a);
    else
        hipLaunchKernelGGL((split_product_kernel<WT, 64>), grid, dim3(kThreads), narrow_bytes, stream, a);
    return hipGetLastError();
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

template <int WT, int TN>
hipError_t allow_stages()
{
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&split_product_kernel<WT, TN>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kStages<TN> * Layout<WT, TN>::kStageBytes);
}
} // namespace

bool split_product_fits(int wdtype, int inner, int out, int split, int split2)
{
    return (wdtype == kF16 || wdtype == kBF16) && inner % kStep == 0 && out % 128 == 0 && split % 128 == 0
           && split2 % 128 == 0 && split <= split2 && split2 <= out;
}

hipError_t split_rows(hipStream_t stream, const float* x, size_t count, int wdtype, void* parts, size_t part_stride)
{
    if (count % 8 != 0 || (wdtype != kF16 && wdtype != kBF16))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) ((count / 8 + kSplitThreads - 1) / kSplitThreads));
    if (wdtype == kF16)
        hipLaunchKernelGGL(split_rows_kernel<kF16>, grid, dim3(kSplitThreads), 0, stream, x, count,
                           static_cast<u16*>(parts), part_stride);
    else
        hipLaunchKernelGGL(split_rows_kernel<kBF16>, grid, dim3(kSplitThreads), 0, stream, x, count,
                           static_cast<u16*>(parts), part_stride);
    return hipGetLastError();
}

bool layernorm_parts_fits(int width)
{
    return width > 0 && width % 4 == 0 && width <= 4 * kWave * kNormRuns;
}

hipError_t layernorm_parts(hipStream_t stream, const float* x, const float* gamma, const float* beta, void* parts,
                           size_t part_stride, int rows, int width, float eps, int wdtype)
{
    if (!layernorm_parts_fits(width) || (wdtype != kF16 && wdtype != kBF16))
        return hipErrorInvalidValue;
    const dim3 grid((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
    if (wdtype == kF16)
        hipLaunchKernelGGL(layernorm_parts_kernel<kF16>, grid, dim3(kNormRowsPerBlock * kWave), 0, stream, x, gamma,
                           beta, rows, width, eps, static_cast<u16*>(parts), part_stride);
    else
        hipLaunchKernelGGL(layernorm_parts_kernel<kBF16>, grid, dim3(kNormRowsPerBlock * kWave), 0, stream, x,
                           gamma, beta, rows, width, eps, static_cast<u16*>(parts), part_stride);
    return hipGetLastError();
}

// 128-column tiles unless they would leave more than an eighth of the CUs
// idle (the 1280-column products at 1500 rows: 120 blocks), then 64.
hipError_t split_product(hipStream_t stream, const SplitProduct& product)
{
    SplitProduct a = product;
    if (a.split2 <= 0 || a.split2 > a.out)
        a.split2 = a.out;
    if (a.split <= 0 || a.split > a.split2)
        a.split = a.split2;
    if (!split_product_fits(a.wdtype, a.inner, a.out, a.split, a.split2))
        return hipErrorInvalidValue;
    static const hipError_t allowed = [] {
        hipError_t e = allow_stages<kF16, 128>();
        if (e == hipSuccess)
            e = allow_stages<kF16, 64>();
        if (e == hipSuccess)
            e = allow_stages<kBF16, 128>();
        if (e == hipSuccess)
            e = allow_stages<kBF16, 64>();
        return e;
    }();
    if (allowed != hipSuccess)
        return allowed;
    const long long wide_blocks = (long long) (a.out / 128) * ((a.rows + kTileRows - 1) / kTileRows);
    const bool wide = 8 * wide_blocks >= 7 * compute_units();
    return a.wdtype == kF16 ? launch<kF16>(stream, a, wide) : launch<kBF16>(stream, a, wide);
}
} // namespace wsp::ops
