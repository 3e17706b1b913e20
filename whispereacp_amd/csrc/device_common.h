// Device helpers shared by the gfx950 kernels: weight widening, wave64
// reductions and the exact GELU. CDNA4 only: waves are 64 lanes wide.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wsp
{
constexpr int kWave = 64;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

enum WeightType : int
{
    kF32 = 0,
    kF16 = 1,
    kBF16 = 2
};

// Global-memory views of pointers the compiler cannot place itself (pointers
// read from LDS or from memory). Accesses through them are global_load /
// global_store, which count only in vmcnt; the same access through a generic
// pointer is a flat access, which also counts in lgkmcnt, so every later LDS
// wait would also wait for it.
template <class T>
using global_ptr = __attribute__((address_space(1))) T*;

template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* global(const T* p)
{
    return (const __attribute__((address_space(1))) T*) p;
}

template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* global_mut(T* p)
{
    return (__attribute__((address_space(1))) T*) p;
}

// Sums within a 16-lane DPP row in a fixed order: swap neighbours, swap
// pairs, mirror within 8 and mirror within 16 leave the row total in every
// lane, each step one v_add_f32_dpp. Every pair is added in an
// order-independent way (a + b == b + a), so every lane of the row holds the
// same bits. Every lane of the row must be active.
// (bound_ctrl set: every pattern used reads a lane of the same row, so no lane
// reads out of range, and the move folds into the consuming add as one
// v_add_f32_dpp.)
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

constexpr int kSwapNeighbours = 0xB1; // quad_perm [1,0,3,2]
constexpr int kSwapPairs = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kMirrorHalfRow = 0x141; // row_half_mirror
constexpr int kMirrorRow = 0x140;     // row_mirror

__device__ __forceinline__ float sum16(float v)
{
    v += dpp<kSwapNeighbours>(v);
    v += dpp<kSwapPairs>(v);
    v += dpp<kMirrorHalfRow>(v);
    v += dpp<kMirrorRow>(v);
    return v;
}

// 16 bytes from global memory.
__device__ __forceinline__ uint4 load_global16(const void* p)
{
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = *global(static_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ float bf16_to_float(uint16_t bits)
{
    return __uint_as_float((uint32_t) bits << 16);
}

// Eight consecutive weights widened to float from one 16-byte load (F16,
// BF16) or two (F32). `index` is an element index, a multiple of 8.
template <int WT>
__device__ __forceinline__ void load8(const void* base, size_t index, float (&w)[8])
{
    if constexpr (WT == kF32)
    {
        const float4v* p = reinterpret_cast<const float4v*>(static_cast<const float*>(base) + index);
        const float4v a = p[0], b = p[1];
        w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
        w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
    }
    else if constexpr (WT == kF16)
    {
        const half8 h = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(base) + index);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[i] = (float) h[i];
    }
    else
    {
        const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + index);
        const uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            w[2 * i] = __uint_as_float(v[i] << 16);
            w[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
        }
    }
}

template <int WT>
__device__ __forceinline__ float load1(const void* base, size_t index)
{
    if constexpr (WT == kF32)
        return static_cast<const float*>(base)[index];
    else if constexpr (WT == kF16)
        return (float) static_cast<const _Float16*>(base)[index];
    else
        return bf16_to_float(static_cast<const uint16_t*>(base)[index]);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v = fmaxf(v, __shfl_xor(v, offset, kWave));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (at most 1024). `scratch`
// holds one float per wave. Every thread returns the total.
__device__ __forceinline__ float block_sum(float v, float* scratch)
{
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int waves = blockDim.x / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0)
        scratch[wave] = v;
    __syncthreads();
    float total = 0.f;
    for (int i = 0; i < waves; ++i)
        total += scratch[i];
    return total;
}

__device__ __forceinline__ float block_max(float v, float* scratch)
{
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int waves = blockDim.x / kWave;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0)
        scratch[wave] = v;
    __syncthreads();
    float best = scratch[0];
    for (int i = 1; i < waves; ++i)
        best = fmaxf(best, scratch[i]);
    return best;
}

// x as exact 16-bit parts for products with 16-bit weights of type WT
// (kF16: fp16 hi + lo, for |x| < 65504; kBF16: three bf16 parts); part p in
// the low 16 bits of bits[p], and x equals the sum of the parts.
template <int WT>
__device__ __forceinline__ void exact_parts(float x, uint32_t (&bits)[3])
{
    if constexpr (WT == kF16)
    {
        const _Float16 hi = (_Float16) x;
        const _Float16 lo = (_Float16) (x - (float) hi);
        bits[0] = __builtin_bit_cast(uint16_t, hi);
        bits[1] = __builtin_bit_cast(uint16_t, lo);
        bits[2] = 0;
    }
    else
    {
        float rest = x;
#pragma unroll
        for (int p = 0; p < 3; ++p)
        {
            const __bf16 b = (__bf16) rest;
            bits[p] = __builtin_bit_cast(uint16_t, b);
            rest -= (float) b;
        }
    }
}

// x * 0.5 * (1 + erf(x / sqrt(2))), the exact form (Kernels/Gelu.h:16-21),
// with the device library's erff.
__device__ __forceinline__ float exact_gelu(float x)
{
    return 0.5f * x * (1.f + erff(x * 0.70710678118654752f));
}
} // namespace wsp
