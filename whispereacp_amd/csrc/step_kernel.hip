// The single-token decoder step (Decoder/Decoder.cpp:151-177 with one token,
// then Argmax over the logits row, Whisper/Whisper.cpp:1164-1184) as ONE
// persistent launch on gfx950 (every workgroup resident at once).
//
// Why one launch: at batch 1 every phase of the step is a dependent GEMV or
// attention of a few MB, so a launch per op (170+ per step) is bound by launch
// and drain latency, not by HBM. Here every workgroup stays resident for the
// whole step and the phases hand activations to each other through
// "exchange words": 64-bit words carrying a float and the step's epoch, stored
// and polled with device-scope relaxed atomics. A consumer sees a value and
// its validity in one load, so a hand-over costs one store-to-load trip
// through the memory side, with no barrier and no flag round trip.
//
// Why it streams at bandwidth: a workgroup issues the loads of its slice of
// the NEXT phase's weights right after it stores the current phase's outputs
// (two register sets alternate), so a phase's weights are in registers when
// its input arrives and HBM traffic overlaps the hand-over chain. The layer table lives
// in LDS, so no phase waits on a pointer load, and every cross-lane reduction
// is a DPP/swizzle tree in a fixed order.
//
// Roles (G workgroups of 512 threads, one per CU):
//   - the first Gg ("row" groups) run every projection and the
//     cross-attention key chunks;
//   - the last Ga = heads * self_split_max ("head" groups) run self-attention,
//     each holding its head's cached keys and values in registers (loaded one
//     layer ahead), and the cross-attention combine of one head;
//   - all of them run the tied logits.
// Per layer the chain is: LN1+QKV -> self attention -> out-proj (+residual)
// -> LN2+cross-q -> cross partials -> cross combine -> cross out (+residual)
// -> LN3+fc1+GELU -> fc2 (+residual). Then final LN + tied logits with a
// per-workgroup top-1, and the argmax fold in the last workgroup.
//
// Every wait is bounded: a watchdog flags the context's status word and all
// workgroups leave, so a broken hand-over ends the launch instead of hanging.
#include "device_common.h"
#include "step_kernel.h"

#include <cmath>

namespace wsp::step
{
namespace
{
constexpr int kKeyLanes = 16;                      // lanes per key row (4 channels each)
constexpr int kKeySlots = kThreads / kKeyLanes;    // keys per pass
constexpr int kSelfPasses = kSelfKeys / kKeySlots; // self keys held per head group
constexpr int kCrossPasses = kCrossKeys / kKeySlots;
constexpr int kRowLanes = 32;                      // lanes per projection row
constexpr int kRowGroups = kThreads / kRowLanes;   // rows in flight per workgroup
constexpr int kChunks = 3;                         // 16-byte chunks per lane per row slice
constexpr int kRing = 5;                           // logits rows in flight per row group (6, 7, 8: slower)
constexpr int kWaves = kThreads / kWave;
constexpr int kSpinLimit = 1 << 21;                // poll rounds before the watchdog trips
constexpr uint32_t kUnchosen = 0xFFFFFFFFu;

static_assert(kSelfKeys % kKeySlots == 0 && kCrossKeys % kKeySlots == 0, "key capacities");
static_assert(kKeySlots / kWaves == 4, "attend() folds four key slots per wave");

// Optional timeline: built with WSP_STEP_TIMELINE, thread 0 of every
// workgroup records the real-time clock (100 MHz) at the points marked
// STEP_STAMP(event, layer) into LDS, and the kernel writes them to
// StepArgs::timeline ([workgroup][kTimelineEvents][kTimelineLayers]) at its
// end. Without it the marks compile to nothing.
// STEP_MARK(event) stamps inside a phase, at the layer the workgroup last
// named with STEP_LAYER (events below 0 are not stamped).
constexpr int kTimelineEvents = 40, kTimelineLayers = 33;
#ifdef WSP_STEP_TIMELINE
#define STEP_STAMP(e, l)                                      \
    do                                                        \
    {                                                         \
        if (threadIdx.x == 0)                                 \
            sh.timeline[(e)][(l)] = wall_clock64();           \
    } while (0)
#define STEP_LAYER(l)                                         \
    do                                                        \
    {                                                         \
        if (threadIdx.x == 0)                                 \
            sh.mark_layer = (l);                              \
    } while (0)
#define STEP_MARK(e)                                          \
    do                                                        \
    {                                                         \
        if (threadIdx.x == 0 && (e) >= 0)                     \
            sh.timeline[(e)][sh.mark_layer] = wall_clock64(); \
    } while (0)
#else
#define STEP_STAMP(e, l) \
    do                   \
    {                    \
    } while (0)
#define STEP_LAYER(l) \
    do                \
    {                 \
    } while (0)
#define STEP_MARK(e) \
    do               \
    {                \
    } while (0)
#endif

// A workgroup-uniform pointer as a value the compiler knows to be uniform, so
// it lives in a scalar register pair (a load's saddr operand, with a 32-bit
// per-lane offset beside it). readfirstlane returns a signed int: each half
// goes through uint32_t so it is zero-extended.
template <class T>
__device__ __forceinline__ T* uniform(T* p)
{
    const uint64_t at = reinterpret_cast<uint64_t>(p);
    const uint32_t high = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (at >> 32));
    const uint32_t low = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) at);
    return reinterpret_cast<T*>(((uint64_t) high << 32) | (uint64_t) low);
}

// ---------------------------------------------------------------------------
// Exchange words
// ---------------------------------------------------------------------------
__device__ __forceinline__ void put(uint64_t* p, float v, uint32_t epoch)
{
    const uint64_t word = ((uint64_t) epoch << 32) | (uint64_t) __float_as_uint(v);
    __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t peek(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Cross-lane sums and maxima in a fixed order. Within a 16-lane row, sum16
// (device_common.h) leaves the row total in every lane; a permlane16 swap
// then adds the neighbouring row (lane l and lane l ^ 16) and a permlane32
// swap the other half of the wave (lane l and lane l ^ 32). Both swaps are
// VALU operations of gfx950: no LDS round trip and no scalar register. Every
// pair is added in an order-independent way (a + b == b + a), so every lane
// of the span holds the same bits. Every lane of the span must be active.
// ---------------------------------------------------------------------------
// Lane l's value and lane (l ^ 16)'s, in an order that depends only on l.
__device__ __forceinline__ void rows_pair_bits(uint32_t v, uint32_t& a, uint32_t& b)
{
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

// Lane l's value and lane (l ^ 32)'s, in an order that depends only on l.
__device__ __forceinline__ void halves_pair_bits(uint32_t v, uint32_t& a, uint32_t& b)
{
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

__device__ __forceinline__ void rows_pair(float v, float& a, float& b)
{
    uint32_t x, y;
    rows_pair_bits(__float_as_uint(v), x, y);
    a = __uint_as_float(x);
    b = __uint_as_float(y);
}

__device__ __forceinline__ void halves_pair(float v, float& a, float& b)
{
    uint32_t x, y;
    halves_pair_bits(__float_as_uint(v), x, y);
    a = __uint_as_float(x);
    b = __uint_as_float(y);
}

__device__ __forceinline__ float add16(float v)
{
    float a, b;
    rows_pair(v, a, b);
    return a + b;
}

__device__ __forceinline__ float add32(float v)
{
    float a, b;
    halves_pair(v, a, b);
    return a + b;
}

__device__ __forceinline__ float halves_sum(float v)
{
    return add32(v);
}

__device__ __forceinline__ float sum32(float v)
{
    return add16(sum16(v));
}

__device__ __forceinline__ float sum64(float v)
{
    return halves_sum(sum32(v));
}

__device__ __forceinline__ float max64(float v)
{
    v = fmaxf(v, dpp<kSwapNeighbours>(v));
    v = fmaxf(v, dpp<kSwapPairs>(v));
    v = fmaxf(v, dpp<kMirrorHalfRow>(v));
    v = fmaxf(v, dpp<kMirrorRow>(v));
    float a, b;
    rows_pair(v, a, b);
    v = fmaxf(a, b);
    halves_pair(v, a, b);
    return fmaxf(a, b);
}

// Per-token rows in LDS: token k's residual row at raw + k * kRawStride, its
// head block (query, new key, new value) at q + k * kQStride, and element i
// of its phase input at x + x_at<T>(k, i). The single-token kernel keeps that
// input contiguous. With T tokens the inputs interleave in blocks of eight
// floats, token k's block c at c * kXBlock<T> + 8 k: a lane's chunk then has
// one address for every token (the tokens sit at immediate offsets of the LDS
// instructions), and a pad of four floats per block spreads the lanes' reads
// over the banks.
constexpr int kRawStride = kMaxWidth;
constexpr int kQStride = 3 * kMaxHeadWidth;
template <int T>
constexpr int kXBlock = T == 1 ? 8 : 8 * T + 4;
constexpr int kXFloats = kMaxFeedForward / 8 * kXBlock<kMaxTokens>;
static_assert(kMaxFeedForward % 8 == 0, "whole blocks");

template <int T>
__device__ __forceinline__ int x_at(int k, int i)
{
    if constexpr (T == 1)
        return i;
    else
        return (i >> 3) * kXBlock<T> + 8 * k + (i & 7);
}

// The large per-token rows come last: every array's base then stays below
// 64 KB, within the 16-bit offset of an LDS instruction, for token 0.
struct Shared
{
    wsp_layer_tensors table[kMaxLayers]; // the layer table, read once per launch
    float comb[kMaxCombine];             // attention partials being combined
    float red[kWaves][kMaxHeadWidth];    // per-wave value rows of an attention chunk
    float q[kMaxTokens * kQStride];      // a head's query, then (self-attention) its new key and value
    float scratch[kMaxTokens][2][kWaves]; // per-wave maxima and sums of an attention chunk, per query
    float fold[kWaves][kMaxTokens][2];   // per-wave sums of (x - K) and (x - K)^2 of a folded LayerNorm
    alignas(16) float part[kMaxTokens * kRowGroups]; // per-row-group partial sums of a projection pass
    float best_v[kRowGroups];
    uint32_t best_i[kRowGroups];
    int abort;
    alignas(16) float raw[kMaxTokens * kRawStride]; // the residual stream as gathered (un-normalised)
    alignas(16) float x[kXFloats];                  // the current phase's input vectors
    float red_more[kMaxTokens - 1][kWaves][kMaxHeadWidth]; // red for the queries of tokens 1.. (multi-token)
#ifdef WSP_STEP_TIMELINE
    uint64_t timeline[kTimelineEvents][kTimelineLayers];
    int mark_layer;
#endif
};

// Waits until the n words map(i) (i < n <= P * 448) of base carry `epoch`
// and copies their floats to dst (LDS). map(i, offset, index) names word i's
// offset from base and its index in dst, or returns false for a slot that
// holds nothing. Waves 1-7 poll; wave 0 — the wave that stores a phase's
// outputs — only waits for its own stores meanwhile, because on this
// architecture a load's completion count also covers earlier stores, so a
// poll issued behind them would see nothing until they were acknowledged.
// Every poll round issues all of a thread's outstanding loads at once. Returns
// false, uniformly over the workgroup, when the watchdog tripped here or
// anywhere else.
static_assert(kPollThreads == kThreads - kWave, "wave 0 does not poll");

// One polling thread's wait for P exchange words (word k at base +
// offset_of(k), a valid offset for every k; the set bits of `pending` name the
// words it waits for) to carry `epoch`; deliver(k, value) receives each
// awaited word's float once. The first round of loads is examined alone: a
// word that was there before the consumer asked costs one trip. After a miss
// two rounds are in flight at once, the second issued kPollStagger sleep units
// (64 clocks each) after the first, and each is issued again as soon as it has
// been examined, so a word is seen about half a trip after it lands instead of
// up to a whole trip. Every round loads all P words, so the number of loads in
// flight is fixed and the compiler's wait for the older round is exact.
// Returns false when the watchdog tripped here or anywhere else.
// Two rounds pay where few workgroups wait for a few words (a head group for
// its q/k/v rows, a cross task for its query, a combining workgroup for its
// head's partials); where every row group polls a whole vector the second
// round's loads slow the hand-over more than they shorten it, so those gathers
// keep one round in flight.
constexpr int kPollStagger = 3;  // sleep units between the two rounds
constexpr int kPollTwoMax = 1;   // poll<P> with P at most this takes two rounds by default

template <int P, class Offset>
__device__ __forceinline__ void issue_round(uint64_t (&w)[P], const uint64_t* base, const Offset& offset_of)
{
#pragma unroll
    for (int k = 0; k < P; ++k)
        w[k] = peek(base + offset_of(k));
}

template <int P, class Deliver>
__device__ __forceinline__ bool take_round(const uint64_t (&w)[P], uint32_t& pending, uint32_t epoch,
                                           const Deliver& deliver)
{
#pragma unroll
    for (int k = 0; k < P; ++k)
        if ((pending & (1u << k)) && (uint32_t) (w[k] >> 32) == epoch)
        {
            deliver(k, __uint_as_float((uint32_t) w[k]));
            pending &= ~(1u << k);
        }
    return pending == 0;
}

// The watchdog, every 32 turns of a poll loop: false when this poll gave up
// or another one did.
__device__ __forceinline__ bool watchdog_ok(int spins, int limit, int* status)
{
    if ((spins & 31) != 0)
        return true;
    if (spins > limit)
    {
        __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
}

template <int P, bool TWO, class Offset, class Deliver>
__device__ __forceinline__ bool poll_words(const uint64_t* base, const Offset& offset_of, uint32_t pending,
                                           uint32_t epoch, int* status, const Deliver& deliver)
{
    if (pending == 0)
        return true;
    uint64_t first[P];
    issue_round(first, base, offset_of);
    if (take_round(first, pending, epoch, deliver))
        return true;
    if constexpr (!TWO)
    {
        // One round in flight where two would not fit in registers.
        for (int spins = 1;; ++spins)
        {
            issue_round(first, base, offset_of);
            if (take_round(first, pending, epoch, deliver))
                return true;
            if (!watchdog_ok(spins, kSpinLimit, status))
                return false;
        }
    }
    else
    {
        uint64_t second[P];
        issue_round(first, base, offset_of);
        if constexpr (kPollStagger > 0)
            asm volatile("s_sleep %0" ::"n"(kPollStagger) : "memory");
        issue_round(second, base, offset_of);
        for (int spins = 1;; ++spins)
        {
            if (take_round(first, pending, epoch, deliver))
                return true;
            issue_round(first, base, offset_of);
            if (take_round(second, pending, epoch, deliver))
                return true;
            issue_round(second, base, offset_of);
            if (!watchdog_ok(spins, kSpinLimit / 2, status))
                return false;
        }
    }
}

template <int P, class Map, bool TWO = (P <= kPollTwoMax)>
__device__ __forceinline__ bool poll(const uint64_t* base, int n, Map map, float* dst, uint32_t epoch, int* status,
                                     Shared& sh)
{
    bool failed = false;
    if (threadIdx.x < kWave)
        __builtin_amdgcn_s_waitcnt(0); // every counter at zero: this wave's stores and loads are done
    else if constexpr (!TWO)
    {
        // Wide gathers (attention partials, the argmax candidates): each round
        // loads only the words still awaited and stores each as it arrives
        // (fewer registers than the fixed rounds below).
        const int t = threadIdx.x - kWave;
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < P; ++k)
        {
            int offset, index;
            if (t + k * kPollThreads < n && map(t + k * kPollThreads, offset, index))
                pending |= 1u << k;
        }
        for (int spins = 1; pending != 0; ++spins)
        {
            uint64_t w[P];
#pragma unroll
            for (int k = 0; k < P; ++k)
                if (pending & (1u << k))
                {
                    int offset, index;
                    map(t + k * kPollThreads, offset, index);
                    w[k] = peek(base + offset);
                }
#pragma unroll
            for (int k = 0; k < P; ++k)
                if ((pending & (1u << k)) && (uint32_t) (w[k] >> 32) == epoch)
                {
                    int offset, index;
                    map(t + k * kPollThreads, offset, index);
                    dst[index] = __uint_as_float((uint32_t) w[k]);
                    pending &= ~(1u << k);
                }
            if (pending != 0 && !watchdog_ok(spins, kSpinLimit, status))
            {
                failed = true;
                break;
            }
        }
    }
    else
    {
        const int t = threadIdx.x - kWave;
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < P; ++k)
        {
            int offset, index;
            if (t + k * kPollThreads < n && map(t + k * kPollThreads, offset, index))
                pending |= 1u << k;
        }
        failed = !poll_words<P, true>(
            base,
            [&](int k) {
                int offset, index;
                return t + k * kPollThreads < n && map(t + k * kPollThreads, offset, index) ? offset : 0;
            },
            pending, epoch, status,
            [&](int k, float v) {
                int offset, index;
                map(t + k * kPollThreads, offset, index);
                dst[index] = v;
            });
    }
    if (failed)
        sh.abort = 1;
    __syncthreads();
    return sh.abort == 0;
}

// n contiguous words.
template <int P, bool TWO = (P <= kPollTwoMax)>
__device__ __forceinline__ bool gather(const uint64_t* src, int n, float* dst, uint32_t epoch, int* status,
                                       Shared& sh)
{
    auto map = [](int i, int& offset, int& index) {
        offset = index = i;
        return true;
    };
    return poll<P, decltype(map), TWO>(src, n, map, dst, epoch, status, sh);
}

// n <= kMaxCombine contiguous words, polled with as few slots per thread as
// the count needs (a poll round costs every unrolled slot's test, so the usual
// vector of a few hundred words takes the two-slot form).
__device__ __forceinline__ bool gather_any(const uint64_t* src, int n, float* dst, uint32_t epoch, int* status,
                                           Shared& sh);

// Row-group outputs live in producer blocks: the workgroup that computes row
// r (r % stride) stores it at slot (r % stride) * 2^log2_block + r / stride,
// so each workgroup's rows share its own cache lines (no line has two
// writers) and a reader polls the slots in order.
__device__ __forceinline__ int block_slot(int row, int stride, int log2_block)
{
    return ((row % stride) << log2_block) + row / stride;
}

// The same for a vector of blocked ownership (`block` rows per workgroup).
__device__ __forceinline__ int blocked_slot(int row, int block, int log2_block)
{
    return ((row / block) << log2_block) + row % block;
}

// The whole `rows`-row vector, read slot by slot in chunks of P * 448 slots.
template <int P>
__device__ __forceinline__ bool gather_blocked(const uint64_t* base, int rows, int log2_block, int stride, float* dst,
                                               uint32_t epoch, int* status, Shared& sh)
{
    const int slots = stride << log2_block;
    const int mask = (1 << log2_block) - 1;
    for (int first = 0; first < slots; first += P * kPollThreads)
    {
        const bool ok = poll<P>(
            base + first, min(P * kPollThreads, slots - first),
            [&](int i, int& offset, int& index) {
                const int slot = first + i;
                offset = i;
                index = (slot & mask) * stride + (slot >> log2_block);
                return index < rows;
            },
            dst, epoch, status, sh);
        if (!ok)
            return false;
    }
    return true;
}

// The same for the long feed-forward vector, eight slots per polling thread
// (slot first + t + 448 k, so each load instruction of a wave reads 64
// consecutive words). A poll round is one inline-assembly statement: eight
// global_load_dwordx2 with the device-scope (sc1) cache policy, then
// s_waitcnt vmcnt(0), so no use of a loaded register can be scheduled between
// the loads and the wait (the compiler's own wait insertion does not see loads
// written in assembly). Each word is read whole: a naturally aligned
// global_load_dwordx2 with sc1 is the instruction LLVM's AMDGPU memory model
// emits on gfx942/gfx950 for a relaxed agent-scope atomic load of 64 bits
// (llvm/docs/AMDGPUUsage.rst, "Memory Model GFX942": load atomic monotonic,
// agent scope, global -> global_load sc1=1), the same access peek() makes.
// Addresses are one scalar base and eight 32-bit byte offsets, each clamped
// into the vector: a slot past it re-reads word 0 and is ignored.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// place(index) is where element `index` goes in dst (the identity for one
// token's contiguous row).
template <int P, class Place>
__device__ __forceinline__ bool gather_words(const uint64_t* base, int rows, int log2_block, int stride, float* dst,
                                             uint32_t epoch, int* status, Shared& sh, Place place)
{
    static_assert(P == 8, "the poll statement below names eight loads");
    const uint64_t scalar_base = reinterpret_cast<uint64_t>(uniform(base));
    const int slots = stride << log2_block;
    const int mask = (1 << log2_block) - 1;
    for (int first = 0; first < slots; first += P * kPollThreads)
    {
        bool failed = false;
        if (threadIdx.x < kWave)
            __builtin_amdgcn_s_waitcnt(0);
        else
        {
            const int t = threadIdx.x - kWave;
            uint32_t pending = 0;
            uint32_t off[P];
#pragma unroll
            for (int k = 0; k < P; ++k)
            {
                const int slot = first + t + k * kPollThreads;
                if (slot < slots && (slot & mask) * stride + (slot >> log2_block) < rows)
                    pending |= 1u << k;
                off[k] = (uint32_t) (slot < slots ? slot : 0) * (uint32_t) sizeof(uint64_t);
            }
            int spins = 0;
            while (pending != 0)
            {
                u32x2 v[P];
                asm volatile("global_load_dwordx2 %0, %8, %16 sc1\n\t"
                             "global_load_dwordx2 %1, %9, %16 sc1\n\t"
                             "global_load_dwordx2 %2, %10, %16 sc1\n\t"
                             "global_load_dwordx2 %3, %11, %16 sc1\n\t"
                             "global_load_dwordx2 %4, %12, %16 sc1\n\t"
                             "global_load_dwordx2 %5, %13, %16 sc1\n\t"
                             "global_load_dwordx2 %6, %14, %16 sc1\n\t"
                             "global_load_dwordx2 %7, %15, %16 sc1\n\t"
                             "s_waitcnt vmcnt(0)"
                             : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                               "=&v"(v[6]), "=&v"(v[7])
                             : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "v"(off[4]), "v"(off[5]),
                               "v"(off[6]), "v"(off[7]), "s"(scalar_base)
                             : "memory");
#pragma unroll
                for (int k = 0; k < P; ++k)
                    if ((pending & (1u << k)) && v[k][1] == epoch)
                    {
                        const int slot = first + t + k * kPollThreads;
                        dst[place((slot & mask) * stride + (slot >> log2_block))] = __uint_as_float(v[k][0]);
                        pending &= ~(1u << k);
                    }
                if (pending != 0 && (++spins & 63) == 0)
                {
                    if (spins > kSpinLimit)
                    {
                        __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        failed = true;
                        break;
                    }
                    if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
                    {
                        failed = true;
                        break;
                    }
                }
            }
        }
        if (failed)
            sh.abort = 1;
        __syncthreads();
        if (sh.abort != 0)
            return false;
    }
    return true;
}

// Words per polling thread for the vectors a phase awaits: kPollBlocked and
// kPollBlockedFF (step_kernel.h) per chunk of a blocked vector; a larger
// vector is polled chunk after chunk.

constexpr int kPollCombine = (kMaxCombine + kPollThreads - 1) / kPollThreads;
constexpr int kPollArgmax = (2 * 256 + kPollThreads - 1) / kPollThreads; // two words per workgroup candidate

__device__ __forceinline__ bool gather_any(const uint64_t* src, int n, float* dst, uint32_t epoch, int* status,
                                           Shared& sh)
{
    if (n <= 2 * kPollThreads)
        return gather<2>(src, n, dst, epoch, status, sh);
    if (n <= 3 * kPollThreads)
        return gather<3>(src, n, dst, epoch, status, sh);
    return gather<kPollCombine>(src, n, dst, epoch, status, sh);
}

// ---------------------------------------------------------------------------
// LayerNorm of sh.raw into sh.x: mean, centred biased variance, then
// (x - mean) * rsqrt(var + eps) * gamma + beta (Kernels/LayerNorm.h:44-89).
// Lane l of a wave holds the runs 4 (l + 64 k) .. + 3 of the row (n is a
// multiple of 4), read from LDS in one batch, and each wave that writes a run
// sums them in the same order, so those waves get the same statistics without
// a barrier. Wave w then writes run w (kNormRuns runs cover the widest row),
// with gamma/beta of that run held in registers since the previous phase. The
// only barrier is the one completing sh.x.
// ---------------------------------------------------------------------------
constexpr int kNormRuns = (kMaxWidth + 4 * kWave - 1) / (4 * kWave);
static_assert(kNormRuns <= kThreads / kWave, "one wave writes each run");

struct NormParams
{
    float4v g;
    float4v b;
};

// The run this thread's wave writes, clamped into the row (a wave past the
// row loads the last run and writes nothing).
__device__ __forceinline__ int norm_run(int n)
{
    const int i = 4 * ((int) (threadIdx.x & (kWave - 1)) + kWave * (int) (threadIdx.x / kWave));
    return min(i, n - 4);
}

__device__ __forceinline__ void load_norm(NormParams& p, const float* gamma, const float* beta, int n)
{
    const int i = norm_run(n);
    p.g = *global(reinterpret_cast<const float4v*>(gamma + i));
    p.b = *global(reinterpret_cast<const float4v*>(beta + i));
}

// The statistics and this wave's run, with R runs per lane (R * 256 >= n).
template <int R, int XB>
__device__ __forceinline__ void norm_row(const NormParams& p, int n, float inv_n, float eps, const float* raw,
                                         float* out, int lane, int own, int mark, Shared& sh)
{
    // Every LDS read is issued before the first is used: the row's runs and
    // this thread's own run.
    float4v v[R];
#pragma unroll
    for (int k = 0; k < R; ++k)
        v[k] = *reinterpret_cast<const float4v*>(&raw[min(4 * (lane + kWave * k), n - 4)]);
    const float4v x = *reinterpret_cast<const float4v*>(&raw[min(own, n - 4)]);
    // Pairwise sums (a fixed order, shallow dependency chains; runs past the
    // row add zeros, so the order does not depend on R).
    float t[R];
#pragma unroll
    for (int k = 0; k < R; ++k)
        t[k] = 4 * (lane + kWave * k) < n ? (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]) : 0.f;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < R; k += 2)
        s += k + 1 < R ? t[k] + t[k + 1] : t[k];
    const float mean = sum64(s) * inv_n;
#pragma unroll
    for (int k = 0; k < R; ++k)
    {
        const float c0 = v[k][0] - mean, c1 = v[k][1] - mean, c2 = v[k][2] - mean, c3 = v[k][3] - mean;
        t[k] = 4 * (lane + kWave * k) < n ? (c0 * c0 + c1 * c1) + (c2 * c2 + c3 * c3) : 0.f;
    }
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < R; k += 2)
        q += k + 1 < R ? t[k] + t[k + 1] : t[k];
    const float scale = rsqrtf(sum64(q) * inv_n + eps);
    STEP_MARK(mark);
    if (own < n)
    {
        float4v y;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            y[c] = __builtin_fmaf((x[c] - mean) * scale, p.g[c], p.b[c]);
        // (own is a multiple of 4: its run sits inside one block of eight.)
        *reinterpret_cast<float4v*>(&out[XB == 8 ? own : (own >> 3) * XB + (own & 7)]) = y;
    }
}

// inv_n = 1 / n (the row means are the sums times inv_n); the rows of tokens
// [0, count) of a T-token launch, one barrier for all of them.
template <int T = 1>
__device__ __forceinline__ void layer_norm(const NormParams& p, int n, float inv_n, float eps, Shared& sh,
                                           int mark = -1, int count = 1)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int own = 4 * (lane + kWave * (int) (threadIdx.x / kWave)); // the run this wave writes
    // Only the waves that write a run compute the statistics; the others go
    // straight to the barrier and leave their SIMDs' issue slots to them.
    if (own - 4 * lane < n)
    {
        for (int k = 0; k < (T == 1 ? 1 : count); ++k)
        {
            const float* raw = sh.raw + k * kRawStride;
            float* out = sh.x + x_at<T>(k, 0);
            switch ((n + 4 * kWave - 1) / (4 * kWave))
            {
                case 1:
                case 2: norm_row<2, kXBlock<T>>(p, n, inv_n, eps, raw, out, lane, own, mark, sh); break;
                case 3: norm_row<3, kXBlock<T>>(p, n, inv_n, eps, raw, out, lane, own, mark, sh); break;
                case 4: norm_row<4, kXBlock<T>>(p, n, inv_n, eps, raw, out, lane, own, mark, sh); break;
                default: norm_row<kNormRuns, kXBlock<T>>(p, n, inv_n, eps, raw, out, lane, own, mark, sh); break;
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// A LayerNorm folded into the projection that consumes it. With
// LN(x)_i = (x_i - mean) rstd gamma_i + beta_i, row r of that projection is
//   (W LN(x))_r + b_r = rstd (sum_i W_ri gamma_i (x_i - K) - (mean - K) g_r) + b'_r
// for any shift K, with g_r = sum_i W_ri gamma_i and b'_r = b_r + sum_i W_ri
// beta_i computed once per weight set (fold_terms_kernel, fused_step.hip). So
// the polling threads write gamma_i (x_i - K) into the dot products' input as
// the words arrive, keep x_i for the residual, and sum their slots' (x_i - K)
// and (x_i - K)^2 in slot order; one reduction of the two sums gives
// mean = K + E[x - K] and var = E[(x - K)^2] - E[x - K]^2, and nothing
// normalises the row before the dot products start. K is the workgroup's
// previous LayerNorm mean (zero before the first), so (mean - K) stays small
// next to the row's spread: neither the variance nor the correction
// (mean - K) g_r loses precision to cancellation while the residual stream's
// mean moves little from one sublayer to the next.
// ---------------------------------------------------------------------------
static_assert(kFoldChunks * kPollBlocked * kPollThreads >= 2 * 768, "two chunks hold d 768 at any row-group count");
constexpr int kFoldSlots = kPollBlocked * kFoldChunks; // a polling thread's slots of a folded row

struct FoldParams
{
    float gamma[kFoldSlots]; // gamma at this thread's slots (zero where a slot holds nothing)
};

// A folded LayerNorm's statistics (fold_stats): rstd, and the mean less the
// shift K the input was written against.
struct FoldStats
{
    float rstd;
    float dmean;
};

// One thread's sums of (x_i - K) and (x_i - K)^2 over the entries it wrote.
struct FoldSums
{
    float s1;
    float s2;
};

// The slot of a blocked vector that polling thread t reads as its k-th
// (chunk k / kPollBlocked, the same order gather_blocked polls in).
__device__ __forceinline__ int fold_slot(int t, int k)
{
    return (k / kPollBlocked) * (kPollBlocked * kPollThreads) + t + (k % kPollBlocked) * kPollThreads;
}

// Loads gamma at this thread's slots of a `rows`-long blocked vector (2^log2
// words per producer, `stride` producers). Every load is issued on every path,
// at a clamped index; wave 0, which does not poll, holds zeros.
__device__ __forceinline__ void load_fold(FoldParams& fp, const float* gamma, int rows, int log2_block, int stride)
{
    const int t = (int) threadIdx.x - kWave;
    const int slots = stride << log2_block;
    const int mask = (1 << log2_block) - 1;
#pragma unroll
    for (int k = 0; k < kFoldSlots; ++k)
    {
        const int slot = fold_slot(t, k);
        const bool valid = t >= 0 && slot < slots && (slot & mask) * stride + (slot >> log2_block) < rows;
        const float g = global(gamma)[valid ? (slot & mask) * stride + (slot >> log2_block) : 0];
        fp.gamma[k] = valid ? g : 0.f;
    }
}

// Each wave's totals of the threads' sums into sh.fold (every lane of the
// wave active), per token; read after the next barrier.
template <int T>
__device__ __forceinline__ void fold_reduce(const FoldSums (&sums)[T], Shared& sh)
{
#pragma unroll
    for (int k = 0; k < T; ++k)
    {
        const float s1 = sum64(sums[k].s1);
        const float s2 = sum64(sums[k].s2);
        if ((threadIdx.x & (kWave - 1)) == 0)
        {
            sh.fold[threadIdx.x / kWave][k][0] = s1;
            sh.fold[threadIdx.x / kWave][k][1] = s2;
        }
    }
}

// gather_blocked for a LayerNorm's input, the whole vector in chunks of
// kPollBlocked * 448 slots: sh.raw[i] = x_i, sh.x[i] = gamma_i (x_i - shift),
// and each wave's sums of (x_i - shift) and (x_i - shift)^2 over its slots (in
// slot order, then a fixed tree) in sh.fold. With T tokens the first `count`
// tokens' vectors (token_words apart) are polled in the same rounds, each
// against its own shift, into its own rows. Returns false, uniformly, when the
// watchdog tripped.
template <int T>
__device__ __forceinline__ bool gather_fold(const uint64_t* base, int token_words, int count, int rows,
                                            int log2_block, int stride, const FoldParams& fp, const float (&shift)[T],
                                            uint32_t epoch, int* status, Shared& sh)
{
    const int slots = stride << log2_block;
    const int mask = (1 << log2_block) - 1;
    FoldSums sums[T];
#pragma unroll
    for (int k = 0; k < T; ++k)
        sums[k] = {0.f, 0.f};
    bool failed = false;
    if (threadIdx.x < kWave)
        __builtin_amdgcn_s_waitcnt(0); // wave 0 stored the last phase's outputs: it only waits for them
    else
    {
        int t = threadIdx.x - kWave;
        // With several tokens the slots' offsets and LDS addresses are
        // recomputed at each call (a few VALU operations) rather than held
        // across the layer loop, where they would not fit in registers.
        if constexpr (T > 1)
            asm volatile("" : "+v"(t));
#pragma unroll
        for (int c = 0; c < kFoldChunks; ++c)
        {
            if (c * kPollBlocked * kPollThreads >= slots || failed) // uniform over the workgroup but for failed
                break;
            uint32_t pending = 0;
            int index[kPollBlocked];
#pragma unroll
            for (int k = 0; k < kPollBlocked; ++k)
            {
                const int slot = fold_slot(t, c * kPollBlocked + k);
                index[k] = (slot & mask) * stride + (slot >> log2_block);
                if (slot < slots && index[k] < rows)
#pragma unroll
                    for (int tok = 0; tok < T; ++tok)
                        if (T == 1 || tok < count)
                            pending |= 1u << (tok * kPollBlocked + k);
            }
            const uint32_t valid = pending;
            float got[T * kPollBlocked] = {};
            if (!poll_words<T * kPollBlocked, false>(
                    base,
                    [&](int w) {
                        const int slot = fold_slot(t, c * kPollBlocked + w % kPollBlocked);
                        return (w / kPollBlocked) * token_words + (slot < slots ? slot : 0);
                    },
                    pending, epoch, status, [&](int w, float v) { got[w] = v; }))
            {
                failed = true;
                break;
            }
            // In slot order: the stores into the row and the two sums.
#pragma unroll
            for (int tok = 0; tok < T; ++tok)
#pragma unroll
                for (int k = 0; k < kPollBlocked; ++k)
                    if (valid & (1u << (tok * kPollBlocked + k)))
                    {
                        const float value = got[tok * kPollBlocked + k];
                        const float dx = value - shift[tok];
                        sh.raw[tok * kRawStride + index[k]] = value;
                        sh.x[x_at<T>(tok, index[k])] = fp.gamma[c * kPollBlocked + k] * dx;
                        sums[tok].s1 += dx;
                        sums[tok].s2 = __builtin_fmaf(dx, dx, sums[tok].s2);
                    }
        }
    }
    fold_reduce<T>(sums, sh);
    if (failed)
        sh.abort = 1;
    __syncthreads();
    return sh.abort == 0;
}

// The statistics from the waves' sums (in wave order): rstd, and the mean
// less the shift, of token k. Every thread computes the same values.
__device__ __forceinline__ FoldStats fold_stats(const Shared& sh, int k, float inv_n, float eps)
{
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
    {
        s1 += sh.fold[w][k][0];
        s2 += sh.fold[w][k][1];
    }
    FoldStats fs;
    fs.dmean = s1 * inv_n;
    fs.rstd = rsqrtf(fmaxf(s2 * inv_n - fs.dmean * fs.dmean, 0.f) + eps);
    return fs;
}

// ---------------------------------------------------------------------------
// Projection rows. A row is cut into `slices` (a power of two) equal runs of
// 16-byte chunks (8 fp16/bf16 or 4 fp32 weights); one slice is walked by a
// row group of 32 lanes, lane l taking chunks l, l+32, l+64 of the run in
// ascending order, and the 32 partials are summed in a fixed order. The slices
// of a row are then added in slice order. Row r of a phase belongs to
// workgroup r % stride; a workgroup's (row, slice) tasks go to its 16 row
// groups in order, with the slice count chosen so every row group has work.
// Loads are issued unconditionally (lanes without a chunk re-read their run's
// first chunk; row groups without a task read chunk 0 of row 0) so the number
// of loads in flight is fixed and the compiler's waits stay exact.
// ---------------------------------------------------------------------------
template <int WT>
struct Storage
{
    static constexpr int kPerChunk = WT == kF32 ? 4 : 8;
    static constexpr int kBytes = WT == kF32 ? 4 : 2;
};

struct RowLoad
{
    uint4 w[kChunks];
};

// The split of one projection phase for this workgroup (identical for every
// layer, so computed once per launch).
struct PhaseShape
{
    int rows;
    int row_bytes;
    int chunks;        // 16-byte chunks per row
    int slice_log2;    // slices = 1 << slice_log2
    int slice_chunks;  // chunks per slice (<= kRowLanes * kChunks)
    int local_rows;    // rows this workgroup owns
    int rows_per_pass; // kRowGroups >> slice_log2
    int passes;
    int block;         // blocked ownership: workgroup w owns rows [w * block, w * block + block); 0: strided
};

// Strided ownership (row r belongs to workgroup r % stride) spreads the rows a
// consumer of the whole vector needs evenly; blocked ownership gives a head's
// rows to a few consecutive workgroups, so a consumer of one head's rows
// polls a few producer blocks instead of one line per row.
template <int WT>
__device__ __forceinline__ PhaseShape phase_shape(int rows, int inner, int group, int stride, bool blocked = false)
{
    PhaseShape ps;
    ps.rows = rows;
    ps.row_bytes = inner * Storage<WT>::kBytes;
    ps.chunks = inner / Storage<WT>::kPerChunk;
    const int most_rows = (rows + stride - 1) / stride;
    int log2 = 0;
    while (log2 < 4 && ((kRowLanes * kChunks << log2) < ps.chunks || (2 << log2) * most_rows <= kRowGroups))
        ++log2;
    ps.slice_log2 = log2;
    ps.slice_chunks = (ps.chunks + (1 << log2) - 1) >> log2;
    ps.block = blocked ? most_rows : 0;
    ps.local_rows = blocked ? max(0, min(most_rows, rows - group * most_rows))
                            : (group < rows ? (rows - group + stride - 1) / stride : 0);
    ps.rows_per_pass = kRowGroups >> log2;
    ps.passes = (ps.local_rows + ps.rows_per_pass - 1) / ps.rows_per_pass;
    return ps;
}

// The row of this workgroup's local row `local`.
__device__ __forceinline__ int phase_row(const PhaseShape& ps, int group, int stride, int local)
{
    return ps.block ? group * ps.block + local : group + stride * local;
}

// This row group's (row, first chunk, end chunk) in `pass`; false when it has
// no task (then the dummy row 0, chunks [0, 0)).
__device__ __forceinline__ bool phase_task(const PhaseShape& ps, int group, int stride, int pass, int& row,
                                           int& first, int& last, int tid = threadIdx.x)
{
    const int task = pass * kRowGroups + tid / kRowLanes;
    if (task >= (ps.local_rows << ps.slice_log2))
    {
        row = 0;
        first = 0;
        last = 0;
        return false;
    }
    row = phase_row(ps, group, stride, task >> ps.slice_log2);
    first = (task & ((1 << ps.slice_log2) - 1)) * ps.slice_chunks;
    last = min(first + ps.slice_chunks, ps.chunks);
    return true;
}

// Loads chunks [first, last) of `row` (lane l taking first + l + 32 i); lanes
// past `last` load the run's first chunk again. The matrix base is uniform
// and every byte offset fits 32 bits (a matrix is far below 4 GiB), so each
// load takes a scalar base and one 32-bit offset register.
__device__ __forceinline__ void load_run(RowLoad& r, const void* weight, int row, int row_bytes, int first, int last,
                                         int tid = threadIdx.x)
{
    const int lane = tid & (kRowLanes - 1);
    const char* base = uniform(static_cast<const char*>(weight));
    const uint32_t row_offset = (uint32_t) row * (uint32_t) row_bytes;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = first + lane + kRowLanes * i;
        r.w[i] = load_global16(base + (row_offset + (uint32_t) (c < last ? c : first) * 16u));
    }
}

// A chunk's weights as floats (4 for fp32 storage, 8 for fp16/bf16).
template <int WT>
struct ChunkWeights
{
    float w[Storage<WT>::kPerChunk];
};

template <int WT>
__device__ __forceinline__ ChunkWeights<WT> chunk_weights(const uint4& u)
{
    ChunkWeights<WT> c;
    if constexpr (WT == kF32)
    {
        c.w[0] = __uint_as_float(u.x);
        c.w[1] = __uint_as_float(u.y);
        c.w[2] = __uint_as_float(u.z);
        c.w[3] = __uint_as_float(u.w);
    }
    else
    {
        const uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            if constexpr (WT == kF16)
            {
                const _Float16* h = reinterpret_cast<const _Float16*>(&v[i]);
                c.w[2 * i] = (float) h[0];
                c.w[2 * i + 1] = (float) h[1];
            }
            else
            {
                c.w[2 * i] = __uint_as_float(v[i] << 16);
                c.w[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
            }
        }
    }
    return c;
}

// The chunk's dot product with x (the same order for every token).
template <int WT>
__device__ __forceinline__ float chunk_dot(const ChunkWeights<WT>& c, const float* x)
{
    float acc = 0.f;
    // Fused multiply-adds written out, so every kernel that inlines this
    // rounds alike.
    if constexpr (WT == kF32)
    {
        const float4v xv = *reinterpret_cast<const float4v*>(x);
        acc = __builtin_fmaf(xv[0], c.w[0], acc);
        acc = __builtin_fmaf(xv[1], c.w[1], acc);
        acc = __builtin_fmaf(xv[2], c.w[2], acc);
        acc = __builtin_fmaf(xv[3], c.w[3], acc);
    }
    else
    {
        const float4v xa = *reinterpret_cast<const float4v*>(x);
        const float4v xb = *reinterpret_cast<const float4v*>(x + 4);
        // Two chains of four (even and odd weights), added at the end.
        float odd = 0.f;
        acc = __builtin_fmaf(xa[0], c.w[0], acc);
        odd = __builtin_fmaf(xa[1], c.w[1], odd);
        acc = __builtin_fmaf(xa[2], c.w[2], acc);
        odd = __builtin_fmaf(xa[3], c.w[3], odd);
        acc = __builtin_fmaf(xb[0], c.w[4], acc);
        odd = __builtin_fmaf(xb[1], c.w[5], odd);
        acc = __builtin_fmaf(xb[2], c.w[6], acc);
        odd = __builtin_fmaf(xb[3], c.w[7], odd);
        acc += odd;
    }
    return acc;
}

template <int WT>
__device__ __forceinline__ float chunk_dot(const uint4& u, const float* x)
{
    return chunk_dot<WT>(chunk_weights<WT>(u), x);
}

// The row slice's dot products with T tokens' inputs (x + x_at<T>(k, .)):
// each chunk is unpacked once and used for every token.
template <int WT, int T>
__device__ __forceinline__ void run_dot(const RowLoad& r, const float* x, int first, int last, int lane,
                                        float (&acc)[T])
{
#pragma unroll
    for (int k = 0; k < T; ++k)
        acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = first + lane + kRowLanes * i;
        if (c < last)
        {
            const ChunkWeights<WT> w = chunk_weights<WT>(r.w[i]);
#pragma unroll
            for (int k = 0; k < T; ++k)
                acc[k] += chunk_dot<WT>(w, x + x_at<T>(k, c * Storage<WT>::kPerChunk));
        }
    }
}

struct Prefetch
{
    RowLoad r;
    float bias; // the bias of the row this thread finishes in pass 0
    float gain; // a folded LayerNorm's sum_i W_ri gamma_i of that row (FOLD phases)
};

// Issues this row group's pass-0 weights and, for the finishing threads, the
// bias of their pass-0 row (and with FOLD its gain).
// A finishing thread's local row: thread t finishes row t % rows_per_pass of
// its pass for token t / rows_per_pass (rows_per_pass is a power of two).
template <int T>
__device__ __forceinline__ int finisher_local(const PhaseShape& ps, int tid = threadIdx.x)
{
    return T == 1 ? tid : tid & (ps.rows_per_pass - 1);
}

template <bool FOLD, int T = 1>
__device__ __forceinline__ void prefetch(Prefetch& p, const void* weight, const float* bias, const float* gain,
                                         const PhaseShape& ps, int group, int stride)
{
    // With several tokens the task's offsets are recomputed at each phase
    // (from an opaque copy of the thread index) rather than held across the
    // layer loop, where registers are short.
    int tid = threadIdx.x;
    if constexpr (T > 1)
        asm volatile("" : "+v"(tid));
    int row, first, last;
    phase_task(ps, group, stride, 0, row, first, last, tid);
    load_run(p.r, weight, row, ps.row_bytes, first, last, tid);
    const int finisher_row = min(phase_row(ps, group, stride, finisher_local<T>(ps, tid)), ps.rows - 1);
    // The load is issued whether or not the phase has a bias (a phase without
    // one reads a weight word and drops it): the compiler counts outstanding
    // loads per program point, and a load skipped on some path makes every
    // later wait for an older load count one load too few, so it would also
    // wait for the newest one — the next phase's weights.
    const float* source = bias != nullptr ? bias : static_cast<const float*>(weight);
    const float b = global(source)[finisher_row];
    p.bias = bias != nullptr ? b : 0.f;
    if constexpr (FOLD)
        p.gain = global(gain)[finisher_row];
}

// The slices of finisher t's row (slots [t << log2, (t + 1) << log2) of
// sh.part), read in one or a few vector reads and added pairwise.
__device__ __forceinline__ float slice_total(const Shared& sh, int token, int t, int log2)
{
    const float* part = sh.part + token * kRowGroups;
    const float4v* run = reinterpret_cast<const float4v*>(part);
    switch (log2)
    {
        case 0: return part[t];
        case 1:
        {
            const float2 v = reinterpret_cast<const float2*>(part)[t];
            return v.x + v.y;
        }
        case 2:
        {
            const float4v v = run[t];
            return (v[0] + v[1]) + (v[2] + v[3]);
        }
        case 3:
        {
            const float4v u = run[2 * t], v = run[2 * t + 1];
            return ((u[0] + u[1]) + (u[2] + u[3])) + ((v[0] + v[1]) + (v[2] + v[3]));
        }
        default:
        {
            const float4v u = run[0], v = run[1], w = run[2], x = run[3];
            return (((u[0] + u[1]) + (u[2] + u[3])) + ((v[0] + v[1]) + (v[2] + v[3])))
                   + (((w[0] + w[1]) + (w[2] + w[3])) + ((x[0] + x[1]) + (x[2] + x[3])));
        }
    }
}
static_assert(kRowGroups == 16, "slice_total covers up to 16 slices");

// Sums a pass's partials, then the finishing threads add the slices of their
// row, turn the dot product into the row's value (value_of: the bias, or a
// folded LayerNorm's correction and bias) and hand it to epi; two barriers
// bracket the shared partial slots. With T tokens thread t finishes token
// t / rows_per_pass (the first `count` tokens only).
template <int T, class Epilogue, class Value>
__device__ __forceinline__ void finish_pass(const float (&acc)[T], bool has_task, int pass, const PhaseShape& ps,
                                            int group, int stride, int count, Shared& sh, Epilogue& epi,
                                            Value value_of)
{
#pragma unroll
    for (int k = 0; k < T; ++k)
    {
        const float total = sum32(acc[k]);
        if (has_task && (threadIdx.x & (kRowLanes - 1)) == 0)
            sh.part[k * kRowGroups + threadIdx.x / kRowLanes] = total;
    }
    __syncthreads();
    int tid = threadIdx.x;
    if constexpr (T > 1)
        asm volatile("" : "+v"(tid)); // recomputed here, not held across the layer loop
    const int lr = finisher_local<T>(ps, tid);
    const int token = T == 1 ? 0 : tid / ps.rows_per_pass;
    const int local = pass * ps.rows_per_pass + lr;
    if ((T == 1 ? tid < ps.rows_per_pass : token < count) && local < ps.local_rows)
    {
        const float v = slice_total(sh, token, lr, ps.slice_log2);
        const int r = phase_row(ps, group, stride, local);
        epi(r, local, token, value_of(token, r, v));
    }
    // Also keeps the other waves from issuing loads (polls, prefetches)
    // ahead of the finishers' stores.
    __syncthreads();
}

// Runs every task of the phase against sh.x. epi(row, local row, token,
// value) receives the dot product plus bias, on thread (local row) %
// rows_per_pass (+ token * rows_per_pass; all in wave 0); with FOLD, sh.x
// holds gamma (x - K) of a LayerNorm's input and the value is
// rstd (dot - (mean - K) gain) + bias, where bias and gain are the row's
// folded terms. Pass 0 is straight-line code whose weights, bias and gain were
// loaded a phase earlier; further passes, which only long rows or narrow grids
// need, load on the spot. after() issues the loads of a later phase (its
// prefetch): every thread calls it once, after pass 0's stores, so they are
// not held up behind the issue. With T tokens every weight chunk is used for
// the first `count` tokens' inputs.
template <int WT, bool FOLD, int T = 1, class Epilogue, class After>
__device__ __forceinline__ void run_phase(const Prefetch& p, const void* weight, const float* bias, const float* gain,
                                          const FoldStats (&fs)[T], const PhaseShape& ps, int group, int stride,
                                          int count, Shared& sh, Epilogue epi, After after, int mark = -1)
{
    const int lane = threadIdx.x & (kRowLanes - 1);
    // The statistics of the token this thread finishes (thread t finishes
    // token t / rows_per_pass), picked before the dot products, off the
    // chain that follows them. By selects on values: an indexed register
    // array would be placed in memory (the empty asm keeps the compiler from
    // turning the selects back into an indexed load).
    float rstd = fs[0].rstd, dmean = fs[0].dmean;
    if constexpr (FOLD && T > 1)
    {
        const int mine = (int) threadIdx.x / ps.rows_per_pass;
#pragma unroll
        for (int i = 1; i < T; ++i)
        {
            float r = fs[i].rstd, m = fs[i].dmean;
            asm volatile("" : "+v"(r), "+v"(m));
            rstd = mine == i ? r : rstd;
            dmean = mine == i ? m : dmean;
        }
    }
    int row, first, last;
    const bool has_task = phase_task(ps, group, stride, 0, row, first, last);
    float acc[T];
    run_dot<WT, T>(p.r, sh.x, first, last, lane, acc);
    const float bias0 = p.bias;
    const float gain0 = FOLD ? p.gain : 0.f;
    // k is always the finishing thread's own token.
    auto value = [&](int, float v, float b, float g) {
        return FOLD ? __builtin_fmaf(rstd, __builtin_fmaf(-dmean, g, v), b) : v + b;
    };
    STEP_MARK(mark);
    if (ps.passes > 0)
        finish_pass<T>(acc, has_task, 0, ps, group, stride, count, sh, epi,
                       [&](int k, int, float v) { return value(k, v, bias0, gain0); });
    STEP_MARK(mark < 0 ? -1 : mark + 1);
    after();
    for (int pass = 1; pass < ps.passes; ++pass)
    {
        const bool task = phase_task(ps, group, stride, pass, row, first, last);
        RowLoad r;
        load_run(r, weight, row, ps.row_bytes, first, last);
        run_dot<WT, T>(r, sh.x, first, last, lane, acc);
        finish_pass<T>(acc, task, pass, ps, group, stride, count, sh, epi, [&](int k, int rr, float v) {
            return value(k, v, bias != nullptr ? global(bias)[rr] : 0.f, FOLD ? global(gain)[rr] : 0.f);
        });
    }
}

// ---------------------------------------------------------------------------
// Single-query attention over keys held in registers: thread t holds channels
// 4*(t%16).. of key slot t/16 for keys slot + 32*p. Scores (scale * q.k),
// their maximum, exp(s - max), the sum and the unnormalised value row — the
// chunk form of Kernels/SingleQueryAttention.h:27-37. Scores are kept in
// base-2 units (scale * log2(e) * q.k), so exp(s - max) is one exp2; the
// maxima written to the exchange, and the combines, use the same units.
// ---------------------------------------------------------------------------
constexpr float kLog2e = 1.44269504088896340736f;

// 2^x for x <= 0 (a softmax weight): the hardware exp2 alone. Results below
// 2^-126, which the library's exp2f would keep as denormals, come out as 0 —
// weights no sum can notice — and the library's range fix-up (a compare, a
// scalar select and an ldexp per call) stays off the dependency chain.
__device__ __forceinline__ float exp2_weight(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

// q . k over a lane's four channels, and acc += e * v, with the fused
// multiply-adds written out: the single- and multi-token kernels then round
// alike (the compiler's own contraction could pair the products differently
// in each).
__device__ __forceinline__ float dot4(const float4v& q, const float4v& k)
{
    return __builtin_fmaf(q[0], k[0], q[1] * k[1]) + __builtin_fmaf(q[2], k[2], q[3] * k[3]);
}

__device__ __forceinline__ void add_scaled(float4v& acc, float e, const float4v& v)
{
    acc[0] = __builtin_fmaf(e, v[0], acc[0]);
    acc[1] = __builtin_fmaf(e, v[1], acc[1]);
    acc[2] = __builtin_fmaf(e, v[2], acc[2]);
    acc[3] = __builtin_fmaf(e, v[3], acc[3]);
}

template <int NP>
struct KeyRows
{
    float4v k[NP];
    float4v v[NP];
};

// Keys [first, first + count) of one head; slots past count re-read key `first`.
template <int NP>
__device__ __forceinline__ void load_keys(KeyRows<NP>& kr, const float* keys, const float* values, int first,
                                          int count, int width, int column, int head_width)
{
    const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
    const int channel = 4 * kl < head_width ? 4 * kl : 0;
    // Uniform bases and 32-bit element offsets (a cache is far below 4 GiB).
    const float* kb = uniform(keys);
    const float* vb = uniform(values);
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        const int key = ks + kKeySlots * p;
        const uint32_t at = (uint32_t) (first + (key < count ? key : 0)) * (uint32_t) width + (uint32_t) (column + channel);
        kr.k[p] = *global(reinterpret_cast<const float4v*>(kb + at));
        kr.v[p] = *global(reinterpret_cast<const float4v*>(vb + at));
    }
}

// Writes (max, sum, row[head_width]) of `count` keys into out (exchange
// words). With `normalized` the row is written already divided by the sum —
// the combine of a single partial, so a consumer of the only partial of a
// head can take the row as it is. Each wave takes the softmax of its own key
// slots against its own maximum; after one barrier the waves' rows are
// rescaled to the largest maximum and added in wave order (the combine of
// Kernels/SingleQueryAttention.h:312-373 over the eight waves). The caller
// writes sh.red and sh.scratch again only after a barrier of its own.
template <int NP>
__device__ __forceinline__ void attend(const KeyRows<NP>& kr, int count, int head_width, float scale2, uint64_t* out,
                                       uint32_t epoch, Shared& sh, bool normalized = false, int mark = -1,
                                       const float* query = nullptr)
{
    // No contraction beyond the fused multiply-adds written out: the single-
    // and multi-token kernels must round every token alike.
#pragma clang fp contract(off)
    const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const bool live = 4 * kl < head_width;
    float4v qv = {0.f, 0.f, 0.f, 0.f};
    if (live)
        qv = *reinterpret_cast<const float4v*>((query != nullptr ? query : sh.q) + 4 * kl);
    float s[NP];
    float local_max = -INFINITY;
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        s[p] = -INFINITY;
        if (kKeySlots * p < count) // uniform: passes past the keys are skipped
        {
            const float part = live ? dot4(qv, kr.k[p]) : 0.f;
            s[p] = scale2 * sum16(part);
            if (ks + kKeySlots * p < count)
                local_max = fmaxf(local_max, s[p]);
        }
    }
    const float m = max64(local_max); // this wave's keys; -inf when it holds none
    STEP_MARK(mark);
    float local_sum = 0.f;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        if (kKeySlots * p < count && ks + kKeySlots * p < count)
        {
            const float e = exp2_weight(s[p] - m);
            if (kl == 0)
                local_sum += e;
            add_scaled(acc, e, kr.v[p]);
        }
    }
    // Fold the wave's four key slots (lanes 16 apart) with the neighbouring
    // row, then the other half of the wave: lanes 0-15 then hold the wave's
    // row, and lane 0 its sum (kept by the kl == 0 lanes).
#pragma unroll
    for (int i = 0; i < 4; ++i)
        acc[i] = add32(add16(acc[i]));
    local_sum = add32(add16(local_sum));
    STEP_MARK(mark < 0 ? -1 : mark + 1);
    if (lane < kKeyLanes && live)
        *reinterpret_cast<float4v*>(&sh.red[wave][4 * kl]) = acc;
    if (lane == 0)
    {
        sh.scratch[0][0][wave] = m;
        sh.scratch[0][1][wave] = local_sum;
    }
    __syncthreads();
    STEP_MARK(mark < 0 ? -1 : mark + 2);
    if ((int) threadIdx.x < head_width)
    {
        float mw[kWaves], lw[kWaves], rw[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
            mw[w] = sh.scratch[0][0][w];
            lw[w] = sh.scratch[0][1][w];
            rw[w] = sh.red[w][threadIdx.x];
        }
        static_assert(kWaves == 8, "three-level trees over the waves");
        const float top = fmaxf(fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3])),
                                fmaxf(fmaxf(mw[4], mw[5]), fmaxf(mw[6], mw[7])));
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
            const float f = lw[w] == 0.f ? 0.f : exp2_weight(mw[w] - top); // a wave without keys adds nothing
            lw[w] *= f;
            rw[w] *= f;
        }
        const float l = ((lw[0] + lw[1]) + (lw[2] + lw[3])) + ((lw[4] + lw[5]) + (lw[6] + lw[7]));
        const float row = ((rw[0] + rw[1]) + (rw[2] + rw[3])) + ((rw[4] + rw[5]) + (rw[6] + rw[7]));
        put(out + 2 + threadIdx.x, normalized ? row * __builtin_amdgcn_rcpf(l) : row, epoch);
        if (threadIdx.x == 0)
        {
            put(out, count > 0 ? top : -INFINITY, epoch);
            put(out + 1, l, epoch);
        }
    }
}

// Token k's per-wave rows of an attention chunk.
__device__ __forceinline__ float (*red_of(Shared& sh, int k))[kMaxHeadWidth]
{
    return k == 0 ? sh.red : sh.red_more[k - 1];
}

// attend() for the queries of Q tokens over the same keys (a cross-attention
// chunk of a multi-token launch): token k's query at query + k * kQStride,
// its (max, sum, row) at out + k * out_stride, for the first `tokens` tokens.
// Every key register is used for all Q queries, and the Q chains of
// reductions run side by side; each token's arithmetic is attend()'s.
template <int NP, int Q>
__device__ __forceinline__ void attend_tokens(const KeyRows<NP>& kr, int count, int tokens, int head_width,
                                              float scale2, uint64_t* out, int out_stride, uint32_t epoch, Shared& sh,
                                              const float* query)
{
    // No contraction beyond the fused multiply-adds written out: the single-
    // and multi-token kernels must round every token alike.
#pragma clang fp contract(off)
    const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const bool live = 4 * kl < head_width;
    float4v qv[Q];
#pragma unroll
    for (int k = 0; k < Q; ++k)
    {
        qv[k] = float4v {0.f, 0.f, 0.f, 0.f};
        if (live)
            qv[k] = *reinterpret_cast<const float4v*>(query + k * kQStride + 4 * kl);
    }
    float s[NP][Q];
    float local_max[Q];
#pragma unroll
    for (int k = 0; k < Q; ++k)
        local_max[k] = -INFINITY;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int k = 0; k < Q; ++k)
        {
            s[p][k] = -INFINITY;
            if (kKeySlots * p < count) // uniform: passes past the keys are skipped
            {
                const float part = live ? dot4(qv[k], kr.k[p]) : 0.f;
                s[p][k] = scale2 * sum16(part);
                if (ks + kKeySlots * p < count)
                    local_max[k] = fmaxf(local_max[k], s[p][k]);
            }
        }
    float m[Q], local_sum[Q];
    float4v acc[Q];
#pragma unroll
    for (int k = 0; k < Q; ++k)
    {
        m[k] = max64(local_max[k]);
        local_sum[k] = 0.f;
        acc[k] = float4v {0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
        if (kKeySlots * p < count && ks + kKeySlots * p < count)
#pragma unroll
            for (int k = 0; k < Q; ++k)
            {
                const float e = exp2_weight(s[p][k] - m[k]);
                if (kl == 0)
                    local_sum[k] += e;
                add_scaled(acc[k], e, kr.v[p]);
            }
#pragma unroll
    for (int k = 0; k < Q; ++k)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc[k][i] = add32(add16(acc[k][i]));
        local_sum[k] = add32(add16(local_sum[k]));
        if (lane < kKeyLanes && live)
            *reinterpret_cast<float4v*>(&red_of(sh, k)[wave][4 * kl]) = acc[k];
        if (lane == 0)
        {
            sh.scratch[k][0][wave] = m[k];
            sh.scratch[k][1][wave] = local_sum[k];
        }
    }
    __syncthreads();
    // Thread k * head_width + c folds channel c of token k (head_width is a
    // power of two here).
    const int k = (int) threadIdx.x / head_width, c = (int) threadIdx.x & (head_width - 1);
    if (k < tokens)
    {
        float mw[kWaves], lw[kWaves], rw[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
            mw[w] = sh.scratch[k][0][w];
            lw[w] = sh.scratch[k][1][w];
            rw[w] = red_of(sh, k)[w][c];
        }
        const float top = fmaxf(fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3])),
                                fmaxf(fmaxf(mw[4], mw[5]), fmaxf(mw[6], mw[7])));
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
            const float f = lw[w] == 0.f ? 0.f : exp2_weight(mw[w] - top); // a wave without keys adds nothing
            lw[w] *= f;
            rw[w] *= f;
        }
        const float l = ((lw[0] + lw[1]) + (lw[2] + lw[3])) + ((lw[4] + lw[5]) + (lw[6] + lw[7]));
        const float row = ((rw[0] + rw[1]) + (rw[2] + rw[3])) + ((rw[4] + rw[5]) + (rw[6] + rw[7]));
        uint64_t* o = out + k * out_stride;
        put(o + 2 + c, row, epoch);
        if (c == 0)
        {
            put(o, count > 0 ? top : -INFINITY, epoch);
            put(o + 1, l, epoch);
        }
    }
}

// Combines `parts` partials (stride apart, as written by attend) into the
// normalised row: rescale each by exp(m_i - max) and divide
// (Kernels/SingleQueryAttention.h:312-373). Empty partials (sum 0) are skipped.
__device__ __forceinline__ float combine(const float* part, int parts, int stride, int c)
{
    float largest = -INFINITY;
    for (int i = 0; i < parts; ++i)
        largest = fmaxf(largest, part[i * stride]);
    float numerator = 0.f, denominator = 0.f;
    for (int i = 0; i < parts; ++i)
    {
        const float* p = part + i * stride;
        if (p[1] == 0.f)
            continue;
        const float factor = exp2_weight(p[0] - largest);
        numerator += factor * p[2 + c];
        denominator += factor * p[1];
    }
    return numerator / denominator;
}

// The same combine for up to 64 partials of one head with the whole
// workgroup: every wave finds the largest maximum, each partial's factor
// exp(m_i - max) (0 for an empty partial) and the denominator itself (no
// barrier); wave w then sums partials w, w + 8, ... of every channel, and the
// eight wave sums are added pairwise. The normalised row goes to out
// (exchange words).
__device__ __forceinline__ void combine_parts(const float* part, int parts, int head_width, uint64_t* out,
                                              uint32_t epoch, Shared& sh)
{
    // No contraction beyond the fused multiply-adds written out: the single-
    // and multi-token kernels must round every token alike.
#pragma clang fp contract(off)
    const int stride = head_width + 2;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const float m = lane < parts ? part[lane * stride] : -INFINITY;
    const float l = lane < parts ? part[lane * stride + 1] : 0.f;
    const float largest = max64(m);
    const float factor = l == 0.f ? 0.f : exp2_weight(m - largest);
    const float denominator = sum64(factor * l);
    if (lane < head_width)
    {
        float acc = 0.f;
        for (int i = wave; i < parts; i += kWaves) // i is uniform over the wave
            acc = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(factor), i)),
                                 part[i * stride + 2 + lane], acc);
        sh.red[wave][lane] = acc;
    }
    __syncthreads();
    if ((int) threadIdx.x < head_width)
    {
        float r[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            r[w] = sh.red[w][threadIdx.x];
        const float numerator = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        put(out + threadIdx.x, numerator * __builtin_amdgcn_rcpf(denominator), epoch);
    }
}

// combine_parts for the first `count` tokens of a T-token launch at once:
// token k's partials at comb + k * n, its row to out + k * out_stride. The
// waves split over the tokens (kWaves / T each); each wave folds the partials
// of the "virtual waves" v = its index within the token + (kWaves / T) j,
// partial i going to virtual wave i % kWaves as in combine_parts, so every
// token's sums run in combine_parts' order.
template <int T>
__device__ __forceinline__ void combine_tokens(const float* comb, int n, int parts, int head_width, uint64_t* out,
                                               int out_stride, int count, uint32_t epoch, Shared& sh)
{
    // No contraction beyond the fused multiply-adds written out: the single-
    // and multi-token kernels must round every token alike.
#pragma clang fp contract(off)
    static_assert(kWaves % T == 0, "whole waves per token");
    constexpr int kPer = kWaves / T;
    const int stride = head_width + 2;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int k = wave / kPer, sub = wave % kPer;
    const bool active = k < count; // a token past the launch's reads nothing
    const float* part = comb + (active ? k : 0) * n;
    const float m = active && lane < parts ? part[lane * stride] : -INFINITY;
    const float l = active && lane < parts ? part[lane * stride + 1] : 0.f;
    const float largest = max64(m);
    const float factor = l == 0.f ? 0.f : exp2_weight(m - largest);
    const float denominator = sum64(factor * l);
    if (active && lane < head_width)
    {
#pragma unroll
        for (int j = 0; j < T; ++j)
        {
            const int v = sub + kPer * j; // kPer * T = kWaves virtual waves per token
            float acc = 0.f;
            for (int i = v; i < parts; i += kWaves) // i is uniform over the wave
                acc = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(factor), i)),
                                 part[i * stride + 2 + lane], acc);
            red_of(sh, k)[v][lane] = acc;
        }
    }
    if (lane == 0 && sub == 0)
        sh.scratch[k][0][0] = denominator;
    __syncthreads();
    const int kk = (int) threadIdx.x / head_width, c = (int) threadIdx.x & (head_width - 1);
    if (kk < count && kk < T)
    {
        float r[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            r[w] = red_of(sh, kk)[w][c];
        const float numerator = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        put(out + kk * out_stride + c, numerator * __builtin_amdgcn_rcpf(sh.scratch[kk][0][0]), epoch);
    }
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi)
{
    if (i == kUnchosen)
        return false;
    if (bi == kUnchosen)
        return true;
    return v > bv || (v == bv && i < bi);
}

// Candidate folds across lanes. better() orders candidates totally (larger
// value, then lower index, an unchosen one last), so which lane of a pair
// holds which candidate does not change the result.
__device__ __forceinline__ void keep_better(float& v, uint32_t& i, float ov, uint32_t oi)
{
    if (better(ov, oi, v, i))
    {
        v = ov;
        i = oi;
    }
}

template <int CTRL>
__device__ __forceinline__ void fold_dpp(float& v, uint32_t& i)
{
    const float ov = dpp<CTRL>(v);
    const uint32_t oi = (uint32_t) __builtin_amdgcn_mov_dpp((int) i, CTRL, 0xF, 0xF, true);
    keep_better(v, i, ov, oi);
}

// Every lane of each 16-lane row ends with the row's best candidate.
__device__ __forceinline__ void fold16(float& v, uint32_t& i)
{
    fold_dpp<kSwapNeighbours>(v, i);
    fold_dpp<kSwapPairs>(v, i);
    fold_dpp<kMirrorHalfRow>(v, i);
    fold_dpp<kMirrorRow>(v, i);
}

// Every lane of the wave ends with the wave's best candidate.
__device__ __forceinline__ void fold64(float& v, uint32_t& i)
{
    fold16(v, i);
    float a, b;
    uint32_t ia, ib;
    rows_pair(v, a, b); // the value and the index pair up the same lanes in the same order
    rows_pair_bits(i, ia, ib);
    v = a;
    i = ia;
    keep_better(v, i, b, ib);
    halves_pair(v, a, b);
    halves_pair_bits(i, ia, ib);
    v = a;
    i = ia;
    keep_better(v, i, b, ib);
}

// ---------------------------------------------------------------------------
// Tied logits. Rows of `lanes` lanes (32 when a row fits 96 chunks, else 64);
// row group g of workgroup w owns rows w + G * (g + groups * j). A ring of
// kRing rows per row group is in flight: finishing row j issues row j + kRing.
// The mask value rides along with each row. Rows past the vocabulary load
// chunk 0 of row 0.
// ---------------------------------------------------------------------------
struct Ring
{
    RowLoad r[kRing];
    float mask[kRing];
};

struct LogitShape
{
    int lanes_log2;
    int groups;    // row groups per workgroup
    int chunks;    // chunks per row
    int row_bytes;
};

__device__ __forceinline__ LogitShape logit_shape(const StepArgs& a)
{
    LogitShape s;
    const int bytes = a.logits_wdtype == kF32 ? 4 : 2;
    s.row_bytes = a.width * bytes;
    s.chunks = s.row_bytes / 16;
    s.lanes_log2 = s.chunks <= kRowLanes * kChunks ? 5 : 6;
    s.groups = kThreads >> s.lanes_log2;
    return s;
}

__device__ __forceinline__ int logit_row(const LogitShape& s, int j)
{
    return blockIdx.x + gridDim.x * ((int) (threadIdx.x >> s.lanes_log2) + s.groups * j);
}

__device__ __forceinline__ void load_logit_row(RowLoad& r, float& mask, const StepArgs& a, const LogitShape& s, int j)
{
    const int row = logit_row(s, j);
    const bool valid = row < a.vocabulary;
    const int lane = threadIdx.x & ((1 << s.lanes_log2) - 1);
    const char* base = uniform(static_cast<const char*>(a.logits_weight));
    const uint32_t row_offset = (uint32_t) (valid ? row : 0) * (uint32_t) s.row_bytes;
    const int last = valid ? s.chunks : 1;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = lane + (i << s.lanes_log2);
        r.w[i] = load_global16(base + (row_offset + (uint32_t) (c < last ? c : 0) * 16u));
    }
    // Issued with or without a mask (then a weight word, dropped), so every
    // path has the same number of loads in flight.
    const float m = *global(a.mask != nullptr ? a.mask + (valid ? row : 0) : static_cast<const float*>(a.logits_weight));
    mask = a.mask != nullptr ? m : 0.f;
}

__device__ __forceinline__ void issue_ring(Ring& ring, const StepArgs& a, const LogitShape& s)
{
#pragma unroll
    for (int k = 0; k < kRing; ++k)
        load_logit_row(ring.r[k], ring.mask[k], a, s, k);
}

// The row's dot products with T tokens' normalised rows (x + x_at<T>(k, .)),
// each chunk unpacked once.
template <int LWT, int T>
__device__ __forceinline__ void logit_dot(const RowLoad& r, const StepArgs& a, const LogitShape& s, int row,
                                          const float* x, float (&v)[T])
{
    const int lanes = 1 << s.lanes_log2;
    const int lane = threadIdx.x & (lanes - 1);
    float acc[T];
#pragma unroll
    for (int k = 0; k < T; ++k)
        acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = lane + i * lanes;
        if (c < s.chunks)
        {
            const ChunkWeights<LWT> w = chunk_weights<LWT>(r.w[i]);
#pragma unroll
            for (int k = 0; k < T; ++k)
                acc[k] += chunk_dot<LWT>(w, x + x_at<T>(k, c * Storage<LWT>::kPerChunk));
        }
    }
    // Rows longer than the ring's share load the rest here.
    for (int c = lane + kChunks * lanes; c < s.chunks; c += lanes)
    {
        const ChunkWeights<LWT> w = chunk_weights<LWT>(*reinterpret_cast<const uint4*>(
            static_cast<const char*>(a.logits_weight) + (size_t) row * s.row_bytes + (size_t) c * 16));
#pragma unroll
        for (int k = 0; k < T; ++k)
            acc[k] += chunk_dot<LWT>(w, x + x_at<T>(k, c * Storage<LWT>::kPerChunk));
    }
#pragma unroll
    for (int k = 0; k < T; ++k)
        v[k] = s.lanes_log2 == 5 ? sum32(acc[k]) : sum64(acc[k]);
}

// The logits of the first `count` tokens; the top-1 under the mask of the
// last of them.
template <int LWT, int T>
__device__ __forceinline__ void logits_loop(Ring& ring, const StepArgs& a, const LogitShape& s, const Shared& sh,
                                            int count, float& best_v, uint32_t& best_i)
{
    const int lane = threadIdx.x & ((1 << s.lanes_log2) - 1);
    for (int j = 0;; j += kRing)
    {
#pragma unroll
        for (int k = 0; k < kRing; ++k)
        {
            const int row = logit_row(s, j + k);
            if (row >= a.vocabulary)
                return;
            float v[T];
            logit_dot<LWT, T>(ring.r[k], a, s, row, sh.x, v);
            const float m = ring.mask[k];
            load_logit_row(ring.r[k], ring.mask[k], a, s, j + k + kRing);
            if (lane == 0)
            {
                float last = v[0];
#pragma unroll
                for (int t = 0; t < T; ++t)
                    if (T == 1 || t < count)
                    {
                        a.logits[(size_t) t * a.vocabulary + row] = v[t];
                        last = v[t];
                    }
                if (m == 0.f && (best_i == kUnchosen || last > best_v))
                {
                    best_v = last;
                    best_i = (uint32_t) row;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// The persistent step.
// ---------------------------------------------------------------------------
// The layer-0 input: the token and position rows (Kernels/Embed.h:9-14); an
// id past the vocabulary poisons the row with NaN (it reads row 0, unused).
// The loads are issued at launch, ahead of the layer table's copy, and the
// two parts are added where the row is written.
constexpr int kEmbedSlots = (kMaxWidth + kThreads - 1) / kThreads;

template <int T>
struct Embedding
{
    float token[T][kEmbedSlots];
    float position[T][kEmbedSlots];
    bool known[T];
};

// Token k (of the first `count`; later slots repeat the last) at position
// position + k.
template <int T>
__device__ __forceinline__ void issue_embedding(Embedding<T>& e, const StepArgs& a)
{
    const int d = a.width;
#pragma unroll
    for (int t = 0; t < T; ++t)
    {
        const int k = T == 1 ? 0 : min(t, a.token_count - 1);
        const uint32_t token = a.tokens[k];
        e.known[t] = token < (uint32_t) a.vocabulary;
        const size_t row = e.known[t] ? (size_t) token * d : 0;
#pragma unroll
        for (int s = 0; s < kEmbedSlots; ++s)
        {
            const int c = min((int) threadIdx.x + kThreads * s, d - 1);
            e.position[t][s] = global(a.position_embedding)[(size_t) (a.position + k) * d + c];
            e.token[t][s] = global(a.token_embedding)[row + c];
        }
    }
}

// The first `count` tokens' n-word vectors (token_words apart from base):
// word j of token k is read at base + k * token_words + offset and written to
// dst[place(k, index)], with map(j, offset, index) as in poll(). The tokens'
// words are polled in order, P * 448 slots a round.
template <int P, class Map, class Place>
__device__ __forceinline__ bool gather_tokens(const uint64_t* base, int token_words, int count, int n, Map map,
                                              float* dst, Place place, uint32_t epoch, int* status, Shared& sh)
{
    const int total = count * n;
    for (int first = 0; first < total; first += P * kPollThreads)
    {
        const bool ok = poll<P>(
            base, min(P * kPollThreads, total - first),
            [&](int i, int& offset, int& index) {
                const int w = first + i;
                const int k = w / n, j = w - k * n;
                int o, x;
                const bool used = map(j, o, x);
                offset = k * token_words + o;
                index = place(k, x);
                return used;
            },
            dst, epoch, status, sh);
        if (!ok)
            return false;
    }
    return true;
}

// Tokens [k0, k0 + TT) (those below `count`) of an n-slot vector each,
// slots [first, first + PT * 448) of it, polled in one round of TT * PT words
// per thread: slot j of a token is word map(j, offset, index) of that token's
// vector (token_words apart from base) and lands in dst[place(token, index)].
template <int PT, int TT, class Map, class Place>
__device__ __forceinline__ bool gather_token_block(const uint64_t* base, int token_words, int k0, int count, int n,
                                                   Map map, float* dst, Place place, uint32_t epoch, int* status,
                                                   Shared& sh, int first = 0)
{
    bool failed = false;
    if (threadIdx.x < kWave)
        __builtin_amdgcn_s_waitcnt(0); // wave 0 stored the last phase's outputs: it only waits for them
    else
    {
        int t = threadIdx.x - kWave;
        asm volatile("" : "+v"(t)); // offsets recomputed per call, not held across the layer loop
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < TT; ++k)
#pragma unroll
            for (int j = 0; j < PT; ++j)
            {
                const int slot = first + t + j * kPollThreads;
                int offset, index;
                if (k0 + k < count && slot < n && map(slot, offset, index))
                    pending |= 1u << (k * PT + j);
            }
        failed = !poll_words<TT * PT, false>(
            base,
            [&](int w) {
                const int slot = first + t + (w % PT) * kPollThreads;
                int offset = 0, index;
                const bool used = slot < n && map(slot, offset, index);
                return (k0 + w / PT) * token_words + (used ? offset : 0);
            },
            pending, epoch, status,
            [&](int w, float v) {
                int offset, index;
                map(first + t + (w % PT) * kPollThreads, offset, index);
                dst[place(k0 + w / PT, index)] = v;
            });
    }
    if (failed)
        sh.abort = 1;
    __syncthreads();
    return sh.abort == 0;
}

template <int WT, int T>
__device__ __forceinline__ bool row_group_layers(const StepArgs& a, Shared& sh, const Embedding<T>& embed)
{
    const int d = a.width, f = a.feed_forward, H = a.heads, hd = d / H;
    const int group = blockIdx.x, stride = a.row_groups;
    const int pos = a.position;
    const int count = T == 1 ? 1 : a.token_count;
    const int tw = a.token_words;
    const uint32_t epoch = a.epoch;
    const PhaseShape qkv_shape = phase_shape<WT>(3 * d, d, group, stride, true); // read per head
    const PhaseShape square_shape = phase_shape<WT>(d, d, group, stride);
    const PhaseShape xq_shape = phase_shape<WT>(d, d, group, stride, true); // read per head
    const PhaseShape fc1_shape = phase_shape<WT>(f, d, group, stride);
    const PhaseShape fc2_shape = phase_shape<WT>(d, f, group, stride);
    // One cross-attention chunk per row group when the split allows it; more
    // tasks than row groups wrap around (and are not prefetched).
    const int tasks = a.cross_splits * H;
    const int task = group;
    const int task_first = (task / H) * a.cross_chunk;
    const int task_count = task < tasks ? min(a.cross_chunk, a.cross_rows - task_first) : 0;

    Prefetch pa, pb;
    FoldParams fold;
    FoldStats fs[T];
    float shift[T]; // per token: the previous LayerNorm's mean (the next one's K)
#pragma unroll
    for (int k = 0; k < T; ++k)
        shift[k] = 0.f;
    KeyRows<kCrossPasses> cross;
    FoldStats none[T];
#pragma unroll
    for (int k = 0; k < T; ++k)
        none[k] = {};
    // After a folded gather every thread reads the statistics (the waves'
    // sums are in sh.fold past its barrier) and moves the shift to this
    // LayerNorm's mean, the next one's K.
    auto statistics = [&] {
#pragma unroll
        for (int k = 0; k < T; ++k)
        {
            fs[k] = fold_stats(sh, k, a.inv_width, a.eps);
            shift[k] += fs[k].dmean;
        }
    };

    {
        // The layer-0 input, folded into LN1 the way gather_fold folds the
        // later layers' (all eight waves hold embedding entries; K = 0).
        const wsp_layer_tensors& L0 = sh.table[0];
        const float* T0 = a.fold_terms;
        prefetch<true, T>(pa, L0.self_qkv_w, T0 + a.terms_qkv_bias, T0 + a.terms_qkv_gain, qkv_shape, group, stride);
        float gamma[kEmbedSlots];
#pragma unroll
        for (int k = 0; k < kEmbedSlots; ++k)
            gamma[k] = global(L0.self_norm_w)[min((int) threadIdx.x + kThreads * k, d - 1)];
        FoldSums sums[T];
#pragma unroll
        for (int t = 0; t < T; ++t)
        {
            sums[t] = {0.f, 0.f};
#pragma unroll
            for (int k = 0; k < kEmbedSlots; ++k)
            {
                const int c = (int) threadIdx.x + kThreads * k;
                if (c < d)
                {
                    const float x = embed.known[t] ? embed.token[t][k] + embed.position[t][k] : __builtin_nanf("");
                    sh.raw[t * kRawStride + c] = x;
                    sh.x[x_at<T>(t, c)] = gamma[k] * x;
                    sums[t].s1 += x;
                    sums[t].s2 = __builtin_fmaf(x, x, sums[t].s2);
                }
            }
        }
        fold_reduce<T>(sums, sh);
        __syncthreads();
    }
    STEP_STAMP(0, 0);

    for (int l = 0; l < a.layer_count; ++l)
    {
        const wsp_layer_tensors& L = sh.table[l];
        const float* TL = a.fold_terms + (size_t) l * a.terms_stride;
        uint64_t* ex = a.exchange + (size_t) l * a.layer_words;
        STEP_LAYER(l);

        // ---- LN1 folded into the fused q/k/v (weights in pa) --------------------
        if (l > 0
            && !gather_fold<T>(a.exchange + (size_t) (l - 1) * a.layer_words + a.off_h4, tw, count, d, a.log2_d,
                               stride, fold, shift, epoch, a.status, sh))
            return false;
        if (l > 0)
            STEP_STAMP(0, l);
        statistics();
        {
            uint64_t* qkv = ex + a.off_qkv;
            run_phase<WT, true, T>(pa, L.self_qkv_w, TL + a.terms_qkv_bias, TL + a.terms_qkv_gain, fs, qkv_shape,
                                   group, stride, count, sh, [&](int r, int j, int k, float v) {
                put(qkv + k * tw + (group << a.log2_qkv) + j, v, epoch);
                // The new key and value rows of token k, at position pos + k.
                const size_t at = (size_t) (pos + k) * d;
                if (r >= 2 * d)
                    global_mut(L.self_values + at)[r - 2 * d] = v;
                else if (r >= d)
                    global_mut(L.self_keys + at)[r - d] = v;
            }, [&] { prefetch<false, T>(pb, L.self_out_w, L.self_out_b, nullptr, square_shape, group, stride); }, 25);
        }
        STEP_STAMP(1, l);

        // This group's cross-attention keys, issued while the self-attention
        // hand-overs are in flight (the workgroup has nothing else to do then)
        // and awaited only when the cross query arrives. Every workgroup issues
        // them (one without a task reads key 0), so the number of loads in
        // flight is the same on every path.
        load_keys<kCrossPasses>(cross, L.cross_keys, L.cross_values, task_count > 0 ? task_first : 0,
                                max(task_count, 1), d, (task % H) * hd, hd);

        // ---- self-attention combine + out-proj + residual (weights in pb) ------
        if (a.self_splits == 1 && (hd & (hd - 1)) == 0)
        {
            // One partial per head, written normalized: its rows are the
            // attention output, gathered straight into sh.x (two poll slots
            // per thread cover 896 words, three the widest row).
            const int shift_hd = 31 - __builtin_clz(hd);
            auto map = [&](int i, int& offset, int& index) {
                offset = (i >> shift_hd) * (hd + 2) + 2 + (i & (hd - 1));
                index = i;
                return true;
            };
            static_assert(3 * kPollThreads >= kMaxWidth, "three slots cover the widest row");
            if constexpr (T == 1)
            {
                if (!(d <= 2 * kPollThreads ? poll<2>(ex + a.off_self, d, map, sh.x, epoch, a.status, sh)
                                            : poll<3>(ex + a.off_self, d, map, sh.x, epoch, a.status, sh)))
                    return false;
            }
            else if (!(d <= 2 * kPollThreads
                           ? gather_token_block<2, T>(ex + a.off_self, tw, 0, count, d, map, sh.x, x_at<T>, epoch,
                                                      a.status, sh)
                           : gather_token_block<3, T>(ex + a.off_self, tw, 0, count, d, map, sh.x, x_at<T>, epoch,
                                                      a.status, sh)))
                return false;
            STEP_STAMP(2, l);
        }
        else
        {
            // (Key splits: the single-token kernel only.)
            if (!gather_any(ex + a.off_self, a.self_splits * H * (hd + 2), sh.comb, epoch, a.status, sh))
                return false;
            STEP_STAMP(2, l);
            for (int c = threadIdx.x; c < d; c += kThreads)
                sh.x[c] = combine(sh.comb + (c / hd) * (hd + 2), a.self_splits, H * (hd + 2), c % hd);
            __syncthreads();
        }
        {
            uint64_t* out = ex + a.off_h2;
            run_phase<WT, false, T>(
                pb, L.self_out_w, L.self_out_b, nullptr, none, square_shape, group, stride, count, sh,
                [&](int r, int j, int k, float v) {
                    put(out + k * tw + (group << a.log2_d) + j, sh.raw[k * kRawStride + r] + v, epoch);
                },
                [&] {
                    prefetch<true, T>(pa, L.cross_q_w, TL + a.terms_xq_bias, TL + a.terms_xq_gain, xq_shape, group,
                                      stride);
                    load_fold(fold, L.cross_norm_w, d, a.log2_d, stride);
                },
                27);
        }
        STEP_STAMP(3, l);

        // ---- LN2 folded into the cross q (weights in pa) --------------------------
        if (!gather_fold<T>(ex + a.off_h2, tw, count, d, a.log2_d, stride, fold, shift, epoch, a.status, sh))
            return false;
        STEP_STAMP(4, l);
        statistics();
        {
            uint64_t* out = ex + a.off_xq;
            run_phase<WT, true, T>(
                pa, L.cross_q_w, TL + a.terms_xq_bias, TL + a.terms_xq_gain, fs, xq_shape, group, stride, count, sh,
                [&](int, int j, int k, float v) { put(out + k * tw + (group << a.log2_d) + j, v, epoch); },
                [&] { prefetch<false, T>(pb, L.cross_out_w, L.cross_out_b, nullptr, square_shape, group, stride); },
                29);
        }
        STEP_STAMP(5, l);

        // ---- cross-attention partials over this group's key chunk(s) ---------------
        for (int t = task; t < tasks; t += stride)
        {
            const int h = t % H, s = t / H;
            const int first = s * a.cross_chunk;
            const int keys = min(a.cross_chunk, a.cross_rows - first);
            if (t != task)
                load_keys<kCrossPasses>(cross, L.cross_keys, L.cross_values, first, keys, d, h * hd, hd);
            auto map = [&](int i, int& offset, int& index) {
                offset = blocked_slot(h * hd + i, xq_shape.block, a.log2_d);
                index = i;
                return true;
            };
            if constexpr (T == 1)
            {
                if (!poll<1>(ex + a.off_xq, hd, map, sh.q, epoch, a.status, sh))
                    return false;
            }
            else if (!gather_tokens<1>(ex + a.off_xq, tw, count, hd, map, sh.q,
                                       [](int k, int i) { return k * kQStride + i; }, epoch, a.status, sh))
                return false;
            if (t == task)
                STEP_STAMP(6, l);
            uint64_t* part = ex + a.off_xpart + (size_t) (h * a.cross_splits + s) * (hd + 2);
            if constexpr (T == 1)
                attend<kCrossPasses>(cross, keys, hd, a.scale * kLog2e, part, epoch, sh, false, t == task ? 22 : -1);
            else
                attend_tokens<kCrossPasses, T>(cross, keys, count, hd, a.scale * kLog2e, part, tw, epoch, sh, sh.q);
        }
        STEP_STAMP(7, l);

        // ---- cross out-proj + residual (weights in pb) --------------------------------
        if constexpr (T == 1)
        {
            if (!gather_any(ex + a.off_xattn, d, sh.x, epoch, a.status, sh))
                return false;
        }
        else
        {
            auto map = [](int i, int& offset, int& index) {
                offset = index = i;
                return true;
            };
            if (!(d <= 2 * kPollThreads
                      ? gather_token_block<2, T>(ex + a.off_xattn, tw, 0, count, d, map, sh.x, x_at<T>, epoch,
                                                 a.status, sh)
                      : gather_token_block<3, T>(ex + a.off_xattn, tw, 0, count, d, map, sh.x, x_at<T>, epoch,
                                                 a.status, sh)))
                return false;
        }
        STEP_STAMP(8, l);
        {
            uint64_t* out = ex + a.off_h3;
            run_phase<WT, false, T>(
                pb, L.cross_out_w, L.cross_out_b, nullptr, none, square_shape, group, stride, count, sh,
                [&](int r, int j, int k, float v) {
                    put(out + k * tw + (group << a.log2_d) + j, sh.raw[k * kRawStride + r] + v, epoch);
                },
                [&] {
                    prefetch<true, T>(pa, L.fc1_w, TL + a.terms_fc1_bias, TL + a.terms_fc1_gain, fc1_shape, group,
                                      stride);
                    load_fold(fold, L.final_norm_w, d, a.log2_d, stride);
                },
                31);
        }
        STEP_STAMP(9, l);

        // ---- LN3 folded into fc1 + GELU (weights in pa) ----------------------------------
        if (!gather_fold<T>(ex + a.off_h3, tw, count, d, a.log2_d, stride, fold, shift, epoch, a.status, sh))
            return false;
        STEP_STAMP(10, l);
        statistics();
        {
            uint64_t* out = ex + a.off_ff;
            run_phase<WT, true, T>(
                pa, L.fc1_w, TL + a.terms_fc1_bias, TL + a.terms_fc1_gain, fs, fc1_shape, group, stride, count, sh,
                [&](int, int j, int k, float v) { put(out + k * tw + (group << a.log2_f) + j, exact_gelu(v), epoch); },
                [&] { prefetch<false, T>(pb, L.fc2_w, L.fc2_b, nullptr, fc2_shape, group, stride); }, 33);
        }
        STEP_STAMP(11, l);

        // ---- fc2 + residual (weights in pb) ------------------------------------------------
        if constexpr (T == 1)
        {
            if (!gather_words<kPollBlockedFF>(ex + a.off_ff, f, a.log2_f, stride, sh.x, epoch, a.status, sh,
                                              [](int i) { return i; }))
                return false;
        }
        else
        {
            // Two tokens a round of sixteen words per thread.
            const int mask = (1 << a.log2_f) - 1, slots = stride << a.log2_f;
            auto map = [&](int i, int& offset, int& index) {
                offset = i;
                index = (i & mask) * stride + (i >> a.log2_f);
                return index < f;
            };
            for (int k = 0; k < count; k += 2)
                for (int first = 0; first < slots; first += kPollBlockedFF * kPollThreads)
                    if (!gather_token_block<kPollBlockedFF, 2>(ex + a.off_ff, tw, k, count, slots, map, sh.x,
                                                               x_at<T>, epoch, a.status, sh, first))
                        return false;
        }
        STEP_STAMP(12, l);
        {
            // After the dot products: the next layer's q/k/v slice, its folded
            // terms and LN1's gamma (the last layer loads its own again, unused,
            // so these loads are issued on every path).
            const int next_layer = min(l + 1, a.layer_count - 1);
            const wsp_layer_tensors& next = sh.table[next_layer];
            const float* TN = a.fold_terms + (size_t) next_layer * a.terms_stride;
            uint64_t* out = ex + a.off_h4;
            run_phase<WT, false, T>(
                pb, L.fc2_w, L.fc2_b, nullptr, none, fc2_shape, group, stride, count, sh,
                [&](int r, int j, int k, float v) {
                    put(out + k * tw + (group << a.log2_d) + j, sh.raw[k * kRawStride + r] + v, epoch);
                },
                [&] {
                    prefetch<true, T>(pa, next.self_qkv_w, TN + a.terms_qkv_bias, TN + a.terms_qkv_gain, qkv_shape,
                                      group, stride);
                    load_fold(fold, next.self_norm_w, d, a.log2_d, stride);
                },
                35);
        }
        STEP_STAMP(13, l);
    }
    return true;
}

__device__ __forceinline__ bool head_group_layers(const StepArgs& a, Shared& sh)
{
    const int d = a.width, H = a.heads, hd = d / H;
    const int index = blockIdx.x - a.row_groups;
    const int qkv_block = (3 * d + a.row_groups - 1) / a.row_groups; // the q/k/v phase's rows per workgroup
    const int head = index % H, split = index / H;
    const int n = a.position + 1; // keys attended, the new one included
    const int first = split * a.self_chunk;
    const int count = min(a.self_chunk, n - first);            // <= 0 for an idle split
    const int cached = max(0, min(count, a.position - first)); // keys read from the cache
    const bool attends = split < a.self_splits;
    const uint32_t epoch = a.epoch;

    KeyRows<kSelfPasses> self;
    if (attends && cached > 0)
        load_keys<kSelfPasses>(self, sh.table[0].self_keys, sh.table[0].self_values, first, cached, d, head * hd, hd);

    for (int l = 0; l < a.layer_count; ++l)
    {
        uint64_t* ex = a.exchange + (size_t) l * a.layer_words;
        const bool last_layer = l + 1 == a.layer_count;
        STEP_LAYER(l);
        if (attends)
        {
            // q, and the new key/value rows, of this head, in one wait.
            if (!poll<1>(
                    ex + a.off_qkv, 3 * hd,
                    [&](int i, int& offset, int& index) {
                        offset = blocked_slot((i / hd) * d + head * hd + i % hd, qkv_block, a.log2_qkv);
                        index = i;
                        return true;
                    },
                    sh.q, epoch, a.status, sh))
                return false;
            STEP_STAMP(14, l);
            if (count > cached)
            {
                // The new key sits at local index `cached` (= position - first).
                const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
                const int c = 4 * min(kl, hd / 4 - 1);
                const float4v nk = *reinterpret_cast<const float4v*>(&sh.q[hd + c]);
                const float4v nv = *reinterpret_cast<const float4v*>(&sh.q[2 * hd + c]);
#pragma unroll
                for (int p = 0; p < kSelfPasses; ++p)
                    if (ks + kKeySlots * p == cached && 4 * kl < hd)
                    {
                        self.k[p] = nk;
                        self.v[p] = nv;
                    }
            }
            attend<kSelfPasses>(self, count, hd, a.scale * kLog2e, ex + a.off_self + (size_t) (split * H + head) * (hd + 2),
                                epoch, sh, a.self_splits == 1, 22);
            STEP_STAMP(15, l);
        }
        // Cross-attention combine of one head; the next layer's keys are
        // loaded after it, so they never hold up its wait.
        if (index < H)
        {
            const int parts = a.cross_splits;
            const uint64_t* src = ex + a.off_xpart + (size_t) head * parts * (hd + 2);
            const int n = parts * (hd + 2);
            if (!(n <= 2 * kPollThreads ? gather<2, true>(src, n, sh.comb, epoch, a.status, sh)
                                        : gather_any(src, n, sh.comb, epoch, a.status, sh)))
                return false;
            STEP_STAMP(16, l);
            combine_parts(sh.comb, parts, hd, ex + a.off_xattn + head * hd, epoch, sh);
            STEP_STAMP(17, l);
        }
        if (!last_layer && attends && cached > 0)
            load_keys<kSelfPasses>(self, sh.table[l + 1].self_keys, sh.table[l + 1].self_values, first, cached, d,
                                   head * hd, hd);
        __syncthreads();
    }
    return true;
}

// The head groups of a multi-token launch: workgroup (query k, head h) —
// index k * H + h past the row groups — attends token k's query of head h
// over the cached keys and the new keys of tokens 0..k (the causal mask of
// Kernels/Attention.h:34-47); its row goes to token k's self slot, normalized.
// The positions stay within one key block (position + count <= kSelfKeys), so
// no key split is combined. The first H of them also combine every token's
// cross-attention partials of their head.
template <int T>
__device__ __forceinline__ bool head_group_tokens(const StepArgs& a, Shared& sh)
{
    const int d = a.width, H = a.heads, hd = d / H;
    const int index = blockIdx.x - a.row_groups;
    const int qkv_block = (3 * d + a.row_groups - 1) / a.row_groups; // the q/k/v phase's rows per workgroup
    const int head = index % H, query = index / H;
    const int count = a.token_count, tw = a.token_words;
    const int cached = a.position;                // keys read from the cache
    const bool attends = query < count;
    const int keys = cached + query + 1;          // keys attended by this query
    const uint32_t epoch = a.epoch;

    KeyRows<kSelfPasses> self;
    if (attends && cached > 0)
        load_keys<kSelfPasses>(self, sh.table[0].self_keys, sh.table[0].self_values, 0, cached, d, head * hd, hd);

    for (int l = 0; l < a.layer_count; ++l)
    {
        uint64_t* ex = a.exchange + (size_t) l * a.layer_words;
        const bool last_layer = l + 1 == a.layer_count;
        STEP_LAYER(l);
        if (attends)
        {
            // q, new key and new value of this head for tokens 0..query, in
            // one wait: token k's block at sh.q + k * kQStride.
            if (!gather_tokens<2>(
                    ex + a.off_qkv, tw, query + 1, 3 * hd,
                    [&](int i, int& offset, int& at) {
                        offset = blocked_slot((i / hd) * d + head * hd + i % hd, qkv_block, a.log2_qkv);
                        at = i;
                        return true;
                    },
                    sh.q, [](int k, int i) { return k * kQStride + i; }, epoch, a.status, sh))
                return false;
            STEP_STAMP(14, l);
            // The new keys sit at local indices cached .. cached + query.
            const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
            const int c = 4 * min(kl, hd / 4 - 1);
#pragma unroll
            for (int p = 0; p < kSelfPasses; ++p)
            {
                const int j = ks + kKeySlots * p - cached; // the new token this slot holds
                if (j >= 0 && j <= query && 4 * kl < hd)
                {
                    self.k[p] = *reinterpret_cast<const float4v*>(&sh.q[j * kQStride + hd + c]);
                    self.v[p] = *reinterpret_cast<const float4v*>(&sh.q[j * kQStride + 2 * hd + c]);
                }
            }
            attend<kSelfPasses>(self, keys, hd, a.scale * kLog2e, ex + query * tw + a.off_self + (size_t) head * (hd + 2),
                                epoch, sh, true, 22, sh.q + query * kQStride);
            STEP_STAMP(15, l);
        }
        // Cross-attention combine of one head for every token.
        if (index < H)
        {
            const int parts = a.cross_splits;
            const int n = parts * (hd + 2);
            if (!gather_tokens<kPollCombine>(
                    ex + a.off_xpart + (size_t) head * n, tw, count, n,
                    [](int i, int& offset, int& at) {
                        offset = at = i;
                        return true;
                    },
                    sh.comb, [n](int k, int i) { return k * n + i; }, epoch, a.status, sh))
                return false;
            STEP_STAMP(16, l);
            combine_tokens<T>(sh.comb, n, parts, hd, ex + a.off_xattn + head * hd, tw, count, epoch, sh);
            STEP_STAMP(17, l);
        }
        if (!last_layer && attends && cached > 0)
            load_keys<kSelfPasses>(self, sh.table[l + 1].self_keys, sh.table[l + 1].self_values, 0, cached, d,
                                   head * hd, hd);
        __syncthreads();
    }
    return true;
}

// Final LN of the last layer's output, the tied logits (Decoder/Decoder.cpp
// :174-176) and this workgroup's top-1 under the mask.
template <int LWT, int T>
__device__ __forceinline__ bool final_phase(const StepArgs& a, Shared& sh, Ring& ring, const NormParams& norm,
                                            float& best_v, uint32_t& best_i)
{
    const int d = a.width;
    const int count = T == 1 ? 1 : a.token_count;
    const uint64_t* h4 = a.exchange + (size_t) (a.layer_count - 1) * a.layer_words + a.off_h4;
    if constexpr (T == 1)
    {
        if (!gather_blocked<kPollBlocked>(h4, d, a.log2_d, a.row_groups, sh.raw, a.epoch, a.status, sh))
            return false;
    }
    else
    {
        const int stride = a.row_groups, mask = (1 << a.log2_d) - 1;
        auto map = [&](int i, int& offset, int& index) {
            offset = i;
            index = (i & mask) * stride + (i >> a.log2_d);
            return index < d;
        };
        auto place = [](int k, int i) { return k * kRawStride + i; };
        const int slots = stride << a.log2_d;
        if (!(slots <= 2 * kPollThreads
                  ? gather_token_block<2, T>(h4, a.token_words, 0, count, slots, map, sh.raw, place, a.epoch,
                                             a.status, sh)
                  : gather_token_block<4, T>(h4, a.token_words, 0, count, slots, map, sh.raw, place, a.epoch,
                                             a.status, sh)))
            return false;
    }
    STEP_STAMP(18, 0);
    // The first logits rows are issued once the last layer's output is in:
    // issued before, they would share the memory pipeline with its polls.
    issue_ring(ring, a, logit_shape(a));
    layer_norm<T>(norm, d, a.inv_width, a.eps, sh, -1, count);
    if (blockIdx.x == 0)
        for (int k = 0; k < count; ++k)
            for (int c = threadIdx.x; c < d; c += kThreads)
                a.hidden[(size_t) k * d + c] = sh.x[x_at<T>(k, c)];
    logits_loop<LWT, T>(ring, a, logit_shape(a), sh, count, best_v, best_i);
    STEP_STAMP(19, 0);
    return true;
}

template <int WT, int T>
__device__ __forceinline__ void step_body(const StepArgs& a, Shared& sh)
{
    if (threadIdx.x == 0)
        sh.abort = 0;
    const bool row_group = (int) blockIdx.x < a.row_groups;
    Embedding<T> embed;
    if (row_group)
        issue_embedding<T>(embed, a);
    {
        // The layer table, once.
        const int words = a.layer_count * (int) (sizeof(wsp_layer_tensors) / sizeof(uint64_t));
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.layers);
        uint64_t* dst = reinterpret_cast<uint64_t*>(sh.table);
        for (int i = threadIdx.x; i < words; i += kThreads)
            dst[i] = src[i];
    }
    __syncthreads();
    STEP_STAMP(21, 0);

    bool ok;
    if constexpr (T == 1)
        ok = row_group ? row_group_layers<WT, 1>(a, sh, embed) : head_group_layers(a, sh);
    else
        ok = row_group ? row_group_layers<WT, T>(a, sh, embed) : head_group_tokens<T>(a, sh);
    if (!ok)
        return;
    // The final norm's parameters are in flight before the last layer's output
    // is awaited.
    Ring ring;
    NormParams norm;
    load_norm(norm, a.final_norm_w, a.final_norm_b, a.width);

    // ---- final LN + tied logits with a per-workgroup top-1 -----------------------
    const int G = gridDim.x;
    const uint32_t epoch = a.epoch;
    float best_v = 0.f;
    uint32_t best_i = kUnchosen;
    bool done;
    switch (a.logits_wdtype)
    {
        case kF32: done = final_phase<kF32, T>(a, sh, ring, norm, best_v, best_i); break;
        case kF16: done = final_phase<kF16, T>(a, sh, ring, norm, best_v, best_i); break;
        default: done = final_phase<kBF16, T>(a, sh, ring, norm, best_v, best_i); break;
    }
    if (!done)
        return;
    const LogitShape ls = logit_shape(a);
    const int rg = threadIdx.x >> ls.lanes_log2;
    if ((threadIdx.x & ((1 << ls.lanes_log2) - 1)) == 0)
    {
        sh.best_v[rg] = best_v;
        sh.best_i[rg] = best_i;
    }
    __syncthreads();
    STEP_LAYER(0);
    STEP_MARK(37); // every row group of this workgroup done with the logits
    if (threadIdx.x < kKeyLanes)
    {
        // The row groups' candidates (at most 16: rows of 32 or 64 lanes) in
        // the first row of wave 0.
        const bool held = (int) threadIdx.x < ls.groups;
        float bv = held ? sh.best_v[threadIdx.x] : 0.f;
        uint32_t bi = held ? sh.best_i[threadIdx.x] : kUnchosen;
        fold16(bv, bi);
        // The candidates packed two words each, so the fold polls few lines.
        if (threadIdx.x == 0)
        {
            put(a.exchange + a.off_argmax + 2 * blockIdx.x, bv, epoch);
            put(a.exchange + a.off_argmax + 2 * blockIdx.x + 1, __uint_as_float(bi), epoch);
        }
    }

    // ---- the argmax fold (Kernels/Argmax.h:145-201) ---------------------------------
    // The last workgroup folds: workgroup 0 also stores the hidden row, and
    // its polls would wait for those stores' acknowledgements.
    if (blockIdx.x != gridDim.x - 1 || a.argmax_out == nullptr)
        return;
    if (!gather<kPollArgmax, false>(a.exchange + a.off_argmax, 2 * G, sh.comb, epoch, a.status, sh))
        return;
    STEP_MARK(38); // every workgroup's candidate arrived
    if (threadIdx.x < kWave)
    {
        float bv = 0.f;
        uint32_t bi = kUnchosen;
        for (int k = threadIdx.x; k < G; k += kWave)
        {
            const float v = sh.comb[2 * k];
            const uint32_t i = __float_as_uint(sh.comb[2 * k + 1]);
            if (better(v, i, bv, bi))
            {
                bv = v;
                bi = i;
            }
        }
        fold64(bv, bi);
        if (threadIdx.x == 0)
        {
            const uint32_t token = bi == kUnchosen ? 0u : bi;
            a.argmax_out[0] = token;
            // Every workgroup's candidate arrived, so none waits any more:
            // the watchdog word is final for this step.
            if (a.host_pair != nullptr)
            {
                __hip_atomic_store(a.host_pair, (int) token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(a.host_pair + 1,
                                   __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        STEP_STAMP(20, 0);
    }
}

template <int WT, int T>
__global__ void __launch_bounds__(kThreads) step_kernel(StepArgs a)
{
    __shared__ Shared sh;
#ifdef WSP_STEP_TIMELINE
    for (int i = threadIdx.x; i < kTimelineEvents * kTimelineLayers; i += kThreads)
        (&sh.timeline[0][0])[i] = 0;
    __syncthreads();
#endif
    step_body<WT, T>(a, sh);
#ifdef WSP_STEP_TIMELINE
    __syncthreads();
    if (a.timeline != nullptr)
        for (int i = threadIdx.x; i < kTimelineEvents * kTimelineLayers; i += kThreads)
            a.timeline[(size_t) blockIdx.x * kTimelineEvents * kTimelineLayers + i] = (&sh.timeline[0][0])[i];
#endif
}
} // namespace

const void* kernel_for(int wdtype, bool multi_token)
{
    switch (wdtype)
    {
        case kF32:
            return multi_token ? reinterpret_cast<const void*>(&step_kernel<kF32, kMaxTokens>)
                               : reinterpret_cast<const void*>(&step_kernel<kF32, 1>);
        case kF16:
            return multi_token ? reinterpret_cast<const void*>(&step_kernel<kF16, kMaxTokens>)
                               : reinterpret_cast<const void*>(&step_kernel<kF16, 1>);
        default:
            return multi_token ? reinterpret_cast<const void*>(&step_kernel<kBF16, kMaxTokens>)
                               : reinterpret_cast<const void*>(&step_kernel<kBF16, 1>);
    }
}
} // namespace wsp::step
