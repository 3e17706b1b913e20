// The single-token decoder step (Decoder/Decoder.cpp:151-177 with one token,
// then Argmax over the logits row, Whisper/Whisper.cpp:1164-1184) as ONE
// persistent cooperative launch on gfx950.
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
// Why it streams at bandwidth: each workgroup issues the loads of its slice of
// the next phase's weights (and of its cross-attention key/value chunk)
// BEFORE it waits for that phase's inputs, so HBM traffic overlaps the
// hand-over chain instead of following it.
//
// Roles (G workgroups of 512 threads, one per CU):
//   - the first Gg ("row" groups) run every projection, the cross-attention
//     key chunks and half of the logits;
//   - the last Ga = heads * self_split_max ("head" groups) run self-attention,
//     each holding its head's cached keys and values in registers (prefetched
//     one layer ahead), and the cross-attention combine of one head.
// Per layer the chain is: LN1+QKV -> self attention -> out-proj (+residual)
// -> LN2+cross-q -> cross partials -> cross combine -> cross out (+residual)
// -> LN3+fc1+GELU -> fc2 (+residual). Then final LN + tied logits with a
// per-workgroup top-1, and the argmax fold in workgroup 0.
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
constexpr int kSpinLimit = 1 << 21;                // poll rounds before the watchdog trips
constexpr uint32_t kUnchosen = 0xFFFFFFFFu;

static_assert(kSelfKeys % kKeySlots == 0 && kCrossKeys % kKeySlots == 0, "key capacities");

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

struct Shared
{
    float raw[kMaxWidth];       // the residual stream as gathered (un-normalised)
    float x[kMaxFeedForward];   // the current phase's input vector
    float comb[kMaxCombine];    // attention partials being combined
    float red[kKeySlots][kMaxHeadWidth]; // per-key-slot value rows
    float q[3 * kMaxHeadWidth]; // a head's query, then (self-attention) its new key and value
    float scratch[kThreads / kWave];
    float part[kRowGroups];     // per-row-group partial sums of a projection pass
    float best_v[kRowGroups];
    uint32_t best_i[kRowGroups];
    int abort;
};

// Waits until the n words (n <= P * 512) at src carry `epoch` and copies their
// floats to dst (LDS). With SEG, word i sits at
// src[(i / segment) * segment_stride + i % segment], so a few equal runs of a
// buffer (a head's q, k and v) are awaited together. Every poll round issues
// all of a thread's outstanding loads at once. Returns false, uniformly over
// the workgroup, when the watchdog tripped here or anywhere else.
template <int P, bool SEG = false>
__device__ __forceinline__ bool gather(const uint64_t* src, int n, float* dst, uint32_t epoch, int* status,
                                       Shared& sh, int segment = 1, int segment_stride = 0)
{
    const uint64_t* at[P];
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < P; ++k)
    {
        const int i = threadIdx.x + k * kThreads;
        if (i < n)
        {
            pending |= 1u << k;
            at[k] = SEG ? src + (i / segment) * segment_stride + i % segment : src + i;
        }
    }
    int spins = 0;
    bool failed = false;
    while (pending != 0)
    {
        uint64_t w[P];
#pragma unroll
        for (int k = 0; k < P; ++k)
            if (pending & (1u << k))
                w[k] = peek(at[k]);
#pragma unroll
        for (int k = 0; k < P; ++k)
            if ((pending & (1u << k)) && (uint32_t) (w[k] >> 32) == epoch)
            {
                dst[threadIdx.x + k * kThreads] = __uint_as_float((uint32_t) w[k]);
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
    if (failed)
        sh.abort = 1;
    __syncthreads();
    return sh.abort == 0;
}

// Words per thread for the vectors a phase awaits.
constexpr int kPollWidth = (kMaxWidth + kThreads - 1) / kThreads;
constexpr int kPollFeedForward = (kMaxFeedForward + kThreads - 1) / kThreads;
constexpr int kPollCombine = (kMaxCombine + kThreads - 1) / kThreads;

// ---------------------------------------------------------------------------
// Reductions over the 512-thread workgroup (fixed order: wave butterfly, then
// the eight wave totals in wave order).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float group_sum(float v, Shared& sh)
{
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0)
        sh.scratch[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / kWave; ++i)
        t += sh.scratch[i];
    return t;
}

__device__ __forceinline__ float group_max(float v, Shared& sh)
{
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0)
        sh.scratch[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = sh.scratch[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i)
        t = fmaxf(t, sh.scratch[i]);
    return t;
}

__device__ __forceinline__ float row_sum(float v)
{
#pragma unroll
    for (int offset = kRowLanes / 2; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, kRowLanes);
    return v;
}

// ---------------------------------------------------------------------------
// LayerNorm of sh.raw into sh.x: mean, centred biased variance, then
// (x - mean) * rsqrt(var + eps) * gamma + beta (Kernels/LayerNorm.h:44-89).
// gamma/beta arrive as registers loaded before the inputs were awaited.
// ---------------------------------------------------------------------------
constexpr int kNormPer = (kMaxWidth + kThreads - 1) / kThreads;

struct NormParams
{
    float g[kNormPer];
    float b[kNormPer];
};

__device__ __forceinline__ void load_norm(NormParams& p, const float* gamma, const float* beta, int n)
{
#pragma unroll
    for (int k = 0; k < kNormPer; ++k)
    {
        const int i = threadIdx.x + k * kThreads;
        p.g[k] = i < n ? gamma[i] : 0.f;
        p.b[k] = i < n ? beta[i] : 0.f;
    }
}

__device__ __forceinline__ void layer_norm(const NormParams& p, int n, float eps, Shared& sh)
{
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kNormPer; ++k)
    {
        const int i = threadIdx.x + k * kThreads;
        if (i < n)
            s += sh.raw[i];
    }
    const float mean = group_sum(s, sh) / (float) n;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < kNormPer; ++k)
    {
        const int i = threadIdx.x + k * kThreads;
        if (i < n)
        {
            const float c = sh.raw[i] - mean;
            q += c * c;
        }
    }
    const float scale = rsqrtf(group_sum(q, sh) / (float) n + eps);
#pragma unroll
    for (int k = 0; k < kNormPer; ++k)
    {
        const int i = threadIdx.x + k * kThreads;
        if (i < n)
            sh.x[i] = (sh.raw[i] - mean) * scale * p.g[k] + p.b[k];
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Projection rows. A row is cut into `slices` equal runs of 16-byte chunks (8
// fp16/bf16 or 4 fp32 weights); one slice is walked by a row group of 32
// lanes, lane l taking chunks l, l+32, l+64 of the run in ascending order, and
// the 32 partials are summed by a fixed butterfly. The slices of a row are then
// added in slice order. Row r of a phase belongs to workgroup r % stride; a
// workgroup's (row, slice) tasks go to its 16 row groups in order, so with the
// slice count chosen per phase every row group has work and holds at most
// kChunks chunks per lane — all of which are in flight before the phase's
// input is awaited.
// ---------------------------------------------------------------------------
constexpr int kChunks = 3;

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

struct Phase
{
    const void* weight;
    const float* bias; // null: none
    int rows;
    int inner;
    int slices;        // a power of two dividing kRowGroups
    int slice_chunks;  // chunks per slice (<= kRowLanes * kChunks)
};

template <int WT>
__device__ __forceinline__ Phase make_phase(const void* weight, const float* bias, int rows, int inner, int stride)
{
    const int chunks = inner / Storage<WT>::kPerChunk;
    const int local_rows = (rows + stride - 1) / stride;
    int slices = 1;
    while (slices < kRowGroups && (slices * kRowLanes * kChunks < chunks || 2 * slices * local_rows <= kRowGroups))
        slices *= 2;
    return Phase {weight, bias, rows, inner, slices, (chunks + slices - 1) / slices};
}

// Loads chunks [first, last) of `row`, lane l taking first + l + 32 i.
template <int WT>
__device__ __forceinline__ void load_run(RowLoad& r, const void* weight, int row, int inner, int first, int last)
{
    const int lane = threadIdx.x & (kRowLanes - 1);
    const char* base = static_cast<const char*>(weight) + (size_t) row * inner * Storage<WT>::kBytes;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = first + lane + kRowLanes * i;
        if (c < last)
            r.w[i] = *reinterpret_cast<const uint4*>(base + (size_t) c * 16);
    }
}

template <int WT>
__device__ __forceinline__ float chunk_dot(const uint4& u, const float* x)
{
    float acc = 0.f;
    if constexpr (WT == kF32)
    {
        const float4v xv = *reinterpret_cast<const float4v*>(x);
        acc += xv[0] * __uint_as_float(u.x);
        acc += xv[1] * __uint_as_float(u.y);
        acc += xv[2] * __uint_as_float(u.z);
        acc += xv[3] * __uint_as_float(u.w);
    }
    else
    {
        const float4v xa = *reinterpret_cast<const float4v*>(x);
        const float4v xb = *reinterpret_cast<const float4v*>(x + 4);
        const uint32_t v[4] = {u.x, u.y, u.z, u.w};
        float w[8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            if constexpr (WT == kF16)
            {
                const _Float16* h = reinterpret_cast<const _Float16*>(&v[i]);
                w[2 * i] = (float) h[0];
                w[2 * i + 1] = (float) h[1];
            }
            else
            {
                w[2 * i] = __uint_as_float(v[i] << 16);
                w[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
            }
        }
        acc += xa[0] * w[0];
        acc += xa[1] * w[1];
        acc += xa[2] * w[2];
        acc += xa[3] * w[3];
        acc += xb[0] * w[4];
        acc += xb[1] * w[5];
        acc += xb[2] * w[6];
        acc += xb[3] * w[7];
    }
    return acc;
}

template <int WT>
__device__ __forceinline__ float run_dot(const RowLoad& r, const float* x, int first, int last)
{
    const int lane = threadIdx.x & (kRowLanes - 1);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
    {
        const int c = first + lane + kRowLanes * i;
        if (c < last)
            acc += chunk_dot<WT>(r.w[i], x + c * Storage<WT>::kPerChunk);
    }
    return acc;
}

// The (row, slice) task of this row group in `pass`, or false when it has none.
__device__ __forceinline__ bool phase_task(const Phase& ph, int group, int stride, int pass, int& row, int& first,
                                           int& last)
{
    const int local_rows = group < ph.rows ? (ph.rows - group + stride - 1) / stride : 0;
    const int task = pass * kRowGroups + (int) (threadIdx.x / kRowLanes);
    if (task >= local_rows * ph.slices)
        return false;
    row = group + stride * (task / ph.slices);
    first = (task % ph.slices) * ph.slice_chunks;
    last = first + ph.slice_chunks;
    return true;
}

template <int WT>
struct Prefetch
{
    RowLoad r;
    float bias; // the bias of the row this thread finishes in pass 0
};

template <int WT>
__device__ __forceinline__ void prefetch_phase(Prefetch<WT>& p, const Phase& ph, int group, int stride)
{
    int row, first, last;
    const int chunks = ph.inner / Storage<WT>::kPerChunk;
    if (phase_task(ph, group, stride, 0, row, first, last))
        load_run<WT>(p.r, ph.weight, row, ph.inner, first, min(last, chunks));
    const int finisher_row = group + stride * (int) threadIdx.x;
    p.bias = 0.f;
    if (ph.bias != nullptr && (int) threadIdx.x < kRowGroups / ph.slices && finisher_row < ph.rows)
        p.bias = ph.bias[finisher_row];
}

// Runs every task of the phase against sh.x. epi(row, value) receives the dot
// product plus bias, on thread (local row) % (16 / slices).
template <int WT, class Epilogue>
__device__ __forceinline__ void run_phase(const Prefetch<WT>& p, const Phase& ph, int group, int stride, Shared& sh,
                                          Epilogue epi)
{
    const int chunks = ph.inner / Storage<WT>::kPerChunk;
    const int local_rows = group < ph.rows ? (ph.rows - group + stride - 1) / stride : 0;
    const int rows_per_pass = kRowGroups / ph.slices;
    const int passes = (local_rows + rows_per_pass - 1) / rows_per_pass;
    for (int pass = 0; pass < passes; ++pass)
    {
        int row, first, last;
        if (phase_task(ph, group, stride, pass, row, first, last))
        {
            float acc;
            if (pass == 0)
                acc = run_dot<WT>(p.r, sh.x, first, min(last, chunks));
            else
            {
                RowLoad r;
                load_run<WT>(r, ph.weight, row, ph.inner, first, min(last, chunks));
                acc = run_dot<WT>(r, sh.x, first, min(last, chunks));
            }
            acc = row_sum(acc);
            if ((threadIdx.x & (kRowLanes - 1)) == 0)
                sh.part[threadIdx.x / kRowLanes] = acc;
        }
        __syncthreads();
        const int local = pass * rows_per_pass + (int) threadIdx.x;
        if ((int) threadIdx.x < rows_per_pass && local < local_rows)
        {
            float v = 0.f;
            for (int s2 = 0; s2 < ph.slices; ++s2)
                v += sh.part[threadIdx.x * ph.slices + s2];
            const int r = group + stride * local;
            const float b = pass == 0 ? p.bias : (ph.bias != nullptr ? ph.bias[r] : 0.f);
            epi(r, v + b);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Single-query attention over keys held in registers: thread t holds channels
// 4*(t%16).. of key slot t/16 for keys slot + 32*p. Scores (scale * q.k),
// their maximum, exp(s - max), the sum and the unnormalised value row — the
// chunk form of Kernels/SingleQueryAttention.h:27-37.
// ---------------------------------------------------------------------------
template <int NP>
struct KeyRows
{
    float4v k[NP];
    float4v v[NP];
};

template <int NP>
__device__ __forceinline__ void load_keys(KeyRows<NP>& kr, const float* keys, const float* values, int first,
                                          int count, int width, int column, int head_width)
{
    const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        const int key = ks + kKeySlots * p;
        if (key < count && 4 * kl < head_width)
        {
            const size_t at = (size_t) (first + key) * width + column + 4 * kl;
            kr.k[p] = *reinterpret_cast<const float4v*>(keys + at);
            kr.v[p] = *reinterpret_cast<const float4v*>(values + at);
        }
    }
}

// Writes (max, sum, row[head_width]) of `count` keys into out (exchange words).
template <int NP>
__device__ __forceinline__ void attend(const KeyRows<NP>& kr, int count, int head_width, float scale, uint64_t* out,
                       uint32_t epoch, Shared& sh)
{
    const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
    float4v qv = {0.f, 0.f, 0.f, 0.f};
    if (4 * kl < head_width)
        qv = *reinterpret_cast<const float4v*>(sh.q + 4 * kl);
    float s[NP];
    float local_max = -INFINITY;
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        float part = 0.f;
        if (4 * kl < head_width)
            part = qv[0] * kr.k[p][0] + qv[1] * kr.k[p][1] + qv[2] * kr.k[p][2] + qv[3] * kr.k[p][3];
#pragma unroll
        for (int offset = kKeyLanes / 2; offset > 0; offset >>= 1)
            part += __shfl_xor(part, offset, kKeyLanes);
        s[p] = scale * part;
        if (ks + kKeySlots * p < count)
            local_max = fmaxf(local_max, s[p]);
    }
    const float m = group_max(local_max, sh);
    float local_sum = 0.f;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NP; ++p)
    {
        if (ks + kKeySlots * p < count)
        {
            const float e = expf(s[p] - m);
            if (kl == 0)
                local_sum += e;
            acc[0] += e * kr.v[p][0];
            acc[1] += e * kr.v[p][1];
            acc[2] += e * kr.v[p][2];
            acc[3] += e * kr.v[p][3];
        }
    }
    const float l = group_sum(local_sum, sh);
    if (4 * kl < head_width)
        *reinterpret_cast<float4v*>(&sh.red[ks][4 * kl]) = acc;
    __syncthreads();
    if ((int) threadIdx.x < head_width)
    {
        float row = 0.f;
        for (int slot = 0; slot < kKeySlots; ++slot)
            row += sh.red[slot][threadIdx.x];
        put(out + 2 + threadIdx.x, row, epoch);
    }
    if (threadIdx.x == 0)
    {
        put(out, count > 0 ? m : -INFINITY, epoch);
        put(out + 1, l, epoch);
    }
    __syncthreads();
}

// Combines `parts` partials (stride head_width + 2, as written by attend)
// into the normalised row: rescale each by exp(m_i - max) and divide
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
        const float factor = expf(p[0] - largest);
        numerator += factor * p[2 + c];
        denominator += factor * p[1];
    }
    return numerator / denominator;
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi)
{
    if (i == kUnchosen)
        return false;
    if (bi == kUnchosen)
        return true;
    return v > bv || (v == bv && i < bi);
}

// ---------------------------------------------------------------------------
// The persistent step.
// ---------------------------------------------------------------------------
template <int WT>
__device__ __forceinline__ void row_group_layers(const StepArgs& a, Shared& sh)
{
    const int d = a.width, f = a.feed_forward, H = a.heads, hd = d / H;
    const int group = blockIdx.x, stride = a.row_groups;
    const int pos = a.position;
    const uint32_t epoch = a.epoch;

    // The layer-0 input: the token and position rows (Kernels/Embed.h:9-14);
    // an id past the vocabulary poisons the row with NaN.
    {
        const uint32_t token = a.tokens[0];
        for (int c = threadIdx.x; c < d; c += kThreads)
            sh.raw[c] = token < (uint32_t) a.vocabulary
                            ? a.token_embedding[(size_t) token * d + c] + a.position_embedding[(size_t) pos * d + c]
                            : __builtin_nanf("");
        __syncthreads();
    }

    // One cross-attention chunk per row group when the split allows it; more
    // tasks than row groups wrap around (and are not prefetched).
    const int tasks = a.cross_splits * H;
    const int task = group;

    for (int l = 0; l < a.layer_count; ++l)
    {
        const wsp_layer_tensors& L = a.layers[l];
        uint64_t* ex = a.exchange + (size_t) l * a.layer_words;
        NormParams norm;
        Prefetch<WT> pre;

        // ---- LN1 + fused q/k/v ---------------------------------------------
        {
            const Phase ph = make_phase<WT>(L.self_qkv_w, L.self_qkv_b, 3 * d, d, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            load_norm(norm, L.self_norm_w, L.self_norm_b, d);
            if (l > 0
                && !gather<kPollWidth>(a.exchange + (size_t) (l - 1) * a.layer_words + a.off_h4, d, sh.raw, epoch,
                                       a.status, sh))
                return;
            layer_norm(norm, d, a.eps, sh);
            uint64_t* qkv = ex + a.off_qkv;
            float* krow = L.self_keys + (size_t) pos * d;
            float* vrow = L.self_values + (size_t) pos * d;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) {
                put(qkv + r, v, epoch);
                if (r >= 2 * d)
                    vrow[r - 2 * d] = v;
                else if (r >= d)
                    krow[r - d] = v;
            });
        }

        // ---- self-attention combine + out-proj + residual --------------------
        {
            const Phase ph = make_phase<WT>(L.self_out_w, L.self_out_b, d, d, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            const int parts = a.self_splits * H * (hd + 2);
            if (!gather<kPollCombine>(ex + a.off_self, parts, sh.comb, epoch, a.status, sh))
                return;
            for (int c = threadIdx.x; c < d; c += kThreads)
                sh.x[c] = combine(sh.comb + (c / hd) * (hd + 2), a.self_splits, H * (hd + 2), c % hd);
            __syncthreads();
            uint64_t* out = ex + a.off_h2;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) { put(out + r, sh.raw[r] + v, epoch); });
        }

        // ---- LN2 + cross q ---------------------------------------------------
        KeyRows<kCrossPasses> cross;
        {
            const Phase ph = make_phase<WT>(L.cross_q_w, L.cross_q_b, d, d, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            load_norm(norm, L.cross_norm_w, L.cross_norm_b, d);
            if (!gather<kPollWidth>(ex + a.off_h2, d, sh.raw, epoch, a.status, sh))
                return;
            if (task < tasks)
            {
                // Issued now, awaited only when the query arrives.
                const int first = (task / H) * a.cross_chunk;
                load_keys<kCrossPasses>(cross, L.cross_keys, L.cross_values, first,
                                        min(a.cross_chunk, a.cross_rows - first), d, (task % H) * hd, hd);
            }
            layer_norm(norm, d, a.eps, sh);
            uint64_t* out = ex + a.off_xq;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) { put(out + r, v, epoch); });
        }

        // ---- cross-attention partials, then out-proj + residual ---------------
        {
            const Phase ph = make_phase<WT>(L.cross_out_w, L.cross_out_b, d, d, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            for (int t = task; t < tasks; t += stride)
            {
                const int h = t % H, s = t / H;
                const int first = s * a.cross_chunk;
                const int count = min(a.cross_chunk, a.cross_rows - first);
                if (t != task)
                    load_keys<kCrossPasses>(cross, L.cross_keys, L.cross_values, first, count, d, h * hd, hd);
                if (!gather<1>(ex + a.off_xq + h * hd, hd, sh.q, epoch, a.status, sh))
                    return;
                attend<kCrossPasses>(cross, count, hd, a.scale,
                                     ex + a.off_xpart + (size_t) (h * a.cross_splits + s) * (hd + 2), epoch, sh);
            }
            if (!gather<kPollWidth>(ex + a.off_xattn, d, sh.x, epoch, a.status, sh))
                return;
            uint64_t* out = ex + a.off_h3;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) { put(out + r, sh.raw[r] + v, epoch); });
        }

        // ---- LN3 + fc1 + GELU ---------------------------------------------------
        {
            const Phase ph = make_phase<WT>(L.fc1_w, L.fc1_b, f, d, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            load_norm(norm, L.final_norm_w, L.final_norm_b, d);
            if (!gather<kPollWidth>(ex + a.off_h3, d, sh.raw, epoch, a.status, sh))
                return;
            layer_norm(norm, d, a.eps, sh);
            uint64_t* out = ex + a.off_ff;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) { put(out + r, exact_gelu(v), epoch); });
        }

        // ---- fc2 + residual ---------------------------------------------------------
        {
            const Phase ph = make_phase<WT>(L.fc2_w, L.fc2_b, d, f, stride);
            prefetch_phase<WT>(pre, ph, group, stride);
            if (!gather<kPollFeedForward>(ex + a.off_ff, f, sh.x, epoch, a.status, sh))
                return;
            uint64_t* out = ex + a.off_h4;
            run_phase<WT>(pre, ph, group, stride, sh, [&](int r, float v) { put(out + r, sh.raw[r] + v, epoch); });
        }
    }
}

__device__ __forceinline__ void head_group_layers(const StepArgs& a, Shared& sh)
{
    const int d = a.width, H = a.heads, hd = d / H;
    const int index = blockIdx.x - a.row_groups;
    const int head = index % H, split = index / H;
    const int n = a.position + 1; // keys attended, the new one included
    const int first = split * kSelfKeys;
    const int count = min(kSelfKeys, n - first); // <= 0 for an idle split
    const int cached = max(0, min(count, a.position - first)); // keys read from the cache
    const uint32_t epoch = a.epoch;

    KeyRows<kSelfPasses> self;
    if (split < a.self_splits && cached > 0)
        load_keys<kSelfPasses>(self, a.layers[0].self_keys, a.layers[0].self_values, first, cached, d, head * hd, hd);

    for (int l = 0; l < a.layer_count; ++l)
    {
        uint64_t* ex = a.exchange + (size_t) l * a.layer_words;
        if (split < a.self_splits)
        {
            // q, and the new key/value rows, of this head, in one wait.
            if (!gather<1, true>(ex + a.off_qkv + head * hd, 3 * hd, sh.q, epoch, a.status, sh, hd, d))
                return;
            if (count > cached)
            {
                // The new key sits at local index `cached` (= position - first).
                const int kl = threadIdx.x % kKeyLanes, ks = threadIdx.x / kKeyLanes;
#pragma unroll
                for (int p = 0; p < kSelfPasses; ++p)
                    if (ks + kKeySlots * p == cached && 4 * kl < hd)
                    {
                        self.k[p] = *reinterpret_cast<const float4v*>(&sh.q[hd + 4 * kl]);
                        self.v[p] = *reinterpret_cast<const float4v*>(&sh.q[2 * hd + 4 * kl]);
                    }
            }
            attend<kSelfPasses>(self, count, hd, a.scale, ex + a.off_self + (size_t) (split * H + head) * (hd + 2),
                                epoch, sh);
            if (l + 1 < a.layer_count && cached > 0)
                load_keys<kSelfPasses>(self, a.layers[l + 1].self_keys, a.layers[l + 1].self_values, first, cached,
                                       d, head * hd, hd);
        }
        // Cross-attention combine of one head.
        if (index < H)
        {
            const int parts = a.cross_splits;
            if (!gather<kPollCombine>(ex + a.off_xpart + (size_t) head * parts * (hd + 2), parts * (hd + 2), sh.comb,
                                      epoch, a.status, sh))
                return;
            if ((int) threadIdx.x < hd)
                put(ex + a.off_xattn + head * hd + threadIdx.x, combine(sh.comb, parts, hd + 2, threadIdx.x), epoch);
            __syncthreads();
        }
    }
}

// Logits rows: row group g of workgroup w owns rows w + G * (g + 16 j); each
// batch keeps kLogitRows rows in flight per row group (two batches
// alternate), the mask value riding along with each row.
constexpr int kLogitRows = 2;

struct LogitBatch
{
    RowLoad r[kLogitRows];
    float mask[kLogitRows];
};

__device__ __forceinline__ int logit_row(int j)
{
    return blockIdx.x + gridDim.x * ((int) (threadIdx.x / kRowLanes) + kRowGroups * j);
}

template <int LWT>
__device__ __forceinline__ void load_logits(LogitBatch& b, const StepArgs& a, int j0)
{
    const int chunks = a.width / Storage<LWT>::kPerChunk;
#pragma unroll
    for (int k = 0; k < kLogitRows; ++k)
    {
        const int row = logit_row(j0 + k);
        if (row < a.vocabulary)
        {
            load_run<LWT>(b.r[k], a.logits_weight, row, a.width, 0, min(chunks, kRowLanes * kChunks));
            b.mask[k] = a.mask != nullptr ? a.mask[row] : 0.f;
        }
    }
}

// Finishes one batch: dot products (chunks past the first run load on the
// spot), logits stores and this row group's running top-1. A row group's rows
// ascend, so a strict ">" keeps the lowest index of a tie.
template <int LWT>
__device__ __forceinline__ void finish_logits(const LogitBatch& b, const StepArgs& a, int j0, const Shared& sh,
                                              float& best_v, uint32_t& best_i)
{
    const int d = a.width, V = a.vocabulary;
    const int chunks = d / Storage<LWT>::kPerChunk;
    const int run = kRowLanes * kChunks;
#pragma unroll
    for (int k = 0; k < kLogitRows; ++k)
    {
        const int row = logit_row(j0 + k);
        if (row >= V)
            break;
        float acc = run_dot<LWT>(b.r[k], sh.x, 0, min(chunks, run));
        for (int c0 = run; c0 < chunks; c0 += run)
        {
            RowLoad t;
            load_run<LWT>(t, a.logits_weight, row, d, c0, min(chunks, c0 + run));
            acc += run_dot<LWT>(t, sh.x, c0, min(chunks, c0 + run));
        }
        acc = row_sum(acc);
        if ((threadIdx.x & (kRowLanes - 1)) == 0)
        {
            a.logits[row] = acc;
            if (b.mask[k] == 0.f && (best_i == kUnchosen || acc > best_v))
            {
                best_v = acc;
                best_i = (uint32_t) row;
            }
        }
    }
}

// Final LN of the last layer's output, the tied logits (Decoder/Decoder.cpp
// :174-176) and this workgroup's top-1 under the mask. The first batch of
// logits rows is in flight before the last layer's output is awaited.
template <int LWT>
__device__ __forceinline__ bool final_phase(const StepArgs& a, Shared& sh, float& best_v, uint32_t& best_i)
{
    const int d = a.width;
    NormParams norm;
    load_norm(norm, a.final_norm_w, a.final_norm_b, d);
    LogitBatch b0, b1;
    load_logits<LWT>(b0, a, 0);
    if (!gather<kPollWidth>(a.exchange + (size_t) (a.layer_count - 1) * a.layer_words + a.off_h4, d, sh.raw, a.epoch,
                            a.status, sh))
        return false;
    layer_norm(norm, d, a.eps, sh);
    if (blockIdx.x == 0)
        for (int c = threadIdx.x; c < d; c += kThreads)
            a.hidden[c] = sh.x[c];
    for (int j0 = 0;; j0 += 2 * kLogitRows)
    {
        if (logit_row(j0) >= a.vocabulary)
            break;
        load_logits<LWT>(b1, a, j0 + kLogitRows);
        finish_logits<LWT>(b0, a, j0, sh, best_v, best_i);
        if (logit_row(j0 + kLogitRows) >= a.vocabulary)
            break;
        load_logits<LWT>(b0, a, j0 + 2 * kLogitRows);
        finish_logits<LWT>(b1, a, j0 + kLogitRows, sh, best_v, best_i);
    }
    return true;
}

template <int WT>
__global__ void __launch_bounds__(kThreads) step_kernel(StepArgs a)
{
    __shared__ Shared sh;
    if (threadIdx.x == 0)
        sh.abort = 0;
    __syncthreads();

    if ((int) blockIdx.x < a.row_groups)
        row_group_layers<WT>(a, sh);
    else
        head_group_layers(a, sh);
    if (sh.abort != 0)
        return;

    // ---- final LN + tied logits with a per-workgroup top-1 -----------------------
    const int G = gridDim.x;
    const uint32_t epoch = a.epoch;
    float best_v = 0.f;
    uint32_t best_i = kUnchosen;
    bool ok;
    switch (a.logits_wdtype)
    {
        case kF32: ok = final_phase<kF32>(a, sh, best_v, best_i); break;
        case kF16: ok = final_phase<kF16>(a, sh, best_v, best_i); break;
        default: ok = final_phase<kBF16>(a, sh, best_v, best_i); break;
    }
    if (!ok)
        return;
    const int rg = threadIdx.x / kRowLanes;
    if ((threadIdx.x & (kRowLanes - 1)) == 0)
    {
        sh.best_v[rg] = best_v;
        sh.best_i[rg] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        float bv = 0.f;
        uint32_t bi = kUnchosen;
        for (int k = 0; k < kRowGroups; ++k)
            if (better(sh.best_v[k], sh.best_i[k], bv, bi))
            {
                bv = sh.best_v[k];
                bi = sh.best_i[k];
            }
        put(a.exchange + a.off_argmax + 2 * blockIdx.x, bv, epoch);
        put(a.exchange + a.off_argmax + 2 * blockIdx.x + 1, __uint_as_float(bi), epoch);
    }

    // ---- the argmax fold (Kernels/Argmax.h:145-201) ---------------------------------
    if (blockIdx.x != 0 || a.argmax_out == nullptr)
        return;
    if (!gather<kPollCombine>(a.exchange + a.off_argmax, 2 * G, sh.comb, epoch, a.status, sh))
        return;
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
#pragma unroll
        for (int offset = kWave / 2; offset > 0; offset >>= 1)
        {
            const float ov = __shfl_xor(bv, offset, kWave);
            const uint32_t oi = __shfl_xor(bi, offset, kWave);
            if (better(ov, oi, bv, bi))
            {
                bv = ov;
                bi = oi;
            }
        }
        if (threadIdx.x == 0)
            a.argmax_out[0] = bi == kUnchosen ? 0u : bi;
    }
}
} // namespace

const void* kernel_for(int wdtype)
{
    switch (wdtype)
    {
        case kF32: return reinterpret_cast<const void*>(&step_kernel<kF32>);
        case kF16: return reinterpret_cast<const void*>(&step_kernel<kF16>);
        default: return reinterpret_cast<const void*>(&step_kernel<kBF16>);
    }
}
} // namespace wsp::step
