// MI355X (gfx950) decode worker: one persistent cooperative kernel per launch that runs
// every worker's instruction stream once per token for up to 64 tokens, with on-GPU greedy
// selection (replaces tileinfer/src/runtime/worker_kernel.cu and ops.cuh).
//
// Synchronization.  The reference separates waves with a grid barrier
// (worker_kernel.cu:105-107,191-192).  On MI355X a flat 256-block barrier costs 4.2 us and a
// contention-spread one 1.9 us, plus a store-acknowledge and a reload around it, against a
// token floor of about 344 us over ~83 waves.  This worker therefore synchronizes through an
// exchange area of 64-bit words, each holding one element of a wave's output in its low half
// and the epoch of the token/layer/phase that wrote it in its high half.  A producer stores
// the word with one device-coherent (sc1) 64-bit store, which is single-copy atomic, and a
// consumer polls the words it needs with device-coherent loads until every epoch matches:
// data and "arrived" travel together, so a dependency costs one coherent round trip.
// Every producer waits for its earlier side-effect stores (the K/V cache rows) to complete
// (s_waitcnt vmcnt(0)) before publishing, so a consumer that sees an epoch also sees them.
// The plan's barrier records therefore compile to nothing; the wave order they encode still
// decides which worker runs which task.
//
// Each operation issues its first weight loads (nontemporal, 16 bytes per lane) before it
// polls its inputs, so HBM latency overlaps the wait.  Weights are bf16 or fp32 with FP32
// accumulation; every bf16 rounding point follows the eager-PyTorch contract of the
// reference (docs/architecture.md:284-312; ops.cuh rounding sites cited per function).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>

#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = kThreads / 64;

// ---------------------------------------------------------------- scalar helpers

__device__ inline float bf16_bits_to_float(uint32_t bits) { return __uint_as_float(bits << 16); }

__device__ inline uint32_t float_to_bf16_bits(float value)
{
    // Round to nearest even; NaN stays a quiet NaN.
    const uint32_t u = __float_as_uint(value);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <bool BF16>
struct Num {
    using T = std::conditional_t<BF16, uint16_t, float>;
    static constexpr int kBytes = BF16 ? 2 : 4;
    static constexpr int kPerVec = 16 / kBytes;  // elements per 16-byte vector
    __device__ static float round(float v)
    {
        if constexpr (BF16)
            return bf16_bits_to_float(float_to_bf16_bits(v));
        else
            return v;
    }
    __device__ static float load(const void* base, size_t index)
    {
        if constexpr (BF16)
            return bf16_bits_to_float(static_cast<const uint16_t*>(base)[index]);
        else
            return static_cast<const float*>(base)[index];
    }
    __device__ static void store(void* base, size_t index, float v)
    {
        if constexpr (BF16)
            static_cast<uint16_t*>(base)[index] = static_cast<uint16_t>(float_to_bf16_bits(v));
        else
            static_cast<float*>(base)[index] = v;
    }
    // An element of a 16-byte vector, widened to FP32.
    __device__ static float elem(const u32x4& v, int j)
    {
        if constexpr (BF16)
            return __uint_as_float((j & 1) ? (v[j >> 1] & 0xffff0000u) : (v[j >> 1] << 16));
        else
            return __uint_as_float(v[j]);
    }
    // The 32-bit payload of a rounded value in an exchange word.
    __device__ static uint32_t payload(float rounded)
    {
        if constexpr (BF16)
            return float_to_bf16_bits(rounded);
        else
            return __float_as_uint(rounded);
    }
    __device__ static float from_payload(uint32_t p)
    {
        if constexpr (BF16)
            return bf16_bits_to_float(p & 0xffffu);
        else
            return __uint_as_float(p);
    }
};

__device__ inline u32x4 load_weights(const void* p) { return __builtin_nontemporal_load(static_cast<const u32x4*>(p)); }

__device__ inline void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Device-coherent 32/64-bit accesses (global_load/store ... sc1).
__device__ inline uint64_t coherent_load64(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_store64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float coherent_loadf(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_storef(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline uint32_t coherent_load32(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_store32(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_store16(uint16_t* p, uint16_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// 16-byte device-coherent load of K/V rows through a buffer resource (sc1).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ inline u32x4 coherent_load128(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset)
{
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 16);
}

__device__ inline float wave_sum(float v, int width)
{
    for (int offset = width >> 1; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset);
    return v;
}
__device__ inline float wave_max(float v, int width)
{
    for (int offset = width >> 1; offset > 0; offset >>= 1)
        v = fmaxf(v, __shfl_xor(v, offset));
    return v;
}

// ---------------------------------------------------------------- launch record

template <bool BF16>
struct Launch {
    const ti_task_record* instructions;
    const ti_worker_task_range* streams;
    ti_layer_layout layout;
    ti_model_shape shape;
    ti_numeric_config numeric;
    ti_stack_config stack;
    const float* rope;
    const void* weights;
    void* input;
    void* output;
    void* scratch;
    void* kv;
    float* partials;
    float* logits;
    float* block_trace;
    float* ffn_trace;
    ti_candidate* selection_out;
    uint64_t* timeline;
    uint64_t* exchange;
    ExchangeLayout xl;
    uint32_t epoch;
    int position;
    int steps;
    ti_token_id token_id;
    const ti_token_id* device_tokens;
    ti_selection selection;
    int selection_slots;
    int workers;

    __device__ size_t kv_width() const { return static_cast<size_t>(shape.kv_heads) * shape.head_dim; }
    __device__ const void* layer_weight(int layer, uint32_t offset) const
    {
        const size_t element = static_cast<size_t>(stack.layer_weights_offset) +
                               static_cast<size_t>(layer) * stack.layer_weight_stride + offset;
        return static_cast<const char*>(weights) + element * Num<BF16>::kBytes;
    }
    __device__ const void* stack_weight(size_t element) const
    {
        return static_cast<const char*>(weights) + element * Num<BF16>::kBytes;
    }
    __device__ void* cache(int layer, uint32_t offset) const
    {
        const size_t element = static_cast<size_t>(layer) * stack.layer_kv_stride + offset;
        return static_cast<char*>(kv) + element * Num<BF16>::kBytes;
    }
    // Epoch of an exchange written at (step, layer, phase); stages use layer == layers.
    __device__ uint32_t epoch_of(int step, int layer, int phase) const
    {
        return epoch + static_cast<uint32_t>(step) * epochs_per_step(stack.layers) +
               static_cast<uint32_t>(layer) * kPhases + static_cast<uint32_t>(phase) + 1u;
    }
};

struct Shared {
    float vec[kMaxHidden];          // a task's input vector (normalized), FP32 values of Scalar
    float region[kRegionFloats];    // scores/probabilities, reductions, FFN product
    float small[kMaxTaskRows];      // reductions over waves, softmax statistics, residual rows
    float rotated[(kMaxGroup + 1) * kMaxHeadDim];
    float vcur[kMaxHeadDim];
    ti_candidate candidates[kWaves];
    int flag;
    int aborted;
    int token;
    uint64_t mark_read;   // timeline: when the instruction's first exchange read returned
    uint64_t mark_ready;  // timeline: when its last exchange wait ended
};

// ---------------------------------------------------------------- exchange polling

// Reads `count` (at most kMaxHidden) exchange words from `src` until each carries `epoch`
// and hands each payload to `sink(index, payload)`.  Block-wide: every thread must call it.
// The first read is optimistic (one coherent round trip when the producers are done).  If any
// word is still missing, only wave 0 keeps polling, one "witness" word every `stride` words
// (every producer writes a run of at least `stride` words), with a back-off; the block then
// re-reads what was missing.  Polling the whole vector from every thread of every worker
// floods the few memory channels that hold it and slows the producers themselves.
template <typename Sink>
__device__ __forceinline__ void poll_words(const uint64_t* src, int count, int stride, uint32_t epoch, uint64_t* exchange,
                                          const ExchangeLayout& xl, Shared& sh, Sink sink)
{
    constexpr int kBatch = (kMaxHidden + kThreads - 1) / kThreads;
    const uint64_t done_word = static_cast<uint64_t>(epoch) << 32;
    uint64_t w[kBatch];
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
        const int index = k * kThreads + static_cast<int>(threadIdx.x);
        w[k] = index < count ? coherent_load64(src + index) : done_word;
        ok &= static_cast<uint32_t>(w[k] >> 32) == epoch;
    }
    const bool all_present = __syncthreads_and(ok);
    if (threadIdx.x == 0 && sh.mark_read == 0)
        sh.mark_read = __builtin_amdgcn_s_memrealtime();
    if (!all_present) {
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            uint32_t spins = 0;
            while (!sh.aborted) {
                bool mine = true;
                for (int j = lane; j * stride < count; j += 64)
                    mine &= static_cast<uint32_t>(coherent_load64(src + j * stride) >> 32) == epoch;
                if (lane == 0)
                    mine &= static_cast<uint32_t>(coherent_load64(src + count - 1) >> 32) == epoch;
                if (__all(mine))
                    break;
                __builtin_amdgcn_s_sleep(2);
                if ((++spins & 63u) == 0 && lane == 0 &&
                    (coherent_load64(exchange + xl.control) != 0 || spins > kSpinLimit)) {
                    sh.aborted = 1;
                    coherent_store64(exchange + xl.control, 1);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int index = k * kThreads + static_cast<int>(threadIdx.x);
            uint32_t spins = 0;
            while (static_cast<uint32_t>(w[k] >> 32) != epoch && !sh.aborted) {
                w[k] = coherent_load64(src + index);
                if (static_cast<uint32_t>(w[k] >> 32) == epoch)
                    break;
                __builtin_amdgcn_s_sleep(2);
                if ((++spins & 63u) == 0 && (coherent_load64(exchange + xl.control) != 0 || spins > kSpinLimit)) {
                    sh.aborted = 1;
                    coherent_store64(exchange + xl.control, 1);
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
        const int index = k * kThreads + static_cast<int>(threadIdx.x);
        if (index < count)
            sink(index, static_cast<uint32_t>(w[k]));
    }
    if (threadIdx.x == 0)
        sh.mark_ready = __builtin_amdgcn_s_memrealtime();
}

// Witness spacing of an exchange written by row tasks that split `n` rows over `workers`
// (plan_core.py:275-278: every task gets at least n / workers rows).
__device__ inline int row_stride(int n, int workers) { return n >= workers ? n / workers : 1; }

template <bool BF16>
__device__ inline void publish(uint64_t* dst, int index, float rounded, uint32_t epoch)
{
    coherent_store64(dst + index, (static_cast<uint64_t>(epoch) << 32) | Num<BF16>::payload(rounded));
}

// ---------------------------------------------------------------- layer input

// The hidden state a layer reads: the token's embedding row for a stack's first layer, the
// host-written input of a block package, or the previous layer's exchanged output.
template <bool BF16>
__device__ __forceinline__ void load_hidden(const Launch<BF16>& L, int layer, int step, ti_token_id token, float* dst, Shared& sh)
{
    const int d = L.shape.hidden_size;
    if (layer == 0) {
        if (L.stack.full_stack) {
            const void* row = L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) + static_cast<size_t>(token) * d);
            for (int i = threadIdx.x; i < d; i += kThreads)
                dst[i] = Num<BF16>::load(row, i);
        } else {
            for (int i = threadIdx.x; i < d; i += kThreads)
                dst[i] = Num<BF16>::load(L.input, i);
        }
        return;
    }
    poll_words(L.exchange + L.xl.hidden(layer % 2), d, row_stride(d, L.workers), L.epoch_of(step, layer - 1, kPhaseY),
               L.exchange, L.xl, sh, [&](int i, uint32_t p) { dst[i] = Num<BF16>::from_payload(p); });
}

// One element of a layer's input, for residual additions.
template <bool BF16>
__device__ __forceinline__ float hidden_element(const Launch<BF16>& L, int layer, int step, ti_token_id token, int i, Shared& sh)
{
    if (layer == 0) {
        if (L.stack.full_stack)
            return Num<BF16>::load(L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) + static_cast<size_t>(token) * L.shape.hidden_size), i);
        return Num<BF16>::load(L.input, i);
    }
    const uint64_t* src = L.exchange + L.xl.hidden(layer % 2) + i;
    const uint32_t epoch = L.epoch_of(step, layer - 1, kPhaseY);
    uint64_t w = coherent_load64(src);
    uint32_t spins = 0;
    while (static_cast<uint32_t>(w >> 32) != epoch && !sh.aborted) {
        __builtin_amdgcn_s_sleep(1);
        w = coherent_load64(src);
        if (++spins > kSpinLimit) {
            sh.aborted = 1;
            coherent_store64(L.exchange + L.xl.control, 1);
        }
    }
    return Num<BF16>::from_payload(static_cast<uint32_t>(w));
}

// ---------------------------------------------------------------- RMSNorm (ops.cuh:145-219)

// In place: v[i] = round(round(v[i] * inv_rms) * scale[i]) for bf16, v[i] * inv_rms * scale[i]
// for fp32 (decoder_reference.py:183-187, decoder_stack.py:126-132).  The statistic is FP32.
template <bool BF16>
__device__ __forceinline__ void rms_norm_lds(float* v, int d, const void* scale, float eps, Shared& sh)
{
    float sum = 0.0f;
    for (int i = threadIdx.x; i < d; i += kThreads)
        sum += v[i] * v[i];
    sum = wave_sum(sum, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0)
        sh.small[wave] = sum;
    __syncthreads();
    float total = 0.0f;
    for (int w = 0; w < kWaves; ++w)
        total += sh.small[w];
    const float inv = 1.0f / sqrtf(total / static_cast<float>(d) + eps);
    for (int i = threadIdx.x; i < d; i += kThreads)
        v[i] = Num<BF16>::round(Num<BF16>::round(v[i] * inv) * Num<BF16>::load(scale, i));
    __syncthreads();
}

// ---------------------------------------------------------------- GEMV over rows

// Dot products of rows [r0, r1) of NM row-major matrices sharing a shape (row length `cols`,
// row stride `stride` elements) with the FP32 vector u (LDS).  One group of
// LR = min(64, vectors per row) lanes owns a row of every matrix; lanes hold their slice of u
// in registers.  `prepare` runs once, block-wide, after the first pass's weight loads are
// issued and before u is read: it polls the inputs and writes u, so weight latency overlaps
// the wait.  emit(row, dots) runs in the group's lane 0 with one dot per matrix.
template <bool BF16, int VPL, int NM, typename Prepare, typename Emit>
__device__ __forceinline__ void gemv_rows(const void* const (&matrices)[NM], size_t stride, int r0, int r1, int cols,
                                         const float* u, Prepare prepare, Emit emit)
{
    using N = Num<BF16>;
    constexpr int PV = N::kPerVec;
    constexpr int kLoads = VPL * NM;
    const int nvec = cols / PV;
    const int LR = nvec < 64 ? nvec : 64;
    const int rows_per_wave = 64 / LR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LR, col = lane % LR;
    const size_t row_bytes = stride * N::kBytes;
    const int pass_rows = kWaves * rows_per_wave;

    auto row_of = [&](int pass) { return r0 + pass * pass_rows + wave * rows_per_wave + sub; };
    auto issue = [&](int row, u32x4* w) {
        const int safe = row < r1 ? row : r0;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const char* p = static_cast<const char*>(matrices[m]) + static_cast<size_t>(safe) * row_bytes +
                            static_cast<size_t>(col) * 16;
#pragma unroll
            for (int k = 0; k < VPL; ++k)
                w[m * VPL + k] = load_weights(p + static_cast<size_t>(k) * LR * 16);
        }
    };

    u32x4 w0[kLoads];
    if (r0 + wave * rows_per_wave < r1)
        issue(row_of(0), w0);
    prepare();
    float ur[VPL][PV];
#pragma unroll
    for (int k = 0; k < VPL; ++k)
#pragma unroll
        for (int j = 0; j < PV; ++j)
            ur[k][j] = u[(col + k * LR) * PV + j];

    auto finish = [&](int row, const u32x4* w) {
        float dots[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int j = 0; j < PV; ++j)
                    acc += N::elem(w[m * VPL + k], j) * ur[k][j];
            dots[m] = wave_sum(acc, LR);
        }
        if (row < r1 && col == 0)
            emit(row, dots);
    };

    if (r0 + wave * rows_per_wave >= r1)
        return;
    int pass = 0;
    if constexpr (kLoads <= 8) {
        // Two passes in flight: issue pass p + 1 before reducing pass p.
        while (true) {
            const bool more = r0 + (pass + 1) * pass_rows + wave * rows_per_wave < r1;
            u32x4 w1[kLoads];
            if (more)
                issue(row_of(pass + 1), w1);
            finish(row_of(pass), w0);
            if (!more)
                break;
#pragma unroll
            for (int k = 0; k < kLoads; ++k)
                w0[k] = w1[k];
            ++pass;
        }
    } else {
        while (true) {
            finish(row_of(pass), w0);
            ++pass;
            if (r0 + pass * pass_rows + wave * rows_per_wave >= r1)
                break;
            issue(row_of(pass), w0);
        }
    }
}

// Runtime vectors-per-lane dispatch (the loader admits rows of 1..512 16-byte vectors).
template <bool BF16, int NM, typename Prepare, typename Emit>
__device__ __forceinline__ void gemv_n(const void* const (&matrices)[NM], size_t stride, int r0, int r1, int cols,
                                      const float* u, Prepare prepare, Emit emit)
{
    const int nvec = cols / Num<BF16>::kPerVec;
    const int vpl = nvec <= 64 ? 1 : nvec / 64;
    switch (vpl) {
    case 1: gemv_rows<BF16, 1, NM>(matrices, stride, r0, r1, cols, u, prepare, emit); break;
    case 2: gemv_rows<BF16, 2, NM>(matrices, stride, r0, r1, cols, u, prepare, emit); break;
    case 4: gemv_rows<BF16, 4, NM>(matrices, stride, r0, r1, cols, u, prepare, emit); break;
    default: gemv_rows<BF16, 8, NM>(matrices, stride, r0, r1, cols, u, prepare, emit); break;
    }
}

template <bool BF16, typename Prepare, typename Emit>
__device__ __forceinline__ void gemv(const void* matrix, size_t stride, int r0, int r1, int cols, const float* u, Prepare prepare,
                                    Emit emit)
{
    const void* const matrices[1] = {matrix};
    gemv_n<BF16, 1>(matrices, stride, r0, r1, cols, u, prepare, [&](int row, const float* dots) { emit(row, dots[0]); });
}

// ---------------------------------------------------------------- operations

// [Q; K; V] rows of the normalized layer input (ops.cuh:266-289): Q and K round to Scalar and
// are published unrotated; V rows also go to the cache row of the current position.
template <bool BF16>
__device__ __forceinline__ void op_qkv(const Launch<BF16>& L, const ti_task_record& t, int step, ti_token_id token, Shared& sh)
{
    const int d = L.shape.hidden_size;
    const int kvw = static_cast<int>(L.kv_width());
    const int layer = static_cast<int>(t.layer);
    const int position = L.position + step;
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseQKV);
    const void* norm = L.layer_weight(layer, L.layout.attn_norm);
    auto prepare = [&]() {
        load_hidden(L, layer, step, token, sh.vec, sh);
        __syncthreads();
        rms_norm_lds<BF16>(sh.vec, d, norm, L.numeric.rms_norm_eps, sh);
    };
    auto emit = [&](int row, float dot) {
        const float value = Num<BF16>::round(dot);
        if (row >= d + kvw) {
            // V rows also go to the cache row of the current position, before publication.
            void* cache = L.cache(layer, L.layout.value);
            const size_t index = static_cast<size_t>(position) * kvw + (row - d - kvw);
            if constexpr (BF16)
                coherent_store16(static_cast<uint16_t*>(cache) + index, static_cast<uint16_t>(float_to_bf16_bits(value)));
            else
                coherent_storef(static_cast<float*>(cache) + index, value);
            wait_stores();
        }
        publish<BF16>(L.exchange + L.xl.qkv, qkv_word(row, L.shape), value, epoch);
    };
    // Rows may span Wq, Wk and Wv; run each matrix's part (they are separate regions).
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    struct Part { uint32_t offset; int first, last, shift; };
    Part parts[3] = {{L.layout.Wq, 0, d, 0}, {L.layout.Wk, d, d + kvw, d}, {L.layout.Wv, d + kvw, d + 2 * kvw, d + kvw}};
    bool prepared = false;
    for (int p = 0; p < 3; ++p) {
        const int lo = begin > parts[p].first ? begin : parts[p].first;
        const int hi = end < parts[p].last ? end : parts[p].last;
        if (lo >= hi)
            continue;
        const void* m = L.layer_weight(layer, parts[p].offset);
        const int shift = parts[p].shift;
        if (!prepared) {
            gemv<BF16>(m, d, lo - shift, hi - shift, d, sh.vec, prepare, [&](int row, float dot) { emit(row + shift, dot); });
            prepared = true;
        } else {
            gemv<BF16>(m, d, lo - shift, hi - shift, d, sh.vec, []() {}, [&](int row, float dot) { emit(row + shift, dot); });
        }
    }
}

__device__ inline int active_chunks(int position, const ti_model_shape& s)
{
    const int length = position + 1;
    if (length <= s.attention_fused_steps)
        return 1;
    const int chunks = (length + s.attention_chunk_steps - 1) / s.attention_chunk_steps;
    return chunks > 2 ? chunks : 2;
}

// Rotate one split-half pair; cos/sin and products round before the sum (ops.cuh:125-140).
template <bool BF16>
__device__ inline void rope_pair(const float* src, float* dst, int pair, int half, float angle)
{
    const float c = Num<BF16>::round(cosf(angle));
    const float s = Num<BF16>::round(sinf(angle));
    const float a = src[pair], b = src[pair + half];
    dst[pair] = Num<BF16>::round(Num<BF16>::round(a * c) - Num<BF16>::round(b * s));
    dst[pair + half] = Num<BF16>::round(Num<BF16>::round(b * c) + Num<BF16>::round(a * s));
}

// One K/V head and context chunk of decode attention (ops.cuh:574-673, re-designed):
// RoPE of the group's query heads and current K; chunk 0 stores rotated K into the cache.
// One active chunk (a prefix of at most attention_fused_steps): scores, exact softmax,
// probabilities rounded to Scalar, P*V, published as the group's attention output.
// Several chunks: each chunk keeps (max, sum of exp, unnormalized P*V) in FP32; the chunk
// that finishes last (an atomic count per head group) merges all of them and publishes.
// Cached K/V rows never change during a token, so the first block of them is loaded before
// the task waits for this token's Q/K/V.
template <bool BF16, int MG>
__device__ __forceinline__ void op_attention(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    constexpr int PV = N::kPerVec;
    const ti_model_shape& s = L.shape;
    const int position = L.position + step;
    const int chunks = active_chunks(position, s);
    const int chunk = static_cast<int>(t.chunk);
    if (chunk >= chunks)
        return;
    const int layer = static_cast<int>(t.layer);
    const int kv_head = static_cast<int>(t.kv_head);
    const int dh = s.head_dim;
    const int group = s.query_heads / s.kv_heads;
    const int first_head = kv_head * group;
    const int kvw = static_cast<int>(L.kv_width());
    const int length = position + 1;
    const int begin = static_cast<int>(static_cast<int64_t>(length) * chunk / chunks);
    const int end = static_cast<int>(static_cast<int64_t>(length) * (chunk + 1) / chunks);
    const int span = end - begin;

    const int LRk = dh / PV;                 // lanes per K/V row (power of two, <= 16)
    const int rows_per_wave = 64 / LRk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LRk, col = lane % LRk;
    const int block_rows = kWaves * rows_per_wave;
    void* key_cache = L.cache(layer, L.layout.key);
    const void* value_cache = L.cache(layer, L.layout.value);
    const uint32_t layer_kv_bytes = static_cast<uint32_t>(static_cast<size_t>(s.max_context) * kvw * N::kBytes);
    const __amdgpu_buffer_rsrc_t krsrc = make_rsrc(key_cache, layer_kv_bytes);
    const __amdgpu_buffer_rsrc_t vrsrc = make_rsrc(value_cache, layer_kv_bytes);
    auto row_time = [&](int first, int u) { return first + u * block_rows + wave * rows_per_wave + sub; };
    auto load_rows = [&](__amdgpu_buffer_rsrc_t rsrc, int first, u32x4* raw) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int time = row_time(first, u);
            const bool cached = time < end && time < position;
            const uint32_t offset =
                static_cast<uint32_t>((static_cast<size_t>(cached ? time : 0) * kvw + kv_head * dh + col * PV) * N::kBytes);
            raw[u] = cached ? coherent_load128(rsrc, offset) : u32x4{0, 0, 0, 0};
        }
    };
    u32x4 kfirst[2], vfirst[2];
    load_rows(krsrc, begin, kfirst);
    load_rows(vrsrc, begin, vfirst);

    // This token's Q heads, K and V of the head group: one packed exchange block.
    const int block = (group + 2) * dh;
    float* incoming = sh.region;  // [group][dh] Q, [dh] K, [dh] V
    poll_words(L.exchange + L.xl.qkv + static_cast<size_t>(kv_head) * block, block,
               row_stride(s.hidden_size + 2 * kvw, L.workers), L.epoch_of(step, layer, kPhaseQKV), L.exchange, L.xl, sh,
               [&](int i, uint32_t p) { incoming[i] = N::from_payload(p); });
    __syncthreads();
    const int half = dh / 2;
    for (int index = threadIdx.x; index < (group + 1) * half; index += kThreads) {
        const int head = index / half, pair = index - head * half;
        const float angle = static_cast<float>(position) * L.rope[pair];
        rope_pair<BF16>(incoming + head * dh, sh.rotated + head * dh, pair, half, angle);
    }
    for (int index = threadIdx.x; index < dh; index += kThreads)
        sh.vcur[index] = incoming[(group + 1) * dh + index];
    __syncthreads();
    if (chunk == 0) {
        for (int index = threadIdx.x; index < (group + 1) * dh; index += kThreads) {
            const float value = sh.rotated[index];
            if (index < group * dh) {
                N::store(L.scratch, L.layout.q_rot + first_head * dh + index, value);
            } else {
                const size_t e = static_cast<size_t>(position) * kvw + kv_head * dh + (index - group * dh);
                if constexpr (BF16)
                    coherent_store16(static_cast<uint16_t*>(key_cache) + e, static_cast<uint16_t>(float_to_bf16_bits(value)));
                else
                    coherent_storef(static_cast<float*>(key_cache) + e, value);
            }
        }
    }

    // Scores of rows [begin, end): LRk lanes hold one 16-byte slice of a K row each.
    const float scale = 1.0f / sqrtf(static_cast<float>(dh));
    const float divisor = sqrtf(static_cast<float>(dh));
    float* scores = sh.region;  // [group][span] (the incoming block is consumed)
    float qreg[MG][PV];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int j = 0; j < PV; ++j)
            qreg[g][j] = g < group ? sh.rotated[g * dh + col * PV + j] : 0.0f;
    float kcur[PV];
#pragma unroll
    for (int j = 0; j < PV; ++j)
        kcur[j] = sh.rotated[group * dh + col * PV + j];
    __syncthreads();  // incoming is dead; scores may overwrite the region
    for (int first = begin; first < end; first += 2 * block_rows) {
        u32x4 raw[2];
        if (first == begin) {
            raw[0] = kfirst[0];
            raw[1] = kfirst[1];
        } else {
            load_rows(krsrc, first, raw);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int time = row_time(first, u);
            const bool current = time == position;
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                float dot = 0.0f;
#pragma unroll
                for (int j = 0; j < PV; ++j)
                    dot += (current ? kcur[j] : N::elem(raw[u], j)) * qreg[g][j];
                dot = wave_sum(dot, LRk);
                if (g < group && col == 0 && time < end) {
                    const float rounded = N::round(dot);
                    scores[g * span + time - begin] = BF16 ? N::round(rounded * scale) : rounded / divisor;
                }
            }
        }
    }
    __syncthreads();

    // Softmax statistics per head: one wave per head.
    float* stat_max = sh.small;
    float* stat_sum = sh.small + kMaxGroup;
    if (wave < group) {
        float m = -INFINITY;
        for (int i = lane; i < span; i += 64)
            m = fmaxf(m, scores[wave * span + i]);
        m = wave_max(m, 64);
        float sum = 0.0f;
        for (int i = lane; i < span; i += 64)
            sum += expf(scores[wave * span + i] - m);
        sum = wave_sum(sum, 64);
        if (lane == 0) {
            stat_max[wave] = m;
            stat_sum[wave] = sum;
        }
    }
    __syncthreads();
    const bool fused = chunks == 1;
    for (int index = threadIdx.x; index < group * span; index += kThreads) {
        const int g = index / span;
        const float e = expf(scores[index] - stat_max[g]);
        scores[index] = fused ? N::round(e / stat_sum[g]) : e;
    }
    __syncthreads();

    // P*V over rows [begin, end): each lane accumulates its slice for every head.
    float acc[MG][PV];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int j = 0; j < PV; ++j)
            acc[g][j] = 0.0f;
    for (int first = begin; first < end; first += 2 * block_rows) {
        u32x4 raw[2];
        if (first == begin) {
            raw[0] = vfirst[0];
            raw[1] = vfirst[1];
        } else {
            load_rows(vrsrc, first, raw);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int time = row_time(first, u);
            if (time >= end)
                continue;
            const bool current = time == position;
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                const float p = g < group ? scores[g * span + time - begin] : 0.0f;
#pragma unroll
                for (int j = 0; j < PV; ++j)
                    acc[g][j] += p * (current ? sh.vcur[col * PV + j] : N::elem(raw[u], j));
            }
        }
    }
    // Reduce over the rows a wave holds (lanes with equal col), then over waves.
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int j = 0; j < PV; ++j)
            for (int offset = LRk; offset < 64; offset <<= 1)
                acc[g][j] += __shfl_xor(acc[g][j], offset);
    __syncthreads();  // probabilities are dead
    float* reduction = sh.region;  // [wave][group][dh]
    if (sub == 0)
#pragma unroll
        for (int g = 0; g < MG; ++g)
            if (g < group)
#pragma unroll
                for (int j = 0; j < PV; ++j)
                    reduction[(wave * group + g) * dh + col * PV + j] = acc[g][j];
    __syncthreads();
    float* out = sh.region + kWaves * group * dh;  // [group][dh] FP32 output of this chunk
    for (int index = threadIdx.x; index < group * dh; index += kThreads) {
        float total = 0.0f;
        for (int w = 0; w < kWaves; ++w)
            total += reduction[w * group * dh + index];
        out[index] = total;
    }
    __syncthreads();

    const uint32_t out_epoch = L.epoch_of(step, layer, kPhaseAttn);
    uint64_t* attn = L.exchange + L.xl.attn + first_head * dh;
    if (fused) {
        wait_stores();  // the K row is in the cache before anyone sees this output
        for (int index = threadIdx.x; index < group * dh; index += kThreads)
            publish<BF16>(attn, index, N::round(out[index]), out_epoch);
        return;
    }
    // Partial of this chunk: [chunk][head][dh] then statistics [chunk][head][2].
    float* partials = L.partials;
    float* stats_base = L.partials + static_cast<size_t>(s.attention_chunks) * s.query_heads * dh;
    float* partial = partials + (static_cast<size_t>(chunk) * s.query_heads + first_head) * dh;
    float* stats = stats_base + (static_cast<size_t>(chunk) * s.query_heads + first_head) * 2;
    for (int index = threadIdx.x; index < group * dh; index += kThreads)
        coherent_storef(partial + index, out[index]);
    if (threadIdx.x < group) {
        coherent_storef(stats + threadIdx.x * 2, stat_max[threadIdx.x]);
        coherent_storef(stats + threadIdx.x * 2 + 1, stat_sum[threadIdx.x]);
    }
    wait_stores();
    __syncthreads();
    uint64_t* counter = L.exchange + L.xl.counters + layer * s.kv_heads + kv_head;
    if (threadIdx.x == 0) {
        const uint64_t before = __hip_atomic_fetch_add(counter, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.flag = before == static_cast<uint64_t>(chunks - 1);
    }
    __syncthreads();
    if (!sh.flag)
        return;
    // Last chunk of this head group: merge every chunk in chunk order.
    if (threadIdx.x < group) {
        const int head = first_head + threadIdx.x;
        float m = -INFINITY;
        for (int c = 0; c < chunks; ++c)
            m = fmaxf(m, coherent_loadf(stats_base + (static_cast<size_t>(c) * s.query_heads + head) * 2));
        float sum = 0.0f;
        for (int c = 0; c < chunks; ++c) {
            const float* st = stats_base + (static_cast<size_t>(c) * s.query_heads + head) * 2;
            sum += coherent_loadf(st + 1) * expf(coherent_loadf(st) - m);
        }
        sh.small[2 * kMaxGroup + threadIdx.x] = m;
        sh.small[3 * kMaxGroup + threadIdx.x] = sum;
    }
    __syncthreads();
    for (int index = threadIdx.x; index < group * dh; index += kThreads) {
        const int g = index / dh;
        const int head = first_head + g;
        const float m = sh.small[2 * kMaxGroup + g];
        float total = 0.0f;
        for (int c = 0; c < chunks; ++c) {
            const float* st = stats_base + (static_cast<size_t>(c) * s.query_heads + head) * 2;
            total += coherent_loadf(partials + (static_cast<size_t>(c) * s.query_heads + first_head) * dh + index) *
                     expf(coherent_loadf(st) - m);
        }
        out[index] = total / sh.small[3 * kMaxGroup + g];
    }
    if (threadIdx.x == 0)
        coherent_store64(counter, 0);
    wait_stores();
    __syncthreads();
    for (int index = threadIdx.x; index < group * dh; index += kThreads)
        publish<BF16>(attn, index, N::round(out[index]), out_epoch);
}

// Wo rows plus the residual (ops.cuh:718-734): r = round(round(Wo a) + x).
template <bool BF16>
__device__ __forceinline__ void op_output_projection(const Launch<BF16>& L, const ti_task_record& t, int step, ti_token_id token, Shared& sh)
{
    const int d = L.shape.hidden_size;
    const int layer = static_cast<int>(t.layer);
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseR);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    float* residual = sh.small;  // rows [begin, end)
    auto prepare = [&]() {
        poll_words(L.exchange + L.xl.attn, d, (L.shape.query_heads / L.shape.kv_heads) * L.shape.head_dim,
                   L.epoch_of(step, layer, kPhaseAttn), L.exchange, L.xl, sh,
                   [&](int i, uint32_t p) { sh.vec[i] = Num<BF16>::from_payload(p); });
        for (int i = begin + static_cast<int>(threadIdx.x); i < end; i += kThreads)
            residual[i - begin] = hidden_element(L, layer, step, token, i, sh);
        __syncthreads();
        if (begin == 0)
            for (int i = threadIdx.x; i < d; i += kThreads)
                Num<BF16>::store(L.scratch, L.layout.attention + i, sh.vec[i]);
    };
    gemv<BF16>(L.layer_weight(layer, L.layout.Wo), d, begin, end, d, sh.vec, prepare, [&](int row, float dot) {
        const float r = Num<BF16>::round(Num<BF16>::round(dot) + residual[row - begin]);
        Num<BF16>::store(L.scratch, L.layout.r + row, r);
        publish<BF16>(L.exchange + L.xl.r, row, r, epoch);
    });
}

// One FFN product chunk (ops.cuh:739-813): z = RMSNorm(r); p = round(round(silu(round(gate)))
// * round(up)) for rows [begin, end); then the chunk's FP32 down partial over every output,
// published for the reduce wave.  Wdown is stored transposed, [intermediate, hidden].
template <bool BF16>
__device__ __forceinline__ void op_ffn(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    const int d = L.shape.hidden_size;
    const int layer = static_cast<int>(t.layer);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const int rows = end - begin;
    float* product = sh.region;             // [rows]
    float* gate = sh.region + rows;         // [rows]
    float* up = sh.region + 2 * rows;       // [rows]
    const void* norm = L.layer_weight(layer, L.layout.ffn_norm);
    auto prepare = [&]() {
        poll_words(L.exchange + L.xl.r, d, row_stride(d, L.workers), L.epoch_of(step, layer, kPhaseR), L.exchange, L.xl, sh,
                   [&](int i, uint32_t p) { sh.vec[i] = N::from_payload(p); });
        __syncthreads();
        rms_norm_lds<BF16>(sh.vec, d, norm, L.numeric.rms_norm_eps, sh);
    };
    // Gate and up rows in one pass (all their loads issue before the input wait).
    const void* const gate_up[2] = {L.layer_weight(layer, L.layout.Wgate), L.layer_weight(layer, L.layout.Wup)};
    gemv_n<BF16, 2>(gate_up, d, begin, end, d, sh.vec, prepare, [&](int row, const float* dots) {
        gate[row - begin] = N::round(dots[0]);
        up[row - begin] = N::round(dots[1]);
    });
    __syncthreads();
    for (int i = threadIdx.x; i < rows; i += kThreads) {
        const float g = gate[i];
        const float silu = N::round(g / (1.0f + expf(-g)));
        const float p = N::round(silu * up[i]);
        product[i] = p;
        N::store(L.scratch, L.layout.product + begin + i, p);
    }
    __syncthreads();
    // Down partial: a thread owns one 16-byte column slice of Wdown^T and a residue class of rows.
    constexpr int PV = N::kPerVec;
    const int nvec = d / PV;
    const int groups = kThreads / nvec;  // >= 1 (the loader bounds hidden_size)
    const int col = threadIdx.x % nvec, grp = threadIdx.x / nvec;
    float acc[PV];
#pragma unroll
    for (int j = 0; j < PV; ++j)
        acc[j] = 0.0f;
    const char* wd = static_cast<const char*>(L.layer_weight(layer, L.layout.Wdown));
    if (grp < groups) {
        int i = grp;
        for (; i + groups < rows; i += 2 * groups) {
            const u32x4 a = load_weights(wd + (static_cast<size_t>(begin + i) * d + col * PV) * N::kBytes);
            const u32x4 b = load_weights(wd + (static_cast<size_t>(begin + i + groups) * d + col * PV) * N::kBytes);
            const float pa = product[i], pb = product[i + groups];
#pragma unroll
            for (int j = 0; j < PV; ++j)
                acc[j] += N::elem(a, j) * pa;
#pragma unroll
            for (int j = 0; j < PV; ++j)
                acc[j] += N::elem(b, j) * pb;
        }
        for (; i < rows; i += groups) {
            const u32x4 a = load_weights(wd + (static_cast<size_t>(begin + i) * d + col * PV) * N::kBytes);
            const float pa = product[i];
#pragma unroll
            for (int j = 0; j < PV; ++j)
                acc[j] += N::elem(a, j) * pa;
        }
    }
    __syncthreads();  // product is dead
    float* reduction = sh.region;  // [groups][d]
    if (grp < groups)
#pragma unroll
        for (int j = 0; j < PV; ++j)
            reduction[grp * d + col * PV + j] = acc[j];
    __syncthreads();
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseFfn);
    uint64_t* partials = L.exchange + L.xl.ffn + static_cast<size_t>(t.chunk) * d;
    for (int i = threadIdx.x; i < d; i += kThreads) {
        float total = 0.0f;
        for (int g = 0; g < groups; ++g)
            total += reduction[g * d + i];
        coherent_store64(partials + i, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(total));
    }
}

// y rows: the chunks' FP32 down partials summed, rounded before the residual (ops.cuh:820-838).
template <bool BF16>
__device__ __forceinline__ void op_ffn_reduce(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    const ti_model_shape& s = L.shape;
    const int d = s.hidden_size;
    const int layer = static_cast<int>(t.layer);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const int rows = end - begin;
    const uint32_t in_epoch = L.epoch_of(step, layer, kPhaseFfn);
    // TPR lanes (a power of two <= 64) sum one row's chunks.
    int tpr = 64;
    while (tpr > 1 && tpr * rows > kThreads)
        tpr >>= 1;
    const int slots = kThreads / tpr;
    const int slot = threadIdx.x / tpr, lane = threadIdx.x % tpr;
    const uint64_t* base = L.exchange + L.xl.ffn;
    for (int first = 0; first < rows; first += slots) {
        const int row = begin + first + slot;
        float total = 0.0f;
        if (first + slot < rows) {
            for (int c = lane; c < s.ffn_chunks; c += tpr) {
                const uint64_t* src = base + static_cast<size_t>(c) * d + row;
                uint64_t w = coherent_load64(src);
                uint32_t spins = 0;
                while (static_cast<uint32_t>(w >> 32) != in_epoch && !sh.aborted) {
                    __builtin_amdgcn_s_sleep(1);
                    w = coherent_load64(src);
                    if (++spins > kSpinLimit) {
                        sh.aborted = 1;
                        coherent_store64(L.exchange + L.xl.control, 1);
                    }
                }
                total += __uint_as_float(static_cast<uint32_t>(w));
            }
        }
        total = wave_sum(total, tpr);
        float r = 0.0f;
        if (first + slot < rows && lane == 0) {
            const uint64_t* src = L.exchange + L.xl.r + row;
            const uint32_t r_epoch = L.epoch_of(step, layer, kPhaseR);
            uint64_t w = coherent_load64(src);
            uint32_t spins = 0;
            while (static_cast<uint32_t>(w >> 32) != r_epoch && !sh.aborted) {
                __builtin_amdgcn_s_sleep(1);
                w = coherent_load64(src);
                if (++spins > kSpinLimit) {
                    sh.aborted = 1;
                    coherent_store64(L.exchange + L.xl.control, 1);
                }
            }
            r = N::from_payload(static_cast<uint32_t>(w));
            const float projected = N::round(total);
            const float y = N::round(projected + r);
            void* hidden = (layer + 1) % 2 == 0 ? L.input : L.output;
            N::store(hidden, row, y);
            if (L.block_trace)
                L.block_trace[static_cast<size_t>(layer) * d + row] = y;
            if (L.ffn_trace)
                L.ffn_trace[row] = projected;
            publish<BF16>(L.exchange + L.xl.hidden((layer + 1) % 2), row, y, L.epoch_of(step, layer, kPhaseY));
        }
    }
}

__device__ inline void keep_better(ti_candidate& best, ti_candidate other)
{
    if (best.id == TI_NON_FINITE)
        return;
    if (other.id == TI_NON_FINITE || other.value > best.value || (other.value == best.value && other.id < best.id))
        best = other;
}

// Final norm of the last layer's output into sh.vec (decoder_stack.py:126-132).
template <bool BF16>
__device__ __forceinline__ void final_normalized(const Launch<BF16>& L, int step, Shared& sh)
{
    const int d = L.shape.hidden_size;
    const int layers = L.stack.layers;
    poll_words(L.exchange + L.xl.hidden(layers % 2), d, row_stride(d, L.workers), L.epoch_of(step, layers - 1, kPhaseY),
               L.exchange, L.xl, sh,
               [&](int i, uint32_t p) { sh.vec[i] = Num<BF16>::from_payload(p); });
    __syncthreads();
    rms_norm_lds<BF16>(sh.vec, d, L.stack_weight(L.stack.final_norm_offset), L.numeric.rms_norm_eps, sh);
}

template <bool BF16>
__device__ __forceinline__ void op_final_rms_norm(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    final_normalized(L, step, sh);
    void* hidden = (L.stack.layers + 1) % 2 == 0 ? L.input : L.output;
    for (int i = static_cast<int>(t.begin) + threadIdx.x; i < static_cast<int>(t.end); i += kThreads)
        Num<BF16>::store(hidden, i, sh.vec[i]);
}

// Vocabulary rows [begin, end) of the LM head and their greedy candidate (ops.cuh:851-889):
// logits round to Scalar, then widen; the largest value wins, the lowest ID among equals,
// and any non-finite logit makes the candidate kNonFinite.
template <bool BF16>
__device__ __forceinline__ void op_logits(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    const int d = L.shape.hidden_size;
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ti_candidate best{-INFINITY, 0x7fffffff};
    auto prepare = [&]() { final_normalized(L, step, sh); };
    gemv<BF16>(L.stack_weight(L.stack.lm_head_offset), d, begin, end, d, sh.vec, prepare, [&](int row, float dot) {
        const float logit = Num<BF16>::round(dot);
        L.logits[row] = logit;
        keep_better(best, {logit, isfinite(logit) ? row : TI_NON_FINITE});
    });
    // Lanes that emitted hold candidates; reduce the wave, then the block.
    for (int offset = 32; offset > 0; offset >>= 1) {
        ti_candidate other{__shfl_xor(best.value, offset), __shfl_xor(best.id, offset)};
        keep_better(best, other);
    }
    if (lane == 0)
        sh.candidates[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        ti_candidate result = sh.candidates[0];
        for (int w = 1; w < kWaves; ++w)
            keep_better(result, sh.candidates[w]);
        L.selection_out[t.chunk] = result;
        const uint32_t epoch = L.epoch_of(step, L.stack.layers, kPhaseCandidate);
        uint64_t* slot = L.exchange + L.xl.candidates + 2 * static_cast<size_t>(t.chunk);
        coherent_store64(slot, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(result.value));
        coherent_store64(slot + 1, (static_cast<uint64_t>(epoch) << 32) | static_cast<uint32_t>(result.id));
    }
}

// Greedy selection over every logits task's candidate (ops.cuh:895-911).  Step 0 of a launch
// reads the candidates a previous launch left (complete at the kernel boundary).
template <bool BF16>
__device__ __forceinline__ ti_token_id greedy(const Launch<BF16>& L, int step, Shared& sh)
{
    const int slots = L.selection_slots;
    if (threadIdx.x < 64) {
        ti_candidate best{-INFINITY, 0x7fffffff};
        const uint32_t epoch = step > 0 ? L.epoch_of(step - 1, L.stack.layers, kPhaseCandidate) : 0u;
        for (int slot = threadIdx.x; slot < slots; slot += 64) {
            const uint64_t* words = L.exchange + L.xl.candidates + 2 * static_cast<size_t>(slot);
            uint64_t a = coherent_load64(words), b = coherent_load64(words + 1);
            if (step > 0) {
                uint32_t spins = 0;
                while ((static_cast<uint32_t>(a >> 32) != epoch || static_cast<uint32_t>(b >> 32) != epoch) && !sh.aborted) {
                    __builtin_amdgcn_s_sleep(1);
                    a = coherent_load64(words);
                    b = coherent_load64(words + 1);
                    if (++spins > kSpinLimit) {
                        sh.aborted = 1;
                        coherent_store64(L.exchange + L.xl.control, 1);
                    }
                }
            }
            keep_better(best, {__uint_as_float(static_cast<uint32_t>(a)), static_cast<ti_token_id>(static_cast<uint32_t>(b))});
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            ti_candidate other{__shfl_xor(best.value, offset), __shfl_xor(best.id, offset)};
            keep_better(best, other);
        }
        if (threadIdx.x == 0)
            sh.token = best.id;
    }
    __syncthreads();
    return sh.token;
}

template <bool BF16>
__device__ __forceinline__ void record_choice(const Launch<BF16>& L, int step, ti_token_id token)
{
    int32_t* status = L.selection.status;
    if (token == TI_NON_FINITE) {
        status[TI_STATUS_ERROR] = TI_DEVICE_NON_FINITE;
    } else if (token < 0 || token >= L.stack.vocab_size) {
        status[TI_STATUS_ERROR] = TI_DEVICE_TOKEN_RANGE;
    } else {
        L.selection.generated[L.selection.first + step] = token;
        status[TI_STATUS_COUNT] = L.selection.first + step + 1;
        if (token == L.selection.eos_id)
            status[TI_STATUS_EOS] = 1;
    }
}

template <bool BF16>
__global__ __launch_bounds__(kThreads, 1) void decoder_worker(Launch<BF16> launch)
{
    __shared__ Shared sh;
    // The launch record lives in LDS: referenced from many inlined operations, a kernel
    // argument would be copied to scratch or spread over (and spilled from) SGPRs.
    __shared__ Launch<BF16> record;
    if (threadIdx.x == 0) {
        record = launch;
        sh.aborted = 0;
        sh.flag = 0;
    }
    __syncthreads();
    const Launch<BF16>& L = record;
    const bool generating = L.selection.generated != nullptr;
    if (generating && (L.selection.status[TI_STATUS_EOS] != 0 || L.selection.status[TI_STATUS_ERROR] != 0))
        return;
    const ti_worker_task_range stream = L.streams[blockIdx.x];
    for (int step = 0; step < L.steps; ++step) {
        ti_token_id token = L.token_id;
        if (generating) {
            token = greedy(L, step, sh);
            if (blockIdx.x == 0 && threadIdx.x == 0)
                record_choice(L, step, token);
        } else if (L.device_tokens != nullptr) {
            token = L.device_tokens[step];
        }
        if (L.stack.full_stack && (token < 0 || token >= L.stack.vocab_size))
            return;
        for (uint32_t index = stream.begin; index < stream.begin + stream.count; ++index) {
            const ti_task_record task = L.instructions[index];
            if (task.opcode == TI_OP_BARRIER)
                continue;  // waves synchronize through the exchange words
            // Optional timeline: 100 MHz device clock (s_memrealtime) at the start of every
            // instruction of the launch's last step, when its first exchange read returned,
            // when its inputs were complete, and at its end (diagnostic_context.cu:257-285).
            if (L.timeline && threadIdx.x == 0) {
                L.timeline[4 * static_cast<size_t>(index)] = __builtin_amdgcn_s_memrealtime();
                sh.mark_read = 0;
                sh.mark_ready = 0;
            }
            switch (task.opcode) {
            case TI_OP_QKV: op_qkv(L, task, step, token, sh); break;
            case TI_OP_ATTENTION_SCORES: op_attention<BF16, kMaxGroup>(L, task, step, sh); break;
            case TI_OP_OUTPUT_PROJECTION: op_output_projection(L, task, step, token, sh); break;
            case TI_OP_FFN: op_ffn(L, task, step, sh); break;
            case TI_OP_FFN_REDUCE: op_ffn_reduce(L, task, step, sh); break;
            case TI_OP_EMBEDDING: {
                const int d = L.shape.hidden_size;
                const void* row = L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) + static_cast<size_t>(token) * d);
                for (int i = static_cast<int>(task.begin) + threadIdx.x; i < static_cast<int>(task.end); i += kThreads)
                    Num<BF16>::store(L.input, i, Num<BF16>::load(row, i));
                break;
            }
            case TI_OP_FINAL_RMS_NORM: op_final_rms_norm(L, task, step, sh); break;
            case TI_OP_LOGITS: op_logits(L, task, step, sh); break;
            default: break;  // attention_values: no work in this worker
            }
            __syncthreads();
            if (L.timeline && threadIdx.x == 0) {
                L.timeline[4 * static_cast<size_t>(index) + 1] = sh.mark_read;
                L.timeline[4 * static_cast<size_t>(index) + 2] = sh.mark_ready;
                L.timeline[4 * static_cast<size_t>(index) + 3] = __builtin_amdgcn_s_memrealtime();
            }
        }
        if (sh.aborted) {
            if (threadIdx.x == 0 && generating && blockIdx.x == 0)
                L.selection.status[TI_STATUS_ERROR] = TI_DEVICE_SYNC_TIMEOUT;
            return;
        }
        if (generating && token == L.selection.eos_id)
            return;
    }
}

} // namespace

// ---------------------------------------------------------------- host side of the launch

namespace {
thread_local char g_message[512];
void set_message(const char* text)
{
    std::strncpy(g_message, text, sizeof g_message - 1);
    g_message[sizeof g_message - 1] = '\0';
}
int fail(int code, const char* text)
{
    set_message(text);
    return code;
}
int hip_fail(hipError_t e, const char* what)
{
    char buffer[400];
    std::snprintf(buffer, sizeof buffer, "%s: %s", what, hipGetErrorString(e));
    set_message(buffer);
    return TI_ERR_HIP;
}

template <bool BF16>
int launch_typed(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                 ti_token_input token, ti_selection selection)
{
    Launch<BF16> L{};
    L.instructions = p.instructions;
    L.streams = p.streams;
    L.layout = p.layout;
    L.shape = p.shape;
    L.numeric = p.numeric;
    L.stack = p.stack;
    L.rope = p.rotary_frequencies;
    L.weights = p.weights;
    L.input = b.input;
    L.output = b.output;
    L.scratch = b.scratch;
    L.kv = b.kv;
    L.partials = b.attention_partials;
    L.logits = b.logits;
    L.block_trace = b.block_trace;
    L.ffn_trace = b.ffn_trace;
    L.selection_out = b.selection;
    L.timeline = b.timeline;
    L.exchange = b.exchange;
    L.xl = exchange_layout(p.shape, p.stack.layers, p.selection_slots);
    L.epoch = b.epoch;
    L.position = position;
    L.steps = token.steps;
    L.token_id = token.immediate;
    L.device_tokens = token.ids;
    L.selection = selection;
    L.selection_slots = p.selection_slots;
    L.workers = p.workers;
    void* args[] = {&L};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&decoder_worker<BF16>), dim3(p.workers),
                                                    dim3(kThreads), args, 0, stream);
    if (e != hipSuccess)
        return hip_fail(e, "cooperative worker launch");
    return TI_OK;
}
} // namespace

const char* last_message() { return g_message; }
void set_last_message(const char* text) { set_message(text); }

template <bool BF16>
const void* worker_function() { return reinterpret_cast<const void*>(&decoder_worker<BF16>); }
template const void* worker_function<true>();
template const void* worker_function<false>();

} // namespace tiles

extern "C" int ti_enqueue_worker(void* stream, const ti_worker_program_view* program, const ti_worker_buffers* buffers,
                                 int32_t position, ti_token_input token, ti_selection selection)
{
    using namespace tiles;
    if (!program || !buffers)
        return fail(TI_ERR_INVALID_ARGUMENT, "null program or buffers");
    if (token.steps < 1 || token.steps > TI_MAX_LAUNCH_STEPS)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid worker launch step count");
    const std::string problem = check_launch_shape(*program, *buffers, position, token.steps);
    if (!problem.empty())
        return fail(TI_ERR_INVALID_ARGUMENT, problem.c_str());
    const hipStream_t s = static_cast<hipStream_t>(stream);
    return program->weight_dtype == TI_DTYPE_BFLOAT16 ? launch_typed<true>(s, *program, *buffers, position, token, selection)
                                                      : launch_typed<false>(s, *program, *buffers, position, token, selection);
}

// ---------------------------------------------------------------- diagnostics kernels (snapshot.cu:8-62)

namespace tiles {
namespace {
// Zeroes cache rows at and after `prefix` (or the generation's end) in every layer.
template <bool BF16>
__global__ void zero_unused_kv(void* kv, size_t count, int layers, int layer_stride, int width, int capacity,
                               int key_offset, int value_offset, int prefix, const int32_t* status)
{
    const int valid = status ? prefix + status[TI_STATUS_COUNT] : prefix;
    const size_t per_layer = static_cast<size_t>(capacity) * width;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < 2 * per_layer * layers;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t layer = i / (2 * per_layer);
        const size_t within = i % (2 * per_layer);
        const size_t table = within / per_layer;  // 0 = K, 1 = V
        const size_t element = within % per_layer;
        if (static_cast<int>(element / width) < valid)
            continue;
        const size_t index = layer * layer_stride + (table ? value_offset : key_offset) + element;
        if (index < count)
            Num<BF16>::store(kv, index, 0.0f);
    }
}

template <bool BF16>
__global__ void widen(const void* source, size_t count, float* destination)
{
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        destination[i] = Num<BF16>::load(source, i);
}
} // namespace

std::string check_shape(const ti_model_shape& s, int dtype)
{
    const int elem = dtype == TI_DTYPE_BFLOAT16 ? 2 : 4;
    auto power_of_two = [](long v) { return v > 0 && (v & (v - 1)) == 0; };
    if (s.hidden_size <= 0 || s.hidden_size > kMaxHidden)
        return "hidden size exceeds the compiled worker's LDS limit";
    const long hidden_vectors = static_cast<long>(s.hidden_size) * elem / 16;
    if (static_cast<long>(s.hidden_size) * elem % 16 != 0 || !(power_of_two(hidden_vectors) || hidden_vectors % 64 == 0) ||
        hidden_vectors > 8 * 64)
        return "hidden size unsupported by the compiled worker's 16-byte row lanes";
    if (s.head_dim > kMaxHeadDim || s.head_dim * elem % 16 != 0 || !power_of_two(s.head_dim * elem / 16))
        return "head_dim unsupported by the compiled worker";
    if (s.kv_heads <= 0 || s.query_heads % s.kv_heads != 0)
        return "invalid GQA grouping";
    const int group = s.query_heads / s.kv_heads;
    if (group > kMaxGroup || group * s.head_dim > kMaxGroupTimesHeadDim)
        return "query group exceeds the compiled worker's limits";
    if (static_cast<long>(s.attention_chunk_steps) * group * elem > kAttentionSharedBytes ||
        static_cast<long>(s.attention_chunk_steps) * group > kRegionFloats)
        return "attention chunk exceeds the compiled worker's LDS";
    if (s.intermediate_size % 2 != 0)
        return "odd intermediate size";
    return {};
}

std::string check_launch_shape(const ti_worker_program_view& p, const ti_worker_buffers& b, int position, int steps)
{
    std::string problem = check_shape(p.shape, p.weight_dtype);
    if (!problem.empty())
        return problem;
    if (!p.instructions || !p.streams || !p.weights || !p.rotary_frequencies)
        return "incomplete program view";
    if (!b.input || !b.output || !b.scratch || !b.kv || !b.logits || !b.attention_partials || !b.selection || !b.exchange)
        return "incomplete worker buffers";
    if (p.workers <= 0 || p.workers > 4096)
        return "invalid worker count";
    if (position < 0 || position + steps > p.shape.max_context)
        return "sequence context capacity reached";
    if (p.stack.full_stack && p.selection_slots <= 0)
        return "stack without selection slots";
    return {};
}
} // namespace tiles

extern "C" const char* ti_error_string(int code)
{
    switch (code) {
    case TI_OK: return "success";
    case TI_ERR_INVALID_ARGUMENT: return "invalid argument";
    case TI_ERR_HIP: return "HIP runtime error";
    case TI_ERR_PLAN: return "invalid decoder package";
    case TI_ERR_RUNTIME: return "runtime error";
    case TI_ERR_NO_DEVICE: return "no HIP device";
    default: return "unknown error";
    }
}

extern "C" const char* ti_last_error_message(void) { return tiles::last_message(); }
extern "C" const char* ti_abi(void) { return tiles::kAbi; }
extern "C" const char* ti_fingerprint(void) { return tiles::kFingerprint; }

extern "C" size_t ti_exchange_words(const ti_model_shape* shape, int32_t layers, int32_t selection_slots)
{
    return shape ? tiles::exchange_layout(*shape, layers, selection_slots).total : 0;
}

extern "C" uint32_t ti_epochs_per_launch(int32_t layers) { return TI_MAX_LAUNCH_STEPS * tiles::epochs_per_step(layers); }

extern "C" int ti_describe_target(ti_target* out)
{
    using namespace tiles;
    if (!out)
        return fail(TI_ERR_INVALID_ARGUMENT, "null target");
    std::memset(out, 0, sizeof *out);
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1)
        return fail(TI_ERR_NO_DEVICE, "no HIP device");
    hipDeviceProp_t props{};
    hipError_t e = hipGetDeviceProperties(&props, 0);
    if (e != hipSuccess)
        return hip_fail(e, "device query");
    std::strncpy(out->name, props.name, sizeof out->name - 1);
    std::strncpy(out->arch, props.gcnArchName, sizeof out->arch - 1);
    out->major = props.major;
    out->minor = props.minor;
    out->sm_count = props.multiProcessorCount;
    out->cooperative_launch = props.cooperativeLaunch ? 1 : 0;
    out->max_threads_per_sm = props.maxThreadsPerMultiProcessor;
    out->global_memory_bytes = props.totalGlobalMem;
    out->threads_per_block = kThreads;
    out->attention_shared_bytes = kAttentionSharedBytes;
    (void)hipDriverGetVersion(&out->driver_version);
    (void)hipRuntimeGetVersion(&out->runtime_version);
    hipFuncAttributes f32{}, bf16{};
    if ((e = hipFuncGetAttributes(&f32, worker_function<false>())) != hipSuccess)
        return hip_fail(e, "FP32 worker attributes");
    if ((e = hipFuncGetAttributes(&bf16, worker_function<true>())) != hipSuccess)
        return hip_fail(e, "BF16 worker attributes");
    int f32_occupancy = 0, bf16_occupancy = 0;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&f32_occupancy, worker_function<false>(), kThreads, 0)) != hipSuccess)
        return hip_fail(e, "FP32 worker occupancy");
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&bf16_occupancy, worker_function<true>(), kThreads, 0)) != hipSuccess)
        return hip_fail(e, "BF16 worker occupancy");
    out->f32_registers = f32.numRegs;
    out->f32_shared_bytes = static_cast<int>(f32.sharedSizeBytes);
    out->f32_active_blocks = f32_occupancy;
    out->bf16_registers = bf16.numRegs;
    out->bf16_shared_bytes = static_cast<int>(bf16.sharedSizeBytes);
    out->bf16_active_blocks = bf16_occupancy;
    out->active_blocks_per_sm = f32_occupancy < bf16_occupancy ? f32_occupancy : bf16_occupancy;
    out->registers_per_thread = f32.numRegs > bf16.numRegs ? f32.numRegs : bf16.numRegs;
    out->static_shared_bytes = static_cast<int>(f32.sharedSizeBytes > bf16.sharedSizeBytes ? f32.sharedSizeBytes : bf16.sharedSizeBytes);
    return TI_OK;
}

extern "C" int ti_enqueue_zero_unused_kv(void* stream, void* kv, int32_t dtype, size_t count, int32_t layers,
                                         int32_t layer_stride, int32_t width, int32_t capacity, int32_t key_offset,
                                         int32_t value_offset, int32_t prefix, const int32_t* generated_status)
{
    using namespace tiles;
    if (!kv || layers <= 0 || width <= 0 || capacity <= 0)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid K/V zeroing request");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == TI_DTYPE_BFLOAT16)
        hipLaunchKernelGGL(zero_unused_kv<true>, dim3(256), dim3(256), 0, s, kv, count, layers, layer_stride, width, capacity,
                           key_offset, value_offset, prefix, generated_status);
    else
        hipLaunchKernelGGL(zero_unused_kv<false>, dim3(256), dim3(256), 0, s, kv, count, layers, layer_stride, width, capacity,
                           key_offset, value_offset, prefix, generated_status);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? TI_OK : hip_fail(e, "K/V zeroing launch");
}

extern "C" int ti_enqueue_widen(void* stream, const void* source, int32_t dtype, size_t count, float* destination)
{
    using namespace tiles;
    if (!source || !destination)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid widen request");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == TI_DTYPE_BFLOAT16)
        hipLaunchKernelGGL(widen<true>, dim3(1024), dim3(256), 0, s, source, count, destination);
    else
        hipLaunchKernelGGL(widen<false>, dim3(1024), dim3(256), 0, s, source, count, destination);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? TI_OK : hip_fail(e, "widen launch");
}

// ---------------------------------------------------------------- streaming-read roofline

namespace tiles {
namespace {
// Reads `n` 16-byte vectors with nontemporal loads, `unroll` independent loads per lane in
// flight (the reference's stream_vectors probe, bandwidth_probe.cu:509-549, re-written).
__global__ void stream_read(const u32x4* __restrict__ src, size_t n, int unroll, unsigned* sink)
{
    u32x4 acc = {0, 0, 0, 0};
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (unroll >= 8) {
        for (; i + 7 * stride < n; i += 8 * stride) {
            u32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                acc ^= v[u];
        }
    } else if (unroll >= 4) {
        for (; i + 3 * stride < n; i += 4 * stride) {
            u32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                acc ^= v[u];
        }
    }
    for (; i < n; i += stride)
        acc ^= __builtin_nontemporal_load(src + i);
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u)
        sink[0] = 1;
}
} // namespace
} // namespace tiles

extern "C" int ti_measure_stream_read(size_t bytes, int32_t repeats, double* best_gbps)
{
    using namespace tiles;
    if (!best_gbps || bytes < (1u << 20) || repeats < 1)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid stream measurement request");
    hipDeviceProp_t props{};
    hipError_t e = hipGetDeviceProperties(&props, 0);
    if (e != hipSuccess)
        return hip_fail(e, "device query");
    void* buffer = nullptr;
    unsigned* sink = nullptr;
    if ((e = hipMalloc(&buffer, bytes)) != hipSuccess)
        return hip_fail(e, "stream buffer");
    if ((e = hipMalloc(&sink, 64)) != hipSuccess) {
        (void)hipFree(buffer);
        return hip_fail(e, "stream sink");
    }
    hipEvent_t a = nullptr, b = nullptr;
    double best = 0.0;
    const size_t n = bytes / 16;
    e = hipMemset(buffer, 1, bytes);
    if (e == hipSuccess)
        e = hipEventCreate(&a);
    if (e == hipSuccess)
        e = hipEventCreate(&b);
    const int cus = props.multiProcessorCount;
    const int grids[] = {1, 2, 4, 8, 16, 32};
    const int blocks[] = {256, 1024};
    const int unrolls[] = {1, 4, 8};
    for (int g = 0; e == hipSuccess && g < 6; ++g)
        for (int bl : blocks)
            for (int u : unrolls) {
                const dim3 grid(static_cast<unsigned>(cus * grids[g]));
                hipLaunchKernelGGL(stream_read, grid, dim3(bl), 0, 0, static_cast<const u32x4*>(buffer), n, u, sink);
                (void)hipEventRecord(a, 0);
                for (int r = 0; r < repeats; ++r)
                    hipLaunchKernelGGL(stream_read, grid, dim3(bl), 0, 0, static_cast<const u32x4*>(buffer), n, u, sink);
                (void)hipEventRecord(b, 0);
                if ((e = hipEventSynchronize(b)) != hipSuccess)
                    break;
                float ms = 0.0f;
                (void)hipEventElapsedTime(&ms, a, b);
                const double gbps = static_cast<double>(bytes) * repeats / (ms * 1e-3) / 1e9;
                best = gbps > best ? gbps : best;
            }
    if (a)
        (void)hipEventDestroy(a);
    if (b)
        (void)hipEventDestroy(b);
    (void)hipFree(buffer);
    (void)hipFree(sink);
    if (e != hipSuccess)
        return hip_fail(e, "stream measurement");
    *best_gbps = best;
    return TI_OK;
}
