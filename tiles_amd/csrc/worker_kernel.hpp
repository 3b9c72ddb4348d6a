// MI355X (gfx950) decode worker: one persistent kernel per launch, all of whose blocks are resident, that runs
// every worker's instruction stream once per token for up to 64 tokens, with on-GPU greedy
// selection (replaces tileinfer/src/runtime/worker_kernel.cu and ops.cuh).
//
// Synchronization.  The reference separates waves with a grid barrier
// (worker_kernel.cu:105-107,191-192).  On MI355X a flat 256-block barrier costs 4.2 us and a
// contention-spread one 1.9 us, plus a store-acknowledge and a reload around it, against a
// token floor of about 342 us over ~83 waves.  This worker therefore synchronizes through an
// exchange area of 64-bit words, each holding one element of a wave's output in its low half
// and the epoch of the token/layer/phase that wrote it in its high half.  A producer stores
// the word with one device-coherent (sc1) 64-bit store, which is single-copy atomic, and a
// consumer reads the words it needs with device-coherent loads until every epoch matches:
// data and "arrived" travel together.  Every producer waits for its earlier side-effect
// stores (K/V cache rows, attention partials) to complete (s_waitcnt vmcnt(0)) before
// publishing, so a consumer that sees an epoch also sees them.  The plan's barrier records
// compile to nothing; the wave order still decides which worker runs which task.
//
// Each operation issues its weight loads (nontemporal, 16 bytes per lane, several passes in
// flight) before it waits for its inputs, so HBM latency overlaps the wait.  The kernel is
// instantiated per storage type, per number of 16-byte vectors a lane holds of a hidden row
// (VPL) and per number of lanes that hold a K/V row (LRK), so that every loop bound and
// cross-lane reduction width is a compile-time constant; worker_bf16.hip and worker_f32.hip
// instantiate the shapes listed in worker_config.hpp.  Every bf16 rounding point follows the eager-PyTorch contract of the reference
// (docs/architecture.md:284-312; ops.cuh sites cited per function).
#pragma once

#include <atomic>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {
namespace {

constexpr int kWaves = kThreads / 64;
constexpr int kResidencyDevices = 64;
constexpr int kBlockThreads = kThreads;
constexpr int kLdsHidden = kMaxHidden;
constexpr int kLdsRegionFloats = kRegionFloats;
constexpr int kLdsStreamRecords = kMaxStreamRecords;

// The thread's index in the block, re-read at each use through an empty asm statement that the
// compiler may neither move nor merge.  Address arithmetic on threadIdx.x is otherwise hoisted
// out of the task loop to the kernel's start: those values then live across every task, exceed
// the 256 VGPRs of a wave at 8 waves per CU, and are spilled to scratch and reloaded from
// memory (behind the weight stream) inside the tasks.
__device__ inline unsigned tid()
{
    unsigned t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// This thread's wave, as a value the compiler knows to be uniform across the wave (a scalar),
// so that branches on it stay scalar branches.
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6); }

// Stress build (compiled with TILES_DELAY_INJECTION, tiles_amd/libtileinfer_amd_delay.so): at the
// start of every task and before every exchange publish, cache-row store and poll, the calling wave
// sleeps a pseudo-random 0 to about 2.5 us (s_sleep 4 is about 108 ns), drawn from a hash of a fixed
// seed, the worker, the wave, the call site and the device clock.  The decode must stay
// bit-identical to the undelayed build: nothing in the exchange protocol may rest on timing.  (The
// reference runs its cases under racecheck/synccheck and with random delays before tasks,
// counter_probe.cu:14-15.)  In the product build the call compiles to nothing.
__device__ inline void inject_delay(uint32_t site)
{
#if defined(TILES_DELAY_INJECTION)
    uint32_t x = 0x2545F491u ^ (blockIdx.x * 0x9E3779B1u) ^ (static_cast<uint32_t>(wave_id()) * 0x85EBCA6Bu) ^
                 (site * 0xC2B2AE35u) ^ static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime());
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    for (uint32_t i = __builtin_amdgcn_readfirstlane(x) % 24u; i > 0; --i)
        __builtin_amdgcn_s_sleep(4);
#else
    (void)site;
#endif
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
    int timeline_fields;  // TI_TIMELINE_FIELDS, or TI_TIMELINE_REFERENCE_FIELDS (the reference's record)
    uint32_t spin_limit;  // polls of one wait before it declares the exchange stuck
    int down_vectors;     // 16-byte vectors of a Wdown row per thread in the down projection (1-4)
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
    // Derived on the host, so that no task divides at run time (an integer division by a
    // run-time value is a chain of about 40 dependent instructions on this target).
    int group;              // query heads per K/V head
    float inv_group;        // 1 / group, rounded
    int hidden_stride;      // row_stride(hidden_size, workers)
    int qkv_stride;         // row_stride(hidden_size + 2 x K/V width, workers)

    __device__ size_t kv_width() const { return static_cast<size_t>(shape.kv_heads) * shape.head_dim; }
    __device__ const char* layer_weight(int layer, uint32_t offset) const
    {
        const size_t element = static_cast<size_t>(stack.layer_weights_offset) +
                               static_cast<size_t>(layer) * stack.layer_weight_stride + offset;
        return static_cast<const char*>(weights) + element * Num<BF16>::kBytes;
    }
    __device__ const char* stack_weight(size_t element) const
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

// The hidden size, a compile-time constant in instantiations with more than one 16-byte vector
// per lane: the launcher admits power-of-two vector counts only, so rows are then exactly
// VPL x 64 vectors.  Loops, bounds and row geometry over it then fold to constants.
template <bool BF16, int VPL>
__device__ __forceinline__ int hidden_size(const Launch<BF16>& L)
{
    return VPL > 1 ? VPL * 64 * Num<BF16>::kPerVec : L.shape.hidden_size;
}

// Elements of a hidden-size vector per thread (an upper bound, exact when VPL > 1): the launcher
// admits at most VPL 16-byte vectors per lane of a row.  Per-element loops over the vector run
// this many times, not kMaxHidden / kThreads.
template <bool BF16, int VPL>
constexpr int hidden_slots()
{
    return (VPL * 64 * Num<BF16>::kPerVec + kThreads - 1) / kThreads;
}

// bf16 elements of the attention's staged V block: one row of (head_dim + 8) per position.  It
// shares LDS with the input vector.  A block holds the most positions (a multiple of 32, at most
// 256) whose rows fit: 256 for 64-dim heads, as many as the K tiles issued before the input wait,
// so that a fused chunk of up to 256 positions stages one block.
constexpr int kVtElements = 256 * (64 + 8) > kLdsHidden * 3 ? 256 * (64 + 8) : kLdsHidden * 3;
constexpr int kMaxThreadsPadded = kThreads;  // floats of a split chunk's own partial in the work region
constexpr int vt_block_positions(int dh)
{
    int positions = 256;
    while (positions > 32 && positions * (dh + 8) > kVtElements)
        positions -= 32;
    return positions;
}
static_assert(vt_block_positions(kMaxHeadDim) * (kMaxHeadDim + 8) <= kVtElements, "V blocks");

struct Shared {
    union {
        struct {
            float vec[kLdsHidden];  // a task's input vector, FP32 values of the storage type
            // The same vector as bf16 bits (bf16 storage): the GEMV reads each lane's slice as
            // one 16-byte vector at consecutive addresses.  Reading it from `vec` (32 bytes per
            // lane, lanes 32 bytes apart) put 16 lanes on each LDS bank.
            uint16_t vbits[kLdsHidden];
        };
        alignas(16) uint16_t vt[kVtElements];  // attention: V rows of a block of positions (no input vector)
    };
    alignas(16) float region[kLdsRegionFloats];  // scores/probabilities, reductions, FFN gate/up/product
    float xsave[kLdsHidden];      // the layer input this worker last read, before the norm
    float rsave[kLdsHidden];      // the attention block output this worker last read
    alignas(16) float small[kMaxTaskRows];  // reductions over waves, softmax statistics, residual rows
    float rotated[(kMaxGroup + 1) * kMaxHeadDim];
    float vcur[kMaxHeadDim];
    // The same rotated Q heads and K row, and V row, as bf16 bits (bf16 storage): a lane's
    // 16-byte matrix operand is then one LDS read instead of eight floats to pack.
    alignas(16) uint16_t rotated_bits[(kMaxGroup + 1) * kMaxHeadDim];
    alignas(16) uint16_t vcur_bits[kMaxHeadDim];
    float rope_cs[kMaxHeadDim];  // the position's RoPE cos (first half) and sin (second half)
    int rope_position;           // the position rope_cs holds, -1 when none
    ti_candidate candidates[kWaves];
    ti_task_record stream[kLdsStreamRecords];  // this worker's instructions but barriers, when they fit
    uint16_t stream_index[kLdsStreamRecords];  // each one's position in the worker's stream
    uint32_t xsave_tag;  // epoch_of(step, layer, kPhaseQKV) of xsave's contents, 0 when empty
    uint32_t rsave_tag;  // epoch_of(step, layer, kPhaseR) of rsave's contents
    int flag;
    int aborted;
    uint32_t spin_limit;  // polls of one wait before it declares the exchange stuck
    int token;
    uint64_t mark_read;   // timeline: when the instruction's first exchange read returned
    uint64_t mark_ready;  // timeline: when its last exchange wait ended
    uint64_t mark_start;         // timeline: 100 MHz device clock at the instruction's start
    uint64_t mark_start_cycles;  // timeline (the reference's record): shader cycle counter at its start
};

// ---------------------------------------------------------------- block synchronization

// LDS words shared between waves, read and written without caching in registers.
__device__ inline int lds_read(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ inline void lds_write(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
// Waits until this wave's LDS accesses completed (s_waitcnt lgkmcnt(0)), leaving vector memory
// operations in flight; also a compiler barrier for memory accesses.
__device__ inline void lds_complete() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }


// Barrier of the waves that run tasks.
__device__ inline void block_sync(Shared& sh)
{
    (void)sh;
    __syncthreads();
}

// Barrier that also returns whether `pred` held in every task thread.
__device__ inline bool block_sync_and(Shared& sh, bool pred)
{
    (void)sh;
    return __syncthreads_and(pred);
}


// ---------------------------------------------------------------- exchange polling

// A wait declares the exchange stuck past the launch's spin limit (ti_set_worker_spin_limit), and
// every 64th spin checks the shared abort word; a stuck wait sets it, so that every worker leaves
// its loops and the kernel drains.
__device__ inline bool stuck(uint64_t* exchange, const ExchangeLayout& xl, uint32_t spins, Shared& sh)
{
    if (sh.aborted)
        return true;
    if (spins > sh.spin_limit || ((spins & 63u) == 0 && coherent_load64(exchange + xl.control) != 0)) {
        sh.aborted = 1;
        coherent_store64(exchange + xl.control, 1);
        return true;
    }
    return false;
}

// The bf16 vectors that every worker reads (layer outputs, the attention output, the attention
// block output) travel as 32-bit halves of exchange words: element i is half i of its region,
// its bf16 bits in the low 16 bits and exchange_tag(epoch) in the high 16.  A producer publishes
// an element with one 4-byte store and a reader gets two elements per 8-byte load: the bytes
// that all 256 workers pull from the few memory channels holding such a vector set the cost of
// reading it.  The tag is never 0 (a cleared word), and two epochs less than 65535 apart have
// different tags.  An element's previous contents are at most one launch older than the epoch
// a reader waits for (every launch writes every element at its first step, and a failed launch
// requires a reset, which clears the exchange): 64 x 8 x (layers + 1) epochs, below 65535 for
// the kMaxTaggedLayers layers the launcher accepts.
// exchange_tag (worker_config.hpp) maps an epoch to that tag.

// Whether exchange word w carries `want`: in its high half (one element per word), or in the
// high 16 bits of both halves (two tagged bf16 elements per word).
template <bool kHalves>
__device__ inline bool word_present(uint64_t w, uint32_t want)
{
    if constexpr (kHalves)
        return static_cast<uint32_t>(w >> 48) == want && (static_cast<uint32_t>(w) >> 16) == want;
    else
        return static_cast<uint32_t>(w >> 32) == want;
}

// Reads `count` (at most kMaxCount) exchange elements from `src` until each carries `epoch`
// and hands each payload to `sink(index, payload)`: one element per word, or with kHalves two
// tagged bf16 elements per word (exchange_tag; `count` even).  Block-wide: every thread must
// call it.
// The first read is optimistic (one coherent round trip when the producers are done).  If any
// word is still missing, every thread re-reads its missing words, with a back-off, until the
// block has them all.  A probe of 256 one-per-CU blocks exchanging a 2048-element vector measured a round
// at 2.46 us this way against 2.64 us with wave 0 first polling one "witness" word per producer
// and the block re-reading after it (1.98 against 2.32 us with 64 producers): the witness scheme
// adds a round trip once the data is there.  (`stride`, the witness spacing, is unused.)  Every
// read issues all its loads before it looks at any of them: a use right after a load waits for
// it, and a loop of such pairs would pay one round trip per word.  `overlap()` runs while the
// first read is in flight.
struct NoOverlap {
    __device__ void operator()() const {}
};

template <bool kHalves, int kMaxCount = kLdsHidden, bool kMeet = true, typename Sink, typename Overlap = NoOverlap>
__device__ __forceinline__ void poll_words(const uint64_t* src, int count, int stride, uint32_t epoch, uint64_t* exchange,
                                          const ExchangeLayout& xl, Shared& sh, Sink sink, Overlap overlap = {})
{
    constexpr int kBatch = ((kHalves ? kMaxCount / 2 : kMaxCount) + kThreads - 1) / kThreads;
    inject_delay(__LINE__);
    const int words = kHalves ? count / 2 : count;
    (void)stride;
    const uint32_t want = kHalves ? exchange_tag(epoch) : epoch;
    uint64_t w[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
        w[k] = kHalves ? (static_cast<uint64_t>(want) << 48) | (want << 16) : static_cast<uint64_t>(want) << 32;
    auto issue_reads = [&]() {
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int index = k * kThreads + static_cast<int>(tid());
            if (k * kThreads < words)  // block-uniform; lanes past the end re-read the last word
                w[k] = coherent_load64(src + (index < words ? index : words - 1));
        }
    };
    auto check = [&]() {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            ok &= word_present<kHalves>(w[k], want);
        return ok;
    };
    // Later rounds re-read only the words still missing: re-reading a whole vector every round,
    // from every worker, floods the memory channels that hold it while the producers and the
    // weight streams still need them (the FFN's 8192 products are 32 KB per worker).
    auto read_missing = [&]() {
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int index = k * kThreads + static_cast<int>(tid());
            if (k * kThreads < words && !word_present<kHalves>(w[k], want))
                w[k] = coherent_load64(src + (index < words ? index : words - 1));
        }
        return check();
    };
    issue_reads();
    issue_fence();
    overlap();
    // Each wave re-reads its own missing words until it has them all, and the block meets once
    // at the end (kMeet; without it, the caller's barrier after the sink is the meeting): a
    // barrier in every round made each wave's next read wait for the slowest wave's last one (a
    // probe of 256 blocks exchanging a 1024-word vector: 2.03 against 2.38 us a round).
    bool mine = check();
    if (tid() == 0 && sh.mark_read == 0)
        sh.mark_read = __builtin_amdgcn_s_memrealtime();
    uint32_t spins = 0;
    while (!__all(mine) && !sh.aborted) {
        __builtin_amdgcn_s_sleep(1);
        if ((tid() & 63) == 0)
            stuck(exchange, xl, ++spins, sh);
        mine = read_missing();
    }
    if constexpr (kMeet)
        block_sync(sh);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
        const int index = k * kThreads + static_cast<int>(tid());
        if (index < words) {
            if constexpr (kHalves) {
                sink(2 * index, static_cast<uint32_t>(w[k]) & 0xffffu);
                sink(2 * index + 1, static_cast<uint32_t>(w[k] >> 32) & 0xffffu);
            } else {
                sink(index, static_cast<uint32_t>(w[k]));
            }
        }
    }
    // This worker's earlier stores (K/V cache rows written after their exchange words) complete
    // before anything it publishes from here on, which is what every later reader of those rows
    // follows.  The loads above already returned, so this waits only for stores.
    wait_stores();
    if (tid() == 0)
        sh.mark_ready = __builtin_amdgcn_s_memrealtime();
}

// The input poll of a GEMV task (a vector exchange: tagged halves in bf16), followed by a
// barrier: the sink's LDS writes are then visible to every wave.  (Polling from wave 0 alone, so
// that the other waves' prefetched weights stay ahead of no reads, measured slower: one wave
// needs more coherent round trips, and a round trip costs about 1.5 us under full HBM load.)
template <bool BF16, typename Sink>
__device__ __forceinline__ void poll_input(const uint64_t* src, int count, int stride, uint32_t epoch, uint64_t* exchange,
                                          const ExchangeLayout& xl, Shared& sh, Sink sink)
{
    poll_words<BF16, kLdsHidden, false>(src, count, stride, epoch, exchange, xl, sh, sink);
    block_sync(sh);
}

// A vector exchange read by the calling wave alone (poll_words's optimistic read and re-reads of
// the missing words, with up to kMaxElements elements), into `sink`; the caller meets the other
// waves at a barrier afterwards.  Its loads return only after every load the wave issued before them,
// so a wave that polls this way keeps few loads of its own in flight.
template <bool BF16, int kMaxElements, typename Sink>
__device__ __forceinline__ void poll_words_one_wave(const uint64_t* src, int count, int stride, uint32_t epoch,
                                                   uint64_t* exchange, const ExchangeLayout& xl, Shared& sh, Sink sink)
{
    constexpr bool kHalves = BF16;
    constexpr int kWords = kHalves ? kMaxElements / 2 : kMaxElements;
    // Rounds of at most 16 words per lane (one round for a 2048-element bf16 vector): more would
    // spill the registers that hold the wave's weight loads.
    constexpr int kBatch = (kWords + 63) / 64 < 16 ? (kWords + 63) / 64 : 16;
    inject_delay(__LINE__);
    const int lane = static_cast<int>(tid() & 63);
    const int words = kHalves ? count / 2 : count;
    (void)stride;
    const uint32_t want = kHalves ? exchange_tag(epoch) : epoch;
    for (int w0 = 0; w0 < words; w0 += 64 * kBatch) {
        uint64_t w[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            w[k] = kHalves ? (static_cast<uint64_t>(want) << 48) | (want << 16) : static_cast<uint64_t>(want) << 32;
        auto read = [&]() {
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int index = w0 + k * 64 + lane;
                if (w0 + k * 64 < words)
                    w[k] = coherent_load64(src + (index < words ? index : words - 1));
            }
            bool ok = true;
#pragma unroll
            for (int k = 0; k < kBatch; ++k)
                ok &= word_present<kHalves>(w[k], want);
            return ok;
        };
        // Later rounds re-read only the missing words, at once (a witness word per producer
        // first, then every word again, cost a round trip more once the data was there).
        auto read_missing = [&]() {
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int index = w0 + k * 64 + lane;
                if (w0 + k * 64 < words && !word_present<kHalves>(w[k], want))
                    w[k] = coherent_load64(src + (index < words ? index : words - 1));
            }
            bool ok = true;
#pragma unroll
            for (int k = 0; k < kBatch; ++k)
                ok &= word_present<kHalves>(w[k], want);
            return ok;
        };
        bool mine = read();
        if (lane == 0 && sh.mark_read == 0)
            sh.mark_read = __builtin_amdgcn_s_memrealtime();
        uint32_t spins = 0;
        while (!__all(mine) && !sh.aborted) {
            __builtin_amdgcn_s_sleep(1);
            if (lane == 0)
                stuck(exchange, xl, ++spins, sh);
            mine = read_missing();
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int index = w0 + k * 64 + lane;
            if (index < words) {
                if constexpr (kHalves) {
                    sink(2 * index, static_cast<uint32_t>(w[k]) & 0xffffu);
                    sink(2 * index + 1, static_cast<uint32_t>(w[k] >> 32) & 0xffffu);
                } else {
                    sink(index, static_cast<uint32_t>(w[k]));
                }
            }
        }
    }
    wait_stores();
    if (lane == 0)
        sh.mark_ready = __builtin_amdgcn_s_memrealtime();
}

// One exchange word, waited for by the calling thread alone.
__device__ inline uint32_t poll_one(const uint64_t* src, uint32_t epoch, uint64_t* exchange, const ExchangeLayout& xl,
                                    Shared& sh)
{
    inject_delay(__LINE__);
    uint64_t w = coherent_load64(src);
    uint32_t spins = 0;
    while (static_cast<uint32_t>(w >> 32) != epoch && !sh.aborted) {
        __builtin_amdgcn_s_sleep(2);
        w = coherent_load64(src);
        stuck(exchange, xl, ++spins, sh);
    }
    return static_cast<uint32_t>(w);
}

// Element `index` of a vector exchange, waited for by the calling thread alone: its payload.
template <bool BF16>
__device__ inline uint32_t poll_element(const uint64_t* region, int index, uint32_t epoch, uint64_t* exchange,
                                        const ExchangeLayout& xl, Shared& sh)
{
    if constexpr (BF16) {
        inject_delay(__LINE__);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(region) + index;
        const uint32_t want = exchange_tag(epoch);
        uint32_t w = coherent_load32(src);
        uint32_t spins = 0;
        while ((w >> 16) != want && !sh.aborted) {
            __builtin_amdgcn_s_sleep(2);
            w = coherent_load32(src);
            stuck(exchange, xl, ++spins, sh);
        }
        return w & 0xffffu;
    } else {
        return poll_one(region + index, epoch, exchange, xl, sh);
    }
}

// Wave 0 waits until each witness word witness(j), j < n, carries `epoch` (8 loads in flight per
// lane, a back-off between rounds); the block then meets at a barrier.  Used after an optimistic
// read came up short: one wave polling one word per producer instead of every thread polling
// every word keeps the waiting workers from flooding the memory system that the others are
// still streaming weights through.  Block-wide: every thread must call it.
template <typename Witness>
__device__ __forceinline__ void wait_witnesses(int n, Witness witness, uint32_t epoch, uint64_t* exchange,
                                              const ExchangeLayout& xl, Shared& sh)
{
    constexpr int kBatch = 8;
    inject_delay(__LINE__);
    if (tid() < 64) {
        const int lane = tid();
        uint32_t spins = 0;
        while (true) {
            bool mine = true;
            for (int j0 = 0; j0 < n; j0 += 64 * kBatch) {
                uint64_t v[kBatch];
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int j = j0 + u * 64 + lane;
                    v[u] = coherent_load64(witness(j < n ? j : n - 1));
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
                    mine &= static_cast<uint32_t>(v[u] >> 32) == epoch;
            }
            if (__all(mine))
                break;
            __builtin_amdgcn_s_sleep(2);
            if (lane == 0)
                stuck(exchange, xl, ++spins, sh);
            if (__any(sh.aborted))
                break;
        }
    }
    block_sync(sh);
}

template <bool BF16>
__device__ inline void publish(uint64_t* dst, int index, float rounded, uint32_t epoch)
{
    inject_delay(__LINE__);
    coherent_store64(dst + index, (static_cast<uint64_t>(epoch) << 32) | Num<BF16>::payload(rounded));
}

// Element `index` of a vector exchange (tagged halves in bf16, words in FP32).
template <bool BF16>
__device__ inline void publish_element(uint64_t* region, int index, float rounded, uint32_t epoch)
{
    inject_delay(__LINE__);
    if constexpr (BF16)
        coherent_store32(reinterpret_cast<uint32_t*>(region) + index, (exchange_tag(epoch) << 16) | Num<BF16>::payload(rounded));
    else
        publish<false>(region, index, rounded, epoch);
}

// Witness spacing of an exchange written by row tasks that split `n` rows over `workers`
// (plan_core.py:275-278: every task gets at least n / workers rows).
__host__ __device__ inline int row_stride(int n, int workers) { return n >= workers ? n / workers : 1; }

// The first half of a block-wide RMSNorm (rms_apply is the second): each wave adds the squares
// its threads accumulated over the elements they delivered and puts the sum in sh.small[wave].
__device__ __forceinline__ void rms_partial(float squares, Shared& sh)
{
    squares = group_sum<64>(squares);
    if ((tid() & 63) == 63)
        sh.small[wave_id()] = squares;
}

// ---------------------------------------------------------------- layer input and residuals

// The hidden state a layer reads, into dst (FP32): the token's embedding row for a stack's
// first layer, the host-written input of a block package, or the previous layer's output.
// A copy stays in sh.xsave for the layer's residual addition.
template <bool BF16, int kSlots>
__device__ __forceinline__ void load_hidden(const Launch<BF16>& L, int d, int layer, int step, ti_token_id token, Shared& sh)
{
    float squares = 0.0f;  // the RMSNorm statistic over the elements this thread delivers
    if (layer == 0) {
        // The token is uniform; as a scalar, its row offset (hoisted to the step's start by the
        // compiler) does not hold two VGPRs across the whole step.
        const int id = __builtin_amdgcn_readfirstlane(token);
        const void* row = L.stack.full_stack
                              ? static_cast<const void*>(L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) +
                                                                        static_cast<size_t>(id) * d))
                              : L.input;
        float v[kSlots];
#pragma unroll
        for (int k = 0; k < kSlots; ++k) {  // all loads in flight together
            const int i = k * kThreads + static_cast<int>(tid());
            v[k] = Num<BF16>::load(row, i < d ? i : 0);
        }
#pragma unroll
        for (int k = 0; k < kSlots; ++k) {
            const int i = k * kThreads + static_cast<int>(tid());
            if (i < d) {
                sh.xsave[i] = v[k];
                squares = fmaf(v[k], v[k], squares);
            }
        }
    } else {
        poll_words<BF16, kLdsHidden, false>(L.exchange + L.xl.hidden(layer % 2), d, L.hidden_stride, L.epoch_of(step, layer - 1, kPhaseY),
                         L.exchange, L.xl, sh, [&](int i, uint32_t p) {
                             const float x = Num<BF16>::from_payload(p);
                             sh.xsave[i] = x;
                             squares = fmaf(x, x, squares);
                         });
    }
    rms_partial(squares, sh);
    block_sync(sh);
    if (tid() == 0)
        sh.xsave_tag = L.epoch_of(step, layer, kPhaseQKV);
}

// Element i of a layer's input (the attention block's residual).
template <bool BF16>
__device__ __forceinline__ float input_element(const Launch<BF16>& L, int layer, int step, ti_token_id token, int i,
                                              Shared& sh)
{
    if (sh.xsave_tag == L.epoch_of(step, layer, kPhaseQKV))
        return sh.xsave[i];
    if (layer == 0)
        return L.stack.full_stack
                   ? Num<BF16>::load(L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) +
                                                    static_cast<size_t>(token) * L.shape.hidden_size),
                                     i)
                   : Num<BF16>::load(L.input, i);
    return Num<BF16>::from_payload(poll_element<BF16>(L.exchange + L.xl.hidden(layer % 2), i,
                                                      L.epoch_of(step, layer - 1, kPhaseY), L.exchange, L.xl, sh));
}

// Element i of a layer's attention block output (the FFN's residual).
template <bool BF16>
__device__ __forceinline__ float attention_output_element(const Launch<BF16>& L, int layer, int step, int i, Shared& sh)
{
    if (sh.rsave_tag == L.epoch_of(step, layer, kPhaseR))
        return sh.rsave[i];
    return Num<BF16>::from_payload(
        poll_element<BF16>(L.exchange + L.xl.r, i, L.epoch_of(step, layer, kPhaseR), L.exchange, L.xl, sh));
}

// ---------------------------------------------------------------- RMSNorm (ops.cuh:145-219)

// A norm's scale elements tid() + k * kThreads, loaded into registers before the task
// waits for its input (a load issued after the wait would add a full memory latency).
template <int kSlots>
struct NormScale {
    float v[kSlots];
};

template <bool BF16, int kSlots>
__device__ __forceinline__ NormScale<kSlots> load_scale(const void* scale, int d)
{
    // Unconditional loads (lanes past d re-read element d - 1, never used): a select on a
    // loaded value would make the load's wait immediate.
    NormScale<kSlots> s;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        const int i = k * kThreads + static_cast<int>(tid());
        s.v[k] = Num<BF16>::load(scale, i < d ? i : d - 1);
    }
    return s;
}

// RMSNorm in two block-wide halves around a barrier of the caller's: rms_partial (above), then
// rms_apply after the barrier: the statistic is the waves' sums in wave order (FP32); then
// element i = tid() + k * kThreads of the raw vector x becomes round(round(x[i] * inv_rms) *
// scale[i]) in bf16, x[i] * inv_rms * scale[i] in fp32 (decoder_reference.py:183-187,
// decoder_stack.py:126-132): into sh.vbits (bf16 bits, the GEMV input) and, for fp32 or when
// asked, into sh.vec.  Ends with a barrier.
// Scale element i (slot k of the calling thread) for rms_apply: from registers, or (bf16) from
// the bits a wave left in sh.vbits, read by the thread that then overwrites them.
template <int kSlots>
struct RegisterScale {
    const NormScale<kSlots>& scale;
    __device__ float operator()(int k, int, const Shared&) const { return scale.v[k]; }
};
struct LdsScale {
    __device__ float operator()(int, int i, const Shared& sh) const { return bf16_bits_to_float(sh.vbits[i]); }
};

template <bool BF16, int kSlots, typename Scale>
__device__ __forceinline__ void rms_apply(const float* x, int d, Scale scale, float eps, Shared& sh, bool fp32_copy = false)
{
    float xv[kSlots];  // all reads first
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        const int i = k * kThreads + static_cast<int>(tid());
        xv[k] = x[i < d ? i : 0];
    }
    static_assert(kWaves == 8, "wave sums read as two float4");
    const float4 s0 = reinterpret_cast<const float4*>(sh.small)[0];
    const float4 s1 = reinterpret_cast<const float4*>(sh.small)[1];
    const float total = ((((((s0.x + s0.y) + s0.z) + s0.w) + s1.x) + s1.y) + s1.z) + s1.w;
    const float inv = 1.0f / sqrtf(total / static_cast<float>(d) + eps);
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        const int i = k * kThreads + static_cast<int>(tid());
        if (i < d) {
            const float y = Num<BF16>::round(Num<BF16>::round(xv[k] * inv) * scale(k, i, sh));
            if (!BF16 || fp32_copy)
                sh.vec[i] = y;
            if constexpr (BF16)
                sh.vbits[i] = static_cast<uint16_t>(float_to_bf16_bits(y));
        }
    }
    block_sync(sh);
}

// ---------------------------------------------------------------- GEMV over rows

// Rows of a hidden-width matrix are owned by lane groups: LR = min(64, vectors per row) lanes
// per row, each holding VPL 16-byte vectors of it; a wave pass covers 64 / LR rows.
template <bool BF16>
struct RowGeometry {
    int lr, rows_per_wave, pass_rows, wave, sub, col;
    __device__ explicit RowGeometry(int cols)
    {
        const int nvec = cols / Num<BF16>::kPerVec;
        lr = nvec < 64 ? nvec : 64;
        rows_per_wave = 64 / lr;
        pass_rows = kWaves * rows_per_wave;
        const int lane = tid() & 63;
        wave = wave_id();
        sub = lane / lr;
        col = lane % lr;
    }
    __device__ int first_row(int r0, int pass) const { return r0 + pass * pass_rows + wave * rows_per_wave; }
};

// The lane's slice of a hidden-width vector u in LDS, one 16-byte vector per k: packed bf16
// pairs for v_dot2_f32_bf16, or four FP32 values.
template <int VPL>
struct InputSlice {
    uint32_t r[VPL * 4];
    __device__ InputSlice() {}
    __device__ InputSlice(const void* u, int col, int lr)
    {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const u32x4 v = static_cast<const u32x4*>(u)[col + k * lr];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                r[k * 4 + q] = v[q];
        }
    }
    // The lane's part of one row's dot product (VPL 16-byte vectors of the row).
    template <bool BF16>
    __device__ float dot(const u32x4* wm) const
    {
        using N = Num<BF16>;
        if constexpr (BF16) {
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // independent chains
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    a[q] = dot2_bf16(wm[k][q], r[k * 4 + q], a[q]);
            return (a[0] + a[1]) + (a[2] + a[3]);
        } else {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int j = 0; j < N::kPerVec; ++j)
                    acc += N::elem(wm[k], j) * __uint_as_float(r[k * 4 + j]);
            return acc;
        }
    }
};

// The normalized GEMV input of a lane: rms_apply to the raw vector x (its statistic already in
// sh.small), then the lane's slice from LDS.
template <bool BF16, int VPL>
struct NormInput {
    static constexpr int kSlots = hidden_slots<BF16, VPL>();
    NormScale<kSlots> scale;
    __device__ NormInput(const void* weights, int d) : scale(load_scale<BF16, kSlots>(weights, d)) {}
    __device__ InputSlice<VPL> operator()(const float* x, Shared& sh, int d, float eps) const
    {
        rms_apply<BF16, kSlots>(x, d, RegisterScale<kSlots>{scale}, eps, sh);
        const RowGeometry<BF16> g(d);
        return InputSlice<VPL>(gemv_input<BF16>(sh), g.col, g.lr);
    }
};

// Dot products of rows [r0, r1) of NM matrices of hidden width with an input vector: prepare()
// (block-wide) waits for the task's inputs, make_slice() then gives each lane its slice of the
// vector (InputSlice).  emit(row, dots), with one dot per matrix, runs once per row after every
// row is done, in any thread.
//
// row_offset(m, row) is the byte offset from `base` of a row of matrix m (below 2 GiB).  D passes
// of loads are in flight; all D issue before `prepare`, which runs block-wide, waits for the
// task's inputs and writes u, so weight latency overlaps the wait.
template <bool BF16, int VPL, int NM, int DEPTH = 0, typename RowOffset, typename Prepare, typename MakeSlice,
          typename Emit>
__device__ __forceinline__ void gemv(const void* base, RowOffset row_offset, int r0, int r1, int cols, Shared& sh,
                                    Prepare prepare, MakeSlice make_slice, Emit emit)
{
    using N = Num<BF16>;
    constexpr int K = VPL * NM;
    constexpr int D = DEPTH > 0 ? DEPTH : (K <= 4 ? 4 : (K <= 8 ? 2 : 1));
    const RowGeometry<BF16> g(cols);
    (void)sh;
    auto active = [&](int pass) { return g.first_row(r0, pass) < r1; };
    // Lanes past the task read the task's first row from its start, 16 bytes apart per k: one
    // cached request per instruction.  Their addresses differ per k on purpose: equal ones let
    // the compiler load once for those lanes and copy, behind a wait for that load.
    auto issue = [&](int pass, u32x4* w) {
        const int row = g.first_row(r0, pass) + g.sub;
        const bool inside = row < r1;
        const uint32_t col = inside ? static_cast<uint32_t>(g.col) * 16u : 0u;
        const uint32_t stride = inside ? static_cast<uint32_t>(g.lr) * 16u : 16u;
        const char* at = static_cast<const char*>(base) + col;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const char* p = at + row_offset(m, inside ? row : r0);
#pragma unroll
            for (int k = 0; k < VPL; ++k)
                w[m * VPL + k] = load_weights(p + k * stride);
        }
    };
    u32x4 w[D][K];
    // Every pass issues.  A conditional issue would leave the compiler unsure how many loads are
    // in flight, and its waits for earlier loads would become waits for all of them.
#pragma unroll
    for (int s = 0; s < D; ++s)
        issue(s, w[s]);
    issue_fence();
    // The input's first read goes out once the first pass has arrived: a read samples the
    // exchange when it is issued and returns after the loads before it, so one issued with the
    // weights found late producers' words missing when it came back, and a second round followed.
    if constexpr (D > 1)
        wait_vmem<(D - 1) * K>();
    prepare();
    const InputSlice<VPL> in = make_slice();
    // Whole groups of D passes without branches (passes past the task compute values nobody
    // keeps), an explicit wait for each pass's loads with the later passes in flight, and no
    // global store inside the loop: the row results wait in LDS (the work region, free once the
    // input slice is read) and are emitted afterwards, one row per thread.  Loads and stores share
    // vmcnt, so a store, or a branch the compiler's count merges over, made each wait a wait for
    // every load in flight.  Every group but the last issues the next group's passes; the last
    // issues nothing, so that no load is in flight when the rows are emitted (loads past the task
    // issued at its end made the first publish wait a whole memory round trip for them).
    float* staged = sh.region;  // [row - r0][NM]
    auto compute = [&](int s, int pass) {
        float dots[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const float part = in.template dot<BF16>(&w[s][m * VPL]);
            dots[m] = VPL > 1 ? group_sum<64>(part) : group_sum(part, g.lr);
        }
        const int row = g.first_row(r0, pass) + g.sub;
        if (row < r1 && g.col == g.lr - 1)
#pragma unroll
            for (int m = 0; m < NM; ++m)
                staged[(row - r0) * NM + m] = dots[m];
    };
    int pass0 = 0;
    for (; active(pass0 + D); pass0 += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            wait_vmem<(D - 1) * K>();
            compute(s, pass0 + s);
            issue(pass0 + s + D, w[s]);
        }
    }
    // The last group: each pass's dot products as its loads arrive, then the reductions of all of
    // them together and the staged stores after those.  Reducing and storing each pass in turn
    // made every pass a serial chain of its own (the masked store between passes split the code
    // into blocks the scheduler does not interleave), also for passes past the task.
    float parts[D * NM];
    unroll<D>([&](auto step) {
        constexpr int s = decltype(step)::value;
        wait_vmem<(D - 1 - s) * K>();
#pragma unroll
        for (int m = 0; m < NM; ++m)
            parts[s * NM + m] = in.template dot<BF16>(&w[s][m * VPL]);
    });
    if constexpr (VPL > 1) {
        group_sum_all<64>(parts);
    } else {
#pragma unroll
        for (int j = 0; j < D * NM; ++j)
            parts[j] = group_sum(parts[j], g.lr);
    }
    if (g.col == g.lr - 1)
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int row = g.first_row(r0, pass0 + s) + g.sub;
            if (row < r1)
#pragma unroll
                for (int m = 0; m < NM; ++m)
                    staged[(row - r0) * NM + m] = parts[s * NM + m];
        }
    block_sync(sh);
    for (int row = r0 + static_cast<int>(tid()); row < r1; row += kThreads) {
        float dots[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m)
            dots[m] = staged[(row - r0) * NM + m];
        emit(row, dots);
    }
    static_assert(kMaxTaskRows * NM <= kLdsRegionFloats, "staged GEMV rows exceed the work region");
    (void)N::kBytes;
}

// ---------------------------------------------------------------- operations

template <bool BF16>
__device__ inline const void* gemv_input(const Shared& sh)
{
    return BF16 ? static_cast<const void*>(sh.vbits) : static_cast<const void*>(sh.vec);
}

// [Q; K; V] rows of the normalized layer input (ops.cuh:266-289), rounded to the storage type
// and published unrotated.  V rows also go to the cache row of the current position; this
// token's attention takes V from the exchange words, and the worker's next input poll waits for
// the cache stores before it publishes anything else, so later tokens find the row complete.
template <bool BF16, int VPL, int LRK>
__device__ __forceinline__ void op_qkv(const Launch<BF16>& L, const ti_task_record& t, int step, ti_token_id token, Shared& sh)
{
    using N = Num<BF16>;
    constexpr int dh = LRK * N::kPerVec;  // the launcher admits only this head_dim for the instantiation
    const int d = hidden_size<BF16, VPL>(L);
    const int kvw = L.shape.kv_heads * dh;
    const int layer = static_cast<int>(t.layer);
    const int position = L.position + step;
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseQKV);
    // Rows may span Wq, Wk and Wv, which are separate regions of the layer's weights: row r of
    // a region that starts at row `first` lies at region + (r - first) d = base + r d, with base
    // = region - first d (mod 2^32).  The base is the V region's plus differences selected
    // against zero: a select among the captured bases became an indexed load from a per-thread
    // copy of them (20 bytes a thread, which the compiler placed in LDS, or in scratch memory
    // once LDS was short), and a select of the launch record's fields branches around loads.
    const uint32_t ud = static_cast<uint32_t>(d), ukvw = static_cast<uint32_t>(kvw);
    const uint32_t base_q = L.layout.Wq, base_k = L.layout.Wk - ud * ud, base_v = L.layout.Wv - (ud + ukvw) * ud;
    const uint32_t to_k = base_k - base_v, to_q = base_q - base_k;
    auto row_offset = [=](int, int row) {
        const bool q = row < d, k = row < d + kvw;
        const uint32_t base = base_v + (k ? to_k : 0u) + (q ? to_q : 0u);
        return (base + static_cast<uint32_t>(row) * ud) * N::kBytes;
    };
    const NormInput<BF16, VPL> norm(L.layer_weight(layer, L.layout.attn_norm), d);
    auto prepare = [&]() { load_hidden<BF16, hidden_slots<BF16, VPL>()>(L, d, layer, step, token, sh); };
    auto make_slice = [&]() { return norm(sh.xsave, sh, d, L.numeric.rms_norm_eps); };
    float* staged_v = sh.small;  // this task's V rows, for the cache stores after the GEMV
    // Read once into registers: inside the row loop every field of the LDS launch record would be
    // re-read after each LDS store.
    uint64_t* const words = L.exchange + L.xl.qkv;
    const int group = L.group;
    const float inv_group = L.inv_group;
    gemv<BF16, VPL, 1, 2>(L.layer_weight(layer, 0), row_offset, begin, end, d, sh, prepare, make_slice,
                       [&](int row, const float* dots) {
        const float value = N::round(dots[0]);
        publish<BF16>(words, qkv_slot<dh>(row, d, kvw, group, inv_group), value, epoch);
        if (row >= d + kvw)
            staged_v[row - begin] = value;
    });
    const int first_v = begin > d + kvw ? begin : d + kvw;
    if (end <= first_v)
        return;
    block_sync(sh);
    // Wave 0 stores the V rows (at most 64 per task); every wave's next input poll waits for its
    // stores before this worker publishes anything else.
    void* cache = L.cache(layer, L.layout.value);
    if (wave_id() != 0)
        return;
    inject_delay(__LINE__);
    for (int row = first_v + (static_cast<int>(tid()) & 63); row < end; row += 64) {
        const size_t index = static_cast<size_t>(position) * kvw + (row - d - kvw);
        if constexpr (BF16)
            coherent_store16(static_cast<uint16_t*>(cache) + index,
                             static_cast<uint16_t>(float_to_bf16_bits(staged_v[row - begin])));
        else
            coherent_storef(static_cast<float*>(cache) + index, staged_v[row - begin]);
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

// One K/V head and context chunk of decode attention (ops.cuh:574-673, re-designed):
// RoPE of the group's query heads and current K; chunk 0 stores rotated K into the cache.
// One active chunk (a prefix of at most attention_fused_steps): scores, exact softmax,
// probabilities rounded to the storage type, P*V, published as the group's attention output.
// Several chunks: each chunk publishes its softmax statistics, merges every chunk's, rounds
// exp(score - M) / S to the storage type and publishes its FP32 partial P*V; each chunk then
// adds one slice of the group's outputs over all chunks' partials, in chunk order, and publishes
// it.  The reference runs the same arithmetic as a scores wave and a values wave
// (ops.cuh:574-673).
//
// bf16 heads of 32, 64 or 128 dims compute Q K^T and P V on the matrix cores
// (v_mfma_f32_16x16x32_bf16): a wave takes 16 positions at a time, lane l holding position
// l % 16 and dims 8 (l / 16) .. + 7 of every 32 (one 16-byte load per 32 dims), against the
// group's query heads padded to 16 rows.  V is transposed through LDS a block of positions at
// a time, so P V runs the positions as the reduced dimension; waves split the head's dims 16
// at a time.  Other shapes use the vector path: LRK lanes hold one K/V row (16 bytes each),
// rows spread over lanes and waves, partial P V sums reduced across them.
// Cached K/V rows never change during a token, so the first rows of the chunk, and the
// position's RoPE angles, are loaded before the task waits for this token's Q/K/V.
template <bool BF16, int LRK>
__device__ __forceinline__ void op_attention(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    constexpr int PV = N::kPerVec;
    constexpr int MG = kMaxGroup;
    constexpr int dh = LRK * PV;
    constexpr bool kMfma = BF16 && dh % 32 == 0;
    constexpr int KS = dh / 32;                      // 32-dim slices of a head (matrix path)
    constexpr int kTile = 16;                        // positions per matrix tile
    constexpr int PB = vt_block_positions(dh);       // positions per staged V block in LDS
    constexpr int kBlockTiles = PB / kTile;
    constexpr int TW = (kBlockTiles + kWaves - 1) / kWaves;  // tiles per wave in a block
    constexpr int kVRow = dh + 8;  // bf16 per staged V row: 4 rows of 16-byte-apart chunks hit distinct banks
    static_assert(!kMfma || PB * kVRow <= kVtElements, "V block exceeds its LDS area");
    static_assert(!kMfma || dh / 16 <= kWaves, "a wave per 16 output dims");
    constexpr int kRowsPerWave = 64 / LRK;
    constexpr int kBlockRows = kWaves * kRowsPerWave;
    constexpr uint32_t kOutside = 0x80000000u;  // past every layer's K/V bytes: the buffer load returns 0
    const ti_model_shape& s = L.shape;
    const int position = L.position + step;
    const int chunks = active_chunks(position, s);
    const int chunk = static_cast<int>(t.chunk);
    if (chunk >= chunks)
        return;
    const int layer = static_cast<int>(t.layer);
    const int kv_head = static_cast<int>(t.kv_head);
    const int group = L.group;
    const int first_head = kv_head * group;
    const int kvw = s.kv_heads * dh;
    const int length = position + 1;
    // 32-bit: the launcher bounds max_context x attention_chunks below 2^31.
    const int begin = chunk == 0 ? 0 : static_cast<int>(static_cast<uint32_t>(length * chunk) / static_cast<uint32_t>(chunks));
    const int end = chunk + 1 == chunks ? length
                                        : static_cast<int>(static_cast<uint32_t>(length * (chunk + 1)) / static_cast<uint32_t>(chunks));
    const int span = end - begin;

    const int lane = tid() & 63, wave = wave_id();
    const int sub = lane / LRK, col = lane % LRK;    // vector path: row and 16-byte slice
    const int tr = lane % kTile, tk = lane / kTile;  // matrix path: tile row and 8-element slice
    void* key_cache = L.cache(layer, L.layout.key);
    const void* value_cache = L.cache(layer, L.layout.value);
    const uint32_t layer_kv_bytes = static_cast<uint32_t>(static_cast<size_t>(s.max_context) * kvw * N::kBytes);
    const __amdgpu_buffer_rsrc_t krsrc = make_rsrc(key_cache, layer_kv_bytes);
    const __amdgpu_buffer_rsrc_t vrsrc = make_rsrc(value_cache, layer_kv_bytes);
    // Rows past the chunk, and the current position (not cached yet), read as zeros.  Their
    // offsets differ per load: equal ones let the compiler merge the loads behind a wait.
    auto row_time = [&](int first, int u) { return first + u * kBlockRows + wave * kRowsPerWave + sub; };
    auto load_rows = [&](__amdgpu_buffer_rsrc_t rsrc, int first, u32x4* raw) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int time = row_time(first, u);
            const bool cached = time < end && time < position;
            const uint32_t offset = static_cast<uint32_t>((static_cast<size_t>(time) * kvw + kv_head * dh + col * PV) * N::kBytes);
            raw[u] = coherent_load128(rsrc, cached ? offset : kOutside + 16u * u);
        }
    };
    // Matrix path: tile `tile` of the chunk, lane l at position begin + 16 tile + l % 16.
    auto load_tile = [&](__amdgpu_buffer_rsrc_t rsrc, int tile, u32x4* raw) {
        const int time = begin + tile * kTile + tr;
        const bool cached = time < end && time < position;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const uint32_t offset =
                static_cast<uint32_t>((static_cast<size_t>(time) * kvw + kv_head * dh + 32 * k + 8 * tk) * N::kBytes);
            raw[k] = coherent_load128(rsrc, cached ? offset : kOutside + 16u * k);
        }
    };
    // Matrix path: tiles wave, wave + 8, ... of the first block; vector path: two rows.
    constexpr int kFirst = kMfma ? KS : 2;
    constexpr int kFirstTiles = kMfma ? TW : 1;
    u32x4 kfirst[kFirstTiles][kFirst], vfirst[kFirstTiles][kFirst];
    if constexpr (kMfma) {
#pragma unroll
        for (int j = 0; j < TW; ++j) {
            load_tile(krsrc, wave + j * kWaves, kfirst[j]);
            load_tile(vrsrc, wave + j * kWaves, vfirst[j]);
        }
    } else {
        load_rows(krsrc, begin, kfirst[0]);
        load_rows(vrsrc, begin, vfirst[0]);
    }
    issue_fence();

    // cos/sin of the position's RoPE angles, rounded (ops.cuh:125-140): the same for every layer
    // of a step, so computed once per position (the tag is read before the poll's barriers and
    // written after them), while the first exchange read is in flight.
    constexpr int half = dh / 2;
    const bool fresh_rope = sh.rope_position != position;
    auto rope_table = [&]() {
        if (fresh_rope)
            for (int pair = tid(); pair < half; pair += kThreads) {
                const float angle = static_cast<float>(position) * global(L.rope)[pair];
                sh.rope_cs[pair] = N::round(cosf(angle));
                sh.rope_cs[half + pair] = N::round(sinf(angle));
            }
    };
    // Matrix path: the first block's cached V rows go to LDS, as stored, while the first read is
    // in flight too (the current position's row, loaded as zeros, is written once it arrives).
    // V rows past the chunk's last 32-position step are never read: P V stops there.
    const int live0 = min(kBlockTiles, 2 * ((min(span, PB) + 31) / 32));
    auto stage_v = [&]() {
        if constexpr (kMfma) {
#pragma unroll
            for (int j = 0; j < TW; ++j)
                if (wave + j * kWaves < live0) {
                    const int row = (wave + j * kWaves) * kTile + tr;
#pragma unroll
                    for (int k = 0; k < KS; ++k)
                        *reinterpret_cast<u32x4*>(sh.vt + row * kVRow + 32 * k + 8 * tk) = vfirst[j][k];
                }
        }
    };

    // This token's Q heads, K and V of the head group: one packed exchange block.  With
    // head_dim <= 64, thread t polls element t and finds its RoPE partner (element t +- dh / 2)
    // in lane t ^ (dh / 2) of its own wave, so it rotates in registers; wider heads go through
    // the work region and a pass of their own.
    constexpr bool kRopeInWave = half <= 32;
    const int block = (group + 2) * dh;
    const int qk = (group + 1) * dh;
    float held = 0.0f;  // kRopeInWave: element tid() of the block
    poll_words<false>(L.exchange + L.xl.qkv + static_cast<size_t>(kv_head) * block, block,
               L.qkv_stride, L.epoch_of(step, layer, kPhaseQKV), L.exchange, L.xl, sh,
               [&](int i, uint32_t p) {
                   const float v = N::from_payload(p);
                   if (i >= qk) {
                       sh.vcur[i - qk] = v;
                       if constexpr (kMfma)
                           sh.vcur_bits[i - qk] = static_cast<uint16_t>(p);
                   }
                   if constexpr (kRopeInWave)
                       held = v;  // i == tid(): block <= kThreads
                   else if (i < qk)
                       sh.region[i] = v;
               }, [&]() {
                   rope_table();
                   stage_v();
               });
    if (tid() == 0)
        sh.rope_position = position;
    // Chunk 0 stores the rotated K row into the cache and the rotated Q heads into scratch.  Every
    // load issued so far has returned (the poll waited for its own, which return after them); an
    // explicit wait says so to the compiler, which would otherwise make later waits for those loads
    // wait for these stores too.
    auto store_rotated = [&](int index, float value) {
        inject_delay(__LINE__);
        if (index < group * dh) {
            if (L.block_trace)  // scratch intermediates only on traced launches
                N::store(L.scratch, L.layout.q_rot + first_head * dh + index, value);
        } else {
            const size_t e = static_cast<size_t>(position) * kvw + kv_head * dh + (index - group * dh);
            if constexpr (BF16)
                coherent_store16(static_cast<uint16_t*>(key_cache) + e, static_cast<uint16_t>(float_to_bf16_bits(value)));
            else
                coherent_storef(static_cast<float*>(key_cache) + e, value);
        }
    };
    if constexpr (kRopeInWave) {
        static_assert((kMaxGroup + 2) * dh <= kThreads, "one block element per thread");
        const int t = static_cast<int>(tid());
        const float partner = __shfl_xor(held, half);  // a wave holds whole heads: dh divides 64
        const int d = t % dh, pair = d % half;
        if (t < qk) {
            const float c = sh.rope_cs[pair], sn = sh.rope_cs[half + pair];
            const float value = d < half ? N::round(N::round(held * c) - N::round(partner * sn))
                                         : N::round(N::round(held * c) + N::round(partner * sn));
            sh.rotated[t] = value;
            if constexpr (kMfma)
                sh.rotated_bits[t] = static_cast<uint16_t>(__float_as_uint(value) >> 16);
            if (chunk == 0) {
                wait_stores();
                store_rotated(t, value);
            }
        }
        block_sync(sh);
    } else {
        block_sync(sh);
        for (int index = tid(); index < (group + 1) * half; index += kThreads) {
            const int head = index / half, pair = index - head * half;
            const float c = sh.rope_cs[pair], sn = sh.rope_cs[half + pair];
            const float a = sh.region[head * dh + pair], b = sh.region[head * dh + pair + half];
            const float lo = N::round(N::round(a * c) - N::round(b * sn));
            const float hi = N::round(N::round(b * c) + N::round(a * sn));
            sh.rotated[head * dh + pair] = lo;
            sh.rotated[head * dh + pair + half] = hi;
            if constexpr (kMfma) {
                sh.rotated_bits[head * dh + pair] = static_cast<uint16_t>(__float_as_uint(lo) >> 16);
                sh.rotated_bits[head * dh + pair + half] = static_cast<uint16_t>(__float_as_uint(hi) >> 16);
            }
        }
        block_sync(sh);  // the region is dead: the scores may overwrite it
        if (chunk == 0)
            for (int index = tid(); index < qk; index += kThreads)
                store_rotated(index, sh.rotated[index]);
    }

    const float scale = 1.0f / sqrtf(static_cast<float>(dh));
    const float divisor = sqrtf(static_cast<float>(dh));
    float* scores = sh.region;  // [group][span]
    auto score_of = [&](float dot) {
        const float rounded = N::round(dot);
        return BF16 ? N::round(rounded * scale) : rounded / divisor;
    };
    // Matrix path: eight bf16 values of `src` as four packed pairs.
    auto pack8 = [](const float* src) {
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            v[q] = pack_bf16(src[2 * q], src[2 * q + 1]);
        return v;
    };
    // Matrix path: V rows of the PB positions from tile first_tile of the chunk; the wave writes
    // its tile wave + 8 j of the block (vb: that tile's rows).
    uint16_t* vt = sh.vt;
    // V is staged as it is stored, a row per position (`kVRow` apart), one 16-byte store per lane
    // and 32 dims; P V's B operand (dim 16 n + tr at 8 positions) then comes from two transposing
    // reads, ds_read_b64_tr_b16: within a 16-lane group, lane j names row 4 h + j / 4, dims
    // 16 n + 4 (j % 4) .. + 3, and lane i receives element i % 4 of lanes 4 e + i / 4, e = 0..3,
    // i.e. dim 16 n + i of the group's four rows.
    auto write_v = [&](int first_tile, int j, const u32x4* vb) {
        const int tile = wave + j * kWaves;
        const int row = tile * kTile + tr;
        const bool current = begin + (first_tile + tile) * kTile + tr == position;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const u32x4 now = *reinterpret_cast<const u32x4*>(sh.vcur_bits + 32 * k + 8 * tk);
            *reinterpret_cast<u32x4*>(vt + row * kVRow + 32 * k + 8 * tk) = current ? now : vb[k];
        }
    };
    auto v_operand = [&](int q, int n) {
        u32x4 out;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = 32 * q + 8 * tk + 4 * h + (tr >> 2);
            typedef short v4s __attribute__((ext_vector_type(4)));
            const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(vt + row * kVRow + 16 * n + 4 * (tr & 3)));
            const uint2 pair = __builtin_bit_cast(uint2, r);
            out[2 * h] = pair.x;
            out[2 * h + 1] = pair.y;
        }
        return out;
    };
    if constexpr (kMfma) {
        // A: query head tr (zero past the group); the current K row stands in for the
        // position's own tile row.
        // Rows past the group read head 0 (one address per tk, a broadcast) and take zeros:
        // reading row tr put the 16 rows, 256 bytes apart, on the same LDS banks.
        u32x4 qa[KS], kc[KS];
        const u32x4 zero = {0u, 0u, 0u, 0u};
        const int qrow = tr < group ? tr : 0;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const u32x4 q = *reinterpret_cast<const u32x4*>(sh.rotated_bits + qrow * dh + 32 * k + 8 * tk);
            qa[k] = tr < group ? q : zero;
            kc[k] = *reinterpret_cast<const u32x4*>(sh.rotated_bits + group * dh + 32 * k + 8 * tk);
        }
        auto tile_scores = [&](int tile, const u32x4* kb) {
            const int time = begin + tile * kTile + tr;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < KS; ++k)
                acc = mfma_16x16x32_bf16(qa[k], time == position ? kc[k] : kb[k], acc);
            // Lanes 0-15 hold heads 0-3 of their position.
            if (tk == 0 && time < end)
#pragma unroll
                for (int g = 0; g < MG; ++g)
                    if (g < group)
                        scores[g * span + time - begin] = score_of(acc[g]);
        };
#pragma unroll
        for (int j = 0; j < TW; ++j)
            if ((wave + j * kWaves) * kTile < span)
                tile_scores(wave + j * kWaves, kfirst[j]);
        // Tiles past the preloaded ones (chunks longer than TW * kWaves tiles): kGroup per wave
        // in flight at once, one wait per group instead of one per tile (tiles past the chunk
        // read zeros without memory traffic).
        constexpr int kGroup = KS <= 2 ? 7 : 4;  // wider heads do not fit seven tiles in registers
        for (int tile0 = wave + TW * kWaves; tile0 * kTile < span; tile0 += kGroup * kWaves) {
            u32x4 kb[kGroup][KS];
#pragma unroll
            for (int gi = 0; gi < kGroup; ++gi)
                load_tile(krsrc, tile0 + gi * kWaves, kb[gi]);
#pragma unroll
            for (int gi = 0; gi < kGroup; ++gi)
                if ((tile0 + gi * kWaves) * kTile < span)
                    tile_scores(tile0 + gi * kWaves, kb[gi]);
        }
        // The current position's V row, where it lies in the first block (staged during the poll).
#pragma unroll
        for (int j = 0; j < TW; ++j) {
            const int tile = wave + j * kWaves;
            if (tile < live0 && begin + tile * kTile + tr == position)
#pragma unroll
                for (int k = 0; k < KS; ++k)
                    *reinterpret_cast<u32x4*>(vt + (tile * kTile + tr) * kVRow + 32 * k + 8 * tk) =
                        *reinterpret_cast<const u32x4*>(sh.vcur_bits + 32 * k + 8 * tk);
        }
    } else {
        // Scores of rows [begin, end).  Every lane holds its slice of all MG query heads (heads
        // past the group compute values that are never stored) and of the current K row.
        constexpr int kWords = BF16 ? 4 : PV;  // registers per 16-byte slice
        uint32_t qreg[MG][kWords];
        uint32_t kcur[kWords];
#pragma unroll
        for (int g = 0; g <= MG; ++g) {
            const float* src = sh.rotated + (g < MG ? g : group) * dh + col * PV;
            uint32_t* dst = g < MG ? qreg[g] : kcur;
#pragma unroll
            for (int q = 0; q < kWords; ++q)
                dst[q] = BF16 ? pack_bf16(src[2 * q], src[2 * q + 1]) : __float_as_uint(src[q]);
        }
        for (int first = begin; first < end; first += 2 * kBlockRows) {
            u32x4 raw[2];
            if (first == begin) {
                raw[0] = kfirst[0][0];
                raw[1] = kfirst[0][1];
            } else {
                load_rows(krsrc, first, raw);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int time = row_time(first, u);
                const bool current = time == position;
                uint32_t kw[kWords];
#pragma unroll
                for (int q = 0; q < kWords; ++q)
                    kw[q] = current ? kcur[q] : raw[u][q];
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    float dot = 0.0f;
                    if constexpr (BF16) {
                        float a = 0.0f, b = 0.0f;
#pragma unroll
                        for (int q = 0; q < 4; q += 2) {
                            a = dot2_bf16(kw[q], qreg[g][q], a);
                            b = dot2_bf16(kw[q + 1], qreg[g][q + 1], b);
                        }
                        dot = a + b;
                    } else {
#pragma unroll
                        for (int j = 0; j < PV; ++j)
                            dot += __uint_as_float(kw[j]) * __uint_as_float(qreg[g][j]);
                    }
                    dot = group_sum<LRK>(dot);
                    if (g < group && col == LRK - 1 && time < end)
                        scores[g * span + time - begin] = score_of(dot);
                }
            }
        }
    }
    block_sync(sh);

    // Softmax per head, one wave each (warp_softmax_statistics, ops.cuh:457-474): the chunk's
    // maximum and its sum of exp(score - maximum), FP32.  One active chunk rounds the probabilities
    // exp / sum to the storage type at once (ops.cuh:612-623).  Several active chunks first
    // exchange their statistics: every chunk merges all of them in chunk order, M = max_c m_c and
    // S = sum_c s_c exp(m_c - M), and rounds P = exp(score - M) / S to the storage type once
    // (attention_values_group, ops.cuh:636-668), so that P V sees the probabilities eager
    // attention rounds whatever the chunking.
    float* stat_max = sh.small;                    // [group] this chunk's statistics
    float* stat_sum = sh.small + kMaxGroup;
    const bool fused = chunks == 1;
    // Matrix path: the rounded probabilities also go to LDS as the bf16 operands of P V, each
    // head's positions contiguous and zero up to the span's last 32-position step, so that one
    // 16-byte read is a lane's 8 positions.  Chunks too long for the work region pack them from the FP32 values.
    const int span_pad = (span + 31) / 32 * 32;  // P V reads P up to the span's last 32-step
    const int p_offset = (group * span + 7) / 8 * 8;  // floats: after the scores, 16-byte aligned
    // A split chunk also keeps every chunk's statistics after the operands (2 group per chunk).
    const int stat_floats = fused ? 0 : chunks * 2 * group;
    const bool packed_p = kMfma && (p_offset + (group * span_pad + 1) / 2 + 3 + stat_floats) <= kLdsRegionFloats;
    uint16_t* pbits = reinterpret_cast<uint16_t*>(scores + p_offset);  // [group][span_pad]
    auto put_p = [&](int g, int i, float v) { pbits[g * span_pad + i] = static_cast<uint16_t>(__float_as_uint(v) >> 16); };
    // Chunks of at most 6 x 64 positions: the wave's scores stay in registers (R per lane), read
    // once; sums in the same order as the loop below.
    auto register_softmax = [&](auto count) {
        constexpr int R = decltype(count)::value;
        const float* row = scores + wave * span;
        float v[R], e[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int i = lane + 64 * k;
            v[k] = i < span ? row[i] : -INFINITY;
        }
        float m = v[0];
#pragma unroll
        for (int k = 1; k < R; ++k)
            m = fmaxf(m, v[k]);
        m = lane_value(group_max(m, 64), 63);
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < R; ++k) {
            e[k] = lane + 64 * k < span ? expf(v[k] - m) : 0.0f;
            sum += e[k];
        }
        sum = lane_value(group_sum<64>(sum), 63);
        if (fused)
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int i = lane + 64 * k;
                if (i < span_pad)
                    put_p(wave, i, N::round(e[k] / sum));  // 0 past the span
            }
        if (lane == 63) {
            stat_max[wave] = m;
            stat_sum[wave] = sum;
        }
    };
    if (wave < group && packed_p && span_pad <= 3 * 64) {
        register_softmax(std::integral_constant<int, 3>{});  // spans up to 192
    } else if (wave < group && packed_p && span <= 4 * 64) {
        register_softmax(std::integral_constant<int, 4>{});  // P V reads P up to the span's last 32-step
    } else if (wave < group && packed_p && span <= 6 * 64) {
        register_softmax(std::integral_constant<int, 6>{});
    } else if (wave < group) {
        // Longer chunks: unrolled, so that several LDS reads are in flight.
        float* row = scores + wave * span;
        float m = -INFINITY;
#pragma unroll 4
        for (int i = lane; i < span; i += 64)
            m = fmaxf(m, row[i]);
        m = lane_value(group_max(m, 64), 63);
        float sum = 0.0f;
#pragma unroll 4
        for (int i = lane; i < span; i += 64) {
            const float e = expf(row[i] - m);
            if (fused)
                row[i] = e;
            sum += e;
        }
        sum = lane_value(group_sum<64>(sum), 63);
        if (fused) {
#pragma unroll 4
            for (int i = lane; i < span; i += 64) {
                const float v = N::round(row[i] / sum);
                row[i] = v;
                if (packed_p)
                    put_p(wave, i, v);
            }
            if (packed_p)
                for (int i = span + lane; i < span_pad; i += 64)
                    put_p(wave, i, 0.0f);
        }
        if (lane == 63) {
            stat_max[wave] = m;
            stat_sum[wave] = sum;
        }
    }
    // One chunk on the matrix path publishes straight from the P V accumulators of waves 0-3:
    // the K row store (and every earlier store) completes before this barrier.
    if (kMfma && fused)
        wait_stores();
    block_sync(sh);

    const int outputs = group * dh;
    // The head's split-attention exchange block: every chunk's (max, sum) per query head, then
    // every chunk's FP32 partials, [chunk][output].  Strides use the plan's chunk count; `chunks`
    // of them are active.  (Read
    // only on the split path: computed before the branch, its launch-record reads cost the fused
    // path 0.1-0.2 us per layer.)
    auto stats_block = [&]() {
        // attention_part_words(s) from the group and the compile-time head width, without its
        // division of the head counts.
        return L.exchange + L.xl.parts + static_cast<size_t>(kv_head) * s.attention_chunks * static_cast<size_t>(group * (dh + 2));
    };
    if (!fused) {
        // This chunk's (max, sum) per head go out as epoch-tagged exchange words; every chunk of
        // the head then reads all chunks' words, this chunk's own from LDS: one load per word
        // (waves past the words issue none), and a round with words missing re-reads only those.
        const uint32_t stat_epoch = L.epoch_of(step, layer, kPhaseAttnStats);
        inject_delay(__LINE__);
        if (tid() < 2 * group) {
            const int g = static_cast<int>(tid()) >> 1;
            const float value = (tid() & 1) ? stat_sum[g] : stat_max[g];
            coherent_store64(stats_block() + static_cast<size_t>(chunk) * 2 * group + tid(),
                             (static_cast<uint64_t>(stat_epoch) << 32) | __float_as_uint(value));
        }
        const int stat_words = stat_floats;  // [chunk][max, sum of each head]
        // After the operands, or after the scores (check_shape: they fit the work region).
        const int stats_offset = packed_p ? (p_offset + (group * span_pad + 1) / 2 + 3) / 4 * 4 : p_offset;
        float* all_stats = scores + stats_offset;
        const uint64_t* stats = stats_block();
        inject_delay(__LINE__);
        for (int base = 0; base < stat_words; base += kThreads) {  // block-uniform
            const int j = base + static_cast<int>(tid());
            const bool wanted = j < stat_words && j / (2 * group) != chunk;
            uint64_t w = 0;
            if (wanted)
                w = coherent_load64(stats + j);
            bool have = !wanted || static_cast<uint32_t>(w >> 32) == stat_epoch;
            uint32_t spins = 0;
            while (!__all(have) && !sh.aborted) {  // per wave, the block meets after the loop
                __builtin_amdgcn_s_sleep(1);
                if ((tid() & 63) == 0)
                    stuck(L.exchange, L.xl, ++spins, sh);
                if (!have) {
                    w = coherent_load64(stats + j);
                    have = static_cast<uint32_t>(w >> 32) == stat_epoch;
                }
            }
            if (j < stat_words) {
                const int k = j % (2 * group);
                all_stats[j] = wanted ? __uint_as_float(static_cast<uint32_t>(w))
                                      : ((k & 1) ? stat_sum[k >> 1] : stat_max[k >> 1]);
            }
        }
        block_sync(sh);
        // The merge, one wave per head: lane c takes chunk c's statistics, M = max_c m_c and
        // S = sum_c s_c exp(m_c - M), summed over the lanes in a fixed tree order.  The reference's
        // values task adds the chunks in chunk order, one thread per head (ops.cuh:644-656); that
        // order is an FP32 summation order, not a rounding point of the contract, and a serial
        // chain here cost 1 us per layer at ctx 4096.
        if (wave < group) {
            const int g = wave;
            float m = -INFINITY;
            for (int c = lane; c < chunks; c += 64)
                m = fmaxf(m, all_stats[c * 2 * group + 2 * g]);
            m = lane_value(group_max(m, 64), 63);
            float part = 0.0f;
            for (int c = lane; c < chunks; c += 64)
                part = fmaf(all_stats[c * 2 * group + 2 * g + 1], expf(all_stats[c * 2 * group + 2 * g] - m), part);
            const float total = lane_value(group_sum<64>(part), 63);
            // The same wave rounds its head's probabilities with the merged statistics: into the
            // packed P V operands only (up to three per lane read at once), or back into the
            // scores, which P V then reads.
            float* row = scores + g * span;
            if (packed_p && span_pad <= 3 * 64) {
                float v[3];
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const int i = lane + 64 * k;
                    v[k] = i < span ? row[i] : 0.0f;
                }
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const int i = lane + 64 * k;
                    if (i < span_pad)
                        put_p(g, i, i < span ? N::round(expf(v[k] - m) / total) : 0.0f);
                }
            } else {
#pragma unroll 4
                for (int i = lane; i < (packed_p ? span_pad : span); i += 64) {
                    const float p = i < span ? N::round(expf(row[i] - m) / total) : 0.0f;
                    if (i < span && !packed_p)
                        row[i] = p;
                    if (packed_p)
                        put_p(g, i, p);
                }
            }
        }
        block_sync(sh);
    }

    // group * dh <= kThreads: each thread owns at most one output element.
    const int mine = tid();
    const bool owner = mine < outputs;
    float out = 0.0f;
    if constexpr (kMfma) {
        // Wave n < dh / 16 accumulates output dims 16 n .. 16 n + 15 of every head over the
        // chunk's positions, PB at a time: A = probabilities of head tr at 8 consecutive
        // positions (zero past the group or the span), B = dim 16 n + tr of the same positions.
        f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
        const int n = wave;
        // The next block's V tiles load while this block's P V runs.
        u32x4 vnext[TW][KS];
        for (int first = 0; first < span; first += PB) {
            const int steps = (min(span - first, PB) + 31) / 32;  // 32-position steps of this block
            if (first > 0) {
                block_sync(sh);  // the previous block's V rows have been read
#pragma unroll
                for (int j = 0; j < TW; ++j)
                    if (wave + j * kWaves < min(kBlockTiles, 2 * steps))
                        write_v(first / kTile, j, vnext[j]);
                block_sync(sh);
            }
            if (first + PB < span)  // block-uniform
#pragma unroll
                for (int j = 0; j < TW; ++j)
                    load_tile(vrsrc, (first + PB) / kTile + wave + j * kWaves, vnext[j]);
            if (n < dh / 16 && packed_p) {
                const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int q = 0; q < PB / 32; ++q) {
                    if (q >= steps)
                        break;
                    const int t0 = first + 32 * q + 8 * tk;
                    const u32x4 vb = v_operand(q, n);
                    const u32x4 p = *reinterpret_cast<const u32x4*>(pbits + (tr < group ? tr : 0) * span_pad + t0);
                    const u32x4 pa = tr < group ? p : zero;
                    o = mfma_16x16x32_bf16(pa, vb, o);
                }
            } else if (n < dh / 16) {
#pragma unroll
                for (int q = 0; q < PB / 32; ++q) {
                    if (q >= steps)
                        break;
                    const int t0 = first + 32 * q + 8 * tk;
                    const u32x4 vb = v_operand(q, n);
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        p[e] = tr < group && t0 + e < span ? scores[tr * span + t0 + e] : 0.0f;
                    o = mfma_16x16x32_bf16(pack8(p), vb, o);  // rounded probabilities: exact
                }
            }
        }
        // Every load of the task has returned (the last block loaded no next V tiles; waves past
        // the live tiles never read theirs): saying so before any store lets the publishes below
        // issue back to back, and leaves the task with no load in flight.  A task that ended
        // with loads the compiler still counted as pending made the dispatcher, where every
        // task's paths merge, wait for vmcnt(2) after each task's end barrier: on a task that
        // had just published, for its stores to complete (about 1 us).
        wait_vmem<0>();
        if (fused) {
            // Lanes 0-15 of wave n hold output dims 16 n + l of every head of the group.  The
            // destination and epoch are read from the LDS launch record once, before the stores
            // (after each store the compiler would read them again).
            const uint32_t out_epoch = L.epoch_of(step, layer, kPhaseAttn);
            uint64_t* const attn_words = L.exchange + L.xl.attn;
            if (n < dh / 16 && tk == 0)
#pragma unroll
                for (int g = 0; g < MG; ++g)
                    if (g < group)
                        publish_element<BF16>(attn_words, (first_head + g) * dh + 16 * n + tr, N::round(o[g]), out_epoch);
            return;
        }
        float* results = sh.rotated;  // [group][dh]: the unrotated heads are dead
        if (n < dh / 16 && tk == 0)
#pragma unroll
            for (int g = 0; g < MG; ++g)
                if (g < group)
                    results[g * dh + 16 * n + tr] = o[g];
        block_sync(sh);
        if (owner)
            out = results[mine];
    } else {
        // P*V over rows [begin, end): each lane accumulates its slice for every head.
        float vnow[PV];
#pragma unroll
        for (int j = 0; j < PV; ++j)
            vnow[j] = sh.vcur[col * PV + j];
        float acc[MG * PV];
#pragma unroll
        for (int n = 0; n < MG * PV; ++n)
            acc[n] = 0.0f;
        for (int first = begin; first < end; first += 2 * kBlockRows) {
            u32x4 raw[2];
            if (first == begin) {
                raw[0] = vfirst[0][0];
                raw[1] = vfirst[0][1];
            } else {
                load_rows(vrsrc, first, raw);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int time = row_time(first, u);
                const bool inside = time < end;
                const bool current = time == position;
                float v[PV];
#pragma unroll
                for (int j = 0; j < PV; ++j)
                    v[j] = current ? vnow[j] : N::elem(raw[u], j);
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    // Rows past the chunk, and heads past the group, read in-bounds LDS and weigh 0.
                    const float read = scores[g * span + time - begin];
                    const float p = inside && g < group ? read : 0.0f;
#pragma unroll
                    for (int j = 0; j < PV; ++j)
                        acc[g * PV + j] += p * v[j];
                }
            }
        }
        // Reduce over the rows a wave holds (lanes with equal col), then over waves.
        residue_sum<LRK>(acc);
        block_sync(sh);  // probabilities are dead
        float* reduction = sh.region;  // [wave][group][dh]
        if (sub == 0)
#pragma unroll
            for (int g = 0; g < MG; ++g)
                if (g < group)
#pragma unroll
                    for (int j = 0; j < PV; ++j)
                        reduction[(wave * group + g) * dh + col * PV + j] = acc[g * PV + j];
        block_sync(sh);
        if (owner)
            for (int w = 0; w < kWaves; ++w)
                out += reduction[w * group * dh + mine];
    }

    const uint32_t out_epoch = L.epoch_of(step, layer, kPhaseAttn);
    uint64_t* attn = L.exchange + L.xl.attn;
    if (fused) {
        wait_stores();  // the K row is in the cache before anyone sees this output
        if (owner)
            publish_element<BF16>(attn, first_head * dh + mine, N::round(out), out_epoch);
        return;
    }
    // Split context: every chunk publishes its FP32 partial P V as exchange words, then merges a
    // block of the group's outputs.  Chunk m merges outputs [m per, (m + 1) per): it reads those
    // outputs' partials from every chunk (a run of `per` adjacent words per chunk, where a
    // cyclic assignment read every word from its own line), adds them in chunk order
    // (output_projection, ops.cuh:718-728), rounds the sum once and publishes it.  The merge is
    // spread over all the head's chunk workers (one merger reading every chunk's whole partial
    // finished about 6 us after the other chunks at ctx 4096), and no arrival counter stands
    // between a chunk and the merge: the words carry the epoch.
    const uint32_t part_epoch = L.epoch_of(step, layer, kPhaseAttnPart);
    if (chunk == 0)
        wait_stores();  // the K row chunk 0 stored is in the cache before any output of the head is published
    const int chunk_stride = s.attention_chunks;
    uint64_t* partial_block = stats_block() + static_cast<size_t>(chunk_stride) * 2 * group;
    inject_delay(__LINE__);
    if (owner)
        coherent_store64(partial_block + static_cast<size_t>(chunk) * outputs + mine,
                         (static_cast<uint64_t>(part_epoch) << 32) | __float_as_uint(out));
    const int per = (outputs + chunks - 1) / chunks;  // outputs per merging chunk
    const int first_out = chunk * per;
    const int owned = max(0, min(per, outputs - first_out));
    const int words = chunks * per;                    // [chunk][output of the block]
    float* own = sh.region;                  // [outputs]: this chunk's partial, for its own slots
    float* merge = sh.region + kMaxThreadsPadded;  // [chunk][per]
    static_assert(2 * kMaxThreadsPadded <= kLdsRegionFloats, "merge slots exceed the work region");
    block_sync(sh);  // P V's LDS reads are done
    if (owner)
        own[mine] = out;
    // One load per slot (this chunk's own from LDS), and a round re-reads only the missing.
    inject_delay(__LINE__);
    for (int base = 0; base < words; base += kThreads) {  // block-uniform
        const int j = base + static_cast<int>(tid());
        const int c = j / per, k = j - c * per;
        const bool wanted = j < words && k < owned && c != chunk;
        const uint64_t* word = partial_block + static_cast<size_t>(c) * outputs + first_out + k;
        uint64_t w = 0;
        if (wanted)
            w = coherent_load64(word);
        bool have = !wanted || static_cast<uint32_t>(w >> 32) == part_epoch;
        uint32_t spins = 0;
        while (!__all(have) && !sh.aborted) {  // per wave, the block meets after the loop
            __builtin_amdgcn_s_sleep(1);
            if ((tid() & 63) == 0)
                stuck(L.exchange, L.xl, ++spins, sh);
            if (!have) {
                w = coherent_load64(word);
                have = static_cast<uint32_t>(w >> 32) == part_epoch;
            }
        }
        if (j < words)
            merge[j] = wanted ? __uint_as_float(static_cast<uint32_t>(w)) : (k < owned ? own[first_out + k] : 0.0f);
    }
    block_sync(sh);
    if (static_cast<int>(tid()) < owned) {
        // In chunk order, 16 LDS reads issued at a time (a loop of read-then-add would pay one
        // LDS round trip per chunk).
        const int k = tid();
        float total = 0.0f;
        for (int c0 = 0; c0 < chunks; c0 += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                v[u] = merge[(c0 + u < chunks ? c0 + u : 0) * per + k];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (c0 + u < chunks)
                    total += v[u];
        }
        publish_element<BF16>(attn, first_head * dh + first_out + k, N::round(total), out_epoch);
    }
}

// Wo rows plus the residual (ops.cuh:718-734): r = round(round(Wo a) + x).
template <bool BF16, int VPL>
__device__ __forceinline__ void op_output_projection(const Launch<BF16>& L, const ti_task_record& t, int step,
                                                    ti_token_id token, Shared& sh, int warm_begin, int warm_end)
{
    using N = Num<BF16>;
    const int d = hidden_size<BF16, VPL>(L);
    const int layer = static_cast<int>(t.layer);
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseR);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    float* residual = sh.small;  // rows [begin, end)
    const uint32_t row_bytes = static_cast<uint32_t>(d) * N::kBytes;
    auto prepare = [&]() {
        // While the attention output is awaited, rows [warm_begin, warm_end) of the layer's FFN,
        // the first weight pass of this worker's next task, come into L2 (gate and up rows, one
        // dword load per 128-byte line); the loads return before the poll's reads issued after them.
        uint32_t warm = 0;
        if (warm_begin >= 0) {
            const int lines_per_row = static_cast<int>(row_bytes / 128u);
            const int line = static_cast<int>(tid());
            const int row = warm_begin + line / (2 * lines_per_row);
            const int part = line % (2 * lines_per_row);
            if (row < warm_end) {
                const char* at = L.layer_weight(layer, part < lines_per_row ? L.layout.Wgate : L.layout.Wup) +
                                 static_cast<size_t>(row) * row_bytes + static_cast<size_t>(part % lines_per_row) * 128u;
                warm = *global(reinterpret_cast<const uint32_t*>(at));
            }
        }
        for (int i = begin + static_cast<int>(tid()); i < end; i += kThreads)
            residual[i - begin] = input_element(L, layer, step, token, i, sh);
        poll_input<BF16>(L.exchange + L.xl.attn, d, L.group * L.shape.head_dim,
                   L.epoch_of(step, layer, kPhaseAttn), L.exchange, L.xl, sh,
                   [&](int i, uint32_t p) {
                       sh.vec[i] = N::from_payload(p);
                       sh.vbits[i] = static_cast<uint16_t>(p);
                   });
        asm volatile("" ::"v"(warm));
        if (begin == 0 && L.block_trace)  // scratch intermediates only on traced launches
            for (int i = tid(); i < d; i += kThreads)
                N::store(L.scratch, L.layout.attention + i, sh.vec[i]);
    };
    gemv<BF16, VPL, 1, 2>(L.layer_weight(layer, L.layout.Wo), [&](int, int row) { return static_cast<uint32_t>(row) * row_bytes; },
                       begin, end, d, sh, prepare,
                       [&]() { return InputSlice<VPL>(gemv_input<BF16>(sh), RowGeometry<BF16>(d).col, RowGeometry<BF16>(d).lr); },
                       [&](int row, const float* dots) {
                           const float r = N::round(N::round(dots[0]) + residual[row - begin]);
                           if (L.block_trace)
                               N::store(L.scratch, L.layout.r + row, r);
                           publish_element<BF16>(L.exchange + L.xl.r, row, r, epoch);
                       });
}

// One FFN product chunk (ops.cuh:739-757): z = RMSNorm(r); p = round(round(silu(round(gate))) *
// round(up)) for rows [begin, end), published into the exchange's product vector (phase
// kPhaseFfn) for the down projection (op_down).
//
// A lane group takes row i's gate and up slices in one pass (2 x VPL 16-byte vectors per lane); D
// passes are in flight per wave.  Waves 1-7 issue all of theirs before the task waits for r; wave
// 0 issues one, polls r alone and issues the rest.  A wave's loads return in issue order, so
// polling from waves with D passes queued saw r only when those passes had drained, 5-7 us after
// the chunk began (the burst is 48 MB across the chip); wave 0 sees it about 2 us sooner.  The
// products wait in LDS and are published after the pass loop: a store inside it would make each
// pass's wait a wait for every load in flight (loads and stores share vmcnt).
template <bool BF16, int VPL>
__device__ __forceinline__ void op_ffn(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    constexpr int PV = N::kPerVec;
    constexpr int NV = 2 * VPL;                      // vectors per lane and row: gate, up
    constexpr int D = VPL >= 8 ? 1 : (VPL >= 4 ? 2 : 4);  // 2 for Llama-3.2-1B: its 4 passes per chunk in two groups
    constexpr int kOut = VPL * PV;                   // hidden elements per lane of a row
    const int d = hidden_size<BF16, VPL>(L);
    const int layer = static_cast<int>(t.layer);
    const int r0 = static_cast<int>(t.begin), r1 = static_cast<int>(t.end);
    const RowGeometry<BF16> g(d);
    const bool traced = L.block_trace != nullptr;  // scratch intermediates only on traced launches
    // Waves 1-7 wait for their earlier stores (V cache rows of a QKV task) before their loads, as
    // the block-wide poll does after its reads, so that every later publish follows those stores.
    if (g.wave != 0)
        wait_stores();
    // The norm's scale.  fp32: every thread's elements in registers.  bf16: wave 0 alone reads it,
    // ahead of its weights, and leaves it in sh.vbits for rms_apply (LdsScale), so that waves 1-7
    // have no reads older than their weights to wait for before the norm.
    const void* norm_weights = L.layer_weight(layer, L.layout.ffn_norm);
    constexpr int kSlots = hidden_slots<BF16, VPL>();
    const NormScale<kSlots> scale = BF16 ? NormScale<kSlots>{} : load_scale<BF16, kSlots>(norm_weights, d);
    constexpr int kScaleVectors = VPL;  // bf16: 16-byte vectors of the scale per lane of wave 0
    u32x4 scale_bits[kScaleVectors];
    if (BF16 && g.wave == 0) {
        const int vectors = d / PV, lane = static_cast<int>(tid() & 63);
#pragma unroll
        for (int j = 0; j < kScaleVectors; ++j) {
            const int v = lane + 64 * j;
            scale_bits[j] = global(static_cast<const u32x4*>(norm_weights))[v < vectors ? v : 0];
        }
    }
    issue_fence();
    auto row_of = [&](int pass) { return g.first_row(r0, pass) + g.sub; };
    const uint32_t row_bytes = static_cast<uint32_t>(d) * N::kBytes;
    const char* gate = L.layer_weight(layer, L.layout.Wgate) + g.col * 16;
    const char* up = L.layer_weight(layer, L.layout.Wup) + g.col * 16;
    // Lanes past the chunk all read the first 16 bytes of its first row (one cached request
    // per instruction); their product is not kept.
    auto issue = [&](int pass, u32x4* w) {
        const int row = row_of(pass);
        const bool inside = row < r1;
        const size_t at = static_cast<size_t>(inside ? row : r0) * row_bytes - (inside ? 0 : g.col * 16);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const size_t o = at + (inside ? static_cast<size_t>(k) * g.lr * 16 : 0);
            w[k] = load_weights(gate + o);
            w[VPL + k] = load_weights(up + o);
        }
    };
    u32x4 w[D][NV];
    float squares = 0.0f;  // wave 0 delivers every element of r, and the norm statistic with them
    if (g.wave == 0) {
        issue(0, w[0]);
        issue_fence();
        poll_words_one_wave<BF16, kOut * 64>(L.exchange + L.xl.r, d, L.hidden_stride, L.epoch_of(step, layer, kPhaseR),
                                             L.exchange, L.xl, sh, [&](int i, uint32_t p) {
                                                 const float x = N::from_payload(p);
                                                 sh.rsave[i] = x;
                                                 squares = fmaf(x, x, squares);
                                             });
#pragma unroll
        for (int s = 1; s < D; ++s)
            issue(s, w[s]);
    } else {
#pragma unroll
        for (int s = 0; s < D; ++s)
            issue(s, w[s]);
    }
    issue_fence();
    if (BF16 && g.wave == 0) {
        // The poll's reads returned after the scale's (wave 0 issued it first).
        const int vectors = d / PV, lane = static_cast<int>(tid() & 63);
#pragma unroll
        for (int j = 0; j < kScaleVectors; ++j)
            if (lane + 64 * j < vectors)
                reinterpret_cast<u32x4*>(sh.vbits)[lane + 64 * j] = scale_bits[j];
    }
    rms_partial(squares, sh);
    block_sync(sh);
    if (tid() == 0)
        sh.rsave_tag = L.epoch_of(step, layer, kPhaseR);
    if constexpr (BF16)
        rms_apply<BF16, kSlots>(sh.rsave, d, LdsScale{}, L.numeric.rms_norm_eps, sh);
    else
        rms_apply<BF16, kSlots>(sh.rsave, d, RegisterScale<kSlots>{scale}, L.numeric.rms_norm_eps, sh);
    const InputSlice<VPL> in(gemv_input<BF16>(sh), g.col, g.lr);
    const int lane = tid() & 63;
    float* staged = sh.small;  // [row - r0]: the chunk's products (rms_apply's barrier freed it)
    // One product row: gate and up dots, p = round(round(silu(round(gate))) * round(up)).
    auto product_row = [&](const u32x4* wg, const u32x4* wu, int row) {
        float gate_dot = VPL > 1 ? group_sum<64>(in.template dot<BF16>(wg)) : group_sum(in.template dot<BF16>(wg), g.lr);
        float up_dot = VPL > 1 ? group_sum<64>(in.template dot<BF16>(wu)) : group_sum(in.template dot<BF16>(wu), g.lr);
        // The group's sums sit in its last lane (in every lane when the group has <= 16).
        if (g.lr == 64) {
            gate_dot = lane_value(gate_dot, 63);
            up_dot = lane_value(up_dot, 63);
        } else if (g.lr == 32) {
            gate_dot = __shfl(gate_dot, (lane & 32) | 31);
            up_dot = __shfl(up_dot, (lane & 32) | 31);
        }
        const float gr = N::round(gate_dot);
        const float silu = N::round(gr / (1.0f + expf(-gr)));
        if (row < r1 && g.col == g.lr - 1)
            staged[row - r0] = N::round(silu * N::round(up_dot));
    };
    // Whole groups of D passes, without branches, and an explicit wait for each pass's loads, the
    // later passes staying in flight: with a branch in the loop the compiler's count, merged at the
    // loop header, waited for every load in flight.  The last group issues nothing.
    int base = 0;
    for (; g.first_row(r0, base + D) < r1; base += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int pass = base + s;
            wait_vmem<(D - 1) * NV>();
            product_row(&w[s][0], &w[s][VPL], row_of(pass));
            issue(pass + D, w[s]);
        }
    }
    unroll<D>([&](auto step) {
        constexpr int s = decltype(step)::value;
        wait_vmem<(D - 1 - s) * NV>();
        product_row(&w[s][0], &w[s][VPL], row_of(base + s));
    });
    block_sync(sh);
    const uint32_t epoch = L.epoch_of(step, layer, kPhaseFfn);
    for (int row = r0 + static_cast<int>(tid()); row < r1; row += kThreads) {
        const float p = staged[row - r0];
        if (traced)
            N::store(L.scratch, L.layout.product + row, p);
        publish_element<BF16>(L.exchange + L.xl.product, row, p, epoch);
    }
}

// Largest intermediate size whose product vector the down projection stages in the work region
// (bf16 bits, or FP32 values), and the 16-byte vectors of a Wdown row one thread holds at most.
template <bool BF16>
constexpr int max_product()
{
    return BF16 ? 2 * kLdsRegionFloats : kLdsRegionFloats;
}
constexpr int kMaxDownVectorsPerThread = 4;

// y rows [begin, end) (ops.cuh:762-838, reorganized for MI355X): the down projection of the FFN's
// product vector over rows of Wdown, which the runtime re-lays out row-major [hidden][intermediate]
// at upload (ti_relayout_weights), rounded before the residual: y = round(round(Wdown[row] . p) +
// r[row]).  The reference has each FFN chunk write an FP32 partial of every output and this wave
// add the chunks' partials in chunk order; the exact sum is the same and the contract rounds once,
// after it, so only the FP32 summation order differs.  Split that way the reduce wave moved no
// weights and waited a whole exchange round for partials (3.1 us per layer at Llama-3.2-1B widths);
// here the task's Wdown rows (16 KB each, 128 KB per worker) are issued before it waits for p and
// stream while the slowest FFN chunks finish and p crosses the exchange, and the FFN chunks stream
// only gate and up.  Thread t holds vectors t, t + 512, ... (VPT of them) of each row, for G = 16 /
// VPT rows at a time, and its slice of p from LDS; the waves' sums meet in LDS in wave order.
template <bool BF16, int VPT>
__device__ __forceinline__ void op_down(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    using N = Num<BF16>;
    constexpr int kLoads = 16;
    constexpr int G = kLoads / VPT;
    static_assert(G * kWaves <= kMaxTaskRows, "down projection wave sums exceed their LDS slots");
    const int f = L.shape.intermediate_size;
    const int d = hidden_size<BF16, 1>(L);
    const int layer = static_cast<int>(t.layer);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const int vectors = f / N::kPerVec;  // 16-byte vectors of a Wdown row (the launcher checks f)
    const size_t row_bytes = static_cast<size_t>(f) * N::kBytes;
    const char* down = L.layer_weight(layer, L.layout.Wdown);
    const int me = static_cast<int>(tid());
    u32x4 w[kLoads];
    // Rows past the task re-read its first row, vectors past a row its last vector (cached
    // requests); neither is kept.  Every load issues: a conditional issue would make the compiler
    // unsure how many are in flight.
    auto issue = [&](int first) {
        unroll<G>([&](auto gi) {
            constexpr int gg = decltype(gi)::value;
            const int row = first + gg < end ? first + gg : begin;
            const char* base = down + static_cast<size_t>(row) * row_bytes;
            unroll<VPT>([&](auto vi) {
                constexpr int v = decltype(vi)::value;
                const int j = v * kThreads + me;
                w[gg * VPT + v] = load_weights(base + static_cast<size_t>(j < vectors ? j : vectors - 1) * 16);
            });
        });
    };
    issue(begin);
    issue_fence();
    // What the rows' emission needs from the LDS launch record, read while the loads are in
    // flight: after the poll's stores and barriers the compiler would read each field again, a
    // chain of LDS round trips between the last product's arrival and the publish.
    const uint32_t y_epoch = L.epoch_of(step, layer, kPhaseY);
    const uint32_t r_epoch = L.epoch_of(step, layer, kPhaseR);
    uint64_t* const y_words = L.exchange + L.xl.hidden((layer + 1) % 2);
    void* const hidden = (layer + 1) % 2 == 0 ? L.input : L.output;
    float* const block_trace = L.block_trace;
    float* const ffn_trace = L.ffn_trace;
    uint16_t* p_bits = reinterpret_cast<uint16_t*>(sh.region);  // bf16: p as bits
    float* p_values = sh.region;                                  // fp32: p as values
    // The products' first read goes out once half of the rows have arrived: a read samples the
    // exchange when it is issued and returns after the loads before it, so one issued with the
    // rows found the slowest FFN chunks' products missing when it came back, and a second round
    // followed the rows' arrival.
    wait_vmem<kLoads / 2>();
    poll_words<BF16, max_product<BF16>(), false>(L.exchange + L.xl.product, f, 1, L.epoch_of(step, layer, kPhaseFfn), L.exchange,
                                         L.xl, sh, [&](int i, uint32_t payload) {
                                             if constexpr (BF16)
                                                 p_bits[i] = static_cast<uint16_t>(payload);
                                             else
                                                 p_values[i] = __uint_as_float(payload);
                                         });
    block_sync(sh);
    const u32x4* p_vectors = reinterpret_cast<const u32x4*>(sh.region);
    float* wave_sums = sh.small;  // [row of the group][wave]
    const int lane = me & 63, wave = wave_id();
    for (int first = begin; first < end; first += G) {  // block-uniform
        if (first != begin) {
            issue(first);
            wait_vmem<0>();
        }
        float acc[G];
#pragma unroll
        for (int gg = 0; gg < G; ++gg)
            acc[gg] = 0.0f;
        unroll<VPT>([&](auto vi) {
            constexpr int v = decltype(vi)::value;
            const int j = v * kThreads + me;
            const u32x4 pv = j < vectors ? p_vectors[j] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                const u32x4& wv = w[gg * VPT + v];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (BF16)
                        acc[gg] = dot2_bf16(wv[q], pv[q], acc[gg]);
                    else
                        acc[gg] = fmaf(__uint_as_float(wv[q]), __uint_as_float(pv[q]), acc[gg]);
                }
            }
        });
        // All G reductions first, then the stores: a store under a lane mask between them made
        // each row's dot products and DPP steps a serial chain of its own (0.5 us per task).
        group_sum_all<64>(acc);
        if (lane == 63)
#pragma unroll
            for (int gg = 0; gg < G; ++gg)
                wave_sums[gg * kWaves + wave] = acc[gg];
        block_sync(sh);
        if (me < G && first + me < end) {
            const int row = first + me;
            float total = 0.0f;
#pragma unroll
            for (int wv = 0; wv < kWaves; ++wv)
                total += wave_sums[me * kWaves + wv];
            // The residual r: in LDS when this worker's FFN task of the layer read it.
            const float r = sh.rsave_tag == r_epoch
                                ? sh.rsave[row]
                                : N::from_payload(poll_element<BF16>(L.exchange + L.xl.r, row, r_epoch, L.exchange, L.xl, sh));
            const float projected = N::round(total);
            const float y = N::round(projected + r);
            N::store(hidden, row, y);
            if (block_trace)
                global(block_trace)[static_cast<size_t>(layer) * d + row] = y;
            if (ffn_trace)
                global(ffn_trace)[static_cast<size_t>(layer) * d + row] = projected;
            publish_element<BF16>(y_words, row, y, y_epoch);
        }
        block_sync(sh);
    }
}

// The down projection for the launch's intermediate size (vectors per thread fixed by the host).
template <bool BF16>
__device__ __forceinline__ void op_ffn_reduce(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    switch (L.down_vectors) {
    case 1: op_down<BF16, 1>(L, t, step, sh); break;
    case 2: op_down<BF16, 2>(L, t, step, sh); break;
    case 3: op_down<BF16, 3>(L, t, step, sh); break;
    default: op_down<BF16, 4>(L, t, step, sh); break;
    }
}

// The last layer's output (the final norm's input, decoder_stack.py:126-132), raw into the work
// region, and its RMSNorm statistic (rms_partial); visible to every wave on return.
template <bool BF16>
__device__ __forceinline__ void final_input(const Launch<BF16>& L, int d, int step, Shared& sh)
{
    const int layers = L.stack.layers;
    float squares = 0.0f;
    poll_words<BF16>(L.exchange + L.xl.hidden(layers % 2), d, L.hidden_stride, L.epoch_of(step, layers - 1, kPhaseY),
                     L.exchange, L.xl, sh, [&](int i, uint32_t p) {
                         const float x = Num<BF16>::from_payload(p);
                         sh.region[i] = x;
                         squares = fmaf(x, x, squares);
                     });
    rms_partial(squares, sh);
    block_sync(sh);
}

template <bool BF16, int VPL>
__device__ __forceinline__ void op_final_rms_norm(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    const int d = hidden_size<BF16, VPL>(L);
    constexpr int kSlots = hidden_slots<BF16, VPL>();
    const NormScale<kSlots> scale = load_scale<BF16, kSlots>(L.stack_weight(L.stack.final_norm_offset), d);
    final_input(L, d, step, sh);
    rms_apply<BF16, kSlots>(sh.region, d, RegisterScale<kSlots>{scale}, L.numeric.rms_norm_eps, sh, true);
    void* hidden = (L.stack.layers + 1) % 2 == 0 ? L.input : L.output;
    for (int i = static_cast<int>(t.begin) + tid(); i < static_cast<int>(t.end); i += kThreads)
        Num<BF16>::store(hidden, i, sh.vec[i]);
}

// Vocabulary rows [begin, end) of the LM head and their greedy candidate (ops.cuh:851-889):
// logits round to the storage type, then widen; the largest value wins, the lowest ID among
// equals, and any non-finite logit makes the candidate kNonFinite.
template <bool BF16, int VPL>
__device__ __forceinline__ void op_logits(const Launch<BF16>& L, const ti_task_record& t, int step, Shared& sh)
{
    const int d = hidden_size<BF16, VPL>(L);
    const int begin = static_cast<int>(t.begin), end = static_cast<int>(t.end);
    const int lane = tid() & 63, wave = wave_id();
    ti_candidate best{-INFINITY, 0x7fffffff};
    const uint32_t row_bytes = static_cast<uint32_t>(d) * Num<BF16>::kBytes;
    const NormInput<BF16, VPL> norm(L.stack_weight(L.stack.final_norm_offset), d);
    gemv<BF16, VPL, 1, 4>(L.stack_weight(L.stack.lm_head_offset), [&](int, int row) { return static_cast<uint32_t>(row) * row_bytes; },
                       begin, end, d, sh, [&]() { final_input(L, d, step, sh); },
                       [&]() { return norm(sh.region, sh, d, L.numeric.rms_norm_eps); },
                       [&](int row, const float* dots) {
                           const float logit = Num<BF16>::round(dots[0]);
                           global(L.logits)[row] = logit;
                           keep_better(best, {logit, isfinite(logit) ? row : TI_NON_FINITE});
                       });
    // Lanes that emitted hold candidates; reduce the wave, then the block.
    for (int offset = 32; offset > 0; offset >>= 1) {
        ti_candidate other{__shfl_xor(best.value, offset), __shfl_xor(best.id, offset)};
        keep_better(best, other);
    }
    if (lane == 0)
        sh.candidates[wave] = best;
    block_sync(sh);
    if (tid() == 0) {
        ti_candidate result = sh.candidates[0];
        for (int w = 1; w < kWaves; ++w)
            keep_better(result, sh.candidates[w]);
        global(&L.selection_out[t.chunk].value)[0] = result.value;
        global(&L.selection_out[t.chunk].id)[0] = result.id;
        const uint32_t epoch = L.epoch_of(step, L.stack.layers, kPhaseCandidate);
        uint64_t* slot = L.exchange + L.xl.candidates + 2 * static_cast<size_t>(t.chunk);
        inject_delay(__LINE__);
        coherent_store64(slot, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(result.value));
        coherent_store64(slot + 1, (static_cast<uint64_t>(epoch) << 32) | static_cast<uint32_t>(result.id));
    }
}

// Greedy selection over every logits task's candidate (ops.cuh:895-911).  Step 0 of a launch
// reads the candidates a previous launch left (complete at the kernel boundary).  Every thread
// reads its slots at once; if some are late, wave 0 waits on their ID words.
template <bool BF16>
__device__ __forceinline__ ti_token_id greedy(const Launch<BF16>& L, int step, Shared& sh)
{
    const int slots = L.selection_slots;
    const uint32_t epoch = step > 0 ? L.epoch_of(step - 1, L.stack.layers, kPhaseCandidate) : 0u;
    ti_candidate best{-INFINITY, 0x7fffffff};
    const uint64_t* candidates = L.exchange + L.xl.candidates;
    inject_delay(__LINE__);
    for (int base = 0; base < slots; base += kThreads) {  // block-uniform
        const int slot = base + static_cast<int>(tid());
        const bool real = slot < slots;
        const uint64_t* words = candidates + 2 * static_cast<size_t>(real ? slot : 0);
        uint64_t a, b;
        auto read = [&]() {
            a = coherent_load64(words);
            b = coherent_load64(words + 1);
            return step == 0 || (static_cast<uint32_t>(a >> 32) == epoch && static_cast<uint32_t>(b >> 32) == epoch);
        };
        if (!block_sync_and(sh, read())) {
            const int n = slots - base < kThreads ? slots - base : kThreads;
            wait_witnesses(n, [&](int j) { return candidates + 2 * static_cast<size_t>(base + j) + 1; }, epoch, L.exchange,
                           L.xl, sh);
            uint32_t spins = 0;
            while (!block_sync_and(sh, read()) && !sh.aborted) {
                __builtin_amdgcn_s_sleep(2);
                if (tid() == 0)
                    stuck(L.exchange, L.xl, ++spins, sh);
            }
        }
        if (real)
            keep_better(best, {__uint_as_float(static_cast<uint32_t>(a)), static_cast<ti_token_id>(static_cast<uint32_t>(b))});
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
        ti_candidate other{__shfl_xor(best.value, offset), __shfl_xor(best.id, offset)};
        keep_better(best, other);
    }
    if ((tid() & 63) == 0)
        sh.candidates[wave_id()] = best;
    block_sync(sh);
    if (tid() == 0) {
        ti_candidate result = sh.candidates[0];
        for (int w = 1; w < kWaves; ++w)
            keep_better(result, sh.candidates[w]);
        sh.token = result.id;
    }
    block_sync(sh);
    return sh.token;
}

template <bool BF16>
__device__ void record_choice(const Launch<BF16>& L, int step, ti_token_id token)
{
    TILES_GLOBAL int32_t* status = global(L.selection.status);
    if (token == TI_NON_FINITE) {
        status[TI_STATUS_ERROR] = TI_DEVICE_NON_FINITE;
    } else if (token < 0 || token >= L.stack.vocab_size) {
        status[TI_STATUS_ERROR] = TI_DEVICE_TOKEN_RANGE;
    } else {
        global(L.selection.generated)[L.selection.first + step] = token;
        status[TI_STATUS_COUNT] = L.selection.first + step + 1;
        if (token == L.selection.eos_id)
            status[TI_STATUS_EOS] = 1;
    }
}

template <bool BF16, int VPL, int LRK>
__global__ __launch_bounds__(kBlockThreads, 1) void decoder_worker(Launch<BF16> launch)
{
    __shared__ Shared sh;
    // The launch record lives in LDS: referenced from many inlined operations, a kernel
    // argument would be copied to scratch or spread over (and spilled from) SGPRs.
    __shared__ Launch<BF16> record;
    if (tid() == 0) {
        record = launch;
        sh.aborted = 0;
        sh.spin_limit = launch.spin_limit;
        sh.rope_position = -1;
        sh.flag = 0;
        sh.xsave_tag = 0;
        sh.rsave_tag = 0;
    }
    __syncthreads();
    const Launch<BF16>& L = record;
    const bool generating = L.selection.generated != nullptr;
    if (generating && (global(L.selection.status)[TI_STATUS_EOS] != 0 || global(L.selection.status)[TI_STATUS_ERROR] != 0))
        return;
    const ti_worker_task_range stream = load_record(L.streams + blockIdx.x);
    // The worker's instruction records move to LDS once: read from memory as each task
    // starts, every record would cost a dependent memory round trip between two tasks.  The
    // barrier records stay behind (waves synchronize through the exchange words; stepping over
    // each one cost an LDS round trip between two tasks), each kept record with its position in
    // the stream, which indexes the timeline.
    const bool cached = stream.count <= static_cast<uint32_t>(kLdsStreamRecords);
    uint32_t tasks = 0;  // records in sh.stream when cached
    if (cached) {
        for (uint32_t first = 0; first < stream.count; first += kBlockThreads) {  // block-uniform
            const uint32_t i = first + tid();
            const bool inside = i < stream.count;
            const ti_task_record r = load_record(L.instructions + stream.begin + (inside ? i : 0));
            const bool keep = inside && r.opcode != TI_OP_BARRIER;
            // Position among the kept records: kept lanes below in this wave, then earlier waves.
            const uint64_t kept = __ballot(keep);
            const uint32_t lane = tid() & 63;
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(kept >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(kept), 0u));
            if (lane == 0)
                sh.candidates[wave_id()].id = static_cast<int>(__builtin_popcountll(kept));  // free until the first step
            __syncthreads();
            uint32_t before = tasks;
            for (int w = 0; w < wave_id(); ++w)
                before += static_cast<uint32_t>(sh.candidates[w].id);
            uint32_t total = tasks;
            for (int w = 0; w < kWaves; ++w)
                total += static_cast<uint32_t>(sh.candidates[w].id);
            if (keep) {
                sh.stream[before + below] = r;
                sh.stream_index[before + below] = static_cast<uint16_t>(i);
            }
            tasks = total;
            __syncthreads();  // the wave counts are read before the next round writes them
        }
    }
    // Read once: the launch record in LDS would be read again at every task's start and end.
    const bool timeline = L.timeline != nullptr;
    // Positions below this have a short attention of one chunk and one staged V block (see the
    // output projection case below).
    const int quiet_attention =
        min(kWarmPositions, min(L.shape.attention_fused_steps, vt_block_positions(L.shape.head_dim)));
    __syncthreads();
    for (int step = 0; step < L.steps; ++step) {
        // The previous step's K/V cache stores complete before this step publishes anything.
        wait_stores();
        ti_token_id token = L.token_id;
        if (generating) {
            token = greedy(L, step, sh);
            if (blockIdx.x == 0 && tid() == 0)
                record_choice(L, step, token);
        } else if (L.device_tokens != nullptr) {
            token = global(L.device_tokens)[step];
        }
        if (L.stack.full_stack && (token < 0 || token >= L.stack.vocab_size)) {
            return;
        }
        const uint32_t records = cached ? tasks : stream.count;
        for (uint32_t k = 0; k < records; ++k) {
            const ti_task_record task = cached ? sh.stream[k] : load_record(L.instructions + stream.begin + k);
            if (task.opcode == TI_OP_BARRIER)
                continue;  // (uncached streams only) waves synchronize through the exchange words
            // Optional timeline of every instruction, the last step's left in the buffer
            // (diagnostic_context.cu:257-285): this build's record, the 100 MHz device clock
            // (s_memrealtime) at the start, when the first exchange read returned, when the inputs
            // were complete and at the end; or the reference's (launch.cuh:25-28), the shader
            // cycle counter (s_memtime) at the start and end and the device clock at the start in ns.
            if (timeline && tid() == 0) {
                sh.mark_start_cycles = __builtin_amdgcn_s_memtime();
                sh.mark_start = __builtin_amdgcn_s_memrealtime();
                sh.mark_read = 0;
                sh.mark_ready = 0;
            }
            inject_delay(__LINE__);
            switch (task.opcode) {
            case TI_OP_QKV: op_qkv<BF16, VPL, LRK>(L, task, step, token, sh); break;
            case TI_OP_ATTENTION_SCORES: op_attention<BF16, LRK>(L, task, step, sh); break;
            case TI_OP_OUTPUT_PROJECTION: {
                // The first weight pass of the worker's next FFN task comes into L2 while the
                // projection awaits the attention output, but only while the attention is one
                // chunk of at most one staged V block, which reads no memory after its input
                // arrives, and short: the burst then delays little the token waits for.  Measured
                // per 64-token launch on Llama-3.2-1B: -10.9 / -5.1 / +3.6 us per token starting at
                // positions 1 / 64 / 128 (the K/V rows the attention loads before its input poll
                // return later behind it), +16 with a second V block and +24 with split chunks.
                // Cached streams only.
                int warm_begin = -1, warm_end = -1;
                if (cached && L.position + step < quiet_attention)
                    for (uint32_t n = k + 1; n < tasks && n < k + 3u; ++n) {
                        const ti_task_record& next = sh.stream[n];
                        if (next.opcode == TI_OP_FFN && next.layer == task.layer) {
                            const RowGeometry<BF16> g(L.shape.hidden_size);
                            warm_begin = static_cast<int>(next.begin);
                            warm_end = min(static_cast<int>(next.end), warm_begin + g.pass_rows);
                            break;
                        }
                    }
                op_output_projection<BF16, VPL>(L, task, step, token, sh, warm_begin, warm_end);
                break;
            }
            case TI_OP_FFN: op_ffn<BF16, VPL>(L, task, step, sh); break;
            case TI_OP_FFN_REDUCE: op_ffn_reduce<BF16>(L, task, step, sh); break;
            case TI_OP_EMBEDDING: {
                const int d = L.shape.hidden_size;
                const void* row = L.stack_weight(static_cast<size_t>(L.stack.embedding_offset) + static_cast<size_t>(token) * d);
                for (int i = static_cast<int>(task.begin) + tid(); i < static_cast<int>(task.end); i += kThreads)
                    Num<BF16>::store(L.input, i, Num<BF16>::load(row, i));
                break;
            }
            case TI_OP_FINAL_RMS_NORM: op_final_rms_norm<BF16, VPL>(L, task, step, sh); break;
            case TI_OP_LOGITS: op_logits<BF16, VPL>(L, task, step, sh); break;
            default: break;  // attention_values: merged inside the scores tasks
            }
            block_sync(sh);
            if (timeline && tid() == 0) {
                const uint32_t index = stream.begin + (cached ? static_cast<uint32_t>(sh.stream_index[k]) : k);
                if (L.timeline_fields == TI_TIMELINE_FIELDS) {
                    TILES_GLOBAL uint64_t* record = global(L.timeline) + TI_TIMELINE_FIELDS * static_cast<size_t>(index);
                    record[0] = sh.mark_start;
                    record[1] = sh.mark_read;
                    record[2] = sh.mark_ready;
                    record[3] = __builtin_amdgcn_s_memrealtime();
                } else {
                    const uint64_t end_cycles = __builtin_amdgcn_s_memtime();
                    TILES_GLOBAL uint64_t* record =
                        global(L.timeline) + TI_TIMELINE_REFERENCE_FIELDS * static_cast<size_t>(index);
                    record[0] = sh.mark_start_cycles;
                    record[1] = end_cycles;
                    record[2] = sh.mark_start * 10u;  // 100 MHz ticks in ns
                }
            }
        }
        if (sh.aborted) {
            if (tid() == 0 && generating && blockIdx.x == 0)
                global(L.selection.status)[TI_STATUS_ERROR] = TI_DEVICE_SYNC_TIMEOUT;
            return;
        }
        if (generating && token == L.selection.eos_id) {
            return;
        }
    }
}

// ---------------------------------------------------------------- host side of the launch

template <bool BF16, int VPL, int LRK>
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
    L.timeline_fields = b.timeline_fields == TI_TIMELINE_FIELDS ? TI_TIMELINE_FIELDS : TI_TIMELINE_REFERENCE_FIELDS;
    L.spin_limit = worker_spin_limit();
    {
        const int row_vectors = p.shape.intermediate_size * (BF16 ? 2 : 4) / 16;
        L.down_vectors = (row_vectors + kBlockThreads - 1) / kBlockThreads;
    }
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
    L.group = p.shape.query_heads / p.shape.kv_heads;
    L.inv_group = 1.0f / static_cast<float>(L.group);
    L.hidden_stride = row_stride(p.shape.hidden_size, p.workers);
    L.qkv_stride = row_stride(p.shape.hidden_size + 2 * p.shape.kv_heads * p.shape.head_dim, p.workers);
    // Every worker waits on the others, so all p.workers blocks must be resident at once: at most
    // CUs x resident blocks per CU, found once per device.  The launch is an ordinary one.  A
    // cooperative launch would check the same bound, but on this runtime it also binds a
    // device-wide resource to the process's queue, and while one process holds it every other
    // process's cooperative launch fails (hipErrorIllegalState): a host running the tile_runtime
    // CLI beside its own context could not decode.  Nothing in the worker needs that resource;
    // its waits are the exchange polls, bounded by the spin limit, so blocks held off the device by
    // another process's kernels end the launch with TI_DEVICE_SYNC_TIMEOUT instead of a hang.
    const void* function = reinterpret_cast<const void*>(&decoder_worker<BF16, VPL, LRK>);
    static std::atomic<int> resident[kResidencyDevices] = {};
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        return hip_fail(e, "current device");
    if (device < 0 || device >= kResidencyDevices)
        return fail(TI_ERR_INVALID_ARGUMENT, "device index beyond the worker residency table");
    if (resident[device].load(std::memory_order_relaxed) == 0) {
        int cus = 0, per_cu = 0;
        if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess)
            return hip_fail(e, "CU count");
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, function, kBlockThreads, 0)) != hipSuccess)
            return hip_fail(e, "worker occupancy");
        resident[device].store(cus * per_cu, std::memory_order_relaxed);
    }
    if (p.workers > resident[device].load(std::memory_order_relaxed))
        return fail(TI_ERR_INVALID_ARGUMENT, "more workers than the device holds resident at once");
    void* args[] = {&L};
    e = hipLaunchKernel(function, dim3(p.workers), dim3(kBlockThreads), args, 0, stream);
    if (e != hipSuccess)
        return hip_fail(e, "worker launch");
    return TI_OK;
}
} // namespace
} // namespace tiles
