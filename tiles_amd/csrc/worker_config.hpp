// Compile-time limits of the gfx950 decode worker and the layout of its exchange area,
// shared by the kernel, the launcher and the host runtime.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "tileinfer_amd.h"

namespace tiles {

inline constexpr int kThreads = 512;                // 8 wave64s per worker (2 per SIMD, 256 VGPRs each), one worker per CU
inline constexpr int kMaxHidden = 4096;             // a task's input vector lives in LDS as FP32
inline constexpr int kMaxHeadDim = 128;
inline constexpr int kMaxGroup = 4;                 // query heads per K/V head (registers hold them all)
inline constexpr int kMaxGroupTimesHeadDim = 512;   // attention P*V reduction in LDS (4 x 128)
inline constexpr int kMaxTaskRows = 512;            // rows of one GEMV task kept in LDS
inline constexpr int kWarmPositions = 128;          // positions below which an output projection warms its worker's next FFN rows
inline constexpr int kMaxStreamRecords = 1536;      // a worker's instruction stream cached in LDS (longer ones are read from memory)
// Shared bytes for one attention task's scores of all its query heads, in the package's
// element type (the planner's chunk capacity, plan_core.py:91-97).  Held as FP32 in LDS.
// 8448 bytes are 1056 bf16 steps for a group of 4: a 32,832-position context then splits into
// 32 chunks per K/V head, one attention task per worker on 256 CUs (1024 steps would give 33
// chunks, 264 tasks, and two tasks on 8 workers).
inline constexpr int kAttentionSharedBytes = 8448;
// >= max(kThreads * 8, attention scores, P*V reduction).  A split chunk of the longest steps
// also keeps its packed bf16 P*V operands here after its FP32 scores: 4 x 1056 scores, then
// 3 parts x 4 heads x 1120 padded positions of bf16 = 10,944 floats.
inline constexpr int kRegionFloats = 11008;
inline constexpr uint64_t kBufferRange = 1ull << 31;   // bytes a weight buffer resource addresses
inline constexpr uint32_t kSpinLimit = TI_DEFAULT_SPIN_LIMIT;  // polls before a wait is declared stuck
inline constexpr const char* kAbi = "tileinfer-decoder-v10";
inline constexpr const char* kFingerprint = "decoder-gfx950-wave64-exchange-v4-b512";

// Exchange phases within one (step, layer); the candidates use layer == layers.
inline constexpr int kPhaseQKV = 0;
inline constexpr int kPhaseAttn = 1;
inline constexpr int kPhaseR = 2;
inline constexpr int kPhaseFfn = 3;        // the FFN's products p (the down projection's input)
inline constexpr int kPhaseY = 4;
inline constexpr int kPhaseAttnPart = 5;   // attention chunk partials of a split context
inline constexpr int kPhaseAttnStats = 6;  // attention chunk softmax statistics of a split context
inline constexpr int kPhaseCandidate = 0;
inline constexpr int kPhases = 8;

__host__ __device__ inline uint32_t epochs_per_step(int layers) { return static_cast<uint32_t>(layers + 1) * kPhases; }

// bf16 vector exchanges carry a 16-bit tag of the epoch, which tells epochs apart that are less
// than 65535 apart; one launch spans 64 x 8 x (layers + 1) epochs.
inline constexpr int kMaxTaggedLayers = 120;
static_assert(TI_MAX_LAUNCH_STEPS * kPhases * (kMaxTaggedLayers + 1) < 65535, "tagged exchange epochs");

// The 16-bit tag of an epoch in a bf16 exchange half: never 0 (a cleared word), and distinct
// for epochs less than 65535 apart.
__host__ __device__ inline uint32_t exchange_tag(uint32_t epoch) { return epoch % 65535u + 1u; }

// Greedy order of candidates (ops.cuh:895-911): the larger value wins, the lower ID among equal
// values, and a non-finite candidate wins over everything and stays.
__host__ __device__ inline void keep_better(ti_candidate& best, ti_candidate other)
{
    if (best.id == TI_NON_FINITE)
        return;
    if (other.id == TI_NON_FINITE || other.value > best.value || (other.value == best.value && other.id < best.id))
        best = other;
}

// Word offsets into the exchange area.  Each word: payload in bits 0-31 (one bf16 or fp32
// element, or a candidate field), writer's epoch in bits 32-63.  In bf16, the vectors every
// worker reads (hidden0/1, attn, r, product) hold two elements per word instead, each a 32-bit
// half with a 16-bit epoch tag (worker_kernel.hpp, exchange_tag), and use the first half of their
// region.
struct ExchangeLayout {
    size_t control;      // [0]: nonzero once a worker declared a wait stuck
    size_t hidden0, hidden1;  // layer outputs, alternating like the hidden buffers
    size_t qkv;          // per K/V head: its group's unrotated Q, then K, then V of the current position
    size_t attn;         // merged attention output
    size_t r;            // attention block output
    size_t product;      // the FFN's products p = SiLU(gate) * up, [intermediate] (tagged halves in bf16)
    size_t candidates;   // greedy candidates, 2 words per slot
    size_t parts;        // split attention, per K/V head: every chunk's (max, sum) per query head, then its FP32 partials [chunk][output]
    size_t total;
    // A conditional, not an indexed array: a dynamic index into the launch record would put
    // the whole record in scratch memory.
    __host__ __device__ size_t hidden(int index) const { return index % 2 == 0 ? hidden0 : hidden1; }
};

// Exchange words per split-attention chunk of one K/V head: its (max, sum) for each of the
// group's query heads and its group x head_dim FP32 partial outputs.
__host__ __device__ inline size_t attention_part_words(const ti_model_shape& s)
{
    const size_t group = s.kv_heads > 0 ? static_cast<size_t>(s.query_heads / s.kv_heads) : 0;
    return group * (static_cast<size_t>(s.head_dim) + 2);
}

__host__ __device__ inline ExchangeLayout exchange_layout(const ti_model_shape& s, int layers, int slots)
{
    ExchangeLayout x{};
    const size_t d = static_cast<size_t>(s.hidden_size);
    const size_t kvw = static_cast<size_t>(s.kv_heads) * s.head_dim;
    x.control = 0;
    x.hidden0 = 8;
    x.hidden1 = x.hidden0 + d;
    x.qkv = x.hidden1 + d;
    x.attn = x.qkv + d + 2 * kvw;
    x.r = x.attn + d;
    x.product = x.r + d;
    x.candidates = x.product + static_cast<size_t>(s.intermediate_size);
    x.parts = x.candidates + 2 * static_cast<size_t>(slots > 0 ? slots : 1);
    x.total = x.parts + static_cast<size_t>(s.kv_heads) * s.attention_chunks * attention_part_words(s);
    (void)layers;
    return x;
}

// Word of [Q; K; V] projection row `row` in the packed per-head exchange block.
__host__ __device__ constexpr int qkv_word(int row, const ti_model_shape& s)
{
    const int d = s.hidden_size, dh = s.head_dim, kvw = s.kv_heads * s.head_dim;
    const int group = s.query_heads / s.kv_heads, block = (group + 2) * dh;
    if (row < d)
        return row / (group * dh) * block + row % (group * dh);
    if (row < d + kvw)
        return (row - d) / dh * block + group * dh + (row - d) % dh;
    return (row - d - kvw) / dh * block + (group + 1) * dh + (row - d - kvw) % dh;
}

// qkv_word without integer division, for a head_dim DH fixed at compile time (a power of two)
// and inv_group = 1 / group rounded to FP32: (head + 0.5) / group lies at least 1 / (2 group)
// from an integer, far beyond the product's rounding error, so truncation gives head / group.
template <int DH>
__host__ __device__ constexpr int qkv_slot(int row, int d, int kvw, int group, float inv_group)
{
    static_assert(DH > 0 && (DH & (DH - 1)) == 0, "head_dim must be a power of two");
    const int block = (group + 2) * DH;
    if (row < d) {
        const int head = row / DH;  // shifts: DH is a compile-time power of two
        const int kv_head = static_cast<int>((static_cast<float>(head) + 0.5f) * inv_group);
        return kv_head * block + (head - kv_head * group) * DH + row % DH;
    }
    const bool key = row < d + kvw;
    const int r = key ? row - d : row - d - kvw;
    return r / DH * block + (key ? group : group + 1) * DH + r % DH;
}

// qkv_slot agrees with qkv_word on every row of a shape (checked at compile time below).
template <int DH>
constexpr bool qkv_slot_agrees(int kv_heads, int group)
{
    ti_model_shape s{};
    s.head_dim = DH;
    s.kv_heads = kv_heads;
    s.query_heads = kv_heads * group;
    s.hidden_size = s.query_heads * DH;
    const int kvw = kv_heads * DH;
    for (int row = 0; row < s.hidden_size + 2 * kvw; ++row)
        if (qkv_slot<DH>(row, s.hidden_size, kvw, group, 1.0f / static_cast<float>(group)) != qkv_word(row, s))
            return false;
    return true;
}
static_assert(qkv_slot_agrees<64>(8, 4) && qkv_slot_agrees<64>(8, 3) && qkv_slot_agrees<128>(8, 4) &&
                  qkv_slot_agrees<32>(4, 2) && qkv_slot_agrees<16>(2, 1) && qkv_slot_agrees<64>(64, 3),
              "qkv_slot must place every row where qkv_word does");

// 16-byte vectors a lane holds of a hidden-width row: rows of `hidden` elements of `elem`
// bytes are split over min(64, vectors) lanes.
__host__ __device__ inline int hidden_vectors_per_lane(int hidden, int elem)
{
    const int vectors = hidden * elem / 16;
    return vectors > 64 ? vectors / 64 : 1;
}

// 16-byte vectors in one K/V row (head_dim elements of `elem` bytes): the lanes that hold it.
__host__ __device__ inline int head_vectors(int head_dim, int elem) { return head_dim * elem / 16; }

// Compiled worker shapes, (hidden_vectors_per_lane, head_vectors) pairs per storage type:
// every loop bound and reduction width of a kernel is a compile-time constant, and a kernel
// carries one attention variant (several in one kernel raise register pressure into spills).
// bf16: hidden 128..512 (1), 1024 (2), 2048 (4), 4096 (8); head_dim 8..128.
#define TILES_BF16_SHAPES(X) X(1, 1) X(1, 2) X(1, 4) X(1, 8) X(1, 16) X(2, 8) X(2, 16) X(4, 8) X(4, 16) X(8, 16)
// fp32: hidden 64..256 (1), 512 (2), 1024 (4), 2048 (8); head_dim 8..128.
#define TILES_F32_SHAPES(X) X(1, 2) X(1, 4) X(1, 8) X(1, 16) X(1, 32) X(2, 16) X(4, 16) X(4, 32) X(8, 16) X(8, 32)

inline bool worker_compiled(int dtype, int vpl, int lrk)
{
#define TILES_MATCH(V, K)                                                                                                \
    if (vpl == V && lrk == K)                                                                                           \
        return true;
    if (dtype == TI_DTYPE_BFLOAT16) {
        TILES_BF16_SHAPES(TILES_MATCH)
    } else {
        TILES_F32_SHAPES(TILES_MATCH)
    }
#undef TILES_MATCH
    return false;
}

// Launch of the compiled worker for the program's shape (TI_ERR_INVALID_ARGUMENT when none).
int launch_worker_bf16(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                       ti_token_input token, ti_selection selection);
int launch_worker_f32(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                      ti_token_input token, ti_selection selection);
// Checked worker launch.  With order_streams, a launch waits on the device for the device's last
// launch from another stream to complete (two launches cannot share the device).
int enqueue_worker(hipStream_t s, const ti_worker_program_view& program, const ti_worker_buffers& buffers, int32_t position,
                   ti_token_input token, ti_selection selection, bool order_streams);
// The LM-head step alone (lm_head.hip): `hidden` (device, hidden_size elements of the weight
// type) published as the last layer's output of a launch at buffers.epoch, one step of `head`
// (a program of the package's logits tasks only), then greedy selection of the candidates into
// `token` (device).  The launch uses exchange epochs [buffers.epoch, + ti_epochs_per_launch).
// worker_start / worker_end (optional) are recorded around the worker launch alone.
int enqueue_lm_head_step(hipStream_t stream, const ti_worker_program_view& head, const ti_worker_buffers& buffers,
                         const void* hidden, ti_token_id* token, hipEvent_t worker_start, hipEvent_t worker_end);
std::vector<const void*> worker_functions_bf16();
std::vector<const void*> worker_functions_f32();

// Polls of one worker wait before it declares the exchange stuck, for launches enqueued from now
// on (ti_set_worker_spin_limit; kSpinLimit unless set).
uint32_t worker_spin_limit();

// Rewrites each layer's Wdown region of the device weights in place from the package's
// transposed [intermediate][hidden] to row-major [hidden][intermediate], the layout the worker's
// down projection and the matrix prefill read (ti_relayout_weights).
int relayout_weights(hipStream_t stream, const ti_worker_program_view& program);

// Thread-local message of the last failed call (ti_last_error_message).
const char* last_message();
void set_last_message(const char* text);
int fail(int code, const char* text);        // sets the message, returns `code`
int hip_fail(int hip_error, const char* what);  // "what: <HIP error string>", returns TI_ERR_HIP

// Empty when the compiled worker supports the shape; otherwise the reason.
std::string check_shape(const ti_model_shape& s, int dtype);
std::string check_launch_shape(const ti_worker_program_view& p, const ti_worker_buffers& b, int position, int steps);

} // namespace tiles
