// Host side of the decode worker's C ABI that is not the worker launch itself: error
// messages, the target description, shape checks, and the small auxiliary kernels (K/V
// snapshot zeroing and widening, snapshot.cu:8-62; the streaming-read roofline probe,
// bandwidth_probe.cu:509-549).
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {

namespace {
thread_local char g_message[512];
} // namespace

const char* last_message() { return g_message; }

void set_last_message(const char* text)
{
    std::strncpy(g_message, text, sizeof g_message - 1);
    g_message[sizeof g_message - 1] = '\0';
}

int fail(int code, const char* text)
{
    set_last_message(text);
    return code;
}

int hip_fail(int hip_error, const char* what)
{
    char buffer[400];
    std::snprintf(buffer, sizeof buffer, "%s: %s", what, hipGetErrorString(static_cast<hipError_t>(hip_error)));
    set_last_message(buffer);
    return TI_ERR_HIP;
}

} // namespace tiles

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
    // Rows split into 16-byte vectors over a power-of-two lane group, 1, 2, 4 or 8 per lane.
    const long hidden_vectors = static_cast<long>(s.hidden_size) * elem / 16;
    if (static_cast<long>(s.hidden_size) * elem % 16 != 0 || !power_of_two(hidden_vectors) || hidden_vectors > 8 * 64)
        return "hidden size unsupported by the compiled worker's 16-byte row lanes";
    if (s.head_dim > kMaxHeadDim || s.head_dim * elem % 16 != 0 || !power_of_two(s.head_dim * elem / 16))
        return "head_dim unsupported by the compiled worker";
    if (!worker_compiled(dtype, hidden_vectors_per_lane(s.hidden_size, elem), head_vectors(s.head_dim, elem)))
        return "no compiled worker for this hidden size and head_dim";
    if (s.kv_heads <= 0 || s.query_heads % s.kv_heads != 0)
        return "invalid GQA grouping";
    const int group = s.query_heads / s.kv_heads;
    if (group > kMaxGroup || group * s.head_dim > kMaxGroupTimesHeadDim)
        return "query group exceeds the compiled worker's limits";
    if (static_cast<long>(s.attention_chunk_steps) * group * elem > kAttentionSharedBytes ||
        static_cast<long>(s.attention_chunk_steps) * group > kRegionFloats)
        return "attention chunk exceeds the compiled worker's LDS";
    // A split chunk keeps its scores and every chunk's statistics in the work region at once.
    if (static_cast<long>(s.attention_chunk_steps) * group + 8 + static_cast<long>(s.attention_chunks) * group * 2 > kRegionFloats)
        return "attention chunk count exceeds the compiled worker's merge capacity";
    if (static_cast<long>(s.max_context) * (s.attention_chunks > 0 ? s.attention_chunks : 1) >= (1L << 31))
        return "context too long for the worker's 32-bit chunk arithmetic";
    // Attention addresses one layer's K (or V) table through a buffer resource with 32-bit
    // offsets, and points rows it masks at offset 2^31, past the table, where the load returns 0.
    if (static_cast<uint64_t>(s.max_context) * static_cast<uint64_t>(s.kv_heads) * static_cast<uint64_t>(s.head_dim) * elem >=
        (1ull << 31))
        return "K/V cache of one layer exceeds the worker's 2 GiB buffer addressing";
    if (s.intermediate_size % 2 != 0)
        return "odd intermediate size";
    // The down projection reads Wdown rows (intermediate elements) as 16-byte vectors, at most
    // kMaxDownVectorsPerThread per thread, and stages the product vector in the work region.
    if (static_cast<long>(s.intermediate_size) * elem % 16 != 0)
        return "intermediate size unsupported by the compiled worker's 16-byte Wdown row vectors";
    if (static_cast<long>(s.intermediate_size) * elem / 16 > 4L * kThreads)
        return "intermediate size exceeds the compiled worker's down projection";
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
    if (b.timeline_fields != 0 && b.timeline_fields != TI_TIMELINE_REFERENCE_FIELDS && b.timeline_fields != TI_TIMELINE_FIELDS)
        return "invalid timeline record size";
    if (p.workers <= 0 || p.workers > 4096)
        return "invalid worker count";
    if (position < 0 || position + steps > p.shape.max_context)
        return "sequence context capacity reached";
    if (p.stack.full_stack && p.selection_slots <= 0)
        return "stack without selection slots";
    if (p.weight_dtype == TI_DTYPE_BFLOAT16 && p.stack.layers > kMaxTaggedLayers)
        return "more layers than the bf16 worker's exchange tags allow (120)";
    // Weight loads address one layer's weights, and the LM head, with 32-bit buffer offsets.
    const uint64_t elem = p.weight_dtype == TI_DTYPE_BFLOAT16 ? 2 : 4;
    if (static_cast<uint64_t>(p.stack.layer_weight_stride) * elem >= kBufferRange ||
        static_cast<uint64_t>(p.stack.vocab_size) * p.shape.hidden_size * elem >= kBufferRange)
        return "weight region exceeds the worker's 2 GiB buffer addressing";
    return {};
}
} // namespace tiles

namespace tiles {
namespace {
std::atomic<uint32_t> g_spin_limit{kSpinLimit};
}
uint32_t worker_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }
} // namespace tiles

extern "C" void ti_set_worker_spin_limit(uint32_t polls) { tiles::g_spin_limit.store(polls, std::memory_order_relaxed); }

namespace tiles {
namespace {
// dst[c][r] = src[r][c] for a rows x cols matrix, through 32 x 32 LDS tiles (256 threads).
template <typename E>
__global__ void transpose_matrix(const E* src, E* dst, int rows, int cols)
{
    __shared__ E tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int y = ty; y < 32; y += 8)
        if (r0 + y < rows && c0 + tx < cols)
            tile[y][tx] = src[static_cast<size_t>(r0 + y) * cols + c0 + tx];
    __syncthreads();
    for (int y = ty; y < 32; y += 8)
        if (c0 + y < cols && r0 + tx < rows)
            dst[static_cast<size_t>(c0 + y) * rows + r0 + tx] = tile[tx][y];
}
} // namespace

int relayout_weights(hipStream_t stream, const ti_worker_program_view& p)
{
    if (!p.weights || p.stack.layers <= 0 || p.shape.hidden_size <= 0 || p.shape.intermediate_size <= 0)
        return fail(TI_ERR_INVALID_ARGUMENT, "incomplete program view");
    const bool bf16 = p.weight_dtype == TI_DTYPE_BFLOAT16;
    const size_t elem = bf16 ? 2 : 4;
    const int f = p.shape.intermediate_size, d = p.shape.hidden_size;
    const size_t bytes = static_cast<size_t>(f) * d * elem;
    void* temporary = nullptr;
    hipError_t e = hipMalloc(&temporary, bytes);
    if (e != hipSuccess)
        return hip_fail(e, "Wdown relayout buffer");
    const dim3 grid((d + 31) / 32, (f + 31) / 32);
    for (int layer = 0; layer < p.stack.layers && e == hipSuccess; ++layer) {
        char* region = static_cast<char*>(const_cast<void*>(p.weights)) +
                       (static_cast<size_t>(p.stack.layer_weights_offset) + static_cast<size_t>(layer) * p.stack.layer_weight_stride +
                        p.layout.Wdown) * elem;
        e = hipMemcpyAsync(temporary, region, bytes, hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess)
            break;
        if (bf16)
            hipLaunchKernelGGL(transpose_matrix<uint16_t>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(temporary),
                               reinterpret_cast<uint16_t*>(region), f, d);
        else
            hipLaunchKernelGGL(transpose_matrix<uint32_t>, grid, dim3(256), 0, stream, static_cast<const uint32_t*>(temporary),
                               reinterpret_cast<uint32_t*>(region), f, d);
        e = hipGetLastError();
    }
    const hipError_t done = hipStreamSynchronize(stream);
    (void)hipFree(temporary);
    if (e != hipSuccess)
        return hip_fail(e, "Wdown relayout");
    if (done != hipSuccess)
        return hip_fail(done, "Wdown relayout");
    return TI_OK;
}
} // namespace tiles

extern "C" int ti_relayout_weights(void* stream, const ti_worker_program_view* program)
{
    if (!program)
        return tiles::fail(TI_ERR_INVALID_ARGUMENT, "null program");
    return tiles::relayout_weights(static_cast<hipStream_t>(stream), *program);
}

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

extern "C" uint32_t ti_epoch_after_generation(uint32_t current, const uint32_t* launch_epochs, int32_t launches,
                                              int32_t generated, int32_t layers)
{
    if (!launch_epochs || launches <= 0)
        return current;
    // The launch that selected the last generated token ran; every later one returned at once.
    const int used = generated > 0 ? (generated + TI_MAX_LAUNCH_STEPS - 1) / TI_MAX_LAUNCH_STEPS : 1;
    if (used >= launches)
        return current;
    const uint32_t step = ti_epochs_per_launch(layers);
    for (int i = used - 1; i + 1 < launches; ++i)
        if (launch_epochs[i + 1] != launch_epochs[i] + step)
            return current;  // wrapped after the stop: the wrap cleared every polled word
    if (current != launch_epochs[launches - 1] + step)
        return current;
    return launch_epochs[used - 1] + step;
}

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
    // Every instantiation of each storage type: the largest registers and LDS, the lowest residency.
    struct Summary { int registers = 0, shared = 0, active = 1 << 30; };
    Summary summary[2];
    for (int bf16 = 0; bf16 < 2; ++bf16) {
        std::vector<std::pair<const void*, int>> functions;
        for (const void* f : bf16 ? worker_functions_bf16() : worker_functions_f32())
            functions.emplace_back(f, kThreads);
        for (const auto& [f, threads] : functions) {
            hipFuncAttributes attributes{};
            int active = 0;
            if ((e = hipFuncGetAttributes(&attributes, f)) != hipSuccess)
                return hip_fail(e, "worker attributes");
            if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&active, f, threads, 0)) != hipSuccess)
                return hip_fail(e, "worker occupancy");
            Summary& t = summary[bf16];
            t.registers = std::max(t.registers, attributes.numRegs);
            t.shared = std::max(t.shared, static_cast<int>(attributes.sharedSizeBytes));
            t.active = std::min(t.active, active);
        }
    }
    out->f32_registers = summary[0].registers;
    out->f32_shared_bytes = summary[0].shared;
    out->f32_active_blocks = summary[0].active;
    out->bf16_registers = summary[1].registers;
    out->bf16_shared_bytes = summary[1].shared;
    out->bf16_active_blocks = summary[1].active;
    out->active_blocks_per_sm = std::min(summary[0].active, summary[1].active);
    out->registers_per_thread = std::max(summary[0].registers, summary[1].registers);
    out->static_shared_bytes = std::max(summary[0].shared, summary[1].shared);
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

namespace tiles {
namespace {

// A worker launch occupies every CU with blocks that wait on each other, so two launches must
// never be on the device together: dispatched side by side from two queues, each could hold CUs
// that the other's remaining blocks need, and both would wait out the spin limit.  Launches from
// different streams of this process (two sequence contexts, say) are therefore ordered here:
// a launch on stream s waits, on the device, for the last launch of another stream on the same
// device to complete.  Launches on one stream are ordered by the stream itself.
struct LaunchOrder {
    std::mutex mutex;
    hipEvent_t last = nullptr;      // recorded after the device's latest ordered launch
    hipStream_t stream = nullptr;   // the stream it was launched on
};
constexpr int kOrderedDevices = 64;
LaunchOrder g_order[kOrderedDevices];

int launch_typed_worker(hipStream_t s, const ti_worker_program_view& program, const ti_worker_buffers& buffers,
                        int32_t position, ti_token_input token, ti_selection selection)
{
    if (program.weight_dtype != TI_DTYPE_BFLOAT16)
        return launch_worker_f32(s, program, buffers, position, token, selection);
    return launch_worker_bf16(s, program, buffers, position, token, selection);
}

} // namespace

int enqueue_worker(hipStream_t s, const ti_worker_program_view& program, const ti_worker_buffers& buffers, int32_t position,
                   ti_token_input token, ti_selection selection, bool order_streams)
{
    if (token.steps < 1 || token.steps > TI_MAX_LAUNCH_STEPS)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid worker launch step count");
    const std::string problem = check_launch_shape(program, buffers, position, token.steps);
    if (!problem.empty())
        return fail(TI_ERR_INVALID_ARGUMENT, problem.c_str());
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &capture);
    if (e != hipSuccess)
        return hip_fail(e, "stream capture status");
    // A captured launch runs when its graph is replayed; the graph's owner orders it.
    if (!order_streams || capture != hipStreamCaptureStatusNone)
        return launch_typed_worker(s, program, buffers, position, token, selection);
    int device = 0;
    if ((e = hipGetDevice(&device)) != hipSuccess)
        return hip_fail(e, "current device");
    if (device < 0 || device >= kOrderedDevices)
        return fail(TI_ERR_INVALID_ARGUMENT, "device index beyond the launch-order table");
    LaunchOrder& order = g_order[device];
    std::lock_guard<std::mutex> lock(order.mutex);
    if (!order.last) {
        if ((e = hipEventCreateWithFlags(&order.last, hipEventDisableTiming)) != hipSuccess) {
            order.last = nullptr;
            return hip_fail(e, "launch-order event");
        }
    } else if (order.stream != s && (e = hipStreamWaitEvent(s, order.last, 0)) != hipSuccess) {
        return hip_fail(e, "order after the previous worker launch");
    }
    const int code = launch_typed_worker(s, program, buffers, position, token, selection);
    if (code != TI_OK)
        return code;
    if ((e = hipEventRecord(order.last, s)) != hipSuccess)
        return hip_fail(e, "record worker launch");
    order.stream = s;
    return TI_OK;
}

} // namespace tiles

extern "C" int ti_enqueue_worker(void* stream, const ti_worker_program_view* program, const ti_worker_buffers* buffers,
                                 int32_t position, ti_token_input token, ti_selection selection)
{
    using namespace tiles;
    if (!program || !buffers)
        return fail(TI_ERR_INVALID_ARGUMENT, "null program or buffers");
    return enqueue_worker(static_cast<hipStream_t>(stream), *program, *buffers, position, token, selection, true);
}
