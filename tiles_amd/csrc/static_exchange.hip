// The worker launch for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc): the exchange area, the only scratch memory the
// worker's kernels use beyond the caller's buffers, lives in a file-scope device array instead of
// a caller-owned allocation.  No counterpart exists in the reference.
#include <cstring>
#include <mutex>
#include <string>

#include "device_common.hpp"
#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {
namespace {

// 16 MiB: the exchange area of a hidden-4096 model with 256 FFN chunks and 32 attention chunks
// per K/V head fits (Llama-3.2-1B needs 4.8 MiB).  Each GPU the library runs on holds its own
// copy until the process ends.
constexpr size_t kStaticExchangeWords = size_t(1) << 21;
static __device__ __align__(256) uint64_t scratch[kStaticExchangeWords];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
uint64_t* g_address[kMaxDevices] = {};  // device address of `scratch` on each device, once known

// Zeroes words [0, keep_begin) and [keep_end, total) of the exchange area: every word a launch
// polls, and the control word.  The greedy candidates in between carry a generation's previous
// step into the next launch's first step (which reads them whatever their epoch).
__global__ void clear_exchange(uint64_t* words, size_t keep_begin, size_t keep_end, size_t total)
{
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        if (i < keep_begin || i >= keep_end)
            words[i] = 0;
}

// 1 when a wait of the launch gave up (the control word is set), else 0.
__global__ void read_control(const uint64_t* words, int32_t* out)
{
    if (threadIdx.x == 0 && blockIdx.x == 0)
        *out = words[0] != 0 ? 1 : 0;
}

// The device address of `scratch` on the current device, found with that device current the
// first time the device is used.  Host code passes this address, never the array's name (a
// host-side stand-in), to kernels.
int static_exchange(uint64_t** out)
{
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        return hip_fail(e, "current device");
    if (device < 0 || device >= kMaxDevices)
        return fail(TI_ERR_INVALID_ARGUMENT, "device index beyond the static exchange table");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_address[device]) {
        void* address = nullptr;
        e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return hip_fail(e, "static exchange address");
        g_address[device] = static_cast<uint64_t*>(address);
    }
    *out = g_address[device];
    return TI_OK;
}

} // namespace
} // namespace tiles

extern "C" size_t ti_static_exchange_words(void) { return tiles::kStaticExchangeWords; }

extern "C" int ti_enqueue_worker_static(void* stream, const ti_worker_program_view* program, const ti_worker_buffers* buffers,
                                        int32_t position, ti_token_input token, ti_selection selection, int32_t* sync_timeout)
{
    using namespace tiles;
    if (!program || !buffers)
        return fail(TI_ERR_INVALID_ARGUMENT, "null program or buffers");
    const ExchangeLayout xl = exchange_layout(program->shape, program->stack.layers, program->selection_slots);
    if (xl.total > kStaticExchangeWords)
        return fail(TI_ERR_INVALID_ARGUMENT, "the model's exchange area exceeds the static array (2097152 words)");
    uint64_t* words = nullptr;
    int code = static_exchange(&words);
    if (code != TI_OK)
        return code;
    ti_worker_buffers b = *buffers;
    b.exchange = words;
    b.epoch = 1;
    // Shapes and step counts are checked before anything is enqueued.
    if (token.steps < 1 || token.steps > TI_MAX_LAUNCH_STEPS)
        return fail(TI_ERR_INVALID_ARGUMENT, "invalid worker launch step count");
    const std::string problem = check_launch_shape(*program, b, position, token.steps);
    if (!problem.empty())
        return fail(TI_ERR_INVALID_ARGUMENT, problem.c_str());
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t keep_end = xl.candidates + 2 * static_cast<size_t>(program->selection_slots > 0 ? program->selection_slots : 1);
    hipLaunchKernelGGL(clear_exchange, dim3(256), dim3(256), 0, s, words, xl.candidates, keep_end, xl.total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return hip_fail(e, "clear static exchange");
    // Callers of this entry order their launches themselves (and it creates no event to do so).
    code = enqueue_worker(s, *program, b, position, token, selection, false);
    if (code != TI_OK)
        return code;
    if (sync_timeout) {
        hipLaunchKernelGGL(read_control, dim3(1), dim3(64), 0, s, words, sync_timeout);
        if ((e = hipGetLastError()) != hipSuccess)
            return hip_fail(e, "read static exchange control");
    }
    return TI_OK;
}
