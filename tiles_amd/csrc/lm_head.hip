// The LM-head step alone: a given hidden vector through the final RMSNorm, the LM-head GEMV and
// greedy selection, run by the decode worker's own logits tasks (op_logits), so that the step is
// timed as one launch of the kernel that runs it inside every decode step.  The worker launch
// takes a program of only the package's logits tasks; its input comes from the exchange, where
// a seed kernel publishes the vector as the last layer's output of the launch's first step.

#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "tileinfer_amd.h"
#include "worker_config.hpp"

namespace tiles {
namespace {

constexpr int kSeedThreads = 256;
constexpr int kSelectThreads = 256;

// Element i of `hidden` (the package's element type) published into the exchange region the
// final norm reads (a bf16 element as a tagged 32-bit half, an fp32 element as an epoch word),
// exactly as the last layer's reduce tasks publish it.
template <bool BF16>
__global__ void __launch_bounds__(kSeedThreads) seed_final_hidden(uint64_t* region, const void* hidden, int d, uint32_t epoch)
{
    for (int i = blockIdx.x * kSeedThreads + threadIdx.x; i < d; i += gridDim.x * kSeedThreads) {
        if constexpr (BF16) {
            const uint32_t bits = static_cast<const uint16_t*>(hidden)[i];
            coherent_store32(reinterpret_cast<uint32_t*>(region) + i, (exchange_tag(epoch) << 16) | bits);
        } else {
            const uint32_t bits = static_cast<const uint32_t*>(hidden)[i];
            coherent_store64(region + i, (static_cast<uint64_t>(epoch) << 32) | bits);
        }
    }
}

// Greedy selection over the logits tasks' candidates (the worker's greedy, ops.cuh:895-911):
// `token` receives the winning ID, or TI_NON_FINITE.  keep_better is associative and
// commutative (a total order on (value, ID) with non-finite first), so the tree order gives the
// sequential result.
__global__ void __launch_bounds__(kSelectThreads) select_candidate(const ti_candidate* slots, int count, ti_token_id* token)
{
    constexpr int kWavesHere = kSelectThreads / 64;
    __shared__ ti_candidate best[kWavesHere];
    ti_candidate mine{-INFINITY, 0x7fffffff};
    for (int i = threadIdx.x; i < count; i += kSelectThreads)
        keep_better(mine, slots[i]);
    for (int offset = 32; offset > 0; offset >>= 1)
        keep_better(mine, ti_candidate{__shfl_xor(mine.value, offset), __shfl_xor(mine.id, offset)});
    if ((threadIdx.x & 63) == 0)
        best[threadIdx.x / 64] = mine;
    __syncthreads();
    if (threadIdx.x == 0) {
        ti_candidate result = best[0];
        for (int w = 1; w < kWavesHere; ++w)
            keep_better(result, best[w]);
        *token = result.id;
    }
}

} // namespace

int enqueue_lm_head_step(hipStream_t stream, const ti_worker_program_view& head, const ti_worker_buffers& b, const void* hidden,
                         ti_token_id* token, hipEvent_t worker_start, hipEvent_t worker_end)
{
    if (!hidden || !token || !b.exchange || !b.selection || head.selection_slots < 1)
        return fail(TI_ERR_INVALID_ARGUMENT, "LM-head step needs a hidden vector, a token slot, the exchange and candidates");
    const int d = head.shape.hidden_size;
    const int layers = head.stack.layers;
    if (d < 1 || layers < 1)
        return fail(TI_ERR_INVALID_ARGUMENT, "LM-head step needs a model with a hidden size and a layer");
    const bool bf16 = head.weight_dtype == TI_DTYPE_BFLOAT16;
    const ExchangeLayout xl = exchange_layout(head.shape, layers, head.selection_slots);
    uint64_t* region = b.exchange + xl.hidden(layers % 2);
    // epoch_of(step 0, layer layers - 1, kPhaseY) of the launch at b.epoch.
    const uint32_t epoch = b.epoch + static_cast<uint32_t>(layers - 1) * kPhases + kPhaseY + 1u;
    const dim3 grid((d + kSeedThreads - 1) / kSeedThreads);
    if (bf16)
        hipLaunchKernelGGL(seed_final_hidden<true>, grid, dim3(kSeedThreads), 0, stream, region, hidden, d, epoch);
    else
        hipLaunchKernelGGL(seed_final_hidden<false>, grid, dim3(kSeedThreads), 0, stream, region, hidden, d, epoch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return hip_fail(e, "LM-head seed launch");
    if (worker_start && (e = hipEventRecord(worker_start, stream)) != hipSuccess)
        return hip_fail(e, "LM-head timing event");
    const int code = enqueue_worker(stream, head, b, 0, ti_token_input{0, nullptr, 1}, ti_selection{}, true);
    if (code != TI_OK)
        return code;
    if (worker_end && (e = hipEventRecord(worker_end, stream)) != hipSuccess)
        return hip_fail(e, "LM-head timing event");
    hipLaunchKernelGGL(select_candidate, dim3(1), dim3(kSelectThreads), 0, stream, b.selection, head.selection_slots, token);
    e = hipGetLastError();
    return e == hipSuccess ? TI_OK : hip_fail(e, "LM-head selection launch");
}

} // namespace tiles
