// Matrix prefill of a bf16 decoder stack: many prompt positions through every layer at once,
// filling the K/V cache the decode worker then continues from.
#pragma once

#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

#include "tileinfer_amd.h"

namespace tiles {

class MatrixPrefill {
  public:
    // Positions per pass through the layers: the activation buffers hold this many rows.
    static constexpr int kChunkRows = 4096;

    explicit MatrixPrefill(const ti_worker_program_view& program);
    ~MatrixPrefill();
    MatrixPrefill(const MatrixPrefill&) = delete;
    MatrixPrefill& operator=(const MatrixPrefill&) = delete;

    // Whether a package of this kind can be prefilled with matrices (bf16 decoder stacks).
    static bool supports(const ti_worker_program_view& program);

    // Enqueues positions [position, position + count) of the prompt whose token ids are at
    // `tokens` (device memory, `count` of them) on `stream`: every layer's K and V rows of those
    // positions go into `kv`.  The positions before `position` must already be in the cache.
    // Returns a TI_* code; the message is in ti_last_error_message().
    int enqueue(hipStream_t stream, void* kv, const ti_token_id* tokens, int position, int count);

  private:
    ti_worker_program_view p_;
    void* buffer_ = nullptr;  // every activation buffer, kChunkRows rows each
    size_t buffer_bytes_ = 0;
    int layer(hipStream_t stream, void* kv, int layer, int position, int rows);
};

} // namespace tiles
