// Decode worker instantiations for bf16 packages: one kernel per compiled shape.
#include "worker_kernel.hpp"

namespace tiles {

int launch_worker_bf16(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                       ti_token_input token, ti_selection selection)
{
    const int vpl = hidden_vectors_per_lane(p.shape.hidden_size, 2);
    const int lrk = head_vectors(p.shape.head_dim, 2);
#define TILES_LAUNCH(V, K)                                                              \
    if (vpl == V && lrk == K)                                                           \
        return launch_typed<true, V, K>(stream, p, b, position, token, selection);
    TILES_BF16_SHAPES(TILES_LAUNCH)
#undef TILES_LAUNCH
    return fail(TI_ERR_INVALID_ARGUMENT, "no compiled worker for this hidden size and head_dim");
}

std::vector<const void*> worker_functions_bf16()
{
#define TILES_FUNCTION(V, K) reinterpret_cast<const void*>(&decoder_worker<true, V, K>),
    return {TILES_BF16_SHAPES(TILES_FUNCTION)};
#undef TILES_FUNCTION
}

} // namespace tiles
