// Decode worker instantiations for fp32 packages: one kernel per compiled shape.
#include "worker_kernel.hpp"

namespace tiles {

int launch_worker_f32(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                       ti_token_input token, ti_selection selection)
{
    const int vpl = hidden_vectors_per_lane(p.shape.hidden_size, 4);
    const int lrk = head_vectors(p.shape.head_dim, 4);
#define TILES_LAUNCH(V, K)                                                              \
    if (vpl == V && lrk == K)                                                           \
        return launch_typed<false, V, K>(stream, p, b, position, token, selection);
    TILES_F32_SHAPES(TILES_LAUNCH)
#undef TILES_LAUNCH
    return fail(TI_ERR_INVALID_ARGUMENT, "no compiled worker for this hidden size and head_dim");
}

std::vector<const void*> worker_functions_f32()
{
#define TILES_FUNCTION(V, K) reinterpret_cast<const void*>(&decoder_worker<false, V, K>),
    return {TILES_F32_SHAPES(TILES_FUNCTION)};
#undef TILES_FUNCTION
}

} // namespace tiles
