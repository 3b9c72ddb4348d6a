// Streaming decode worker instantiations: bf16 packages of hidden size 2048 (Llama-3.2-1B and
// its relatives), head_dim 64 or 128.  The same kernel source as the exchange worker, built
// with 4 streamer waves that move every weight row through an LDS ring.
#define TILES_RING 1
#include "worker_kernel.hpp"

namespace tiles {

#define TILES_RING_SHAPES(X) X(4, 8) X(4, 16)

bool ring_worker_compiled(const ti_model_shape& s, int dtype)
{
    if (dtype != TI_DTYPE_BFLOAT16 || s.hidden_size != kRingHidden || s.kv_heads <= 0)
        return false;
    const int vpl = hidden_vectors_per_lane(s.hidden_size, 2);
    const int lrk = head_vectors(s.head_dim, 2);
    const long group = s.query_heads / s.kv_heads;
    if (static_cast<long>(s.attention_chunk_steps) * group + 8 + static_cast<long>(s.attention_chunks) * group * 2 >
        kRingRegionFloats)
        return false;
    // An FFN chunk's products stay in LDS between its two phases.
    if (s.ffn_chunks <= 0 || (s.intermediate_size + s.ffn_chunks - 1) / s.ffn_chunks > kMaxTaskRows)
        return false;
#define TILES_MATCH(V, K)                                                                                                \
    if (vpl == V && lrk == K)                                                                                           \
        return true;
    TILES_RING_SHAPES(TILES_MATCH)
#undef TILES_MATCH
    return false;
}

int launch_worker_ring(hipStream_t stream, const ti_worker_program_view& p, const ti_worker_buffers& b, int position,
                       ti_token_input token, ti_selection selection)
{
    const int vpl = hidden_vectors_per_lane(p.shape.hidden_size, 2);
    const int lrk = head_vectors(p.shape.head_dim, 2);
#define TILES_LAUNCH(V, K)                                                              \
    if (vpl == V && lrk == K)                                                           \
        return launch_typed<true, V, K>(stream, p, b, position, token, selection);
    TILES_RING_SHAPES(TILES_LAUNCH)
#undef TILES_LAUNCH
    return fail(TI_ERR_INVALID_ARGUMENT, "no compiled streaming worker for this hidden size and head_dim");
}

std::vector<const void*> worker_functions_ring()
{
#define TILES_FUNCTION(V, K) reinterpret_cast<const void*>(&decoder_worker<true, V, K>),
    return {TILES_RING_SHAPES(TILES_FUNCTION)};
#undef TILES_FUNCTION
}

} // namespace tiles
