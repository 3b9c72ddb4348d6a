// Device helpers shared by the gfx950 kernels: bf16 rounding, 16-byte vectors, device-coherent
// (sc1) accesses and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace tiles {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ inline float bf16_bits_to_float(uint32_t bits) { return __uint_as_float(bits << 16); }

__device__ inline uint32_t float_to_bf16_bits(float value)
{
    // Round to nearest even; NaN stays a quiet NaN.
    const uint32_t u = __float_as_uint(value);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Storage type of weights, activations and K/V: bf16 (as raw bits) or fp32; math is FP32.
template <bool BF16>
struct Num {
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
    // Element j of a 16-byte vector, widened to FP32.
    __device__ static float elem(const u32x4& v, int j)
    {
        if constexpr (BF16)
            return __uint_as_float((j & 1) ? (v[j >> 1] & 0xffff0000u) : (v[j >> 1] << 16));
        else
            return __uint_as_float(v[j]);
    }
    // The 32-bit payload of a rounded value in an exchange word, and back.
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

// Weights stream once per token: nontemporal 16-byte loads (global_load_dwordx4 ... nt).
__device__ inline u32x4 load_weights(const void* p) { return __builtin_nontemporal_load(static_cast<const u32x4*>(p)); }

// Waits until every earlier memory operation of the wave completed (s_waitcnt vmcnt(0)).
__device__ inline void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Device-coherent accesses: relaxed agent-scope atomics, global_load/store ... sc1.
__device__ inline uint64_t coherent_load64(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_store64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float coherent_loadf(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_storef(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void coherent_store16(uint16_t* p, uint16_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// 16-byte device-coherent loads of K/V rows through a buffer resource (sc1).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ inline u32x4 coherent_load128(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset)
{
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 16);
}

// Butterfly sum / max over aligned groups of `width` lanes (a power of two <= 64).
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

} // namespace tiles
