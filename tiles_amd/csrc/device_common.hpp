// Device helpers shared by the gfx950 kernels: bf16 rounding, 16-byte vectors, device-coherent
// (sc1) accesses and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace tiles {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Device memory as the global address space.  Kernels reach their buffers through pointers
// held in a launch record, which the compiler cannot prove global; a generic pointer compiles
// to flat_* instructions, and a flat access also counts against the LDS wait counter, so every
// later LDS wait would also wait for all outstanding weight loads.  global_* instructions
// keep the two counters apart.
#define TILES_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ inline TILES_GLOBAL T* global(T* p)
{
    return (TILES_GLOBAL T*)(p);
}

// A record of 32-bit fields read from device memory (a struct cannot be copied through a
// global-address-space reference).
template <typename T>
__device__ inline T load_record(const T* p)
{
    static_assert(sizeof(T) % 4 == 0, "records are made of 32-bit fields");
    uint32_t words[sizeof(T) / 4];
    const TILES_GLOBAL uint32_t* src = global(reinterpret_cast<const uint32_t*>(p));
#pragma unroll
    for (unsigned i = 0; i < sizeof(T) / 4; ++i)
        words[i] = src[i];
    T out;
    __builtin_memcpy(&out, words, sizeof(T));
    return out;
}

__device__ inline float bf16_bits_to_float(uint32_t bits) { return __uint_as_float(bits << 16); }

// Round to nearest even (NaN stays a NaN) with gfx950's v_cvt_pk_bf16_f32: one instruction,
// where the bit arithmetic with its NaN case compiled to a divergent branch.
__device__ inline uint32_t float_to_bf16_bits(float value)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
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
            return bf16_bits_to_float(global(static_cast<const uint16_t*>(base))[index]);
        else
            return global(static_cast<const float*>(base))[index];
    }
    __device__ static void store(void* base, size_t index, float v)
    {
        if constexpr (BF16)
            global(static_cast<uint16_t*>(base))[index] = static_cast<uint16_t>(float_to_bf16_bits(v));
        else
            global(static_cast<float*>(base))[index] = v;
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

// Two bf16 values in one register, element 0 in the low half.  Exact for values that are
// already bf16 (rounded FP32 values of a bf16 computation).
__device__ inline uint32_t pack_bf16(float lo, float hi)
{
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// c + a.lo * b.lo + a.hi * b.hi for packed bf16 pairs, accumulated in FP32 (v_dot2_f32_bf16).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c)
{
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// D = A B + C on 16x16 FP32 tiles with K = 32 bf16 (v_mfma_f32_16x16x32_bf16): lane l holds
// row l % 16 of A and column l % 16 of B, elements 8 (l / 16) .. 8 (l / 16) + 7 of each as four
// packed pairs, and rows 4 (l / 16) .. 4 (l / 16) + 3 of column l % 16 of C and D.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ inline f32x4 mfma_16x16x32_bf16(const u32x4& a, const u32x4& b, const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Weights stream once per token: nontemporal 16-byte global loads (global_load_dwordx4 ... nt).
// Measured on the FFN's access pattern, these stream at about 7.0 TB/s and buffer-resource loads
// at 5.2-6.0 TB/s, so a lane with no row to load re-reads a row of its task (a cache hit) rather
// than a range-checked buffer load reading zeros.
__device__ inline u32x4 load_weights(const void* p) { return __builtin_nontemporal_load(global(static_cast<const u32x4*>(p))); }

// Keeps memory operations issued before it from being moved after it (and the reverse) by
// the compiler; emits no instruction.  Loads issued before a task waits for its inputs would
// otherwise be sunk next to their first use, after the wait, and their latency would no
// longer overlap it.
__device__ inline void issue_fence() { asm volatile("" ::: "memory"); }

// Waits until every earlier memory operation of the wave completed (s_waitcnt vmcnt(0)).
__device__ inline void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Waits until at most N vector memory operations of the wave are in flight (s_waitcnt vmcnt(N),
// the other counters untouched).  The compiler takes explicit waits into its own count: where
// code paths with different loads in flight merge, it otherwise picks counts that are right for
// one path and make the other wait for loads it does not need.
template <int N>
__device__ inline void wait_vmem()
{
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// f(std::integral_constant<int, I>{}) for I = 0 .. N - 1, in order: an unrolled loop whose index
// is a constant expression in the body (a template argument of wait_vmem, say).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll(const F& f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        unroll<N, I + 1>(f);
    }
}

// Device-coherent accesses: relaxed agent-scope atomics, global_load/store ... sc1.
__device__ inline uint64_t coherent_load64(const uint64_t* p)
{
    return __hip_atomic_load(global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void coherent_store64(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float coherent_loadf(const float* p)
{
    return __hip_atomic_load(global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void coherent_storef(float* p, float v)
{
    __hip_atomic_store(global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t coherent_load32(const uint32_t* p)
{
    return __hip_atomic_load(global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void coherent_store32(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void coherent_store16(uint16_t* p, uint16_t v)
{
    __hip_atomic_store(global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t coherent_fetch_add64(uint64_t* p, uint64_t v)
{
    return __hip_atomic_fetch_add(global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// e^x for x <= 0, bit for bit the device library's expf (verified over every non-positive float
// on gfx950): x log2(e) as a head ph = x * c and a tail pl (the product's rounding error by FMA
// plus x times the tail of log2(e)), then 2^(ph - rint(ph) + pl) by v_exp_f32 scaled by
// 2^rint(ph), and 0 below ln(2^-149).  Without expf's overflow branch, which no x <= 0 takes: 3
// of its 15 instructions.  The constants are the ones that library's code on gfx950 uses.
__device__ __forceinline__ float exp_nonpositive(float x)
{
#pragma clang fp contract(off)
    constexpr float kLog2eHead = 0x1.715476p+0f, kLog2eTail = 0x1.4ae0bep-26f, kUnderflow = -0x1.9d1da0p+6f;
    const float ph = x * kLog2eHead;
    float pl = fmaf(x, kLog2eHead, -ph);
    pl = fmaf(x, kLog2eTail, pl);
    const float e = rintf(ph);
    const float r = __builtin_ldexpf(__builtin_amdgcn_exp2f((ph - e) + pl), static_cast<int>(e));
    return x < kUnderflow ? 0.0f : r;
}

// a / b correctly rounded, from r = 1 / b (itself correctly rounded): q0 = a r is within an ulp of
// a / b, the FMA residual a - b q0 is exact, and q0 + residual * r rounds to a / b (Markstein's
// theorem) while a / b is a normal number, which for b in [1, 2^31) holds from a = kQuotientFloor
// up, and a = 0 gives 0 (callers divide other a in full: quotient_needs_division).  Three
// instructions instead of the division's eleven; equal to IEEE division on 2^32 sampled pairs
// with b in [1, 2^17) and a in [2^-30, 1], and on 2^32 with a in [2^-94, 2^-30).
constexpr float kQuotientFloor = 0x1p-94f;
__device__ __forceinline__ float divide_by(float a, float b, float r)
{
#pragma clang fp contract(off)
    const float q0 = a * r;
    return fmaf(fmaf(-b, q0, a), r, q0);
}
__device__ __forceinline__ bool quotient_needs_division(float a) { return a > 0.0f && a < kQuotientFloor; }

// 16-byte device-coherent loads of K/V rows through a buffer resource (sc1).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ inline u32x4 coherent_load128(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset)
{
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 16);
}

// ---------------------------------------------------------------- cross-lane reductions
//
// DPP lane permutations (GFX9 encodings) run at VALU speed; a __shfl_xor is an LDS-pipe
// permute with its own latency.  Reductions inside 16-lane rows therefore use DPP only.
inline constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]: lane i <- i ^ 1
inline constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]: lane i <- i ^ 2
inline constexpr int kDppRowHalfMirror = 0x141;  // lane i <- 7 - i within each 8 lanes
inline constexpr int kDppRowMirror = 0x140;    // lane i <- 15 - i within each row
inline constexpr int kDppRowRor = 0x120;       // + n: lane i <- (i - n) mod 16 within each row
inline constexpr int kDppRowBcast15 = 0x142;   // lane 15 of each row -> the whole next row
inline constexpr int kDppRowBcast31 = 0x143;   // lane 31 -> rows 2 and 3

// v from the lane the permutation selects; lanes of rows outside kRowMask read 0.
template <int kCtrl, int kRowMask = 0xF>
__device__ inline float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask, 0xF, false));
}

// Sum over aligned groups of `width` lanes (a power of two <= 64, the same in every lane).
// The total lands in the group's last lane, and in every lane of the group when width <= 16.
__device__ inline float group_sum(float v, int width)
{
    if (width >= 2)
        v += dpp<kDppQuadXor1>(v);
    if (width >= 4)
        v += dpp<kDppQuadXor2>(v);
    if (width >= 8)
        v += dpp<kDppRowHalfMirror>(v);
    if (width >= 16)
        v += dpp<kDppRowMirror>(v);
    if (width >= 32)
        v += dpp<kDppRowBcast15, 0xA>(v);  // rows 1, 3 += rows 0, 2
    if (width >= 64)
        v += dpp<kDppRowBcast31, 0xC>(v);  // row 3 += row 1
    return v;
}

// group_sum for a width known at compile time.
template <int W>
__device__ inline float group_sum(float v)
{
    if constexpr (W >= 2)
        v += dpp<kDppQuadXor1>(v);
    if constexpr (W >= 4)
        v += dpp<kDppQuadXor2>(v);
    if constexpr (W >= 8)
        v += dpp<kDppRowHalfMirror>(v);
    if constexpr (W >= 16)
        v += dpp<kDppRowMirror>(v);
    if constexpr (W >= 32)
        v += dpp<kDppRowBcast15, 0xA>(v);
    if constexpr (W >= 64)
        v += dpp<kDppRowBcast31, 0xC>(v);
    return v;
}

// group_sum<W> of N independent values, one DPP step of all of them at a time: the chains
// interleave instead of each paying its dependent-step latency in turn.
template <int W, int N>
__device__ inline void group_sum_all(float (&v)[N])
{
    if constexpr (W >= 2)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppQuadXor1>(v[n]);
    if constexpr (W >= 4)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppQuadXor2>(v[n]);
    if constexpr (W >= 8)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowHalfMirror>(v[n]);
    if constexpr (W >= 16)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowMirror>(v[n]);
    if constexpr (W >= 32)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowBcast15, 0xA>(v[n]);
    if constexpr (W >= 64)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowBcast31, 0xC>(v[n]);
}

// Maximum with the same lane layout as group_sum.
__device__ inline float group_max(float v, int width)
{
    if (width >= 2)
        v = fmaxf(v, dpp<kDppQuadXor1>(v));
    if (width >= 4)
        v = fmaxf(v, dpp<kDppQuadXor2>(v));
    if (width >= 8)
        v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    if (width >= 16)
        v = fmaxf(v, dpp<kDppRowMirror>(v));
    if (width >= 32) {
        const float other = dpp<kDppRowBcast15, 0xA>(v);
        v = (threadIdx.x & 16) ? fmaxf(v, other) : v;
    }
    if (width >= 64) {
        const float other = dpp<kDppRowBcast31, 0xC>(v);
        v = (threadIdx.x & 32) ? fmaxf(v, other) : v;
    }
    return v;
}

// v of lane `lane` (uniform), in every lane.
__device__ inline float lane_value(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// residue_sum for a width known at compile time.
template <int W, int N>
__device__ inline void residue_sum(float (&v)[N])
{
    if constexpr (W <= 1)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 1>(v[n]);
    if constexpr (W <= 2)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 2>(v[n]);
    if constexpr (W <= 4)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 4>(v[n]);
    if constexpr (W <= 8)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 8>(v[n]);
    if constexpr (W <= 16)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += __shfl_xor(v[n], 16);
    if constexpr (W <= 32)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += __shfl_xor(v[n], 32);
}

// For each of N values: the sum over the lanes that share lane % width (width a power of two
// <= 64, the same in every lane).  Lanes 0 .. width-1 end with their residue class's total.
// In-row steps rotate by width, 2 width, ... 8 (DPP); the steps across rows are batched
// permutes, N independent ones per step.
template <int N>
__device__ inline void residue_sum(float (&v)[N], int width)
{
    if (width <= 1)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 1>(v[n]);
    if (width <= 2)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 2>(v[n]);
    if (width <= 4)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 4>(v[n]);
    if (width <= 8)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += dpp<kDppRowRor + 8>(v[n]);
    if (width <= 16)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += __shfl_xor(v[n], 16);
    if (width <= 32)
#pragma unroll
        for (int n = 0; n < N; ++n)
            v[n] += __shfl_xor(v[n], 32);
}

} // namespace tiles
