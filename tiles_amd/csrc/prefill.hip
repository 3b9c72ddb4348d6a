// Matrix prefill of a bf16 decoder stack.  The reference prefills a prompt one position per
// worker step and leaves a matrix prefill as an open question (docs/development.md:331); this
// one runs up to kChunkRows positions through each layer at once.  Its arithmetic is the
// reference's full causal block (decoder_reference.py:273-312, recompute_prefix) with every
// rounding point of the decode path (docs/architecture.md:284-312), so that the cache rows it
// writes are the ones a position-by-position prefill writes, up to the FP32 summation order of
// the dot products:
//
//   u = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * attn_norm)      rms_rows
//   q, k, v = bf16(W u)                                          gemm_bf16 (MFMA, FP32 sums)
//   q, k rotated as the worker rotates them; K, V rows -> cache  rope_rows
//   s = bf16(bf16(q . k) * (1 / sqrt(dh)));                       attention_tiles (causal: M the
//   P = bf16(exp(s - M) / S); attention = bf16(sum P v)          row's maximum, S its FP32 exp-sum)
//   r = bf16(bf16(Wo attention) + x)                             GEMM, add_rows
//   z = RMSNorm(r) with ffn_norm                                 rms_rows
//   p = bf16(bf16(silu(bf16(Wgate z))) * bf16(Wup z))            GEMMs, silu_rows
//   y = bf16(bf16(Wdown p) + r)                                  GEMM, add_rows
//
// The GEMMs are this file's MFMA kernel rather than a library's: rocBLAS, linked into this
// library, conflicted with the different rocBLAS build PyTorch ships, and a process that loaded
// this library before importing torch crashed.
#include "prefill.hpp"

#include <algorithm>
#include <type_traits>
#include <string>

#include "device_common.hpp"
#include "worker_config.hpp"

namespace tiles {
namespace {

using Bf = Num<true>;
constexpr int kRowThreads = 256;
constexpr int kTile = 64;  // key positions per attention tile

__device__ inline float bf(uint16_t bits) { return bf16_bits_to_float(bits); }
__device__ inline uint16_t bits16(float v) { return static_cast<uint16_t>(float_to_bf16_bits(v)); }

// Sum over the block's threads (kRowThreads), in a fixed order.
__device__ float block_sum(float v, float* partial)
{
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset);
    if ((threadIdx.x & 63) == 0)
        partial[threadIdx.x / 64] = v;
    __syncthreads();
    float total = 0.0f;
    for (int w = 0; w < kRowThreads / 64; ++w)
        total += partial[w];
    __syncthreads();
    return total;
}

// x[r] = the embedding row of tokens[r].
__global__ void __launch_bounds__(kRowThreads) gather_rows(const uint16_t* embedding, const ti_token_id* tokens, int d,
                                                           uint16_t* x)
{
    const uint16_t* src = embedding + static_cast<size_t>(tokens[blockIdx.x]) * d;
    uint16_t* dst = x + static_cast<size_t>(blockIdx.x) * d;
    for (int i = threadIdx.x; i < d; i += kRowThreads)
        dst[i] = src[i];
}

// out[r] = bf16(bf16(x[r] * inv_rms) * scale), inv_rms = 1 / sqrt(mean(x[r]^2) + eps) in FP32,
// as the worker's rms_apply computes it.
__global__ void __launch_bounds__(kRowThreads) rms_rows(const uint16_t* x, const uint16_t* scale, int d, float eps,
                                                        uint16_t* out)
{
    __shared__ float partial[kRowThreads / 64];
    const uint16_t* row = x + static_cast<size_t>(blockIdx.x) * d;
    float squares = 0.0f;
    for (int i = threadIdx.x; i < d; i += kRowThreads) {
        const float v = bf(row[i]);
        squares = fmaf(v, v, squares);
    }
    const float total = block_sum(squares, partial);
    const float inv = 1.0f / sqrtf(total / static_cast<float>(d) + eps);
    uint16_t* dst = out + static_cast<size_t>(blockIdx.x) * d;
    for (int i = threadIdx.x; i < d; i += kRowThreads)
        dst[i] = bits16(Bf::round(Bf::round(bf(row[i]) * inv) * bf(scale[i])));
}

// Row r of qkv ([q heads | k heads | v heads], bf16) at position `position + r`: the query and
// key heads rotated (split halves; cos and sin of position * frequency rounded to bf16, each
// product rounded, then the difference or sum), the query heads to q_rot, the key and value
// heads to the cache row of the position.
__global__ void __launch_bounds__(kRowThreads) rope_rows(const uint16_t* qkv, int position, const float* frequencies, int nq,
                                                         int nkv, int dh, uint16_t* q_rot, uint16_t* key_cache,
                                                         uint16_t* value_cache)
{
    const int r = blockIdx.x;
    const int pos = position + r;
    const int half = dh / 2;
    const uint16_t* src = qkv + static_cast<size_t>(r) * (nq + 2 * nkv) * dh;
    for (int index = threadIdx.x; index < (nq + nkv) * half; index += kRowThreads) {
        const int head = index / half, pair = index - head * half;
        const float angle = static_cast<float>(pos) * frequencies[pair];
        const float c = Bf::round(cosf(angle)), s = Bf::round(sinf(angle));
        const float a = bf(src[head * dh + pair]), b = bf(src[head * dh + pair + half]);
        const uint16_t lo = bits16(Bf::round(Bf::round(a * c) - Bf::round(b * s)));
        const uint16_t hi = bits16(Bf::round(Bf::round(b * c) + Bf::round(a * s)));
        uint16_t* dst = head < nq ? q_rot + (static_cast<size_t>(r) * nq + head) * dh
                                  : key_cache + (static_cast<size_t>(pos) * nkv + head - nq) * dh;
        dst[pair] = lo;
        dst[pair + half] = hi;
    }
    for (int index = threadIdx.x; index < nkv * dh; index += kRowThreads)
        value_cache[static_cast<size_t>(pos) * nkv * dh + index] = src[(nq + nkv) * dh + index];
}

// Causal attention on the matrix cores, for 64 rows (positions position + r0 ..) and every
// query head of K/V head blockIdx.y: wave w takes rows r0 + 16 w .. + 15.  Scores are
// computed transposed, S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A: 16 key rows, B: the 16
// query rows of one head), so that lane l holds query l % 16 against keys 4 (l / 16) + i of each
// 16-key subtile.  Each score is bf16(bf16(dot) * scale) (the decode worker's score_of), keys past
// the query's position are masked (tiles past the block's first row only; rows past the chunk
// compute finite values nobody stores).  Pass 1 keeps each lane's running maximum and exp-sum per
// head, rescaled when the maximum grows, and merges the four lanes of a query at the end (exact
// maximum M, FP32 S).  Pass 2 recomputes the scores, rounds P = exp(s - M) / S to bf16 in
// registers and takes P V on the matrix cores with P as the A operand straight from the score
// layout: a 32-key step's k-elements 8 g .. 8 g + 7 of lane group g are keys 4 g .. 4 g + 3 and
// 16 + 4 g .. + 3 of the step (the sum over keys does not depend on their order), and two
// transposing LDS reads of the V rows supply the same keys.  The block stages each 64-key tile's
// K rows (and, in pass 2, V rows) in LDS once for its four waves, as stored, while the next
// tile's rows load into registers.
// The output is rounded once.  Keys past the block's last position are clamped to it when loaded
// and masked.
constexpr int kAttnThreads = 256;
constexpr int kAttnRows = 64;  // query positions per block: 16 per wave

// Two waves per SIMD for head_dim 64 (256 registers a lane at most; unbounded, the compiler
// took 276 and ran one); 128 needs more than 256 in either case.
template <int DH>
__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(DH == 64 ? 2 : 1)))
attention_tiles(const uint16_t* q_rot, int position, int rows, int nq, int nkv,
                                                                const uint16_t* key_cache, const uint16_t* value_cache,
                                                                float scale, uint16_t* out)
{
    constexpr int KS = DH / 32;                              // 32-dim steps of a score
    constexpr int NT = DH / 16;                              // 16-dim output tiles
    constexpr int kVStride = DH + 8;                         // bf16 per staged V row
    constexpr int kKStride = DH + 8;                         // bf16 per staged K row
    constexpr int kVectors = DH / 8;                         // 16-byte vectors of a K or V row
    constexpr int kLoads = kTile * kVectors / kAttnThreads;  // vectors per thread per tile
    static_assert(kTile * kVectors % kAttnThreads == 0, "whole vectors per thread");
    __shared__ __attribute__((aligned(16))) uint16_t vs[kTile * kVStride];
    __shared__ __attribute__((aligned(16))) uint16_t ks[kTile * kKStride];
    // Causal blocks differ in work by their row block (block x reads x + 1 key tiles at position
    // 0).  Every block is resident at once, two per CU, and the dispatcher gives blocks L and L + H
    // (H = half the grid) the same CU; launched in row-block order those two were alike, and the
    // CUs holding two of the last row blocks set the kernel's time.  So block L takes the L-th
    // heaviest (row block, head) and block L + H the L-th lightest: the two add up to one
    // average pair.  Any assignment covers every (row block, head) once.
    const int row_blocks = gridDim.x, items = gridDim.x * gridDim.y, half = (items + 1) / 2;
    const int linear = blockIdx.x + gridDim.x * blockIdx.y;
    const int heaviest = linear < half ? linear : items - 1 - (linear - half);  // index in descending weight
    const int h = heaviest % nkv, group = nq / nkv;
    const int lane = threadIdx.x & 63, wave = threadIdx.x / 64;
    const int col = lane & 15, g4 = lane >> 4;
    const int r0 = (row_blocks - 1 - heaviest / nkv) * kAttnRows;
    const int last_row = min(r0 + kAttnRows, rows) - 1;
    const int last_key = position + last_row;  // the block's last key: every load stays at or below it
    const int tiles = last_key / kTile + 1;
    const int full_tiles = (position + r0 + 1) / kTile;  // tiles every row of the block sees whole
    const int qrow = r0 + 16 * wave + col;     // this lane's query row (B operand, output column)
    const int qpos = position + qrow;

    // B operands of the scores: query row qrow of each head, dims 32 k + 8 g4 .. + 7.
    u32x4 qb[kMaxGroup][KS];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const bool live = g < group && qrow < rows;
            const size_t at = (static_cast<size_t>(live ? qrow : 0) * nq + h * group + (live ? g : 0)) * DH + 32 * k + 8 * g4;
            qb[g][k] = live ? *reinterpret_cast<const u32x4*>(q_rot + at) : u32x4{0u, 0u, 0u, 0u};
        }
    // This thread's vectors of tile kt's rows (K or V cache), keys clamped to the last key.
    auto load_rows = [&](const uint16_t* cache, int kt, u32x4 (&r)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int index = threadIdx.x + i * kAttnThreads, t = index / kVectors, v = index - t * kVectors;
            const int key = min(kt * kTile + t, last_key);
            r[i] = *reinterpret_cast<const u32x4*>(cache + (static_cast<size_t>(key) * nkv + h) * DH + 8 * v);
        }
    };
    auto stage_k = [&](const u32x4 (&r)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int index = threadIdx.x + i * kAttnThreads, t = index / kVectors, v = index - t * kVectors;
            *reinterpret_cast<u32x4*>(ks + t * kKStride + 8 * v) = r[i];
        }
    };
    auto stage_v = [&](const u32x4 (&r)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int index = threadIdx.x + i * kAttnThreads, t = index / kVectors, v = index - t * kVectors;
            *reinterpret_cast<u32x4*>(vs + t * kVStride + 8 * v) = r[i];
        }
    };
    // B operand of P V for dims 16 n .. + 15 over keys 4 g4 .. + 3 and 16 + 4 g4 .. + 3 of the
    // 32-key step: two transposing reads (ds_read_b64_tr_b16) of the V rows as stored.  Within a
    // 16-lane group lane j names key row 4 e + .. (e = j / 4) and dims 16 n + 4 (j % 4) .. + 3;
    // lane `col` receives dim 16 n + col of the four rows.
    auto v_operand = [&](int step, int n) {
        u32x4 out;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            typedef short v4s __attribute__((ext_vector_type(4)));
            const int row = 32 * step + 16 * h + 4 * g4 + (col >> 2);
            const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4s*)(vs + row * kVStride + 16 * n + 4 * (col & 3)));
            const uint2 pair = __builtin_bit_cast(uint2, v);
            out[2 * h] = pair.x;
            out[2 * h + 1] = pair.y;
        }
        return out;
    };
    // Scores of subtile j of the staged tile kt for every head: s[g][i] at key 64 kt + 16 j + 4 g4 + i.
    auto scores = [&](auto masked, int kt, int j, float (&s)[kMaxGroup][4]) {
        u32x4 ka[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k)
            ka[k] = *reinterpret_cast<const u32x4*>(ks + (16 * j + col) * kKStride + 32 * k + 8 * g4);
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < KS; ++k)
                acc = mfma_16x16x32_bf16(ka[k], qb[g][k], acc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // With head_dim 64 the scale is 2^-3: the product of a bf16 value and it is a bf16
                // value already (short of the subnormal range), so the second rounding is the identity.
                const float score = DH == 64 ? Bf::round(acc[i]) * 0.125f : Bf::round(Bf::round(acc[i]) * scale);
                if constexpr (decltype(masked)::value)
                    s[g][i] = kt * kTile + 16 * j + 4 * g4 + i <= qpos ? score : -INFINITY;
                else
                    s[g][i] = score;
            }
        }
    };

    // Pass 1: this lane's running maximum and exp-sum per head, over its keys.
    float m[kMaxGroup], total[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        m[g] = -INFINITY;
        total[g] = 0.0f;
    }
    u32x4 kr[kLoads], vr[kLoads];
    auto pass1_tile = [&](auto masked, int kt) {
        __syncthreads();  // the previous tile's K reads are done
        stage_k(kr);
        load_rows(key_cache, kt + 1, kr);  // the next tile (clamped past the last) in flight
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float s[kMaxGroup][4];
            scores(masked, kt, j, s);
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g) {
                const float grown = fmaxf(m[g], fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3])));
                if constexpr (decltype(masked)::value)
                    if (grown == -INFINITY)
                        continue;  // every key so far masked
                // total exp(m - grown) + e_0 + ... + e_3, the first two terms as one FMA; the factor
                // (0 for the first subtile's m = -inf) is exactly 1 where the maximum held, and is
                // skipped when it held in every lane of the wave.
                const float first = exp_nonpositive(s[g][0] - grown);
                float sum;
                if (__builtin_amdgcn_ballot_w64(grown != m[g]) != 0)
                    sum = fmaf(total[g], exp_nonpositive(m[g] - grown), first);
                else
                    sum = total[g] + first;
#pragma unroll
                for (int i = 1; i < 4; ++i)
                    sum += exp_nonpositive(s[g][i] - grown);
                total[g] = sum;
                m[g] = grown;
            }
        }
    };
    load_rows(key_cache, 0, kr);
    int kt = 0;
    for (; kt < full_tiles; ++kt)
        pass1_tile(std::false_type{}, kt);
    for (; kt < tiles; ++kt)
        pass1_tile(std::true_type{}, kt);
    // The four lanes of a query (lane groups g4 = 0..3) merge: M exact, S rescaled to it.
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int offset = 16; offset < 64; offset <<= 1) {
            const float om = __shfl_xor(m[g], offset), ot = __shfl_xor(total[g], offset);
            const float grown = fmaxf(m[g], om);
            if (grown != -INFINITY) {
                total[g] = total[g] * exp_nonpositive(m[g] - grown) + ot * exp_nonpositive(om - grown);
                m[g] = grown;
            }
        }
    float inverse[kMaxGroup];  // 1 / S, correctly rounded
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
        inverse[g] = 1.0f / total[g];

    // Pass 2: P = bf16(exp(s - M) / S) as A operands, P V against the staged V rows.
    f32x4 o[kMaxGroup][NT];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int n = 0; n < NT; ++n)
            o[g][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto pass2_tile = [&](auto masked, int kt) {
        __syncthreads();  // the previous tile's K and V reads are done
        stage_k(kr);
        stage_v(vr);
        load_rows(key_cache, kt + 1, kr);
        load_rows(value_cache, kt + 1, vr);
        __syncthreads();
#pragma unroll
        for (int step = 0; step < 2; ++step) {  // keys 32 step .. + 31 of the tile
            float s0[kMaxGroup][4], s1[kMaxGroup][4];
            scores(masked, kt, 2 * step, s0);
            scores(masked, kt, 2 * step + 1, s1);
            u32x4 vb[NT];
#pragma unroll
            for (int n = 0; n < NT; ++n)
                vb[n] = v_operand(step, n);
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g) {
                if (g >= group)
                    continue;
                float p[8];  // exp(s - M), masked keys exp(-inf) = 0; then P
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p[i] = exp_nonpositive(s0[g][i] - m[g]);
                    p[4 + i] = exp_nonpositive(s1[g][i] - m[g]);
                }
                const float least = fminf(fminf(fminf(p[0], p[1]), fminf(p[2], p[3])), fminf(fminf(p[4], p[5]), fminf(p[6], p[7])));
                if (__builtin_expect(least >= kQuotientFloor, 1)) {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        p[i] = divide_by(p[i], total[g], inverse[g]);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        p[i] = p[i] / total[g];
                }
                // Rounded to bf16 in pairs (v_cvt_pk_bf16_f32).
                auto pair = [](float lo, float hi) { return __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(lo), static_cast<__bf16>(hi)}); };
                const u32x4 pa = {pair(p[0], p[1]), pair(p[2], p[3]), pair(p[4], p[5]), pair(p[6], p[7])};
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    o[g][n] = mfma_16x16x32_bf16(pa, vb[n], o[g][n]);
            }
        }
    };
    load_rows(key_cache, 0, kr);
    load_rows(value_cache, 0, vr);
    for (kt = 0; kt < full_tiles; ++kt)
        pass2_tile(std::false_type{}, kt);
    for (; kt < tiles; ++kt)
        pass2_tile(std::true_type{}, kt);
    // o[g][n]: lane l holds query rows r0 + 16 wave + 4 g4 + i, dim 16 n + col.
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 16 * wave + 4 * g4 + i;
            if (g < group && r < rows)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    out[(static_cast<size_t>(r) * nq + h * group + g) * DH + 16 * n + col] = bits16(Bf::round(o[g][n][i]));
        }
}

// out = bf16(a + b) elementwise (a and b bf16).
__global__ void __launch_bounds__(kRowThreads) add_rows(const uint16_t* a, const uint16_t* b, size_t count, uint16_t* out)
{
    for (size_t i = blockIdx.x * static_cast<size_t>(kRowThreads) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kRowThreads)
        out[i] = bits16(Bf::round(bf(a[i]) + bf(b[i])));
}

// out = bf16(bf16(silu(gate)) * up), silu(g) = g / (1 + exp(-g)) in FP32 (gate and up bf16).
__global__ void __launch_bounds__(kRowThreads) silu_rows(const uint16_t* gate, const uint16_t* up, size_t count, uint16_t* out)
{
    for (size_t i = blockIdx.x * static_cast<size_t>(kRowThreads) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kRowThreads) {
        const float g = bf(gate[i]);
        out[i] = bits16(Bf::round(Bf::round(g / (1.0f + expf(-g))) * bf(up[i])));
    }
}

// C = A B^T (kBRows: B is [N][K], a weight matrix whose rows are output features) or C = A B
// (!kBRows: B is [K][N], Wdown as stored), all bf16 and row-major, A [M][K]; C rounded to bf16
// from FP32 sums (ldc: C's row stride).  Tiles of 128 x 128 per block of 4 waves, each wave
// 64 x 64 as 4 x 4 v_mfma_f32_16x16x32_bf16 tiles, K in steps of 32 through LDS (rows padded to
// 40 elements: 16-byte operand reads of 16 rows 80 bytes apart fall on distinct bank groups; a
// [K][N] B tile stays as loaded and its operands come from gfx950's transposing LDS reads), the
// next step's tile loaded into registers while this one's MFMAs run.  K % 32 == 0 and N % 16 == 0
// (the launcher checks); rows and columns past M and N are clamped on load and not stored.
constexpr int kGemmTile = 128, kGemmK = 32, kGemmStride = kGemmK + 8;

template <bool kBRows>
__global__ void __launch_bounds__(256) gemm_bf16(const uint16_t* a, const uint16_t* b, uint16_t* c, int m, int n, int k, int ldc)
{
    __shared__ __attribute__((aligned(16))) uint16_t as[kGemmTile * kGemmStride];
    // kBRows: B as [n][k] rows; !kBRows: B as loaded, [k][n] rows kBkStride apart, its operands
    // read by transposing LDS reads.
    __shared__ __attribute__((aligned(16))) uint16_t bs[kGemmTile * kGemmStride];
    constexpr int kBkStride = kGemmTile + 16;  // 288-byte rows: four rows of a transposing read on distinct banks
    static_assert(kGemmK * kBkStride <= kGemmTile * kGemmStride, "B tile exceeds its LDS area");
    const int t = threadIdx.x, lane = t & 63, wave = t / 64;
    const int m0 = blockIdx.y * kGemmTile, n0 = blockIdx.x * kGemmTile;
    const int wm = (wave / 2) * 64, wn = (wave % 2) * 64;
    // Loads of one K step: A rows t / 2 (16 elements each half), B likewise (kBRows) or B rows
    // k = t / 8 of 16 columns each (!kBRows).
    const int arow = min(m0 + t / 2, m - 1), acol = (t % 2) * 16;
    const int brow = kBRows ? min(n0 + t / 2, n - 1) : t / 8;
    const int bcol = kBRows ? (t % 2) * 16 : min(n0 + (t % 8) * 16, n - 16);
    u32x4 ra[2], rb[2];
    auto load = [&](int k0) {
        const u32x4* pa = reinterpret_cast<const u32x4*>(a + static_cast<size_t>(arow) * k + k0 + acol);
        ra[0] = pa[0];
        ra[1] = pa[1];
        const u32x4* pb = kBRows ? reinterpret_cast<const u32x4*>(b + static_cast<size_t>(brow) * k + k0 + bcol)
                                 : reinterpret_cast<const u32x4*>(b + static_cast<size_t>(k0 + brow) * n + bcol);
        rb[0] = pb[0];
        rb[1] = pb[1];
    };
    auto store = [&]() {
        u32x4* da = reinterpret_cast<u32x4*>(as + (t / 2) * kGemmStride + acol);
        da[0] = ra[0];
        da[1] = ra[1];
        if constexpr (kBRows) {
            u32x4* db = reinterpret_cast<u32x4*>(bs + (t / 2) * kGemmStride + bcol);
            db[0] = rb[0];
            db[1] = rb[1];
        } else {
            u32x4* db = reinterpret_cast<u32x4*>(bs + brow * kBkStride + (t % 8) * 16);
            db[0] = rb[0];
            db[1] = rb[1];
        }
    };
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int r = lane % 16, q = (lane / 16) * 8;
    load(0);
    for (int k0 = 0; k0 < k; k0 += kGemmK) {
        __syncthreads();  // the previous step's operand reads are done
        store();
        __syncthreads();
        if (k0 + kGemmK < k)
            load(k0 + kGemmK);
        u32x4 fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            fa[i] = *reinterpret_cast<const u32x4*>(as + (wm + i * 16 + r) * kGemmStride + q);
            if constexpr (kBRows) {
                fb[i] = *reinterpret_cast<const u32x4*>(bs + (wn + i * 16 + r) * kGemmStride + q);
            } else {
                // ds_read_b64_tr_b16: within a 16-lane group, lane j names row q + 4 h + j / 4,
                // columns wn + 16 i + 4 (j % 4) .. + 3, and lane r receives column wn + 16 i + r
                // of the group's four rows.
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    typedef short v4s __attribute__((ext_vector_type(4)));
                    const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s*)(bs + (q + 4 * h + (r >> 2)) * kBkStride + wn + i * 16 + 4 * (r & 3)));
                    const uint2 pair = __builtin_bit_cast(uint2, v);
                    fb[i][2 * h] = pair.x;
                    fb[i][2 * h + 1] = pair.y;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = mfma_16x16x32_bf16(fa[i], fb[j], acc[i][j]);
    }
    // Lane l holds rows 4 (l / 16) .. + 3 of column l % 16 of each 16 x 16 tile.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn + j * 16 + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm + i * 16 + (lane / 16) * 4 + e;
                if (row < m && col < n)
                    c[static_cast<size_t>(row) * ldc + col] = bits16(Bf::round(acc[i][j][e]));
            }
        }
}

} // namespace

bool MatrixPrefill::supports(const ti_worker_program_view& p)
{
    const ti_model_shape& s = p.shape;
    const int dh = s.head_dim;
    if (p.weight_dtype != TI_DTYPE_BFLOAT16 || !p.stack.full_stack || (dh != 64 && dh != 128) || s.kv_heads <= 0 ||
        s.query_heads % s.kv_heads != 0 || s.query_heads / s.kv_heads > kMaxGroup)
        return false;
    // Every GEMM of MatrixPrefill::layer, as (K, N): Q/K/V (d, heads x dh), Wo (query width, d),
    // gate/up (d, f), down (f, d).  gemm() takes K a multiple of kGemmK and N a multiple of 16; the
    // head widths are multiples of 64 already.  A stack outside these prefills through the worker.
    auto gemm_shape = [](int k, int n) { return k >= kGemmK && k % kGemmK == 0 && n >= 16 && n % 16 == 0; };
    const int d = s.hidden_size, f = s.intermediate_size, qw = s.query_heads * dh, kvw = s.kv_heads * dh;
    return gemm_shape(d, qw) && gemm_shape(d, kvw) && gemm_shape(qw, d) && gemm_shape(d, f) && gemm_shape(f, d);
}

MatrixPrefill::MatrixPrefill(const ti_worker_program_view& program) : p_(program) {}

MatrixPrefill::~MatrixPrefill()
{
    if (buffer_)
        (void)hipFree(buffer_);
}

namespace {
struct Views {
    uint16_t *x, *u, *qkv, *q, *attention, *projected, *r, *gate, *up;
};
size_t row_elements(const ti_model_shape& s)
{
    const size_t d = s.hidden_size, f = s.intermediate_size;
    const size_t qkv = static_cast<size_t>(s.query_heads + 2 * s.kv_heads) * s.head_dim;
    const size_t q = static_cast<size_t>(s.query_heads) * s.head_dim;
    return 5 * d + qkv + q + 2 * f;  // x, u, attention, projected, r | qkv | q | gate, up
}
Views views(void* buffer, const ti_model_shape& s, size_t rows)
{
    const size_t d = s.hidden_size, f = s.intermediate_size;
    uint16_t* at = static_cast<uint16_t*>(buffer);
    auto take = [&](size_t per_row) {
        uint16_t* v = at;
        at += rows * per_row;
        return v;
    };
    Views v{};
    v.x = take(d);
    v.u = take(d);
    v.attention = take(d);
    v.projected = take(d);
    v.r = take(d);
    v.qkv = take(static_cast<size_t>(s.query_heads + 2 * s.kv_heads) * s.head_dim);
    v.q = take(static_cast<size_t>(s.query_heads) * s.head_dim);
    v.gate = take(f);
    v.up = take(f);
    return v;
}

// C (rows x n, row stride ldc) = X (rows x k) W^T, W (n x k) row-major; or = X W with W (k x n).
int gemm(hipStream_t stream, bool w_rows, const uint16_t* x, int rows, int k, const uint16_t* w, int n, uint16_t* c, int ldc)
{
    if (rows < 1 || k % kGemmK != 0 || n % 16 != 0 || n < 16 || ldc < n)
        return fail(TI_ERR_INVALID_ARGUMENT, "prefill GEMM shape (K a multiple of 32, N of 16)");
    const dim3 grid((n + kGemmTile - 1) / kGemmTile, (rows + kGemmTile - 1) / kGemmTile);
    if (w_rows)
        hipLaunchKernelGGL(gemm_bf16<true>, grid, dim3(256), 0, stream, x, w, c, rows, n, k, ldc);
    else
        hipLaunchKernelGGL(gemm_bf16<false>, grid, dim3(256), 0, stream, x, w, c, rows, n, k, ldc);
    return TI_OK;
}
} // namespace

int MatrixPrefill::layer(hipStream_t stream, void* kv, int layer, int position, int rows)
{
    const ti_model_shape& s = p_.shape;
    const int d = s.hidden_size, f = s.intermediate_size, dh = s.head_dim, nq = s.query_heads, nkv = s.kv_heads;
    const int qw = nq * dh, kvw = nkv * dh, qkvw = qw + 2 * kvw;
    const Views v = views(buffer_, s, kChunkRows);
    const uint16_t* base = static_cast<const uint16_t*>(p_.weights) + p_.stack.layer_weights_offset +
                           static_cast<size_t>(layer) * p_.stack.layer_weight_stride;
    const ti_layer_layout& w = p_.layout;
    uint16_t* cache = static_cast<uint16_t*>(kv) + static_cast<size_t>(layer) * p_.stack.layer_kv_stride;
    const float eps = p_.numeric.rms_norm_eps;
    const size_t hidden_count = static_cast<size_t>(rows) * d, ffn_count = static_cast<size_t>(rows) * f;
    const dim3 elementwise(static_cast<unsigned>(std::min<size_t>(4096, (ffn_count + kRowThreads - 1) / kRowThreads)));
    int code = TI_OK;
    auto gemm_ok = [&](int status) {
        code = status;
        return status == TI_OK;
    };

    hipLaunchKernelGGL(rms_rows, dim3(rows), dim3(kRowThreads), 0, stream, v.x, base + w.attn_norm, d, eps, v.u);
    // Wq, Wk and Wv are consecutive in the package's layer layout (plan.cpp checks the regions):
    // one GEMM over their rows, which also fills the chip (Wk and Wv alone are 4 column tiles).
    if (w.Wk == w.Wq + static_cast<uint32_t>(qw) * d && w.Wv == w.Wk + static_cast<uint32_t>(kvw) * d) {
        if (!gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wq, qkvw, v.qkv, qkvw)))
            return code;
    } else if (!gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wq, qw, v.qkv, qkvw)) ||
               !gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wk, kvw, v.qkv + qw, qkvw)) ||
               !gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wv, kvw, v.qkv + qw + kvw, qkvw))) {
        return code;
    }
    hipLaunchKernelGGL(rope_rows, dim3(rows), dim3(kRowThreads), 0, stream, v.qkv, position, p_.rotary_frequencies, nq, nkv, dh,
                       v.q, cache + w.key, cache + w.value);
    const float scale = 1.0f / sqrtf(static_cast<float>(dh));
    const dim3 attention_grid((rows + kAttnRows - 1) / kAttnRows, nkv);
    if (dh == 64)
        hipLaunchKernelGGL(attention_tiles<64>, attention_grid, dim3(kAttnThreads), 0, stream, v.q, position, rows, nq, nkv,
                           cache + w.key, cache + w.value, scale, v.attention);
    else
        hipLaunchKernelGGL(attention_tiles<128>, attention_grid, dim3(kAttnThreads), 0, stream, v.q, position, rows, nq, nkv,
                           cache + w.key, cache + w.value, scale, v.attention);
    if (!gemm_ok(gemm(stream, true, v.attention, rows, qw, base + w.Wo, d, v.projected, d)))
        return code;
    hipLaunchKernelGGL(add_rows, elementwise, dim3(kRowThreads), 0, stream, v.projected, v.x, hidden_count, v.r);
    hipLaunchKernelGGL(rms_rows, dim3(rows), dim3(kRowThreads), 0, stream, v.r, base + w.ffn_norm, d, eps, v.u);
    if (!gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wgate, f, v.gate, f)) ||
        !gemm_ok(gemm(stream, true, v.u, rows, d, base + w.Wup, f, v.up, f)))
        return code;
    hipLaunchKernelGGL(silu_rows, elementwise, dim3(kRowThreads), 0, stream, v.gate, v.up, ffn_count, v.gate);
    // Wdown row-major [hidden][intermediate] on the device (ti_relayout_weights).
    if (!gemm_ok(gemm(stream, true, v.gate, rows, f, base + w.Wdown, d, v.projected, d)))
        return code;
    hipLaunchKernelGGL(add_rows, elementwise, dim3(kRowThreads), 0, stream, v.projected, v.r, hidden_count, v.x);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return hip_fail(e, "prefill kernel launch");
    return TI_OK;
}

int MatrixPrefill::enqueue(hipStream_t stream, void* kv, const ti_token_id* tokens, int position, int count)
{
    if (!supports(p_))
        return fail(TI_ERR_INVALID_ARGUMENT, "matrix prefill needs a bf16 decoder stack with head_dim 64 or 128");
    if (count <= 0)
        return TI_OK;
    if (position < 0 || position + count > p_.shape.max_context)
        return fail(TI_ERR_INVALID_ARGUMENT, "sequence context capacity reached");
    if (!buffer_) {
        buffer_bytes_ = row_elements(p_.shape) * kChunkRows * sizeof(uint16_t);
        const hipError_t e = hipMalloc(&buffer_, buffer_bytes_);
        if (e != hipSuccess) {
            buffer_ = nullptr;
            return hip_fail(e, "prefill buffers");
        }
    }
    const Views v = views(buffer_, p_.shape, kChunkRows);
    const uint16_t* embedding = static_cast<const uint16_t*>(p_.weights) + p_.stack.embedding_offset;
    for (int first = 0; first < count; first += kChunkRows) {
        const int rows = std::min(kChunkRows, count - first);
        hipLaunchKernelGGL(gather_rows, dim3(rows), dim3(kRowThreads), 0, stream, embedding, tokens + first, p_.shape.hidden_size,
                           v.x);
        for (int layer = 0; layer < p_.stack.layers; ++layer) {
            const int code = this->layer(stream, kv, layer, position + first, rows);
            if (code != TI_OK)
                return code;
        }
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return hip_fail(e, "prefill kernel launch");
    return TI_OK;
}

} // namespace tiles
