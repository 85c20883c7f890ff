// mvh_gemv.hip -- decode GEMVs over weights in native GGUF block layout.
//
// Q4_0 x Q8 (tensor_matvec Q4_0 branch, src/gguf_kernels.cpp:246 + dot_q4_q8
// :189): per row the reference runs sum = fma(d_w*d_a, float(isum_b), sum)
// over blocks b in order.  The kernels split that into two phases:
//   1. every lane turns whole 18-byte blocks into (p_b = d_w*d_a, f_b =
//      float(isum_b)) pairs -- integer dots with v_dot4_i32_i8, exact;
//   2. one lane per row folds the pairs in block order with v_fma_f32.
// Phase 2 is the reference's own chain, so y is bit-identical.
//
// Weight units are groups of 8 blocks (144 bytes = 9 x 16 B, so every unit
// starts 16-byte aligned when K % 256 == 0); other K take a 1-block path.
#include "mvh_kernels.hpp"

#include <algorithm>
#include <cstdlib>

namespace mvh {
namespace {

constexpr int kActPitch = 272;     // LDS bytes per 8-block activation group (256 + 16 pad)
constexpr int kXPitchF = 260;      // LDS floats per 8-block fp32 activation group (256 + 4 pad)
constexpr int kGemvThreads = 128;

__device__ __forceinline__ int dot_nibbles(const uint32_t (&qs)[4], const uint4 a0, const uint4 a1) {
    // qs byte i holds element i (low nibble) and element 16+i (high nibble).
    constexpr uint32_t M = 0x0f0f0f0fu;
    int s = 0;
    s = __builtin_amdgcn_sdot4(static_cast<int>(qs[0] & M), static_cast<int>(a0.x), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(qs[1] & M), static_cast<int>(a0.y), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(qs[2] & M), static_cast<int>(a0.z), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(qs[3] & M), static_cast<int>(a0.w), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((qs[0] >> 4) & M), static_cast<int>(a1.x), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((qs[1] >> 4) & M), static_cast<int>(a1.y), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((qs[2] >> 4) & M), static_cast<int>(a1.z), s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>((qs[3] >> 4) & M), static_cast<int>(a1.w), s, false);
    return s;
}

// Fold the per-block pairs of `rows` rows in block order (phase 2).
__device__ __forceinline__ void fold_pairs(const float2* s_pair, int pitch, int rows, int nb, float* y) {
    for (int r = threadIdx.x; r < rows; r += blockDim.x) {
        const float2* pr = s_pair + r * pitch;
        float sum = 0.0f;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float2 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = pr[b + j];
#pragma unroll
            for (int j = 0; j < 8; ++j) sum = fmaf(v[j].x, v[j].y, sum);
        }
        for (; b < nb; ++b) sum = fmaf(pr[b].x, pr[b].y, sum);
        y[r] = sum;
    }
}

// Weight load modes of the 8-block path:
//   kLoadStream  each lane reads its own 144-byte unit (9 x 16 B, lane stride 144 B), non-temporal;
//   kLoadCached  the same pattern through the caches;
//   kLoadStaged  the tile is read with coalesced 16-byte loads (consecutive lanes, consecutive
//                bytes) into LDS, and every lane then reads its unit from LDS.
enum { kLoadStream = 0, kLoadCached = 1, kLoadStaged = 2 };

// blockIdx.y = token: its Q8 row at aq + token * K, scales at ad + token * nb,
// outputs at y + token * N (one launch for a batch, each token's chains as for one)
template <int G, int MODE>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_0_kernel(const uint8_t* __restrict__ W,
                                                                  const int8_t* __restrict__ aq,
                                                                  const float* __restrict__ ad, float* __restrict__ y,
                                                                  int N, int nb, int rows_per_wg) {
    extern __shared__ __align__(16) uint8_t smem[];
    aq += static_cast<size_t>(blockIdx.y) * nb * 32;
    ad += static_cast<size_t>(blockIdx.y) * nb;
    y += static_cast<size_t>(blockIdx.y) * N;
    const int ngrp = (nb + 7) >> 3;
    uint8_t* s_aq = smem;
    float* s_ad = reinterpret_cast<float*>(smem + ngrp * kActPitch);
    int* s_as = reinterpret_cast<int*>(s_ad + nb);
    float2* s_pair = reinterpret_cast<float2*>(s_as + nb);
    const int pitch = nb + 1;

    // stage the Q8 activation (all rows of this tile share it)
    const int K = nb * 32;
    for (int c = threadIdx.x; c < K / 16; c += blockDim.x)
        *reinterpret_cast<uint4*>(s_aq + (c >> 4) * kActPitch + (c & 15) * 16) = reinterpret_cast<const uint4*>(aq)[c];
    for (int b = threadIdx.x; b < nb; b += blockDim.x) s_ad[b] = ad[b];
    __syncthreads();
    // s_b = sum of the 32 activation bytes of block b, for the "-8" nibble bias
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const uint4* a = reinterpret_cast<const uint4*>(s_aq + (b >> 3) * kActPitch + (b & 7) * 32);
        const uint4 a0 = a[0], a1 = a[1];
        constexpr int ones = 0x01010101;
        int t = 0;
        t = __builtin_amdgcn_sdot4(static_cast<int>(a0.x), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a0.y), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a0.z), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a0.w), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a1.x), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a1.y), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a1.z), ones, t, false);
        t = __builtin_amdgcn_sdot4(static_cast<int>(a1.w), ones, t, false);
        s_as[b] = t;
    }
    __syncthreads();

    const int r0 = blockIdx.x * rows_per_wg;
    const int rows = min(rows_per_wg, N - r0);
    const int upr = nb / G;
    const int nunits = rows * upr;
    const uint8_t* tile = W + static_cast<size_t>(r0) * nb * 18;
    // raw weight tile (staged mode), 16-byte aligned after the pair buffer
    uint8_t* s_raw = smem + ((reinterpret_cast<uint8_t*>(s_pair + rows_per_wg * pitch) - smem + 15) & ~15);
    if constexpr (MODE == kLoadStaged && G == 8) {
        const int nchunks = rows * nb * 18 / 16;  // nb % 8 == 0: whole 16-byte chunks
        for (int c = threadIdx.x; c < nchunks; c += blockDim.x)
            reinterpret_cast<uint4*>(s_raw)[c] = ld_stream16(reinterpret_cast<const uint4*>(tile) + c);
        __syncthreads();
    }

    for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
        const int row = u / upr;
        const int b0 = (u - row * upr) * G;
        float2* pout = s_pair + row * pitch + b0;
        if constexpr (G == 8) {
            uint32_t w[36];
            const uint4* src = MODE == kLoadStaged ? reinterpret_cast<const uint4*>(s_raw + u * 144)
                                                   : reinterpret_cast<const uint4*>(tile + static_cast<size_t>(u) * 144);
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const uint4 v = MODE == kLoadStream ? ld_stream16(src + k) : src[k];
                w[4 * k] = v.x;
                w[4 * k + 1] = v.y;
                w[4 * k + 2] = v.z;
                w[4 * k + 3] = v.w;
            }
            const uint8_t* agrp = s_aq + (b0 >> 3) * kActPitch;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int o = 18 * j;  // byte offset of block j inside the unit
                uint32_t dbits, qs[4];
                if ((j & 1) == 0) {
                    dbits = w[o / 4] & 0xffffu;
#pragma unroll
                    for (int k = 0; k < 4; ++k) qs[k] = align16(w[o / 4 + k + 1], w[o / 4 + k]);
                } else {
                    dbits = w[o / 4] >> 16;
#pragma unroll
                    for (int k = 0; k < 4; ++k) qs[k] = w[(o + 2) / 4 + k];
                }
                const uint4* a = reinterpret_cast<const uint4*>(agrp + j * 32);
                const int b = b0 + j;
                const int isum = dot_nibbles(qs, a[0], a[1]) - 8 * s_as[b];
                pout[j] = make_float2(h2f(dbits) * s_ad[b], static_cast<float>(isum));
            }
        } else {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(tile + static_cast<size_t>(u) * 18);
            uint32_t h[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) h[k] = src[k];
            const uint32_t qs[4] = {h[1] | (h[2] << 16), h[3] | (h[4] << 16), h[5] | (h[6] << 16), h[7] | (h[8] << 16)};
            const uint4* a = reinterpret_cast<const uint4*>(s_aq + (b0 >> 3) * kActPitch + (b0 & 7) * 32);
            const int isum = dot_nibbles(qs, a[0], a[1]) - 8 * s_as[b0];
            pout[0] = make_float2(h2f(h[0]) * s_ad[b0], static_cast<float>(isum));
        }
    }
    __syncthreads();
    fold_pairs(s_pair, pitch, rows, nb, y + r0);
}

// fp32-activation block dots (dot_q4_0_fp32 :93-109, dot_q8_0_fp32 :111-120,
// src/gguf_kernels.cpp): per block, lane j of 8 accumulates elements j, 8+j,
// 16+j, 24+j by fma from zero, s = 0+t0+..+t7; then sum = fma(d, s, sum) over
// blocks.  Phase 1 produces (d_b, s_b) per block, phase 2 folds them per row.
// blockIdx.y = token (tensor_matmul_batch's y[b*rows + r]).
template <uint32_t TYPE>
struct Blk;
template <>
struct Blk<kQ4_0> {
    static constexpr int kBytes = 18, kQdw = 4, kScale = 2;
    static __device__ __forceinline__ float scale(uint32_t bits) { return h2f(bits); }
    // element e: low nibble of byte e (e < 16) or high nibble of byte e-16, minus 8
    static __device__ __forceinline__ int value(const uint32_t (&qs)[kQdw], int e) {
        const int byte = e & 15;
        const uint32_t b = (qs[byte >> 2] >> (8 * (byte & 3))) & 0xffu;
        return static_cast<int>(e < 16 ? (b & 15u) : (b >> 4)) - 8;
    }
};
template <>
struct Blk<kQ8_0> {
    static constexpr int kBytes = 34, kQdw = 8, kScale = 2;
    static __device__ __forceinline__ float scale(uint32_t bits) { return h2f(bits); }
    static __device__ __forceinline__ int value(const uint32_t (&qs)[kQdw], int e) {
        return static_cast<int>(static_cast<int8_t>(qs[e >> 2] >> (8 * (e & 3))));
    }
};
// native BlockQ4_0 (src/quant.cpp:79-81): f32 d, element e = nibble e & 1 of
// byte e >> 1, minus 8 (dot_q4_0 unpacks them back to element order, :121-128)
template <>
struct Blk<kNQ4_0> {
    static constexpr int kBytes = 20, kQdw = 4, kScale = 4;
    static __device__ __forceinline__ float scale(uint32_t bits) { return __uint_as_float(bits); }
    static __device__ __forceinline__ int value(const uint32_t (&qs)[kQdw], int e) {
        return static_cast<int>((qs[e >> 3] >> (8 * ((e >> 1) & 3) + 4 * (e & 1))) & 15u) - 8;
    }
};
// native BlockQ8_0: f32 d, int8 qs[32]
template <>
struct Blk<kNQ8_0> {
    static constexpr int kBytes = 36, kQdw = 8, kScale = 4;
    static __device__ __forceinline__ float scale(uint32_t bits) { return __uint_as_float(bits); }
    static __device__ __forceinline__ int value(const uint32_t (&qs)[kQdw], int e) {
        return static_cast<int>(static_cast<int8_t>(qs[e >> 2] >> (8 * (e & 3))));
    }
};

template <uint32_t TYPE>
__device__ __forceinline__ float f32act_block_sum(const uint32_t (&qs)[Blk<TYPE>::kQdw], const float* xb) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const float4 x0 = *reinterpret_cast<const float4*>(xb + k);
        const float4 x1 = *reinterpret_cast<const float4*>(xb + k + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = fmaf(static_cast<float>(Blk<TYPE>::value(qs, k + j)), xv[j], t[j]);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s = s + t[j];
    return s;
}

// Block j of an 8-block unit held in registers w[]: scale bits and quant dwords.
template <uint32_t TYPE>
__device__ __forceinline__ void unit_block(const uint32_t* w, int j, uint32_t& dbits,
                                           uint32_t (&qs)[Blk<TYPE>::kQdw]) {
    const int o = Blk<TYPE>::kBytes * j;
    if constexpr (Blk<TYPE>::kScale == 4) {  // native blocks: scale and quants dword aligned
        dbits = w[o / 4];
#pragma unroll
        for (int k = 0; k < Blk<TYPE>::kQdw; ++k) qs[k] = w[o / 4 + 1 + k];
    } else if ((o & 3) == 0) {
        dbits = w[o / 4] & 0xffffu;
#pragma unroll
        for (int k = 0; k < Blk<TYPE>::kQdw; ++k) qs[k] = align16(w[o / 4 + k + 1], w[o / 4 + k]);
    } else {
        dbits = w[o / 4] >> 16;
#pragma unroll
        for (int k = 0; k < Blk<TYPE>::kQdw; ++k) qs[k] = w[(o + 2) / 4 + k];
    }
}

template <uint32_t TYPE, int G>
__global__ __launch_bounds__(kGemvThreads) void gemv_f32act_kernel(const uint8_t* __restrict__ W,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int N, int nb,
                                                                    int rows_per_wg) {
    constexpr int BB = Blk<TYPE>::kBytes;
    constexpr int UNIT16 = 8 * BB / 16;  // 16-byte loads per 8-block unit
    extern __shared__ __align__(16) uint8_t smem[];
    const int ngrp = (nb + 7) >> 3;
    float* s_x = reinterpret_cast<float*>(smem);
    float2* s_pair = reinterpret_cast<float2*>(smem + static_cast<size_t>(ngrp) * kXPitchF * 4);
    const int pitch = nb + 1;
    const int K = nb * 32;
    const float* xt = x + static_cast<size_t>(blockIdx.y) * K;
    for (int c = threadIdx.x; c < K / 4; c += blockDim.x)
        *reinterpret_cast<float4*>(s_x + (c >> 6) * kXPitchF + (c & 63) * 4) = reinterpret_cast<const float4*>(xt)[c];
    __syncthreads();

    const int r0 = blockIdx.x * rows_per_wg;
    const int rows = min(rows_per_wg, N - r0);
    const int upr = nb / G;
    const int nunits = rows * upr;
    const uint8_t* tile = W + static_cast<size_t>(r0) * nb * BB;
    for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
        const int row = u / upr;
        const int b0 = (u - row * upr) * G;
        float2* pout = s_pair + row * pitch + b0;
        if constexpr (G == 8) {
            uint32_t w[4 * UNIT16];
            const uint4* src = reinterpret_cast<const uint4*>(tile + static_cast<size_t>(u) * 8 * BB);
#pragma unroll
            for (int k = 0; k < UNIT16; ++k) {
                const uint4 v = ld_stream16(src + k);
                w[4 * k] = v.x;
                w[4 * k + 1] = v.y;
                w[4 * k + 2] = v.z;
                w[4 * k + 3] = v.w;
            }
            const float* xg = s_x + (b0 >> 3) * kXPitchF;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t dbits, qs[Blk<TYPE>::kQdw];
                unit_block<TYPE>(w, j, dbits, qs);
                pout[j] = make_float2(Blk<TYPE>::scale(dbits), f32act_block_sum<TYPE>(qs, xg + j * 32));
            }
        } else {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(tile + static_cast<size_t>(u) * BB);
            constexpr int S = Blk<TYPE>::kScale / 2;  // 16-bit words of the scale
            uint32_t qs[Blk<TYPE>::kQdw];
#pragma unroll
            for (int k = 0; k < Blk<TYPE>::kQdw; ++k)
                qs[k] = src[S + 2 * k] | (static_cast<uint32_t>(src[S + 1 + 2 * k]) << 16);
            const uint32_t dbits = S == 1 ? src[0] : src[0] | (static_cast<uint32_t>(src[1]) << 16);
            pout[0] = make_float2(Blk<TYPE>::scale(dbits),
                                  f32act_block_sum<TYPE>(qs, s_x + (b0 >> 3) * kXPitchF + (b0 & 7) * 32));
        }
    }
    __syncthreads();
    fold_pairs(s_pair, pitch, rows, nb, y + static_cast<size_t>(blockIdx.y) * N + r0);
}

// The same two phases for TT tokens per workgroup (nb % 8 == 0): each 8-block
// unit is loaded once and turned into pairs for every token of the group (the
// per-token kernel reloads the weights for every token); the folds then run
// one thread per (row, token).  Token t of the group is t0 + t, t < B - t0.
template <uint32_t TYPE, int TT>
__global__ __launch_bounds__(kGemvThreads) void gemv_f32act_tokens_kernel(const uint8_t* __restrict__ W,
                                                                           const float* __restrict__ x,
                                                                           float* __restrict__ y, int N, int nb,
                                                                           int rows_per_wg, int B) {
    constexpr int BB = Blk<TYPE>::kBytes;
    constexpr int UNIT16 = 8 * BB / 16;
    extern __shared__ __align__(16) uint8_t smem[];
    const int ngrp = nb >> 3;
    const int xstride = ngrp * kXPitchF;  // floats per token
    float* s_x = reinterpret_cast<float*>(smem);
    float2* s_pair = reinterpret_cast<float2*>(smem + static_cast<size_t>(TT) * xstride * 4);
    const int pitch = nb + 1;
    const int K = nb * 32;
    const int t0 = blockIdx.y * TT, nt = min(TT, B - t0);
    for (int tk = 0; tk < nt; ++tk) {
        const float* xt = x + static_cast<size_t>(t0 + tk) * K;
        for (int c = threadIdx.x; c < K / 4; c += blockDim.x)
            *reinterpret_cast<float4*>(s_x + tk * xstride + (c >> 6) * kXPitchF + (c & 63) * 4) =
                reinterpret_cast<const float4*>(xt)[c];
    }
    __syncthreads();

    const int r0 = blockIdx.x * rows_per_wg;
    const int rows = min(rows_per_wg, N - r0);
    const int upr = nb / 8;
    const int nunits = rows * upr;
    const uint8_t* tile = W + static_cast<size_t>(r0) * nb * BB;
    for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
        const int row = u / upr;
        const int b0 = (u - row * upr) * 8;
        uint32_t w[4 * UNIT16];
        const uint4* src = reinterpret_cast<const uint4*>(tile + static_cast<size_t>(u) * 8 * BB);
#pragma unroll
        for (int k = 0; k < UNIT16; ++k) {
            const uint4 v = ld_stream16(src + k);
            w[4 * k] = v.x;
            w[4 * k + 1] = v.y;
            w[4 * k + 2] = v.z;
            w[4 * k + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t dbits, qs[Blk<TYPE>::kQdw];
            unit_block<TYPE>(w, j, dbits, qs);
            const float d = Blk<TYPE>::scale(dbits);
            for (int tk = 0; tk < nt; ++tk)
                s_pair[(tk * rows_per_wg + row) * pitch + b0 + j] =
                    make_float2(d, f32act_block_sum<TYPE>(qs, s_x + tk * xstride + (b0 >> 3) * kXPitchF + j * 32));
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < rows * nt; i += blockDim.x) {
        const int tk = i / rows, r = i - tk * rows;
        const float2* pr = s_pair + (tk * rows_per_wg + r) * pitch;
        float sum = 0.0f;
        for (int b = 0; b < nb; ++b) sum = fmaf(pr[b].x, pr[b].y, sum);
        y[static_cast<size_t>(t0 + tk) * N + r0 + r] = sum;
    }
}

// Default batched prefill numerics (q4_row_batch4_fp32 / q8_row_batch4_fp32,
// src/gguf_kernels.cpp:191-209; batch8 = two batch4, :211-216): per
// (row, token) eight lane accumulators run over ALL blocks without reset,
// term = fma(float(q)*d, x, acc) with the product float(q)*d rounded first;
// result = t0+t1+..+t7.  One thread per (row, token); blockIdx.y = token.
template <uint32_t TYPE>
__global__ __launch_bounds__(256) void batch4_f32act_kernel(const uint8_t* __restrict__ W,
                                                             const float* __restrict__ x, float* __restrict__ y,
                                                             int N, int nb) {
    constexpr int BB = Blk<TYPE>::kBytes;
    extern __shared__ __align__(16) float s_xt[];
    const int K = nb * 32;
    const float* xt = x + static_cast<size_t>(blockIdx.y) * K;
    for (int c = threadIdx.x; c < K / 4; c += blockDim.x)
        reinterpret_cast<float4*>(s_xt)[c] = reinterpret_cast<const float4*>(xt)[c];
    __syncthreads();
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= N) return;
    const uint8_t* rowp = W + static_cast<size_t>(r) * nb * BB;
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(rowp + static_cast<size_t>(b) * BB);
        uint32_t qs[Blk<TYPE>::kQdw];
#pragma unroll
        for (int k = 0; k < Blk<TYPE>::kQdw; ++k)
            qs[k] = src[1 + 2 * k] | (static_cast<uint32_t>(src[2 + 2 * k]) << 16);
        const float d = h2f(src[0]);
        const float* xb = s_xt + b * 32;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float q = static_cast<float>(Blk<TYPE>::value(qs, e)) * d;
            t[e & 7] = fmaf(q, xb[e], t[e & 7]);
        }
    }
    float s = t[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) s = s + t[j];
    y[static_cast<size_t>(blockIdx.y) * N + r] = s;
}

// dot_q8_0_fp32 / dot_q4_0_fp32 per row (tensor_matvec's Q8_0 branch and the
// fp32-activation Q4_0 dot, src/gguf_kernels.cpp:93-120) for one token, K %
// 256 == 0, K / 256 <= 64, in the structure of the persistent Q4_0 x Q8 GEMV:
// lane (r, u) of a wave owns unit u (8 blocks) of row r of the wave's tile of
// TR = 64 / (K/256) rows, turns its 8 blocks into (d_b, s_b) pairs (s_b the
// block's exact 8-lane sum, f32act_block_sum) against the activation staged
// in LDS, and the row's chain sum = fma(d_b, s_b, sum) then walks the lanes
// in unit order (DPP shift by one lane per stage).  Persistent waves stride
// over the tiles; every weight load is unconditional (clamped rows).
template <uint32_t TYPE, int UB>
__device__ __forceinline__ void gemv_f32act_persistent(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                       float* __restrict__ y, int N, int nb, int ntiles) {
    // a unit is UB blocks (8, or 4 to halve the weights each lane holds),
    // loaded with 8-byte loads (a 4-block unit is only 8-byte aligned)
    constexpr int kU2 = UB * Blk<TYPE>::kBytes / 8;
    extern __shared__ __align__(16) uint8_t smem[];
    float* s_x = reinterpret_cast<float*>(smem);
    const int upr = nb / UB;
    const size_t row_bytes = static_cast<size_t>(nb) * Blk<TYPE>::kBytes;
    const int t = threadIdx.x, lane = t & 63;
    const int TR = 64 / upr;
    const int r = lane / upr, u = lane - r * upr;
    const bool worker = r < TR;
    const int uu = worker ? u : 0;
    const int gw = blockIdx.x * 4 + (t >> 6), GW = gridDim.x * 4;
    auto load = [&](uint32_t (&w)[2 * kU2], int tl) {
        const int grow = min(tl * TR + (worker ? r : 0), N - 1);
        const uint2* src = reinterpret_cast<const uint2*>(W + static_cast<size_t>(grow) * row_bytes +
                                                          static_cast<size_t>(uu) * UB * Blk<TYPE>::kBytes);
#pragma unroll
        for (int k = 0; k < kU2; ++k) {
            const uint2 v = src[k];
            w[2 * k] = v.x;
            w[2 * k + 1] = v.y;
        }
    };
    // the wave's first two tiles go out before the activation staging
    uint32_t wa[2 * kU2], wb[2 * kU2];
    int tile = gw;
    load(wa, min(tile, ntiles - 1));
    load(wb, min(tile + GW, ntiles - 1));
    for (int c = t; c < nb * 8; c += 256)
        *reinterpret_cast<float4*>(s_x + (c >> 6) * kXPitchF + (c & 63) * 4) = reinterpret_cast<const float4*>(x)[c];
    __syncthreads();
    const float* xg = s_x + (uu * UB >> 3) * kXPitchF + (uu * UB & 7) * 32;
    auto tile_step = [&](int tl, const uint32_t (&w)[2 * kU2]) {
        const int grow = tl * TR + r;
        float2 pr[UB];
#pragma unroll
        for (int j = 0; j < UB; ++j) {
            uint32_t dbits, qs[Blk<TYPE>::kQdw];
            unit_block<TYPE>(w, j, dbits, qs);
            pr[j] = make_float2(Blk<TYPE>::scale(dbits), f32act_block_sum<TYPE>(qs, xg + j * 32));
        }
        // lane u's value is final from stage u on; after upr stages the last
        // lane of each row holds the in-order chain
        float sum = 0.0f;
        for (int st = 0; st < upr; ++st) {
            const float in = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x138, 0xf, 0xf, false));
            float acc = u == 0 ? 0.0f : in;
#pragma unroll
            for (int j = 0; j < UB; ++j) acc = fmaf(pr[j].x, pr[j].y, acc);
            sum = acc;
        }
        if (worker && grow < N && u == upr - 1) y[grow] = sum;
    };
    while (tile < ntiles) {
        tile_step(tile, wa);
        if (tile + 2 * GW < ntiles) load(wa, tile + 2 * GW);
        tile += GW;
        if (tile >= ntiles) break;
        tile_step(tile, wb);
        if (tile + 2 * GW < ntiles) load(wb, tile + 2 * GW);
        tile += GW;
    }
}

__global__ __launch_bounds__(256) void gemv_f32act_persistent_q4_0(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int N, int nb, int ntiles) {
    gemv_f32act_persistent<kQ4_0, 4>(W, x, y, N, nb, ntiles);
}
__global__ __launch_bounds__(256) void gemv_f32act_persistent_q8_0(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int N, int nb, int ntiles) {
    gemv_f32act_persistent<kQ8_0, 4>(W, x, y, N, nb, ntiles);
}
// dot_q8_0_fp32 for one token (src/gguf_kernels.cpp:111-120), K = 16 * UB
// blocks: the row-group layout of the Q4_0 x Q8 decode GEMV.  A wave holds 4
// rows, one per 16-lane group; lane g of a group owns the row's blocks
// UB*g .. UB*g + UB - 1 (UB * 34 contiguous bytes, 8-byte loads issued before
// the activation staging), turns them into (d_b, s_b) pairs (s_b the block's
// exact eight-lane sum, f32act_block_sum), and the row's chain
// sum = fma(d_b, s_b, sum) walks the group's lanes in block order: at stage st
// every lane redoes its UB fmas from its left neighbour's value (DPP
// row_ror:1), lane g's value being final from stage g on.  The activation is
// staged once per workgroup (4 waves, 16 rows), block b at float
// 32b + 4*(b / UB): the 16 lanes of a group then read 16 different bank
// quads at every step.
__device__ __forceinline__ float dpp_row_ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));
}

template <int UB>
__global__ __launch_bounds__(256) void gemv_q8_0_f32act_rows16(const uint8_t* __restrict__ W,
                                                                const float* __restrict__ x, float* __restrict__ y,
                                                                int N) {
    constexpr int nb = 16 * UB, kW2 = UB * 34 / 8;  // blocks per row, 8-byte words per lane
    __shared__ __align__(16) float s_x[32 * nb + 4 * 16];
    const int t = threadIdx.x, lane = t & 63, g = lane & 15;
    const int row = blockIdx.x * 16 + (t >> 6) * 4 + (lane >> 4);
    // rows past N read row N - 1 and are not written
    const uint2* src = reinterpret_cast<const uint2*>(W + static_cast<size_t>(min(row, N - 1)) * (nb * 34) +
                                                      static_cast<size_t>(g) * (UB * 34));
    uint32_t w[2 * kW2];
#pragma unroll
    for (int k = 0; k < kW2; ++k) {
        const uint2 v = src[k];
        w[2 * k] = v.x;
        w[2 * k + 1] = v.y;
    }
    for (int c = t; c < nb * 8; c += 256) {
        const int b = c >> 3;
        *reinterpret_cast<float4*>(s_x + 32 * b + 4 * (b / UB) + 4 * (c & 7)) = reinterpret_cast<const float4*>(x)[c];
    }
    __syncthreads();
    float pd[UB], ps[UB];
#pragma unroll
    for (int j = 0; j < UB; ++j) {
        uint32_t dbits, qs[Blk<kQ8_0>::kQdw];
        unit_block<kQ8_0>(w, j, dbits, qs);
        const int b = UB * g + j;
        pd[j] = Blk<kQ8_0>::scale(dbits);
        ps[j] = f32act_block_sum<kQ8_0>(qs, s_x + 32 * b + 4 * g);
    }
    float sum = 0.0f;
#pragma unroll
    for (int st = 0; st < 16; ++st) {
        const float in = dpp_row_ror1(sum);
        float acc = g == 0 ? 0.0f : in;
#pragma unroll
        for (int j = 0; j < UB; ++j) acc = fmaf(pd[j], ps[j], acc);
        sum = acc;
    }
    if (g == 15 && row < N) y[row] = sum;
}

__global__ __launch_bounds__(256) void gemv_f32act_persistent_nq4_0(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int N, int nb, int ntiles) {
    gemv_f32act_persistent<kNQ4_0, 4>(W, x, y, N, nb, ntiles);
}
__global__ __launch_bounds__(256) void gemv_f32act_persistent_nq8_0(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int N, int nb, int ntiles) {
    gemv_f32act_persistent<kNQ8_0, 4>(W, x, y, N, nb, ntiles);
}

// The same numerics for K % 256 == 0 with the work spread over lanes: lane
// (row, j) owns accumulator j of its row for kBT tokens, i.e. elements j,
// j+8, j+16, j+24 of every block in that order (the reference's 8-wide
// vector lane j); eight lanes per row, eight rows per wave, 32 rows per
// workgroup.  Each dequantized float(q)*d feeds the kBT tokens' fmas.  The
// weights come in 8-block units (16-byte loads; the eight lanes of a row load
// the same bytes); the activations of the kBT tokens come through LDS one
// 8-block chunk at a time, stored as [token][block][j][m] so lane j reads its
// four elements x[32b + j + 8m] with one 16-byte read.  The final
// t0 + t1 + ... + t7 runs in order through LDS.
constexpr int kBT = 8;         // tokens per workgroup
constexpr int kBRows = 32;     // rows per workgroup
constexpr int kBChunk = 256;   // activation elements per LDS chunk (one 8-block unit)

template <uint32_t TYPE>
struct Unit;
template <>
struct Unit<kQ4_0> {
    static constexpr int kU4 = 9;  // 16-byte loads per 8 blocks (144 bytes)
    // block jb of the unit: f16 scale bits and the 16 quant bytes as 4 dwords
    static __device__ __forceinline__ void block(const uint32_t (&w)[4 * kU4], int jb, uint32_t& dbits,
                                                 uint32_t (&qs)[4]) {
        const int o = 18 * jb;
        if ((jb & 1) == 0) {
            dbits = w[o / 4] & 0xffffu;
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = align16(w[o / 4 + k + 1], w[o / 4 + k]);
        } else {
            dbits = w[o / 4] >> 16;
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = w[(o + 2) / 4 + k];
        }
    }
    // elements j, j+8, j+16, j+24: low nibbles of bytes j, 8+j, high nibbles of the same
    static __device__ __forceinline__ void lane_values(const uint32_t (&qs)[4], int j, int (&v)[4]) {
        const uint32_t sh = 8u * static_cast<uint32_t>(j & 3);
        const uint32_t b0 = ((j & 4) ? qs[1] : qs[0]) >> sh, b1 = ((j & 4) ? qs[3] : qs[2]) >> sh;
        v[0] = static_cast<int>(b0 & 15u) - 8;
        v[1] = static_cast<int>(b1 & 15u) - 8;
        v[2] = static_cast<int>((b0 >> 4) & 15u) - 8;
        v[3] = static_cast<int>((b1 >> 4) & 15u) - 8;
    }
};
template <>
struct Unit<kQ8_0> {
    static constexpr int kU4 = 17;  // 272 bytes
    static __device__ __forceinline__ void block(const uint32_t (&w)[4 * kU4], int jb, uint32_t& dbits,
                                                 uint32_t (&qs)[8]) {
        const int o = 34 * jb;
        if ((jb & 1) == 0) {
            dbits = w[o / 4] & 0xffffu;
#pragma unroll
            for (int k = 0; k < 8; ++k) qs[k] = align16(w[o / 4 + k + 1], w[o / 4 + k]);
        } else {
            dbits = w[o / 4] >> 16;
#pragma unroll
            for (int k = 0; k < 8; ++k) qs[k] = w[(o + 2) / 4 + k];
        }
    }
    // elements j + 8m: byte j + 8m of the 32 int8 values
    static __device__ __forceinline__ void lane_values(const uint32_t (&qs)[8], int j, int (&v)[4]) {
        const uint32_t sh = 8u * static_cast<uint32_t>(j & 3);
#pragma unroll
        for (int m = 0; m < 4; ++m)
            v[m] = static_cast<int>(static_cast<int8_t>(((j & 4) ? qs[2 * m + 1] : qs[2 * m]) >> sh));
    }
};

template <uint32_t TYPE>
__global__ __launch_bounds__(256) void batch_f32act_lanes_kernel(const uint8_t* __restrict__ W,
                                                                 const float* __restrict__ x, float* __restrict__ y,
                                                                 int N, int nb) {
    using U = Unit<TYPE>;
    constexpr int kQdw = Blk<TYPE>::kQdw;
    __shared__ __align__(16) float s_x[2][kBT * kBChunk];  // [token][block][j][m], double-buffered
    const int t = threadIdx.x, j = t & 7;
    const int rl = t >> 3;  // row within the workgroup
    const int r = blockIdx.x * kBRows + rl;
    const int tok0 = blockIdx.y * kBT;
    const int K = nb * 32, units = nb / 8;
    const size_t row_bytes = static_cast<size_t>(nb) * Blk<TYPE>::kBytes;
    const uint4* wrow = reinterpret_cast<const uint4*>(W + static_cast<size_t>(min(r, N - 1)) * row_bytes);

    // chunk c of the kBT activation rows: 2 float4 per thread (kBT * 256
    // floats) into registers, written to LDS after the current unit's fmas,
    // so the wait for them neither delays those fmas nor covers the weight
    // loads issued after them
    constexpr int kSt = kBT * kBChunk / 4 / 256;
    auto stage_load = [&](int c, float4 (&v)[kSt]) {
#pragma unroll
        for (int k = 0; k < kSt; ++k) {
            const int f = t + 256 * k;  // float4 index within the chunk: token f / 64, element 4 (f % 64)
            v[k] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(tok0 + (f >> 6)) * K + c * kBChunk +
                                                    4 * (f & 63));
        }
    };
    auto stage_store = [&](const float4 (&v)[kSt], int buf) {
#pragma unroll
        for (int k = 0; k < kSt; ++k) {
            const int f = t + 256 * k;
            const int tk = f >> 6, e = 4 * (f & 63);
            const float vv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // element e+i: block (e+i)/32, lane (e+i)%8, m = ((e+i)%32)/8
                const int ei = e + i;
                s_x[buf][((tk * 8 + (ei >> 5)) * 8 + (ei & 7)) * 4 + ((ei & 31) >> 3)] = vv[i];
            }
        }
    };

    float acc[kBT];
#pragma unroll
    for (int k = 0; k < kBT; ++k) acc[k] = 0.0f;
    uint32_t w[4 * U::kU4];
    auto load = [&](int u) {
#pragma unroll
        for (int k = 0; k < U::kU4; ++k) {
            const uint4 v = wrow[u * U::kU4 + k];
            w[4 * k] = v.x;
            w[4 * k + 1] = v.y;
            w[4 * k + 2] = v.z;
            w[4 * k + 3] = v.w;
        }
    };
    float4 xs[kSt];
    stage_load(0, xs);
    load(0);
    stage_store(xs, 0);
    __syncthreads();
    for (int u = 0; u < units; ++u) {
        const int buf = u & 1;
        // the next unit's loads and staging run unconditionally (the last
        // unit reloads itself and restages into the idle buffer), so no
        // branch lets the compiler move the staging stores ahead of the fmas
        const int nu = min(u + 1, units - 1);
        uint32_t cur[4 * U::kU4];
#pragma unroll
        for (int k = 0; k < 4 * U::kU4; ++k) cur[k] = w[k];
        stage_load(nu, xs);
        load(nu);
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
            uint32_t dbits, qs[kQdw];
            U::block(cur, jb, dbits, qs);
            const float d = h2f(dbits);
            int v[4];
            U::lane_values(qs, j, v);
            float q[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) q[m] = static_cast<float>(v[m]) * d;
#pragma unroll
            for (int k = 0; k < kBT; ++k) {
                const float4 xv = *reinterpret_cast<const float4*>(&s_x[buf][((k * 8 + jb) * 8 + j) * 4]);
                acc[k] = fmaf(q[0], xv.x, acc[k]);
                acc[k] = fmaf(q[1], xv.y, acc[k]);
                acc[k] = fmaf(q[2], xv.z, acc[k]);
                acc[k] = fmaf(q[3], xv.w, acc[k]);
            }
            // each block's LDS reads stay with its fmas, and the staging
            // stores stay after the last block: hoisted, the reads take a
            // register set per block and the stores wait for the activation
            // loads in the middle of the fmas
            __builtin_amdgcn_sched_barrier(0);
        }
        stage_store(xs, buf ^ 1);  // s_x[buf ^ 1] was last read by unit u - 1
        __syncthreads();  // s_x[buf ^ 1] is complete; s_x[buf] is free for unit u + 2
    }
    // t0 + t1 + ... + t7 per (row, token), in order, through LDS
    float* s_red = &s_x[0][0];  // [row][token][j]
#pragma unroll
    for (int k = 0; k < kBT; ++k) s_red[(rl * kBT + k) * 8 + j] = acc[k];
    __syncthreads();
    {
        const int tk = t / kBRows, row = t % kBRows;  // one output per thread, rows fastest
        const float* p = s_red + (row * kBT + tk) * 8;
        float sum = p[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) sum = sum + p[i];
        const int orow = blockIdx.x * kBRows + row;
        if (orow < N) y[static_cast<size_t>(tok0 + tk) * N + orow] = sum;
    }
}

// q4/q8_row_batch4_fp32 numerics (src/gguf_kernels.cpp:191-216) for Q4_0 and
// Q8_0 with K % 256 == 0, each activation read feeding two rows: lane (row
// pair, j) owns accumulator j of two rows for kR2T tokens, elements j, j+8,
// j+16, j+24 of every block in that order (the reference's 8-wide vector
// lane j).  A workgroup covers 32 rows x 2*kR2T tokens; per 8-block unit it
// stages the 32 rows' raw bytes (one copy, 16-byte loads) and the activations
// ([token][block][j][m], as batch_f32act_lanes_kernel) in LDS, double
// buffered.  Lane j reads its four weights of a block and the f16 scale:
// Q4_0 bytes j and j+8 of the nibbles, float(q - 8) * d with q - 8 formed
// exactly in float; Q8_0 bytes j, j+8, j+16, j+24, float(q) * d.  Each row's
// t0 + t1 + ... + t7 then runs in order through LDS.  Against
// batch_f32act_lanes_kernel: fewer VALU instructions per fma (the eight lanes
// of a row no longer each unpack the whole unit from registers) and half the
// activation reads from LDS per fma.
//
// BS = true: dot_q4_0_fp32 / dot_q8_0_fp32 numerics (src/gguf_kernels.cpp:
// 93-120; tensor_matmul_batch, and tensor_matmul_batch_v06 with
// MEMVANTA_FORCE_Q8_ACT for Q8_0 weights): per block, lane j's t_j over
// elements j, j+8, j+16, j+24 from zero, s = t0 + ... + t7 in order, then
// sum = fma(d, s, sum) over the blocks in order.  The same tile and staging;
// thread (block jb, row pair, token group) owns block jb of each unit for two
// rows x kR2T tokens, all eight lanes of it, so a block's in-order lane sum
// stays in the thread.  The block sums go to LDS, and after a barrier thread
// t carries the chains of (row, token) t and t + 256 over the unit's eight
// blocks.  The activation blocks are padded to 36 floats in LDS so the eight
// blocks of a token fall in different banks.
constexpr int kR2T = 8;       // tokens per thread (16 measured slower: 214 VGPRs, half the workgroups)
constexpr int kR2Rows = 32;   // rows per workgroup
constexpr int kR2Tok = 2 * kR2T;
constexpr int kBsPitch = kR2Tok + 4;                 // block sums: floats per row (16-byte aligned)
constexpr int kBsBlk = kR2Rows * kBsPitch + 4;       // block sums: floats per block of the unit

template <uint32_t TYPE, bool BS>
__global__ __launch_bounds__(256) void batch_f32act_rows2_kernel(const uint8_t* __restrict__ W,
                                                                 const float* __restrict__ x,
                                                                 float* __restrict__ y, int N, int nb) {
    constexpr int kB = Blk<TYPE>::kBytes;     // 18 or 34
    constexpr int kU = 8 * kB;                // bytes of an 8-block unit of one row (144 or 272)
    constexpr int kP = kU / 16;               // 16-byte pieces per row and unit (9 or 17)
    constexpr int kNP = (kR2Rows * kP + 255) / 256;  // pieces per thread (2 or 3)
    constexpr int kXP = BS ? 36 : 32;         // LDS floats per activation block
    __shared__ __align__(16) uint8_t s_w[2][kR2Rows * kU + 16];  // + a 16-byte slot for unused stores
    __shared__ __align__(16) float s_x[2][kR2Tok * 8 * kXP];     // [token][block][j][m]
    __shared__ __align__(16) float s_bs[BS ? 8 * kBsBlk : 1];    // [block][row][token]
    __shared__ float s_d[BS ? 8 * kR2Rows : 1];                  // [block][row]
    const int t = threadIdx.x, j = t & 7, slot = t >> 3;
    const int rp = slot & 15, tg = slot >> 4;  // rows 2rp, 2rp+1; tokens tg*kR2T ..
    const int row0 = blockIdx.x * kR2Rows;
    const int tok0 = blockIdx.y * kR2Tok;
    const int K = nb * 32, units = nb / 8;
    const size_t row_bytes = static_cast<size_t>(nb) * kB;

    // staging of unit c: pieces t + 256 i of the 32 rows' 16-byte pieces (row
    // p / kP, bytes 16 (p % kP); pieces past the last load it again and store
    // to the spare slot); kR2Tok * 64 float4 of activations, kXs per thread
    constexpr int kXs = kR2Tok * kBChunk / 4 / 256;
    const uint8_t* wsrc[kNP];
    int wdst[kNP];
#pragma unroll
    for (int i = 0; i < kNP; ++i) {
        const int p = t + 256 * i, pc = min(p, kR2Rows * kP - 1);
        wsrc[i] = W + static_cast<size_t>(min(row0 + pc / kP, N - 1)) * row_bytes + 16 * (pc % kP);
        wdst[i] = p < kR2Rows * kP ? (pc / kP) * kU + 16 * (pc % kP) : kR2Rows * kU;
    }
    auto stage_load = [&](int c, uint4 (&w)[kNP], float4 (&v)[kXs]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kNP; ++i) w[i] = *reinterpret_cast<const uint4*>(wsrc[i] + static_cast<size_t>(c) * kU);
#pragma unroll
        for (int k = 0; k < kXs; ++k) {
            const int f = t + 256 * k;  // token f / 64, element 4 (f % 64)
            v[k] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(tok0 + (f >> 6)) * K + c * kBChunk +
                                                    4 * (f & 63));
        }
    };
    auto stage_store = [&](const uint4 (&w)[kNP], const float4 (&v)[kXs], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kNP; ++i) *reinterpret_cast<uint4*>(&s_w[buf][wdst[i]]) = w[i];
#pragma unroll
        for (int k = 0; k < kXs; ++k) {
            const int f = t + 256 * k;
            const int tk = f >> 6, e = 4 * (f & 63);
            const float vv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // element e+i: block (e+i)/32, lane (e+i)%8, m = ((e+i)%32)/8
                const int ei = e + i;
                s_x[buf][(tk * 8 + (ei >> 5)) * kXP + (ei & 7) * 4 + ((ei & 31) >> 3)] = vv[i];
            }
        }
    };

    float acc[2][kR2T];  // BS: the block sums of the current unit
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int k = 0; k < kR2T; ++k) acc[r][k] = 0.0f;
    float chain[2] = {0.0f, 0.0f};  // BS: sums of (row, token) = (c / 16, c % 16), c = t and t + 256
    uint4 ws[kNP];
    float4 xs[kXs];
    stage_load(0, ws, xs);
    stage_store(ws, xs, 0);
    __syncthreads();
    for (int u = 0; u < units; ++u) {
        const int buf = u & 1;
        // the next unit's loads and staging run unconditionally (the last
        // unit reloads itself into the idle buffer)
        stage_load(min(u + 1, units - 1), ws, xs);
        if constexpr (!BS) {
#pragma unroll
            for (int jb = 0; jb < 8; ++jb) {
                float q[2][4];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const uint8_t* blk = &s_w[buf][(2 * rp + r) * kU + kB * jb];
                    const float d = h2f(*reinterpret_cast<const uint16_t*>(blk));
                    if constexpr (TYPE == kQ4_0) {
                        // bytes j and j + 8 of the nibbles: elements j, j + 8 (low
                        // nibbles), j + 16, j + 24 (high).  q ^ 8 read as a signed
                        // 4-bit field is q - 8, so one signed extract (v_bfe_i32,
                        // written as shifts: __builtin_amdgcn_sbfe's result is
                        // converted as unsigned by this compiler) gives it;
                        // float(q - 8) * d is then the reference's product
                        const uint32_t px =
                            (static_cast<uint32_t>(blk[2 + j]) | (static_cast<uint32_t>(blk[10 + j]) << 8)) ^ 0x8888u;
                        q[r][0] = static_cast<float>(static_cast<int>(px << 28) >> 28) * d;
                        q[r][1] = static_cast<float>(static_cast<int>(px << 20) >> 28) * d;
                        q[r][2] = static_cast<float>(static_cast<int>(px << 24) >> 28) * d;
                        q[r][3] = static_cast<float>(static_cast<int>(px << 16) >> 28) * d;
                    } else {
#pragma unroll
                        for (int m = 0; m < 4; ++m)
                            q[r][m] = static_cast<float>(static_cast<int8_t>(blk[2 + j + 8 * m])) * d;
                    }
                }
#pragma unroll
                for (int k = 0; k < kR2T; ++k) {
                    const float4 xv = *reinterpret_cast<const float4*>(
                        &s_x[buf][((tg * kR2T + k) * 8 + jb) * kXP + j * 4]);
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        acc[r][k] = fmaf(q[r][0], xv.x, acc[r][k]);
                        acc[r][k] = fmaf(q[r][1], xv.y, acc[r][k]);
                        acc[r][k] = fmaf(q[r][2], xv.z, acc[r][k]);
                        acc[r][k] = fmaf(q[r][3], xv.w, acc[r][k]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            stage_store(ws, xs, buf ^ 1);  // buffer buf ^ 1 was last read by unit u - 1
            __syncthreads();
        } else {
            // block j of the unit: lane sums t_l, l = 0..7, each from zero,
            // added into s in lane order
            const uint8_t* blk0 = &s_w[buf][(2 * rp) * kU + kB * j];
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int k = 0; k < kR2T; ++k) acc[r][k] = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                float q[2][4];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const uint8_t* blk = blk0 + r * kU;
                    if constexpr (TYPE == kQ4_0) {
                        const uint32_t pair =
                            static_cast<uint32_t>(blk[2 + l]) | (static_cast<uint32_t>(blk[10 + l]) << 8);
                        const uint32_t lo = pair & 0x0f0fu, hi = (pair >> 4) & 0x0f0fu;
                        q[r][0] = static_cast<float>(lo & 0xffu) - 8.0f;
                        q[r][1] = static_cast<float>(lo >> 8) - 8.0f;
                        q[r][2] = static_cast<float>(hi & 0xffu) - 8.0f;
                        q[r][3] = static_cast<float>(hi >> 8) - 8.0f;
                    } else {
#pragma unroll
                        for (int m = 0; m < 4; ++m) q[r][m] = static_cast<float>(static_cast<int8_t>(blk[2 + l + 8 * m]));
                    }
                }
#pragma unroll
                for (int k = 0; k < kR2T; ++k) {
                    const float4 xv = *reinterpret_cast<const float4*>(
                        &s_x[buf][((tg * kR2T + k) * 8 + j) * kXP + l * 4]);
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        float tl = fmaf(q[r][0], xv.x, 0.0f);
                        tl = fmaf(q[r][1], xv.y, tl);
                        tl = fmaf(q[r][2], xv.z, tl);
                        tl = fmaf(q[r][3], xv.w, tl);
                        acc[r][k] = acc[r][k] + tl;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float* dst = &s_bs[j * kBsBlk + (2 * rp + r) * kBsPitch + tg * kR2T];
#pragma unroll
                for (int k = 0; k < kR2T; k += 4)
                    *reinterpret_cast<float4*>(dst + k) = make_float4(acc[r][k], acc[r][k + 1], acc[r][k + 2], acc[r][k + 3]);
                if (tg == 0) s_d[j * kR2Rows + 2 * rp + r] = h2f(*reinterpret_cast<const uint16_t*>(blk0 + r * kU));
            }
            stage_store(ws, xs, buf ^ 1);  // buffer buf ^ 1 was last read by unit u - 1
            __syncthreads();
            // sum = fma(d, s, sum) over the unit's blocks in order
#pragma unroll
            for (int o = 0; o < 2; ++o) {
                const int c = t + 256 * o, row = c >> 4, tk = c & 15;
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    chain[o] = fmaf(s_d[b * kR2Rows + row], s_bs[b * kBsBlk + row * kBsPitch + tk], chain[o]);
            }
            __syncthreads();  // the reads of s_bs / s_d end before the next unit's writes
        }
    }
    if constexpr (BS) {
#pragma unroll
        for (int o = 0; o < 2; ++o) {
            const int c = t + 256 * o, row = c >> 4, tk = c & 15;
            const int orow = row0 + row;
            if (orow < N) y[static_cast<size_t>(tok0 + tk) * N + orow] = chain[o];
        }
        return;
    }
    // t0 + t1 + ... + t7 per (row, token), in order, through LDS
    float* s_red = &s_x[0][0];  // [row][token][j]: 32 * kR2Tok * 8 floats
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int k = 0; k < kR2T; ++k) s_red[((2 * rp + r) * kR2Tok + tg * kR2T + k) * 8 + j] = acc[r][k];
    __syncthreads();
#pragma unroll
    for (int o = 0; o < kR2Rows * kR2Tok / 256; ++o) {
        const int idx = t + 256 * o, tk = idx / kR2Rows, row = idx % kR2Rows;  // rows fastest
        const float* p = s_red + (row * kR2Tok + tk) * 8;
        float sum = p[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) sum = sum + p[i];
        const int orow = row0 + row;
        if (orow < N) y[static_cast<size_t>(tok0 + tk) * N + orow] = sum;
    }
}

// Q6_K with fp32 activations (dot_q6_k_fp32, src/gguf_kernels.cpp:138-146):
// w = (d*sc[i/16])*q in f32, exact products summed in double.  LPR lanes per
// row (64: one row per wave; 32: two; the launch picks by K), each lane
// working on R rows at once (the launch picks by row count); each lane sums
// 64-element units (a half super-block's sixteen-column group) into its own
// double partial per row, the row's lanes add the partials as a tree and
// round to f32 once.  The double sum order differs from the reference's element order, so
// a row can differ from it only when the exact sum lies within ~1e-13
// (relative) of an f32 rounding boundary.
constexpr int kQ6Threads = 256;

template <int LPR, int R, int T = kQ6Threads>
__global__ __launch_bounds__(T) void gemv_q6_k_kernel(const uint8_t* __restrict__ W,
                                                               const float* __restrict__ x, float* __restrict__ y,
                                                               int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* s_x = reinterpret_cast<float*>(smem);
    constexpr int kRpw = 64 / LPR;  // rows per wave
    const int nsb = K / 256;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l = lane % LPR;
    // a lane sums the same units of R consecutive rows (each activation value
    // converted once for all R)
    const int row = (blockIdx.x * (T / 64) * kRpw + wave * kRpw + lane / LPR) * R;
    // rows past N sum row N - 1 (the lane groups reduce together) and are not written
    const uint8_t* rb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rb[r] = W + static_cast<size_t>(min(row + r, N - 1)) * nsb * 210;
    const int units = 4 * nsb;
    // unit u of the row: ql bytes g*64 + h*16 (elements j = 0, 2) and
    // g*64 + 32 + h*16 (j = 1, 3), qh bytes 128 + g*32 + h*16, scales
    // 192 + g*8 + h + 2j, d at 208; the bytes are 2-aligned (16-bit loads)
    struct Raw {
        uint32_t qa[4], qb[4], qh[4];
        int sc[4];
        uint32_t d;
    };
    auto load_unit = [&](int u, const uint8_t* rbase, Raw& w) __attribute__((always_inline)) {
        const int sb = u >> 2, g = (u >> 1) & 1, h = u & 1;
        const uint8_t* b = rbase + static_cast<size_t>(sb) * 210;
        const uint16_t* pa = reinterpret_cast<const uint16_t*>(b + g * 64 + h * 16);
        const uint16_t* pb = reinterpret_cast<const uint16_t*>(b + g * 64 + 32 + h * 16);
        const uint16_t* ph = reinterpret_cast<const uint16_t*>(b + 128 + g * 32 + h * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w.qa[i] = pa[2 * i] | (static_cast<uint32_t>(pa[2 * i + 1]) << 16);
            w.qb[i] = pb[2 * i] | (static_cast<uint32_t>(pb[2 * i + 1]) << 16);
            w.qh[i] = ph[2 * i] | (static_cast<uint32_t>(ph[2 * i + 1]) << 16);
        }
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + g * 8 + h);
#pragma unroll
        for (int j = 0; j < 4; ++j) w.sc[j] = sc[2 * j];
        w.d = *reinterpret_cast<const uint16_t*>(b + 208);
    };
    // Every weight w = (d*sc)*q is exact in f32 (d*sc has at most 18
    // significant bits, |q| <= 32 at most 5), so w*x = (d*sc) * (q*x) with
    // q*x exact in double: each 16-element group (one scale) sums q*x in
    // double and adds (d*sc) times that sum -- the reference's exact terms,
    // added in another order (as the partials and the lane tree already do)
    double acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0;
    auto sum_unit = [&](int u, const Raw (&w)[R]) __attribute__((always_inline)) {
        const int sb = u >> 2, g = (u >> 1) & 1, h = u & 1;
        // float4 f of the activation sits at f ^ swz(f) (the staging below);
        // here f = base + 8j + c, so bits 0..1 (c) and 3 (j's bit 0) move
        const float4* xb = reinterpret_cast<const float4*>(s_x) + sb * 64 + g * 32 + h * 4;
        const int kv = (u >> 1) & 7, klo = kv & 3, kb = kv >> 2;
        double part[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) part[r][j] = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // columns 4c .. 4c+3 of the group
            // the 6-bit codes u = q + 32 of element group j as four bytes
            // (low nibbles (j = 0, 1) or high nibbles (j = 2, 3) of ql, bits
            // 2j..2j+1 of qh above them), bit 5 flipped: a byte's low six bits
            // are then q in two's complement
            // (bits 6..7 of a byte are left as they come: the six-bit field
            // extraction ignores them; bit 5 is flipped in qh once for all four)
            uint32_t u[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t qa = w[r].qa[c], qb = w[r].qb[c], hx = w[r].qh[c] ^ 0xaaaaaaaau;
                constexpr uint32_t kLo = 0x0f0f0f0fu;
                u[r][0] = (qa & kLo) | ((hx << 4) & ~kLo);  // v_bfi_b32
                u[r][1] = (qb & kLo) | ((hx << 2) & ~kLo);
                u[r][2] = ((qa >> 4) & kLo) | (hx & ~kLo);
                u[r][3] = ((qb >> 4) & kLo) | ((hx >> 2) & ~kLo);
            }
            const float4* pc = xb + (c ^ klo);
            const float4* pe = pc + 8 * kb;  // j = 0, 2
            const float4* po = pc - 8 * kb;  // j = 1, 3
            const float4 xv[4] = {pe[0], po[8], pe[16], po[24]};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float xe = e == 0 ? xv[j].x : e == 1 ? xv[j].y : e == 2 ? xv[j].z : xv[j].w;
                    const double xd = static_cast<double>(xe);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int q = static_cast<int>(u[r][j] << (26 - 8 * e)) >> 26;  // v_bfe_i32
                        part[r][j] = fma(static_cast<double>(q), xd, part[r][j]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = h2f(w[r].d);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[r] = fma(static_cast<double>(d * static_cast<float>(w[r].sc[j])), part[r][j], acc[r]);
        }
    };
    // the activation staged first, then each lane's units loaded and summed in
    // turn (loading every unit before the staging, which keeps three units'
    // bytes in registers, measured slower at every shape: 4096->32000 61 against
    // 39 us, 2048->32000 29 against 21 us, 5632->2048 10 against 8 us)
    const float* xt = x + static_cast<size_t>(blockIdx.y) * K;
    // stored swizzled: float4 f at f ^ swz(f), swz taking bits 5..7 of f to
    // bits 0, 1 and 3, so the 32 units the lanes of a row read at once spread
    // over all 64 banks instead of two sets of four
    for (int c = threadIdx.x; c < K / 4; c += T) {
        const int kv = (c >> 5) & 7;
        reinterpret_cast<float4*>(s_x)[c ^ ((kv & 3) | ((kv & 4) << 1))] = reinterpret_cast<const float4*>(xt)[c];
    }
    __syncthreads();
    for (int u = l; u < units; u += LPR) {
        Raw w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) load_unit(u, rb[r], w[r]);
        sum_unit(u, w);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        double tot;
        if constexpr (LPR == 64) {
            tot = wave_sum(acc[r]);
        } else {  // within each 32-lane half
            double a = acc[r];
            a += swz_xor<16>(a);
            a += swz_xor<8>(a);
            a += swz_xor<4>(a);
            a += swz_xor<2>(a);
            a += swz_xor<1>(a);
            tot = a;
        }
        if (l == 0 && row + r < N) y[static_cast<size_t>(blockIdx.y) * N + row + r] = static_cast<float>(tot);
    }
}

// Q6_K for whole groups of 16 tokens on the f64 matrix pipe
// (v_mfma_f64_16x16x4f64): the same exact products ((d*sc)*q)*x in double
// as dot_q6_k_fp32 (src/gguf_kernels.cpp:138-146), accumulated by the
// MFMA in double.  A workgroup covers 16 rows x 16 tokens; its kQ6FWaves
// waves take consecutive shares of the super-blocks and their partials are
// added in wave order through LDS.  In a wave, lane (i = lane % 16, g =
// lane / 16) gives the A operand (row i) and the B operand (token i) of
// the 64-element unit g of each super-block (half g / 2, sixteen-column
// group g % 2, as gemv_q6_k_kernel's units): step (j, c) of a super-block
// is element 128*(g/2) + 32j + 16*(g%2) + c of both, so one MFMA adds four
// elements' products for all 16 x 16 (row, token) pairs; each weight is
// formed once for the 16 tokens (signed 6-bit extract, int -> double, times
// d*sc: exact), each activation converted once for the 16 rows.  Four
// accumulators take the steps in turn.  The MFMA's 16 x 16 result: lane L,
// element r = row 4r + L/16, token L % 16.  The sum order differs from the
// reference's element order, with the same bound on the difference as the
// other Q6_K kernels.
constexpr int kQ6FWaves = 8;  // 8 against 4: 5632->2048 at 32 tokens 23.8 against 27.4 us
constexpr int kQ6FAcc = 4;    // accumulators taking the steps in turn
typedef double v4f64 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(64 * kQ6FWaves) void gemv_q6_k_batch_f64_kernel(const uint8_t* __restrict__ W,
                                                                             const float* __restrict__ x,
                                                                             float* __restrict__ y, int N, int K) {
    __shared__ v4f64 s_red[kQ6FWaves][64];
    const int nsb = K / 256;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, g = lane >> 4, half = g >> 1, hg = g & 1;
    const int r0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
    // rows past N use row N - 1 (not written)
    const uint8_t* rb = W + static_cast<size_t>(min(r0 + li, N - 1)) * nsb * 210;
    const float* xt = x + static_cast<size_t>(t0 + li) * K + 128 * half + 16 * hg;
    const int s_beg = wave * nsb / kQ6FWaves, s_end = (wave + 1) * nsb / kQ6FWaves;
    struct Raw {
        uint32_t qa[4], qb[4], qh[4];
        int sc[4];
        uint32_t d;
    };
    // the unit's bytes: ql g/2*64 + hg*16 (j = 0, 2) and +32 (j = 1, 3), qh
    // 128 + g/2*32 + hg*16, scales 192 + g/2*8 + hg + 2j, d at 208
    auto load_unit = [&](int sb, Raw& w) __attribute__((always_inline)) {
        const uint8_t* b = rb + static_cast<size_t>(sb) * 210;
        const uint16_t* pa = reinterpret_cast<const uint16_t*>(b + half * 64 + hg * 16);
        const uint16_t* pb = reinterpret_cast<const uint16_t*>(b + half * 64 + 32 + hg * 16);
        const uint16_t* ph = reinterpret_cast<const uint16_t*>(b + 128 + half * 32 + hg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w.qa[i] = pa[2 * i] | (static_cast<uint32_t>(pa[2 * i + 1]) << 16);
            w.qb[i] = pb[2 * i] | (static_cast<uint32_t>(pb[2 * i + 1]) << 16);
            w.qh[i] = ph[2 * i] | (static_cast<uint32_t>(ph[2 * i + 1]) << 16);
        }
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + half * 8 + hg);
#pragma unroll
        for (int j = 0; j < 4; ++j) w.sc[j] = sc[2 * j];
        w.d = *reinterpret_cast<const uint16_t*>(b + 208);
    };
    v4f64 acc[kQ6FAcc];
#pragma unroll
    for (int a = 0; a < kQ6FAcc; ++a) acc[a] = v4f64{0.0, 0.0, 0.0, 0.0};
    if (s_beg < s_end) {
        Raw cur;
        load_unit(s_beg, cur);
        for (int sb = s_beg; sb < s_end; ++sb) {
            Raw nxt;
            load_unit(min(sb + 1, s_end - 1), nxt);  // the next unit in flight (the last one loads itself again)
            // the lane's 64 activations of the super-block, all requested at once
            const float* xs = xt + static_cast<size_t>(sb) * 256;
            float4 xa[4][4];
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
                for (int j = 0; j < 4; ++j) xa[c4][j] = reinterpret_cast<const float4*>(xs + 32 * j)[c4];
            const float d = h2f(cur.d);
            double dsc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dsc[j] = static_cast<double>(d * static_cast<float>(cur.sc[j]));
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {  // columns 4c4 .. 4c4+3 of the unit's four groups
                const float4* xv = xa[c4];
                // 6-bit codes q + 32 four to a dword, bit 5 flipped (bits 6..7 ignored by the extract)
                const uint32_t qa = cur.qa[c4], qb = cur.qb[c4], hx = cur.qh[c4] ^ 0xaaaaaaaau;
                constexpr uint32_t kLo = 0x0f0f0f0fu;
                const uint32_t u[4] = {(qa & kLo) | ((hx << 4) & ~kLo), (qb & kLo) | ((hx << 2) & ~kLo),
                                       ((qa >> 4) & kLo) | (hx & ~kLo), ((qb >> 4) & kLo) | ((hx >> 2) & ~kLo)};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int q = static_cast<int>(u[j] << (26 - 8 * e)) >> 26;
                        const double a = static_cast<double>(q) * dsc[j];  // w, exact
                        const float xe = e == 0 ? xv[j].x : e == 1 ? xv[j].y : e == 2 ? xv[j].z : xv[j].w;
                        const double bx = static_cast<double>(xe);
                        v4f64& ac = acc[(4 * e + j) % kQ6FAcc];
                        ac = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bx, ac, 0, 0, 0);
                    }
                }
            }
            cur = nxt;
        }
    }
    v4f64 part = acc[0];
#pragma unroll
    for (int a = 1; a < kQ6FAcc; ++a) part += acc[a];
    s_red[wave][lane] = part;
    __syncthreads();
    if (wave == 0) {
        v4f64 tot = s_red[0][lane];
#pragma unroll
        for (int w = 1; w < kQ6FWaves; ++w) tot += s_red[w][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + 4 * r + g;
            if (row < N) y[static_cast<size_t>(t0 + li) * N + row] = static_cast<float>(tot[r]);
        }
    }
}

// rows x tokens of the Q6_K token-group tile
constexpr int kQ6BRows = 16, kQ6BTok = 16;

// F32 weights (dot_f32_simd, src/gguf_kernels.cpp:228-234, as tensor_matvec
// and tensor_matmul_batch call it): per (row, token) eight accumulators
// t_j = fma(w[i+j], x[i+j], t_j) over i = 0, 8, .. (< cols & ~7), held by a
// lane pair (t0..t3 and t4..t7); s = t0+t1+..+t7; then the scalar tail as the
// compiled reference runs it -- 4 elements at a time with rounded products
// and in-order adds, the last cols % 4 fused.
constexpr int kF32T = 256;
__global__ __launch_bounds__(kF32T) void gemv_f32_kernel(const float* __restrict__ W, const float* __restrict__ x,
                                                         float* __restrict__ y, int N, int K) {
    const int g = static_cast<int>((static_cast<size_t>(blockIdx.x) * kF32T + threadIdx.x) >> 1);
    const int h = threadIdx.x & 1;
    const bool live = g < N;
    const int r = live ? g : N - 1;  // lanes past the last row mirror it (results dropped)
    const float* wr = W + static_cast<size_t>(r) * K;
    const float* xb = x + static_cast<size_t>(blockIdx.y) * K;
    float t[4] = {0.f, 0.f, 0.f, 0.f};
    const int n8 = K & ~7;
    for (int i = 4 * h; i < n8; i += 8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = fmaf(wr[i + e], xb[i + e], t[e]);
    }
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = __shfl_xor(t[e], 1);  // the partner's four accumulators
    if (h == 0 && live) {
        float s = t[0];
        s = s + t[1];
        s = s + t[2];
        s = s + t[3];
        s = s + o[0];
        s = s + o[1];
        s = s + o[2];
        s = s + o[3];
        int i = n8;
        for (; i + 4 <= K; i += 4)
#pragma unroll
            for (int e = 0; e < 4; ++e) s = s + wr[i + e] * xb[i + e];
        for (; i < K; ++i) s = fmaf(wr[i], xb[i], s);
        y[static_cast<size_t>(blockIdx.y) * N + r] = s;
    }
}

// F16 weights (tensor_matvec / tensor_matmul_batch, src/gguf_kernels.cpp:250,
// :257): s = sum of double(f16(w))*x in double, rounded to f32 once.  One wave
// per (row, token); each lane keeps a double partial over elements l, l+64,
// .. (the products are exact in double), the wave adds them as a tree -- the
// reference adds in element order, so a result can differ from it only when
// the exact sum lies within ~1e-13 (relative) of an f32 rounding boundary.
constexpr int kF16T = 256;
__global__ __launch_bounds__(kF16T) void gemv_f16_kernel(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                                         float* __restrict__ y, int N, int K) {
    const int row = blockIdx.x * (kF16T / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= N) return;  // whole waves leave together
    const uint16_t* wr = W + static_cast<size_t>(row) * K;
    const float* xb = x + static_cast<size_t>(blockIdx.y) * K;
    double acc = 0.0;
    for (int c = lane; c < K; c += 64) acc = fma(static_cast<double>(h2f(wr[c])), static_cast<double>(xb[c]), acc);
    const double tot = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(blockIdx.y) * N + row] = static_cast<float>(tot);
}

int pick_rows_per_wg(size_t rows, size_t nb, size_t pair_budget) {
    // enough rows per workgroup that every lane owns at least one 8-block
    // unit, capped by the LDS budget of the pair buffer
    int r = static_cast<int>((kGemvThreads * 8 + nb - 1) / nb);
    if (r < 1) r = 1;
    const int cap = static_cast<int>(pair_budget / ((nb + 1) * sizeof(float2)));
    if (r > cap) r = cap;
    if (r < 1) r = 1;
    (void)rows;
    return r;
}

}  // namespace

hipError_t launch_gemv_q4_0(const uint8_t* W, const int8_t* aq, const float* ad, float* y, size_t rows, size_t cols,
                            hipStream_t st, size_t batch) {
    if (!rows || !batch) return hipSuccess;
    if (gemv_q4_0_rows16_ok(cols)) {  // one token per launch
        const size_t nbk = cols / 32;
        for (size_t b = 0; b < batch; ++b)
            if (hipError_t e = launch_gemv_q4_0_rows16(W, nullptr, aq + b * cols, ad + b * nbk, y + b * rows, rows,
                                                       cols, st))
                return e;
        return hipSuccess;
    }
    static const int mode = [] {
        const char* e = getenv("MVH_GEMV_LOAD");
        return e ? atoi(e) : kLoadStaged;
    }();
    const int nb = static_cast<int>(cols / 32);
    const int ngrp = (nb + 7) / 8;
    const size_t fixed = static_cast<size_t>(ngrp) * kActPitch + 8u * nb;
    const bool staged = mode == kLoadStaged && nb % 8 == 0;
    // staged tiles also hold the raw weight bytes of every row in LDS
    const size_t per_row = (nb + 1) * sizeof(float2) + (staged ? 18u * nb : 0u);
    int rpw = pick_rows_per_wg(rows, nb, 60 * 1024 - fixed);
    rpw = std::max(1, std::min<int>(rpw, static_cast<int>((60 * 1024 - fixed) / per_row)));
    const size_t lds = fixed + static_cast<size_t>(rpw) * per_row + 16;
    const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw), static_cast<unsigned>(batch));
    const int n = static_cast<int>(rows);
    if (nb % 8 != 0)
        gemv_q4_0_kernel<1, kLoadCached><<<grid, kGemvThreads, lds, st>>>(W, aq, ad, y, n, nb, rpw);
    else if (mode == kLoadStream)
        gemv_q4_0_kernel<8, kLoadStream><<<grid, kGemvThreads, lds, st>>>(W, aq, ad, y, n, nb, rpw);
    else if (mode == kLoadCached)
        gemv_q4_0_kernel<8, kLoadCached><<<grid, kGemvThreads, lds, st>>>(W, aq, ad, y, n, nb, rpw);
    else
        gemv_q4_0_kernel<8, kLoadStaged><<<grid, kGemvThreads, lds, st>>>(W, aq, ad, y, n, nb, rpw);
    return hipGetLastError();
}

template <uint32_t TYPE>
static hipError_t launch_f32act(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                                hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    const int nb = static_cast<int>(cols / 32);
    const int ngrp = (nb + 7) / 8;
    const size_t fixed = static_cast<size_t>(ngrp) * kXPitchF * 4;
    if (batch >= 2 && nb % 8 == 0) {
        // token groups of 4 (or 2) when their activations leave room for a few rows of pairs
        const int tt = 4 * fixed <= 36 * 1024 ? 4 : 2 * fixed <= 36 * 1024 ? 2 : 1;
        if (tt > 1) {
            const size_t budget = 60 * 1024 - tt * fixed;
            const int rpw = std::max(1, std::min(pick_rows_per_wg(rows, nb, budget / tt),
                                                 static_cast<int>(budget / (tt * (nb + 1) * sizeof(float2)))));
            const size_t lds = tt * fixed + static_cast<size_t>(tt) * rpw * (nb + 1) * sizeof(float2);
            const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw), static_cast<unsigned>((batch + tt - 1) / tt));
            if (tt == 4)
                gemv_f32act_tokens_kernel<TYPE, 4><<<grid, kGemvThreads, lds, st>>>(
                    W, x, y, static_cast<int>(rows), nb, rpw, static_cast<int>(batch));
            else
                gemv_f32act_tokens_kernel<TYPE, 2><<<grid, kGemvThreads, lds, st>>>(
                    W, x, y, static_cast<int>(rows), nb, rpw, static_cast<int>(batch));
            return hipGetLastError();
        }
    }
    const int rpw = pick_rows_per_wg(rows, nb, 60 * 1024 - fixed);
    const size_t lds = fixed + static_cast<size_t>(rpw) * (nb + 1) * sizeof(float2);
    const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw), static_cast<unsigned>(batch));
    if (nb % 8 == 0)
        gemv_f32act_kernel<TYPE, 8><<<grid, kGemvThreads, lds, st>>>(W, x, y, static_cast<int>(rows), nb, rpw);
    else
        gemv_f32act_kernel<TYPE, 1><<<grid, kGemvThreads, lds, st>>>(W, x, y, static_cast<int>(rows), nb, rpw);
    return hipGetLastError();
}

// One token, K % 256 == 0, K <= 16384: the persistent kernel; otherwise the
// two-phase kernel per token.
template <uint32_t TYPE>
static hipError_t launch_f32act_any(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols,
                                    size_t batch, hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    if constexpr (TYPE == kQ8_0) {
        // one token at K = 2048 / 4096: the row-group kernel
        if (batch == 1 && (cols == 2048 || cols == 4096) && (reinterpret_cast<uintptr_t>(W) & 7) == 0) {
            const unsigned grid = static_cast<unsigned>((rows + 15) / 16);
            if (cols == 2048)
                gemv_q8_0_f32act_rows16<4><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows));
            else
                gemv_q8_0_f32act_rows16<8><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows));
            return hipGetLastError();
        }
    }
    if (batch == 1 && cols % 256 == 0 && cols / 128 <= 64) {
        static const int cus = [] {
            int dev = 0;
            hipDeviceProp_t prop;
            if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                prop.multiProcessorCount > 0)
                return prop.multiProcessorCount;
            return 256;
        }();
        const int nb = static_cast<int>(cols / 32);
        const int tr = 64 / (nb / 4);
        const int ntiles = static_cast<int>((rows + tr - 1) / tr);
        const int waves = std::min(ntiles, cus * 16);
        const size_t lds = static_cast<size_t>(nb / 8) * kXPitchF * 4;
        const int g = (waves + 3) / 4, n = static_cast<int>(rows);
        if constexpr (TYPE == kQ4_0)
            gemv_f32act_persistent_q4_0<<<g, 256, lds, st>>>(W, x, y, n, nb, ntiles);
        else if constexpr (TYPE == kQ8_0)
            gemv_f32act_persistent_q8_0<<<g, 256, lds, st>>>(W, x, y, n, nb, ntiles);
        else if constexpr (TYPE == kNQ4_0)
            gemv_f32act_persistent_nq4_0<<<g, 256, lds, st>>>(W, x, y, n, nb, ntiles);
        else
            gemv_f32act_persistent_nq8_0<<<g, 256, lds, st>>>(W, x, y, n, nb, ntiles);
        return hipGetLastError();
    }
    if constexpr (TYPE == kQ4_0 || TYPE == kQ8_0) {
        if (cols % 256 == 0 && batch >= kR2Tok) {
            // whole groups of kR2Tok tokens on the staged two-row kernel, the rest below
            const size_t groups = batch / kR2Tok;
            const dim3 grid(static_cast<unsigned>((rows + kR2Rows - 1) / kR2Rows), static_cast<unsigned>(groups));
            batch_f32act_rows2_kernel<TYPE, true><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows),
                                                                        static_cast<int>(cols / 32));
            const size_t done = groups * kR2Tok;
            if (done == batch) return hipGetLastError();
            x += done * cols;
            y += done * rows;
            batch -= done;
        }
    }
    return launch_f32act<TYPE>(W, x, y, rows, cols, batch, st);
}

hipError_t launch_gemv_q8_0(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                            hipStream_t st) {
    return launch_f32act_any<kQ8_0>(W, x, y, rows, cols, batch, st);
}

hipError_t launch_gemv_q4_0_f32act(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                                   hipStream_t st) {
    return launch_f32act_any<kQ4_0>(W, x, y, rows, cols, batch, st);
}

// dot_q4_0 / dot_q8_0 of the native blocks (src/quant.cpp:87-156): the same
// eight-lane block sums and in-order sum = fma(s, d, sum) as dot_q4_0_fp32 /
// dot_q8_0_fp32, over 20- / 36-byte blocks with an f32 scale.
hipError_t launch_gemv_native_f32act(uint32_t type, const uint8_t* W, const float* x, float* y, size_t rows,
                                     size_t cols, size_t batch, hipStream_t st) {
    if (type == kNQ4_0) return launch_f32act_any<kNQ4_0>(W, x, y, rows, cols, batch, st);
    if (type == kNQ8_0) return launch_f32act_any<kNQ8_0>(W, x, y, rows, cols, batch, st);
    return hipErrorInvalidValue;
}

hipError_t launch_batch4_f32act(uint32_t type, const uint8_t* W, const float* x, float* y, size_t rows, size_t cols,
                                size_t batch, hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    const int nb = static_cast<int>(cols / 32);
    static_assert(kBT * kBRows == 256, "one output per thread in the final sum");
    if (cols % 256 == 0 && batch >= kR2Tok) {
        // whole groups of kR2Tok tokens with two rows per lane, the rest below
        const size_t groups = batch / kR2Tok;
        const dim3 grid(static_cast<unsigned>((rows + kR2Rows - 1) / kR2Rows), static_cast<unsigned>(groups));
        if (type == kQ4_0)
            batch_f32act_rows2_kernel<kQ4_0, false><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows), nb);
        else
            batch_f32act_rows2_kernel<kQ8_0, false><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows), nb);
        const size_t done = groups * kR2Tok;
        if (done == batch) return hipGetLastError();
        x += done * cols;
        y += done * rows;
        batch -= done;
    }
    if (cols % 256 == 0 && batch >= kBT) {
        // whole groups of kBT tokens on the lane-spread kernel, the rest per token below
        const size_t groups = batch / kBT;
        const dim3 grid(static_cast<unsigned>((rows + kBRows - 1) / kBRows), static_cast<unsigned>(groups));
        if (type == kQ4_0)
            batch_f32act_lanes_kernel<kQ4_0><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows), nb);
        else
            batch_f32act_lanes_kernel<kQ8_0><<<grid, 256, 0, st>>>(W, x, y, static_cast<int>(rows), nb);
        const size_t done = groups * kBT;
        if (done == batch) return hipGetLastError();
        x += done * cols;
        y += done * rows;
        batch -= done;
    }
    const dim3 grid(static_cast<unsigned>((rows + 255) / 256), static_cast<unsigned>(batch));
    if (type == kQ4_0)
        batch4_f32act_kernel<kQ4_0><<<grid, 256, cols * sizeof(float), st>>>(W, x, y, static_cast<int>(rows), nb);
    else
        batch4_f32act_kernel<kQ8_0><<<grid, 256, cols * sizeof(float), st>>>(W, x, y, static_cast<int>(rows), nb);
    return hipGetLastError();
}

hipError_t launch_gemv_f32(const float* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                           hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((2 * rows + kF32T - 1) / kF32T), static_cast<unsigned>(batch));
    gemv_f32_kernel<<<grid, kF32T, 0, st>>>(W, x, y, static_cast<int>(rows), static_cast<int>(cols));
    return hipGetLastError();
}

hipError_t launch_gemv_f16(const uint16_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                           hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((rows + kF16T / 64 - 1) / (kF16T / 64)), static_cast<unsigned>(batch));
    gemv_f16_kernel<<<grid, kF16T, 0, st>>>(W, x, y, static_cast<int>(rows), static_cast<int>(cols));
    return hipGetLastError();
}

size_t gemv_decode_rows_per_wg(uint32_t type, size_t rows, size_t cols) {
    switch (type) {
        case kQ4_0: return gemv_q4_0_rows16_ok(cols) ? 16 : 0;
        case kQ8_0: return cols == 2048 || cols == 4096 ? 16 : 0;  // gemv_q8_0_f32act_rows16
        case kQ6_K: {  // the one-token choice of launch_gemv_q6_k below
            if (cols % 256) return 0;
            const size_t units = cols / 64;
            const bool half = units <= 64;
            const size_t rpw1 = half ? 8 : 4;
            const bool two = rows >= 1024 * 2 * rpw1;
            return half ? (two ? 16 : 8) : 8;
        }
    }
    return 0;
}

hipError_t launch_gemv_q6_k(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                            hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    if (batch >= kQ6BTok) {
        // whole groups of kQ6BTok tokens on the batch kernel, the rest per token below
        const size_t groups = batch / kQ6BTok;
        const dim3 bgrid(static_cast<unsigned>((rows + kQ6BRows - 1) / kQ6BRows), static_cast<unsigned>(groups));
        gemv_q6_k_batch_f64_kernel<<<bgrid, 64 * kQ6FWaves, 0, st>>>(W, x, y, static_cast<int>(rows),
                                                                     static_cast<int>(cols));
        const size_t done = groups * kQ6BTok;
        if (done == batch) return hipGetLastError();
        x += done * cols;
        y += done * rows;
        batch -= done;
    }
    // 32 lanes per row up to 64 units, 64 beyond; two rows per lane when that
    // still leaves at least four workgroups per CU (4096->32000 34-36 against
    // 38 us, 2048->32000 19 against 20 us; 5632->2048 stays at one row per
    // lane: 7.0 against 8.0 us)
    const size_t units = cols / 64;  // 64-element units per row
    const bool half = units <= 64;
    const size_t rpw1 = half ? 8 : 4;  // rows per workgroup at one row per lane
    const bool two = rows >= 1024 * 2 * rpw1;
    const size_t rpw = two ? 2 * rpw1 : rpw1;
    const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw), static_cast<unsigned>(batch));
    const size_t lds = cols * sizeof(float);
    const int n = static_cast<int>(rows), k = static_cast<int>(cols);
    if (half) {
        if (two)
            gemv_q6_k_kernel<32, 2><<<grid, kQ6Threads, lds, st>>>(W, x, y, n, k);
        else
            gemv_q6_k_kernel<32, 1><<<grid, kQ6Threads, lds, st>>>(W, x, y, n, k);
    } else {
        if (two) {
            gemv_q6_k_kernel<64, 2><<<grid, kQ6Threads, lds, st>>>(W, x, y, n, k);
        } else {
            // 8 waves (8 rows) per workgroup: the activation staged once for
            // twice the rows (5632->2048 6.7 against 7.0 us; 16 waves 8.8)
            const dim3 g8(static_cast<unsigned>((rows + 7) / 8), static_cast<unsigned>(batch));
            gemv_q6_k_kernel<64, 1, 512><<<g8, 512, lds, st>>>(W, x, y, n, k);
        }
    }
    return hipGetLastError();
}

}  // namespace mvh
