// mvh_gemv_q4.hip -- Q4 x Q8 decode GEMV (K % 256 == 0, K <= 16384) for both
// block formats of the path.
//
// Numerics, per row, over blocks b in order (one fma per block, no split):
//   GGUF block_q4_0 (tensor_matvec's Q4_0 branch, dot_q4_q8,
//   src/gguf_kernels.cpp:189,246):   sum = fma(f16(d_w) * d_a, float(isum_b), sum)
//   native BlockQ4_0 (dot_q4_q8, src/quant_kernels.cpp:52-66):
//                                    sum = fma(float(isum_b) * d_w, d_x, sum)
// isum_b is the exact integer block dot, v_dot4_i32_i8 on the raw nibbles
// minus 8 * (the block's activation byte sum).
//
// Work split.  One wave = one tile of 4 rows; lanes form four 16-lane row
// groups (DPP "rows"), lane g of group r owning, in pass p, unit 16p + g of
// tile row r (a unit = 8 consecutive blocks = 144 or 160 bytes of the row,
// 16-byte loads).  Passes are column-major in K: pass 0 holds the first 16
// units of all four rows, so, vector loads completing in issue order, the
// front of K arrives first.  Per pass every lane turns its unit into 8
// (p_b, f_b) pairs in registers, then the rows' fma chains walk the group's
// lanes in unit order (DPP row_ror:1: at each stage a lane continues from its
// left neighbour's value; lane 0 starts a pass from lane 15's value at the end
// of the previous pass).  Pass p + 1's loads are issued just before pass p is
// computed, so a pass's chain runs while the next pass's units are still
// arriving; only the last pass's stages follow the last byte.
//
// The activation (Q8 bytes, per-block scale and byte sum) is staged once per
// workgroup of 4 waves in LDS.  Its global loads are issued before the weight
// loads and the staging stores are branch-free (lanes past the end write a
// dummy slot): a load used only under a branch is sunk into it by the
// compiler, behind the weight loads, and waiting for it then waits for every
// weight load (vector loads complete in issue order).  Q8 bytes of a block
// are stored as 16 bytes paired with the low nibbles, then 16 paired with the
// high nibbles: natural order for GGUF (elements 0..15, 16..31), even/odd
// elements for the native interleaved nibbles (element 2i = low nibble of
// byte i).
#include "mvh_kernels.hpp"

#include <algorithm>

namespace mvh {
namespace {

constexpr int kActPitch = 272;  // LDS bytes per 8-block group of Q8 bytes (256 + 16 pad)
constexpr int kDasPitch = 80;   // LDS bytes per 8-block group of (d, byte sum) pairs (64 + 16 pad)

enum { kSrcQ8 = 0, kSrcF32 = 1, kSrcNative = 2 };

struct Q4Gguf {  // 18-byte block: f16 d, qs[16] (element i low nibble, 16+i high)
    static constexpr int kBytes = 18, kUnit16 = 9;
    static __device__ __forceinline__ void block(const uint32_t* w, int j, uint32_t& dbits, uint32_t (&qs)[4]) {
        const int o = 18 * j;
        if ((j & 1) == 0) {
            dbits = w[o / 4] & 0xffffu;
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = align16(w[o / 4 + k + 1], w[o / 4 + k]);
        } else {
            dbits = w[o / 4] >> 16;
#pragma unroll
            for (int k = 0; k < 4; ++k) qs[k] = w[(o + 2) / 4 + k];
        }
    }
    static __device__ __forceinline__ float2 pair(uint32_t dbits, float da, int isum) {
        return make_float2(h2f(dbits) * da, static_cast<float>(isum));
    }
};

struct Q4Native {  // 20-byte block: f32 d, qs[16] (element 2i low nibble, 2i+1 high)
    static constexpr int kBytes = 20, kUnit16 = 10;
    static __device__ __forceinline__ void block(const uint32_t* w, int j, uint32_t& dbits, uint32_t (&qs)[4]) {
        dbits = w[5 * j];
#pragma unroll
        for (int k = 0; k < 4; ++k) qs[k] = w[5 * j + 1 + k];
    }
    static __device__ __forceinline__ float2 pair(uint32_t dbits, float dx, int isum) {
        return make_float2(static_cast<float>(isum) * __uint_as_float(dbits), dx);
    }
};

__device__ __forceinline__ int dot_nib(const uint32_t (&qs)[4], const uint4 a0, const uint4 a1) {
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

__device__ __forceinline__ int byte_sum16(uint4 a) {
    constexpr int ones = 0x01010101;
    int s = __builtin_amdgcn_sdot4(static_cast<int>(a.x), ones, 0, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(a.y), ones, s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(a.z), ones, s, false);
    return __builtin_amdgcn_sdot4(static_cast<int>(a.w), ones, s, false);
}

// DPP row_ror:1 -- lane g of each 16-lane row receives lane (g - 1) mod 16.
__device__ __forceinline__ float row_ror1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));
}

// NP passes (one per 128 blocks of K); CH activation loads per thread: 16-byte
// Q8 chunks (kSrcQ8, nb * 2 <= 256 CH), native blocks (kSrcNative, nb <= 256 CH)
// or fp32 float4s (kSrcF32, nb * 8 <= 256 CH), all issued before the weights.
// W, act and ad are deliberately not __restrict__: with it the compiler may
// sink the weight loads past the staging barrier (nothing could write
// restrict-qualified read-only memory), and they would then be issued only
// after the activation is staged.
template <class F, int SRC, int NP, int CH>
__global__ __launch_bounds__(256) void gemv_q4_rows16(const uint8_t* W, const void* act, const float* ad,
                                                      float* __restrict__ y, int N, int nb, int ntiles) {
    constexpr int kW = 4 * F::kUnit16;  // dwords of one unit
    extern __shared__ __align__(16) uint8_t smem[];
    const int upr = nb >> 3;
    uint8_t* s_aq = smem;
    uint8_t* s_das = smem + upr * kActPitch;
    uint8_t* dummy = s_das + upr * kDasPitch;  // 64 bytes: staging stores of lanes past the end
    const int t = threadIdx.x, lane = t & 63;
    const int r = lane >> 4, g = lane & 15;
    const int tile = blockIdx.x * 4 + (t >> 6);
    const size_t row_bytes = static_cast<size_t>(nb) * F::kBytes;

    // 1. activation loads, before any weight load
    uint4 aqv[SRC == kSrcQ8 ? CH : 1];
    float adv[SRC == kSrcQ8 ? CH : 1];
    uint32_t anv[SRC == kSrcNative ? CH : 1][9];
    float4 axv[SRC == kSrcF32 ? CH : 1];
    if constexpr (SRC == kSrcF32) {  // fp32 input: CH float4 per thread, all issued here
        const float4* x4 = static_cast<const float4*>(act);
#pragma unroll
        for (int i = 0; i < CH; ++i) axv[i] = x4[min(t + 256 * i, nb * 8 - 1)];
    } else if constexpr (SRC == kSrcQ8) {
        const uint4* aq4 = static_cast<const uint4*>(act);
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = min(t + 256 * i, nb * 2 - 1);
            aqv[i] = aq4[c];
            adv[i] = ad[c >> 1];
        }
    } else if constexpr (SRC == kSrcNative) {
        const uint32_t* xb = static_cast<const uint32_t*>(act);
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int b = min(t + 256 * i, nb - 1);
#pragma unroll
            for (int k = 0; k < 9; ++k) anv[i][k] = xb[9 * b + k];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the tile's weight units of the first pass (every load unconditional:
    // rows past N and units past the row reload the last valid ones); pass
    // p + 1 is issued just before pass p is computed, so a wave reaches the
    // staging barrier after issuing one pass, not all of them (a wave stalls at
    // the issue of a load while the memory system holds too many of its
    // requests, and its chain could then only start once nearly all of its
    // bytes had arrived)
    uint32_t w[NP][kW];
    const int grow_c = min(min(tile, ntiles - 1) * 4 + r, N - 1);
    auto issue = [&](int p) {
        const int u = min(16 * p + g, upr - 1);
        const uint4* src = reinterpret_cast<const uint4*>(W + static_cast<size_t>(grow_c) * row_bytes +
                                                          static_cast<size_t>(u) * 8 * F::kBytes);
#pragma unroll
        for (int k = 0; k < F::kUnit16; ++k) {
            const uint4 v = src[k];
            w[p][4 * k] = v.x;
            w[p][4 * k + 1] = v.y;
            w[p][4 * k + 2] = v.z;
            w[p][4 * k + 3] = v.w;
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the passes' loads in K order
    };
    issue(0);

    // 3. the activation into LDS: Q8 bytes, then (d, byte sum) per block
    if constexpr (SRC == kSrcQ8) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = t + 256 * i;
            const int s = byte_sum16(aqv[i]);
            const int both = s + __builtin_amdgcn_mov_dpp(s, 0xb1, 0xf, 0xf, false);  // chunks c, c^1: one block
            const bool v = c < nb * 2;
            const int b = v ? c >> 1 : 0;
            *reinterpret_cast<uint4*>(v ? s_aq + (b >> 3) * kActPitch + (b & 7) * 32 + (c & 1) * 16 : dummy) = aqv[i];
            *reinterpret_cast<int2*>(v && (c & 1) == 0 ? s_das + (b >> 3) * kDasPitch + (b & 7) * 8 : dummy + 32) =
                make_int2(__float_as_int(adv[i]), both);
        }
    } else if constexpr (SRC == kSrcNative) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int b0 = t + 256 * i;
            const bool v = b0 < nb;
            const int b = v ? b0 : 0;
            const uint32_t* q = anv[i] + 1;
            uint4 ev, od;  // bytes of the even / odd elements
            ev.x = __builtin_amdgcn_perm(q[1], q[0], 0x06040200u);
            ev.y = __builtin_amdgcn_perm(q[3], q[2], 0x06040200u);
            ev.z = __builtin_amdgcn_perm(q[5], q[4], 0x06040200u);
            ev.w = __builtin_amdgcn_perm(q[7], q[6], 0x06040200u);
            od.x = __builtin_amdgcn_perm(q[1], q[0], 0x07050301u);
            od.y = __builtin_amdgcn_perm(q[3], q[2], 0x07050301u);
            od.z = __builtin_amdgcn_perm(q[5], q[4], 0x07050301u);
            od.w = __builtin_amdgcn_perm(q[7], q[6], 0x07050301u);
            uint8_t* dst = v ? s_aq + (b >> 3) * kActPitch + (b & 7) * 32 : dummy;
            *reinterpret_cast<uint4*>(dst) = ev;
            *reinterpret_cast<uint4*>(dst + 16) = od;
            *reinterpret_cast<int2*>(v ? s_das + (b >> 3) * kDasPitch + (b & 7) * 8 : dummy + 32) =
                make_int2(static_cast<int>(anv[i][0]), byte_sum16(ev) + byte_sum16(od));
        }
    } else {  // kSrcF32: quantize_q8 of the fp32 input, 8 lanes per block
        const int n4 = nb * 8;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i = t + 256 * c;
            float d;
            int s;
            const uint32_t q = quantize_q8_x4(axv[c], d, s);
            const bool ok = i < n4;
            const int b = ok ? i >> 3 : 0;
            *reinterpret_cast<uint32_t*>(ok ? s_aq + (b >> 3) * kActPitch + (b & 7) * 32 + (i & 7) * 4 : dummy) = q;
            *reinterpret_cast<int2*>(ok && (i & 7) == 0 ? s_das + (b >> 3) * kDasPitch + (b & 7) * 8 : dummy + 32) =
                make_int2(__float_as_int(d), s);
        }
    }
    __syncthreads();

    // 4. pass by pass: the next pass's loads, pairs in registers, then the chain stages
    float sum = 0.0f;
    int last = 15;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if (p + 1 < NP) issue(p + 1);
        const int uu = min(16 * p + g, upr - 1);
        const uint8_t* ag = s_aq + uu * kActPitch;
        const uint8_t* dg = s_das + uu * kDasPitch;
        float2 pr[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t dbits, qs[4];
            F::block(w[p], j, dbits, qs);
            const uint4 a0 = *reinterpret_cast<const uint4*>(ag + 32 * j);
            const uint4 a1 = *reinterpret_cast<const uint4*>(ag + 32 * j + 16);
            const int2 ds = *reinterpret_cast<const int2*>(dg + 8 * j);
            const int isum = dot_nib(qs, a0, a1) - 8 * ds.y;
            pr[j] = F::pair(dbits, __int_as_float(ds.x), isum);
        }
        // lane 0 starts from the row's chain so far (lane 15 at the end of the
        // previous, whole, pass); at stage st every lane redoes its 8 fmas from
        // its left neighbour's value, lane g's value being final from stage g on
        const float carry = p == 0 ? 0.0f : row_ror1(sum);
        const int ng = min(16, upr - 16 * p);
        for (int st = 0; st < ng; ++st) {
            const float in = row_ror1(sum);
            float acc = g == 0 ? carry : in;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = fmaf(pr[j].x, pr[j].y, acc);
            sum = acc;
        }
        last = ng - 1;
        if (NP > 1) __builtin_amdgcn_sched_barrier(0);  // the next pass's loads stay ahead of its pairs
    }
    const int grow = tile * 4 + r;
    if (tile < ntiles && grow < N && g == last) y[grow] = sum;
}

template <class F, int SRC, int NP>
hipError_t launch_np(const uint8_t* W, const void* act, const float* ad, float* y, int N, int nb, hipStream_t st) {
    const int ntiles = (N + 3) / 4;
    const unsigned grid = static_cast<unsigned>((ntiles + 3) / 4);
    const size_t lds = static_cast<size_t>(nb / 8) * (kActPitch + kDasPitch) + 64;
    if constexpr (SRC == kSrcNative) {  // native blocks per thread: nb / 256
        if (nb <= 256)
            gemv_q4_rows16<F, SRC, NP, 1><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, ntiles);
        else
            gemv_q4_rows16<F, SRC, NP, 2><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, ntiles);
    } else if constexpr (SRC == kSrcF32) {  // float4 per thread: nb * 8 / 256 <= 4 * NP
        gemv_q4_rows16<F, SRC, NP, 4 * NP><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, ntiles);
    } else {  // Q8 chunks per thread: nb * 2 / 256 = NP
        gemv_q4_rows16<F, SRC, NP, NP><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, ntiles);
    }
    return hipGetLastError();
}

template <class F, int SRC>
hipError_t launch_rows16(const uint8_t* W, const void* act, const float* ad, float* y, size_t rows, size_t cols,
                         hipStream_t st) {
    if (!rows) return hipSuccess;
    const int nb = static_cast<int>(cols / 32), N = static_cast<int>(rows);
    switch ((nb + 127) / 128) {  // passes of 16 units = 128 blocks
        case 1: return launch_np<F, SRC, 1>(W, act, ad, y, N, nb, st);
        case 2: return launch_np<F, SRC, 2>(W, act, ad, y, N, nb, st);
        case 3: return launch_np<F, SRC, 3>(W, act, ad, y, N, nb, st);
        default: return launch_np<F, SRC, 4>(W, act, ad, y, N, nb, st);
    }
}

}  // namespace

bool gemv_q4_0_rows16_ok(size_t cols) { return cols % 256 == 0 && cols >= 256 && cols <= 16384; }

hipError_t launch_gemv_q4_0_rows16(const uint8_t* W, const float* x, const int8_t* aq, const float* ad, float* y,
                                   size_t rows, size_t cols, hipStream_t st) {
    if (x) return launch_rows16<Q4Gguf, kSrcF32>(W, x, nullptr, y, rows, cols, st);
    return launch_rows16<Q4Gguf, kSrcQ8>(W, aq, ad, y, rows, cols, st);
}

hipError_t launch_gemv_q4q8_native_rows16(const uint8_t* W, const uint8_t* xq, float* y, size_t rows, size_t cols,
                                          hipStream_t st) {
    return launch_rows16<Q4Native, kSrcNative>(W, xq, nullptr, y, rows, cols, st);
}

}  // namespace mvh
