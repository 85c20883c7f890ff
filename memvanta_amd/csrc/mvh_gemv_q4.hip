// mvh_gemv_q4.hip -- persistent Q4_0 x Q8 decode GEMV for K % 256 == 0.
//
// Numerics are those of tensor_matvec's Q4_0 branch (src/gguf_kernels.cpp:246):
// x is quantized with quantize_q8 (:160-172), then per row
//   sum = fma(f16(d_w) * d_a, float(isum_b), sum)   over blocks b in order (:189).
// Work split (one wave = one tile of TR = 64/(K/256) whole rows):
//   * lane (r, u) owns "unit" u of row r -- 8 consecutive blocks = 144 bytes,
//     the units of a row sit in consecutive lanes -- loads it with 9 x 16-byte
//     loads and turns its 8 blocks into (p_b = d_w*d_a, f_b = float(isum_b))
//     pairs held in registers (isum via v_dot4_i32_i8, exact);
//   * the row's fma chain then walks the lanes in unit order: at every stage
//     each lane takes its left neighbour's running value (DPP wave_shr:1) and
//     applies its 8 fmas; after K/256 stages the last lane of the row holds
//     the reference's in-order chain, bit for bit.
// Throughput structure: persistent waves walk tiles with a stride of the
// grid's wave count; the units of the next two tiles are in flight in
// registers while a tile is reduced; the fp32 input is quantized into LDS by
// every workgroup (no separate launch) while the first loads are in flight.
#include "mvh_kernels.hpp"

#include <algorithm>
#include <cstdlib>

namespace mvh {
namespace {

constexpr int kActPitch = 272;  // LDS bytes per 8-block activation group (256 + 16 pad)

__device__ __forceinline__ void load_unit(const uint8_t* __restrict__ W, size_t row_bytes, int grow, int unit,
                                          uint32_t (&w)[36]) {
    const uint4* src = reinterpret_cast<const uint4*>(W + static_cast<size_t>(grow) * row_bytes + unit * 144);
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const uint4 v = src[k];
        w[4 * k] = v.x;
        w[4 * k + 1] = v.y;
        w[4 * k + 2] = v.z;
        w[4 * k + 3] = v.w;
    }
}

__device__ __forceinline__ int dot_nib(const uint32_t (&qs)[4], const uint4 a0, const uint4 a1) {
    // qs byte i holds element i (low nibble) and element 16+i (high nibble)
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

// 8 pairs of one unit; agrp = the unit's activation group, b0 = first block.
__device__ __forceinline__ void unit_pairs(const uint32_t (&w)[36], const uint8_t* agrp, const float* s_ad,
                                           const int* s_as, int b0, float2* dst) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int o = 18 * j;  // block j starts at byte 18j of the unit
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
        const int isum = dot_nib(qs, a[0], a[1]) - 8 * s_as[b0 + j];
        dst[j] = make_float2(h2f(dbits) * s_ad[b0 + j], static_cast<float>(isum));
    }
}

// DPP wave_shr:1 -- lane l receives lane l-1's value (lane 0 gets `old`).
__device__ __forceinline__ float shift_up1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, false));
}

template <bool QUANT, int kT>
__global__ __launch_bounds__(kT) void gemv_q4_0_persistent_v1(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                           const int8_t* __restrict__ aq,
                                                           const float* __restrict__ ad, float* __restrict__ y, int N,
                                                           int nb, int ntiles) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int upr = nb >> 3;  // units (8 blocks, 144 bytes) per row; upr <= 64
    uint8_t* s_aq = smem;
    float* s_ad = reinterpret_cast<float*>(smem + upr * kActPitch);
    int* s_as = reinterpret_cast<int*>(s_ad + nb);
    const size_t row_bytes = static_cast<size_t>(nb) * 18;

    // wave-local tiles of TR whole rows: lane = (row r, unit u), units of a
    // row in consecutive lanes
    const int t = threadIdx.x, lane = t & 63;
    const int TR = 64 / upr;
    const int r = lane / upr, u = lane - r * upr;
    const bool worker = r < TR;
    const int gw = blockIdx.x * (kT / 64) + (t >> 6);
    const int GW = gridDim.x * (kT / 64);

    // weight units of this wave's first two tiles go out first
    uint32_t wa[36], wb[36];
    int tile = gw;
    if (worker && tile < ntiles && tile * TR + r < N) load_unit(W, row_bytes, tile * TR + r, u, wa);
    if (worker && tile + GW < ntiles && (tile + GW) * TR + r < N) load_unit(W, row_bytes, (tile + GW) * TR + r, u, wb);

    // stage the Q8 activation (padded 8-block groups) while they are in flight
    if constexpr (QUANT) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const int n4 = nb * 8;  // float4s; a group of 8 lanes = one 32-element block
        for (int i0 = 0; i0 < n4; i0 += 4 * kT) {
            float4 v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = i0 + k * kT + t;
                v[k] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (i0 + k * kT >= n4) break;  // uniform: skip slices past the end
                const int i = i0 + k * kT + t;
                float d;
                int s;
                const uint32_t q = quantize_q8_x4(v[k], d, s);
                if (i < n4) {
                    const int b = i >> 3;
                    *reinterpret_cast<uint32_t*>(s_aq + (b >> 3) * kActPitch + (b & 7) * 32 + (i & 7) * 4) = q;
                    if ((i & 7) == 0) {
                        s_ad[b] = d;
                        s_as[b] = s;
                    }
                }
            }
        }
    } else {
        for (int c = t; c < nb * 2; c += kT)  // 16-byte chunks of the int8 activation
            *reinterpret_cast<uint4*>(s_aq + (c >> 4) * kActPitch + (c & 15) * 16) = reinterpret_cast<const uint4*>(aq)[c];
        for (int b = t; b < nb; b += kT) s_ad[b] = ad[b];
        __syncthreads();
        for (int b = t; b < nb; b += kT) {  // s_b = sum of the block's 32 activation bytes
            const uint4* a = reinterpret_cast<const uint4*>(s_aq + (b >> 3) * kActPitch + (b & 7) * 32);
            const uint4 a0 = a[0], a1 = a[1];
            constexpr int ones = 0x01010101;
            int s = 0;
            s = __builtin_amdgcn_sdot4(static_cast<int>(a0.x), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a0.y), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a0.z), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a0.w), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a1.x), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a1.y), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a1.z), ones, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(a1.w), ones, s, false);
            s_as[b] = s;
        }
    }
    __syncthreads();

    const uint8_t* agrp = s_aq + (worker ? u : 0) * kActPitch;
    const int b0 = (worker ? u : 0) * 8;
    // One tile: pairs in registers, then the row chains run through the lanes
    // in unit order: at stage s the lane holding unit s of each row continues
    // the fma chain from the running sum its left neighbour produced at s-1.
    auto tile_step = [&](int tl, const uint32_t (&w)[36]) {
        const int grow = tl * TR + r;
        const bool live = worker && grow < N;
        float2 pr[8];
        if (live) unit_pairs(w, agrp, s_ad, s_as, b0, pr);
        // every lane redoes its 8 fmas from its left neighbour's value at every
        // stage; lane u's value is final from stage u on (its neighbour's was
        // final at u-1), so after upr stages the last lane of each row holds
        // the complete in-order chain
        float sum = 0.0f;
        for (int st = 0; st < upr; ++st) {
            const float in = shift_up1(sum);
            float acc = u == 0 ? 0.0f : in;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = fmaf(pr[j].x, pr[j].y, acc);
            sum = acc;
        }
        if (live && u == upr - 1) y[grow] = sum;
    };

    while (tile < ntiles) {
        tile_step(tile, wa);
        if (worker && tile + 2 * GW < ntiles && (tile + 2 * GW) * TR + r < N)
            load_unit(W, row_bytes, (tile + 2 * GW) * TR + r, u, wa);
        tile += GW;
        if (tile >= ntiles) break;
        tile_step(tile, wb);
        if (worker && tile + 2 * GW < ntiles && (tile + 2 * GW) * TR + r < N)
            load_unit(W, row_bytes, (tile + 2 * GW) * TR + r, u, wb);
        tile += GW;
    }
}

int g_cu_count = 0;

}  // namespace

// LDS bytes of the persistent kernel for a given K (activation only).
static size_t persistent_lds(int nb) { return static_cast<size_t>(nb / 8) * kActPitch + 8u * nb; }


static hipError_t launch_gemv_q4_0_persistent_v1(const uint8_t* W, const float* x, const int8_t* aq, const float* ad, float* y,
                                       size_t rows, size_t cols, hipStream_t st) {
    if (!rows) return hipSuccess;
    if (!g_cu_count) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            g_cu_count = prop.multiProcessorCount;
        if (g_cu_count <= 0) g_cu_count = 256;
    }
    const int nb = static_cast<int>(cols / 32);
    const int tr = 64 / (nb / 8);
    const int ntiles = static_cast<int>((rows + tr - 1) / tr);
    const size_t lds = persistent_lds(nb);
    static const int wpc = [] {  // resident waves per CU (tuning override)
        const char* e = getenv("MVH_GEMV_WPC");
        return e && atoi(e) > 0 ? atoi(e) : 16;
    }();
    const int waves = std::min(ntiles, g_cu_count * wpc);
    if (x) {
        // fp32 input: every workgroup quantizes it into LDS
        constexpr int T = 256;
        const int grid = (waves + T / 64 - 1) / (T / 64);
        gemv_q4_0_persistent_v1<true, T><<<grid, T, lds, st>>>(W, x, nullptr, nullptr, y, static_cast<int>(rows), nb,
                                                            ntiles);
    } else {
        // workgroup size (tuning override): every workgroup stages the
        // activation once, so larger groups stage it fewer times
        static const int wg = [] {
            const char* e = getenv("MVH_GEMV_WG");
            const int v = e ? atoi(e) : 256;
            return v == 512 || v == 1024 ? v : 256;
        }();
        const int grid = (waves + wg / 64 - 1) / (wg / 64);
        if (wg == 1024)
            gemv_q4_0_persistent_v1<false, 1024><<<grid, 1024, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                       nb, ntiles);
        else if (wg == 512)
            gemv_q4_0_persistent_v1<false, 512><<<grid, 512, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                     nb, ntiles);
        else
            gemv_q4_0_persistent_v1<false, 256><<<grid, 256, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                     nb, ntiles);
    }
    return hipGetLastError();
}


namespace {

// ============================================================================
// Q4 x Q8 decode GEMV, second structure (both block formats of the path).
//
// Numerics, per row, over blocks b in order (one fma per block, no split):
//   GGUF block_q4_0 (dot_q4_q8, src/gguf_kernels.cpp:189):
//       sum = fma(f16(d_w) * d_a, float(isum_b), sum)
//   native BlockQ4_0 (dot_q4_q8, src/quant_kernels.cpp:52-66):
//       sum = fma(float(isum_b) * d_w, d_x, sum)
// isum_b is the exact integer block dot, from v_dot4_i32_i8 on the raw
// nibbles minus 8 * (sum of the block's activation bytes).
//
// Work split.  A workgroup of 4 waves; each wave walks tiles of TR rows
// (persistent, stride = the grid's wave count).  The TR * K/256 "units" of a
// tile (8 blocks = 144 or 160 contiguous bytes of one row, 16-byte loads) are
// dealt to the wave's 64 lanes in NP passes (unit v -> lane v % 64, pass
// v / 64).  Each lane turns its units into (p_b, f_b) pairs and stores them in
// the wave's LDS rows; then lane r < TR runs row r's in-order fma chain over
// the row's pairs (2 pairs per 16-byte LDS read).  The chain of a tile thus
// costs ~K/32 dependent fmas of one wave for TR rows together.
//
// The activation (Q8 values + per-block scale and byte sum) is staged once per
// workgroup in LDS, its global loads issued before the first weight loads so
// that waiting for them does not wait for the weights (vector loads complete
// in issue order).  Q8 bytes of a block are stored as 16 bytes paired with the
// low nibbles then 16 paired with the high nibbles: natural order for GGUF
// (elements 0..15, 16..31), even/odd elements for the native interleaved
// nibbles (element 2i = low nibble of byte i).
// ============================================================================

constexpr int kDasPitch = 80;   // LDS bytes per 8-block group of (d, byte sum) pairs (64 + 16 pad)
constexpr int kPairUnit = 80;   // LDS bytes per unit of 8 chain pairs (64 + 16 pad)

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

__device__ __forceinline__ int byte_sum16(uint4 a) {
    constexpr int ones = 0x01010101;
    int s = __builtin_amdgcn_sdot4(static_cast<int>(a.x), ones, 0, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(a.y), ones, s, false);
    s = __builtin_amdgcn_sdot4(static_cast<int>(a.z), ones, s, false);
    return __builtin_amdgcn_sdot4(static_cast<int>(a.w), ones, s, false);
}

template <class F, int SRC, int NP, int RING>
__global__ __launch_bounds__(256) void gemv_q4_persistent(const uint8_t* __restrict__ W, const void* __restrict__ act,
                                                          const float* __restrict__ ad, float* __restrict__ y, int N,
                                                          int nb, int TR, int ntiles) {
    constexpr int kW = 4 * F::kUnit16;  // dwords of one unit
    extern __shared__ __align__(16) uint8_t smem[];
    const int upr = nb >> 3;
    uint8_t* s_aq = smem;
    uint8_t* s_das = smem + upr * kActPitch;
    const int rowpitch = upr * kPairUnit + 16;
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    uint8_t* s_pair = s_das + upr * kDasPitch + wid * TR * rowpitch;
    const int gw = blockIdx.x * 4 + wid, GW = gridDim.x * 4;
    const size_t row_bytes = static_cast<size_t>(nb) * F::kBytes;
    const int units = TR * upr;

    // the lane's unit in each pass (invalid units load row 0's unit 0 and are
    // discarded), fixed for every tile
    int prow[NP], punit[NP];
    bool pval[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int v = lane + 64 * p;
        pval[p] = v < units;
        const int vv = pval[p] ? v : 0;
        prow[p] = vv / upr;
        punit[p] = vv - prow[p] * upr;
    }

    // 1. activation loads (before any weight load)
    constexpr int kAQ = 4;  // 16-byte chunks per thread: nb * 2 <= 1024
    uint4 aqv[kAQ];
    float adv[kAQ];
    constexpr int kAN = 2;  // native blocks per thread: nb <= 512
    uint32_t anv[kAN][9];
    if constexpr (SRC == kSrcQ8) {
        const uint4* aq4 = static_cast<const uint4*>(act);
#pragma unroll
        for (int i = 0; i < kAQ; ++i) {
            const int c = min(t + 256 * i, nb * 2 - 1);
            aqv[i] = aq4[c];
            adv[i] = ad[c >> 1];
        }
    } else if constexpr (SRC == kSrcNative) {
        const uint32_t* xb = static_cast<const uint32_t*>(act);
#pragma unroll
        for (int i = 0; i < kAN; ++i) {
            const int b = min(t + 256 * i, nb - 1);
#pragma unroll
            for (int k = 0; k < 9; ++k) anv[i][k] = xb[9 * b + k];
        }
    }

    // 2. the weight units of the wave's first tile(s)
    auto load = [&](uint32_t (&w)[NP][kW], int tl) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int grow = min(tl * TR + prow[p], N - 1);
            const uint4* src = reinterpret_cast<const uint4*>(W + static_cast<size_t>(grow) * row_bytes +
                                                              static_cast<size_t>(punit[p]) * 8 * F::kBytes);
#pragma unroll
            for (int k = 0; k < F::kUnit16; ++k) {
                const uint4 v = src[k];
                w[p][4 * k] = v.x;
                w[p][4 * k + 1] = v.y;
                w[p][4 * k + 2] = v.z;
                w[p][4 * k + 3] = v.w;
            }
        }
    };
    uint32_t wa[NP][kW];
    uint32_t wb[RING > 1 ? NP : 1][RING > 1 ? kW : 1];
    int tile = gw;
    load(wa, min(tile, ntiles - 1));
    if constexpr (RING > 1) load(wb, min(tile + GW, ntiles - 1));

    // 3. activation into LDS: bytes, then (d, byte sum) per block
    if constexpr (SRC == kSrcQ8) {
#pragma unroll
        for (int i = 0; i < kAQ; ++i) {
            const int c = t + 256 * i;
            const int s = byte_sum16(aqv[i]);
            const int both = s + __builtin_amdgcn_mov_dpp(s, 0xb1, 0xf, 0xf, false);  // lanes c, c^1 of a block
            if (c < nb * 2) {
                const int b = c >> 1;
                *reinterpret_cast<uint4*>(s_aq + (b >> 3) * kActPitch + (b & 7) * 32 + (c & 1) * 16) = aqv[i];
                if ((c & 1) == 0)
                    *reinterpret_cast<int2*>(s_das + (b >> 3) * kDasPitch + (b & 7) * 8) =
                        make_int2(__float_as_int(adv[i]), both);
            }
        }
    } else if constexpr (SRC == kSrcNative) {
#pragma unroll
        for (int i = 0; i < kAN; ++i) {
            const int b = t + 256 * i;
            if (b < nb) {
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
                uint8_t* dst = s_aq + (b >> 3) * kActPitch + (b & 7) * 32;
                *reinterpret_cast<uint4*>(dst) = ev;
                *reinterpret_cast<uint4*>(dst + 16) = od;
                *reinterpret_cast<int2*>(s_das + (b >> 3) * kDasPitch + (b & 7) * 8) =
                    make_int2(static_cast<int>(anv[i][0]), byte_sum16(ev) + byte_sum16(od));
            }
        }
    } else {  // kSrcF32: quantize_q8 of the fp32 input, 8 lanes per block
        const float4* x4 = static_cast<const float4*>(act);
        const int n4 = nb * 8;
        for (int i0 = 0; i0 < n4; i0 += 256) {
            const int i = i0 + t;
            const float4 v = x4[min(i, n4 - 1)];
            float d;
            int s;
            const uint32_t q = quantize_q8_x4(v, d, s);
            if (i < n4) {
                const int b = i >> 3;
                *reinterpret_cast<uint32_t*>(s_aq + (b >> 3) * kActPitch + (b & 7) * 32 + (i & 7) * 4) = q;
                if ((i & 7) == 0)
                    *reinterpret_cast<int2*>(s_das + (b >> 3) * kDasPitch + (b & 7) * 8) =
                        make_int2(__float_as_int(d), s);
            }
        }
    }
    __syncthreads();

    // 4. per tile: pairs into the wave's LDS rows, then one lane per row chains
    auto tile_step = [&](int tl, const uint32_t (&w)[NP][kW]) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if (pval[p]) {
                const uint8_t* ag = s_aq + punit[p] * kActPitch;
                const uint8_t* dg = s_das + punit[p] * kDasPitch;
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
                float4* dst = reinterpret_cast<float4*>(s_pair + prow[p] * rowpitch + punit[p] * kPairUnit);
#pragma unroll
                for (int k = 0; k < 4; ++k) dst[k] = make_float4(pr[2 * k].x, pr[2 * k].y, pr[2 * k + 1].x, pr[2 * k + 1].y);
            }
        }
        if (lane < TR) {
            const uint8_t* src = s_pair + lane * rowpitch;
            float sum = 0.0f;
#pragma unroll 2
            for (int u = 0; u < upr; ++u) {
                const float4* q = reinterpret_cast<const float4*>(src + u * kPairUnit);
                const float4 q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
                sum = fmaf(q0.x, q0.y, sum);
                sum = fmaf(q0.z, q0.w, sum);
                sum = fmaf(q1.x, q1.y, sum);
                sum = fmaf(q1.z, q1.w, sum);
                sum = fmaf(q2.x, q2.y, sum);
                sum = fmaf(q2.z, q2.w, sum);
                sum = fmaf(q3.x, q3.y, sum);
                sum = fmaf(q3.z, q3.w, sum);
            }
            const int grow = tl * TR + lane;
            if (grow < N) y[grow] = sum;
        }
    };

    if constexpr (RING == 1) {
        while (tile < ntiles) {
            tile_step(tile, wa);
            tile += GW;
            if (tile < ntiles) load(wa, tile);
        }
    } else {
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
}

int g_cu_count2 = 0;

int cu_count() {
    if (!g_cu_count2) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            g_cu_count2 = prop.multiProcessorCount;
        if (g_cu_count2 <= 0) g_cu_count2 = 256;
    }
    return g_cu_count2;
}

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e && atoi(e) > 0 ? atoi(e) : dflt;
}

// Tile shape for K/256 units per row: NP passes of 64 lanes, TR rows.
struct TileShape {
    int tr, np;
};
TileShape pick_tile(int upr) {
    static const int force_np = env_int("MVH_GEMV_NP", 0), force_tr = env_int("MVH_GEMV_TR", 0);
    if (force_np >= 1 && force_np <= 4 && force_tr >= 1 && force_tr * upr <= 64 * force_np) return {force_tr, force_np};
    TileShape best{0, 0};
    double best_eff = 0.0;
    for (int np = 1; np <= 4; ++np) {
        const int tr = std::min(16, 64 * np / upr);
        if (tr < 1) continue;
        const double eff = static_cast<double>(tr * upr) / (64.0 * np);
        if (np == 1 && eff >= 0.75) return {tr, 1};
        if (eff > best_eff + 0.05) {
            best_eff = eff;
            best = {tr, np};
        }
    }
    return best;
}

size_t q4_lds_bytes(int upr, int tr) {
    return static_cast<size_t>(upr) * (kActPitch + kDasPitch) + 4u * tr * (upr * kPairUnit + 16);
}

template <class F, int SRC, int NP>
hipError_t launch_q4_np(const uint8_t* W, const void* act, const float* ad, float* y, int N, int nb, int tr,
                        int ntiles, hipStream_t st) {
    static const int wpc = env_int("MVH_GEMV_WPC", 8);  // resident waves per CU (tuning override)
    const int waves = std::min(ntiles, cu_count() * wpc);
    const int grid = (waves + 3) / 4;
    const size_t lds = q4_lds_bytes(nb / 8, tr);
    if (ntiles > grid * 4)
        gemv_q4_persistent<F, SRC, NP, 2><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, tr, ntiles);
    else
        gemv_q4_persistent<F, SRC, NP, 1><<<grid, 256, lds, st>>>(W, act, ad, y, N, nb, tr, ntiles);
    return hipGetLastError();
}

template <class F, int SRC>
hipError_t launch_q4(const uint8_t* W, const void* act, const float* ad, float* y, size_t rows, size_t cols,
                     hipStream_t st) {
    if (!rows) return hipSuccess;
    const int nb = static_cast<int>(cols / 32);
    const TileShape ts = pick_tile(nb / 8);
    const int ntiles = static_cast<int>((rows + ts.tr - 1) / ts.tr);
    const int N = static_cast<int>(rows);
    switch (ts.np) {
        case 1: return launch_q4_np<F, SRC, 1>(W, act, ad, y, N, nb, ts.tr, ntiles, st);
        case 2: return launch_q4_np<F, SRC, 2>(W, act, ad, y, N, nb, ts.tr, ntiles, st);
        case 3: return launch_q4_np<F, SRC, 3>(W, act, ad, y, N, nb, ts.tr, ntiles, st);
        default: return launch_q4_np<F, SRC, 4>(W, act, ad, y, N, nb, ts.tr, ntiles, st);
    }
}

}  // namespace

// K % 256 == 0, K <= 16384 (the activation staging holds nb * 2 <= 1024
// 16-byte chunks, or nb <= 512 native blocks, per workgroup's 256 threads),
// and a tile shape whose LDS fits
bool gemv_q4_0_persistent_ok(size_t cols) {
    if (cols % 256 || cols / 256 > 64) return false;
    const int upr = static_cast<int>(cols / 256);
    const TileShape ts = pick_tile(upr);
    return ts.np >= 1 && q4_lds_bytes(upr, ts.tr) <= 96 * 1024;
}

hipError_t launch_gemv_q4_0_persistent(const uint8_t* W, const float* x, const int8_t* aq, const float* ad, float* y,
                                       size_t rows, size_t cols, hipStream_t st) {
    // GGUF Q4_0 keeps the lane-chained kernel (faster at the 7B decode shapes);
    // MVH_GEMV_V2=1 selects the pass/LDS-chain structure the native format uses
    static const bool v2 = env_int("MVH_GEMV_V2", 0) == 1;
    if (!v2) return launch_gemv_q4_0_persistent_v1(W, x, aq, ad, y, rows, cols, st);
    if (x) return launch_q4<Q4Gguf, kSrcF32>(W, x, nullptr, y, rows, cols, st);
    return launch_q4<Q4Gguf, kSrcQ8>(W, aq, ad, y, rows, cols, st);
}

bool gemv_q4q8_native_ok(size_t cols) { return gemv_q4_0_persistent_ok(cols); }

hipError_t launch_gemv_q4q8_native(const uint8_t* W, const uint8_t* xq, float* y, size_t rows, size_t cols,
                                   hipStream_t st) {
    return launch_q4<Q4Native, kSrcNative>(W, xq, nullptr, y, rows, cols, st);
}

}  // namespace mvh
