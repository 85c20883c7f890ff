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
__global__ __launch_bounds__(kT) void gemv_q4_0_persistent(const uint8_t* __restrict__ W, const float* __restrict__ x,
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

bool gemv_q4_0_persistent_ok(size_t cols) {
    // whole rows inside one wave: at most 64 units of 8 blocks
    return cols % 256 == 0 && cols / 256 <= 64;
}

hipError_t launch_gemv_q4_0_persistent(const uint8_t* W, const float* x, const int8_t* aq, const float* ad, float* y,
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
        gemv_q4_0_persistent<true, T><<<grid, T, lds, st>>>(W, x, nullptr, nullptr, y, static_cast<int>(rows), nb,
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
            gemv_q4_0_persistent<false, 1024><<<grid, 1024, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                       nb, ntiles);
        else if (wg == 512)
            gemv_q4_0_persistent<false, 512><<<grid, 512, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                     nb, ntiles);
        else
            gemv_q4_0_persistent<false, 256><<<grid, 256, lds, st>>>(W, nullptr, aq, ad, y, static_cast<int>(rows),
                                                                     nb, ntiles);
    }
    return hipGetLastError();
}

}  // namespace mvh
