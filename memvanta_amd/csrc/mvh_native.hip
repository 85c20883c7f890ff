// mvh_native.hip -- MemVanta's native (non-GGUF) block formats on the device.
//
// src/quant.cpp / src/quant_kernels.cpp keep their own blocks:
//   BlockQ4_0 {float d; uint8 qs[16]}  20 bytes, element 2i = low nibble of
//             qs[i], element 2i+1 = high nibble (src/quant.cpp:79-81)
//   BlockQ8_0 {float d; int8 qs[32]}   36 bytes
// Here: the two quantizers (quantize_q8_0 / quantize_q4_0, src/quant.cpp:44-85)
// and matvec_q4_q8 (src/quant_kernels.cpp:68-76) for any cols % 32 == 0; the
// K % 256 == 0 shapes of matvec_q4_q8 run on the Q4 x Q8 GEMV of
// mvh_gemv_q4.hip, the fp32-activation dots on the kernels of mvh_gemv.hip.
#include "mvh_kernels.hpp"

namespace mvh {

namespace {

// quantize_q8_0 / quantize_q4_0 (src/quant.cpp:44-85), 8 lanes per block of 32
// (4 consecutive floats each): amax = max|p| (NaN skipped, as std::max keeps
// amax), d = amax/127 (amax/7) or 0 when amax == 0, a block whose d is 0 is
// all zero bytes; else q = clamp(nearbyint(p * (1/d))) with round half to even
// (a non-finite p*(1/d), 1/d having overflowed, converts to INT_MIN: the low
// clamp), Q4 nibbles q + 8 with even elements in the low nibble.
template <bool Q4>
__global__ __launch_bounds__(256) void quantize_native_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                              int nblocks) {
    const int i = blockIdx.x * 256 + threadIdx.x;  // float4 index; 8 per block
    const int b = i >> 3, l = i & 7;
    const bool live = b < nblocks;
    const float4 v = live ? reinterpret_cast<const float4*>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = group_max<8>(m);
    const float d = m == 0.0f ? 0.0f : __fdiv_rn(m, Q4 ? 7.0f : 127.0f);
    const float id = __fdiv_rn(1.0f, d);
    if (!live) return;
    constexpr int kB = Q4 ? 20 : 36;
    uint8_t* o = out + static_cast<size_t>(b) * kB;
    if (l == 0) *reinterpret_cast<float*>(o) = d;
    if constexpr (Q4) {
        auto nib = [&](float p) { return static_cast<uint32_t>(static_cast<int>(q_round_even(p * id, -8.0f, 7.0f)) + 8); };
        uint32_t two = 0;  // bytes 2l, 2l+1: elements 4l..4l+3
        if (d != 0.0f) two = nib(v.x) | (nib(v.y) << 4) | (nib(v.z) << 8) | (nib(v.w) << 12);
        *reinterpret_cast<uint16_t*>(o + 4 + 2 * l) = static_cast<uint16_t>(two);
    } else {
        auto qz = [&](float p) {
            return static_cast<uint32_t>(static_cast<int>(q_round_even(p * id, -127.0f, 127.0f))) & 0xffu;
        };
        uint32_t four = 0;
        if (d != 0.0f) four = qz(v.x) | (qz(v.y) << 8) | (qz(v.z) << 16) | (qz(v.w) << 24);
        *reinterpret_cast<uint32_t*>(o + 4 + 4 * l) = four;
    }
}

// matvec_q4_q8 for any cols % 32 == 0: one wave per row; per chunk of 64
// blocks every lane forms its block's (float(isum) * d_w, d_x) pair in the
// wave's LDS slots, then lane 0 continues the row's in-order chain
// sum = fma(float(isum) * d_w, d_x, sum) (dot_q4_q8, src/quant_kernels.cpp:52-66).
constexpr int kRowWaves = 4;
__global__ __launch_bounds__(64 * kRowWaves) void q4q8_native_rows_kernel(const uint8_t* __restrict__ W,
                                                                          const uint8_t* __restrict__ xq,
                                                                          float* __restrict__ y, int N, int nb) {
    __shared__ float2 s_pair[kRowWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row = blockIdx.x * kRowWaves + w;
    if (row >= N) return;  // whole wave
    const uint8_t* wr = W + static_cast<size_t>(row) * nb * 20;
    float sum = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 64) {
        const int b = b0 + lane;
        if (b < nb) {
            const uint32_t* wb = reinterpret_cast<const uint32_t*>(wr + 20 * b);
            const uint32_t* ab = reinterpret_cast<const uint32_t*>(xq + 36 * static_cast<size_t>(b));
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q[k] = ab[1 + k];
            constexpr uint32_t M = 0x0f0f0f0fu;
            int s = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t qw = wb[1 + k];  // elements 8k..8k+7: even ones in the low nibbles
                const uint32_t ev = __builtin_amdgcn_perm(q[2 * k + 1], q[2 * k], 0x06040200u);
                const uint32_t od = __builtin_amdgcn_perm(q[2 * k + 1], q[2 * k], 0x07050301u);
                s = __builtin_amdgcn_sdot4(static_cast<int>(qw & M), static_cast<int>(ev), s, false);
                s = __builtin_amdgcn_sdot4(static_cast<int>((qw >> 4) & M), static_cast<int>(od), s, false);
                constexpr int ones = 0x01010101;
                s -= 8 * (__builtin_amdgcn_sdot4(static_cast<int>(ev), ones, 0, false) +
                          __builtin_amdgcn_sdot4(static_cast<int>(od), ones, 0, false));
            }
            s_pair[w][lane] = make_float2(static_cast<float>(s) * __uint_as_float(wb[0]), __uint_as_float(ab[0]));
        }
        // the wave's LDS slots: every lane's store visible to lane 0 before it
        // reads them, and lane 0's reads done before the next chunk's stores
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) {
            const int n = min(64, nb - b0);
            for (int j = 0; j < n; ++j) sum = fmaf(s_pair[w][j].x, s_pair[w][j].y, sum);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (lane == 0) y[row] = sum;
}

}  // namespace

hipError_t launch_quantize_native(uint32_t type, const float* x, uint8_t* out, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    const int nblocks = static_cast<int>(n / 32);
    const unsigned grid = static_cast<unsigned>((static_cast<size_t>(nblocks) * 8 + 255) / 256);
    if (type == kNQ4_0)
        quantize_native_kernel<true><<<grid, 256, 0, st>>>(x, out, nblocks);
    else if (type == kNQ8_0)
        quantize_native_kernel<false><<<grid, 256, 0, st>>>(x, out, nblocks);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_matvec_q4q8_native(const uint8_t* W, const uint8_t* xq, float* y, size_t rows, size_t cols,
                                     hipStream_t st) {
    if (!rows) return hipSuccess;
    if (gemv_q4_0_rows16_ok(cols)) return launch_gemv_q4q8_native_rows16(W, xq, y, rows, cols, st);
    const unsigned grid = static_cast<unsigned>((rows + kRowWaves - 1) / kRowWaves);
    q4q8_native_rows_kernel<<<grid, 64 * kRowWaves, 0, st>>>(W, xq, y, static_cast<int>(rows),
                                                             static_cast<int>(cols / 32));
    return hipGetLastError();
}

}  // namespace mvh
