// mvh_gemm_q4.hip -- batched-prefill Q4_0 x Q8 GEMM on int8 MFMA.
//
// Numerics: tensor_matmul_batch_v06 with MEMVANTA_FORCE_Q8_ACT=1
// (src/gguf_kernels.cpp:265-267): every token's activation row is quantized
// with quantize_q8, and every (row, token) output is dot_q4_q8 (:189):
//   sum = fma(f16(d_w[b]) * d_a[b], float(isum_b), sum)   over blocks b in order,
// with isum_b the exact integer dot of block b.  One v_mfma_i32_16x16x32_i8
// has K = 32 = one block, so it yields isum_b for a 16 x 16 (token x row)
// tile exactly (int8 x int8 -> int32, no rounding); each lane then applies
// the reference's fma for its 4 outputs, block after block, so every output
// is the reference's chain bit for bit.  No split-K, no reassociation.
//
// Data path per K-chunk of 8 blocks (256 elements), workgroup tile = 32 rows
// x 32 tokens, 4 waves = (row half, token half):
//   1. coalesced 16-byte loads of the tile's raw Q4_0 bytes (32 rows x 144 B,
//      rows of a chunk are 16-byte aligned when K % 256 == 0), of the int8
//      activations (32 tokens x 256 B, stored [block][token][32] so operand
//      reads are conflict-free) and of the activation scales;
//   2. the raw blocks are expanded in LDS to int8 (q - 8) in element order
//      plus an f32 weight scale per (block, row) -- one (row, block) per thread;
//   3. every wave runs 8 MFMAs (one per block) with operands read from LDS
//      (8-byte reads) and folds each block's 4 products into its accumulators.
// The loads of chunks c+1 and c+2 are in flight while chunk c is expanded
// and summed.
#include "mvh_kernels.hpp"

namespace mvh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGT = 256;        // threads per workgroup
constexpr int kRows = 32;       // weight rows per workgroup
constexpr int kToks = 32;       // tokens per workgroup
constexpr int kChunk = 8;       // blocks per K-chunk
constexpr int kUnit = 144;      // bytes of 8 Q4_0 blocks of one row
constexpr int kWPieces = kRows * kUnit / 16;   // 288 16-byte pieces of raw weights per chunk
constexpr int kAPieces = kToks * kChunk * 2;   // 512 16-byte pieces of activations per chunk

// bytes (q - 8) of four nibbles held one per byte (0..15): (n + 120) ^ 0x80
__device__ __forceinline__ uint32_t nib_to_s8(uint32_t n) {
    return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

__global__ __launch_bounds__(kGT) void gemm_q4_0_q8_mfma_kernel(const uint8_t* __restrict__ W,
                                                                const int8_t* __restrict__ aq,
                                                                const float* __restrict__ ad,
                                                                float* __restrict__ y, int N, int nb, int B) {
    __shared__ __align__(16) uint8_t s_raw[kRows * kUnit];             // raw Q4_0 blocks [row][8 blocks]
    __shared__ __align__(16) uint8_t s_exp[kChunk * kRows * 32];       // int8 (q-8) [block][row][32]
    __shared__ float s_dw[kChunk * kRows];                             // weight scales [block][row]
    __shared__ __align__(16) uint8_t s_act[kChunk * kToks * 32];       // int8 activations [block][token][32]
    __shared__ __align__(16) float s_da[kChunk * kToks];               // activation scales [block][token]

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r0 = blockIdx.x * kRows, t0 = blockIdx.y * kToks;
    const size_t row_bytes = static_cast<size_t>(nb) * 18, K = static_cast<size_t>(nb) * 32;
    const int nchunks = nb / kChunk;

    // global -> register prefetch of one chunk (two register sets: chunks
    // c+1 and c+2 are in flight while chunk c is expanded and summed)
    struct Regs {
        uint4 w[2], a[2];
        float d;
    };
    auto fetch = [&](Regs& r, int c) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = t + i * kGT;
            if (idx < kWPieces) {
                const int row = min(r0 + idx / 9, N - 1), piece = idx % 9;
                r.w[i] = ld_global16(W + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(c) * kUnit +
                                     piece * 16);
            }
            const int tok = min(t0 + idx / 16, B - 1), piece = idx % 16;
            r.a[i] = ld_global16(aq + static_cast<size_t>(tok) * K + static_cast<size_t>(c) * 256 + piece * 16);
        }
        const int tok = min(t0 + t / kChunk, B - 1);
        r.d = ad[static_cast<size_t>(tok) * nb + c * kChunk + t % kChunk];
    };
    auto store = [&](const Regs& r) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = t + i * kGT;
            if (idx < kWPieces) *reinterpret_cast<uint4*>(s_raw + (idx / 9) * kUnit + (idx % 9) * 16) = r.w[i];
            const int tok = idx >> 4, piece = idx & 15;  // piece p = block p/2, half p%2
            *reinterpret_cast<uint4*>(s_act + ((piece >> 1) * kToks + tok) * 32 + (piece & 1) * 16) = r.a[i];
        }
        s_da[(t % kChunk) * kToks + t / kChunk] = r.d;
    };

    // MFMA lane roles: token group tg, row group rg; operand index i = lane & 15,
    // k group h = lane >> 4 (elements 8h .. 8h+7 of a block)
    const int rg = w >> 1, tg = w & 1, li = lane & 15, h = lane >> 4;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};

    // one chunk, its data already in LDS: expand, then MFMA + chains
    auto compute = [&]() {
        {
            // expand (row, block) = (t % 32, t / 32) to int8 (q - 8)
            const int row = t & 31, j = t >> 5;
            const uint8_t* blk = s_raw + row * kUnit + 18 * j;
            uint32_t q[4], dbits;
            if ((j & 1) == 0) {  // block starts 4-byte aligned: d in bytes 0-1, qs from byte 2
                const uint32_t* p = reinterpret_cast<const uint32_t*>(blk);
                const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
                dbits = w0 & 0xffffu;
                q[0] = align16(w1, w0);
                q[1] = align16(w2, w1);
                q[2] = align16(w3, w2);
                q[3] = align16(w4, w3);
            } else {  // block starts 2 bytes past a dword: d in the high half, qs aligned
                const uint32_t* p = reinterpret_cast<const uint32_t*>(blk - 2);
                dbits = p[0] >> 16;
                q[0] = p[1];
                q[1] = p[2];
                q[2] = p[3];
                q[3] = p[4];
            }
            uint4 lo, hi;  // elements 0..15 (low nibbles), 16..31 (high nibbles)
            lo.x = nib_to_s8(q[0] & 0x0f0f0f0fu);
            lo.y = nib_to_s8(q[1] & 0x0f0f0f0fu);
            lo.z = nib_to_s8(q[2] & 0x0f0f0f0fu);
            lo.w = nib_to_s8(q[3] & 0x0f0f0f0fu);
            hi.x = nib_to_s8((q[0] >> 4) & 0x0f0f0f0fu);
            hi.y = nib_to_s8((q[1] >> 4) & 0x0f0f0f0fu);
            hi.z = nib_to_s8((q[2] >> 4) & 0x0f0f0f0fu);
            hi.w = nib_to_s8((q[3] >> 4) & 0x0f0f0f0fu);
            uint4* dst = reinterpret_cast<uint4*>(s_exp + (j * kRows + row) * 32);
            dst[0] = lo;
            dst[1] = hi;
            s_dw[j * kRows + row] = h2f(dbits);
        }
        __syncthreads();
        const int wrow = 16 * rg + li, atok = 16 * tg + li;
        // all eight block MFMAs first (independent, back to back), then the
        // per-block fma chain in block order on their finished results
        v4i isum[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const long bop = *reinterpret_cast<const long*>(s_exp + (j * kRows + wrow) * 32 + 8 * h);
            const long aop = *reinterpret_cast<const long*>(s_act + (j * kToks + atok) * 32 + 8 * h);
            isum[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, v4i{0, 0, 0, 0}, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const float dw = s_dw[j * kRows + wrow];
            const float4 da = *reinterpret_cast<const float4*>(s_da + j * kToks + 16 * tg + 4 * h);
            acc[0] = fmaf(dw * da.x, static_cast<float>(isum[j][0]), acc[0]);
            acc[1] = fmaf(dw * da.y, static_cast<float>(isum[j][1]), acc[1]);
            acc[2] = fmaf(dw * da.z, static_cast<float>(isum[j][2]), acc[2]);
            acc[3] = fmaf(dw * da.w, static_cast<float>(isum[j][3]), acc[3]);
        }
        __syncthreads();
    };

    Regs ra, rb;
    fetch(ra, 0);
    if (nchunks > 1) fetch(rb, 1);
    for (int c = 0; c < nchunks; c += 2) {
        store(ra);
        __syncthreads();
        if (c + 2 < nchunks) fetch(ra, c + 2);
        compute();
        if (c + 1 >= nchunks) break;
        store(rb);
        __syncthreads();
        if (c + 3 < nchunks) fetch(rb, c + 3);
        compute();
    }

    // lane holds outputs (token 16*tg + 4h + v, row 16*rg + li)
    const int orow = r0 + 16 * rg + li;
    if (orow < N) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tok = t0 + 16 * tg + 4 * h + v;
            if (tok < B) y[static_cast<size_t>(tok) * N + orow] = acc[v];
        }
    }
}

}  // namespace

bool gemm_q4_0_mfma_ok(size_t cols) { return cols >= 256 && cols % 256 == 0; }

hipError_t launch_gemm_q4_0_q8_mfma(const uint8_t* W, const int8_t* aq, const float* ad, float* y, size_t rows,
                                    size_t cols, size_t batch, hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    if (!gemm_q4_0_mfma_ok(cols)) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((rows + kRows - 1) / kRows), static_cast<unsigned>((batch + kToks - 1) / kToks));
    gemm_q4_0_q8_mfma_kernel<<<grid, kGT, 0, st>>>(W, aq, ad, y, static_cast<int>(rows), static_cast<int>(cols / 32),
                                                   static_cast<int>(batch));
    return hipGetLastError();
}

}  // namespace mvh
