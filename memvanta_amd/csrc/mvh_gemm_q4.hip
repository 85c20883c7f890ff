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
// Work split: one wave per tile of 16 weight rows x 16*TG tokens, independent
// of every other wave (wave-private LDS, no workgroup barriers).  Per K-chunk
// of 8 blocks (256 elements):
//   1. the tile's raw Q4_0 bytes (16 rows x 144 B; a row's chunk is 16-byte
//      aligned when K % 256 == 0) come in with 16-byte loads, the int8
//      activation operands straight into registers (8 bytes per lane and
//      block), the activation scales as one 16-byte load per lane -- the
//      next chunk's loads are in flight while this chunk is computed;
//   2. the raw blocks are expanded in LDS to int8 (q - 8) in element order
//      plus an f32 weight scale per (block, row), two (row, block) per lane;
//   3. per block TG MFMAs (token groups) share the expanded weight operand;
//      each lane then applies the reference's fma to its 4 outputs per group.
#include "mvh_kernels.hpp"

namespace mvh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;   // weight rows per wave
constexpr int kChunk = 8;   // blocks per K-chunk
constexpr int kUnit = 144;  // bytes of 8 Q4_0 blocks of one row
constexpr int kWPieces = kRows * kUnit / 16;  // 144 16-byte pieces of raw weights per chunk

// bytes (q - 8) of four nibbles held one per byte (0..15): (n + 120) ^ 0x80
__device__ __forceinline__ uint32_t nib_to_s8(uint32_t n) {
    return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

template <int TG>
struct ChunkRegs {
    uint4 w[3];           // raw weight pieces l, l+64, l+128
    long a[TG][kChunk];   // A operands: token group g, block j
    float4 d;             // activation scales of 16*TG tokens x 8 blocks
};

// TG token groups of 16 per wave: TG = 1 gives twice the waves (small
// batches, where the per-wave chain length bounds the time), TG = 2 shares
// each expanded weight operand between two MFMAs.
template <int TG>
__global__ __launch_bounds__(64) void gemm_q4_0_q8_mfma_kernel(const uint8_t* __restrict__ W,
                                                               const int8_t* __restrict__ aq,
                                                               const float* __restrict__ ad,
                                                               float* __restrict__ y, int N, int nb, int B) {
    constexpr int kToks = 16 * TG;
    __shared__ __align__(16) uint8_t s_raw[kRows * kUnit];        // raw blocks [row][8 blocks]
    __shared__ __align__(16) uint8_t s_exp[kChunk * kRows * 32];  // int8 (q-8) [block][row][32]
    __shared__ float s_dw[kChunk * kRows];                        // weight scales [block][row]
    __shared__ __align__(16) float s_da[kChunk * kToks];          // activation scales [block][token]

    const int l = threadIdx.x, li = l & 15, h = l >> 4;
    const int r0 = blockIdx.x * kRows, t0 = blockIdx.y * kToks;
    const size_t row_bytes = static_cast<size_t>(nb) * 18, K = static_cast<size_t>(nb) * 32;
    const int nchunks = nb / kChunk;

    auto fetch = [&](ChunkRegs<TG>& r, int c) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int p = l + 64 * i;
            if (p < kWPieces) {
                const int row = min(r0 + p / 9, N - 1);
                r.w[i] = ld_global16(W + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(c) * kUnit +
                                     (p % 9) * 16);
            }
        }
#pragma unroll
        for (int g = 0; g < TG; ++g) {
            const int tok = min(t0 + 16 * g + li, B - 1);
            const int8_t* base = aq + static_cast<size_t>(tok) * K + static_cast<size_t>(c) * 256 + 8 * h;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) r.a[g][j] = *reinterpret_cast<const long*>(base + 32 * j);
        }
        // lane -> (token l/2, blocks 4*(l%2) .. +3); TG = 1 uses lanes 0..31
        const int tok = min(t0 + min(l >> 1, kToks - 1), B - 1);
        r.d = *reinterpret_cast<const float4*>(ad + static_cast<size_t>(tok) * nb + c * kChunk + 4 * (l & 1));
    };

    float acc[TG][4];
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;

    auto compute = [&](const ChunkRegs<TG>& r) {
        // stage the raw bytes and the scales (LDS operations of one wave are
        // performed in order, so the reads below see these writes)
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int p = l + 64 * i;
            if (p < kWPieces) *reinterpret_cast<uint4*>(s_raw + (p / 9) * kUnit + (p % 9) * 16) = r.w[i];
        }
        if ((l >> 1) < kToks) {
            const int tok = l >> 1, j0 = 4 * (l & 1);
            s_da[(j0 + 0) * kToks + tok] = r.d.x;
            s_da[(j0 + 1) * kToks + tok] = r.d.y;
            s_da[(j0 + 2) * kToks + tok] = r.d.z;
            s_da[(j0 + 3) * kToks + tok] = r.d.w;
        }
        __builtin_amdgcn_wave_barrier();
        // expand (row li, blocks h and h+4) to int8 (q - 8)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = h + 4 * jj;
            const uint8_t* blk = s_raw + li * kUnit + 18 * j;
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
            uint4* dst = reinterpret_cast<uint4*>(s_exp + (j * kRows + li) * 32);
            dst[0] = lo;
            dst[1] = hi;
            s_dw[j * kRows + li] = h2f(dbits);
        }
        __builtin_amdgcn_wave_barrier();
        // four blocks at a time: their MFMAs back to back, then the chains
#pragma unroll
        for (int half = 0; half < kChunk; half += 4) {
            v4i is[TG][4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int j = half + jj;
                const long bop = *reinterpret_cast<const long*>(s_exp + (j * kRows + li) * 32 + 8 * h);
#pragma unroll
                for (int g = 0; g < TG; ++g)
                    is[g][jj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(r.a[g][j], bop, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int j = half + jj;
                const float dw = s_dw[j * kRows + li];
#pragma unroll
                for (int g = 0; g < TG; ++g) {
                    const float4 da = *reinterpret_cast<const float4*>(s_da + j * kToks + 16 * g + 4 * h);
                    acc[g][0] = fmaf(dw * da.x, static_cast<float>(is[g][jj][0]), acc[g][0]);
                    acc[g][1] = fmaf(dw * da.y, static_cast<float>(is[g][jj][1]), acc[g][1]);
                    acc[g][2] = fmaf(dw * da.z, static_cast<float>(is[g][jj][2]), acc[g][2]);
                    acc[g][3] = fmaf(dw * da.w, static_cast<float>(is[g][jj][3]), acc[g][3]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    ChunkRegs<TG> ra, rb;
    fetch(ra, 0);
    for (int c = 0; c < nchunks; c += 2) {
        if (c + 1 < nchunks) fetch(rb, c + 1);
        compute(ra);
        if (c + 1 >= nchunks) break;
        if (c + 2 < nchunks) fetch(ra, c + 2);
        compute(rb);
    }

    // lane holds (token 16g + 4h + v, row li) of each token group g
    const int orow = r0 + li;
    if (orow < N) {
#pragma unroll
        for (int g = 0; g < TG; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tk = t0 + 16 * g + 4 * h + v;
                if (tk < B) y[static_cast<size_t>(tk) * N + orow] = acc[g][v];
            }
    }
}

}  // namespace

bool gemm_q4_0_mfma_ok(size_t cols) { return cols >= 256 && cols % 256 == 0; }

hipError_t launch_gemm_q4_0_q8_mfma(const uint8_t* W, const int8_t* aq, const float* ad, float* y, size_t rows,
                                    size_t cols, size_t batch, hipStream_t st) {
    if (!rows || !batch) return hipSuccess;
    if (!gemm_q4_0_mfma_ok(cols)) return hipErrorInvalidValue;
    const unsigned gx = static_cast<unsigned>((rows + kRows - 1) / kRows);
    if (batch <= 32) {  // short chains per wave matter more than operand sharing
        gemm_q4_0_q8_mfma_kernel<1><<<dim3(gx, static_cast<unsigned>((batch + 15) / 16)), 64, 0, st>>>(
            W, aq, ad, y, static_cast<int>(rows), static_cast<int>(cols / 32), static_cast<int>(batch));
    } else {
        gemm_q4_0_q8_mfma_kernel<2><<<dim3(gx, static_cast<unsigned>((batch + 31) / 32)), 64, 0, st>>>(
            W, aq, ad, y, static_cast<int>(rows), static_cast<int>(cols / 32), static_cast<int>(batch));
    }
    return hipGetLastError();
}

}  // namespace mvh
