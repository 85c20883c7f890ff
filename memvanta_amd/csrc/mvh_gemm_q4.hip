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
// of every other wave (wave-private LDS, no workgroup barriers); the
// activation operands come in the MFMA operand order (q8_op_offset), so one
// block's A operand is one fully used 512-byte load.  Per K-chunk of 8 blocks
// (256 elements):
//   1. the tile's raw Q4_0 bytes (16 rows x 144 B; a row's chunk is 16-byte
//      aligned when K % 256 == 0) come in with 16-byte loads, D chunks ahead;
//   2. they are staged in a wave-private LDS copy and each lane reads back
//      its own MFMA operand bytes and the row's f16 scale;
//   3. per block and token group two MFMAs give the exact block sum (the
//      nibbles as they are, the -8 through the accumulator); each lane then
//      applies the reference's fma to its 4 outputs.
#include "mvh_kernels.hpp"

#include <cstdlib>

namespace mvh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;   // weight rows per wave
constexpr int kChunk = 8;   // blocks per K-chunk
constexpr int kUnit = 144;  // bytes of 8 Q4_0 blocks of one row
constexpr int kWPieces = kRows * kUnit / 16;  // 144 16-byte pieces of raw weights per chunk

// bytes (q - 8) of four nibbles held one per byte (0..15) are not formed:
// the MFMA takes the nibbles as they are (0..15 is a valid int8) and the
// -8 offset comes in through the accumulator, C = A x (-8), an exact int32.
constexpr long kMinus8 = static_cast<long>(0xF8F8F8F8F8F8F8F8ull);

template <int TG>
struct ChunkRegs {
    uint4 w[3];           // raw weight pieces l, l+64, l+128 (16 rows x 144 B)
    long a[TG][kChunk];   // A operands: token group g, block j
    float da[2 * TG];     // activation scales: token l / (4/TG), blocks 2*TG*(l % (4/TG)) ..
};

// One wave per tile of 16 weight rows x 16*TG tokens, independent of every
// other wave.  The tile's K-chunks (8 blocks, 144 bytes per row) stream
// through a ring of D register sets, D chunks ahead of the chunk being
// computed; every load is issued unconditionally (clamped addresses), so the
// compiler's wait counts stay exact and never wait for the ring's later
// chunks.  Per chunk:
//   1. the raw bytes go to a wave-private LDS copy, the scales next to it;
//   2. each lane reads back the 8 quant bytes of its MFMA operand (row li,
//      elements 8h .. 8h+7 of the block: low nibbles of qs[8(h&1) ..] for
//      h < 2, high nibbles for h >= 2) and the row's scale, in registers;
//   3. per block and token group: C = A x (-8), D = A x nibbles + C -- the
//      exact block sum -- then the reference's fma for the lane's 4 outputs.
template <int TG, int D>
__global__ __launch_bounds__(64) void gemm_q4_0_q8_mfma_kernel(const uint8_t* __restrict__ W,
                                                               const int8_t* __restrict__ aq,
                                                               const float* __restrict__ ad,
                                                               float* __restrict__ y, int N, int nb, int B) {
    constexpr int kToks = 16 * TG;
    constexpr int kDaL = 4 / TG;  // lanes per token in the scale load
    __shared__ __align__(16) uint8_t s_raw[kRows * kUnit];
    __shared__ __align__(16) float s_da[kChunk * kToks];  // [block][token]

    const int l = threadIdx.x, li = l & 15, h = l >> 4;
    const int r0 = blockIdx.x * kRows, t0 = blockIdx.y * kToks;
    const size_t row_bytes = static_cast<size_t>(nb) * 18, K = static_cast<size_t>(nb) * 32;
    const int nchunks = nb / kChunk;
    // raw piece p of the chunk: row p / 9, bytes 16 (p % 9); lanes past 143 reload piece 0
    const uint8_t* wp[3];
    int wo[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int p = l + 64 * i, pc = p < kWPieces ? p : 0;
        wp[i] = W + static_cast<size_t>(min(r0 + pc / 9, N - 1)) * row_bytes + (pc % 9) * 16;
        wo[i] = p < kWPieces ? (p / 9) * kUnit + (p % 9) * 16 : -1;
    }
    // A operands in operand order: slab of 16 tokens, then 4 KB per chunk,
    // 512 B per block (lane l's 8 bytes at 8l); a partial group past the last
    // slab reads the last slab again (its outputs are not stored)
    const int8_t* ap[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g)
        ap[g] = aq + static_cast<size_t>(min(blockIdx.y * TG + g, (B - 1) / 16)) * 16 * K + 8 * l;
    const int da_t = l / kDaL, da_b = (l % kDaL) * 2 * TG;
    const float* dp = ad + static_cast<size_t>(min(t0 + da_t, B - 1)) * nb + da_b;

    // the scheduling barriers keep every chunk's loads in ring order: loads
    // reordered across chunks would make the wait for the oldest chunk also
    // wait for the newer ones
    auto fetch = [&](ChunkRegs<TG>& r, int c) {
        __builtin_amdgcn_sched_barrier(0);
        c = min(c, nchunks - 1);
        const size_t wc = static_cast<size_t>(c) * kUnit;
#pragma unroll
        for (int i = 0; i < 3; ++i) r.w[i] = ld_global16(wp[i] + wc);
#pragma unroll
        for (int g = 0; g < TG; ++g)
#pragma unroll
            for (int j = 0; j < kChunk; ++j)
                r.a[g][j] = *reinterpret_cast<const long*>(ap[g] + static_cast<size_t>(c) * 4096 + 512 * j);
        if constexpr (TG == 2) {
            const float4 v = *reinterpret_cast<const float4*>(dp + c * kChunk);
            r.da[0] = v.x; r.da[1] = v.y; r.da[2] = v.z; r.da[3] = v.w;
        } else {
            const float2 v = *reinterpret_cast<const float2*>(dp + c * kChunk);
            r.da[0] = v.x; r.da[1] = v.y;
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    float acc[TG][4];
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;

    // the lane's operand bytes: row li, qs[8(h&1) .. +8) of each block, nibble half h >> 1
    const uint8_t* my_q = s_raw + li * kUnit + 2 + 8 * (h & 1);
    const uint32_t nib_shift = 4u * static_cast<uint32_t>(h >> 1);

    auto compute = [&](const ChunkRegs<TG>& r) {
        // LDS operations of one wave are performed in order, so the reads
        // below see these writes and the next chunk's writes come after them
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            // pieces past the tile's 144 go to piece 0's place with piece 0's bytes
            *reinterpret_cast<uint4*>(s_raw + (wo[i] < 0 ? 0 : wo[i])) = r.w[i];
        }
#pragma unroll
        for (int e = 0; e < 2 * TG; ++e) s_da[(da_b + e) * kToks + da_t] = r.da[e];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            uint32_t q0, q1;
            if ((j & 1) == 0) {  // 18j + 2 + 8(h&1) is 2 mod 4: three dwords, shifted by 2 bytes
                const uint32_t* p = reinterpret_cast<const uint32_t*>(my_q + 18 * j - 2);
                const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
                q0 = align16(w1, w0);
                q1 = align16(w2, w1);
            } else {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(my_q + 18 * j);
                q0 = p[0];
                q1 = p[1];
            }
            const uint32_t n0 = (q0 >> nib_shift) & 0x0f0f0f0fu, n1 = (q1 >> nib_shift) & 0x0f0f0f0fu;
            const long bop = static_cast<long>((static_cast<unsigned long>(n1) << 32) | n0);
            const float dw = h2f(*reinterpret_cast<const uint16_t*>(s_raw + li * kUnit + 18 * j));
#pragma unroll
            for (int g = 0; g < TG; ++g) {
                const v4i c8 = __builtin_amdgcn_mfma_i32_16x16x32_i8(r.a[g][j], kMinus8, v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4i is = __builtin_amdgcn_mfma_i32_16x16x32_i8(r.a[g][j], bop, c8, 0, 0, 0);
                const float4 da = *reinterpret_cast<const float4*>(s_da + j * kToks + 16 * g + 4 * h);
                acc[g][0] = fmaf(dw * da.x, static_cast<float>(is[0]), acc[g][0]);
                acc[g][1] = fmaf(dw * da.y, static_cast<float>(is[1]), acc[g][1]);
                acc[g][2] = fmaf(dw * da.z, static_cast<float>(is[2]), acc[g][2]);
                acc[g][3] = fmaf(dw * da.w, static_cast<float>(is[3]), acc[g][3]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    ChunkRegs<TG> ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) fetch(ring[d], d);
    for (int c = 0; c < nchunks; c += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (c + d < nchunks) compute(ring[d]);
            fetch(ring[d], c + d + D);
        }
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
    const int N = static_cast<int>(rows), nb = static_cast<int>(cols / 32), Bn = static_cast<int>(batch);
    const size_t g16 = (batch + 15) / 16, g32 = (batch + 31) / 32;
    // 16-token tiles while the grid is small (more waves, shorter chains);
    // 32-token tiles share each weight operand when there are waves to spare.
    // The deeper ring pays where few waves each stream a long K.
    // From 512 row tiles (N >= 8192: the fused q|k|v and gate|up) 32-token
    // tiles pay even at M <= 32: the raw-weight staging and unpack is shared
    // by two token groups (pp512 +1.5%); below it the 16-token tiles keep
    // the wave count up.  Tuning override: MVH_GEMM_TG2_ROWTILES.
    static const size_t tg2_min = [] {
        const char* e = getenv("MVH_GEMM_TG2_ROWTILES");
        return e ? static_cast<size_t>(atoll(e)) : static_cast<size_t>(512);
    }();
    if ((batch <= 32 && gx < tg2_min) || gx * g32 <= 1024) {
        if (gx * g16 <= 1024)
            gemm_q4_0_q8_mfma_kernel<1, 4><<<dim3(gx, static_cast<unsigned>(g16)), 64, 0, st>>>(W, aq, ad, y, N, nb, Bn);
        else
            gemm_q4_0_q8_mfma_kernel<1, 2><<<dim3(gx, static_cast<unsigned>(g16)), 64, 0, st>>>(W, aq, ad, y, N, nb, Bn);
    } else {
        gemm_q4_0_q8_mfma_kernel<2, 2><<<dim3(gx, static_cast<unsigned>(g32)), 64, 0, st>>>(W, aq, ad, y, N, nb, Bn);
    }
    return hipGetLastError();
}

}  // namespace mvh
