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

// The same numerics with a workgroup of 4 waves sharing one LDS copy of each
// K-chunk: 64 weight rows (wave w computes rows 16w .. 16w+15) x 16*TG
// tokens.  The chunk's raw weights (64 rows x 144 B), activation operands (TG
// x 4 KB, operand order) and scales come in with 16-byte loads one chunk
// ahead into registers, go to the idle half of a double-buffered LDS copy
// after the current chunk's compute, and one workgroup barrier per chunk
// hands them over; the staging also copies each row's f16 block scales to a
// [block][row] table.  The weights are the MFMA's A operand, so a lane holds
// rows 4h .. 4h+3 of one token (li) and reads, per block, four row scales
// (8 bytes) and one activation scale per token group; C = (-8) x A for the
// next block is issued before the current block's sums are used.  Against
// the wave-private kernel: no register ring of activation operands (about
// half the VGPRs, twice the resident waves), a quarter of the activation
// traffic and a third of the LDS bytes per block.
template <int TG>
__global__ __launch_bounds__(256) void gemm_q4_0_q8_mfma_wg_kernel(const uint8_t* __restrict__ W,
                                                                   const int8_t* __restrict__ aq,
                                                                   const float* __restrict__ ad,
                                                                   float* __restrict__ y, int N, int nb, int B) {
    constexpr int kToks = 16 * TG;
    constexpr int kWgRows = 64;
    constexpr int kRaw = kWgRows * kUnit;        // 9216 bytes of raw weights per chunk
    constexpr int kPieces = kRaw / 16;           // 576
    constexpr int kWLd = (kPieces + 255) / 256;  // 3 weight loads per thread
    constexpr int kA = TG * 4096;                // activation operand bytes per chunk
    constexpr int kDa = kChunk * kToks;          // activation scales per chunk
    __shared__ __align__(16) uint8_t s_raw[2][kRaw + 16];                // + a spare slot for unused stores
    __shared__ __align__(16) uint16_t s_dw[2][kChunk * kWgRows + 8];      // [block][row] f16 scales + spare
    __shared__ __align__(16) int8_t s_a[2][kA];
    __shared__ __align__(16) float s_da[2][kDa];                          // [block][token]

    const int t = threadIdx.x, l = t & 63, wv = t >> 6, li = l & 15, h = l >> 4;
    const int r0 = blockIdx.x * kWgRows, t0 = blockIdx.y * kToks;
    const size_t row_bytes = static_cast<size_t>(nb) * 18, K = static_cast<size_t>(nb) * 32;
    const int nchunks = nb / kChunk;

    // weight piece p = t + 256 i: row p / 9, unit bytes 16 (p % 9); piece k < 8 of a
    // row holds block k's scale at its byte 2k
    const uint8_t* wsrc[kWLd];
    int wdst[kWLd], sdst[kWLd], sdw[kWLd];
#pragma unroll
    for (int i = 0; i < kWLd; ++i) {
        const int p = t + 256 * i, pc = min(p, kPieces - 1), k = pc % 9;
        wsrc[i] = W + static_cast<size_t>(min(r0 + pc / 9, N - 1)) * row_bytes + k * 16;
        wdst[i] = p < kPieces ? (pc / 9) * kUnit + k * 16 : kRaw;
        sdst[i] = p < kPieces && k < 8 ? k * kWgRows + pc / 9 : kChunk * kWgRows;
        sdw[i] = k & 7;  // the scale's halfword within the piece
    }
    const int8_t* asrc[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g)
        asrc[g] = aq + static_cast<size_t>(min(blockIdx.y * TG + g, (B - 1) / 16)) * 16 * K + 16 * t;
    // scale e = t + 256 i: token e / 8, block e % 8 (TG = 1: threads t, t + 128 load the same scale)
    constexpr int kDL = (kDa + 255) / 256;
    const float* dsrc[kDL];
    int ddst[kDL];
#pragma unroll
    for (int i = 0; i < kDL; ++i) {
        const int e = (t + 256 * i) % kDa, d_tok = e / 8, d_blk = e % 8;
        dsrc[i] = ad + static_cast<size_t>(min(t0 + d_tok, B - 1)) * nb + d_blk;
        ddst[i] = d_blk * kToks + d_tok;
    }

    uint4 wreg[kWLd];
    uint4 areg[TG];
    float dreg[kDL];
    auto load = [&](int c) {
        const size_t wc = static_cast<size_t>(c) * kUnit;
#pragma unroll
        for (int i = 0; i < kWLd; ++i) wreg[i] = ld_global16(wsrc[i] + wc);
#pragma unroll
        for (int g = 0; g < TG; ++g) areg[g] = ld_global16(asrc[g] + static_cast<size_t>(c) * 4096);
#pragma unroll
        for (int i = 0; i < kDL; ++i) dreg[i] = dsrc[i][c * kChunk];
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kWLd; ++i) {
            *reinterpret_cast<uint4*>(&s_raw[buf][wdst[i]]) = wreg[i];
            // halfword sdw[i] of the piece (dword sdw / 2, half sdw % 2)
            const bool upper = (sdw[i] & 4) != 0;
            const uint32_t d0 = upper ? wreg[i].z : wreg[i].x, d1 = upper ? wreg[i].w : wreg[i].y;
            const uint32_t dd = (sdw[i] & 2) ? d1 : d0;
            s_dw[buf][sdst[i]] = static_cast<uint16_t>(dd >> (16 * (sdw[i] & 1)));
        }
#pragma unroll
        for (int g = 0; g < TG; ++g) *reinterpret_cast<uint4*>(&s_a[buf][g * 4096 + 16 * t]) = areg[g];
#pragma unroll
        for (int i = 0; i < kDL; ++i) s_da[buf][ddst[i]] = dreg[i];
    };

    float acc[TG][4];
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;
    // the lane's weight operand bytes: row 16 wv + li, qs[8(h&1) .. +8) of each block, nibble half h >> 1
    const int my_row = (16 * wv + li) * kUnit;
    const uint32_t nib_shift = 4u * static_cast<uint32_t>(h >> 1);

    load(0);
    store(0);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        load(min(c + 1, nchunks - 1));  // unconditional: the last chunk reloads itself
        const uint8_t* my_q = &s_raw[buf][my_row + 2 + 8 * (h & 1)];
        long a_cur[TG];
        v4i c8_cur[TG];
#pragma unroll
        for (int g = 0; g < TG; ++g) {
            a_cur[g] = *reinterpret_cast<const long*>(&s_a[buf][g * 4096 + 8 * l]);
            c8_cur[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(kMinus8, a_cur[g], v4i{0, 0, 0, 0}, 0, 0, 0);
        }
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
            const long wop = static_cast<long>((static_cast<unsigned long>(n1) << 32) | n0);
            // f16 scales of rows 16 wv + 4h .. +3
            const uint2 dwb = *reinterpret_cast<const uint2*>(&s_dw[buf][j * kWgRows + 16 * wv + 4 * h]);
            const float dw[4] = {h2f(dwb.x & 0xffffu), h2f(dwb.x >> 16), h2f(dwb.y & 0xffffu), h2f(dwb.y >> 16)};
            long a_nxt[TG];
            v4i c8_nxt[TG];
#pragma unroll
            for (int g = 0; g < TG; ++g) {
                const v4i is = __builtin_amdgcn_mfma_i32_16x16x32_i8(wop, a_cur[g], c8_cur[g], 0, 0, 0);
                if (j + 1 < kChunk) {
                    a_nxt[g] = *reinterpret_cast<const long*>(&s_a[buf][g * 4096 + (j + 1) * 512 + 8 * l]);
                    c8_nxt[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(kMinus8, a_nxt[g], v4i{0, 0, 0, 0}, 0, 0, 0);
                }
                const float da = s_da[buf][j * kToks + 16 * g + li];
                acc[g][0] = fmaf(dw[0] * da, static_cast<float>(is[0]), acc[g][0]);
                acc[g][1] = fmaf(dw[1] * da, static_cast<float>(is[1]), acc[g][1]);
                acc[g][2] = fmaf(dw[2] * da, static_cast<float>(is[2]), acc[g][2]);
                acc[g][3] = fmaf(dw[3] * da, static_cast<float>(is[3]), acc[g][3]);
            }
            if (j + 1 < kChunk) {
#pragma unroll
                for (int g = 0; g < TG; ++g) {
                    a_cur[g] = a_nxt[g];
                    c8_cur[g] = c8_nxt[g];
                }
            }
        }
        store(buf ^ 1);  // the idle buffer was last read in chunk c - 1, before the barrier that ended it
        __syncthreads();
    }

    // lane holds (row 16 wv + 4h + v, token 16g + li) of each token group g
#pragma unroll
    for (int g = 0; g < TG; ++g) {
        const int tk = t0 + 16 * g + li;
        if (tk < B) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int orow = r0 + 16 * wv + 4 * h + v;
                if (orow < N) y[static_cast<size_t>(tk) * N + orow] = acc[g][v];
            }
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
    // From 256 tokens the workgroup kernel (64 rows x 32 tokens per workgroup)
    // is a few percent faster (M = 512: 68-69 against 70-71 us at 4096^2,
    // 160 against 165-172 us at the other two shapes); at M = 128 it is slower.
    // Tuning override: MVH_GEMM_WG=0 never, 1 at every batch size.
    static const int wg_mode = [] {
        const char* e = getenv("MVH_GEMM_WG");
        return e ? atoi(e) : -1;
    }();
    const size_t gw = (rows + 63) / 64;
    if (wg_mode == 1 || (wg_mode != 0 && batch >= 256)) {
        gemm_q4_0_q8_mfma_wg_kernel<2><<<dim3(static_cast<unsigned>(gw), static_cast<unsigned>(g32)), 256, 0, st>>>(
            W, aq, ad, y, N, nb, Bn);
        return hipGetLastError();
    }
    // (17..32 tokens: the row-tile count alone decides -- the fused q|k|v's
    // 768 row tiles on 32-token tiles, pp512 11.84 -> 11.95-12.03 K tok/s;
    // up to 16 tokens a 32-token tile would be half empty)
    if (batch <= 32 ? batch <= 16 || gx < tg2_min : gx * g32 <= 1024) {
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
