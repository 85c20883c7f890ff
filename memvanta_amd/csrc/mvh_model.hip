// mvh_model.hip -- the element-wise pieces of LlamaModel's decode and
// prefill steps (src/llama_model.cpp:237-259), kept on the device so a whole
// step runs without host round trips.  Positions and token ids can be read
// from device memory, so one captured HIP graph serves every decode step.
#include "mvh_kernels.hpp"
#define MVH_EXPF_QUAL __device__ __forceinline__
#define MVH_EXPF_TABLE static __constant__ const
#include "mvh_expf.h"

namespace mvh {

// One element of row `row` of a GGUF tensor, dequantized the way
// tensor_read_row_f32 does it (src/gguf_kernels.cpp:226).
__device__ __forceinline__ float dequant_elem(uint32_t type, const uint8_t* W, int cols, size_t row, int i) {
    if (type == kF32) return reinterpret_cast<const float*>(W)[row * cols + i];
    if (type == kF16) return h2f(reinterpret_cast<const uint16_t*>(W)[row * cols + i]);
    if (type == kQ4_0) {
        const uint8_t* b = W + (row * (cols / 32) + i / 32) * 18;
        const int e = i & 31;
        const uint32_t byte = b[2 + (e & 15)];
        const int q = static_cast<int>(e < 16 ? (byte & 15u) : (byte >> 4)) - 8;
        return h2f(b[0] | (static_cast<uint32_t>(b[1]) << 8)) * static_cast<float>(q);
    }
    if (type == kQ8_0) {
        const uint8_t* b = W + (row * (cols / 32) + i / 32) * 34;
        return h2f(b[0] | (static_cast<uint32_t>(b[1]) << 8)) * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31)]));
    }
    const uint8_t* b = W + (row * (cols / 256) + i / 256) * 210;  // Q6_K
    const int e = i & 255;
    const int row32 = e / 32, j = e % 32, group = row32 / 4, local = row32 % 4;
    const int lo = (b[group * 64 + (local % 2) * 32 + j] >> (local < 2 ? 0 : 4)) & 0x0f;
    const int hi = (b[128 + group * 32 + j] >> (2 * local)) & 0x03;
    const float d = h2f(b[208] | (static_cast<uint32_t>(b[209]) << 8));
    return (d * static_cast<float>(static_cast<int8_t>(b[192 + e / 16]))) * static_cast<float>((lo | (hi << 4)) - 32);
}

namespace {

// Embedding rows of B tokens (token ids in device memory).
__global__ __launch_bounds__(256) void embed_kernel(uint32_t type, int cols, int half, const uint8_t* __restrict__ W,
                                                    const int* __restrict__ tokens, float* __restrict__ out,
                                                    const int* __restrict__ d_pos, const float* __restrict__ cos_t,
                                                    const float* __restrict__ sin_t, float* __restrict__ rope_cur) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= cols) return;
    out[static_cast<size_t>(blockIdx.y) * cols + i] = dequant_elem(type, W, cols, static_cast<size_t>(tokens[blockIdx.y]), i);
    if (rope_cur && i < half) {  // the decode attention's RoPE row, read without waiting for the position
        const size_t p = static_cast<size_t>(*d_pos);
        rope_cur[i] = cos_t[p * half + i];
        rope_cur[half + i] = sin_t[p * half + i];
    }
}

// x += add (when add != null), then LlamaModel::rmsnorm (src/llama_model.cpp:237)
// of each row and optionally its Q8 activation: rmsnorm_row, one workgroup
// per row; workgroups past the rows warm the next GEMV's weights (l2_warm).
constexpr int kNormT = 1024;
constexpr int kNormV = 4;  // float4s per thread: D <= 16384, all held in registers
__global__ __launch_bounds__(kNormT) void rmsnorm_kernel(int rows, int D, float eps, bool q_op, float* __restrict__ x,
                                                         const float* __restrict__ add, const float* __restrict__ w,
                                                         float* __restrict__ n, int8_t* __restrict__ q,
                                                         float* __restrict__ qd, L2Warm warm) {
    __shared__ double red[kNormT / 64];
    const size_t row = blockIdx.x;
    if (static_cast<int>(blockIdx.x) >= rows) {
        l2_warm<kNormT>(warm, static_cast<int>(blockIdx.x), rows, static_cast<int>(gridDim.x) - rows);
        return;
    }
    rmsnorm_row<kNormT, kNormV>(x + row * D, add ? add + row * D : nullptr, w, n + row * D, q, qd, row, D, eps, q_op,
                                red);
}

// RoPE (LlamaModel::rope_ptr, src/llama_model.cpp:238; half-split pairs,
// GCC's contraction fma(x0,c,-(x1*s)) / fma(x0,s,x1*c)) on q and k of B
// tokens at positions pos..pos+B-1, in place, then (pt_k != null)
// PagedKVCache::write of k and v: F16 pages through the reference's
// fp32_to_fp16 (:22), F32 pages as they are (kv_f32).
// One thread per (token, head, i).
__global__ __launch_bounds__(256) void rope_kv_kernel(float* __restrict__ q, int q_pitch, float* __restrict__ k,
                                                      const float* __restrict__ v, int kv_pitch,
                                                      const float* __restrict__ cos_t,
                                                      const float* __restrict__ sin_t, const int* __restrict__ d_pos,
                                                      int pos0, int B, int n_head, int n_kv, int hd,
                                                      void* const* __restrict__ pt_k,
                                                      void* const* __restrict__ pt_v, int page_tokens,
                                                      int kv_f32) {
    const int half = hd / 2, heads = n_head + n_kv;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= B * heads * half) return;
    const int b = idx / (heads * half), rem = idx - b * heads * half, h = rem / half, i = rem - h * half;
    const int pos = (d_pos ? *d_pos : pos0) + b;
    const float c = cos_t[static_cast<size_t>(pos) * half + i], s = sin_t[static_cast<size_t>(pos) * half + i];
    const int KV = n_kv * hd;
    float* z = h < n_head ? q + static_cast<size_t>(b) * q_pitch + h * hd
                          : k + static_cast<size_t>(b) * kv_pitch + (h - n_head) * hd;
    const float x0 = z[i], x1 = z[i + half];
    const float r0 = fmaf(x0, c, -(x1 * s)), r1 = fmaf(x0, s, x1 * c);
    z[i] = r0;
    z[i + half] = r1;
    if (h >= n_head && pt_k) {
        const int kh = h - n_head;
        const size_t off = static_cast<size_t>(pos % page_tokens) * KV + kh * hd;
        const float* vv = v + static_cast<size_t>(b) * kv_pitch + kh * hd;
        if (kv_f32) {  // F32 pages: the row as it is (PagedKVCache::write's memcpy)
            float* kp = static_cast<float*>(pt_k[pos / page_tokens]) + off;
            float* vp = static_cast<float*>(pt_v[pos / page_tokens]) + off;
            kp[i] = r0;
            kp[i + half] = r1;
            vp[i] = vv[i];
            vp[i + half] = vv[i + half];
        } else {
            uint16_t* kp = static_cast<uint16_t*>(pt_k[pos / page_tokens]) + off;
            uint16_t* vp = static_cast<uint16_t*>(pt_v[pos / page_tokens]) + off;
            kp[i] = f2h_ref(r0);
            kp[i + half] = f2h_ref(r1);
            vp[i] = f2h_ref(vv[i]);
            vp[i + half] = f2h_ref(vv[i + half]);
        }
    }
}

// SwiGLU (src/llama_model.cpp:249,257): ff = (g/(1+expf(-g)))*u, with expf as
// the C library computes it; optionally the Q8 activation of ff (row-major,
// or in the prefill GEMM's operand order when q_op).  Row b of g/u at
// g + b*pitch, u + b*pitch; ff and q rows are F long.  F % 32 == 0
// (F % 256 == 0 with q_op).  One row (gridDim.y == 1): workgroups from
// nblk on warm the next GEMV's weights (l2_warm).
__global__ __launch_bounds__(256) void swiglu_kernel(int nblk, int pitch, const float* __restrict__ g,
                                                     const float* __restrict__ u, float* __restrict__ ff,
                                                     int8_t* __restrict__ q, float* __restrict__ qd, int F, bool q_op,
                                                     L2Warm warm) {
    __shared__ uint64_t s_tab[32];
    if (static_cast<int>(blockIdx.x) >= nblk) {
        l2_warm<256>(warm, static_cast<int>(blockIdx.x), nblk, static_cast<int>(gridDim.x) - nblk);
        return;
    }
    const int i = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    const int n4 = F / 4;
    const bool live = i < n4;  // n4 % 8 == 0: 8-lane groups are whole blocks
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a, o = a;
    if (live) {
        a = reinterpret_cast<const float4*>(g + static_cast<size_t>(b) * pitch)[i];
        c = reinterpret_cast<const float4*>(u + static_cast<size_t>(b) * pitch)[i];
    }
    const uint64_t tab_v = mvh_expf_tab(threadIdx.x);
    if (threadIdx.x < 32) s_tab[threadIdx.x] = tab_v;
    __syncthreads();
    if (live) {
        auto f = [&](float z, float up) { return __fdiv_rn(z, 1.0f + mvh_expf_tabbed(-z, s_tab)) * up; };
        o = make_float4(f(a.x, c.x), f(a.y, c.y), f(a.z, c.z), f(a.w, c.w));
        reinterpret_cast<float4*>(ff + static_cast<size_t>(b) * F)[i] = o;
    }
    if (q) {
        float d;
        int s;
        const uint32_t packed = quantize_q8_x4(o, d, s);
        if (live) {
            if (q_op)
                *reinterpret_cast<uint32_t*>(q + q8_op_offset(b, 4 * static_cast<size_t>(i), F)) = packed;
            else
                reinterpret_cast<uint32_t*>(q + static_cast<size_t>(b) * F)[i] = packed;
            if ((i & 7) == 0) qd[static_cast<size_t>(b) * (F / 32) + (i >> 3)] = d;
        }
    }
}

// Greedy sampling (Sampler, src/llama_model.cpp:60: first index of the max)
// of each of B rows; writes token ids and, when d_pos != null, records the
// token in hist[*d_pos] (if hist) and advances *d_pos.
constexpr int kArgT = 1024;
__global__ __launch_bounds__(kArgT) void argmax_kernel(const float* __restrict__ logits, int V, int* __restrict__ out,
                                                       int* __restrict__ d_pos, int* __restrict__ hist) {
    __shared__ float sv[kArgT / 64];
    __shared__ int si[kArgT / 64];
    const float* l = logits + static_cast<size_t>(blockIdx.x) * V;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i0 = threadIdx.x; i0 < V; i0 += 8 * kArgT) {  // eight loads in flight per thread
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = i0 + k * kArgT;
            v[k] = i < V ? l[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = i0 + k * kArgT;
            if (i < V && (v[k] > best || bi == 0x7fffffff)) {  // indices increase: strict > keeps the first max
                best = v[k];
                bi = i;
            }
        }
    }
    auto better = [](float v, int i, float bv, int bj) { return v > bv || (v == bv && i < bj); };
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best, m);
        const int oi = __shfl_xor(bi, m);
        if (better(ov, oi, best, bi)) {
            best = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kArgT / 64; ++k)
            if (better(sv[k], si[k], best, bi)) {
                best = sv[k];
                bi = si[k];
            }
        out[blockIdx.x] = bi;
        if (d_pos && blockIdx.x == 0) {  // decode loop: record the token at its position, advance
            if (hist) hist[*d_pos] = bi;
            *d_pos += 1;
        }
    }
}

}  // namespace

hipError_t launch_embed(uint32_t type, const uint8_t* W, size_t cols, const int* tokens, size_t B, float* out,
                        hipStream_t st, const int* d_pos, const float* cos_t, const float* sin_t, size_t half,
                        float* rope_cur) {
    if (!B) return hipSuccess;
    if (rope_cur && (B != 1 || !d_pos || !cos_t || !sin_t || half > cols)) return hipErrorInvalidValue;
    embed_kernel<<<dim3(static_cast<unsigned>((cols + 255) / 256), static_cast<unsigned>(B)), 256, 0, st>>>(
        type, static_cast<int>(cols), static_cast<int>(half), W, tokens, out, d_pos, cos_t, sin_t, rope_cur);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(float* x, const float* add, const float* w, float* n, int8_t* q, float* qd, size_t B,
                          size_t D, float eps, hipStream_t st, bool q_op, const L2Warm& warm) {
    if (!B) return hipSuccess;
    if (D % 32 || D > static_cast<size_t>(4 * kNormT * kNormV) || (q_op && D % 256)) return hipErrorInvalidValue;
    const unsigned extra = warm.c1 > warm.c0 && B < kWarmWgs ? kWarmWgs - static_cast<unsigned>(B) : 0u;
    rmsnorm_kernel<<<static_cast<unsigned>(B) + extra, kNormT, 0, st>>>(static_cast<int>(B), static_cast<int>(D), eps,
                                                                        q && q_op, x, add, w, n, q, qd, warm);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* q, size_t q_pitch, float* k, const float* v, size_t kv_pitch, const float* cos_t,
                          const float* sin_t, const int* d_pos, size_t pos0, size_t B, size_t n_head, size_t n_kv,
                          size_t hd, int kv_type, void* const* pt_k, void* const* pt_v, size_t page_tokens,
                          hipStream_t st) {
    const size_t n = B * (n_head + n_kv) * (hd / 2);
    if (!n) return hipSuccess;
    rope_kv_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(
        q, static_cast<int>(q_pitch), k, v, static_cast<int>(kv_pitch), cos_t, sin_t, d_pos, static_cast<int>(pos0),
        static_cast<int>(B), static_cast<int>(n_head), static_cast<int>(n_kv), static_cast<int>(hd), pt_k, pt_v,
        static_cast<int>(page_tokens), kv_type == kKvF32 ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, size_t pitch, float* ff, int8_t* q, float* qd, size_t B,
                         size_t F, hipStream_t st, bool q_op, const L2Warm& warm) {
    const size_t n4 = F / 4;
    if (!n4 || !B) return hipSuccess;
    if (q_op && F % 256) return hipErrorInvalidValue;
    const unsigned nblk = static_cast<unsigned>((n4 + 255) / 256);
    const unsigned extra = warm.c1 > warm.c0 && B == 1 && nblk < kWarmWgs ? kWarmWgs - nblk : 0u;
    swiglu_kernel<<<dim3(nblk + extra, static_cast<unsigned>(B)), 256, 0, st>>>(
        static_cast<int>(nblk), static_cast<int>(pitch), g, u, ff, q, qd, static_cast<int>(F), q && q_op, warm);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, size_t V, size_t B, int* out, int* d_pos, int* hist, hipStream_t st) {
    if (!B) return hipSuccess;
    argmax_kernel<<<static_cast<unsigned>(B), kArgT, 0, st>>>(logits, static_cast<int>(V), out, d_pos, hist);
    return hipGetLastError();
}

}  // namespace mvh
