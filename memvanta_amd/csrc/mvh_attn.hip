// mvh_attn.hip -- paged F16 KV cache write and decode attention.
//
// Layout in HBM: per layer a page table of `max_pages` entries; page p holds
// positions [p*page_tokens, (p+1)*page_tokens) as [slot][kv_dim] fp16, K and V
// in separate arrays -- the PagedKVCache layout of src/llama_model.cpp:18-22.
#include "mvh_kernels.hpp"
#define MVH_EXPF_QUAL __device__ __forceinline__
#include "mvh_expf.h"

namespace mvh {
namespace {

// PagedKVCache::write, F16 branch (src/llama_model.cpp:22): every element goes
// through the reference's fp32_to_fp16 routine (f2h_ref).
__global__ __launch_bounds__(256) void kv_write_kernel(uint16_t* const* __restrict__ pt_k,
                                                       uint16_t* const* __restrict__ pt_v,
                                                       const float* __restrict__ k, const float* __restrict__ v,
                                                       int pos, int n_tokens, int kv_dim, int page_tokens) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(n_tokens) * kv_dim) return;
    const int t = static_cast<int>(i / kv_dim), d = static_cast<int>(i % kv_dim);
    const int p = pos + t;
    const size_t off = static_cast<size_t>(p % page_tokens) * kv_dim + d;
    pt_k[p / page_tokens][off] = f2h_ref(k[i]);
    pt_v[p / page_tokens][off] = f2h_ref(v[i]);
}

// Scores of query token b (grid z) and head h (grid x) against positions
// 0..upto, upto = pos + b (dot_key, src/llama_model.cpp:23-39, divided by
// sqrtf(hd) as at :248/:256): lane e of 8 accumulates fma(q[d], k[d]) for
// d = e, e+8, ...; sum = t0+t1+..+t7; a tail beyond a multiple of 8 is
// fma-accumulated into the sum.  pos comes from *d_pos when d_pos != null, so
// the launch (sized for the largest position) can be replayed from a graph.
__global__ __launch_bounds__(64) void attn_scores_kernel(const uint16_t* const* __restrict__ pt_k,
                                                         const float* __restrict__ q, float* __restrict__ scores,
                                                         const int* __restrict__ d_pos, int pos_arg, int n_head,
                                                         int group, int hd, int kv_dim, int page_tokens,
                                                         int score_pitch) {
    extern __shared__ float s_q[];
    const int h = blockIdx.x, b = blockIdx.z;
    const int upto = (d_pos ? *d_pos : pos_arg) + b;
    const int t0 = blockIdx.y * blockDim.x;
    if (t0 > upto) return;  // whole block past the causal limit
    const float* qh = q + (static_cast<size_t>(b) * n_head + h) * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) s_q[i] = qh[i];
    __syncthreads();
    const int t = t0 + threadIdx.x;
    if (t > upto) return;
    const int kh = h / group;
    const uint16_t* krow = pt_k[t / page_tokens] + static_cast<size_t>(t % page_tokens) * kv_dim + kh * hd;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    int c = 0;
    for (; c + 8 <= hd; c += 8) {
        const uint4 kv8 = *reinterpret_cast<const uint4*>(krow + c);
        const uint32_t w[4] = {kv8.x, kv8.y, kv8.z, kv8.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(s_q[c + e], h2f((w[e >> 1] >> (16 * (e & 1))) & 0xffffu), acc[e]);
    }
    float sum = acc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) sum = sum + acc[e];
    for (; c < hd; ++c) sum = fmaf(s_q[c], h2f(krow[c]), sum);
    scores[(static_cast<size_t>(b) * n_head + h) * score_pitch + t] = __fdiv_rn(sum, sqrt_rn(static_cast<float>(hd)));
}

__device__ __forceinline__ float wave_max(float v) {
    v = group_max<32>(v);
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
}

// Softmax and the value sum (src/llama_model.cpp:248,256): mx = max s,
// e = expf(s-mx), den = sum of e in double, inv = float(1/den),
// out[d] = fma(e_t*inv, V_t[d], out[d]) over t in order.  One wave per
// (head, 64-wide slice of head_dim, query token); every output element's
// value chain runs in t order in its own lane, as in the reference.  The
// double `den` is added as a tree instead of in t order.
__global__ __launch_bounds__(64) void attn_softmax_v_kernel(const uint16_t* const* __restrict__ pt_v,
                                                            const float* __restrict__ scores, float* __restrict__ out,
                                                            const int* __restrict__ d_pos, int pos_arg, int n_head,
                                                            int group, int hd, int kv_dim, int page_tokens,
                                                            int score_pitch) {
    extern __shared__ float s_a[];
    const int h = blockIdx.x, b = blockIdx.z;
    const int n = (d_pos ? *d_pos : pos_arg) + b + 1;
    const float* sc = scores + (static_cast<size_t>(b) * n_head + h) * score_pitch;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < n; t += 64) mx = fmaxf(mx, sc[t]);
    mx = wave_max(mx);
    double den = 0.0;
    for (int t = threadIdx.x; t < n; t += 64) {
        const float e = mvh_expf(sc[t] - mx);
        s_a[t] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    const float inv = static_cast<float>(1.0 / den);
    __syncthreads();
    for (int t = threadIdx.x; t < n; t += 64) s_a[t] = s_a[t] * inv;
    __syncthreads();
    const int d = blockIdx.y * 64 + threadIdx.x;
    if (d >= hd) return;
    const int kh = h / group;
    float acc = 0.0f;
    for (int p0 = 0; p0 < n; p0 += page_tokens) {
        const uint16_t* vp = pt_v[p0 / page_tokens] + kh * hd + d;
        const int m = min(page_tokens, n - p0);
        int i = 0;
        for (; i + 8 <= m; i += 8) {
            float vv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) vv[j] = h2f(vp[static_cast<size_t>(i + j) * kv_dim]);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = fmaf(s_a[p0 + i + j], vv[j], acc);
        }
        for (; i < m; ++i) acc = fmaf(s_a[p0 + i], h2f(vp[static_cast<size_t>(i) * kv_dim]), acc);
    }
    out[(static_cast<size_t>(b) * n_head + h) * hd + d] = acc;
}

}  // namespace

hipError_t launch_kv_write(uint16_t* const* pt_k, uint16_t* const* pt_v, const float* k, const float* v, size_t pos,
                           size_t n_tokens, size_t kv_dim, size_t page_tokens, hipStream_t st) {
    const size_t n = n_tokens * kv_dim;
    if (!n) return hipSuccess;
    kv_write_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(
        pt_k, pt_v, k, v, static_cast<int>(pos), static_cast<int>(n_tokens), static_cast<int>(kv_dim),
        static_cast<int>(page_tokens));
    return hipGetLastError();
}

hipError_t launch_attn(const uint16_t* const* pt_k, const uint16_t* const* pt_v, const float* q, float* scores,
                       float* out, const int* d_pos, size_t pos, size_t max_pos, size_t B, size_t n_head,
                       size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st) {
    if (!B) return hipSuccess;
    const int group = static_cast<int>(n_head / n_head_kv);
    const int pitch = static_cast<int>(max_pos);  // scores row pitch >= last position + 1
    const dim3 g1(static_cast<unsigned>(n_head), static_cast<unsigned>((max_pos + 63) / 64), static_cast<unsigned>(B));
    attn_scores_kernel<<<g1, 64, hd * sizeof(float), st>>>(pt_k, q, scores, d_pos, static_cast<int>(pos),
                                                           static_cast<int>(n_head), group, static_cast<int>(hd),
                                                           static_cast<int>(kv_dim), static_cast<int>(page_tokens),
                                                           pitch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 g2(static_cast<unsigned>(n_head), static_cast<unsigned>((hd + 63) / 64), static_cast<unsigned>(B));
    attn_softmax_v_kernel<<<g2, 64, max_pos * sizeof(float), st>>>(pt_v, scores, out, d_pos, static_cast<int>(pos),
                                                                    static_cast<int>(n_head), group,
                                                                    static_cast<int>(hd), static_cast<int>(kv_dim),
                                                                    static_cast<int>(page_tokens), pitch);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const uint16_t* const* pt_k, const uint16_t* const* pt_v, const float* q, float* scores,
                              float* out, size_t pos, size_t n_head, size_t n_head_kv, size_t hd, size_t kv_dim,
                              size_t page_tokens, hipStream_t st) {
    return launch_attn(pt_k, pt_v, q, scores, out, nullptr, pos, pos + 1, 1, n_head, n_head_kv, hd, kv_dim,
                       page_tokens, st);
}

}  // namespace mvh
