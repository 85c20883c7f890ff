// mvh_attn.hip -- paged KV cache write and attention (decode and prefill).
//
// Layout in HBM: per layer a page table of `max_pages` entries; page p holds
// positions [p*page_tokens, (p+1)*page_tokens) as [slot][kv_dim] elements of
// the cache type (F32, F16, or Q8 with one float scale per slot after the
// elements: kv_page_bytes), K and V in separate pages -- the PagedKVCache
// layout of src/llama_model.cpp:18-22.
#include "mvh_kernels.hpp"
#define MVH_EXPF_QUAL __device__ __forceinline__
#define MVH_EXPF_TABLE static __constant__ const
#include "mvh_expf.h"

namespace mvh {
namespace {

// PagedKVCache::write, F32 and F16 branches (src/llama_model.cpp:22): F32
// copies, F16 sends every element through the reference's fp32_to_fp16
// routine (f2h_ref).  Token t's k/v row at k + t*pitch, v + t*pitch; its
// position is pos + t, pos = *d_pos when d_pos != null.
template <int KT>
__global__ __launch_bounds__(256) void kv_write_kernel(void* const* __restrict__ pt_k, void* const* __restrict__ pt_v,
                                                       const float* __restrict__ k, const float* __restrict__ v,
                                                       int pitch, const int* __restrict__ d_pos, int pos_arg,
                                                       int n_tokens, int kv_dim, int page_tokens) {
    typedef typename KvElem<KT>::T E;
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(n_tokens) * kv_dim) return;
    const int t = static_cast<int>(i / kv_dim), d = static_cast<int>(i % kv_dim);
    const int p = (d_pos ? *d_pos : pos_arg) + t;
    const size_t off = static_cast<size_t>(p % page_tokens) * kv_dim + d;
    const float kx = k[static_cast<size_t>(t) * pitch + d], vx = v[static_cast<size_t>(t) * pitch + d];
    E* kp = static_cast<E*>(pt_k[p / page_tokens]);
    E* vp = static_cast<E*>(pt_v[p / page_tokens]);
    if constexpr (KT == kKvF16) {
        kp[off] = f2h_ref(kx);
        vp[off] = f2h_ref(vx);
    } else {
        kp[off] = kx;
        vp[off] = vx;
    }
}

// PagedKVCache::write, Q8 branch (src/llama_model.cpp:22): one scale per
// token and row (K, V), s = max|x|/127 over the whole kv_dim row (1 when the
// row is all zero; fmaxf skips a NaN as std::max(m, NaN) keeps m), then
// q = clamp(round_half_away(x / s), -127, 127) with an IEEE division (a
// non-finite quotient -- s underflowed to 0 -- clamps to -127, as lround's
// x86 result does).  Workgroup = (token,
// K or V); each thread holds up to kKWV groups of 4 elements in registers, so
// the row is read once (kv_dim <= 4 * kKW * kKWV).
constexpr int kKW = 1024;
constexpr int kKWV = 4;
__global__ __launch_bounds__(kKW) void kv_write_q8_kernel(void* const* __restrict__ pt_k,
                                                          void* const* __restrict__ pt_v,
                                                          const float* __restrict__ k, const float* __restrict__ v,
                                                          int pitch, const int* __restrict__ d_pos, int pos_arg,
                                                          int kv_dim, int page_tokens) {
    __shared__ float red[kKW / 64];
    const int t = blockIdx.x, which = blockIdx.y;
    const float* x = (which ? v : k) + static_cast<size_t>(t) * pitch;
    float4 xv[kKWV];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kKWV; ++j) {
        const int d = 4 * (j * kKW + static_cast<int>(threadIdx.x));
        xv[j] = d < kv_dim ? *reinterpret_cast<const float4*>(x + d) : make_float4(0.f, 0.f, 0.f, 0.f);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[j].x), fabsf(xv[j].y)), fmaxf(fabsf(xv[j].z), fabsf(xv[j].w))));
    }
    m = group_max<32>(m);
    m = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kKW / 64; ++w) m = fmaxf(m, red[w]);
    const float s = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const int p = (d_pos ? *d_pos : pos_arg) + t, slot = p % page_tokens;
    uint8_t* page = static_cast<uint8_t*>((which ? pt_v : pt_k)[p / page_tokens]);
    int8_t* row = reinterpret_cast<int8_t*>(page) + static_cast<size_t>(slot) * kv_dim;
    auto qz = [&](float z) {
        const float r = q_round_away(__fdiv_rn(z, s), 127.0f);
        return static_cast<uint32_t>(static_cast<int>(r)) & 0xffu;
    };
#pragma unroll
    for (int j = 0; j < kKWV; ++j) {
        const int d = 4 * (j * kKW + static_cast<int>(threadIdx.x));
        if (d < kv_dim)
            *reinterpret_cast<uint32_t*>(row + d) =
                qz(xv[j].x) | (qz(xv[j].y) << 8) | (qz(xv[j].z) << 16) | (qz(xv[j].w) << 24);
    }
    if (threadIdx.x == 0) reinterpret_cast<float*>(page + kv_scale_offset(page_tokens, kv_dim))[slot] = s;
}

// PagedKVCache::dot_key (src/llama_model.cpp:23-39) of one stored key row
// (krow = the head's first element) with q (LDS): lane e of 8 accumulates
// fma(q[d], k[d]) for d = e, e+8, ...; sum = t0+t1+..+t7; then the tail as
// the compiled reference runs it -- F16/Q8: fused; F32 (dot_f32_simd): 4
// elements at a time with rounded products and in-order adds, the last
// hd % 4 fused.  The Q8 row scale is applied by the caller.
template <int KT>
__device__ __forceinline__ float kv_dot_row(const void* krow, const float* q, int hd) {
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    int c = 0;
    for (; c + 8 <= hd; c += 8) {
        float kf[8];
        kv_load8<KT>(krow, c, kf);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(q[c + e], kf[e], acc[e]);
    }
    float sum = acc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) sum = sum + acc[e];
    if constexpr (KT == kKvF32) {
        for (; c + 4 <= hd; c += 4)
#pragma unroll
            for (int j = 0; j < 4; ++j) sum = sum + q[c + j] * kv_to_f<KT>(krow, c + j);
    }
    for (; c < hd; ++c) sum = fmaf(q[c], kv_to_f<KT>(krow, c), sum);
    return sum;
}

// Address of element `e` of slot `slot` in a page of the cache type.
template <int KT>
__device__ __forceinline__ const void* kv_elem_ptr(const void* page, size_t slot, size_t kv_dim, size_t e) {
    return static_cast<const typename KvElem<KT>::T*>(page) + slot * kv_dim + e;
}

// Scores of query token b (grid z) and head h (grid x) against positions
// 0..upto, upto = pos + b (dot_key, src/llama_model.cpp:23-39, times the Q8
// row scale, divided by sqrtf(hd) as at :248/:256; kv_dot_row).  pos comes
// from *d_pos when d_pos != null, so the launch (sized for the largest
// position) can be replayed from a graph.
template <int KT>
__global__ __launch_bounds__(64) void attn_scores_kernel(const void* const* __restrict__ pt_k,
                                                         const float* __restrict__ q, int q_pitch,
                                                         float* __restrict__ scores,
                                                         const int* __restrict__ d_pos, int pos_arg, int n_head,
                                                         int group, int hd, int kv_dim, int page_tokens,
                                                         int score_pitch) {
    extern __shared__ float s_q[];
    const int h = blockIdx.x, b = blockIdx.z;
    const int upto = (d_pos ? *d_pos : pos_arg) + b;
    const int t0 = blockIdx.y * blockDim.x;
    if (t0 > upto) return;  // whole block past the causal limit
    const float* qh = q + static_cast<size_t>(b) * q_pitch + h * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) s_q[i] = qh[i];
    __syncthreads();
    const int t = t0 + threadIdx.x;
    if (t > upto) return;
    const int kh = h / group;
    const void* page = pt_k[t / page_tokens];
    float sum = kv_dot_row<KT>(kv_elem_ptr<KT>(page, t % page_tokens, kv_dim, kh * hd), s_q, hd);
    if constexpr (KT == kKvQ8) sum = sum * kv_row_scale<KT>(page, t % page_tokens, page_tokens, kv_dim);
    scores[(static_cast<size_t>(b) * n_head + h) * score_pitch + t] = __fdiv_rn(sum, sqrt_rn(static_cast<float>(hd)));
}

// Softmax and the value sum (src/llama_model.cpp:248,256): mx = max s,
// e = expf(s-mx), den = sum of e in double, inv = float(1/den), a_t = e_t*inv,
// out[d] = fma(w_t, V_t[d], out[d]) over t in order with w_t = a_t, or
// a_t * (V_t's row scale) for Q8 (add_value, :40-48).  One wave per
// (head, 64-wide slice of head_dim, query token); every output element's
// value chain runs in t order in its own lane, as in the reference.  The
// double `den` is added as a tree instead of in t order.  With q8 (hd % 32
// == 0) the output's quantize_q8 blocks are written too, row-major or in the
// prefill GEMM's operand order (q8_op, rows of n_head*hd).
template <int KT>
__global__ __launch_bounds__(64) void attn_softmax_v_kernel(const void* const* __restrict__ pt_v,
                                                            const float* __restrict__ scores, float* __restrict__ out,
                                                            const int* __restrict__ d_pos, int pos_arg, int n_head,
                                                            int group, int hd, int kv_dim, int page_tokens,
                                                            int score_pitch, int8_t* __restrict__ q8,
                                                            float* __restrict__ q8d, bool q8_op) {
    extern __shared__ float s_a[];  // [score_pitch] weights; Q8: then [score_pitch] V row scales
    __shared__ uint64_t s_tab[32];
    const uint64_t tab_v = mvh_expf_tab(threadIdx.x);  // the expf table, stored to LDS after the other loads
    const int h = blockIdx.x, b = blockIdx.z;
    const int n = (d_pos ? *d_pos : pos_arg) + b + 1;
    if constexpr (KT == kKvQ8) {  // V row scales: loads issued before the softmax, in flight meanwhile
        float* s_vs = s_a + score_pitch;
#pragma unroll 4
        for (int t = threadIdx.x; t < n; t += 64)
            s_vs[t] = kv_row_scale<KT>(pt_v[t / page_tokens], t % page_tokens, page_tokens, kv_dim);
    }
    if (threadIdx.x < 32) s_tab[threadIdx.x] = tab_v;
    __syncthreads();
    const float* sc = scores + (static_cast<size_t>(b) * n_head + h) * score_pitch;
    float mx = -INFINITY;
#pragma unroll 4
    for (int t = threadIdx.x; t < n; t += 64) mx = fmaxf(mx, sc[t]);
    mx = wave_max_all(mx);
    double den = 0.0;
    for (int t = threadIdx.x; t < n; t += 64) {
        const float e = mvh_expf_tabbed(sc[t] - mx, s_tab);
        s_a[t] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    const float inv = static_cast<float>(1.0 / den);
    __syncthreads();
    const int kh = h / group;
    for (int t = threadIdx.x; t < n; t += 64) {
        float a = s_a[t] * inv;
        if constexpr (KT == kKvQ8) a = a * s_a[score_pitch + t];
        s_a[t] = a;
    }
    __syncthreads();
    const int d = blockIdx.y * 64 + threadIdx.x;
    const bool live = d < hd;
    float acc = 0.0f;
    if (live) {
        for (int p0 = 0; p0 < n; p0 += page_tokens) {
            const void* vp = kv_elem_ptr<KT>(pt_v[p0 / page_tokens], 0, kv_dim, kh * hd + d);
            const int m = min(page_tokens, n - p0);
            int i = 0;
            for (; i + 8 <= m; i += 8) {
                float vv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) vv[j] = kv_to_f<KT>(vp, (i + j) * kv_dim);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = fmaf(s_a[p0 + i + j], vv[j], acc);
            }
            for (; i < m; ++i) acc = fmaf(s_a[p0 + i], kv_to_f<KT>(vp, i * kv_dim), acc);
        }
    }
    const size_t o = (static_cast<size_t>(b) * n_head + h) * hd + d;
    if (live) out[o] = acc;
    if (q8 && live) {  // quantize_q8 of this lane's 32-element block (hd % 32 == 0): the o projection's input
        const float mq = group_max<32>(fabsf(acc));
        const float dq = mq > 0.0f ? __fdiv_rn(mq, 127.0f) : 1.0f;
        const float id = __fdiv_rn(1.0f, dq);
        const float rq = q_round_away(acc * id, 127.0f);
        const int col = h * hd + d, D = n_head * hd;
        q8[q8_op ? q8_op_offset(b, col, D) : o] = static_cast<int8_t>(rq);
        if ((threadIdx.x & 31) == 0) q8d[o / 32] = dq;
    }
}


// ---- fused decode attention --------------------------------------------------
//
// One decode token, one launch, for the model's preallocated F16 KV slab (page
// p of a layer at kbase / vbase + p * page_stride: rows are addressed without a
// page-table load).  Workgroup (head h, slice j) owns output elements
// [j*SW, (j+1)*SW) of head h:
//  1. RoPE of q (head h) and k (kv head h/group) at position p = *d_pos
//     (LlamaModel::rope_ptr numerics), k and v rounded through the
//     reference's fp32_to_fp16; the first workgroup of each kv head writes
//     the K/V row of position p into its page; every workgroup keeps the
//     rounded values of position p in LDS and uses them for t = p;
//  2. s_t = dot_key(q, K_t) / sqrtf(hd) for t = 0..p (thread per position,
//     lane-of-8 fma accumulation, t0+..+t7);
//  3. mx, e_t = expf(s_t - mx), den = double sum, a_t = e_t * float(1/den);
//  4. out[d] = fma(a_t, V_t[d], out[d]) for t = 0..p in order, one lane per
//     output element, the V slice staged through LDS in rounds of kRV rows,
//     transposed so a lane reads 8 rows with one 16-byte LDS load (the
//     global loads of round r+1 are in flight while round r is summed);
//  5. with SW == 32 the slice is one Q8 block of the output: quantize_q8 of
//     it (the o-projection's activation) is written beside it.
// One memory round trip on the critical path: the position, q/k/v, the
// RoPE row of the position (copied to a fixed buffer by the token's embedding
// launch), the first K row of each thread (row t) and V round 0 (rows
// 0..kRV-1) are all issued together, none of their addresses depending on the
// position (rows past the position are read and ignored; at positions below
// kAT that is the price of not waiting for the position first).  Later K rows
// and V rounds follow the position.  The scores are recomputed by every slice
// of a head (K is read from L2).
constexpr int kAT = 256;
constexpr int kRV = 256;        // V rows per staging round
constexpr int kRVP = kRV + 8;   // LDS pitch of a transposed V dimension: 528 bytes (132
                                // dwords, 4 mod 32), so the lanes' 16-byte row reads fall in
                                // different banks (at a multiple of 128 bytes they collide)
constexpr int kMaxPages = 128;  // KV pages a context may span

// HD != 0 fixes head_dim at compile time (the loops over it unroll and the
// LDS reads of q are scheduled ahead of their use); HD == 0 reads hd_arg.
template <int SW, int HD>
__global__ __launch_bounds__(kAT) void attn_decode_fused_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ rope, const int* __restrict__ d_pos, uint16_t* kbase, uint16_t* vbase,
    int page_tokens, size_t page_stride, int rows_alloc, float* __restrict__ out, int8_t* __restrict__ q8,
    float* __restrict__ q8d, int group, int hd_arg, int kv_dim, int ctx_pad, int nslice) {
    const int hd = HD ? HD : hd_arg;
    constexpr int kCh = SW / 8;                        // 16-byte chunks per V row slice
    constexpr int kVPT = (kRV * kCh + kAT - 1) / kAT;  // chunks per thread per round
    extern __shared__ __align__(16) float sm[];
    float* s_q = sm;
    float* s_k = sm + hd;
    float* s_v = sm + 2 * hd;
    float* s_a = sm + 3 * hd;
    uint16_t* s_vt = reinterpret_cast<uint16_t*>(s_a + ctx_pad);  // [SW][kRVP]
    __shared__ float red_f[kAT / 64];
    __shared__ double red_d[kAT / 64];
    __shared__ uint64_t s_tab[32];

    const int h = blockIdx.x / nslice, slice = blockIdx.x - h * nslice;
    const int kh = h / group, t = threadIdx.x, half = hd >> 1;
    const int dbase = slice * SW;
    auto krow_of = [&](int tt) {
        return kbase + static_cast<size_t>(tt / page_tokens) * page_stride + static_cast<size_t>(tt % page_tokens) * kv_dim +
               kh * hd;
    };
    auto vrow_of = [&](int tt) {
        return vbase + static_cast<size_t>(tt / page_tokens) * page_stride + static_cast<size_t>(tt % page_tokens) * kv_dim +
               kh * hd;
    };

    // The one round trip: position, q/k/v, the RoPE row, row t of K, V round
    // 0.  Every load is unconditional (threads without a use read an in-bounds
    // element and ignore it) and issued in this order (the scheduling
    // barriers keep it): vector loads complete in issue order, so RoPE waits
    // for q/k/v and the RoPE row alone while the K rows and V are in flight (a
    // load under a branch makes the compiler's wait cover all of them).
    const int pos = *d_pos;
    const uint64_t tab_v = mvh_expf_tab(t);  // the expf table, stored to LDS after the other loads
    const int th = t < half ? t : 0;
    const float* qh = q + static_cast<size_t>(h) * hd;
    const float* kk = k + static_cast<size_t>(kh) * hd;
    const float* vv = v + static_cast<size_t>(kh) * hd;
    const float q0 = qh[th], q1 = qh[th + half], k0 = kk[th], k1 = kk[th + half], v0 = vv[th], v1 = vv[th + half];
    const float cs = rope[th];
    const float sn = rope[half + th];
    __builtin_amdgcn_sched_barrier(0);
    uint4 kv[16];
    auto load_k = [&](int tt, int c0) {
        const uint16_t* kr = krow_of(tt) + c0;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (c0 + 8 * j < hd) kv[j] = ld_global16(kr + 8 * j);
    };
    load_k(min(t, rows_alloc - 1), 0);  // rows at or past pos: read, unused
    uint4 vr[kVPT];
    auto load_round = [&](int r0, int nrows) {
        // branch-free: chunks past the round's rows re-read row r0 (ignored)
        const int lim = nrows * kCh;
#pragma unroll
        for (int i = 0; i < kVPT; ++i) {
            const int c = i * kAT + t < lim ? i * kAT + t : 0;
            vr[i] = ld_global16(vrow_of(r0 + c / kCh) + dbase + (c % kCh) * 8);
        }
    };
    load_round(0, min(kRV, rows_alloc));  // the whole first round, whatever pos is
    __builtin_amdgcn_sched_barrier(0);

    // 1. RoPE, K/V of the current position (computed by every thread, so the
    // cos/sin loads are used outside a branch; threads t >= half drop it)
    const float rq0 = fmaf(q0, cs, -(q1 * sn)), rq1 = fmaf(q0, sn, q1 * cs);
    const uint16_t hk0 = f2h_ref(fmaf(k0, cs, -(k1 * sn))), hk1 = f2h_ref(fmaf(k0, sn, k1 * cs));
    const uint16_t hv0 = f2h_ref(v0), hv1 = f2h_ref(v1);
    if (t < half) {
        s_q[t] = rq0;
        s_q[t + half] = rq1;
        s_k[t] = h2f(hk0);
        s_k[t + half] = h2f(hk1);
        s_v[t] = h2f(hv0);
        s_v[t + half] = h2f(hv1);
        if (slice == 0 && h % group == 0) {  // one writer per kv head
            uint16_t* kc = krow_of(pos);
            uint16_t* vc = vrow_of(pos);
            kc[t] = hk0;
            kc[t + half] = hk1;
            vc[t] = hv0;
            vc[t + half] = hv1;
        }
    }
    if (t < 32) s_tab[t] = tab_v;
    __syncthreads();

    // 2. scores
    const float scale = sqrt_rn(static_cast<float>(hd));
    float mx = -INFINITY;
    for (int tt = t; tt <= pos; tt += kAT) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
        if (tt == pos) {
            for (int c = 0; c < hd; c += 8) {
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] = fmaf(s_q[c + e], s_k[c + e], acc[e]);
            }
        } else {
            for (int c0 = 0; c0 < hd; c0 += 128) {
                if (tt != t || c0 != 0) load_k(tt, c0);  // the first group of the first row is in flight already
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    if (c0 + 8 * j >= hd) break;
                    const half8 hk = as_half8(kv[j]);
                    const float4 qa = *reinterpret_cast<const float4*>(s_q + c0 + 8 * j);
                    const float4 qb = *reinterpret_cast<const float4*>(s_q + c0 + 8 * j + 4);
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] = fmaf(qv[e], static_cast<float>(hk[e]), acc[e]);
                }
            }
        }
        float sum = acc[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) sum = sum + acc[e];
        const float sc = __fdiv_rn(sum, scale);
        s_a[tt] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = wave_max_all(mx);
    if ((t & 63) == 0) red_f[t >> 6] = mx;
    __syncthreads();
    mx = red_f[0];
#pragma unroll
    for (int w = 1; w < kAT / 64; ++w) mx = fmaxf(mx, red_f[w]);

    // 3. softmax weights
    double den = 0.0;
    for (int tt = t; tt <= pos; tt += kAT) {
        const float e = mvh_expf_tabbed(s_a[tt] - mx, s_tab);
        s_a[tt] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    if ((t & 63) == 0) red_d[t >> 6] = den;
    __syncthreads();
    den = red_d[0];
#pragma unroll
    for (int w = 1; w < kAT / 64; ++w) den += red_d[w];
    const float inv = static_cast<float>(1.0 / den);
    for (int tt = t; tt <= pos; tt += kAT) s_a[tt] = s_a[tt] * inv;

    // 4. value chain over t = 0..pos in order
    float acc = 0.0f;
    for (int r0 = 0; r0 < pos; r0 += kRV) {
        const int rows = min(kRV, pos - r0);
        // transpose into [dim][row] so each lane's rows are contiguous
#pragma unroll
        for (int i = 0; i < kVPT; ++i) {
            const int c = i * kAT + t;
            if (c < rows * kCh) {
                const int row = c / kCh, d0 = (c % kCh) * 8;
                const uint32_t w[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    s_vt[(d0 + e) * kRVP + row] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
            }
        }
        __syncthreads();  // also orders the s_a writes above before their reads
        if (r0 + kRV < pos) load_round(r0 + kRV, min(kRV, pos - r0 - kRV));
        if (t < SW) {
            const uint16_t* vl = s_vt + t * kRVP;
            const float* al = s_a + r0;
            // 16-row steps with two register sets used in turn (A even, B
            // odd).  Every LDS read is unconditional -- the read for a step
            // past the last one re-reads the last step (in bounds, unused) --
            // so the wait counts only cover the set being summed and the
            // next set's reads stay in flight during the fma chain.
            const int nsteps = rows >> 4;
            auto ld = [&](int st, uint4& v0, uint4& v1, float4 (&a)[4]) {
                const int j0 = min(st, nsteps - 1) << 4;
                v0 = *reinterpret_cast<const uint4*>(vl + j0);
                v1 = *reinterpret_cast<const uint4*>(vl + j0 + 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const float4*>(al + j0 + 4 * i);
            };
            auto step = [&](float c, const uint4& v0, const uint4& v1, const float4 (&a)[4]) {
                const half8 h0 = as_half8(v0), h1 = as_half8(v1);
                const float av[16] = {a[0].x, a[0].y, a[0].z, a[0].w, a[1].x, a[1].y, a[1].z, a[1].w,
                                      a[2].x, a[2].y, a[2].z, a[2].w, a[3].x, a[3].y, a[3].z, a[3].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) c = fmaf(av[e], static_cast<float>(h0[e]), c);
#pragma unroll
                for (int e = 0; e < 8; ++e) c = fmaf(av[8 + e], static_cast<float>(h1[e]), c);
                return c;
            };
            if (nsteps > 0) {
                uint4 va0, va1, vb0, vb1;
                float4 aa[4], ab[4];
                ld(0, va0, va1, aa);
                for (int st = 0; st < nsteps; st += 2) {
                    // scheduling barriers keep each set's reads ahead of the
                    // other set's fma chain
                    ld(st + 1, vb0, vb1, ab);
                    __builtin_amdgcn_sched_barrier(0);
                    acc = step(acc, va0, va1, aa);
                    __builtin_amdgcn_sched_barrier(0);
                    ld(st + 2, va0, va1, aa);
                    __builtin_amdgcn_sched_barrier(0);
                    // the odd step always runs (no branch for its reads to sink
                    // into) and is kept only when it exists
                    const float nb = step(acc, vb0, vb1, ab);
                    acc = st + 1 < nsteps ? nb : acc;
                }
            }
            int j = nsteps << 4;
            for (; j < rows; ++j) acc = fmaf(al[j], h2f(vl[j]), acc);
        }
        __syncthreads();
    }
    if (pos == 0) __syncthreads();  // s_a writes before the read below
    if (t < SW) {
        acc = fmaf(s_a[pos], s_v[dbase + t], acc);
        const size_t o = static_cast<size_t>(h) * hd + dbase + t;
        out[o] = acc;
        if constexpr (SW == 32) {
            if (q8) {  // quantize_q8 of this 32-element block of the output
                const float m = group_max<32>(fabsf(acc));
                const float d = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
                const float id = __fdiv_rn(1.0f, d);
                const float rq = q_round_away(acc * id, 127.0f);
                q8[o] = static_cast<int8_t>(rq);
                if (t == 0) q8d[o / 32] = d;
            }
        }
    }
}

// ---- fused decode attention, K and V staged through LDS ----------------------
//
// The same step as attn_decode_fused_kernel (RoPE of q and k at position
// p = *d_pos, the F16 K/V row of p written through fp32_to_fp16, scores
// dot_key / sqrtf(hd), mx, e = expf(s - mx), den in double, a_t = e_t *
// float(1/den), out[d] = fma(a_t, V_t[d], out[d]) for t = 0..p in order, Q8
// of each 32-element block of the output), arranged so that every K and V
// byte crosses the memory system once per workgroup in full 16-byte pieces of
// whole rows:
//  * workgroup (head h, slice s of NS) owns output elements [s*SW, (s+1)*SW),
//    SW = HD / NS; the NS slices of a head run on one XCD (consecutive
//    blockIdx modulo the eight XCDs), so their K rows come from one L2;
//  * K rows are staged in rounds of kHR rows: thread t loads 16-byte pieces
//    t, t + 256, ... of the round (CPR = HD/8 pieces per row, so a wave's
//    load covers whole rows), stores them to an LDS tile of pitch
//    2*HD + 16 bytes, and after one barrier computes the score of row t of
//    the round from the tile with the reference's eight-lane fma order;
//  * V rows of the slice are loaded after the K tile is stored (the loads
//    then queue behind K's instead of ahead of them: a workgroup's loads are
//    accepted at a bounded rate) and arrive during the scores; a group of
//    eight lanes loads eight consecutive rows of one 8-element chunk, lane
//    pairs exchange halves (DPP) and each writes one 16-byte piece of a tile
//    laid out as [row pair][element][2 rows], so the value chain reads two
//    rows of its element with one LDS load;
//  * the value chain runs in wave 0, lane l owning DPL = SW/64 (or 1) output
//    elements, two steps of 8 rows in flight;
//  * round 0 of K (rows 0..kHR-1, whatever the position: rows past it are
//    read and ignored) is issued with q/k/v and the RoPE row, so the kernel
//    has one memory round trip below kHR positions; the position's own K and
//    V rows are taken from the RoPE'd k and the rounded v (the cache row is
//    written by this launch), not from the staged copy;
//  * the max and the double denominator are reduced across each wave by DPP
//    (wave_max_all, wave_sum), then across the four waves through LDS.
constexpr int kHT = 256;        // threads
constexpr int kHR = 256;        // rows per staging round
constexpr int kHMaxCtx = 2048;  // positions the LDS score array holds

template <int HD, int NS>
struct HeadCfg {
    static constexpr int SW = HD / NS;                   // output elements per workgroup
    static constexpr int CPR = HD / 8;                   // 16-byte K pieces per row
    static constexpr int KPT = kHR * CPR / kHT;          // K pieces per thread per round
    static constexpr int CV = SW / 8;                    // 16-byte V pieces per row of the slice
    static constexpr int VPT = kHR * CV / kHT;           // V pieces per thread per round
    static constexpr int KP = 2 * HD + 16;               // K tile pitch (bytes)
    static constexpr int VPP = SW + 16;                  // V tile pitch per row pair (dwords)
    static constexpr int DPL = SW >= 128 ? SW / 64 : 1;  // output elements per chain lane
    static constexpr int LANES = SW / DPL;               // chain lanes (<= 64: wave 0)
    static_assert(kHR * CPR % kHT == 0 && kHR * CV % kHT == 0 && LANES <= 64 && DPL <= 2, "head attention shape");
};

// The arguments the first instructions need come first: the 14 dwords the
// dispatch preloads into SGPRs hold nwg .. kbase (q, k and v are one buffer:
// k at q + n_head * HD, v at k + kv_dim).
template <int HD, int NS>
__global__ __launch_bounds__(kHT) void attn_decode_head_kernel(
    int nwg, int group, int page_tokens, int kv_dim, int rows_alloc, int page_stride, const float* __restrict__ q,
    const float* __restrict__ rope, const int* __restrict__ d_pos, uint16_t* kbase, uint16_t* vbase,
    float* __restrict__ out, int8_t* __restrict__ q8, float* __restrict__ q8d, L2Warm warm, L2Warm warm2) {
    using C = HeadCfg<HD, NS>;
    constexpr int SW = C::SW, CPR = C::CPR, KPT = C::KPT, CV = C::CV, VPT = C::VPT, KP = C::KP, VPP = C::VPP,
                  DPL = C::DPL, half = HD / 2;
    __shared__ __align__(16) uint8_t s_kt[kHR * KP];
    __shared__ __align__(16) uint32_t s_vt[kHR / 2 * VPP];
    __shared__ __align__(16) float s_q[HD];
    __shared__ __align__(16) float s_a[kHMaxCtx];
    __shared__ float red_f[kHT / 64];
    __shared__ double red_d[kHT / 64];
    __shared__ uint64_t s_tab[32];

    // blockIdx -> (head, slice): the slices of a head on one XCD; workgroups
    // from nwg on warm the weights of the GEMVs after it instead (l2_warm;
    // the o projection's, then a share of the next one's)
    const int G = nwg, b = blockIdx.x;
    if (b >= G) {
        l2_warm<kHT>(warm, b, G, static_cast<int>(gridDim.x) - G);
        l2_warm<kHT>(warm2, b, G, static_cast<int>(gridDim.x) - G);
        return;
    }
    const int hs = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    const int h = hs / NS, slice = hs - h * NS;
    const int kh = h / group, t = threadIdx.x, dbase = slice * SW;
    const float* k = q + static_cast<size_t>(G / NS) * HD;
    const float* v = k + kv_dim;
    auto row_off = [&](int tt) {
        return static_cast<size_t>(tt / page_tokens) * page_stride + static_cast<size_t>(tt % page_tokens) * kv_dim +
               kh * HD;
    };
    // this thread's V pieces: rows 8 * rg + vi of chunk vc (the same chunk in every round)
    const int vi = t & 7, vc = (t >> 3) % CV;

    // the one round trip: position, q/k/v, the RoPE row, K round 0 and this
    // thread's chunk of the position's v (the position by a vector load, made
    // uniform only after the K loads are issued: a scalar load of it would
    // hold up the K loads, whose addresses wait for the kernel's argument
    // loads on the same counter)
    const int pos_v = ld_global_lanes(d_pos);
    const uint64_t tab_v = mvh_expf_tab(t);  // the expf table, stored to LDS after the RoPE
    const int th = t < half ? t : 0;
    const float* qh = q + static_cast<size_t>(h) * HD;
    const float* kk = k + static_cast<size_t>(kh) * HD;
    const float* vv = v + static_cast<size_t>(kh) * HD;
    const float q0 = qh[th], q1 = qh[th + half], k0 = kk[th], k1 = kk[th + half], v0 = vv[th], v1 = vv[th + half];
    const float cs = rope[th];
    const float sn = rope[half + th];
    const float4 pv0 = *reinterpret_cast<const float4*>(vv + dbase + 8 * vc);
    const float4 pv1 = *reinterpret_cast<const float4*>(vv + dbase + 8 * vc + 4);
    __builtin_amdgcn_sched_barrier(0);
    uint4 kr[KPT], vr[VPT];
    auto load_k = [&](int r0) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int pc = i * kHT + t, row = min(r0 + pc / CPR, rows_alloc - 1);
            kr[i] = ld_global16(kbase + row_off(row) + (pc % CPR) * 8);
        }
    };
    auto load_v = [&](int r0) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int rg = (i * kHT + t) / (8 * CV), row = min(r0 + 8 * rg + vi, rows_alloc - 1);
            vr[i] = ld_global16(vbase + row_off(row) + dbase + vc * 8);
        }
    };
    load_k(0);
    __builtin_amdgcn_sched_barrier(0);
    const int pos = __builtin_amdgcn_readfirstlane(pos_v);

    // RoPE (every thread computes it so the loads are used outside a branch)
    const float rq0 = fmaf(q0, cs, -(q1 * sn)), rq1 = fmaf(q0, sn, q1 * cs);
    const uint16_t hk0 = f2h_ref(fmaf(k0, cs, -(k1 * sn))), hk1 = f2h_ref(fmaf(k0, sn, k1 * cs));
    const uint16_t hv0 = f2h_ref(v0), hv1 = f2h_ref(v1);
    const uint4 vpos = make_uint4(f2h_ref(pv0.x) | (static_cast<uint32_t>(f2h_ref(pv0.y)) << 16),
                                  f2h_ref(pv0.z) | (static_cast<uint32_t>(f2h_ref(pv0.w)) << 16),
                                  f2h_ref(pv1.x) | (static_cast<uint32_t>(f2h_ref(pv1.y)) << 16),
                                  f2h_ref(pv1.z) | (static_cast<uint32_t>(f2h_ref(pv1.w)) << 16));
    if (t < half) {
        s_q[t] = rq0;
        s_q[t + half] = rq1;
        if (slice == 0 && h % group == 0) {  // one writer of the cache row per kv head
            uint16_t* kc = kbase + row_off(pos);
            uint16_t* vc_ = vbase + row_off(pos);
            kc[t] = hk0;
            kc[t + half] = hk1;
            vc_[t] = hv0;
            vc_[t + half] = hv1;
        }
    }
    if (t < 32) s_tab[t] = tab_v;
    // stores of the staged registers, the position's row replaced by the RoPE'd k
    auto store_k = [&](int r0) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int pc = i * kHT + t, row = pc / CPR;
            if (r0 + row != pos) *reinterpret_cast<uint4*>(s_kt + row * KP + (pc % CPR) * 16) = kr[i];
        }
        if (pos >= r0 && pos < r0 + kHR && t < half) {
            uint16_t* kt = reinterpret_cast<uint16_t*>(s_kt + (pos - r0) * KP);
            kt[t] = hk0;
            kt[t + half] = hk1;
        }
    };
    // V pieces to the [row pair][element][2] tile: the position's row taken
    // from the rounded v; lanes 2j, 2j+1 (rows r, r+1 of the chunk) swap the
    // elements 4..7 of row r for 0..3 of row r+1, then each writes its four
    // elements of both rows
    auto store_v = [&](int r0) {
        const bool odd = t & 1;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int rg = (i * kHT + t) / (8 * CV), row = 8 * rg + vi;
            const uint4 w = r0 + row == pos ? vpos : vr[i];
            const uint32_t s0 = odd ? w.x : w.z, s1 = odd ? w.y : w.w;
            const uint32_t x0 = static_cast<uint32_t>(dpp_mov<0xb1>(static_cast<int>(s0)));
            const uint32_t x1 = static_cast<uint32_t>(dpp_mov<0xb1>(static_cast<int>(s1)));
            const uint32_t e0 = odd ? x0 : w.x, e1 = odd ? x1 : w.y;  // even row's elements
            const uint32_t o0 = odd ? w.z : x0, o1 = odd ? w.w : x1;  // odd row's elements
            const uint4 pr = make_uint4(__builtin_amdgcn_perm(o0, e0, 0x05040100u), __builtin_amdgcn_perm(o0, e0, 0x07060302u),
                                        __builtin_amdgcn_perm(o1, e1, 0x05040100u), __builtin_amdgcn_perm(o1, e1, 0x07060302u));
            *reinterpret_cast<uint4*>(s_vt + (row >> 1) * VPP + vc * 8 + (odd ? 4 : 0)) = pr;
        }
    };

    // scores, round by round; the next round's K loads in flight meanwhile
    const float scale = sqrt_rn(static_cast<float>(HD));
    float mx = -INFINITY;
    for (int r0 = 0; r0 <= pos; r0 += kHR) {
        if (r0) __syncthreads();  // the previous round's tile reads are done
        store_k(r0);
        if (r0 + kHR <= pos) load_k(r0 + kHR);
        if (r0 == 0) load_v(0);
        __syncthreads();
        const int tt = r0 + t;
        if (tt <= pos) {
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
            const uint8_t* kt = s_kt + t * KP;
#pragma unroll
            for (int c = 0; c < CPR; ++c) {
                const half8 hk = as_half8(*reinterpret_cast<const uint4*>(kt + 16 * c));
                const float4 qa = *reinterpret_cast<const float4*>(s_q + 8 * c);
                const float4 qb = *reinterpret_cast<const float4*>(s_q + 8 * c + 4);
                const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] = fmaf(qv[e], static_cast<float>(hk[e]), acc[e]);
            }
            float sum = acc[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) sum = sum + acc[e];
            const float sc = __fdiv_rn(sum, scale);
            s_a[tt] = sc;
            mx = fmaxf(mx, sc);
        }
    }
    store_v(0);  // round 0 of V, arrived during the scores
    mx = wave_max_all(mx);
    if ((t & 63) == 0) red_f[t >> 6] = mx;
    __syncthreads();
    mx = red_f[0];
#pragma unroll
    for (int w = 1; w < kHT / 64; ++w) mx = fmaxf(mx, red_f[w]);

    // softmax weights
    double den = 0.0;
    for (int tt = t; tt <= pos; tt += kHT) {
        const float e = mvh_expf_tabbed(s_a[tt] - mx, s_tab);
        s_a[tt] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    if ((t & 63) == 0) red_d[t >> 6] = den;
    __syncthreads();
    den = red_d[0];
#pragma unroll
    for (int w = 1; w < kHT / 64; ++w) den += red_d[w];
    const float inv = static_cast<float>(1.0 / den);
    for (int tt = t; tt <= pos; tt += kHT) s_a[tt] = s_a[tt] * inv;

    // value chain over t = 0..pos in order, round by round
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;
    const int lane = t;  // wave 0
    for (int r0 = 0; r0 <= pos; r0 += kHR) {
        if (r0) {
            __syncthreads();  // the previous round's chain is done
            store_v(r0);
        }
        if (r0 + kHR <= pos) load_v(r0 + kHR);
        __syncthreads();  // the tile (and, in round 0, the weights) written
        if (t < C::LANES) {
            const int rows = min(kHR, pos + 1 - r0);
            const uint32_t* vl = s_vt + lane * DPL;
            const float* al = s_a + r0;
            // steps of 4 row pairs (8 rows), three register sets in turn, two
            // steps in flight; every read is unconditional (a step past the
            // last one re-reads the last), so the wait counts cover only the
            // set being summed
            const int nsteps = rows >> 3;
            struct Set {
                uint32_t w[4][DPL];
                float4 a[2];
            };
            auto ld = [&](int st, Set& s) {
                const int j0 = min(st, max(nsteps - 1, 0)) << 3;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    if constexpr (DPL == 2) {
                        const uint2 x = *reinterpret_cast<const uint2*>(vl + ((j0 >> 1) + p) * VPP);
                        s.w[p][0] = x.x;
                        s.w[p][DPL - 1] = x.y;
                    } else {
                        s.w[p][0] = vl[((j0 >> 1) + p) * VPP];
                    }
                }
                s.a[0] = *reinterpret_cast<const float4*>(al + j0);
                s.a[1] = *reinterpret_cast<const float4*>(al + j0 + 4);
            };
            auto step = [&](const Set& s) {
                const float av[8] = {s.a[0].x, s.a[0].y, s.a[0].z, s.a[0].w, s.a[1].x, s.a[1].y, s.a[1].z, s.a[1].w};
#pragma unroll
                for (int p = 0; p < 4; ++p) {
#pragma unroll
                    for (int i = 0; i < DPL; ++i) acc[i] = fmaf(av[2 * p], h2f(s.w[p][i] & 0xffffu), acc[i]);
#pragma unroll
                    for (int i = 0; i < DPL; ++i) acc[i] = fmaf(av[2 * p + 1], h2f(s.w[p][i] >> 16), acc[i]);
                }
            };
            if (nsteps > 0) {
                Set sa, sb, sc;
                ld(0, sa);
                ld(1, sb);
                for (int st = 0; st < nsteps; st += 3) {
                    ld(st + 2, sc);
                    __builtin_amdgcn_sched_barrier(0);
                    step(sa);
                    __builtin_amdgcn_sched_barrier(0);
                    ld(st + 3, sa);
                    __builtin_amdgcn_sched_barrier(0);
                    if (st + 1 < nsteps) step(sb);
                    __builtin_amdgcn_sched_barrier(0);
                    ld(st + 4, sb);
                    __builtin_amdgcn_sched_barrier(0);
                    if (st + 2 < nsteps) step(sc);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            for (int j = nsteps << 3; j < rows; ++j) {
                const int p = j >> 1, sh = 16 * (j & 1);
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] = fmaf(al[j], h2f((vl[p * VPP + i] >> sh) & 0xffffu), acc[i]);
            }
        }
    }
    if (t < C::LANES) {
        const size_t o = static_cast<size_t>(h) * HD + dbase + lane * DPL;
        if constexpr (DPL == 2) {
            *reinterpret_cast<float2*>(out + o) = make_float2(acc[0], acc[DPL - 1]);
        } else {
            out[o] = acc[0];
        }
        // quantize_q8 of each 32-element block of the output (32 / DPL lanes;
        // a slice narrower than a block is launched without q8)
        if (SW % 32 == 0 && q8) {
            constexpr int L = 32 / DPL;
            float m = fabsf(acc[0]);
            if constexpr (DPL == 2) m = fmaxf(m, fabsf(acc[DPL - 1]));
            m = group_max<L>(m);
            const float d = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
            const float id = __fdiv_rn(1.0f, d);
#pragma unroll
            for (int i = 0; i < DPL; ++i) q8[o + i] = static_cast<int8_t>(q_round_away(acc[i] * id, 127.0f));
            if ((lane & (L - 1)) == 0) q8d[o / 32] = d;
        }
    }
}

// ---- prefill chunk attention: scores + softmax once, values shared ----------
//
// Scores and softmax weights of query token b (grid y) and head h (grid x)
// over positions 0..pos0+b, one workgroup: the same arithmetic as
// attn_scores_kernel (kv_dot_row, Q8 row scale, / sqrtf(hd)) and
// attn_softmax_v_kernel (mx, e = expf(s - mx), den in double, a = e *
// float(1/den), times V_t's row scale for Q8); writes that weight to
// a[(b*n_head + h)*pitch + t].  The double den is a tree over the
// workgroup's threads (not in t order).
constexpr int kSM = 256;
template <int KT>
__global__ __launch_bounds__(kSM) void attn_scores_softmax_kernel(const void* const* __restrict__ pt_k,
                                                                  const void* const* __restrict__ pt_v,
                                                                  const float* __restrict__ q, int q_pitch,
                                                                  float* __restrict__ a_out,
                                                                  const int* __restrict__ d_pos, int pos_arg,
                                                                  int n_head, int group, int hd, int kv_dim,
                                                                  int page_tokens, int pitch) {
    extern __shared__ float sm_s[];  // [hd] q, then [pitch] scores / weights
    float* s_q = sm_s;
    float* s_s = sm_s + hd;
    __shared__ float red_f[kSM / 64];
    __shared__ double red_d[kSM / 64];
    __shared__ uint64_t s_tab[32];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int n = (d_pos ? *d_pos : pos_arg) + b + 1;
    const int kh = h / group;
    const float* qh = q + static_cast<size_t>(b) * q_pitch + static_cast<size_t>(h) * hd;
    const uint64_t tab_v = mvh_expf_tab(t);
    for (int i = t; i < hd; i += kSM) s_q[i] = qh[i];
    if (t < 32) s_tab[t] = tab_v;
    __syncthreads();
    const float scale = sqrt_rn(static_cast<float>(hd));
    float mx = -INFINITY;
    for (int tt = t; tt < n; tt += kSM) {
        const void* page = pt_k[tt / page_tokens];
        float sum = kv_dot_row<KT>(kv_elem_ptr<KT>(page, tt % page_tokens, kv_dim, kh * hd), s_q, hd);
        if constexpr (KT == kKvQ8) sum = sum * kv_row_scale<KT>(page, tt % page_tokens, page_tokens, kv_dim);
        const float sc = __fdiv_rn(sum, scale);
        s_s[tt] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = wave_max_all(mx);
    if ((t & 63) == 0) red_f[t >> 6] = mx;
    __syncthreads();
    mx = red_f[0];
#pragma unroll
    for (int w = 1; w < kSM / 64; ++w) mx = fmaxf(mx, red_f[w]);
    double den = 0.0;
    for (int tt = t; tt < n; tt += kSM) {
        const float e = mvh_expf_tabbed(s_s[tt] - mx, s_tab);
        s_s[tt] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    if ((t & 63) == 0) red_d[t >> 6] = den;
    __syncthreads();
    den = red_d[0];
#pragma unroll
    for (int w = 1; w < kSM / 64; ++w) den += red_d[w];
    const float inv = static_cast<float>(1.0 / den);
    float* ar = a_out + (static_cast<size_t>(b) * n_head + h) * pitch;
    for (int tt = t; tt < n; tt += kSM) {
        float a = s_s[tt] * inv;
        if constexpr (KT == kKvQ8)
            a = a * kv_row_scale<KT>(pt_v[tt / page_tokens], tt % page_tokens, page_tokens, kv_dim);
        ar[tt] = a;
    }
}

// Scores of a prefill chunk for F16 pages, K read once per head and row
// block: workgroup (head h, block of kTR positions), every query token of the
// chunk (B <= 32).  The block's K rows come in with 16-byte loads (a wave's
// load covers whole rows) into an LDS tile; the chunk's q rows are staged
// beside it; thread t scores tile row t % kTR for tokens t / kTR + 4k
// (k = 0..7), with kv_dot_row's order (eight-lane fma over the elements,
// t0 + .. + t7) and the division by sqrtf(hd).  Writes the raw score of every
// (token b, position p <= pos0 + b) to s[(b*n_head + h)*pitch + p]; the
// softmax then runs per (head, token) on those rows (attn_softmax_rows_kernel).
// Against one workgroup per (head, token) reading its K rows itself, K crosses
// the caches once per head instead of once per token.
constexpr int kTR = 64;
template <int HD>
__global__ __launch_bounds__(256) void attn_scores_tile_kernel(const void* const* __restrict__ pt_k,
                                                               const float* __restrict__ q, int q_pitch,
                                                               float* __restrict__ s_out, int pos0, int B,
                                                               int n_head, int group, int kv_dim, int page_tokens,
                                                               int pitch) {
    constexpr int CPR = HD / 8, KP = 2 * HD + 16;
    __shared__ __align__(16) uint8_t s_kt[kTR * KP];
    __shared__ __align__(16) float s_q[32 * HD];
    const int h = blockIdx.x, r0 = blockIdx.y * kTR, t = threadIdx.x, kh = h / group;
    const int nmax = pos0 + B;  // rows 0..nmax-1 hold keys (this chunk's included)
#pragma unroll
    for (int i = 0; i < kTR * CPR / 256; ++i) {
        const int pc = i * 256 + t, row = min(r0 + pc / CPR, nmax - 1);
        const uint16_t* src = static_cast<const uint16_t*>(pt_k[row / page_tokens]) +
                              static_cast<size_t>(row % page_tokens) * kv_dim + kh * HD + (pc % CPR) * 8;
        *reinterpret_cast<uint4*>(s_kt + (pc / CPR) * KP + (pc % CPR) * 16) = ld_global16(src);
    }
    for (int i = t; i < B * (HD / 4); i += 256) {
        const int b = i / (HD / 4), c = i % (HD / 4);
        reinterpret_cast<float4*>(s_q)[i] =
            *reinterpret_cast<const float4*>(q + static_cast<size_t>(b) * q_pitch + static_cast<size_t>(h) * HD + 4 * c);
    }
    __syncthreads();
    const int rr = t % kTR, tb = t / kTR, r = r0 + rr;
    float acc[8][8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[k][e] = 0.0f;
    const uint8_t* kt = s_kt + rr * KP;
#pragma unroll 4
    for (int c = 0; c < CPR; ++c) {
        const half8 hk = as_half8(*reinterpret_cast<const uint4*>(kt + 16 * c));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int b = min(tb + 4 * k, B - 1);  // the waves' tokens: one per wave and k (LDS broadcast)
            const float4 qa = *reinterpret_cast<const float4*>(s_q + b * HD + 8 * c);
            const float4 qb = *reinterpret_cast<const float4*>(s_q + b * HD + 8 * c + 4);
            const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[k][e] = fmaf(qv[e], static_cast<float>(hk[e]), acc[k][e]);
        }
    }
    const float scale = sqrt_rn(static_cast<float>(HD));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int b = tb + 4 * k;
        float sum = acc[k][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) sum = sum + acc[k][e];
        if (b < B && r <= pos0 + b)
            s_out[(static_cast<size_t>(b) * n_head + h) * pitch + r] = __fdiv_rn(sum, scale);
    }
}

// Softmax of the raw scores attn_scores_tile_kernel wrote, in place, one
// workgroup per (head h, token b) over positions 0..pos0+b: the arithmetic
// and thread mapping of attn_scores_softmax_kernel's second half (mx,
// e = expf(s - mx), den in double as the same tree, a = e * float(1/den)).
__global__ __launch_bounds__(kSM) void attn_softmax_rows_kernel(float* __restrict__ s_io, int pos0, int n_head,
                                                                int pitch) {
    __shared__ float red_f[kSM / 64];
    __shared__ double red_d[kSM / 64];
    __shared__ uint64_t s_tab[32];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int n = pos0 + b + 1;
    float* sr = s_io + (static_cast<size_t>(b) * n_head + h) * pitch;
    const uint64_t tab_v = mvh_expf_tab(t);
    float mx = -INFINITY;
    for (int tt = t; tt < n; tt += kSM) mx = fmaxf(mx, sr[tt]);
    mx = wave_max_all(mx);
    if ((t & 63) == 0) red_f[t >> 6] = mx;
    if (t < 32) s_tab[t] = tab_v;
    __syncthreads();
    mx = red_f[0];
#pragma unroll
    for (int w = 1; w < kSM / 64; ++w) mx = fmaxf(mx, red_f[w]);
    double den = 0.0;
    for (int tt = t; tt < n; tt += kSM) {
        const float e = mvh_expf_tabbed(sr[tt] - mx, s_tab);
        sr[tt] = e;
        den += static_cast<double>(e);
    }
    den = wave_sum(den);
    if ((t & 63) == 0) red_d[t >> 6] = den;
    __syncthreads();
    den = red_d[0];
#pragma unroll
    for (int w = 1; w < kSM / 64; ++w) den += red_d[w];
    const float inv = static_cast<float>(1.0 / den);
    for (int tt = t; tt < n; tt += kSM) sr[tt] = sr[tt] * inv;
}

// Value chains of a prefill chunk: workgroup (head h, 32-element slice of
// head_dim, group of 32 query tokens); thread = (token b, 4 consecutive
// elements), out[d] = fma(w_t, V_t[d], out[d]) over t = 0..pos0+b in order,
// as in the reference (w_t the weights attn_scores_softmax_kernel wrote).  V rows come in 64-row tiles staged once in LDS for all
// 32 tokens (the next tile's loads in flight while a tile is summed); the
// weights of rows past a token's last position are 0 there, an exact no-op
// (those rows are the chunk's later tokens, finite).  With q8 the output's
// quantize_q8 blocks (one per token and slice) are written too, row-major or
// in the prefill GEMM's operand order (q8_op).
constexpr int kPV = 256;
constexpr int kPVRows = 64;
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
// V tile row: the slice's 32 elements plus 16 bytes of padding
template <int KT>
struct PvTile {
    typedef typename KvElem<KT>::T E;
    static constexpr int kPitch = 32 + 16 / static_cast<int>(sizeof(E));
};
// Four consecutive stored elements of one V row, as read from the LDS tile.
template <int KT>
struct PvRaw;
template <>
struct PvRaw<kKvF32> {
    typedef float4 T;
    static __device__ __forceinline__ float at(const T& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }
};
template <>
struct PvRaw<kKvF16> {
    typedef half4v T;  // f16 operands go straight into v_fma_mix
    static __device__ __forceinline__ float at(const T& v, int k) { return static_cast<float>(v[k]); }
};
template <>
struct PvRaw<kKvQ8> {
    typedef uint32_t T;
    static __device__ __forceinline__ float at(const T& v, int k) {
        return static_cast<float>(static_cast<int8_t>(v >> (8 * k)));
    }
};
template <int KT>
__global__ __launch_bounds__(kPV) void attn_pv_chunk_kernel(int pos_arg, int B, int n_head, int group, int hd,
                                                            int kv_dim, int page_tokens, int pitch,
                                                            const void* const* __restrict__ pt_v,
                                                            const float* __restrict__ a, const int* __restrict__ d_pos,
                                                            float* __restrict__ out, int8_t* __restrict__ q8,
                                                            float* __restrict__ q8d, bool q8_op) {
    typedef typename KvElem<KT>::T E;
    __shared__ __align__(16) E s_v[kPVRows][PvTile<KT>::kPitch];  // V tile: rows x the slice's 32 elements
    __shared__ __align__(16) float s_at[32][kPVRows + 4];       // weights: token x tile row
    const int h = blockIdx.x, slice = blockIdx.y, t = threadIdx.x;
    const int b0 = blockIdx.z * 32, kh = h / group;
    const int pos0 = d_pos ? *d_pos : pos_arg;
    const int nmax = pos0 + min(B, b0 + 32);  // rows 0..nmax-1 are written (this chunk's included)
    const int tb = t >> 3, dq = (t & 7) * 4;  // chain: token b0 + tb, elements dq..dq+3 of the slice
    const int b = b0 + tb, nb = b < B ? pos0 + b + 1 : 0;
    const int vr = t >> 2, vc = (t & 3) * 8;  // V staging: tile row vr, elements vc..vc+7
    const int ar_ = t >> 3, ac = (t & 7) * 8;  // weight staging: token b0 + ar_, tile rows ac..ac+7
    const int ab = b0 + ar_, nab = ab < B ? pos0 + ab + 1 : 0;
    const float* arow = a + (static_cast<size_t>(min(ab, B - 1)) * n_head + h) * pitch;
    uint4 vreg[KT == kKvF32 ? 2 : 1];
    uint2 vreg8;
    float areg[8];
    auto fetch = [&](int r0) {
        const int r = r0 + vr < nmax ? r0 + vr : 0;  // rows past the written ones re-read row 0 (weight 0)
        const void* src = kv_elem_ptr<KT>(pt_v[r / page_tokens], r % page_tokens, kv_dim, kh * hd + slice * 32 + vc);
        if constexpr (KT == kKvF32) {
            vreg[0] = ld_global16(src);
            vreg[1] = ld_global16(static_cast<const float*>(src) + 4);
        } else if constexpr (KT == kKvF16) {
            vreg[0] = ld_global16(src);
        } else {
            vreg8 = ld_global8(src);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int rr = r0 + ac + j;
            areg[j] = rr < nab ? arow[rr] : 0.0f;
        }
    };
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    fetch(0);
    for (int r0 = 0; r0 < nmax; r0 += kPVRows) {
        if constexpr (KT == kKvF32) {
            *reinterpret_cast<uint4*>(&s_v[vr][vc]) = vreg[0];
            *reinterpret_cast<uint4*>(&s_v[vr][vc + 4]) = vreg[1];
        } else if constexpr (KT == kKvF16) {
            *reinterpret_cast<uint4*>(&s_v[vr][vc]) = vreg[0];
        } else {
            *reinterpret_cast<uint2*>(&s_v[vr][vc]) = vreg8;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s_at[ar_][ac + j] = areg[j];
        __syncthreads();
        if (r0 + kPVRows < nmax) fetch(r0 + kPVRows);
        // rows past nmax in the last tile carry weight 0 (areg) over finite rows: no-ops
        const int rows4 = min(kPVRows, (nmax - r0 + 3) & ~3);
        // 4-row steps with two register sets used in turn; every LDS read is
        // unconditional (a step past the last re-reads the last one, unused)
        // and the scheduling barriers keep the next set's reads ahead of the
        // current set's fmas, so the wait counts never cover them
        typedef typename PvRaw<KT>::T R;
        const int nst = rows4 >> 2;
        auto ld = [&](int st, float4& w, R (&v)[4]) {
            const int r = min(st, nst - 1) << 2;
            w = *reinterpret_cast<const float4*>(&s_at[tb][r]);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const R*>(&s_v[r + i][dq]);
        };
        auto step = [&](float (&c)[4], const float4& w4, const R (&v)[4]) {
            const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) c[k] = fmaf(w[i], PvRaw<KT>::at(v[i], k), c[k]);
        };
        float4 wa, wb;
        R va[4], vb[4];
        ld(0, wa, va);
        for (int st = 0; st < nst; st += 2) {
            ld(st + 1, wb, vb);
            __builtin_amdgcn_sched_barrier(0);
            step(acc, wa, va);
            __builtin_amdgcn_sched_barrier(0);
            ld(st + 2, wa, va);
            __builtin_amdgcn_sched_barrier(0);
            float nx[4] = {acc[0], acc[1], acc[2], acc[3]};  // the odd step, kept when it exists
            step(nx, wb, vb);
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = st + 1 < nst ? nx[k] : acc[k];
        }
        __syncthreads();
    }
    if (b >= B) return;  // whole 8-lane groups (one token) leave together
    const int col = h * hd + slice * 32 + dq;
    const size_t o = static_cast<size_t>(b) * n_head * hd + col;
    *reinterpret_cast<float4*>(out + o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    if (q8) {  // quantize_q8 of the token's 32-element block, 4 elements per lane
        const float m4 = fmaxf(fmaxf(fabsf(acc[0]), fabsf(acc[1])), fmaxf(fabsf(acc[2]), fabsf(acc[3])));
        const float mq = group_max<8>(m4);
        const float dqs = mq > 0.0f ? __fdiv_rn(mq, 127.0f) : 1.0f;
        const float id = __fdiv_rn(1.0f, dqs);
        uint32_t packed = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float rq = q_round_away(acc[k] * id, 127.0f);
            packed |= (static_cast<uint32_t>(static_cast<int>(rq)) & 0xffu) << (8 * k);
        }
        const size_t qo = q8_op ? q8_op_offset(b, col, static_cast<size_t>(n_head) * hd) : o;
        *reinterpret_cast<uint32_t*>(q8 + qo) = packed;
        if ((t & 7) == 0) q8d[o / 32] = dqs;
    }
}

}  // namespace

hipError_t launch_kv_write(int kv_type, void* const* pt_k, void* const* pt_v, const float* k, const float* v,
                           size_t pitch, const int* d_pos, size_t pos, size_t n_tokens, size_t kv_dim,
                           size_t page_tokens, hipStream_t st) {
    if (!n_tokens) return hipSuccess;
    const int ip = static_cast<int>(pitch), ipos = static_cast<int>(pos), nt = static_cast<int>(n_tokens);
    const int kd = static_cast<int>(kv_dim), pt = static_cast<int>(page_tokens);
    const unsigned blocks = static_cast<unsigned>((n_tokens * kv_dim + 255) / 256);
    switch (kv_type) {
    case kKvF32:
        kv_write_kernel<kKvF32><<<blocks, 256, 0, st>>>(pt_k, pt_v, k, v, ip, d_pos, ipos, nt, kd, pt);
        break;
    case kKvF16:
        kv_write_kernel<kKvF16><<<blocks, 256, 0, st>>>(pt_k, pt_v, k, v, ip, d_pos, ipos, nt, kd, pt);
        break;
    case kKvQ8:
        if (kv_dim % 4 || kv_dim > 4 * kKW * kKWV || pitch % 4) return hipErrorInvalidValue;
        kv_write_q8_kernel<<<dim3(static_cast<unsigned>(n_tokens), 2), kKW, 0, st>>>(pt_k, pt_v, k, v, ip, d_pos, ipos,
                                                                                  kd, pt);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
template <int KT>
hipError_t attn_typed(const void* const* pt_k, const void* const* pt_v, const float* q, size_t q_pitch, float* scores,
                      float* out, const int* d_pos, size_t pos, size_t max_pos, size_t B, size_t n_head,
                      size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st, int8_t* q8,
                      float* q8d, bool q8_op) {
    const int group = static_cast<int>(n_head / n_head_kv);
    const int pitch = static_cast<int>(max_pos);  // scores row pitch >= last position + 1
    const dim3 g1(static_cast<unsigned>(n_head), static_cast<unsigned>((max_pos + 63) / 64), static_cast<unsigned>(B));
    attn_scores_kernel<KT><<<g1, 64, hd * sizeof(float), st>>>(pt_k, q, static_cast<int>(q_pitch), scores, d_pos,
                                                               static_cast<int>(pos), static_cast<int>(n_head), group,
                                                               static_cast<int>(hd), static_cast<int>(kv_dim),
                                                               static_cast<int>(page_tokens), pitch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 g2(static_cast<unsigned>(n_head), static_cast<unsigned>((hd + 63) / 64), static_cast<unsigned>(B));
    attn_softmax_v_kernel<KT><<<g2, 64, (KT == kKvQ8 ? 2 : 1) * max_pos * sizeof(float), st>>>(
        pt_v, scores, out, d_pos, static_cast<int>(pos), static_cast<int>(n_head), group, static_cast<int>(hd),
        static_cast<int>(kv_dim), static_cast<int>(page_tokens), pitch, q8, q8d, q8_op);
    return hipGetLastError();
}

// Tuning override MVH_ATTN_SCORES_TILE=0: the per-(head, token) scores kernel for every chunk.
const bool kScoresTile = [] {
    const char* e = getenv("MVH_ATTN_SCORES_TILE");
    return !(e && atoi(e) == 0);
}();

template <int KT>
hipError_t attn_prefill_typed(const void* const* pt_k, const void* const* pt_v, const float* q, size_t q_pitch,
                              float* a_scratch, float* out, int8_t* q8, float* q8d, bool q8_op, const int* d_pos,
                              size_t pos, size_t max_pos, size_t B, size_t n_head, size_t n_head_kv, size_t hd,
                              size_t kv_dim, size_t page_tokens, hipStream_t st) {
    const int group = static_cast<int>(n_head / n_head_kv);
    const int pitch = static_cast<int>(max_pos);  // weight row pitch >= last position + 1
    if (kScoresTile && KT == kKvF16 && !d_pos && B >= 8 && B <= 32 && (hd == 128 || hd == 64) && q_pitch % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(q) & 15) == 0) {
        // F16 chunks of 8..32 tokens, q rows 16-byte aligned: K staged once per (head, 64-row block)
        const dim3 gs(static_cast<unsigned>(n_head), static_cast<unsigned>((pos + B + kTR - 1) / kTR));
        if (hd == 128)
            attn_scores_tile_kernel<128><<<gs, 256, 0, st>>>(pt_k, q, static_cast<int>(q_pitch), a_scratch,
                                                             static_cast<int>(pos), static_cast<int>(B),
                                                             static_cast<int>(n_head), group, static_cast<int>(kv_dim),
                                                             static_cast<int>(page_tokens), pitch);
        else
            attn_scores_tile_kernel<64><<<gs, 256, 0, st>>>(pt_k, q, static_cast<int>(q_pitch), a_scratch,
                                                            static_cast<int>(pos), static_cast<int>(B),
                                                            static_cast<int>(n_head), group, static_cast<int>(kv_dim),
                                                            static_cast<int>(page_tokens), pitch);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        attn_softmax_rows_kernel<<<dim3(static_cast<unsigned>(n_head), static_cast<unsigned>(B)), kSM, 0, st>>>(
            a_scratch, static_cast<int>(pos), static_cast<int>(n_head), pitch);
    } else {
    // one workgroup per (head, token): all of a chunk's workgroups resident
    // at once (a 128-wide compile-time head_dim that hoists the K loads, or
    // several tokens per workgroup sharing them, need more registers and run
    // slower)
    attn_scores_softmax_kernel<KT><<<dim3(static_cast<unsigned>(n_head), static_cast<unsigned>(B)), kSM,
                                     (hd + max_pos) * sizeof(float), st>>>(
        pt_k, pt_v, q, static_cast<int>(q_pitch), a_scratch, d_pos, static_cast<int>(pos), static_cast<int>(n_head),
        group, static_cast<int>(hd), static_cast<int>(kv_dim), static_cast<int>(page_tokens), pitch);
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const dim3 g(static_cast<unsigned>(n_head), static_cast<unsigned>(hd / 32), static_cast<unsigned>((B + 31) / 32));
    attn_pv_chunk_kernel<KT><<<g, kPV, 0, st>>>(static_cast<int>(pos), static_cast<int>(B), static_cast<int>(n_head),
                                                group, static_cast<int>(hd), static_cast<int>(kv_dim),
                                                static_cast<int>(page_tokens), pitch, pt_v, a_scratch, d_pos, out, q8,
                                                q8d, q8_op);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_attn(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q, size_t q_pitch,
                       float* scores, float* out, const int* d_pos, size_t pos, size_t max_pos, size_t B,
                       size_t n_head, size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st,
                       int8_t* q8, float* q8d, bool q8_op) {
    if (!B) return hipSuccess;
    if (q8 && (hd % 32 || !q8d || (q8_op && (n_head * hd) % 256))) return hipErrorInvalidValue;
    switch (kv_type) {
    case kKvF32:
        return attn_typed<kKvF32>(pt_k, pt_v, q, q_pitch, scores, out, d_pos, pos, max_pos, B, n_head, n_head_kv, hd,
                                  kv_dim, page_tokens, st, q8, q8d, q8_op);
    case kKvF16:
        return attn_typed<kKvF16>(pt_k, pt_v, q, q_pitch, scores, out, d_pos, pos, max_pos, B, n_head, n_head_kv, hd,
                                  kv_dim, page_tokens, st, q8, q8d, q8_op);
    case kKvQ8:
        return attn_typed<kKvQ8>(pt_k, pt_v, q, q_pitch, scores, out, d_pos, pos, max_pos, B, n_head, n_head_kv, hd,
                                 kv_dim, page_tokens, st, q8, q8d, q8_op);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_attn_prefill(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q,
                               size_t q_pitch, float* a_scratch, float* out, int8_t* q8, float* q8d, bool q8_op,
                               const int* d_pos, size_t pos, size_t max_pos, size_t B, size_t n_head,
                               size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st) {
    if (!B) return hipSuccess;
    if (hd % 32 || hd < 32 || (q8 && !q8d) || (q8_op && (n_head * hd) % 256)) return hipErrorInvalidValue;
    switch (kv_type) {
    case kKvF32:
        return attn_prefill_typed<kKvF32>(pt_k, pt_v, q, q_pitch, a_scratch, out, q8, q8d, q8_op, d_pos, pos, max_pos,
                                          B, n_head, n_head_kv, hd, kv_dim, page_tokens, st);
    case kKvF16:
        return attn_prefill_typed<kKvF16>(pt_k, pt_v, q, q_pitch, a_scratch, out, q8, q8d, q8_op, d_pos, pos, max_pos,
                                          B, n_head, n_head_kv, hd, kv_dim, page_tokens, st);
    case kKvQ8:
        return attn_prefill_typed<kKvQ8>(pt_k, pt_v, q, q_pitch, a_scratch, out, q8, q8d, q8_op, d_pos, pos, max_pos,
                                         B, n_head, n_head_kv, hd, kv_dim, page_tokens, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_attn_decode(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q,
                              float* scores, float* out, size_t pos, size_t n_head, size_t n_head_kv, size_t hd,
                              size_t kv_dim, size_t page_tokens, hipStream_t st) {
    if (hd % 32 == 0)  // V tiles staged in LDS by whole workgroups (latency-bound otherwise)
        return launch_attn_prefill(kv_type, pt_k, pt_v, q, n_head * hd, scores, out, nullptr, nullptr, false, nullptr,
                                   pos, pos + 1, 1, n_head, n_head_kv, hd, kv_dim, page_tokens, st);
    return launch_attn(kv_type, pt_k, pt_v, q, n_head * hd, scores, out, nullptr, pos, pos + 1, 1, n_head, n_head_kv,
                       hd, kv_dim, page_tokens, st);
}

hipError_t launch_attn_decode_fused(const float* q, const float* k, const float* v, const float* rope,
                                    const int* d_pos, uint16_t* kbase, uint16_t* vbase, size_t page_tokens,
                                    size_t page_stride, float* out, int8_t* q8, float* q8d, size_t n_head,
                                    size_t n_head_kv, size_t hd, size_t max_ctx, hipStream_t st, const L2Warm& warm,
                                    const L2Warm& warm2) {
    if (!attn_decode_fused_ok(hd, max_ctx, page_tokens)) return hipErrorInvalidValue;
    const int rows_alloc = static_cast<int>((max_ctx + page_tokens - 1) / page_tokens * page_tokens);
    // head dims 64 and 128 up to kHMaxCtx positions: the LDS-staged kernel,
    // NS slices per head.  Tuning override MVH_ATTN_NS: 1, 2 or 4 slices, 0 =
    // the register-staged kernel below.
    static const int ns_env = [] {
        const char* e = getenv("MVH_ATTN_NS");
        return e ? atoi(e) : -1;
    }();
    // default: four slices per head at head_dim 128 (tg128 562.9 against
    // 561.8 tok/s with two, 543 with one); at 64 four when no Q8 output is
    // written (16-element slices; the TinyLlama shape 1256.6 against 1250.9
    // tok/s with two), else two
    const int ns = ns_env >= 0 ? ns_env : hd == 128 || !q8 ? 4 : 2;
    // the LDS-staged kernel takes q, k and v as one buffer (the decode step's q|k|v)
    const bool qkv_one = k == q + n_head * hd && v == k + n_head_kv * hd && page_stride <= INT32_MAX;
    if ((hd == 128 || hd == 64) && max_ctx <= static_cast<size_t>(kHMaxCtx) && ns > 0 && qkv_one) {
        const int group = static_cast<int>(n_head / n_head_kv), kvd = static_cast<int>(n_head_kv * hd);
        auto warm_wgs = [&](size_t g) {
            return (warm.c1 > warm.c0 || warm2.c1 > warm2.c0) && g < kWarmWgs ? kWarmWgs - static_cast<unsigned>(g) : 0u;
        };
#define MVH_ATTN_HEAD(HD_, NS_)                                                                                   \
    attn_decode_head_kernel<HD_, NS_>                                                                             \
        <<<dim3(static_cast<unsigned>(n_head * NS_) + warm_wgs(n_head * NS_)), kHT, 0, st>>>(                     \
            static_cast<int>(n_head * NS_), group, static_cast<int>(page_tokens), kvd, rows_alloc,                \
            static_cast<int>(page_stride), q, rope, d_pos, kbase, vbase, out, q8, q8d, warm, warm2)
        if (hd == 128 && ns == 1) MVH_ATTN_HEAD(128, 1);
        else if (hd == 128 && ns == 4) MVH_ATTN_HEAD(128, 4);
        else if (hd == 128) MVH_ATTN_HEAD(128, 2);
        else if (ns == 1) MVH_ATTN_HEAD(64, 1);
        else if (ns == 4 && !q8) MVH_ATTN_HEAD(64, 4);  // 16-element slices: no Q8 blocks of the output
        else MVH_ATTN_HEAD(64, 2);
#undef MVH_ATTN_HEAD
        return hipGetLastError();
    }
    const int sw = hd % 32 == 0 ? 32 : hd % 16 == 0 ? 16 : 8;
    const int nslice = static_cast<int>(hd) / sw;
    const int ctx_pad = static_cast<int>((max_ctx + 3) / 4 * 4);
    const size_t lds = (3 * hd + ctx_pad) * sizeof(float) + static_cast<size_t>(kRVP) * sw * sizeof(uint16_t);
    const dim3 grid(static_cast<unsigned>(n_head * nslice));
    const int group = static_cast<int>(n_head / n_head_kv), kvd = static_cast<int>(n_head_kv * hd);
#define MVH_ATTN_FUSED(SW_, HD_)                                                                                     \
    attn_decode_fused_kernel<SW_, HD_><<<grid, kAT, lds, st>>>(q, k, v, rope, d_pos, kbase, vbase,                 \
                                                               static_cast<int>(page_tokens), page_stride, rows_alloc, \
                                                               out, q8, q8d, group, static_cast<int>(hd), kvd,        \
                                                               ctx_pad, nslice)
    if (sw == 32 && hd == 128) MVH_ATTN_FUSED(32, 128);
    else if (sw == 32 && hd == 64) MVH_ATTN_FUSED(32, 64);
    else if (sw == 32) MVH_ATTN_FUSED(32, 0);
    else if (sw == 16) MVH_ATTN_FUSED(16, 0);
    else MVH_ATTN_FUSED(8, 0);
#undef MVH_ATTN_FUSED
    return hipGetLastError();
}

bool attn_decode_fused_ok(size_t hd, size_t max_ctx, size_t page_tokens) {
    const size_t sw = hd % 32 == 0 ? 32 : hd % 16 == 0 ? 16 : 8;
    const size_t lds = (3 * hd + (max_ctx + 3) / 4 * 4) * sizeof(float) + kRVP * sw * sizeof(uint16_t);
    return hd >= 8 && hd % 8 == 0 && hd <= 2 * kAT && max_ctx >= 1 && page_tokens >= 1 &&
           (max_ctx + page_tokens - 1) / page_tokens <= kMaxPages && lds <= 56 * 1024;
}

}  // namespace mvh
