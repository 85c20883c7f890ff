// mvh_device.hpp -- device helpers shared by the gfx950 kernels.
//
// All HIP sources are compiled with -ffp-contract=off: every fused
// multiply-add is written as fmaf()/fma(), every other product rounds on its
// own, so each kernel reproduces the reference's operation order exactly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace mvh {

constexpr int kWave = 64;

// ---- fp16 ------------------------------------------------------------------

// Exact binary16 -> binary32 (v_cvt_f32_f16; f16 denormals are kept, as in
// fp16_to_fp32, src/gguf.cpp:110-119).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// The reference's binary32 -> binary16 routine (src/gguf_kernels.cpp:242):
// ties away from zero, and a mantissa carry is OR-ed (not added) into the
// exponent field.  The F16 KV cache must hold exactly these bits, so this is
// integer code, not v_cvt_f16_f32.
// The reference's branches are all evaluated and one is selected: as branches
// every conversion costs a few exec-mask round trips even when all lanes
// agree.
__device__ __forceinline__ uint16_t f2h_ref(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u, mant = x & 0x7fffffu;
    const int e = static_cast<int>((x >> 23) & 0xffu) - 112;  // -127 + 15
    const uint32_t sh = static_cast<uint32_t>(min(max(1 - e, 0), 31));  // 1..11 where used
    const uint32_t sub = sign + ((((mant | 0x800000u) >> sh) + 0x1000u) >> 13);            // -10 <= e <= 0
    const uint32_t nrm = sign | (static_cast<uint32_t>(e) << 10) | ((mant + 0x1000u) >> 13);  // 1 <= e <= 30
    const uint32_t r = e <= 0 ? (e < -10 ? sign : sub) : (e >= 31 ? (sign | 0x7c00u) : nrm);
    return static_cast<uint16_t>(r);
}

// ---- correctly rounded sqrt ---------------------------------------------------

// sqrtf rounded to nearest even.  HIP's __fsqrt_rn is the native v_sqrt_f32
// (within 1 ulp) unless OCML_BASIC_ROUNDED_OPERATIONS is defined; the
// llvm.sqrt.f32 lowering behind __builtin_sqrtf is correctly rounded under
// hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt (checked equal to
// the host's sqrtf on every positive normal float on gfx950).
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// ---- cross-lane --------------------------------------------------------------

// ds_swizzle in bit-mask mode (offset[15]=0): lane' = ((lane & and) | or) ^ xor
// inside each group of 32 lanes.  No LDS memory is touched.
template <int XOR>
__device__ __forceinline__ int swz_xor(int v) {
    return __builtin_amdgcn_ds_swizzle(v, (XOR << 10) | 0x1f);
}
template <int XOR>
__device__ __forceinline__ float swz_xor(float v) {
    return __int_as_float(swz_xor<XOR>(__float_as_int(v)));
}
template <int XOR>
__device__ __forceinline__ double swz_xor(double v) {
    int lo = __double2loint(v), hi = __double2hiint(v);
    return __hiloint2double(swz_xor<XOR>(hi), swz_xor<XOR>(lo));
}

// DPP lane moves (VALU operand modifiers, no LDS round trip): quad_perm
// [1,0,3,2] = 0xb1 and [2,3,0,1] = 0x4e, row_half_mirror = 0x141 (lane i of
// each 8 reads lane 7 - i), row_mirror = 0x140 (lane i of each 16 reads 15 - i).
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(dpp_mov<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_mov(double v) {
    return __hiloint2double(dpp_mov<CTRL>(__double2hiint(v)), dpp_mov<CTRL>(__double2loint(v)));
}

// Reductions over aligned groups of N lanes (N = 2..32), result in every lane
// of the group (every lane of it must be active): the quad steps, then the
// half-row and row mirrors pair lanes holding the reductions of disjoint
// halves; across 16-lane rows a swizzle.
template <int N>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (N >= 2) v = fmaxf(v, dpp_mov<0xb1>(v));
    if constexpr (N >= 4) v = fmaxf(v, dpp_mov<0x4e>(v));
    if constexpr (N >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if constexpr (N >= 32) v = fmaxf(v, swz_xor<16>(v));
    return v;
}
template <int N>
__device__ __forceinline__ int group_sum(int v) {
    if constexpr (N >= 2) v += dpp_mov<0xb1>(v);
    if constexpr (N >= 4) v += dpp_mov<0x4e>(v);
    if constexpr (N >= 8) v += dpp_mov<0x141>(v);
    if constexpr (N >= 16) v += dpp_mov<0x140>(v);
    if constexpr (N >= 32) v += swz_xor<16>(v);
    return v;
}
// Double sum over the full wave, the same value in every lane: DPP within each
// 16-lane row (the lanes of a row then hold equal sums), then the four rows
// read and added in row order.
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_mov<0xb1>(v);
    v += dpp_mov<0x4e>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    const int lo = __double2loint(v), hi = __double2hiint(v);
    auto rd = [&](int l) { return __hiloint2double(__builtin_amdgcn_readlane(hi, l), __builtin_amdgcn_readlane(lo, l)); };
    return ((rd(0) + rd(16)) + rd(32)) + rd(48);
}
// Max over the full wave, in every lane.
__device__ __forceinline__ float wave_max_all(float v) {
    v = group_max<16>(v);
    auto rd = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
    return fmaxf(fmaxf(rd(0), rd(16)), fmaxf(rd(32), rd(48)));
}

// clamp(lround(v), -lim, lim) as the reference's x86 build evaluates it: a
// finite v rounds half away from zero and clamps; a non-finite v (a scale so
// small that 1/d overflowed, or 0/0) converts to LONG_MIN, i.e. -lim.
__device__ __forceinline__ float q_round_away(float v, float lim) {
    return __builtin_isfinite(v) ? fminf(fmaxf(roundf(v), -lim), lim) : -lim;
}
// clamp((int)nearbyint(v), lo, hi) likewise: round half to even, a non-finite v
// converts to INT_MIN, i.e. lo.
__device__ __forceinline__ float q_round_even(float v, float lo, float hi) {
    return __builtin_isfinite(v) ? fminf(fmaxf(__builtin_rintf(v), lo), hi) : lo;
}

// quantize_q8 (src/gguf_kernels.cpp:160-172) for one 32-element block held as
// 4 consecutive floats in each lane of an aligned group of 8 lanes:
//   mx = max|z| (exact in any order), d = mx > 0 ? mx/127 : 1, inv = 1/d,
//   q = clamp(round_half_away(z*inv), -127, 127).
// Returns the lane's 4 int8 values packed; d and the block sum s = sum(q)
// are the same in all 8 lanes.  Every lane of the group must call it.
__device__ __forceinline__ uint32_t quantize_q8_x4(float4 v, float& d, int& s) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = group_max<8>(m);
    d = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, d);
    auto qz = [&](float z) { return static_cast<int>(q_round_away(z * inv, 127.0f)); };
    const int q0 = qz(v.x), q1 = qz(v.y), q2 = qz(v.z), q3 = qz(v.w);
    s = group_sum<8>(q0 + q1 + q2 + q3);
    return (static_cast<uint32_t>(q0) & 0xffu) | ((static_cast<uint32_t>(q1) & 0xffu) << 8) |
           ((static_cast<uint32_t>(q2) & 0xffu) << 16) | (static_cast<uint32_t>(q3) << 24);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight binary16 values of a 16-byte load; fmaf(a, float(h[e]), c) on them
// compiles to v_fma_mix_f32 (exact f16->f32 conversion fused into the FMA,
// one rounding, as cvt + fmaf).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ half8 as_half8(uint4 w) {
    const u32x4 v = {w.x, w.y, w.z, w.w};
    return __builtin_bit_cast(half8, v);
}

// 16-byte load through a pointer that is known to address global memory but
// was itself loaded from memory (a page table): the address-space cast makes
// it a global_load instead of a flat_load, whose LDS/VMEM counter coupling
// serialises consecutive loads.
__device__ __forceinline__ uint4 ld_global16(const void* p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)(reinterpret_cast<uintptr_t>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A uniform int read by a vector load in every lane (the address offset by a
// zero the compiler cannot see through), where a scalar load would share its
// wait counter with the kernel's argument loads: the first wait for an
// argument would then also wait for this load's trip to memory.  Vector
// loads complete in issue order, so its value is waited for where it is used.
__device__ __forceinline__ int ld_global_lanes(const int* p) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return *(const __attribute__((address_space(1))) int*)(reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(z));
}

// 8-byte form of ld_global16.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld_global8(const void* p) {
    const u32x2 v = *(const __attribute__((address_space(1))) u32x2*)(reinterpret_cast<uintptr_t>(p));
    return make_uint2(v.x, v.y);
}

// 16-byte streaming load (weights are read once per call: nontemporal hint).
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// L2 warm-up of a coming decode GEMV's weights by spare workgroups of a
// launch before it (a norm or the attention, which leave most CUs and HBM
// idle).  The GEMV's workgroup c reads the contiguous chunk [c*chunk,
// (c+1)*chunk) of base and runs on XCD c % 8 (a launch's workgroups go to the
// eight XCDs in turn, each XCD with its own L2), so the warm-up workgroup `id`
// (of `count` such workgroups starting at grid index `first`, 1-D grid) reads
// the chunks c in [c0, c1) with c % 8 == id % 8 that fall to it: each chunk
// lands in the L2 its reader looks in.  Loads only; their values are consumed
// by an empty asm statement.  c0 == c1: nothing to warm.
struct L2Warm {
    const uint8_t* base = nullptr;
    unsigned chunk = 0;  // bytes, a multiple of 16
    unsigned c0 = 0, c1 = 0;
};

template <int NT>
__device__ __forceinline__ void l2_warm(const L2Warm& w, int id, int first, int count) {
    const int x = id & 7;
    const int fx = first + ((x - first) & 7);  // first warm-up workgroup on XCD x
    const int nx = (first + count - 1 - fx) / 8 + 1;
    const int c16 = static_cast<int>(w.chunk / 16);
    const unsigned c_x = w.c0 + ((static_cast<unsigned>(x) - w.c0) & 7u);  // first chunk of [c0, c1) on XCD x
    for (unsigned c = c_x + 8u * static_cast<unsigned>((id - fx) >> 3); c < w.c1; c += 8u * static_cast<unsigned>(nx)) {
        const uint4* src = reinterpret_cast<const uint4*>(w.base + static_cast<size_t>(c) * w.chunk);
        for (int i0 = static_cast<int>(threadIdx.x); i0 < c16; i0 += 8 * NT) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u * NT;
                v[u] = i < c16 ? src[i] : make_uint4(0u, 0u, 0u, 0u);
            }
            uint32_t acc = 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
            asm volatile("" ::"v"(acc));
        }
    }
}

// Bytes [2*sel, 2*sel+4) of the 8-byte value hi:lo (v_alignbyte_b32).
__device__ __forceinline__ uint32_t align16(uint32_t hi, uint32_t lo) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// Q8 activations of B tokens x K elements (K % 256 == 0) in the operand
// order of the prefill GEMM's int8 MFMA: 16-token slabs; within a slab, per
// 256-element chunk, per block j and 8-byte quarter h, the 16 tokens' bytes
// 8h .. 8h+7 of block j -- the A operand of one v_mfma_i32_16x16x32_i8 as 512
// contiguous bytes.  Four consecutive elements (k % 4 == 0) stay contiguous.
__host__ __device__ constexpr size_t q8_op_offset(size_t t, size_t k, size_t K) {
    return (t / 16) * 16 * K + (k / 256) * 4096 + ((k % 256) / 32 * 4 + (k % 32) / 8) * 128 + (t % 16) * 8 + k % 8;
}
// bytes of that layout for B tokens (the last slab is whole)
__host__ __device__ constexpr size_t q8_op_bytes(size_t B, size_t K) { return (B + 15) / 16 * 16 * K; }

// One row of LlamaModel::rmsnorm (src/llama_model.cpp:237) by a workgroup of
// kT threads, D <= 4 * kT * kV, D % 32 == 0 (D % 256 == 0 with q_op):
// x += add (when add != null), ss = sum of x*x in double,
// inv = 1/sqrtf(float(ss/D) + eps), n = (x*inv)*w, and (q != null) the Q8
// activation of n (quantize_q8, bit-exact; row-major, or in the prefill
// GEMM's operand order when q_op).  Thread t owns float4s t, t + kT, ...; the
// double sum is added as a tree (per thread, per wave, then the waves in
// order), not in the reference's element order: the two can differ only when
// the exact sum of squares lies within ~1e-15 (relative) of an f32 rounding
// boundary of ss/D.  red: kT/64 doubles of LDS.  Every thread must call it.
template <int kT, int kV>
__device__ __forceinline__ void rmsnorm_row(float* __restrict__ xr_, const float* __restrict__ add,
                                            const float* __restrict__ w, float* __restrict__ n_row,
                                            int8_t* __restrict__ q, float* __restrict__ qd, size_t row, int D,
                                            float eps, bool q_op, double* red) {
    const int t = threadIdx.x;
    float4* xr = reinterpret_cast<float4*>(xr_);
    const float4* ar = reinterpret_cast<const float4*>(add);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const int D4 = D / 4;
    // one memory round trip: x, the residual and the norm weights together
    float4 v[kV], g[kV], a[kV];
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int i = t + k * kT;
        v[k] = g[k] = a[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < D4) {
            v[k] = xr[i];
            g[k] = w4[i];
            if (ar) a[k] = ar[i];
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int i = t + k * kT;
        if (i >= D4) continue;
        if (ar) {
            v[k] = make_float4(v[k].x + a[k].x, v[k].y + a[k].y, v[k].z + a[k].z, v[k].w + a[k].w);
            xr[i] = v[k];
        }
        ss = fma(static_cast<double>(v[k].x), static_cast<double>(v[k].x), ss);
        ss = fma(static_cast<double>(v[k].y), static_cast<double>(v[k].y), ss);
        ss = fma(static_cast<double>(v[k].z), static_cast<double>(v[k].z), ss);
        ss = fma(static_cast<double>(v[k].w), static_cast<double>(v[k].w), ss);
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    ss = red[0];
#pragma unroll
    for (int k = 1; k < kT / 64; ++k) ss += red[k];
    const float inv = __fdiv_rn(1.0f, sqrt_rn(static_cast<float>(ss / static_cast<double>(D)) + eps));
    float4* nr = reinterpret_cast<float4*>(n_row);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int i = t + k * kT;
        if (k * kT >= D4) break;  // uniform; D4 % 8 == 0: 8-lane groups are whole blocks
        const float4 o = make_float4((v[k].x * inv) * g[k].x, (v[k].y * inv) * g[k].y, (v[k].z * inv) * g[k].z,
                                     (v[k].w * inv) * g[k].w);
        if (i < D4) nr[i] = o;
        if (q) {
            float d;
            int s;
            const uint32_t packed = quantize_q8_x4(o, d, s);
            if (i < D4) {
                if (q_op)
                    *reinterpret_cast<uint32_t*>(q + q8_op_offset(row, 4 * static_cast<size_t>(i), D)) = packed;
                else
                    reinterpret_cast<uint32_t*>(q + row * D)[i] = packed;
                if ((i & 7) == 0) qd[row * (D / 32) + (i >> 3)] = d;
            }
        }
    }
}

// ---- paged KV cache element types ------------------------------------------
//
// PagedKVCache's KVCacheType (F32, F16, Q8 in that order).  One page of K (or
// V) is [page_tokens][kv_dim] elements of the type: float, fp16 bits, or int8;
// a Q8 page then holds its page_tokens float row scales at a 16-byte aligned
// offset after the elements.
enum KvType : int { kKvF32 = 0, kKvF16 = 1, kKvQ8 = 2 };
__host__ __device__ constexpr size_t kv_elem_bytes(int kt) { return kt == kKvF32 ? 4 : kt == kKvF16 ? 2 : 1; }
__host__ __device__ constexpr size_t kv_scale_offset(size_t page_tokens, size_t kv_dim) {
    return (page_tokens * kv_dim + 15) / 16 * 16;
}
__host__ __device__ constexpr size_t kv_page_bytes(int kt, size_t page_tokens, size_t kv_dim) {
    return kt == kKvQ8 ? kv_scale_offset(page_tokens, kv_dim) + 4 * page_tokens : page_tokens * kv_dim * kv_elem_bytes(kt);
}
// bytes PagedKVCache::bytes_allocated counts per page index (K and V; the
// Q8 alignment padding is not counted)
__host__ __device__ constexpr size_t kv_page_pair_bytes_ref(int kt, size_t page_tokens, size_t kv_dim) {
    return 2 * (page_tokens * kv_dim * kv_elem_bytes(kt) + (kt == kKvQ8 ? 4 * page_tokens : 0));
}

template <int KT>
struct KvElem;
template <>
struct KvElem<kKvF32> {
    typedef float T;
};
template <>
struct KvElem<kKvF16> {
    typedef uint16_t T;
};
template <>
struct KvElem<kKvQ8> {
    typedef int8_t T;
};

// Element e of a stored row, converted exactly to float.
template <int KT>
__device__ __forceinline__ float kv_to_f(const void* row, int e) {
    if constexpr (KT == kKvF32) return static_cast<const float*>(row)[e];
    else if constexpr (KT == kKvF16) return h2f(static_cast<const uint16_t*>(row)[e]);
    else return static_cast<float>(static_cast<const int8_t*>(row)[e]);
}

// Eight consecutive stored elements (16/8/4-byte aligned for F32/F16/Q8) of
// a row: kv_raw8 loads them as stored, kv_cvt8 converts them exactly.
template <int KT>
struct KvRaw8 {
    uint4 a, b;  // F32: two 16-byte halves
};
template <>
struct KvRaw8<kKvF16> {
    uint4 a;
};
template <>
struct KvRaw8<kKvQ8> {
    uint2 a;
};
template <int KT>
__device__ __forceinline__ KvRaw8<KT> kv_raw8(const void* row, int e) {
    KvRaw8<KT> r;
    if constexpr (KT == kKvF32) {
        const float* p = static_cast<const float*>(row) + e;
        r.a = ld_global16(p);
        r.b = ld_global16(p + 4);
    } else if constexpr (KT == kKvF16) {
        r.a = ld_global16(static_cast<const uint16_t*>(row) + e);
    } else {
        r.a = ld_global8(static_cast<const int8_t*>(row) + e);
    }
    return r;
}
template <int KT>
__device__ __forceinline__ void kv_cvt8(const KvRaw8<KT>& r, float (&f)[8]) {
    if constexpr (KT == kKvF32) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = __uint_as_float(w[j]);
    } else if constexpr (KT == kKvF16) {
        const half8 h = as_half8(r.a);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = static_cast<float>(h[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            f[j] = static_cast<float>(static_cast<int8_t>((j < 4 ? r.a.x : r.a.y) >> (8 * (j & 3))));
    }
}
template <int KT>
__device__ __forceinline__ void kv_load8(const void* row, int e, float (&f)[8]) {
    kv_cvt8<KT>(kv_raw8<KT>(row, e), f);
}

// Q8 row scale of slot `slot` of a page (1 for the other types).
template <int KT>
__device__ __forceinline__ float kv_row_scale(const void* page, int slot, int page_tokens, int kv_dim) {
    if constexpr (KT == kKvQ8)
        return reinterpret_cast<const float*>(static_cast<const uint8_t*>(page) +
                                              kv_scale_offset(page_tokens, kv_dim))[slot];
    else return 1.0f;
}

}  // namespace mvh
