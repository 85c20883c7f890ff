/*
 * mv_oracle.c -- CPU restatement of MemVanta's quantized-matmul + paged KV
 * attention path.  TEST INFRASTRUCTURE ONLY: used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the
 * product.  Compiled with -ffp-contract=off: every fused multiply-add the
 * reference's GCC build performs is an explicit fmaf() here, every other
 * product is rounded on its own.  Citations are MemVanta file:line.
 */
#define _GNU_SOURCE
#include "mv_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static void set_err(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
const char* mvo_last_error(void) { return g_err; }

/* ------------------------------------------------------------------ */
/* fp16 <-> fp32                                                        */
/* ------------------------------------------------------------------ */

/* Exact binary16 -> binary32, subnormals normalised (src/gguf.cpp:110-119). */
float mvo_fp16_to_fp32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) & 1u, e = (uint32_t)(h >> 10) & 0x1fu, f = h & 0x3ffu, bits;
    if (e == 0) {
        if (f == 0) {
            bits = s << 31;
        } else {
            uint32_t ee = 113; /* 127 - 15 + 1 */
            while ((f & 0x400u) == 0) { f <<= 1; --ee; }
            bits = (s << 31) | (ee << 23) | ((f & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = (s << 31) | 0x7f800000u | (f << 13);
    } else {
        bits = (s << 31) | ((e + 112u) << 23) | (f << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* The reference's binary32 -> binary16 routine (src/gguf_kernels.cpp:242).
 * It is NOT round-to-nearest-even: it adds half an ulp (ties away from zero)
 * and, when the mantissa carry overflows, ORs the carry into the exponent
 * field instead of adding it.  The F16 KV cache stores exactly these bits. */
uint16_t mvo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, mant = x & 0x7fffffu;
    int exp = (int)((x >> 23) & 0xffu) - 127 + 15;
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)sign;
        mant = (mant | 0x800000u) >> (1 - exp);
        return (uint16_t)(sign + ((mant + 0x1000u) >> 13));
    }
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)exp << 10) | ((mant + 0x1000u) >> 13));
}

void mvo_fp32_to_fp16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mvo_fp32_to_fp16(x[i]);
}

void mvo_fp32_to_fp16_bits(uint32_t first, uint64_t count, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        uint32_t b = first + (uint32_t)i;
        float f;
        memcpy(&f, &b, 4);
        out[i] = mvo_fp32_to_fp16(f);
    }
}

uint64_t mvo_fp32_to_fp16_count_mismatch(uint32_t first, uint64_t count, const uint16_t* out) {
    uint64_t bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        uint32_t b = first + (uint32_t)i;
        float f;
        memcpy(&f, &b, 4);
        bad += mvo_fp32_to_fp16(f) != out[i];
    }
    return bad;
}

static inline float blk_d(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return mvo_fp16_to_fp32(h);
}

/* ------------------------------------------------------------------ */
/* activation quantization                                              */
/* ------------------------------------------------------------------ */

/* quantize_q8 (src/gguf_kernels.cpp:160-172): per 32-block, mx = max|z|,
 * d = mx > 0 ? mx/127 : 1, inv = 1/d, q = clamp(lround(z*inv), -127, 127).
 * The scale is kept as f32 (not the 34-byte GGUF Q8_0 block). */
int mvo_quantize_q8(const float* x, size_t cols, int8_t* q, float* d) {
    if (cols % 32) {
        set_err("Q8 activation quantization requires cols multiple of 32");
        return -1;
    }
    for (size_t bi = 0; bi < cols / 32; ++bi) {
        const float* z = x + bi * 32;
        float mx = 0.0f;
        for (int k = 0; k < 32; ++k) {
            float a = fabsf(z[k]);
            if (mx < a) mx = a;
        }
        float dd = mx > 0 ? mx / 127.0f : 1.0f;
        float inv = 1.0f / dd;
        d[bi] = dd;
        for (int k = 0; k < 32; ++k) {
            long r = lroundf(z[k] * inv);
            if (r < -127) r = -127;
            if (r > 127) r = 127;
            q[bi * 32 + k] = (int8_t)r;
        }
    }
    return 0;
}

/* quantize_activations_q8 (src/gguf_kernels.cpp:174-178): row by row. */
int mvo_quantize_act_q8(const float* x, size_t batch, size_t cols, int8_t* q, float* d) {
    for (size_t b = 0; b < batch; ++b)
        if (mvo_quantize_q8(x + b * cols, cols, q + b * cols, d + b * (cols / 32))) return -1;
    return 0;
}

/* ------------------------------------------------------------------ */
/* row dots                                                              */
/* ------------------------------------------------------------------ */

/* Sum of 8 lane accumulators the way `float s=0; for(v:tmp) s+=v;` does. */
static inline float hsum8_from_zero(const float t[8]) {
    float s = 0.0f;
    for (int j = 0; j < 8; ++j) s = s + t[j];
    return s;
}
/* `t[0]+t[1]+...+t[7]` left to right. */
static inline float hsum8(const float t[8]) {
    float s = t[0];
    for (int j = 1; j < 8; ++j) s = s + t[j];
    return s;
}

/* Exact int dot of one Q4_0 block with 32 int8 activations
 * (dot_q4_q8_block + dot_i8_16, src/gguf_kernels.cpp:148-158,180-188).
 * Element i < 16 is (qs[i]&15)-8, element 16+i is (qs[i]>>4)-8. */
static inline int dot_q4_q8_block(const uint8_t* blk, const int8_t* aq) {
    const uint8_t* qs = blk + 2;
    int s = 0;
    for (int i = 0; i < 16; ++i) {
        s += ((int)(qs[i] & 15) - 8) * (int)aq[i];
        s += ((int)(qs[i] >> 4) - 8) * (int)aq[16 + i];
    }
    return s;
}

/* dot_q4_q8 (src/gguf_kernels.cpp:189): the GCC build contracts
 * `sum += d_w*d_a*float(isum)` to fma(d_w*d_a, float(isum), sum). */
float mvo_dot_q4_q8(const uint8_t* w, const int8_t* aq, const float* ad, size_t nb) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = w + 18 * b;
        float p = blk_d(blk) * ad[b];
        sum = fmaf(p, (float)dot_q4_q8_block(blk, aq + 32 * b), sum);
    }
    return sum;
}

/* dot_q4_0_fp32 (src/gguf_kernels.cpp:93-109): per block, lane j of 8
 * accumulates elements j, 8+j, 16+j, 24+j by fma from zero; s = 0+t0+..+t7;
 * sum = fma(d, s, sum). */
float mvo_dot_q4_0_fp32(const uint8_t* w, const float* x, size_t n) {
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t* blk = w + 18 * b;
        const uint8_t* qs = blk + 2;
        float d = blk_d(blk);
        float t[8] = {0};
        for (int h = 0; h < 2; ++h)
            for (int k = 0; k < 16; k += 8)
                for (int j = 0; j < 8; ++j) {
                    int qi = h ? (qs[k + j] >> 4) - 8 : (qs[k + j] & 15) - 8;
                    t[j] = fmaf((float)qi, x[b * 32 + h * 16 + k + j], t[j]);
                }
        sum = fmaf(d, hsum8_from_zero(t), sum);
    }
    return sum;
}

/* dot_q8_0_fp32 (src/gguf_kernels.cpp:111-120): lane j accumulates elements
 * j, 8+j, 16+j, 24+j; s = 0+t0+..+t7; sum = fma(d, s, sum). */
float mvo_dot_q8_0_fp32(const uint8_t* w, const float* x, size_t n) {
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t* blk = w + 34 * b;
        const int8_t* qs = (const int8_t*)(blk + 2);
        float d = blk_d(blk);
        float t[8] = {0};
        for (int k = 0; k < 32; k += 8)
            for (int j = 0; j < 8; ++j) t[j] = fmaf((float)qs[k + j], x[b * 32 + k + j], t[j]);
        sum = fmaf(d, hsum8_from_zero(t), sum);
    }
    return sum;
}

/* q6_k_value (src/gguf_kernels.cpp:122-136): element i of a 210-byte Q6_K
 * block {ql[128], qh[64], scales[16], d}. */
int mvo_q6_k_value(const uint8_t* b, size_t i) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    size_t row32 = i / 32, j = i % 32, group = row32 / 4, local = row32 % 4;
    size_t ql_index = group * 64 + (local % 2) * 32 + j;
    unsigned ql_shift = local < 2 ? 0u : 4u;
    size_t qh_index = group * 32 + j;
    unsigned qh_shift = (unsigned)(local * 2);
    int lo = (ql[ql_index] >> ql_shift) & 0x0f;
    int hi = (qh[qh_index] >> qh_shift) & 0x03;
    return (lo | (hi << 4)) - 32;
}

/* dot_q6_k_fp32 (src/gguf_kernels.cpp:138-146): w = (d*sc[i/16])*q in f32,
 * sum in double in element order (the double product is exact). */
float mvo_dot_q6_k_fp32(const uint8_t* w, const float* x, size_t n) {
    double sum = 0.0;
    for (size_t bi = 0; bi < n / 256; ++bi) {
        const uint8_t* b = w + 210 * bi;
        const int8_t* sc = (const int8_t*)(b + 192);
        float d = blk_d(b + 208);
        const float* xv = x + bi * 256;
        for (size_t i = 0; i < 256; ++i) {
            float wv = (d * (float)sc[i / 16]) * (float)mvo_q6_k_value(b, i);
            sum = sum + (double)wv * (double)xv[i];
        }
    }
    return (float)sum;
}

/* dot_f32_simd (src/gguf_kernels.cpp:228-234): 8 fma lanes, t0+..+t7, then
 * the tail. */
float mvo_dot_f32(const float* a, const float* b, size_t n) {
    float t[8] = {0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) t[j] = fmaf(a[i + j], b[i + j], t[j]);
    float s = hsum8(t);
    /* the scalar tail `s += a*b` as the compiled reference runs it: GCC -O3
     * vectorizes it 4 elements at a time (products rounded, adds in order),
     * the last n % 4 are fused (pinned by the reference's F32 KV dots at every
     * tail length 1..7) */
    for (; i + 4 <= n; i += 4)
        for (int j = 0; j < 4; ++j) s = s + a[i + j] * b[i + j];
    for (; i < n; ++i) s = fmaf(a[i], b[i], s);
    return s;
}

/* q4_row_batch4_fp32 (src/gguf_kernels.cpp:191-199): 4 tokens share one
 * weight decode; q = float(qi)*d is rounded, acc = fma(q, x, acc); the 8 lane
 * accumulators persist over all blocks; out = t0+t1+..+t7. */
static void q4_row_batch4(const uint8_t* w, const float* x, size_t stride, size_t nb, float out[4]) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = w + 18 * b;
        const uint8_t* qs = blk + 2;
        float d = blk_d(blk);
        for (int h = 0; h < 2; ++h)
            for (int k = 0; k < 16; k += 8)
                for (int j = 0; j < 8; ++j) {
                    int qi = h ? (qs[k + j] >> 4) - 8 : (qs[k + j] & 15) - 8;
                    float q = (float)qi * d;
                    size_t off = b * 32 + h * 16 + k + j;
                    for (int t = 0; t < 4; ++t) acc[t][j] = fmaf(q, x[t * stride + off], acc[t][j]);
                }
    }
    for (int t = 0; t < 4; ++t) out[t] = hsum8(acc[t]);
}

/* q8_row_batch4_fp32 (src/gguf_kernels.cpp:201-209). */
static void q8_row_batch4(const uint8_t* w, const float* x, size_t stride, size_t nb, float out[4]) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = w + 34 * b;
        const int8_t* qs = (const int8_t*)(blk + 2);
        float d = blk_d(blk);
        for (int k = 0; k < 32; k += 8)
            for (int j = 0; j < 8; ++j) {
                float q = (float)qs[k + j] * d;
                size_t off = b * 32 + k + j;
                for (int t = 0; t < 4; ++t) acc[t][j] = fmaf(q, x[t * stride + off], acc[t][j]);
            }
    }
    for (int t = 0; t < 4; ++t) out[t] = hsum8(acc[t]);
}

/* ------------------------------------------------------------------ */
/* tensor-level entry points                                            */
/* ------------------------------------------------------------------ */

static size_t row_bytes(int type, size_t cols) {
    switch (type) {
        case MVO_F32: return cols * 4;
        case MVO_F16: return cols * 2;
        case MVO_Q4_0: return cols / 32 * 18;
        case MVO_Q8_0: return cols / 32 * 34;
        case MVO_Q6_K: return cols / 256 * 210;
        default: return 0;
    }
}

static float dot_f16_double(const uint16_t* a, const float* x, size_t cols) {
    double s = 0;
    for (size_t c = 0; c < cols; ++c) s = s + (double)mvo_fp16_to_fp32(a[c]) * (double)x[c];
    return (float)s;
}

/* One (row, fp32-activation vector) product with the dispatch of
 * tensor_matmul_batch (src/gguf_kernels.cpp:255-259). */
static float fp32_row_dot(const uint8_t* w, int type, size_t cols, size_t r, const float* xv) {
    const uint8_t* row = w + r * row_bytes(type, cols);
    switch (type) {
        case MVO_Q4_0: return mvo_dot_q4_0_fp32(row, xv, cols);
        case MVO_Q8_0: return mvo_dot_q8_0_fp32(row, xv, cols);
        case MVO_Q6_K: return mvo_dot_q6_k_fp32(row, xv, cols);
        case MVO_F32: return mvo_dot_f32((const float*)row, xv, cols);
        case MVO_F16: return dot_f16_double((const uint16_t*)row, xv, cols);
    }
    return 0.0f;
}

static int nthreads(int threads) { return threads > 0 ? threads : 1; }

/* tensor_matvec (src/gguf_kernels.cpp:244-253).  Q4_0 quantizes x to Q8 and
 * uses dot_q4_q8; Q8_0/Q6_K/F32/F16 use fp32 activations. */
int mvo_matvec(const void* wv, int type, size_t rows, size_t cols, const float* x, float* y, int threads) {
    const uint8_t* w = (const uint8_t*)wv;
    if (type == MVO_Q4_0) {
        if (cols % 32) { set_err("Q4_0 matrix row not block aligned"); return -1; }
        size_t nb = cols / 32;
        int8_t* aq = (int8_t*)malloc(cols);
        float* ad = (float*)malloc(nb * sizeof(float));
        mvo_quantize_q8(x, cols, aq, ad);
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
        for (int64_t r = 0; r < (int64_t)rows; ++r) y[r] = mvo_dot_q4_q8(w + (size_t)r * nb * 18, aq, ad, nb);
        free(aq);
        free(ad);
        return 0;
    }
    if (type == MVO_Q6_K && cols % 256) { set_err("Q6_K matrix row not block aligned"); return -1; }
    if (type != MVO_Q8_0 && type != MVO_Q6_K && type != MVO_F32 && type != MVO_F16) {
        set_err("unsupported matvec tensor type %d", type);
        return -1;
    }
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t r = 0; r < (int64_t)rows; ++r) y[r] = fp32_row_dot(w, type, cols, (size_t)r, x);
    return 0;
}

/* tensor_matmul_batch (src/gguf_kernels.cpp:255-259): y[b*rows + r]. */
int mvo_matmul_batch(const void* wv, int type, size_t rows, size_t cols, const float* x, float* y,
                     size_t batch, int threads) {
    const uint8_t* w = (const uint8_t*)wv;
    if (type == MVO_Q6_K && cols % 256) { set_err("Q6_K batch matrix row not block aligned"); return -1; }
    if (type != MVO_Q4_0 && type != MVO_Q8_0 && type != MVO_Q6_K && type != MVO_F32 && type != MVO_F16) {
        set_err("unsupported batch matmul tensor type %d", type);
        return -1;
    }
    int64_t jobs = (int64_t)(batch * rows);
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t j = 0; j < jobs; ++j) {
        size_t bi = (size_t)j / rows, r = (size_t)j % rows;
        y[bi * rows + r] = fp32_row_dot(w, type, cols, r, x + bi * cols);
    }
    return 0;
}

/* tensor_matmul_batch_v06 (src/gguf_kernels.cpp:261-271). */
int mvo_matmul_batch_v06(const void* wv, int type, size_t rows, size_t cols, int is_ffn, int force_q8,
                         const float* x, float* y, size_t batch, int threads) {
    const uint8_t* w = (const uint8_t*)wv;
    if (batch < 2 || (type != MVO_Q4_0 && type != MVO_Q8_0) || cols % 32)
        return mvo_matmul_batch(wv, type, rows, cols, x, y, batch, threads);
    size_t nb = cols / 32, rb = row_bytes(type, cols);
    if (force_q8) {
        int8_t* aq = NULL;
        float* ad = NULL;
        if (type == MVO_Q4_0) {
            aq = (int8_t*)malloc(batch * cols);
            ad = (float*)malloc(batch * nb * sizeof(float));
            mvo_quantize_act_q8(x, batch, cols, aq, ad);
        }
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
        for (int64_t r = 0; r < (int64_t)rows; ++r)
            for (size_t b = 0; b < batch; ++b) {
                const uint8_t* row = w + (size_t)r * rb;
                y[b * rows + r] = type == MVO_Q4_0 ? mvo_dot_q4_q8(row, aq + b * cols, ad + b * nb, nb)
                                                   : mvo_dot_q8_0_fp32(row, x + b * cols, cols);
            }
        free(aq);
        free(ad);
        return 0;
    }
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t rr = 0; rr < (int64_t)rows; ++rr) {
        size_t r = (size_t)rr, b = 0;
        const uint8_t* row = w + r * rb;
        /* FFN tensors use batch8 (= two batch4 calls), others batch4. */
        size_t step = is_ffn ? 8 : 4;
        for (; b + step <= batch; b += step)
            for (size_t h = 0; h < step; h += 4) {
                float o[4];
                if (type == MVO_Q4_0) q4_row_batch4(row, x + (b + h) * cols, cols, nb, o);
                else q8_row_batch4(row, x + (b + h) * cols, cols, nb, o);
                for (int j = 0; j < 4; ++j) y[(b + h + j) * rows + r] = o[j];
            }
        for (; b < batch; ++b)
            y[b * rows + r] = type == MVO_Q4_0 ? mvo_dot_q4_0_fp32(row, x + b * cols, cols)
                                               : mvo_dot_q8_0_fp32(row, x + b * cols, cols);
    }
    return 0;
}

/* tensor_read_row_f32 (src/gguf_kernels.cpp:226). */
int mvo_read_row_f32(const void* wv, int type, size_t rows, size_t cols, size_t row, float* out) {
    const uint8_t* w = (const uint8_t*)wv;
    if (row >= rows) { set_err("tensor row shape mismatch"); return -1; }
    const uint8_t* p = w + row * row_bytes(type, cols);
    switch (type) {
        case MVO_F32: memcpy(out, p, cols * 4); return 0;
        case MVO_F16:
            for (size_t i = 0; i < cols; ++i) {
                uint16_t h;
                memcpy(&h, p + 2 * i, 2);
                out[i] = mvo_fp16_to_fp32(h);
            }
            return 0;
        case MVO_Q4_0:
            for (size_t b = 0; b < cols / 32; ++b) {
                const uint8_t* blk = p + 18 * b;
                float d = blk_d(blk);
                for (int i = 0; i < 16; ++i) {
                    out[b * 32 + i] = d * (float)((int)(blk[2 + i] & 15) - 8);
                    out[b * 32 + 16 + i] = d * (float)((int)(blk[2 + i] >> 4) - 8);
                }
            }
            return 0;
        case MVO_Q8_0:
            for (size_t b = 0; b < cols / 32; ++b) {
                const uint8_t* blk = p + 34 * b;
                float d = blk_d(blk);
                for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
            }
            return 0;
        case MVO_Q6_K:
            if (cols % 256) { set_err("Q6_K embedding row not block aligned"); return -1; }
            for (size_t b = 0; b < cols / 256; ++b) {
                const uint8_t* blk = p + 210 * b;
                float d = blk_d(blk + 208);
                const int8_t* sc = (const int8_t*)(blk + 192);
                for (size_t i = 0; i < 256; ++i)
                    out[b * 256 + i] = d * (float)sc[i / 16] * (float)mvo_q6_k_value(blk, i);
            }
            return 0;
    }
    set_err("unsupported embedding row type %d", type);
    return -1;
}

/* ------------------------------------------------------------------ */
/* paged KV cache, F32 / F16 / Q8 pages (src/llama_model.cpp:16-56)      */
/* ------------------------------------------------------------------ */

/* parse_kv_cache_type / kv_cache_type_name (src/llama_model.cpp:16-17) */
int mvo_kv_parse_type(const char* s) {
    if (!strcmp(s, "f32")) return MVO_KV_F32;
    if (!strcmp(s, "f16")) return MVO_KV_F16;
    if (!strcmp(s, "q8") || !strcmp(s, "q8_0")) return MVO_KV_Q8;
    set_err("unknown KV cache type: %s", s);
    return -1;
}
const char* mvo_kv_type_name(int type) {
    switch (type) {
    case MVO_KV_F32: return "f32";
    case MVO_KV_F16: return "f16";
    case MVO_KV_Q8: return "q8";
    }
    return "?";
}

/* One page of K or V: [page_tokens][kv_dim] elements of the cache type
 * (float, fp16 bits or int8), and for Q8 one float scale per slot
 * (PagedKVCache::Page, src/llama_model.cpp:18). */
typedef struct {
    uint8_t* e;
    float* s;
} kvpage;

struct mvo_kv {
    size_t kv_dim, page_tokens, n_pages;
    int type;
    kvpage* k; /* page -> K page (e == NULL: not allocated) */
    kvpage* v;
};

static size_t kv_elem_bytes(int type) { return type == MVO_KV_F32 ? 4 : type == MVO_KV_F16 ? 2 : 1; }

mvo_kv* mvo_kv_create(size_t kv_dim, size_t page_tokens, int type) {
    if (type != MVO_KV_F32 && type != MVO_KV_F16 && type != MVO_KV_Q8) {
        set_err("unknown KV cache type id %d", type);
        return NULL;
    }
    mvo_kv* kv = (mvo_kv*)calloc(1, sizeof *kv);
    kv->kv_dim = kv_dim;
    kv->page_tokens = page_tokens ? page_tokens : 128;
    kv->type = type;
    return kv;
}

int mvo_kv_type(const mvo_kv* kv) { return kv->type; }

void mvo_kv_reset(mvo_kv* kv) {
    for (size_t p = 0; p < kv->n_pages; ++p) {
        free(kv->k[p].e);
        free(kv->k[p].s);
        free(kv->v[p].e);
        free(kv->v[p].s);
    }
    free(kv->k);
    free(kv->v);
    kv->k = kv->v = NULL;
    kv->n_pages = 0;
}

void mvo_kv_destroy(mvo_kv* kv) {
    if (!kv) return;
    mvo_kv_reset(kv);
    free(kv);
}

/* PagedKVCache::ensure: pages are allocated lazily, one per page index. */
static void kv_ensure(mvo_kv* kv, size_t p) {
    if (p >= kv->n_pages) {
        kv->k = (kvpage*)realloc(kv->k, (p + 1) * sizeof(kvpage));
        kv->v = (kvpage*)realloc(kv->v, (p + 1) * sizeof(kvpage));
        for (size_t i = kv->n_pages; i <= p; ++i) {
            kv->k[i].e = kv->v[i].e = NULL;
            kv->k[i].s = kv->v[i].s = NULL;
        }
        kv->n_pages = p + 1;
    }
    if (!kv->k[p].e) {
        size_t eb = kv_elem_bytes(kv->type);
        kv->k[p].e = (uint8_t*)calloc(kv->page_tokens * kv->kv_dim, eb);
        kv->v[p].e = (uint8_t*)calloc(kv->page_tokens * kv->kv_dim, eb);
        if (kv->type == MVO_KV_Q8) {
            kv->k[p].s = (float*)calloc(kv->page_tokens, sizeof(float));
            kv->v[p].s = (float*)calloc(kv->page_tokens, sizeof(float));
        }
    }
}

/* The Q8 row of one token (src/llama_model.cpp:22, Q8 branch): one scale for
 * the whole kv_dim row, s = max|x|/127 (1 for an all-zero row; the running
 * max keeps its value when compared with a NaN, as std::max does), then
 * q = clamp(lround(x/s), -127, 127) -- a division, not a product with 1/s. */
static float kv_quant_row(const float* x, size_t n, int8_t* q) {
    float m = 0.0f;
    for (size_t d = 0; d < n; ++d) {
        float a = fabsf(x[d]);
        if (m < a) m = a;
    }
    float s = m > 0.0f ? m / 127.0f : 1.0f;
    for (size_t d = 0; d < n; ++d) {
        long r = lroundf(x[d] / s);
        q[d] = (int8_t)(r < -127 ? -127 : r > 127 ? 127 : r);
    }
    return s;
}

/* PagedKVCache::write (src/llama_model.cpp:22): F32 copies, F16 through the
 * reference's fp32_to_fp16, Q8 per-token scale + int8. */
void mvo_kv_write(mvo_kv* kv, size_t pos, const float* k, const float* v) {
    size_t p = pos / kv->page_tokens, i = pos % kv->page_tokens;
    kv_ensure(kv, p);
    size_t off = i * kv->kv_dim;
    if (kv->type == MVO_KV_F32) {
        memcpy((float*)kv->k[p].e + off, k, kv->kv_dim * sizeof(float));
        memcpy((float*)kv->v[p].e + off, v, kv->kv_dim * sizeof(float));
    } else if (kv->type == MVO_KV_F16) {
        uint16_t* kh = (uint16_t*)kv->k[p].e + off;
        uint16_t* vh = (uint16_t*)kv->v[p].e + off;
        for (size_t d = 0; d < kv->kv_dim; ++d) {
            kh[d] = mvo_fp32_to_fp16(k[d]);
            vh[d] = mvo_fp32_to_fp16(v[d]);
        }
    } else {
        kv->k[p].s[i] = kv_quant_row(k, kv->kv_dim, (int8_t*)kv->k[p].e + off);
        kv->v[p].s[i] = kv_quant_row(v, kv->kv_dim, (int8_t*)kv->v[p].e + off);
    }
}

/* Raw stored row of `pos`: K (which = 0) or V (which = 1), kv_dim elements
 * of the cache type; *scale gets the Q8 scale (1 for F32/F16) when non-NULL. */
const void* mvo_kv_row(const mvo_kv* kv, size_t pos, int which, float* scale) {
    size_t p = pos / kv->page_tokens, i = pos % kv->page_tokens;
    if (p >= kv->n_pages || !kv->k[p].e) return NULL;
    const kvpage* pg = which ? &kv->v[p] : &kv->k[p];
    if (scale) *scale = kv->type == MVO_KV_Q8 ? pg->s[i] : 1.0f;
    return pg->e + i * kv->kv_dim * kv_elem_bytes(kv->type);
}

/* element d of a stored row, converted exactly to float */
static inline float kv_elem(const void* row, int type, size_t d) {
    if (type == MVO_KV_F32) return ((const float*)row)[d];
    if (type == MVO_KV_F16) return mvo_fp16_to_fp32(((const uint16_t*)row)[d]);
    return (float)((const int8_t*)row)[d];
}

/* PagedKVCache::dot_key (src/llama_model.cpp:23-39), every type: lane j of 8
 * accumulates fma(q[d], k[d]) for d = j, j+8, ...; sum = t0+..+t7; the F16
 * and Q8 tails `sum += q*k` are contracted, F32 is dot_f32_simd (its tail is
 * not, src/gguf_kernels.cpp:228-233); Q8 returns sum*scale (rounded product). */
float mvo_kv_dot_key(const mvo_kv* kv, size_t pos, size_t offset, const float* q, size_t n) {
    float sc;
    const void* k = mvo_kv_row(kv, pos, 0, &sc);
    if (!k) return NAN;
    if (kv->type == MVO_KV_F32) return mvo_dot_f32(q, (const float*)k + offset, n); /* dot_f32_simd */
    float t[8] = {0};
    size_t d = 0;
    for (; d + 8 <= n; d += 8)
        for (int j = 0; j < 8; ++j) t[j] = fmaf(q[d + j], kv_elem(k, kv->type, offset + d + j), t[j]);
    float sum = hsum8(t);
    for (; d < n; ++d) sum = fmaf(q[d], kv_elem(k, kv->type, offset + d), sum);
    return kv->type == MVO_KV_Q8 ? sum * sc : sum;
}

/* PagedKVCache::add_value (src/llama_model.cpp:40-48): out[d] =
 * fma(w, v[d], out[d]) with w = alpha (F32, F16) or alpha*scale (Q8,
 * rounded once before the chain). */
void mvo_kv_add_value(const mvo_kv* kv, size_t pos, size_t offset, float alpha, float* out, size_t n) {
    float sc;
    const void* v = mvo_kv_row(kv, pos, 1, &sc);
    if (!v) return;
    float w = kv->type == MVO_KV_Q8 ? alpha * sc : alpha;
    for (size_t d = 0; d < n; ++d) out[d] = fmaf(w, kv_elem(v, kv->type, offset + d), out[d]);
}

/* PagedKVCache::bytes_allocated (src/llama_model.cpp:49-55): element bytes of
 * both arrays of every allocated page, plus 4 bytes per slot per Q8 scale array. */
size_t mvo_kv_bytes_allocated(const mvo_kv* kv) {
    size_t n = 0, per = 2 * kv->page_tokens * kv->kv_dim * kv_elem_bytes(kv->type);
    if (kv->type == MVO_KV_Q8) per += 2 * kv->page_tokens * sizeof(float);
    for (size_t p = 0; p < kv->n_pages; ++p)
        if (kv->k[p].e) n += per;
    return n;
}

/* Decode attention for one layer (src/llama_model.cpp:256): per head h with
 * KV head h/(n_head/n_head_kv): s_t = dot_key/sqrtf(hd), mx = max s_t,
 * e_t = expf(s_t - mx), den = sum in double (t order), inv = float(1/den),
 * out += (e_t*inv) * V_t accumulated in t order; out starts at zero. */
void mvo_attn_decode(const mvo_kv* kv, const float* q, size_t pos, size_t n_head, size_t n_head_kv,
                     size_t hd, float* out) {
    size_t group = n_head / n_head_kv;
    float* scores = (float*)malloc((pos + 1) * sizeof(float));
    float sq = sqrtf((float)hd);
    memset(out, 0, n_head * hd * sizeof(float));
    for (size_t h = 0; h < n_head; ++h) {
        size_t kb = (h / group) * hd, qb = h * hd;
        float mx = -INFINITY;
        for (size_t t = 0; t <= pos; ++t) {
            float sf = mvo_kv_dot_key(kv, t, kb, q + qb, hd) / sq;
            scores[t] = sf;
            if (mx < sf) mx = sf;
        }
        double den = 0;
        for (size_t t = 0; t <= pos; ++t) {
            scores[t] = expf(scores[t] - mx);
            den += scores[t];
        }
        float inv = (float)(1.0 / den);
        for (size_t t = 0; t <= pos; ++t) mvo_kv_add_value(kv, t, kb, scores[t] * inv, out + qb, hd);
    }
    free(scores);
}

/* ------------------------------------------------------------------ */
/* elementwise model pieces                                             */
/* ------------------------------------------------------------------ */

/* LlamaModel::rmsnorm (src/llama_model.cpp:237): double sum of squares,
 * inv = 1/sqrtf(float(ss/n) + eps), o = (x*inv)*w. */
void mvo_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out) {
    double ss = 0;
    for (size_t i = 0; i < n; ++i) ss = ss + (double)x[i] * (double)x[i];
    float inv = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (size_t i = 0; i < n; ++i) out[i] = (x[i] * inv) * w[i];
}

/* RoPE table (src/llama_model.cpp:233): inv = powf(theta, -2i/hd),
 * a = float(p)*inv, cosf/sinf from the C library. */
void mvo_rope_table(size_t n_ctx, size_t hd, float theta, float* co, float* si) {
    size_t half = hd / 2;
    for (size_t p = 0; p < n_ctx; ++p)
        for (size_t i = 0; i < half; ++i) {
            float inv = powf(theta, -2.0f * (float)i / (float)hd);
            float a = (float)p * inv;
            co[p * half + i] = cosf(a);
            si[p * half + i] = sinf(a);
        }
}

/* LlamaModel::rope_ptr (src/llama_model.cpp:238): half-split pairs
 * (i, i+half).  GCC contracts `x0*c - x1*s` to fma(x0, c, -(x1*s)) and
 * `x0*s + x1*c` to fma(x0, s, x1*c) (pinned by the model golden vectors). */
static void rot(float* z, size_t heads, size_t hd, const float* co, const float* si) {
    size_t half = hd / 2;
    for (size_t h = 0; h < heads; ++h) {
        float* b = z + h * hd;
        for (size_t i = 0; i < half; ++i) {
            float x0 = b[i], x1 = b[i + half], c = co[i], s = si[i];
            b[i] = fmaf(x0, c, -(x1 * s));
            b[i + half] = fmaf(x0, s, x1 * c);
        }
    }
}
void mvo_rope(float* q, float* k, size_t n_head, size_t n_head_kv, size_t hd, const float* co,
              const float* si) {
    rot(q, n_head, hd, co, si);
    rot(k, n_head_kv, hd, co, si);
}

/* SwiGLU (src/llama_model.cpp:257): (g/(1+expf(-g)))*u. */
void mvo_swiglu(const float* g, const float* u, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float z = g[i];
        out[i] = (z / (1.0f + expf(-z))) * u[i];
    }
}

/* Sampler greedy branch (src/llama_model.cpp:60): first index of the max. */
int mvo_argmax(const float* x, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (x[best] < x[i]) best = i;
    return (int)best;
}

/* ------------------------------------------------------------------ */
/* minimal GGUF reader (subset of src/gguf.cpp:121-139)                 */
/* ------------------------------------------------------------------ */

typedef struct {
    char name[96];
    uint64_t ne0, ne1;
    int type;
    const uint8_t* data;
} otensor;

typedef struct {
    char key[96];
    int kind; /* 0 int, 1 float, 2 string */
    uint64_t u;
    double f;
    char s[64];
} okv;

typedef struct {
    void* map;
    size_t size;
    otensor* t;
    size_t nt;
    okv* kv;
    size_t nkv;
} ogguf;

typedef struct {
    const uint8_t* p;
    size_t n, off;
    int bad;
} rdr;

static int rd(rdr* r, void* out, size_t k) {
    if (r->bad || k > r->n || r->off > r->n - k) {
        r->bad = 1;
        memset(out, 0, k);
        return -1;
    }
    memcpy(out, r->p + r->off, k);
    r->off += k;
    return 0;
}
static uint64_t rd_u64(rdr* r) { uint64_t v; rd(r, &v, 8); return v; }
static uint32_t rd_u32(rdr* r) { uint32_t v; rd(r, &v, 4); return v; }
static void rd_str(rdr* r, char* out, size_t cap) {
    uint64_t len = rd_u64(r);
    if (r->bad || len > r->n - r->off) { r->bad = 1; if (cap) out[0] = 0; return; }
    size_t c = len < cap - 1 ? (size_t)len : cap - 1;
    memcpy(out, r->p + r->off, c);
    out[c] = 0;
    r->off += (size_t)len;
}
static const size_t scalar_size[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

static void rd_scalar(rdr* r, uint32_t ty, okv* kv) {
    union { uint8_t u8; int8_t i8; uint16_t u16; int16_t i16; uint32_t u32; int32_t i32; float f32;
            uint64_t u64; int64_t i64; double f64; } v;
    memset(&v, 0, sizeof v);
    if (ty == 8) { kv->kind = 2; rd_str(r, kv->s, sizeof kv->s); return; }
    if (ty > 12 || ty == 9) { r->bad = 1; return; }
    rd(r, &v, scalar_size[ty]);
    kv->kind = 0;
    switch (ty) {
        case 0: kv->u = v.u8; break;
        case 1: kv->u = (uint64_t)(int64_t)v.i8; break;
        case 2: kv->u = v.u16; break;
        case 3: kv->u = (uint64_t)(int64_t)v.i16; break;
        case 4: kv->u = v.u32; break;
        case 5: kv->u = (uint64_t)(int64_t)v.i32; break;
        case 6: kv->kind = 1; kv->f = v.f32; break;
        case 7: kv->u = v.u8 != 0; break;
        case 10: kv->u = v.u64; break;
        case 11: kv->u = (uint64_t)v.i64; break;
        case 12: kv->kind = 1; kv->f = v.f64; break;
    }
}

static void gguf_close(ogguf* g) {
    if (g->map) munmap(g->map, g->size);
    free(g->t);
    free(g->kv);
    memset(g, 0, sizeof *g);
}

static int gguf_open(const char* path, ogguf* g) {
    memset(g, 0, sizeof *g);
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err("open failed: %s", path); return -1; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size == 0) { close(fd); set_err("empty file"); return -1; }
    g->size = (size_t)st.st_size;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) { g->map = NULL; set_err("mmap failed"); return -1; }
    rdr r = {(const uint8_t*)g->map, g->size, 0, 0};
    char magic[4];
    rd(&r, magic, 4);
    if (memcmp(magic, "GGUF", 4)) { set_err("not a GGUF file"); gguf_close(g); return -1; }
    uint32_t ver = rd_u32(&r);
    if (ver < 2 || ver > 3) { set_err("unsupported GGUF version"); gguf_close(g); return -1; }
    uint64_t nt = rd_u64(&r), nkv = rd_u64(&r);
    if (nt > 1000000 || nkv > 1000000) { set_err("implausible GGUF counts"); gguf_close(g); return -1; }
    g->kv = (okv*)calloc(nkv ? nkv : 1, sizeof(okv));
    g->nkv = (size_t)nkv;
    for (uint64_t i = 0; i < nkv && !r.bad; ++i) {
        okv* kv = &g->kv[i];
        rd_str(&r, kv->key, sizeof kv->key);
        uint32_t ty = rd_u32(&r);
        if (ty == 9) { /* arrays: skipped, the oracle needs none of them */
            uint32_t et = rd_u32(&r);
            uint64_t n = rd_u64(&r);
            kv->kind = 3;
            for (uint64_t j = 0; j < n && !r.bad; ++j) {
                if (et == 8) {
                    uint64_t len = rd_u64(&r);
                    if (len > r.n - r.off) r.bad = 1; else r.off += (size_t)len;
                } else if (et <= 12 && et != 9) {
                    size_t k = scalar_size[et];
                    if (k > r.n - r.off) r.bad = 1; else r.off += k;
                } else {
                    r.bad = 1;
                }
            }
        } else {
            rd_scalar(&r, ty, kv);
        }
    }
    g->t = (otensor*)calloc(nt ? nt : 1, sizeof(otensor));
    g->nt = (size_t)nt;
    uint64_t* rel = (uint64_t*)calloc(nt ? nt : 1, 8);
    for (uint64_t i = 0; i < nt && !r.bad; ++i) {
        otensor* t = &g->t[i];
        rd_str(&r, t->name, sizeof t->name);
        uint32_t nd = rd_u32(&r);
        if (nd == 0 || nd > 4) { r.bad = 1; break; }
        uint64_t dims[4] = {1, 1, 1, 1};
        for (uint32_t d = 0; d < nd; ++d) dims[d] = rd_u64(&r);
        t->ne0 = dims[0];
        t->ne1 = dims[1] * dims[2] * dims[3];
        t->type = (int)rd_u32(&r);
        rel[i] = rd_u64(&r);
    }
    if (r.bad) { free(rel); set_err("truncated GGUF"); gguf_close(g); return -1; }
    uint64_t align = 32;
    for (size_t i = 0; i < g->nkv; ++i)
        if (!strcmp(g->kv[i].key, "general.alignment") && g->kv[i].kind == 0) align = g->kv[i].u;
    size_t data_off = (r.off + align - 1) & ~(size_t)(align - 1);
    for (size_t i = 0; i < g->nt; ++i) {
        if (data_off + rel[i] > g->size) { free(rel); set_err("tensor out of file bounds"); gguf_close(g); return -1; }
        g->t[i].data = (const uint8_t*)g->map + data_off + rel[i];
    }
    free(rel);
    return 0;
}

static const otensor* gguf_tensor(const ogguf* g, const char* name) {
    for (size_t i = 0; i < g->nt; ++i)
        if (!strcmp(g->t[i].name, name)) return &g->t[i];
    return NULL;
}
static const okv* gguf_kv(const ogguf* g, const char* key) {
    for (size_t i = 0; i < g->nkv; ++i)
        if (!strcmp(g->kv[i].key, key)) return &g->kv[i];
    return NULL;
}

/* ------------------------------------------------------------------ */
/* model (LlamaModel, src/llama_model.cpp:222-262)                      */
/* ------------------------------------------------------------------ */

typedef struct {
    const otensor *q, *k, *v, *o, *gate, *up, *down;
    float *attn_norm, *ffn_norm;
} olayer;

struct mvo_model {
    ogguf g;
    size_t n_ctx, n_embd, n_ff, n_layer, n_head, n_head_kv, vocab, hd, kv_dim, pos;
    float eps, theta;
    int threads, force_q8;
    const otensor *embd, *output;
    float* output_norm;
    olayer* L;
    mvo_kv** kv;
    float *rope_cos, *rope_sin;
    float *x, *n, *q, *k, *v, *att, *proj, *g_, *u_, *ff, *out;
};

static float* norm_vec(const otensor* t, size_t n) {
    float* o = (float*)malloc(n * sizeof(float));
    if (t->type == MVO_F32) memcpy(o, t->data, n * 4);
    else
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, t->data + 2 * i, 2);
            o[i] = mvo_fp16_to_fp32(h);
        }
    return o;
}

void mvo_model_close(mvo_model* m) {
    if (!m) return;
    if (m->L)
        for (size_t i = 0; i < m->n_layer; ++i) {
            free(m->L[i].attn_norm);
            free(m->L[i].ffn_norm);
            if (m->kv) mvo_kv_destroy(m->kv[i]);
        }
    free(m->L);
    free(m->kv);
    free(m->output_norm);
    free(m->rope_cos);
    free(m->rope_sin);
    free(m->x); free(m->n); free(m->q); free(m->k); free(m->v); free(m->att);
    free(m->proj); free(m->g_); free(m->u_); free(m->ff); free(m->out);
    gguf_close(&m->g);
    free(m);
}

mvo_model* mvo_model_open(const char* path, size_t ctx_override, size_t page_tokens, int kv_type, int threads,
                          int force_q8) {
    if (kv_type != MVO_KV_F32 && kv_type != MVO_KV_F16 && kv_type != MVO_KV_Q8) {
        set_err("unknown KV cache type id %d", kv_type);
        return NULL;
    }
    mvo_model* m = (mvo_model*)calloc(1, sizeof *m);
    if (gguf_open(path, &m->g)) { free(m); return NULL; }
    const okv* a = gguf_kv(&m->g, "general.architecture");
    if (!a || a->kind != 2 || strcmp(a->s, "llama")) { set_err("GGUF architecture is not llama"); mvo_model_close(m); return NULL; }
#define REQ(field, key)                                                    \
    do {                                                                   \
        const okv* e = gguf_kv(&m->g, key);                                \
        if (!e || e->kind != 0) { set_err("missing GGUF metadata: %s", key); mvo_model_close(m); return NULL; } \
        m->field = (size_t)e->u;                                           \
    } while (0)
    REQ(n_ctx, "llama.context_length");
    REQ(n_embd, "llama.embedding_length");
    REQ(n_ff, "llama.feed_forward_length");
    REQ(n_layer, "llama.block_count");
    REQ(n_head, "llama.attention.head_count");
#undef REQ
    const okv* e = gguf_kv(&m->g, "llama.attention.head_count_kv");
    m->n_head_kv = e && e->kind == 0 ? (size_t)e->u : m->n_head;
    e = gguf_kv(&m->g, "llama.attention.layer_norm_rms_epsilon");
    m->eps = e && e->kind == 1 ? (float)e->f : 1e-5f;
    e = gguf_kv(&m->g, "llama.rope.freq_base");
    m->theta = e && e->kind == 1 ? (float)e->f : 10000.0f;
    m->embd = gguf_tensor(&m->g, "token_embd.weight");
    if (!m->embd || m->embd->ne0 != m->n_embd) { set_err("token embedding shape mismatch"); mvo_model_close(m); return NULL; }
    m->vocab = (size_t)m->embd->ne1;
    if (ctx_override && ctx_override < m->n_ctx) m->n_ctx = ctx_override;
    if (m->n_embd % m->n_head || !m->n_head_kv || m->n_head % m->n_head_kv) { set_err("invalid Llama head configuration"); mvo_model_close(m); return NULL; }
    m->hd = m->n_embd / m->n_head;
    m->kv_dim = m->n_head_kv * m->hd;
    const otensor* on = gguf_tensor(&m->g, "output_norm.weight");
    if (!on) { set_err("missing tensor: output_norm.weight"); mvo_model_close(m); return NULL; }
    m->output = gguf_tensor(&m->g, "output.weight");
    if (!m->output) m->output = m->embd;
    m->output_norm = norm_vec(on, m->n_embd);
    m->threads = threads;
    m->force_q8 = force_q8;
    m->L = (olayer*)calloc(m->n_layer, sizeof(olayer));
    m->kv = (mvo_kv**)calloc(m->n_layer, sizeof(mvo_kv*));
    for (size_t i = 0; i < m->n_layer; ++i) {
        char nm[96];
#define T(field, suffix)                                                              \
    do {                                                                              \
        snprintf(nm, sizeof nm, "blk.%zu%s", i, suffix);                              \
        m->L[i].field = gguf_tensor(&m->g, nm);                                       \
        if (!m->L[i].field) { set_err("missing tensor: %s", nm); mvo_model_close(m); return NULL; } \
    } while (0)
        const otensor *an, *fn;
        snprintf(nm, sizeof nm, "blk.%zu.attn_norm.weight", i);
        an = gguf_tensor(&m->g, nm);
        snprintf(nm, sizeof nm, "blk.%zu.ffn_norm.weight", i);
        fn = gguf_tensor(&m->g, nm);
        if (!an || !fn) { set_err("missing norm tensor in layer %zu", i); mvo_model_close(m); return NULL; }
        T(q, ".attn_q.weight");
        T(k, ".attn_k.weight");
        T(v, ".attn_v.weight");
        T(o, ".attn_output.weight");
        T(gate, ".ffn_gate.weight");
        T(up, ".ffn_up.weight");
        T(down, ".ffn_down.weight");
#undef T
        m->L[i].attn_norm = norm_vec(an, m->n_embd);
        m->L[i].ffn_norm = norm_vec(fn, m->n_embd);
        m->kv[i] = mvo_kv_create(m->kv_dim, page_tokens ? page_tokens : 128, kv_type);
    }
    size_t half = m->hd / 2;
    m->rope_cos = (float*)malloc(m->n_ctx * half * sizeof(float));
    m->rope_sin = (float*)malloc(m->n_ctx * half * sizeof(float));
    mvo_rope_table(m->n_ctx, m->hd, m->theta, m->rope_cos, m->rope_sin);
    m->x = (float*)malloc(m->n_embd * 4);
    m->n = (float*)malloc(m->n_embd * 4);
    m->q = (float*)malloc(m->n_embd * 4);
    m->k = (float*)malloc(m->kv_dim * 4);
    m->v = (float*)malloc(m->kv_dim * 4);
    m->att = (float*)malloc(m->n_embd * 4);
    m->proj = (float*)malloc(m->n_embd * 4);
    m->g_ = (float*)malloc(m->n_ff * 4);
    m->u_ = (float*)malloc(m->n_ff * 4);
    m->ff = (float*)malloc(m->n_ff * 4);
    m->out = (float*)malloc(m->n_embd * 4);
    return m;
}

void mvo_model_reset(mvo_model* m) {
    m->pos = 0;
    for (size_t i = 0; i < m->n_layer; ++i) mvo_kv_reset(m->kv[i]);
}

void mvo_model_config(const mvo_model* m, size_t out[7]) {
    out[0] = m->n_ctx; out[1] = m->n_embd; out[2] = m->n_ff; out[3] = m->n_layer;
    out[4] = m->n_head; out[5] = m->n_head_kv; out[6] = m->vocab;
}
size_t mvo_model_position(const mvo_model* m) { return m->pos; }
size_t mvo_model_kv_bytes(const mvo_model* m) {
    size_t n = 0;
    for (size_t i = 0; i < m->n_layer; ++i) n += mvo_kv_bytes_allocated(m->kv[i]);
    return n;
}

static int mv(const mvo_model* m, const otensor* t, const float* x, float* y) {
    return mvo_matvec(t->data, t->type, (size_t)t->ne1, (size_t)t->ne0, x, y, m->threads);
}

/* LlamaModel::forward (src/llama_model.cpp:253-259). */
int mvo_model_forward(mvo_model* m, int token, float* logits) {
    if (token < 0 || (size_t)token >= m->vocab) { set_err("token id out of range"); return -1; }
    if (m->pos >= m->n_ctx) { set_err("context exhausted"); return -1; }
    size_t D = m->n_embd, F = m->n_ff, half = m->hd / 2;
    if (mvo_read_row_f32(m->embd->data, m->embd->type, (size_t)m->embd->ne1, D, (size_t)token, m->x)) return -1;
    for (size_t li = 0; li < m->n_layer; ++li) {
        olayer* L = &m->L[li];
        mvo_rmsnorm(m->x, L->attn_norm, D, m->eps, m->n);
        if (mv(m, L->q, m->n, m->q) || mv(m, L->k, m->n, m->k) || mv(m, L->v, m->n, m->v)) return -1;
        mvo_rope(m->q, m->k, m->n_head, m->n_head_kv, m->hd, m->rope_cos + m->pos * half, m->rope_sin + m->pos * half);
        mvo_kv_write(m->kv[li], m->pos, m->k, m->v);
        mvo_attn_decode(m->kv[li], m->q, m->pos, m->n_head, m->n_head_kv, m->hd, m->att);
        if (mv(m, L->o, m->att, m->proj)) return -1;
        for (size_t i = 0; i < D; ++i) m->x[i] = m->x[i] + m->proj[i];
        mvo_rmsnorm(m->x, L->ffn_norm, D, m->eps, m->n);
        if (mv(m, L->gate, m->n, m->g_) || mv(m, L->up, m->n, m->u_)) return -1;
        mvo_swiglu(m->g_, m->u_, m->ff, F);
        if (mv(m, L->down, m->ff, m->out)) return -1;
        for (size_t i = 0; i < D; ++i) m->x[i] = m->x[i] + m->out[i];
    }
    ++m->pos;
    if (logits) {
        mvo_rmsnorm(m->x, m->output_norm, D, m->eps, m->n);
        if (mv(m, m->output, m->n, logits)) return -1;
    }
    return 0;
}

static int v06(const mvo_model* m, const otensor* t, int ffn, const float* x, float* y, size_t B) {
    return mvo_matmul_batch_v06(t->data, t->type, (size_t)t->ne1, (size_t)t->ne0, ffn, m->force_q8, x, y, B,
                                m->threads);
}

/* LlamaModel::forward_batch_impl (src/llama_model.cpp:240-252). */
static int forward_batch(mvo_model* m, const int* tokens, size_t B, float* logits) {
    if (!B) return 0;
    if (m->pos + B > m->n_ctx) { set_err("context exhausted"); return -1; }
    for (size_t b = 0; b < B; ++b)
        if (tokens[b] < 0 || (size_t)tokens[b] >= m->vocab) { set_err("token id out of range"); return -1; }
    size_t D = m->n_embd, F = m->n_ff, K = m->kv_dim, hd = m->hd, half = hd / 2, start = m->pos;
    size_t group = m->n_head / m->n_head_kv;
    float* X = (float*)malloc(B * D * 4);
    float* N = (float*)malloc(B * D * 4);
    float* Q = (float*)malloc(B * D * 4);
    float* KK = (float*)malloc(B * K * 4);
    float* VV = (float*)malloc(B * K * 4);
    float* ATT = (float*)malloc(B * D * 4);
    float* PROJ = (float*)malloc(B * D * 4);
    float* G = (float*)malloc(B * F * 4);
    float* U = (float*)malloc(B * F * 4);
    float* FF = (float*)malloc(B * F * 4);
    float* OUT = (float*)malloc(B * D * 4);
    float* scores = (float*)malloc((start + B) * 4);
    int rc = 0;
    float sq = sqrtf((float)hd);
    for (size_t b = 0; b < B; ++b)
        mvo_read_row_f32(m->embd->data, m->embd->type, (size_t)m->embd->ne1, D, (size_t)tokens[b], X + b * D);
    for (size_t li = 0; li < m->n_layer && !rc; ++li) {
        olayer* L = &m->L[li];
        for (size_t b = 0; b < B; ++b) mvo_rmsnorm(X + b * D, L->attn_norm, D, m->eps, N + b * D);
        rc = v06(m, L->q, 0, N, Q, B) || v06(m, L->k, 0, N, KK, B) || v06(m, L->v, 0, N, VV, B);
        if (rc) break;
        for (size_t b = 0; b < B; ++b) {
            mvo_rope(Q + b * D, KK + b * K, m->n_head, m->n_head_kv, hd, m->rope_cos + (start + b) * half,
                     m->rope_sin + (start + b) * half);
            mvo_kv_write(m->kv[li], start + b, KK + b * K, VV + b * K);
        }
        memset(ATT, 0, B * D * 4);
        for (size_t job = 0; job < B * m->n_head; ++job) {
            size_t b = job / m->n_head, h = job % m->n_head, kb = (h / group) * hd, qb = h * hd, upto = start + b;
            float mx = -INFINITY;
            for (size_t t = 0; t <= upto; ++t) {
                float sf = mvo_kv_dot_key(m->kv[li], t, kb, Q + b * D + qb, hd) / sq;
                scores[t] = sf;
                if (mx < sf) mx = sf;
            }
            double den = 0;
            for (size_t t = 0; t <= upto; ++t) {
                scores[t] = expf(scores[t] - mx);
                den += scores[t];
            }
            float inv = (float)(1.0 / den);
            for (size_t t = 0; t <= upto; ++t)
                mvo_kv_add_value(m->kv[li], t, kb, scores[t] * inv, ATT + b * D + qb, hd);
        }
        rc = v06(m, L->o, 0, ATT, PROJ, B);
        if (rc) break;
        for (size_t i = 0; i < B * D; ++i) X[i] = X[i] + PROJ[i];
        for (size_t b = 0; b < B; ++b) mvo_rmsnorm(X + b * D, L->ffn_norm, D, m->eps, N + b * D);
        rc = v06(m, L->gate, 1, N, G, B) || v06(m, L->up, 1, N, U, B);
        if (rc) break;
        mvo_swiglu(G, U, FF, B * F);
        rc = v06(m, L->down, 1, FF, OUT, B);
        if (rc) break;
        for (size_t i = 0; i < B * D; ++i) X[i] = X[i] + OUT[i];
    }
    if (!rc) {
        m->pos += B;
        if (logits) {
            mvo_rmsnorm(X + (B - 1) * D, m->output_norm, D, m->eps, m->n);
            rc = mv(m, m->output, m->n, logits);
        }
    }
    free(X); free(N); free(Q); free(KK); free(VV); free(ATT); free(PROJ);
    free(G); free(U); free(FF); free(OUT); free(scores);
    return rc ? -1 : 0;
}

/* LlamaModel::prefill (src/llama_model.cpp:260). */
int mvo_model_prefill(mvo_model* m, const int* tokens, size_t n, size_t batch, float* logits) {
    if (!n) return 0;
    if (!batch) batch = 1;
    for (size_t i = 0; i < n; i += batch) {
        size_t c = n - i < batch ? n - i : batch;
        if (forward_batch(m, tokens + i, c, i + c == n ? logits : NULL)) return -1;
    }
    return 0;
}

/* ======================================================================
 * Native (non-GGUF) block formats of src/quant.cpp / quant_kernels.cpp.
 * BlockQ4_0 = {float d; uint8 qs[16]} (20 bytes), element 2i = low nibble of
 * qs[i], element 2i+1 = high nibble (src/quant.cpp:79-81); BlockQ8_0 =
 * {float d; int8 qs[32]} (36 bytes) (include/memvanta/quant.hpp:9-13).
 * ====================================================================== */

static float nq_d(const uint8_t* blk) {
    float d;
    memcpy(&d, blk, 4);
    return d;
}

/* quantize_q8_0 (src/quant.cpp:44-62): amax = max|p| (fabs, NaN-skipping
 * std::max), d = amax/127 or 0, q = clamp(nearbyint(p*(1/d)), -127, 127) in
 * the default round-half-even mode; a zero block stores d = 0 and q = 0. */
int mvo_nq_quantize_q8_0(const float* src, size_t n, uint8_t* out) {
    if (n % 32) { set_err("q8_0 length must be multiple of 32"); return -1; }
    for (size_t b = 0; b < n / 32; ++b) {
        const float* p = src + 32 * b;
        uint8_t* o = out + 36 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) { float a = fabsf(p[i]); if (amax < a) amax = a; }
        float d = amax == 0.0f ? 0.0f : amax / 127.0f;
        memcpy(o, &d, 4);
        if (d == 0.0f) { memset(o + 4, 0, 32); continue; }
        float id = 1.0f / d;
        for (int i = 0; i < 32; ++i) {
            int q = (int)nearbyintf(p[i] * id);
            q = q < -127 ? -127 : q > 127 ? 127 : q;
            o[4 + i] = (uint8_t)(int8_t)q;
        }
    }
    return 0;
}

/* quantize_q4_0 (src/quant.cpp:64-85): d = amax/7 or 0, q = clamp(nearbyint(
 * p*(1/d)), -8, 7), nibble q+8, even elements in the low nibble. */
int mvo_nq_quantize_q4_0(const float* src, size_t n, uint8_t* out) {
    if (n % 32) { set_err("q4_0 length must be multiple of 32"); return -1; }
    for (size_t b = 0; b < n / 32; ++b) {
        const float* p = src + 32 * b;
        uint8_t* o = out + 20 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) { float a = fabsf(p[i]); if (amax < a) amax = a; }
        float d = amax == 0.0f ? 0.0f : amax / 7.0f;
        memcpy(o, &d, 4);
        memset(o + 4, 0, 16);
        if (d == 0.0f) continue;
        float id = 1.0f / d;
        for (int i = 0; i < 32; ++i) {
            int q = (int)nearbyintf(p[i] * id);
            q = q < -8 ? -8 : q > 7 ? 7 : q;
            uint8_t nib = (uint8_t)(q + 8);
            if ((i & 1) == 0) o[4 + i / 2] = nib;
            else o[4 + i / 2] |= (uint8_t)(nib << 4);
        }
    }
    return 0;
}

/* dot_q4_q8 (src/quant_kernels.cpp:52-66): isum exact per block, then
 * sum += float(isum) * a.d * x.d, which GCC contracts into
 * fma(float(isum) * a.d, x.d, sum) (the left product rounded first). */
float mvo_nq_dot_q4_q8(const uint8_t* a, const uint8_t* x, size_t nb) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* wa = a + 20 * b;
        const uint8_t* xb = x + 36 * b;
        int isum = 0;
        for (int k = 0; k < 32; ++k) {
            uint8_t packed = wa[4 + k / 2];
            int q4 = ((k & 1) ? (packed >> 4) : (packed & 0x0f)) - 8;
            isum += q4 * (int)(int8_t)xb[4 + k];
        }
        float p = (float)isum * nq_d(wa);
        sum = fmaf(p, nq_d(xb), sum);
    }
    return sum;
}

/* The AVX2 block dot shared by dot_q4_0 / dot_q8_0 (src/quant.cpp:87-156):
 * lane j of eight accumulates elements j, 8+j, 16+j, 24+j by fma from zero,
 * s = 0 + t0 + ... + t7 in order, then sum = fma(s, d, sum). */
static float nq_block_sum(const int* q, const float* x) {
    float t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < 32; k += 8)
        for (int j = 0; j < 8; ++j) t[j] = fmaf((float)q[k + j], x[k + j], t[j]);
    float s = 0.0f;
    for (int j = 0; j < 8; ++j) s = s + t[j];
    return s;
}

/* dot_q4_0 (src/quant.cpp:110-156): the nibbles unpacked back to natural
 * element order (0..31), minus 8. */
float mvo_nq_dot_q4_0(const uint8_t* a, const float* x, size_t n) {
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t* wa = a + 20 * b;
        int q[32];
        for (int k = 0; k < 32; ++k) {
            uint8_t packed = wa[4 + k / 2];
            q[k] = ((k & 1) ? (packed >> 4) : (packed & 0x0f)) - 8;
        }
        sum = fmaf(nq_block_sum(q, x + 32 * b), nq_d(wa), sum);
    }
    return sum;
}

/* dot_q8_0 (src/quant.cpp:87-108). */
float mvo_nq_dot_q8_0(const uint8_t* a, const float* x, size_t n) {
    float sum = 0.0f;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t* wa = a + 36 * b;
        int q[32];
        for (int k = 0; k < 32; ++k) q[k] = (int)(int8_t)wa[4 + k];
        sum = fmaf(nq_block_sum(q, x + 32 * b), nq_d(wa), sum);
    }
    return sum;
}

/* matvec_q4_q8 (src/quant_kernels.cpp:68-76): y[r] = dot_q4_q8(row r, x). */
int mvo_nq_matvec_q4_q8(const uint8_t* A, const uint8_t* x, float* y, size_t rows, size_t cols, int threads) {
    if (cols % 32) { set_err("q4_q8 cols must be multiple of 32"); return -1; }
    size_t nb = cols / 32;
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (size_t r = 0; r < rows; ++r) y[r] = mvo_nq_dot_q4_q8(A + r * nb * 20, x, nb);
    return 0;
}

/* matmul_q4_0_batch (src/quant_kernels.cpp:78-91): y[b*rows + r] = dot_q4_0(row r, x + b*cols). */
int mvo_nq_matmul_q4_0_batch(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                             int threads) {
    if (cols % 32) { set_err("q4_0 cols must be multiple of 32"); return -1; }
    size_t nb = cols / 32;
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < batch; ++b) y[b * rows + r] = mvo_nq_dot_q4_0(A + r * nb * 20, x + b * cols, cols);
    return 0;
}

/* matvec_q4_0 / matvec_q8_0 (src/quant.cpp:158-174). */
int mvo_nq_matvec_q4_0(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, int threads) {
    if (cols % 32) { set_err("q4_0 cols must be multiple of 32"); return -1; }
    size_t nb = cols / 32;
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (size_t r = 0; r < rows; ++r) y[r] = mvo_nq_dot_q4_0(A + r * nb * 20, x, cols);
    return 0;
}

int mvo_nq_matvec_q8_0(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, int threads) {
    if (cols % 32) { set_err("q8_0 cols must be multiple of 32"); return -1; }
    size_t nb = cols / 32;
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (size_t r = 0; r < rows; ++r) y[r] = mvo_nq_dot_q8_0(A + r * nb * 36, x, cols);
    return 0;
}
