// mvh_quant.hip -- activation Q8 quantizer and fp16 conversion kernels.
#include "mvh_kernels.hpp"

namespace mvh {

// quantize_q8 (src/gguf_kernels.cpp:160-172), one 32-element block per 8
// lanes, 4 elements per lane (one 16-byte load, one 4-byte store).  Besides q
// and the f32 scale d it writes s = sum of the 32 q values.  With op_cols != 0
// q is written in the prefill GEMM's operand order (q8_op_offset, rows of
// op_cols elements) instead of row-major.
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float4* __restrict__ x, uint32_t* __restrict__ q,
                                                          float* __restrict__ d, int* __restrict__ s, size_t n4,
                                                          int op_cols) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const bool live = i < n4;  // n4 % 8 == 0, so an 8-lane group is all-live or all-dead
    const float4 v = live ? x[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    float dd;
    int bsum;
    const uint32_t packed = quantize_q8_x4(v, dd, bsum);
    if (live) {
        if (op_cols) {
            const size_t K = static_cast<size_t>(op_cols);
            q[q8_op_offset(4 * i / K, 4 * i % K, K) / 4] = packed;
        } else {
            q[i] = packed;
        }
        if ((threadIdx.x & 7) == 0) {
            d[i >> 3] = dd;
            s[i >> 3] = bsum;
        }
    }
}

// fp32_to_fp16 (src/gguf_kernels.cpp:242) over an array.
__global__ __launch_bounds__(256) void f2h_kernel(const float* __restrict__ x, uint16_t* __restrict__ out, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2h_ref(x[i]);
}

// fp32_to_fp16 of the bit patterns first .. first+n-1 (exhaustive checks).
__global__ __launch_bounds__(256) void f2h_bits_kernel(uint32_t first, uint16_t* __restrict__ out, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2h_ref(__uint_as_float(first + static_cast<uint32_t>(i)));
}

// fp16_to_fp32 (src/gguf.cpp:110-119) over an array of bit patterns.
__global__ __launch_bounds__(256) void h2f_kernel(const uint16_t* __restrict__ h, float* __restrict__ out, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = h2f(h[i]);
}

// tensor_read_row_f32 (src/gguf_kernels.cpp:226): dequantize one row.
// Q4_0: d*float(q-8); Q8_0: d*float(q); Q6_K: (d*float(sc))*float(q).
__global__ __launch_bounds__(256) void read_row_kernel(uint32_t type, const uint8_t* __restrict__ W, int cols,
                                                       size_t row, float* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= cols) return;
    if (type == kF32) {
        out[i] = reinterpret_cast<const float*>(W)[row * cols + i];
    } else if (type == kF16) {
        out[i] = h2f(reinterpret_cast<const uint16_t*>(W)[row * cols + i]);
    } else if (type == kQ4_0) {
        const uint8_t* b = W + (row * (cols / 32) + i / 32) * 18;
        const int e = i & 31;
        const uint32_t byte = b[2 + (e & 15)];
        const int q = static_cast<int>(e < 16 ? (byte & 15u) : (byte >> 4)) - 8;
        out[i] = h2f(b[0] | (static_cast<uint32_t>(b[1]) << 8)) * static_cast<float>(q);
    } else if (type == kQ8_0) {
        const uint8_t* b = W + (row * (cols / 32) + i / 32) * 34;
        out[i] = h2f(b[0] | (static_cast<uint32_t>(b[1]) << 8)) * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31)]));
    } else if (type == kQ6_K) {
        const uint8_t* b = W + (row * (cols / 256) + i / 256) * 210;
        const int e = i & 255;
        const int row32 = e / 32, j = e % 32, group = row32 / 4, local = row32 % 4;
        const int lo = (b[group * 64 + (local % 2) * 32 + j] >> (local < 2 ? 0 : 4)) & 0x0f;
        const int hi = (b[128 + group * 32 + j] >> (2 * local)) & 0x03;
        const float d = h2f(b[208] | (static_cast<uint32_t>(b[209]) << 8));
        const float sc = static_cast<float>(static_cast<int8_t>(b[192 + e / 16]));
        out[i] = (d * sc) * static_cast<float>((lo | (hi << 4)) - 32);
    }
}

hipError_t launch_read_row(uint32_t type, const uint8_t* W, size_t cols, size_t row, float* out, hipStream_t st) {
    if (!cols) return hipSuccess;
    read_row_kernel<<<static_cast<unsigned>((cols + 255) / 256), 256, 0, st>>>(type, W, static_cast<int>(cols), row, out);
    return hipGetLastError();
}

hipError_t launch_quantize_q8(const float* x, int8_t* q, float* d, int* s, size_t rows, size_t cols, hipStream_t st,
                              bool q_op) {
    const size_t n4 = rows * cols / 4;
    if (!n4) return hipSuccess;
    if (q_op && cols % 256) return hipErrorInvalidValue;
    const unsigned grid = static_cast<unsigned>((n4 + 255) / 256);
    quantize_q8_kernel<<<grid, 256, 0, st>>>(reinterpret_cast<const float4*>(x), reinterpret_cast<uint32_t*>(q), d,
                                             s, n4, q_op ? static_cast<int>(cols) : 0);
    return hipGetLastError();
}

hipError_t launch_f2h(const float* x, uint16_t* out, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    f2h_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(x, out, n);
    return hipGetLastError();
}

hipError_t launch_f2h_bits(uint32_t first, uint16_t* out, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    f2h_bits_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(first, out, n);
    return hipGetLastError();
}

hipError_t launch_h2f(const uint16_t* h, float* out, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    h2f_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(h, out, n);
    return hipGetLastError();
}

}  // namespace mvh
