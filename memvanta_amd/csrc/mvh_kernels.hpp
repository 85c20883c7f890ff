// mvh_kernels.hpp -- launchers of the gfx950 kernels (host-callable).
#pragma once
#include "mvh_device.hpp"

#include <algorithm>

namespace mvh {

// GGML type ids used on the device side, and the native (non-GGUF) block
// formats of src/quant.cpp: BlockQ4_0 {float d; uint8 qs[16]} (20 bytes,
// element 2i = low nibble of qs[i]) and BlockQ8_0 {float d; int8 qs[32]} (36 bytes).
enum : uint32_t { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ6_K = 14, kNQ4_0 = 0x1002, kNQ8_0 = 0x1008 };

// Grid of the launches that carry L2 warm-up workgroups (warm.c1 > warm.c0): their
// own workgroups and the warm-up ones fill kWarmWgs (one per CU of the 256)
constexpr unsigned kWarmWgs = 256;

// ---- activation quantization / conversions (mvh_quant.hip) ----
// q_op: q in the prefill GEMM's operand order (q8_op_offset; cols % 256 == 0,
// q8_op_bytes(rows, cols) bytes), else row-major
hipError_t launch_quantize_q8(const float* x, int8_t* q, float* d, int* s, size_t rows, size_t cols, hipStream_t st,
                              bool q_op = false);
hipError_t launch_f2h(const float* x, uint16_t* out, size_t n, hipStream_t st);
hipError_t launch_f2h_bits(uint32_t first, uint16_t* out, size_t n, hipStream_t st);
hipError_t launch_h2f(const uint16_t* h, float* out, size_t n, hipStream_t st);
hipError_t launch_read_row(uint32_t type, const uint8_t* W, size_t cols, size_t row, float* out, hipStream_t st);

// ---- decode GEMV (mvh_gemv.hip); W is the tensor in native GGUF layout ----
// y[N] = W[N x K] . x[K]; `rows` are N, `cols` are K.
// aq must be 16-byte aligned; the kernel derives the per-block sums of aq itself.
// batch tokens: rows of aq / ad / y at strides cols / cols/32 / rows (one
// launch unless cols takes the row-group kernel, which runs one per token)
hipError_t launch_gemv_q4_0(const uint8_t* W, const int8_t* aq, const float* ad, float* y, size_t rows, size_t cols,
                            hipStream_t st, size_t batch = 1);
hipError_t launch_gemv_q8_0(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                            hipStream_t st);
hipError_t launch_gemv_q6_k(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                            hipStream_t st);
// F32 / F16 weights with fp32 activations, y[b*rows + r] (dot_f32_simd / the double F16 sum)
hipError_t launch_gemv_f32(const float* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                           hipStream_t st);
hipError_t launch_gemv_f16(const uint16_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                           hipStream_t st);
// Q4_0 x Q8 GEMV in 16-lane row groups (cols % 256 == 0, 256 <= cols <= 16384):
// x != nullptr quantizes the fp32 input inside the kernel; otherwise aq
// (16-byte aligned) / ad are the Q8 input.
bool gemv_q4_0_rows16_ok(size_t cols);
// Rows each workgroup of the one-token decode GEMV of a Q4_0 (pre-quantized
// Q8 input), Q8_0 or Q6_K (fp32 input) tensor reads: workgroup c reads rows
// [c*r, (c+1)*r), one contiguous chunk of the tensor, and runs on XCD c % 8
// (the L2 warm-up's map); 0 when that kernel reads no such chunks.
size_t gemv_decode_rows_per_wg(uint32_t type, size_t rows, size_t cols);
hipError_t launch_gemv_q4_0_rows16(const uint8_t* W, const float* x, const int8_t* aq, const float* ad, float* y,
                                   size_t rows, size_t cols, hipStream_t st);
// the same kernel over native BlockQ4_0 x BlockQ8_0 (xq 4-byte aligned)
hipError_t launch_gemv_q4q8_native_rows16(const uint8_t* W, const uint8_t* xq, float* y, size_t rows, size_t cols,
                                          hipStream_t st);
// Native BlockQ4_0 x BlockQ8_0 (matvec_q4_q8, src/quant_kernels.cpp:68-76):
// y[r] = dot_q4_q8(row r, xq); xq is rows' cols/32 BlockQ8_0 (36 bytes each,
// 4-byte aligned).  Any cols % 32 == 0.
hipError_t launch_matvec_q4q8_native(const uint8_t* W, const uint8_t* xq, float* y, size_t rows, size_t cols,
                                     hipStream_t st);
// Native-format fp32-activation dots, y[b*rows + r]: dot_q4_0 (type kNQ4_0,
// matvec_q4_0 / matmul_q4_0_batch) and dot_q8_0 (kNQ8_0, matvec_q8_0)
hipError_t launch_gemv_native_f32act(uint32_t type, const uint8_t* W, const float* x, float* y, size_t rows,
                                     size_t cols, size_t batch, hipStream_t st);
// quantize_q8_0 / quantize_q4_0 of n floats (n % 32 == 0) into native blocks
hipError_t launch_quantize_native(uint32_t type, const float* x, uint8_t* out, size_t n, hipStream_t st);
// dot_q4_0_fp32 per (row, token): y[b*rows + r]
hipError_t launch_gemv_q4_0_f32act(const uint8_t* W, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                                   hipStream_t st);
// q4/q8_row_batch4_fp32 numerics per (row, token) for Q4_0 / Q8_0
hipError_t launch_batch4_f32act(uint32_t type, const uint8_t* W, const float* x, float* y, size_t rows, size_t cols,
                                size_t batch, hipStream_t st);

// ---- batched prefill on int8 MFMA (mvh_gemm_q4.hip) ----
// y[b*rows + r] = dot_q4_q8(W row r, Q8 activation row b) for b < batch
// (MEMVANTA_FORCE_Q8_ACT numerics); aq in operand order (q8_op_offset,
// q8_op_bytes(batch, cols) bytes, as launch_quantize_q8 with q_op writes it),
// ad [batch][cols/32]; needs cols % 256 == 0.
bool gemm_q4_0_mfma_ok(size_t cols);
hipError_t launch_gemm_q4_0_q8_mfma(const uint8_t* W, const int8_t* aq, const float* ad, float* y, size_t rows,
                                    size_t cols, size_t batch, hipStream_t st);

// ---- paged KV (F32 / F16 / Q8 pages, KvType) + attention (mvh_attn.hip) ----
// PagedKVCache::write of n_tokens rows (token t's k/v at k + t*pitch, v + t*pitch)
// at positions pos..pos+n-1 (pos = *d_pos when d_pos != null)
hipError_t launch_kv_write(int kv_type, void* const* pt_k, void* const* pt_v, const float* k, const float* v,
                           size_t pitch, const int* d_pos, size_t pos, size_t n_tokens, size_t kv_dim,
                           size_t page_tokens, hipStream_t st);
// B query tokens at positions pos..pos+B-1 (pos = *d_pos when d_pos != null),
// causal; q of token b at q + b*q_pitch; scores needs B * n_head * max_pos
// floats, max_pos > last position
hipError_t launch_attn(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q, size_t q_pitch,
                       float* scores, float* out, const int* d_pos, size_t pos, size_t max_pos, size_t B,
                       size_t n_head, size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st,
                       int8_t* q8 = nullptr, float* q8d = nullptr, bool q8_op = false);
// The same attention for a prefill chunk (hd % 32 == 0): scores and softmax
// weights once per (token, head) into a_scratch (B * n_head * max_pos floats),
// then the value chains with the V tiles shared by groups of 32 tokens; with
// q8 also the output's quantize_q8 blocks (row-major, or the prefill GEMM's
// operand order when q8_op).
hipError_t launch_attn_prefill(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q,
                               size_t q_pitch, float* a_scratch, float* out, int8_t* q8, float* q8d, bool q8_op,
                               const int* d_pos, size_t pos, size_t max_pos, size_t B, size_t n_head,
                               size_t n_head_kv, size_t hd, size_t kv_dim, size_t page_tokens, hipStream_t st);
// One decode token in one launch (F16 pages): RoPE of q and k at position
// *d_pos, the F16 K/V write at that position, scores, softmax and the value sum, and
// (when q8 != null, hd % 32 == 0) the Q8 activation of the output.  One
// workgroup per query head; max_ctx bounds the position.
bool attn_decode_fused_ok(size_t hd, size_t max_ctx, size_t page_tokens);  // LDS and shape limits of the fused kernel
// rope: cos then sin of the position (hd/2 floats each); K/V rows of page p at
// kbase / vbase + p * page_stride (elements) + (row % page_tokens) * kv_dim
hipError_t launch_attn_decode_fused(const float* q, const float* k, const float* v, const float* rope,
                                    const int* d_pos, uint16_t* kbase, uint16_t* vbase, size_t page_tokens,
                                    size_t page_stride, float* out, int8_t* q8, float* q8d, size_t n_head,
                                    size_t n_head_kv, size_t hd, size_t max_ctx, hipStream_t st,
                                    const L2Warm& warm = {}, const L2Warm& warm2 = {});
// scores needs n_head * (pos+1) floats of scratch
hipError_t launch_attn_decode(int kv_type, const void* const* pt_k, const void* const* pt_v, const float* q,
                              float* scores, float* out, size_t pos, size_t n_head, size_t n_head_kv, size_t hd,
                              size_t kv_dim, size_t page_tokens, hipStream_t st);

// ---- measurement probe (mvh_probe.hip) ----
// reads bytes (a multiple of 16) of buf once; sink holds sink_words words (at
// least 256 x the grid: 8 workgroups per CU)
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, size_t sink_words, hipStream_t st);

// ---- model step pieces (mvh_model.hip) ----
// with rope_cur (one token): also copies cos/sin row *d_pos of the RoPE
// tables (half floats each) to rope_cur[0 .. 2*half)
hipError_t launch_embed(uint32_t type, const uint8_t* W, size_t cols, const int* tokens, size_t B, float* out,
                        hipStream_t st, const int* d_pos = nullptr, const float* cos_t = nullptr,
                        const float* sin_t = nullptr, size_t half = 0, float* rope_cur = nullptr);
// x += add (if add), n = rmsnorm(x)*w, and q/qd = Q8 of n (if q); B rows of D;
// warm.c1 > warm.c0: the launch also warms the next GEMV's weights in L2 (L2Warm)
hipError_t launch_rmsnorm(float* x, const float* add, const float* w, float* n, int8_t* q, float* qd, size_t B,
                          size_t D, float eps, hipStream_t st, bool q_op = false, const L2Warm& warm = {});
// q/k/v of token b at q + b*q_pitch, k + b*kv_pitch, v + b*kv_pitch; the
// rotated k and v go to the pages when pt_k != null, F16 or F32 (kv_type;
// Q8 pages are written by launch_kv_write), k is rotated in place either way
hipError_t launch_rope_kv(float* q, size_t q_pitch, float* k, const float* v, size_t kv_pitch, const float* cos_t,
                          const float* sin_t, const int* d_pos, size_t pos0, size_t B, size_t n_head, size_t n_kv,
                          size_t hd, int kv_type, void* const* pt_k, void* const* pt_v, size_t page_tokens,
                          hipStream_t st);
// B rows: g/u row b at g + b*pitch, u + b*pitch; ff/q rows of F
hipError_t launch_swiglu(const float* g, const float* u, size_t pitch, float* ff, int8_t* q, float* qd, size_t B,
                         size_t F, hipStream_t st, bool q_op = false, const L2Warm& warm = {});
hipError_t launch_argmax(const float* logits, size_t V, size_t B, int* out, int* d_pos, int* hist, hipStream_t st);

}  // namespace mvh
