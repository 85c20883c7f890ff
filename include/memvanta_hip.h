/*
 * memvanta_hip.h -- C ABI of the MI355X (gfx950) backend for MemVanta's
 * quantized-matmul + paged-KV attention hot path.
 *
 * Plain C: pointers, sizes and int status codes; no exceptions or C++/torch
 * types cross it.  Every call returns MVH_OK (0) or an MVH_E_* code and leaves
 * a message in mvh_last_error() (thread-local) that carries the same text the
 * reference throws (e.g. "Q4_0 matrix row not block aligned: <tensor>").
 *
 * Weights are uploaded once in their native GGUF block layout (Q4_0 18-byte,
 * Q8_0 34-byte, Q6_K 210-byte blocks; GGML order ne0 = cols, ne1 = rows) and
 * are never repacked.  Activation/result pointers are host memory
 * (MVH_HOST: the call stages, launches and synchronises) or device memory
 * (MVH_DEVICE: the call only enqueues on the context's stream).  Device fp32
 * activation inputs (the x of the matvec / matmul / quantize entry points)
 * must be 16-byte aligned: the kernels read them as 16-byte vectors, and a
 * misaligned pointer fails with MVH_E_INVALID.
 *
 * Reference interfaces replaced (MemVanta file:line):
 *   mvh_matvec            tensor_matvec            include/memvanta/gguf_kernels.hpp:26,
 *                                                  src/gguf_kernels.cpp:244-253
 *   mvh_matmul_batch      tensor_matmul_batch      gguf_kernels.hpp:27, src/gguf_kernels.cpp:255-259
 *   mvh_matmul_batch_v06  tensor_matmul_batch_v06  gguf_kernels.hpp:30, src/gguf_kernels.cpp:261-271
 *   mvh_read_row_f32      tensor_read_row_f32      gguf_kernels.hpp:25, src/gguf_kernels.cpp:226
 *   mvh_quantize_q8       quantize_q8 / quantize_activations_q8 (file-local)
 *                                                  src/gguf_kernels.cpp:160-178
 *   mvh_fp32_to_fp16      fp32_to_fp16             gguf_kernels.hpp:34, src/gguf_kernels.cpp:242
 *   mvh_fp16_to_fp32      fp16_to_fp32             include/memvanta/gguf.hpp:80, src/gguf.cpp:110-119
 *   mvh_kv_*              PagedKVCache             include/memvanta/llama_model.hpp:32-52,
 *                                                  src/llama_model.cpp:18-56
 *   mvh_kv_parse_type     parse_kv_cache_type      llama_model.hpp:29, src/llama_model.cpp:16
 *   mvh_kv_type_name      kv_cache_type_name       llama_model.hpp:30, src/llama_model.cpp:17
 *   mvh_attn_decode       the per-head dot_key/softmax/add_value loop of
 *                         LlamaModel::forward      src/llama_model.cpp:256
 *   mvh_attn_batch        the per-(token, head) loop of
 *                         LlamaModel::forward_batch_impl  src/llama_model.cpp:248
 *   mvh_tensor_upload     GgufFile::tensor_data    include/memvanta/gguf.hpp:57, src/gguf.cpp:139
 *                         (the bytes it returns are copied to HBM once)
 *   mvh_model_*           LlamaModel               include/memvanta/llama_model.hpp:100-138,
 *                                                  src/llama_model.cpp:222-262 (device resident)
 *   mvh_argmax            Sampler::sample (greedy) include/memvanta/llama_model.hpp:54-66, src/llama_model.cpp:60
 *   mvh_quantize_q8_0     quantize_q8_0            include/memvanta/quant.hpp:15, src/quant.cpp:44-62
 *   mvh_quantize_q4_0     quantize_q4_0            quant.hpp:16, src/quant.cpp:64-85
 *   mvh_matvec_q4_q8      matvec_q4_q8             quant.hpp:27, src/quant_kernels.cpp:68-76 (dot_q4_q8 :52-66)
 *   mvh_matmul_q4_0_batch matmul_q4_0_batch        quant.hpp:29, src/quant_kernels.cpp:78-91
 *   mvh_matvec_q4_0       matvec_q4_0              quant.hpp:25, src/quant.cpp:167-174 (dot_q4_0 :110-156)
 *   mvh_matvec_q8_0       matvec_q8_0              quant.hpp:23, src/quant.cpp:158-165 (dot_q8_0 :87-108)
 */
#ifndef MEMVANTA_HIP_H
#define MEMVANTA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MVH_OK 0
#define MVH_E_INVALID 1  /* null handle / bad argument */
#define MVH_E_SHAPE 2    /* shape or block-alignment error */
#define MVH_E_TYPE 3     /* unsupported GGML tensor type */
#define MVH_E_DEVICE 4   /* HIP runtime error */
#define MVH_E_RANGE 5    /* position / row / layer out of range, missing KV page */
#define MVH_E_NOMEM 6    /* device allocation failed */

/* where activation / result pointers live */
#define MVH_HOST 0
#define MVH_DEVICE 1

/* numerics of the batched (prefill) matmul, tensor_matmul_batch_v06 */
#define MVH_ACT_REF 0 /* default: fp32 activations, 4/8-token blocking (q4/q8_row_batch4_fp32) */
#define MVH_ACT_Q8 1  /* MEMVANTA_FORCE_Q8_ACT=1: per-token Q8 activations; Q4_0 on int8 MFMA */

/* KV cache element types (KVCacheType, include/memvanta/llama_model.hpp:28, same order) */
#define MVH_KV_F32 0
#define MVH_KV_F16 1 /* LlamaModel's default */
#define MVH_KV_Q8 2  /* int8 with one float scale per token and K/V row */

/* GGML type ids accepted by mvh_tensor_upload */
#define MVH_TYPE_F32 0
#define MVH_TYPE_F16 1
#define MVH_TYPE_Q4_0 2
#define MVH_TYPE_Q8_0 8
#define MVH_TYPE_Q6_K 14
/* MemVanta's native (non-GGUF) blocks, include/memvanta/quant.hpp:9-13: BlockQ4_0 {float d; uint8 qs[16]}
 * (20 bytes; element 2i = low nibble of qs[i], 2i+1 = high nibble) and BlockQ8_0 {float d; int8 qs[32]}
 * (36 bytes).  A native matrix is rows (ne1) of cols/32 blocks (ne0 = cols), uploaded with
 * mvh_tensor_upload like the GGUF types; only the mvh_matvec_q4_q8 / mvh_matmul_q4_0_batch /
 * mvh_matvec_q4_0 / mvh_matvec_q8_0 entry points accept them. */
#define MVH_TYPE_NATIVE_Q4_0 0x1002
#define MVH_TYPE_NATIVE_Q8_0 0x1008

typedef struct mvh_context mvh_context;
typedef struct mvh_tensor mvh_tensor;
typedef struct mvh_kv_cache mvh_kv_cache;
typedef struct mvh_model mvh_model;

/* ---- library / context ---- */
const char* mvh_last_error(void);
int mvh_version(void);
int mvh_device_count(int* count);
/* one context = one device + one HIP stream (default priority) */
int mvh_context_create(int device, mvh_context** out);
int mvh_context_destroy(mvh_context* ctx);
/* the hipStream_t every call of this context is enqueued on */
int mvh_context_stream(mvh_context* ctx, void** stream);
int mvh_context_synchronize(mvh_context* ctx);

/* ---- weights (GgufFile::tensor_data bytes, uploaded once) ---- */
int mvh_tensor_upload(mvh_context* ctx, const char* name, uint32_t ggml_type, uint64_t ne0, uint64_t ne1,
                      const void* host_bytes, uint64_t nbytes, mvh_tensor** out);
/* borrow device memory the caller owns (already in the native layout) */
int mvh_tensor_wrap(mvh_context* ctx, const char* name, uint32_t ggml_type, uint64_t ne0, uint64_t ne1,
                    const void* device_bytes, uint64_t nbytes, mvh_tensor** out);
int mvh_tensor_free(mvh_tensor* t);
int mvh_tensor_info(const mvh_tensor* t, uint32_t* ggml_type, uint64_t* ne0, uint64_t* ne1, uint64_t* nbytes,
                    const void** device_bytes);

/* ---- kernels ---- */
/* quantize_activations_q8: x[batch][cols] -> q[batch][cols] int8 + d[batch][cols/32] f32 */
int mvh_quantize_q8(mvh_context* ctx, const float* x, size_t batch, size_t cols, int8_t* q, float* d, int ptr_kind);
/* tensor_matvec: y[ne1] = W . x[ne0] */
int mvh_matvec(mvh_context* ctx, const mvh_tensor* w, const float* x, float* y, int ptr_kind);
/* Q4_0 weights x an already quantized Q8 activation (the q/d pair mvh_quantize_q8 returns): the
 * per-row kernel of tensor_matvec's Q4_0 branch (dot_q4_q8, src/gguf_kernels.cpp:189) without the
 * quantization, so one quantized input can feed several tensors.  Device q must be 16-byte aligned. */
int mvh_matvec_q8(mvh_context* ctx, const mvh_tensor* w, const int8_t* q, const float* d, float* y, int ptr_kind);
/* tensor_matmul_batch: y[b*ne1 + r] = row r . x[b*ne0 ..], fp32 activations */
int mvh_matmul_batch(mvh_context* ctx, const mvh_tensor* w, const float* x, float* y, size_t batch, int ptr_kind);
/* tensor_matmul_batch_v06 with its fallbacks; act_mode MVH_ACT_REF or MVH_ACT_Q8.  As in the
 * reference, tensors named *.ffn_gate.* / *.ffn_up.* / *.ffn_down.* use 8-token blocking (it changes
 * which tokens of a batch fall in the unblocked tail). */
int mvh_matmul_batch_v06(mvh_context* ctx, const mvh_tensor* w, const float* x, float* y, size_t batch,
                         int act_mode, int ptr_kind);
/* No counterpart in the reference: tensor_matmul_batch_v06 (same numerics, fallbacks and errors as
 * mvh_matmul_batch_v06) for callers that cannot allocate device memory -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  x [batch][ne0] and y [batch][ne1] are device
 * pointers; the call only enqueues on the context's stream and calls no hipMalloc / hipFree.  The FORCE_Q8
 * Q4_0 branch quantizes into a static per-device array of MVH_NOALLOC_SCRATCH_BYTES (held by every device
 * the library runs on until the process ends); a batch whose activations need more fails with MVH_E_RANGE
 * (8 MiB covers 512 tokens at K = 11008).  Every call on one device shares that array: calls that overlap
 * on one device (other streams, other contexts, other threads) race.  Not recorded by the kernel profiler. */
#define MVH_NOALLOC_SCRATCH_BYTES (8u << 20)
int mvh_matmul_batch_v06_noalloc(mvh_context* ctx, const mvh_tensor* w, const float* x, float* y, size_t batch,
                                 int act_mode);
/* tensor_read_row_f32 (embedding row): out[cols] = row `row` of w; cols must equal ne0 and row < ne1, else
 * MVH_E_RANGE with the reference's "tensor row shape mismatch: <name>" */
int mvh_read_row_f32(mvh_context* ctx, const mvh_tensor* w, size_t row, float* out, size_t cols, int ptr_kind);
/* No counterpart in the reference (a measurement probe): reads the bytes (a multiple of 16, 16-byte aligned)
 * of the device buffer buf once with coalesced 16-byte loads on the context's stream.  sink is a device
 * buffer of sink_words words (>= 256 x 8 x the CU count) that receives nothing in practice.  Timed on a
 * buffer larger than the 256 MB Infinity Cache it gives the device's streaming-read bandwidth. */
int mvh_stream_read(mvh_context* ctx, const void* buf, size_t bytes, uint32_t* sink, size_t sink_words);
/* greedy sampling, Sampler::sample with temperature <= 0 (src/llama_model.cpp:60): out[r] = the first index of
 * the maximum of logits[r*n .. r*n+n) (std::max_element), for rows rows of NaN-free logits; n == 0 fails with
 * "empty logits" */
int mvh_argmax(mvh_context* ctx, const float* logits, size_t n, size_t rows, int* out, int ptr_kind);
/* fp32_to_fp16 (the reference's rounding, bit for bit) and the exact fp16_to_fp32 */
int mvh_fp32_to_fp16(mvh_context* ctx, const float* x, uint16_t* out, size_t n, int ptr_kind);
int mvh_fp16_to_fp32(mvh_context* ctx, const uint16_t* h, float* out, size_t n, int ptr_kind);

/* ---- native block formats (src/quant.cpp, src/quant_kernels.cpp) ----
 * Errors carry the reference's text ("q4_q8 cols must be multiple of 32", "q8_0 length must be multiple of
 * 32", ...).  Device block pointers must be 4-byte aligned. */
/* quantize_q8_0 / quantize_q4_0: x[n] (n % 32 == 0) -> n/32 blocks of 36 / 20 bytes (round half to even,
 * d = amax/127 or amax/7, an all-zero block stores d = 0 and zero bytes) */
int mvh_quantize_q8_0(mvh_context* ctx, const float* x, size_t n, void* blocks, int ptr_kind);
int mvh_quantize_q4_0(mvh_context* ctx, const float* x, size_t n, void* blocks, int ptr_kind);
/* matvec_q4_q8: y[r] = dot_q4_q8(row r of a MVH_TYPE_NATIVE_Q4_0 matrix, xq); xq = cols/32 BlockQ8_0 */
int mvh_matvec_q4_q8(mvh_context* ctx, const mvh_tensor* a, const void* xq, float* y, int ptr_kind);
/* matmul_q4_0_batch: y[b*rows + r] = dot_q4_0(row r, x + b*cols), fp32 activations */
int mvh_matmul_q4_0_batch(mvh_context* ctx, const mvh_tensor* a, const float* x, float* y, size_t batch,
                          int ptr_kind);
/* matvec_q4_0 / matvec_q8_0: y[r] = dot_q4_0 / dot_q8_0(row r, x), fp32 activations */
int mvh_matvec_q4_0(mvh_context* ctx, const mvh_tensor* a, const float* x, float* y, int ptr_kind);
int mvh_matvec_q8_0(mvh_context* ctx, const mvh_tensor* a, const float* x, float* y, int ptr_kind);

/* ---- paged KV cache (F32 / F16 / Q8 pages): all layers of one model on one device ---- */
/* parse_kv_cache_type: "f32", "f16", "q8" or "q8_0"; anything else fails with
 * "unknown KV cache type: <s>" */
int mvh_kv_parse_type(const char* s, int* kv_type);
/* kv_cache_type_name: "f32", "f16", "q8", or "?" */
const char* mvh_kv_type_name(int kv_type);
int mvh_kv_create(mvh_context* ctx, size_t n_layer, size_t kv_dim, size_t page_tokens, size_t max_tokens,
                  int kv_type, mvh_kv_cache** out);
int mvh_kv_destroy(mvh_kv_cache* kv);
int mvh_kv_reset(mvh_kv_cache* kv);
/* PagedKVCache::bytes_allocated: element bytes of K and V of every page any write touched, plus 4 bytes per
 * slot per Q8 scale array */
int mvh_kv_bytes_allocated(const mvh_kv_cache* kv, size_t* bytes);
int mvh_kv_type(const mvh_kv_cache* kv, int* kv_type);
/* PagedKVCache::write for n_tokens consecutive positions pos..pos+n-1; k/v are [n][kv_dim] fp32 */
int mvh_kv_write(mvh_context* ctx, mvh_kv_cache* kv, size_t layer, size_t pos, size_t n_tokens, const float* k,
                 const float* v, int ptr_kind);
/* copy the stored row of (layer, pos): which = 0 for K, 1 for V; out is host memory for kv_dim elements of the
 * cache type (float, fp16 bits or int8); scale (may be NULL) receives the Q8 row scale, 1 for F32/F16 */
int mvh_kv_read_row(mvh_context* ctx, const mvh_kv_cache* kv, size_t layer, size_t pos, int which, void* out,
                    float* scale);
/* decode attention of one layer over positions 0..pos: q[n_head*hd] -> out[n_head*hd] */
int mvh_attn_decode(mvh_context* ctx, const mvh_kv_cache* kv, size_t layer, const float* q, size_t pos,
                    size_t n_head, size_t n_head_kv, size_t head_dim, float* out, int ptr_kind);
/* the batched causal attention of LlamaModel::forward_batch_impl (the per-(token, head) loop at
 * src/llama_model.cpp:248) for n_tokens query tokens at positions pos..pos+n_tokens-1, whose K/V rows are
 * already written: token b attends over positions 0..pos+b; q[n_tokens][n_head*hd] -> out[n_tokens][n_head*hd] */
int mvh_attn_batch(mvh_context* ctx, const mvh_kv_cache* kv, size_t layer, const float* q, size_t pos,
                   size_t n_tokens, size_t n_head, size_t n_head_kv, size_t head_dim, float* out, int ptr_kind);

/* ---- kernel profiler: enable_kernel_profiling, reset_kernel_profile, kernel_profile_snapshot,
 * kernel_profile_kind_name (include/memvanta/gguf_kernels.hpp:11-23, src/gguf_kernels.cpp:34-73,:219-222) ----
 * While enabled, every mvh_matvec / mvh_matvec_q8 / mvh_matmul_batch / mvh_matmul_batch_v06 call, and
 * every GEMV / GEMM of a model step, is timed on the device with a HIP event pair on its stream (host
 * staging copies excluded; a profiled call waits for its end event) and added to the entry of its
 * (layer, kind, tensor, batch), with layer and kind taken from the tensor name as tensor_layer and
 * classify_tensor take them.  A model step runs without its HIP graph while profiling; a launch over
 * fused weights is one entry named by its members joined with '+'.  Process-wide, like the reference. */
#define MVH_PROF_Q_PROJ 0
#define MVH_PROF_K_PROJ 1
#define MVH_PROF_V_PROJ 2
#define MVH_PROF_O_PROJ 3
#define MVH_PROF_FFN_GATE 4
#define MVH_PROF_FFN_UP 5
#define MVH_PROF_FFN_DOWN 6
#define MVH_PROF_OUTPUT 7
#define MVH_PROF_OTHER 8
typedef struct mvh_profile_entry {
    int layer;         /* -1 when the name has no "blk.N." prefix */
    int kind;          /* MVH_PROF_* */
    char tensor[192];  /* NUL-terminated, truncated to 191 bytes */
    size_t calls;
    size_t batch;
    double ms;
} mvh_profile_entry;
void mvh_profile_enable(int enabled);
void mvh_profile_reset(void);
/* *n_total = the number of entries; the first min(cap, *n_total) are copied to out (may be NULL when cap is 0) */
int mvh_profile_snapshot(mvh_profile_entry* out, size_t cap, size_t* n_total);
/* "q_proj", "k_proj", "v_proj", "o_proj", "ffn_gate", "ffn_up", "ffn_down", "output", "other" */
const char* mvh_profile_kind_name(int kind);

/* ---- whole model: LlamaModel on one device (weights, paged KV and activations in HBM) ---- */
/* kv_type is LlamaModel's kv_type argument (MVH_KV_F16 is its default); act_mode selects the prefill numerics
 * (MVH_ACT_REF / MVH_ACT_Q8); max_batch bounds the prefill chunk */
int mvh_model_open(const char* gguf_path, int device, size_t ctx_override, size_t kv_page_tokens, int kv_type,
                   int act_mode, size_t max_batch, mvh_model** out);
int mvh_model_close(mvh_model* m);
/* n_ctx, n_embd, n_ff, n_layer, n_head, n_head_kv, vocab */
int mvh_model_config(const mvh_model* m, size_t out[7]);
int mvh_model_reset(mvh_model* m);
/* LlamaModel::forward: one decode step; logits (host, vocab floats) may be NULL */
int mvh_model_forward(mvh_model* m, int token, float* logits);
/* LlamaModel::prefill: chunks of `batch`; logits of the last token when logits != NULL.  Consecutive chunks
 * run on three internal streams (chunk c + 1's layer l beside chunk c's layer l + 1, results identical to a
 * chunk-by-chunk run); every stream is drained before the call returns, also when a later chunk's error is
 * returned after the earlier chunks completed */
int mvh_model_prefill(mvh_model* m, const int* tokens, size_t n, size_t batch, float* logits);
/* n greedy decode steps from `token`, run on the device from one HIP graph (the argmax of each step
 * feeds the next); out_tokens (host) receives the n sampled ids, last_logits (host) may be NULL */
int mvh_model_generate_greedy(mvh_model* m, int token, size_t n, int* out_tokens, float* last_logits);
int mvh_model_position(const mvh_model* m, size_t* pos);
int mvh_model_kv_bytes(const mvh_model* m, size_t* bytes);
int mvh_model_kv_type(const mvh_model* m, int* kv_type); /* LlamaModel::kv_type */
/* the stream decode steps run on (prefill's first lane) */
int mvh_model_stream(mvh_model* m, void** stream);

#ifdef __cplusplus
}
#endif
#endif /* MEMVANTA_HIP_H */
