/*
 * mv_oracle.h -- CPU restatement of MemVanta's quantized-matmul and paged-KV
 * attention path.  TEST INFRASTRUCTURE ONLY: tests/ and __graft_entry__.smoke()
 * check results against it, bench.py's cpu_baseline leg times it.  Nothing
 * in the product (memvanta_amd/, include/) links or calls it.
 *
 * Every function restates one reference function; the citation names the
 * reference file:line it follows (paths relative to the MemVanta repo root).
 * Every floating-point operation is spelled out: the file is compiled with
 * -ffp-contract=off, so each fmaf() below stands for a fused multiply-add the
 * reference's GCC build forms (explicit _mm256_fmadd_ps, or -ffp-contract=fast
 * contraction of `s += a*b`), and every other product is rounded on its own.
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   fp16_to_fp32 ........ exhaustive 65,536 vs the hardware/IEEE conversion
 *   fp32_to_fp16 ........ exhaustive 2^32 vs the compiled reference (oracle/_ref)
 *                         and committed golden vectors (tests/golden)
 *   quantize_q8 ......... closed form + golden matvec vectors (a wrong q or d
 *                         changes y); probe matrices recover each q exactly
 *   matvec / matmul ..... bit-exact golden vectors from the compiled reference,
 *                         plus an fp64 brute-force bound
 *   kv / attention ...... bit-exact golden vectors from the compiled reference
 *                         for F32, F16 and Q8 pages (dots, value sums, one-hot
 *                         probes of the stored values, bytes), model runs with
 *                         each cache type, plus an fp64 softmax bound
 *   model ............... bit-exact logits + greedy ids vs the compiled reference
 *                         (the tiny MHA model and a 2-layer GQA model, 32/4 heads)
 *   native blocks ....... quantize_q8_0 / quantize_q4_0 / matvec_q4_q8 /
 *                         matmul_q4_0_batch / matvec_q4_0 / matvec_q8_0
 *                         bit-exact vs golden vectors of the compiled
 *                         reference (ties, zero blocks, saturation, K 32..11008)
 */
#ifndef MV_ORACLE_H
#define MV_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML tensor type ids (GGUF on-disk values). */
enum { MVO_F32 = 0, MVO_F16 = 1, MVO_Q4_0 = 2, MVO_Q8_0 = 8, MVO_Q6_K = 14 };

/* ---- scalar conversions ---- */
float    mvo_fp16_to_fp32(uint16_t h);
uint16_t mvo_fp32_to_fp16(float f);
void     mvo_fp32_to_fp16_n(const float* x, uint16_t* out, size_t n);
/* out[i] = fp32_to_fp16(bits(first + i)), i < count; used for exhaustive sweeps */
void     mvo_fp32_to_fp16_bits(uint32_t first, uint64_t count, uint16_t* out);
/* number of i in [first, first+count) where mvo_fp32_to_fp16 disagrees with out[] */
uint64_t mvo_fp32_to_fp16_count_mismatch(uint32_t first, uint64_t count, const uint16_t* out);

/* ---- activation quantization (returns 0, or -1 when cols % 32 != 0) ---- */
int mvo_quantize_q8(const float* x, size_t cols, int8_t* q, float* d);
int mvo_quantize_act_q8(const float* x, size_t batch, size_t cols, int8_t* q, float* d);

/* ---- per-row dots over one weight row in native GGUF layout ---- */
float mvo_dot_q4_q8(const uint8_t* w_row, const int8_t* aq, const float* ad, size_t nb);
float mvo_dot_q4_0_fp32(const uint8_t* w_row, const float* x, size_t n);
float mvo_dot_q8_0_fp32(const uint8_t* w_row, const float* x, size_t n);
float mvo_dot_q6_k_fp32(const uint8_t* w_row, const float* x, size_t n);
int   mvo_q6_k_value(const uint8_t* block, size_t i);
float mvo_dot_f32(const float* a, const float* b, size_t n);

/* ---- tensor-level entry points (rows = ne1, cols = ne0) ----
 * return 0 on success, -1 on a shape/type error (message in mvo_last_error()) */
const char* mvo_last_error(void);
int mvo_matvec(const void* w, int type, size_t rows, size_t cols,
               const float* x, float* y, int threads);
int mvo_matmul_batch(const void* w, int type, size_t rows, size_t cols,
                     const float* x, float* y, size_t batch, int threads);
int mvo_matmul_batch_v06(const void* w, int type, size_t rows, size_t cols, int is_ffn,
                         int force_q8, const float* x, float* y, size_t batch, int threads);
int mvo_read_row_f32(const void* w, int type, size_t rows, size_t cols, size_t row, float* out);

/* ---- paged KV cache: F32, F16 or Q8 pages (PagedKVCache's KVCacheType order) ---- */
enum { MVO_KV_F32 = 0, MVO_KV_F16 = 1, MVO_KV_Q8 = 2 };
int         mvo_kv_parse_type(const char* s);   /* -1 (message in mvo_last_error()) when unknown */
const char* mvo_kv_type_name(int type);
typedef struct mvo_kv mvo_kv;
mvo_kv* mvo_kv_create(size_t kv_dim, size_t page_tokens, int type);  /* NULL for an unknown type */
void    mvo_kv_destroy(mvo_kv* kv);
void    mvo_kv_reset(mvo_kv* kv);
int     mvo_kv_type(const mvo_kv* kv);
void    mvo_kv_write(mvo_kv* kv, size_t pos, const float* k, const float* v);
float   mvo_kv_dot_key(const mvo_kv* kv, size_t pos, size_t offset, const float* q, size_t n);
void    mvo_kv_add_value(const mvo_kv* kv, size_t pos, size_t offset, float alpha, float* out, size_t n);
size_t  mvo_kv_bytes_allocated(const mvo_kv* kv);
/* raw page access for layout tests: the stored K (which=0) or V (which=1) row of `pos`
 * (kv_dim floats, fp16 bits or int8); *scale = the Q8 row scale (1 otherwise) if non-NULL */
const void* mvo_kv_row(const mvo_kv* kv, size_t pos, int which, float* scale);
/* decode attention for one layer: q [n_head*hd] -> out [n_head*hd] over positions 0..pos */
void    mvo_attn_decode(const mvo_kv* kv, const float* q, size_t pos, size_t n_head,
                        size_t n_head_kv, size_t hd, float* out);

/* ---- elementwise pieces of the model step ---- */
void mvo_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out);
void mvo_rope_table(size_t n_ctx, size_t hd, float theta, float* cos_out, float* sin_out);
void mvo_rope(float* q, float* k, size_t n_head, size_t n_head_kv, size_t hd,
              const float* cos_row, const float* sin_row);
void mvo_swiglu(const float* g, const float* u, float* out, size_t n);
int  mvo_argmax(const float* x, size_t n);

/* ---- whole model (GGUF llama, paged KV of any type) ---- */
typedef struct mvo_model mvo_model;
mvo_model* mvo_model_open(const char* gguf_path, size_t ctx_override, size_t page_tokens,
                          int kv_type, int threads, int force_q8);
void   mvo_model_close(mvo_model* m);
void   mvo_model_reset(mvo_model* m);
/* config: n_ctx, n_embd, n_ff, n_layer, n_head, n_head_kv, vocab */
void   mvo_model_config(const mvo_model* m, size_t out[7]);
/* one decode step; writes vocab logits when logits != NULL. returns 0 / -1 */
int    mvo_model_forward(mvo_model* m, int token, float* logits);
/* chunked batched prefill; logits of the last token when logits != NULL */
int    mvo_model_prefill(mvo_model* m, const int* tokens, size_t n, size_t batch, float* logits);
size_t mvo_model_position(const mvo_model* m);
size_t mvo_model_kv_bytes(const mvo_model* m);

/* ---- native block formats (src/quant.cpp, src/quant_kernels.cpp): BlockQ4_0 20 bytes,
 * BlockQ8_0 36 bytes; 0 / -1 with the reference's message in mvo_last_error() ---- */
int   mvo_nq_quantize_q8_0(const float* src, size_t n, uint8_t* out);
int   mvo_nq_quantize_q4_0(const float* src, size_t n, uint8_t* out);
float mvo_nq_dot_q4_q8(const uint8_t* a, const uint8_t* x, size_t nb);
float mvo_nq_dot_q4_0(const uint8_t* a, const float* x, size_t n);
float mvo_nq_dot_q8_0(const uint8_t* a, const float* x, size_t n);
int   mvo_nq_matvec_q4_q8(const uint8_t* A, const uint8_t* x, float* y, size_t rows, size_t cols, int threads);
int   mvo_nq_matmul_q4_0_batch(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                               int threads);
int   mvo_nq_matvec_q4_0(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, int threads);
int   mvo_nq_matvec_q8_0(const uint8_t* A, const float* x, float* y, size_t rows, size_t cols, int threads);

#ifdef __cplusplus
}
#endif
#endif
