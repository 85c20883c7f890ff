// llama_model.hpp -- device-resident Llama decode/prefill with the public
// surface of MemVanta's LlamaModel (include/memvanta/llama_model.hpp:100-138):
// construct from a GGUF path, reset(), forward(token), prefill(tokens, batch,
// logits_last), position(), kv_bytes_allocated(), kv_type().  Numerics
// follow the reference step for step (src/llama_model.cpp:222-262); the paged
// KV cache (F32, F16 or Q8 pages) lives in HBM.  generate_greedy() runs the decode loop from a captured
// HIP graph, the greedy token of each step feeding the next on the device.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "profile.hpp"

namespace memvanta {
namespace hip {

class GgufFile;

struct LlamaConfig {
    std::size_t n_ctx{}, n_embd{}, n_ff{}, n_layer{}, n_head{}, n_head_kv{}, vocab{};
    float rms_eps{1e-5f}, rope_theta{10000.0f};
    std::size_t head_dim() const { return n_embd / n_head; }
    std::size_t kv_dim() const { return n_head_kv * head_dim(); }
};

// numerics of the batched prefill matmuls (tensor_matmul_batch_v06)
enum class PrefillMode { Reference = 0, Q8 = 1 };  // Q8 = MEMVANTA_FORCE_Q8_ACT=1

class LlamaModel {
public:
    // kv_type: KVCacheType order, 0 = F32, 1 = F16 (the reference's default), 2 = Q8
    LlamaModel(const std::string& gguf_path, int device = 0, std::size_t ctx_override = 0,
               std::size_t kv_page_tokens = 128, int kv_type = 1, PrefillMode mode = PrefillMode::Q8,
               std::size_t max_batch = 64);
    ~LlamaModel();
    LlamaModel(const LlamaModel&) = delete;
    LlamaModel& operator=(const LlamaModel&) = delete;

    const LlamaConfig& config() const { return c_; }
    void reset();
    const std::vector<float>& forward(int token, bool compute_logits = true);
    const std::vector<float>& prefill(const std::vector<int>& tokens, std::size_t batch_size = 64,
                                      bool compute_logits_last = true);
    // n greedy steps starting from `token`; returns the n sampled ids
    std::vector<int> generate_greedy(int token, std::size_t n);
    std::size_t position() const { return pos_; }
    std::size_t kv_bytes_allocated() const;
    int kv_type() const { return kv_type_; }
    hipStream_t stream() const { return lanes_[0].st; }
    const std::vector<float>& logits();  // copies the device logits of the last step

private:
    struct Tensor {
        std::string sname;
        std::string pname;  // profiler name: sname, or the fused members joined with '+'
        std::uint32_t type{};
        std::size_t rows{}, cols{};
        void* d{};
    };
    struct Layer {
        Tensor q, k, v, o, gate, up, down;
        // q|k|v and gate|up with rows concatenated in one allocation when the
        // parts share type and K (one GEMV launch each)
        Tensor qkv, gate_up;
        bool fused_qkv{}, fused_gu{};
        float *attn_norm{}, *ffn_norm{};
    };
    // where the q/k/v (or gate/up) rows of B tokens land in qkv_ (gu_)
    struct QkvLayout {
        float *q, *k, *v;
        std::size_t q_pitch, kv_pitch;
    };
    QkvLayout qkv_layout(const Layer& L, std::size_t B) const;

    void upload(Tensor& t, const std::string& name);
    bool upload_fused(Tensor& t, const std::vector<std::string>& names);
    float* upload_vector(const std::string& name);
    void gemv(const Tensor& w, const float* x, const int8_t* q8, const float* q8d, float* y);
    // q8/q8d: the Q8 activations of x when already quantized (null: quantize
    // here); q8_op: q8 is in the MFMA GEMM's operand order (mfma_gemm(w) holds)
    void gemm(const Tensor& w, const float* x, const int8_t* q8, const float* q8d, float* y, std::size_t B,
              bool q8_op = false);
    static bool mfma_gemm(const Tensor& w);
    hipError_t fp32_gemv(const Tensor& w, const float* x, float* y, std::size_t B);
    void decode_step(const int* d_token, bool logits, bool argmax);
    void store_kv(const QkvLayout& lay, void* const* pk, void* const* pv, const int* d_pos, std::size_t pos,
                  std::size_t B);
    // one prefill chunk on lane ln_; prev_lane >= 0: the previous chunk runs on
    // that lane and this chunk's attention of layer l waits for its KV of layer l
    void batch_step(const int* tokens, std::size_t B, bool logits, int prev_lane = -1);
    void check(hipError_t e, const char* what) const;

    // A lane: a stream and the activation buffers of one step in flight
    // ([max_batch][...] for prefill; row 0 for decode).  Decode runs on lane 0;
    // consecutive prefill chunks take the lanes in turn, so chunk c + 1
    // computes layer l while chunk c computes layer l + 1.
    struct Lane {
        hipStream_t st{};
        float *x{}, *n{}, *qkv{}, *att{}, *proj{}, *gu{}, *ff{}, *scores{};
        float* ffo{};  // down-projection output (the residual added by the next norm)
        int8_t *q8{}, *q8s{};
        float *q8d{}, *q8sd{};
        int* q8ss{};  // block sums written by the stand-alone quantizer
    };

    std::unique_ptr<GgufFile> file_;
    LlamaConfig c_;
    int device_{};
    // three lanes: pp512 of the 7B shape 7.55 K (one) / 10.3 K (two) / 11.1 K
    // (three) / 10.1 K (four) tok/s; GPU_MAX_HW_QUEUES is 4
    static constexpr int kLanes = 3;
    Lane lanes_[kLanes];
    Lane* ln_{&lanes_[0]};             // the lane the step helpers launch on
    std::vector<hipEvent_t> kv_done_;  // [lane][layer]: the KV rows of the lane's chunk at that layer are written
    int kv_type_{1};
    PrefillMode mode_;
    std::size_t page_tokens_{}, max_pages_{}, max_batch_{}, pos_{}, kv_hi_{};
    Tensor embd_, out_;
    float* out_norm_{};
    std::vector<Layer> layers_;
    std::vector<void*> allocs_;
    // paged KV: one slab per kind, page tables per layer ([layer][max_pages])
    void** pt_k_{};
    void** pt_v_{};
    float *rope_cos_{}, *rope_sin_{};
    float* rope_cur_{};                  // cos/sin row of the decode position (written by the embedding launch)
    uint8_t *kslab_{}, *vslab_{};        // every layer's KV pages, page i of layer l at slab + (l * max_pages_ + i) * kv_stride_
    std::size_t kv_stride_{};
    float* logits_d_{};
    int *d_tok_{}, *d_pos_{}, *d_hist_{};  // d_hist_[p] = greedy token sampled at position p
    int* d_prompt_{};                       // token ids of a prefill call, chunk i's at d_prompt_ + i
    int* pin_{};         // pinned host staging
    std::vector<float> logits_;
    hipGraphExec_t graph_{};   // one decode step (token and position read from device memory)
    hipGraphExec_t graphk_{};  // gsteps_ consecutive decode steps (gsteps_ > 1)
    static constexpr int kGraphSteps = 8;
    int gsteps_ = 1;
    bool fused_attn_{};  // decode attention in one launch (launch_attn_decode_fused; F16 pages)
    // L2 warm-up during a decode step (l2_warm), as shares of a GEMV's
    // weights: q|k|v by the RMSNorm before it, o by the attention, gate|up by
    // the RMSNorm before it, down by the SwiGLU, and a first share of gate|up
    // by the attention (the RMSNorm's share then follows it)
    static constexpr int kWarmSites = 5;
    float warm_frac_[kWarmSites]{};
    // kernel profiler: GEMV / GEMM launches of a step are timed while it is on
    std::unique_ptr<prof::Recorder> rec_;
    bool profiling_{};
    void prof_start();
    void prof_stop(const Tensor& w, std::size_t batch);
    void prof_flush();
};

}  // namespace hip
}  // namespace memvanta
