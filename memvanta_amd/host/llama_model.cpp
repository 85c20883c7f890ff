// llama_model.cpp -- device-resident LlamaModel (see llama_model.hpp).
// Step structure and numerics follow src/llama_model.cpp:222-262 of the
// reference: decode uses tensor_matvec numerics (Q4_0 with Q8 activations),
// prefill chunks use tensor_matmul_batch_v06 numerics in the chosen mode.
#include "llama_model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

#include "gguf.hpp"
#include "mvh_kernels.hpp"

namespace memvanta {
namespace hip {
namespace {

bool is_ffn(const std::string& n) {
    return n.find(".ffn_gate.") != std::string::npos || n.find(".ffn_up.") != std::string::npos ||
           n.find(".ffn_down.") != std::string::npos;
}

float fp16_to_fp32_host(std::uint16_t h) {
    const std::uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu;
    std::uint32_t f = h & 0x3ffu, out;
    if (e == 0) {
        if (f == 0) {
            out = s << 31;
        } else {
            std::uint32_t ee = 113;
            while ((f & 0x400u) == 0) {
                f <<= 1;
                --ee;
            }
            out = (s << 31) | (ee << 23) | ((f & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        out = (s << 31) | 0x7f800000u | (f << 13);
    } else {
        out = (s << 31) | ((e + 112u) << 23) | (f << 13);
    }
    float r;
    std::memcpy(&r, &out, 4);
    return r;
}

}  // namespace

void LlamaModel::check(hipError_t e, const char* what) const {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

LlamaModel::LlamaModel(const std::string& path, int device, std::size_t ctx_override, std::size_t kv_page_tokens,
                       int kv_type, PrefillMode mode, std::size_t max_batch)
    : file_(std::make_unique<GgufFile>(path)), device_(device), kv_type_(kv_type), mode_(mode),
      page_tokens_(kv_page_tokens ? kv_page_tokens : 128), max_batch_(std::max<std::size_t>(1, max_batch)) {
    if (kv_type != mvh::kKvF32 && kv_type != mvh::kKvF16 && kv_type != mvh::kKvQ8)
        throw std::runtime_error("unknown KV cache type id " + std::to_string(kv_type));
    const auto arch = file_->get_string("general.architecture").value_or("");
    if (arch != "llama")
        throw std::runtime_error("MemVanta real-model path currently supports GGUF architecture=llama, got: " + arch);
    auto req = [&](const char* k) {
        auto v = file_->get_u64(k);
        if (!v) throw std::runtime_error(std::string("missing GGUF metadata: ") + k);
        return static_cast<std::size_t>(*v);
    };
    c_.n_ctx = req("llama.context_length");
    c_.n_embd = req("llama.embedding_length");
    c_.n_ff = req("llama.feed_forward_length");
    c_.n_layer = req("llama.block_count");
    c_.n_head = req("llama.attention.head_count");
    c_.n_head_kv = static_cast<std::size_t>(file_->get_u64("llama.attention.head_count_kv").value_or(c_.n_head));
    c_.rms_eps = static_cast<float>(file_->get_f64("llama.attention.layer_norm_rms_epsilon").value_or(1e-5));
    c_.rope_theta = static_cast<float>(file_->get_f64("llama.rope.freq_base").value_or(10000.0));
    const auto& te = file_->tensor("token_embd.weight");
    c_.vocab = static_cast<std::size_t>(te.ne(1));
    if (te.ne(0) != c_.n_embd) throw std::runtime_error("token embedding shape mismatch");
    if (ctx_override) c_.n_ctx = std::min(c_.n_ctx, ctx_override);
    if (c_.n_embd % c_.n_head || !c_.n_head_kv || c_.n_head % c_.n_head_kv)
        throw std::runtime_error("invalid Llama head configuration");
    if (c_.n_embd % 32 || c_.n_ff % 32 || c_.head_dim() % 8)
        throw std::runtime_error("device path needs n_embd, n_ff % 32 == 0 and head_dim % 8 == 0");

    check(hipSetDevice(device_), "hipSetDevice");
    check(hipStreamCreateWithFlags(&lanes_[0].st, hipStreamNonBlocking), "hipStreamCreate");
    auto dalloc = [&](std::size_t bytes) {
        void* p = nullptr;
        check(hipMalloc(&p, std::max<std::size_t>(bytes, 16)), "hipMalloc");
        allocs_.push_back(p);
        return p;
    };

    upload(embd_, "token_embd.weight");
    if (file_->has_tensor("output.weight")) upload(out_, "output.weight");
    else out_ = embd_;  // tied output (src/llama_model.cpp:228)
    out_norm_ = upload_vector("output_norm.weight");
    layers_.resize(c_.n_layer);
    for (std::size_t i = 0; i < c_.n_layer; ++i) {
        auto n = [&](const char* s) { return "blk." + std::to_string(i) + s; };
        auto& L = layers_[i];
        L.attn_norm = upload_vector(n(".attn_norm.weight"));
        L.fused_qkv = upload_fused(L.qkv, {n(".attn_q.weight"), n(".attn_k.weight"), n(".attn_v.weight")});
        if (!L.fused_qkv) {
            upload(L.q, n(".attn_q.weight"));
            upload(L.k, n(".attn_k.weight"));
            upload(L.v, n(".attn_v.weight"));
        }
        upload(L.o, n(".attn_output.weight"));
        L.ffn_norm = upload_vector(n(".ffn_norm.weight"));
        L.fused_gu = upload_fused(L.gate_up, {n(".ffn_gate.weight"), n(".ffn_up.weight")});
        if (!L.fused_gu) {
            upload(L.gate, n(".ffn_gate.weight"));
            upload(L.up, n(".ffn_up.weight"));
        }
        upload(L.down, n(".ffn_down.weight"));
        const auto rows = [&](const Tensor& f, const Tensor& a) { return f.d ? f.rows : a.rows; };
        if (rows(L.qkv, L.q) != (L.fused_qkv ? c_.n_embd + 2 * c_.kv_dim() : c_.n_embd) ||
            (!L.fused_qkv && (L.k.rows != c_.kv_dim() || L.v.rows != c_.kv_dim())) || L.o.rows != c_.n_embd ||
            rows(L.gate_up, L.gate) != (L.fused_gu ? 2 * c_.n_ff : c_.n_ff) || L.down.rows != c_.n_embd ||
            L.down.cols != c_.n_ff)
            throw std::runtime_error("layer " + std::to_string(i) + ": weight shapes do not match the config");
    }

    // RoPE table computed on the host with the C library, as the reference
    // does (src/llama_model.cpp:233), then uploaded
    const std::size_t hd = c_.head_dim(), half = hd / 2;
    std::vector<float> co(c_.n_ctx * half), si(c_.n_ctx * half);
    for (std::size_t p = 0; p < c_.n_ctx; ++p)
        for (std::size_t i = 0; i < half; ++i) {
            const float inv = std::pow(c_.rope_theta, -2.0f * static_cast<float>(i) / static_cast<float>(hd));
            const float a = static_cast<float>(p) * inv;
            co[p * half + i] = std::cos(a);
            si[p * half + i] = std::sin(a);
        }
    rope_cos_ = static_cast<float*>(dalloc(co.size() * 4));
    rope_sin_ = static_cast<float*>(dalloc(si.size() * 4));
    check(hipMemcpy(rope_cos_, co.data(), co.size() * 4, hipMemcpyHostToDevice), "upload rope");
    check(hipMemcpy(rope_sin_, si.data(), si.size() * 4, hipMemcpyHostToDevice), "upload rope");
    rope_cur_ = static_cast<float*>(dalloc(c_.head_dim() * 4));

    // paged KV cache: the pages of every layer preallocated in HBM, addressed
    // through per-layer page tables; page stride 256-byte aligned (a Q8 page
    // ends with its float row scales)
    max_pages_ = (c_.n_ctx + page_tokens_ - 1) / page_tokens_;
    const std::size_t stride = (mvh::kv_page_bytes(kv_type_, page_tokens_, c_.kv_dim()) + 255) / 256 * 256;
    auto* kslab = static_cast<uint8_t*>(dalloc(c_.n_layer * max_pages_ * stride));
    auto* vslab = static_cast<uint8_t*>(dalloc(c_.n_layer * max_pages_ * stride));
    kslab_ = kslab;
    vslab_ = vslab;
    kv_stride_ = stride;
    std::vector<void*> tk(c_.n_layer * max_pages_), tv(c_.n_layer * max_pages_);
    for (std::size_t i = 0; i < tk.size(); ++i) {
        tk[i] = kslab + i * stride;
        tv[i] = vslab + i * stride;
    }
    pt_k_ = static_cast<void**>(dalloc(tk.size() * sizeof(void*)));
    pt_v_ = static_cast<void**>(dalloc(tv.size() * sizeof(void*)));
    check(hipMemcpy(pt_k_, tk.data(), tk.size() * sizeof(void*), hipMemcpyHostToDevice), "page table");
    check(hipMemcpy(pt_v_, tv.data(), tv.size() * sizeof(void*), hipMemcpyHostToDevice), "page table");

    const std::size_t B = max_batch_, D = c_.n_embd, F = c_.n_ff, KV = c_.kv_dim(), W = std::max(D, F);
    for (Lane& l : lanes_) {
        if (&l != &lanes_[0]) check(hipStreamCreateWithFlags(&l.st, hipStreamNonBlocking), "hipStreamCreate");
        l.x = static_cast<float*>(dalloc(B * D * 4));
        l.n = static_cast<float*>(dalloc(B * D * 4));
        l.qkv = static_cast<float*>(dalloc(B * (D + 2 * KV) * 4));
        l.att = static_cast<float*>(dalloc(B * D * 4));
        l.proj = static_cast<float*>(dalloc(B * D * 4));
        l.gu = static_cast<float*>(dalloc(B * 2 * F * 4));
        l.ff = static_cast<float*>(dalloc(B * F * 4));
        l.scores = static_cast<float*>(dalloc(B * c_.n_head * c_.n_ctx * 4));
        l.ffo = static_cast<float*>(dalloc(B * D * 4));
        l.q8 = static_cast<int8_t*>(dalloc(mvh::q8_op_bytes(B, W)));  // row-major or operand order
        l.q8d = static_cast<float*>(dalloc(B * (W / 32) * 4));
        l.q8s = static_cast<int8_t*>(dalloc(mvh::q8_op_bytes(B, W)));
        l.q8sd = static_cast<float*>(dalloc(B * (W / 32) * 4));
        l.q8ss = static_cast<int*>(dalloc(B * (W / 32) * 4));
    }
    kv_done_.assign(kLanes * c_.n_layer, nullptr);
    for (hipEvent_t& e : kv_done_) check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    logits_d_ = static_cast<float*>(dalloc(c_.vocab * 4));
    d_tok_ = static_cast<int*>(dalloc(16));
    d_hist_ = static_cast<int*>(dalloc(4 * (c_.n_ctx + 1)));
    d_pos_ = static_cast<int*>(dalloc(16));
    d_prompt_ = static_cast<int*>(dalloc(4 * (c_.n_ctx + B)));
    rec_ = std::make_unique<prof::Recorder>(lanes_[0].st);
    check(hipHostMalloc(reinterpret_cast<void**>(&pin_), 4 * (c_.n_ctx + B + 8), hipHostMallocDefault),
          "hipHostMalloc");
    logits_.resize(c_.vocab);
    fused_attn_ = kv_type_ == mvh::kKvF16 && mvh::attn_decode_fused_ok(c_.head_dim(), c_.n_ctx, page_tokens_);
    // default shares: what the RMSNorm and attention launches can fetch while
    // their own work runs (the SwiGLU launch warming ffn_down measured
    // slower); with Q8_0 layers (the TinyLlama shape's 5.6 MB q|k|v) the
    // attention norm warms all of q|k|v.  MVH_L2_WARM=0 turns the warm-up
    // off, "a,b,c,d,e" sets the five shares
    const bool q8_layers = !layers_.empty() && (layers_[0].fused_qkv ? layers_[0].qkv : layers_[0].q).type == 8;
    const float defaults_q4[kWarmSites] = {0.5f, 1.0f, 0.3f, 0.0f, 0.15f};
    const float defaults_q8[kWarmSites] = {1.0f, 1.0f, 0.3f, 0.0f, 0.15f};
    std::copy(q8_layers ? defaults_q8 : defaults_q4, (q8_layers ? defaults_q8 : defaults_q4) + kWarmSites, warm_frac_);
    if (const char* e = getenv("MVH_L2_WARM")) {
        float f[kWarmSites] = {};
        const int n = std::sscanf(e, "%f,%f,%f,%f,%f", &f[0], &f[1], &f[2], &f[3], &f[4]);
        if (n == kWarmSites || (n == 1 && f[0] == 0.0f))
            for (int i = 0; i < kWarmSites; ++i) warm_frac_[i] = std::clamp(f[i], 0.0f, 1.0f);
    }
    reset();
}

LlamaModel::~LlamaModel() {
    (void)hipSetDevice(device_);
    for (Lane& l : lanes_)
        if (l.st) (void)hipStreamSynchronize(l.st);
    if (graph_) (void)hipGraphExecDestroy(graph_);
    if (graphk_) (void)hipGraphExecDestroy(graphk_);
    for (hipEvent_t e : kv_done_)
        if (e) (void)hipEventDestroy(e);
    for (void* p : allocs_) (void)hipFree(p);
    if (pin_) (void)hipHostFree(pin_);
    for (Lane& l : lanes_)
        if (l.st) (void)hipStreamDestroy(l.st);
}

void LlamaModel::upload(Tensor& t, const std::string& name) {
    const auto& g = file_->tensor(name);
    if (g.dims.size() < 2) throw std::runtime_error("matvec requires rank-2 tensor: " + name);
    t.sname = t.pname = name;
    t.type = g.type;
    t.cols = static_cast<std::size_t>(g.ne(0));
    t.rows = static_cast<std::size_t>(g.ne(1));
    if (t.type != 0 && t.type != 1 && t.type != 2 && t.type != 8 && t.type != 14)
        throw std::runtime_error(std::string("unsupported device tensor type ") + type_name(t.type) + ": " + name);
    if (!g.nbytes) throw std::runtime_error("bad tensor size: " + name);
    check(hipMalloc(&t.d, g.nbytes), "hipMalloc tensor");
    allocs_.push_back(t.d);
    check(hipMemcpy(t.d, file_->tensor_data(g), g.nbytes, hipMemcpyHostToDevice), "tensor upload");
}

// One allocation holding the rows of `names` back to back (same type and K).
bool LlamaModel::upload_fused(Tensor& t, const std::vector<std::string>& names) {
    std::size_t bytes = 0, rows = 0;
    const auto& g0 = file_->tensor(names[0]);
    for (const auto& nm : names) {
        const auto& g = file_->tensor(nm);
        if (g.dims.size() < 2 || g.type != g0.type || g.ne(0) != g0.ne(0) || !g.nbytes) return false;
        if (g.type != 0 && g.type != 1 && g.type != 2 && g.type != 8 && g.type != 14) return false;
        bytes += g.nbytes;
        rows += static_cast<std::size_t>(g.ne(1));
    }
    t.sname = t.pname = names[0];
    for (std::size_t i = 1; i < names.size(); ++i) t.pname += "+" + names[i];
    t.type = g0.type;
    t.cols = static_cast<std::size_t>(g0.ne(0));
    t.rows = rows;
    check(hipMalloc(&t.d, bytes), "hipMalloc tensor");
    allocs_.push_back(t.d);
    std::size_t off = 0;
    for (const auto& nm : names) {
        const auto& g = file_->tensor(nm);
        check(hipMemcpy(static_cast<uint8_t*>(t.d) + off, file_->tensor_data(g), g.nbytes, hipMemcpyHostToDevice),
              "tensor upload");
        off += g.nbytes;
    }
    return true;
}

LlamaModel::QkvLayout LlamaModel::qkv_layout(const Layer& L, std::size_t B) const {
    const std::size_t D = c_.n_embd, KV = c_.kv_dim();
    if (L.fused_qkv) return {ln_->qkv, ln_->qkv + D, ln_->qkv + D + KV, D + 2 * KV, D + 2 * KV};
    return {ln_->qkv, ln_->qkv + B * D, ln_->qkv + B * (D + KV), D, KV};
}

float* LlamaModel::upload_vector(const std::string& name) {
    const auto& g = file_->tensor(name);
    if (g.elements() != c_.n_embd) throw std::runtime_error("tensor vector size mismatch: " + name);
    std::vector<float> h(c_.n_embd);
    const std::byte* p = file_->tensor_data(g);
    if (g.type == 0) {
        std::memcpy(h.data(), p, h.size() * 4);
    } else if (g.type == 1) {
        for (std::size_t i = 0; i < h.size(); ++i) {
            std::uint16_t v;
            std::memcpy(&v, p + 2 * i, 2);
            h[i] = fp16_to_fp32_host(v);
        }
    } else {
        throw std::runtime_error(std::string("unsupported vector tensor type ") + type_name(g.type) + ": " + name);
    }
    void* d = nullptr;
    check(hipMalloc(&d, h.size() * 4), "hipMalloc");
    allocs_.push_back(d);
    check(hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice), "vector upload");
    return static_cast<float*>(d);
}

// tensor_matvec numerics (src/gguf_kernels.cpp:244-253)
void LlamaModel::prof_start() {
    if (profiling_) check(rec_->start(), "profiler event");
}

void LlamaModel::prof_stop(const Tensor& w, std::size_t batch) {
    if (profiling_) check(rec_->stop(w.pname, batch), "profiler event");
}

void LlamaModel::prof_flush() {
    if (profiling_) check(rec_->flush(), "profiler events");
}

void LlamaModel::gemv(const Tensor& w, const float* x, const int8_t* q8, const float* q8d, float* y) {
    const auto* W = static_cast<const uint8_t*>(w.d);
    hipError_t e;
    prof_start();
    switch (w.type) {
        case 2:
            if (q8) {
                e = mvh::launch_gemv_q4_0(W, q8, q8d, y, w.rows, w.cols, ln_->st);
            } else if (mvh::gemv_q4_0_rows16_ok(w.cols)) {
                e = mvh::launch_gemv_q4_0_rows16(W, x, nullptr, nullptr, y, w.rows, w.cols, ln_->st);
            } else {
                e = mvh::launch_quantize_q8(x, ln_->q8s, ln_->q8sd, ln_->q8ss, 1, w.cols, ln_->st);
                if (e == hipSuccess) e = mvh::launch_gemv_q4_0(W, ln_->q8s, ln_->q8sd, y, w.rows, w.cols, ln_->st);
            }
            break;
        default: e = fp32_gemv(w, x, y, 1); break;
    }
    check(e, w.sname.c_str());
    prof_stop(w, 1);
}

// tensor_matvec / tensor_matmul_batch with fp32 activations for Q8_0, Q6_K,
// F32 and F16 weights (src/gguf_kernels.cpp:247-250,:257): y[b*rows + r]
hipError_t LlamaModel::fp32_gemv(const Tensor& w, const float* x, float* y, std::size_t B) {
    const auto* W = static_cast<const uint8_t*>(w.d);
    switch (w.type) {
        case 8: return mvh::launch_gemv_q8_0(W, x, y, w.rows, w.cols, B, ln_->st);
        case 14: return mvh::launch_gemv_q6_k(W, x, y, w.rows, w.cols, B, ln_->st);
        case 0: return mvh::launch_gemv_f32(reinterpret_cast<const float*>(W), x, y, w.rows, w.cols, B, ln_->st);
        case 1: return mvh::launch_gemv_f16(reinterpret_cast<const uint16_t*>(W), x, y, w.rows, w.cols, B, ln_->st);
    }
    return hipErrorInvalidValue;
}

bool LlamaModel::mfma_gemm(const Tensor& w) { return w.type == 2 && mvh::gemm_q4_0_mfma_ok(w.cols); }

// tensor_matmul_batch_v06 numerics (src/gguf_kernels.cpp:261-271) over B rows
void LlamaModel::gemm(const Tensor& w, const float* x, const int8_t* q8, const float* q8d, float* y, std::size_t B,
                      bool q8_op) {
    const auto* W = static_cast<const uint8_t*>(w.d);
    const std::size_t rows = w.rows, cols = w.cols, nb = cols / 32;
    hipError_t e = hipSuccess;
    prof_start();
    if (B < 2 || (w.type != 2 && w.type != 8) || cols % 32) {  // tensor_matmul_batch: fp32 per token
        if (w.type == 2) e = mvh::launch_gemv_q4_0_f32act(W, x, y, rows, cols, B, ln_->st);
        else e = fp32_gemv(w, x, y, B);
    } else if (mode_ == PrefillMode::Q8) {
        if (w.type == 2) {
            if (!q8) {
                q8_op = mfma_gemm(w);
                e = mvh::launch_quantize_q8(x, ln_->q8s, ln_->q8sd, ln_->q8ss, B, cols, ln_->st, q8_op);
                q8 = ln_->q8s;
                q8d = ln_->q8sd;
            }
            if (q8_op && !mfma_gemm(w))
                throw std::logic_error("operand-order activations for a non-MFMA tensor: " + w.sname);
            if (e == hipSuccess && q8_op) {
                e = mvh::launch_gemm_q4_0_q8_mfma(W, q8, q8d, y, rows, cols, B, ln_->st);
            } else {
                e = mvh::launch_gemv_q4_0(W, q8, q8d, y, rows, cols, ln_->st, B);
            }
        } else {
            e = mvh::launch_gemv_q8_0(W, x, y, rows, cols, B, ln_->st);
        }
    } else {
        const std::size_t step = is_ffn(w.sname) ? 8 : 4, blocked = B / step * step;
        e = mvh::launch_batch4_f32act(w.type, W, x, y, rows, cols, blocked, ln_->st);
        if (e == hipSuccess && blocked < B) {
            if (w.type == 2)
                e = mvh::launch_gemv_q4_0_f32act(W, x + blocked * cols, y + blocked * rows, rows, cols, B - blocked,
                                                 ln_->st);
            else
                e = mvh::launch_gemv_q8_0(W, x + blocked * cols, y + blocked * rows, rows, cols, B - blocked, ln_->st);
        }
    }
    check(e, w.sname.c_str());
    prof_stop(w, B);
}

// The L2 warm-up of a decode GEMV's weights (mvh::l2_warm): a GEMV whose
// one-token kernel reads one contiguous chunk of rows per workgroup
// (mvh::gemv_decode_rows_per_wg: Q4_0, Q8_0 at K = 2048 / 4096, Q6_K) has its
// chunks from the fraction `from` to from + share pulled into the L2 of the
// XCD that will read them; other GEMVs get none.
static mvh::L2Warm l2_warm_for(std::uint32_t type, std::size_t rows, std::size_t cols, const void* d, float from,
                               float share) {
    mvh::L2Warm r;
    const std::size_t per_wg = mvh::gemv_decode_rows_per_wg(type, rows, cols);
    const std::size_t row_bytes = type == 2 ? cols / 32 * 18 : type == 8 ? cols / 32 * 34 : cols / 256 * 210;
    if (!per_wg || share <= 0.0f || (per_wg * row_bytes) % 16) return r;
    const float chunks = static_cast<float>((rows + per_wg - 1) / per_wg);
    const unsigned whole = static_cast<unsigned>(rows / per_wg);  // a partial last chunk is left cold
    r.base = static_cast<const uint8_t*>(d);
    r.chunk = static_cast<unsigned>(per_wg * row_bytes);
    r.c0 = std::min(whole, static_cast<unsigned>(from * chunks));
    r.c1 = std::min(whole, static_cast<unsigned>((from + share) * chunks));
    return r;
}

// One decode step (LlamaModel::forward, src/llama_model.cpp:253-259) for the
// token in *d_token at position *d_pos_.
void LlamaModel::decode_step(const int* d_token, bool logits, bool argmax) {
    const Lane& a = *ln_;
    const std::size_t D = c_.n_embd, F = c_.n_ff, hd = c_.head_dim();
    // the embedding launch also copies the RoPE row of the position for the fused attention
    check(mvh::launch_embed(embd_.type, static_cast<const uint8_t*>(embd_.d), D, d_token, 1, a.x, a.st, d_pos_,
                            rope_cos_, rope_sin_, hd / 2, fused_attn_ ? rope_cur_ : nullptr),
          "embed");
    auto warm = [&](const Tensor& w, float from, float share) {
        return l2_warm_for(w.type, w.rows, w.cols, w.d, from, share);
    };
    for (std::size_t li = 0; li < c_.n_layer; ++li) {
        auto& L = layers_[li];
        const auto lay = qkv_layout(L, 1);
        const bool q8_in = L.fused_qkv ? L.qkv.type == 2 : (L.q.type == 2 || L.k.type == 2 || L.v.type == 2);
        check(mvh::launch_rmsnorm(a.x, li ? a.ffo : nullptr, L.attn_norm, a.n, q8_in ? a.q8 : nullptr, a.q8d, 1, D,
                                  c_.rms_eps, a.st, false,
                                  warm(L.fused_qkv ? L.qkv : L.q, 0.0f, warm_frac_[0])),
              "rmsnorm");
        if (L.fused_qkv) {
            gemv(L.qkv, a.n, L.qkv.type == 2 ? a.q8 : nullptr, a.q8d, a.qkv);
        } else {
            gemv(L.q, a.n, L.q.type == 2 ? a.q8 : nullptr, a.q8d, lay.q);
            gemv(L.k, a.n, L.k.type == 2 ? a.q8 : nullptr, a.q8d, lay.k);
            gemv(L.v, a.n, L.v.type == 2 ? a.q8 : nullptr, a.q8d, lay.v);
        }
        void* const* pk = pt_k_ + li * max_pages_;
        void* const* pv = pt_v_ + li * max_pages_;
        // the attention kernels write the o projection's Q8 activations (32-element head slices are Q8 blocks)
        const bool o_q8 = L.o.type == 2 && hd % 32 == 0 && L.o.cols == c_.n_head * hd;
        if (fused_attn_) {
            const std::size_t layer_off = li * max_pages_ * kv_stride_;
            check(mvh::launch_attn_decode_fused(lay.q, lay.k, lay.v, rope_cur_, d_pos_,
                                                reinterpret_cast<uint16_t*>(kslab_ + layer_off),
                                                reinterpret_cast<uint16_t*>(vslab_ + layer_off), page_tokens_,
                                                kv_stride_ / 2, a.att,
                                                o_q8 ? a.q8 : nullptr, a.q8d, c_.n_head, c_.n_head_kv, hd, c_.n_ctx,
                                                a.st, warm(L.o, 0.0f, warm_frac_[1]),
                                                warm(L.fused_gu ? L.gate_up : L.gate, 0.0f, warm_frac_[4])),
                  "attention");
        } else if (hd % 32 == 0) {  // F32 / Q8 pages: the chunk kernels with one query token
            store_kv(lay, pk, pv, d_pos_, 0, 1);
            check(mvh::launch_attn_prefill(kv_type_, pk, pv, lay.q, lay.q_pitch, a.scores, a.att, o_q8 ? a.q8 : nullptr,
                                           a.q8d, false, d_pos_, 0, c_.n_ctx, 1, c_.n_head, c_.n_head_kv, hd,
                                           c_.kv_dim(), page_tokens_, a.st),
                  "attention");
        } else {
            store_kv(lay, pk, pv, d_pos_, 0, 1);
            check(mvh::launch_attn(kv_type_, pk, pv, lay.q, lay.q_pitch, a.scores, a.att, d_pos_, 0, c_.n_ctx, 1,
                                   c_.n_head, c_.n_head_kv, hd, c_.kv_dim(), page_tokens_, a.st,
                                   o_q8 ? a.q8 : nullptr, a.q8d),
                  "attention");
        }
        gemv(L.o, a.att, o_q8 ? a.q8 : nullptr, a.q8d, a.proj);
        const bool q8_ffn = L.fused_gu ? L.gate_up.type == 2 : (L.gate.type == 2 || L.up.type == 2);
        check(mvh::launch_rmsnorm(a.x, a.proj, L.ffn_norm, a.n, q8_ffn ? a.q8 : nullptr, a.q8d, 1, D, c_.rms_eps, a.st,
                                  false,
                                  warm(L.fused_gu ? L.gate_up : L.gate, warm_frac_[4], warm_frac_[2])),
              "rmsnorm");
        float* g = a.gu;
        float* u = a.gu + F;  // one token: the fused and the separate layouts coincide
        if (L.fused_gu) {
            gemv(L.gate_up, a.n, L.gate_up.type == 2 ? a.q8 : nullptr, a.q8d, a.gu);
        } else {
            gemv(L.gate, a.n, L.gate.type == 2 ? a.q8 : nullptr, a.q8d, g);
            gemv(L.up, a.n, L.up.type == 2 ? a.q8 : nullptr, a.q8d, u);
        }
        check(mvh::launch_swiglu(g, u, 2 * F, a.ff, L.down.type == 2 ? a.q8 : nullptr, a.q8d, 1, F, a.st, false,
                                 warm(L.down, 0.0f, warm_frac_[3])),
              "swiglu");
        gemv(L.down, a.ff, L.down.type == 2 ? a.q8 : nullptr, a.q8d, a.ffo);
    }
    if (logits || argmax) {
        check(mvh::launch_rmsnorm(a.x, a.ffo, out_norm_, a.n, out_.type == 2 ? a.q8 : nullptr, a.q8d, 1, D, c_.rms_eps,
                                  a.st),
              "rmsnorm");
        gemv(out_, a.n, out_.type == 2 ? a.q8 : nullptr, a.q8d, logits_d_);
    }
    if (argmax) check(mvh::launch_argmax(logits_d_, c_.vocab, 1, d_tok_, d_pos_, d_hist_, a.st), "argmax");
}

// One prefill chunk (LlamaModel::forward_batch_impl, src/llama_model.cpp:240-252).
void LlamaModel::batch_step(const int* d_tokens, std::size_t B, bool logits, int prev_lane) {
    const Lane& a = *ln_;
    const int lane = static_cast<int>(ln_ - lanes_);
    const std::size_t D = c_.n_embd, F = c_.n_ff, hd = c_.head_dim();
    check(mvh::launch_embed(embd_.type, static_cast<const uint8_t*>(embd_.d), D, d_tokens, B, a.x, a.st), "embed");
    const bool q8mode = mode_ == PrefillMode::Q8 && B >= 2;
    for (std::size_t li = 0; li < c_.n_layer; ++li) {
        auto& L = layers_[li];
        const auto lay = qkv_layout(L, B);
        // the norm / SwiGLU kernels write the Q8 activations in the MFMA
        // GEMM's operand order when every consumer of them is that GEMM
        const bool op_qkv = q8mode && (L.fused_qkv ? mfma_gemm(L.qkv)
                                                   : mfma_gemm(L.q) && mfma_gemm(L.k) && mfma_gemm(L.v));
        const bool op_gu = q8mode && (L.fused_gu ? mfma_gemm(L.gate_up) : mfma_gemm(L.gate) && mfma_gemm(L.up));
        const bool op_down = q8mode && mfma_gemm(L.down);
        check(mvh::launch_rmsnorm(a.x, li ? a.ffo : nullptr, L.attn_norm, a.n, q8mode ? a.q8 : nullptr, a.q8d, B, D,
                                  c_.rms_eps, a.st, op_qkv),
              "rmsnorm");
        if (L.fused_qkv) {
            gemm(L.qkv, a.n, q8mode ? a.q8 : nullptr, a.q8d, a.qkv, B, op_qkv);
        } else {
            gemm(L.q, a.n, q8mode ? a.q8 : nullptr, a.q8d, lay.q, B, op_qkv);
            gemm(L.k, a.n, q8mode ? a.q8 : nullptr, a.q8d, lay.k, B, op_qkv);
            gemm(L.v, a.n, q8mode ? a.q8 : nullptr, a.q8d, lay.v, B, op_qkv);
        }
        void* const* pk = pt_k_ + li * max_pages_;
        void* const* pv = pt_v_ + li * max_pages_;
        store_kv(lay, pk, pv, nullptr, pos_, B);
        // this chunk's attention of the layer reads the rows of every earlier
        // chunk: it waits for the previous chunk's event, and records its own
        // only after that wait, so the event of chunk c stands for the rows
        // of chunks 0..c (with three lanes chunk c - 2 runs on a third stream)
        if (prev_lane >= 0)
            check(hipStreamWaitEvent(a.st, kv_done_[prev_lane * c_.n_layer + li], 0), "event wait");
        check(hipEventRecord(kv_done_[lane * c_.n_layer + li], a.st), "event record");
        // the softmax-V kernel also writes the o projection's Q8 activations
        // (32-element head slices are Q8 blocks), in the MFMA GEMM's operand
        // order when the projection runs there
        const bool o_q8 = q8mode && L.o.type == 2 && hd % 32 == 0 && L.o.cols == c_.n_head * hd;
        const bool o_op = o_q8 && mfma_gemm(L.o);
        if (hd % 32 == 0) {  // scores + softmax once per (token, head), V tiles shared by the chunk's tokens
            check(mvh::launch_attn_prefill(kv_type_, pk, pv, lay.q, lay.q_pitch, a.scores, a.att, o_q8 ? a.q8 : nullptr,
                                           a.q8d,
                                           o_op, nullptr, pos_, pos_ + B, B, c_.n_head, c_.n_head_kv, hd,
                                           c_.kv_dim(), page_tokens_, a.st),
                  "attention");
        } else {
            check(mvh::launch_attn(kv_type_, pk, pv, lay.q, lay.q_pitch, a.scores, a.att, nullptr, pos_, pos_ + B, B,
                                   c_.n_head,
                                   c_.n_head_kv, hd, c_.kv_dim(), page_tokens_, a.st, o_q8 ? a.q8 : nullptr, a.q8d,
                                   o_op),
                  "attention");
        }
        gemm(L.o, a.att, o_q8 ? a.q8 : nullptr, a.q8d, a.proj, B, o_op);
        check(mvh::launch_rmsnorm(a.x, a.proj, L.ffn_norm, a.n, q8mode ? a.q8 : nullptr, a.q8d, B, D, c_.rms_eps, a.st,
                                  op_gu),
              "rmsnorm");
        float* g = a.gu;
        float* u = L.fused_gu ? a.gu + F : a.gu + B * F;
        const std::size_t pitch = L.fused_gu ? 2 * F : F;
        if (L.fused_gu) {
            gemm(L.gate_up, a.n, q8mode ? a.q8 : nullptr, a.q8d, a.gu, B, op_gu);
        } else {
            gemm(L.gate, a.n, q8mode ? a.q8 : nullptr, a.q8d, g, B, op_gu);
            gemm(L.up, a.n, q8mode ? a.q8 : nullptr, a.q8d, u, B, op_gu);
        }
        check(mvh::launch_swiglu(g, u, pitch, a.ff, q8mode ? a.q8 : nullptr, a.q8d, B, F, a.st, op_down), "swiglu");
        gemm(L.down, a.ff, q8mode ? a.q8 : nullptr, a.q8d, a.ffo, B, op_down);
    }
    if (logits) {
        float* xl = a.x + (B - 1) * D;
        check(mvh::launch_rmsnorm(xl, a.ffo + (B - 1) * D, out_norm_, a.n, out_.type == 2 ? a.q8 : nullptr, a.q8d, 1, D,
                                  c_.rms_eps, a.st),
              "rmsnorm");
        gemv(out_, a.n, out_.type == 2 ? a.q8 : nullptr, a.q8d, logits_d_);
    }
}

void LlamaModel::reset() {
    pos_ = 0;
    kv_hi_ = 0;
}

std::size_t LlamaModel::kv_bytes_allocated() const {
    // pages are allocated lazily in the reference (PagedKVCache::ensure):
    // every page any written position touched, in every layer
    const std::size_t pages = (kv_hi_ + page_tokens_ - 1) / page_tokens_;
    return c_.n_layer * pages * mvh::kv_page_pair_bytes_ref(kv_type_, page_tokens_, c_.kv_dim());
}

// RoPE of q and k of B tokens at positions pos.. (*d_pos when non-null), then
// PagedKVCache::write of k and v: fused into the RoPE kernel for F16 pages,
// a write kernel of its own for F32 / Q8 (Q8 needs the whole row's max).
void LlamaModel::store_kv(const QkvLayout& lay, void* const* pk, void* const* pv, const int* d_pos, std::size_t pos,
                          std::size_t B) {
    // F16 and F32 rows are written by the RoPE launch; a Q8 row's scale
    // spans every head, so Q8 pages get their own write launch
    const bool fused = kv_type_ != mvh::kKvQ8;
    check(mvh::launch_rope_kv(lay.q, lay.q_pitch, lay.k, lay.v, lay.kv_pitch, rope_cos_, rope_sin_, d_pos, pos, B,
                              c_.n_head, c_.n_head_kv, c_.head_dim(), kv_type_, fused ? pk : nullptr,
                              fused ? pv : nullptr, page_tokens_, ln_->st),
          "rope/kv");
    if (!fused)
        check(mvh::launch_kv_write(kv_type_, pk, pv, lay.k, lay.v, lay.kv_pitch, d_pos, pos, B, c_.kv_dim(),
                                   page_tokens_, ln_->st),
              "kv write");
}

const std::vector<float>& LlamaModel::logits() {
    check(hipMemcpyAsync(logits_.data(), logits_d_, c_.vocab * 4, hipMemcpyDeviceToHost, ln_->st), "logits copy");
    check(hipStreamSynchronize(ln_->st), "sync");
    return logits_;
}

const std::vector<float>& LlamaModel::forward(int token, bool compute_logits) {
    ln_ = &lanes_[0];
    if (token < 0 || static_cast<std::size_t>(token) >= c_.vocab) throw std::runtime_error("token id out of range");
    if (pos_ >= c_.n_ctx) throw std::runtime_error("context exhausted");
    check(hipSetDevice(device_), "hipSetDevice");
    pin_[0] = token;
    pin_[1] = static_cast<int>(pos_);
    check(hipMemcpyAsync(d_tok_, &pin_[0], 4, hipMemcpyHostToDevice, ln_->st), "token upload");
    check(hipMemcpyAsync(d_pos_, &pin_[1], 4, hipMemcpyHostToDevice, ln_->st), "pos upload");
    profiling_ = prof::enabled();
    decode_step(d_tok_, compute_logits, false);
    prof_flush();
    ++pos_;
    kv_hi_ = std::max(kv_hi_, pos_);
    if (compute_logits) return logits();
    check(hipStreamSynchronize(ln_->st), "sync");
    return logits_;
}

const std::vector<float>& LlamaModel::prefill(const std::vector<int>& tokens, std::size_t batch_size,
                                              bool compute_logits_last) {
    if (tokens.empty()) return logits_;
    batch_size = std::max<std::size_t>(1, batch_size);
    if (batch_size > max_batch_) throw std::runtime_error("prefill batch larger than the model's max_batch");
    check(hipSetDevice(device_), "hipSetDevice");
    // chunks take the lanes in turn (one lane while profiling: the profiler's
    // events live on lane 0); a chunk's tokens are staged at its own offset,
    // so no staging slot is reused before the final sync
    profiling_ = prof::enabled();
    const int lanes = profiling_ ? 1 : kLanes;
    int prev = -1;
    std::size_t chunk = 0;
    // every lane drained and lane 0 current again before the call returns,
    // also when it throws: a later forward / reset / generate on lane 0 must
    // not race with chunks still writing the shared KV slab
    auto drain = [&](bool quiet) {
        hipError_t first = hipSuccess;
        for (Lane& l : lanes_) {
            const hipError_t e = hipStreamSynchronize(l.st);
            if (first == hipSuccess) first = e;
        }
        ln_ = &lanes_[0];
        if (!quiet) check(first, "sync");
    };
    try {
        for (std::size_t i = 0; i < tokens.size(); i += batch_size, ++chunk) {
            const std::size_t B = std::min(batch_size, tokens.size() - i);
            const char* err = nullptr;
            if (pos_ + B > c_.n_ctx) err = "context exhausted";
            for (std::size_t b = 0; b < B && !err; ++b)
                if (tokens[i + b] < 0 || static_cast<std::size_t>(tokens[i + b]) >= c_.vocab)
                    err = "token id out of range";
            if (err) throw std::runtime_error(err);  // the chunks before this one complete (drained below)
            const bool last = compute_logits_last && i + B == tokens.size();
            const int lane = static_cast<int>(chunk % lanes);
            ln_ = &lanes_[lane];
            std::memcpy(pin_ + i, tokens.data() + i, B * 4);
            check(hipMemcpyAsync(d_prompt_ + i, pin_ + i, B * 4, hipMemcpyHostToDevice, ln_->st), "token upload");
            batch_step(d_prompt_ + i, B, last, lanes > 1 ? prev : -1);
            prof_flush();
            prev = lane;
            pos_ += B;
            kv_hi_ = std::max(kv_hi_, pos_);
            if (last)
                check(hipMemcpyAsync(logits_.data(), logits_d_, c_.vocab * 4, hipMemcpyDeviceToHost, ln_->st),
                      "logits copy");
        }
    } catch (...) {
        drain(true);  // secondary errors ignored: the first one is what the caller sees
        throw;
    }
    drain(false);
    return logits_;
}

std::vector<int> LlamaModel::generate_greedy(int token, std::size_t n) {
    ln_ = &lanes_[0];
    if (token < 0 || static_cast<std::size_t>(token) >= c_.vocab) throw std::runtime_error("token id out of range");
    if (pos_ + n > c_.n_ctx) throw std::runtime_error("context exhausted");
    std::vector<int> out(n);
    if (!n) return out;
    check(hipSetDevice(device_), "hipSetDevice");
    pin_[0] = token;
    pin_[1] = static_cast<int>(pos_);
    check(hipMemcpyAsync(d_tok_, &pin_[0], 4, hipMemcpyHostToDevice, ln_->st), "token upload");
    check(hipMemcpyAsync(d_pos_, &pin_[1], 4, hipMemcpyHostToDevice, ln_->st), "pos upload");
    profiling_ = prof::enabled();
    if (profiling_) {
        // the same steps without the graph, so every GEMV can be timed
        for (std::size_t i = 0; i < n; ++i) {
            decode_step(d_tok_, true, true);
            prof_flush();
        }
    } else if (!graph_) {
        // the step reads token and position from device memory and its argmax
        // writes the next token and advances the position: one graph serves
        // every step; a second graph of gsteps_ consecutive steps is launched
        // while at least that many tokens remain (one graph launch per 8
        // tokens instead of per token: 7B-shape tg128 666.0 -> 670.2 tok/s with
        // 4 steps, 670.5 with 16; MVH_GRAPH_STEPS overrides, 1 = per token)
        static const int gsteps = [] {
            const char* e = getenv("MVH_GRAPH_STEPS");
            return e ? std::max(1, atoi(e)) : kGraphSteps;
        }();
        gsteps_ = gsteps;
        auto capture = [&](int steps, hipGraphExec_t* exec) {
            hipGraph_t g{};
            check(hipStreamBeginCapture(ln_->st, hipStreamCaptureModeThreadLocal), "begin capture");
            try {
                for (int i = 0; i < steps; ++i) decode_step(d_tok_, true, true);
            } catch (...) {  // leave the stream out of capture mode for the calls that follow
                if (hipStreamEndCapture(ln_->st, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
                throw;
            }
            check(hipStreamEndCapture(ln_->st, &g), "end capture");
            const hipError_t e = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            check(e, "graph instantiate");
        };
        capture(1, &graph_);
        if (gsteps_ > 1) capture(gsteps_, &graphk_);
    }
    if (!profiling_) {
        std::size_t i = 0;
        if (graphk_)
            for (; i + gsteps_ <= n; i += gsteps_) check(hipGraphLaunch(graphk_, ln_->st), "graph launch");
        for (; i < n; ++i) check(hipGraphLaunch(graph_, ln_->st), "graph launch");
    }
    check(hipMemcpyAsync(pin_, d_hist_ + pos_, n * 4, hipMemcpyDeviceToHost, ln_->st), "token copy");
    check(hipStreamSynchronize(ln_->st), "sync");
    std::memcpy(out.data(), pin_, n * 4);
    pos_ += n;
    kv_hi_ = std::max(kv_hi_, pos_);
    return out;
}

}  // namespace hip
}  // namespace memvanta
