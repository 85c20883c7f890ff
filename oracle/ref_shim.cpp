// ref_shim.cpp -- extern "C" wrapper over MemVanta's PUBLIC C++ API so tests
// can call the compiled reference through ctypes.  TEST INFRASTRUCTURE ONLY:
// oracle/Makefile compiles it together with the reference's own sources (read
// in place under the reference checkout) into oracle/_ref/libmvref.so; it is
// used to pin the C restatement (mv_oracle.c), to write the golden vectors in
// tests/golden/, and as bench.py's "reference" CPU baseline.  No reference
// source is copied into this repository.
#include "memvanta/gguf.hpp"
#include "memvanta/gguf_kernels.hpp"
#include "memvanta/llama_model.hpp"
#include "memvanta/quant.hpp"

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

namespace {
thread_local std::string g_err;
template <class F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}
struct ForceQ8 {  // MEMVANTA_FORCE_Q8_ACT is read per call (src/gguf_kernels.cpp:265)
    explicit ForceQ8(int on) {
        if (on) setenv("MEMVANTA_FORCE_Q8_ACT", "1", 1);
        else unsetenv("MEMVANTA_FORCE_Q8_ACT");
    }
    ~ForceQ8() { unsetenv("MEMVANTA_FORCE_Q8_ACT"); }
};
}  // namespace

extern "C" {

const char* mvr_last_error(void) { return g_err.c_str(); }

void mvr_fp32_to_fp16_bits(uint32_t first, uint64_t count, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
        uint32_t b = first + static_cast<uint32_t>(i);
        float f;
        std::memcpy(&f, &b, 4);
        out[i] = memvanta::fp32_to_fp16(f);
    }
}

float mvr_fp16_to_fp32(uint16_t h) { return memvanta::fp16_to_fp32(h); }

// ---- native block formats (memvanta/quant.hpp): blocks are copied in and out
// as raw bytes (BlockQ4_0 20 B, BlockQ8_0 36 B) ----
int mvr_nq_quantize_q8_0(const float* src, size_t n, void* out) {
    return guard([&] {
        auto v = memvanta::quantize_q8_0(src, n);
        std::memcpy(out, v.data(), v.size() * sizeof(memvanta::BlockQ8_0));
    });
}
int mvr_nq_quantize_q4_0(const float* src, size_t n, void* out) {
    return guard([&] {
        auto v = memvanta::quantize_q4_0(src, n);
        std::memcpy(out, v.data(), v.size() * sizeof(memvanta::BlockQ4_0));
    });
}
int mvr_nq_dot_q4_q8(const void* a, const void* x, size_t n, float* out) {
    return guard([&] {
        *out = memvanta::dot_q4_q8(static_cast<const memvanta::BlockQ4_0*>(a), static_cast<const memvanta::BlockQ8_0*>(x), n);
    });
}
int mvr_nq_matvec_q4_q8(const void* A, const void* x, float* y, size_t rows, size_t cols, unsigned threads) {
    return guard([&] {
        memvanta::matvec_q4_q8(static_cast<const memvanta::BlockQ4_0*>(A), static_cast<const memvanta::BlockQ8_0*>(x),
                               y, rows, cols, threads);
    });
}
int mvr_nq_matmul_q4_0_batch(const void* A, const float* x, float* y, size_t rows, size_t cols, size_t batch,
                             unsigned threads) {
    return guard([&] {
        memvanta::matmul_q4_0_batch(static_cast<const memvanta::BlockQ4_0*>(A), x, y, rows, cols, batch, threads);
    });
}
int mvr_nq_matvec_q4_0(const void* A, const float* x, float* y, size_t rows, size_t cols, unsigned threads) {
    return guard([&] { memvanta::matvec_q4_0(static_cast<const memvanta::BlockQ4_0*>(A), x, y, rows, cols, threads); });
}
int mvr_nq_matvec_q8_0(const void* A, const float* x, float* y, size_t rows, size_t cols, unsigned threads) {
    return guard([&] { memvanta::matvec_q8_0(static_cast<const memvanta::BlockQ8_0*>(A), x, y, rows, cols, threads); });
}

void* mvr_gguf_open(const char* path) {
    memvanta::GgufFile* f = nullptr;
    if (guard([&] { f = new memvanta::GgufFile(path); })) return nullptr;
    return f;
}
void mvr_gguf_close(void* h) { delete static_cast<memvanta::GgufFile*>(h); }

int mvr_matvec(void* h, const char* name, const float* x, float* y, unsigned threads) {
    auto* f = static_cast<memvanta::GgufFile*>(h);
    return guard([&] { memvanta::tensor_matvec(*f, f->tensor(name), x, y, threads, nullptr); });
}

int mvr_matmul_batch(void* h, const char* name, const float* x, float* y, size_t batch, unsigned threads) {
    auto* f = static_cast<memvanta::GgufFile*>(h);
    return guard([&] { memvanta::tensor_matmul_batch(*f, f->tensor(name), x, y, batch, threads, nullptr); });
}

int mvr_matmul_batch_v06(void* h, const char* name, const float* x, float* y, size_t batch, unsigned threads,
                         int force_q8) {
    auto* f = static_cast<memvanta::GgufFile*>(h);
    ForceQ8 env(force_q8);
    return guard([&] { memvanta::tensor_matmul_batch_v06(*f, f->tensor(name), x, y, batch, threads, nullptr); });
}

int mvr_read_row(void* h, const char* name, size_t row, float* out, size_t cols) {
    auto* f = static_cast<memvanta::GgufFile*>(h);
    return guard([&] { memvanta::tensor_read_row_f32(*f, f->tensor(name), row, out, cols); });
}

// type: 0 = F32, 1 = F16, 2 = Q8 (KVCacheType's order)
void* mvr_kv_create(size_t kv_dim, size_t page_tokens, int type) {
    return new memvanta::PagedKVCache(kv_dim, page_tokens, static_cast<memvanta::KVCacheType>(type));
}
int mvr_kv_parse_type(const char* s, int* type) {
    return guard([&] { *type = static_cast<int>(memvanta::parse_kv_cache_type(s)); });
}
const char* mvr_kv_type_name(int type) {
    return memvanta::kv_cache_type_name(static_cast<memvanta::KVCacheType>(type));
}
void mvr_kv_destroy(void* kv) { delete static_cast<memvanta::PagedKVCache*>(kv); }
int mvr_kv_write(void* kv, size_t pos, const float* k, const float* v) {
    return guard([&] { static_cast<memvanta::PagedKVCache*>(kv)->write(pos, k, v); });
}
int mvr_kv_dot_key(void* kv, size_t pos, size_t offset, const float* q, size_t n, float* out) {
    return guard([&] { *out = static_cast<memvanta::PagedKVCache*>(kv)->dot_key(pos, offset, q, n); });
}
int mvr_kv_add_value(void* kv, size_t pos, size_t offset, float alpha, float* out, size_t n) {
    return guard([&] { static_cast<memvanta::PagedKVCache*>(kv)->add_value(pos, offset, alpha, out, n); });
}
size_t mvr_kv_bytes(void* kv) { return static_cast<memvanta::PagedKVCache*>(kv)->bytes_allocated(); }

struct RefModel {
    std::unique_ptr<memvanta::LlamaModel> m;
    int force_q8{};
};

void* mvr_model_open(const char* path, unsigned threads, size_t ctx, size_t page, int kv_type, int force_q8) {
    auto* r = new RefModel;
    r->force_q8 = force_q8;
    if (guard([&] {
            r->m = std::make_unique<memvanta::LlamaModel>(path, threads, ctx, page,
                                                          static_cast<memvanta::KVCacheType>(kv_type));
        })) {
        delete r;
        return nullptr;
    }
    return r;
}
void mvr_model_close(void* h) { delete static_cast<RefModel*>(h); }
void mvr_model_reset(void* h) { static_cast<RefModel*>(h)->m->reset(); }
void mvr_model_config(void* h, size_t out[7]) {
    const auto& c = static_cast<RefModel*>(h)->m->config();
    out[0] = c.n_ctx; out[1] = c.n_embd; out[2] = c.n_ff; out[3] = c.n_layer;
    out[4] = c.n_head; out[5] = c.n_head_kv; out[6] = c.vocab;
}
int mvr_model_forward(void* h, int token, float* logits) {
    auto* r = static_cast<RefModel*>(h);
    ForceQ8 env(r->force_q8);
    return guard([&] {
        const auto& l = r->m->forward(token, logits != nullptr);
        if (logits) std::memcpy(logits, l.data(), l.size() * sizeof(float));
    });
}
int mvr_model_prefill(void* h, const int* tokens, size_t n, size_t batch, float* logits) {
    auto* r = static_cast<RefModel*>(h);
    ForceQ8 env(r->force_q8);
    return guard([&] {
        std::vector<int> t(tokens, tokens + n);
        const auto& l = r->m->prefill(t, batch, logits != nullptr);
        if (logits) std::memcpy(logits, l.data(), l.size() * sizeof(float));
    });
}
size_t mvr_model_position(void* h) { return static_cast<RefModel*>(h)->m->position(); }
size_t mvr_model_kv_bytes(void* h) { return static_cast<RefModel*>(h)->m->kv_bytes_allocated(); }

// kernel profiler (include/memvanta/gguf_kernels.hpp:11-23)
void mvr_profile_enable(int on) { memvanta::enable_kernel_profiling(on != 0); }
void mvr_profile_reset(void) { memvanta::reset_kernel_profile(); }
const char* mvr_profile_kind_name(int kind) {
    return memvanta::kernel_profile_kind_name(static_cast<memvanta::KernelProfileKind>(kind));
}
// entries in snapshot order: the first `cap` go to the arrays, their tensor
// names (NUL-separated) to names[names_cap]; returns the entry count
size_t mvr_profile_snapshot(int* layer, int* kind, size_t* calls, size_t* batch, char* names, size_t names_cap,
                            size_t cap) {
    const auto es = memvanta::kernel_profile_snapshot();
    size_t off = 0;
    for (size_t i = 0; i < es.size() && i < cap; ++i) {
        layer[i] = es[i].layer;
        kind[i] = static_cast<int>(es[i].kind);
        calls[i] = es[i].calls;
        batch[i] = es[i].batch;
        const size_t n = es[i].tensor.size() + 1;
        if (off + n <= names_cap) std::memcpy(names + off, es[i].tensor.c_str(), n);
        off += n;
    }
    return es.size();
}

}  // extern "C"
