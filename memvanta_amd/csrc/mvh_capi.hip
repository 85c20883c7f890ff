// mvh_capi.hip -- the C ABI declared in include/memvanta_hip.h.
//
// Host-side dispatch mirrors the reference's branches and error texts
// (src/gguf_kernels.cpp:244-271); all arithmetic runs in the gfx950 kernels.
#include "memvanta_hip.h"
#include "mvh_kernels.hpp"
#include "llama_model.hpp"
#include "profile.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

struct mvh_context {
    int device = 0;
    hipStream_t stream = nullptr;
    struct Buf {
        void* p = nullptr;
        size_t cap = 0;
    };
    Buf act;      // Q8 activations: q | d | s
    Buf xin;      // host-pointer staging of inputs
    Buf yout;     // host-pointer staging of outputs
    Buf scores;   // attention scores
};

struct mvh_tensor {
    int device = 0;  // a tensor outlives nothing but its device: freeing it never touches the context
    std::string name;
    uint32_t type = 0;
    uint64_t ne0 = 0, ne1 = 0, nbytes = 0;
    void* d = nullptr;
    bool owned = false;
};

struct mvh_kv_cache {
    int device = 0;  // reset/destroy synchronise the device, so they never touch a context
    int type = mvh::kKvF16;
    size_t n_layer = 0, kv_dim = 0, page_tokens = 0, max_tokens = 0, max_pages = 0;
    std::vector<uint8_t*> hk, hv;  // host mirror of the page tables, [layer*max_pages + page]
    void** dk = nullptr;           // device page tables
    void** dv = nullptr;
    std::vector<uint8_t*> pool;    // released page slabs (K page, then V page at page_stride())
    size_t live_pages = 0;
    size_t page_bytes() const { return mvh::kv_page_bytes(type, page_tokens, kv_dim); }
    size_t page_stride() const { return (page_bytes() + 255) / 256 * 256; }
};

// Scratch of mvh_matmul_batch_v06_noalloc (the Q8 activations of its
// FORCE_Q8 Q4_0 branch): a fixed array in every device's copy of the code
// object, never allocated or freed at run time.  Host code must not pass this
// name to a kernel or copy: its device address comes from hipGetSymbolAddress,
// looked up once per device when a context is created on it (g_scratch_dev).
static __device__ __align__(256) uint8_t scratch[MVH_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};  // device address of `scratch` on each device, once looked up

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define MVH_HIP(expr)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return fail(MVH_E_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

const char* type_name(uint32_t t) {
    switch (t) {
        case MVH_TYPE_F32: return "F32";
        case MVH_TYPE_F16: return "F16";
        case MVH_TYPE_Q4_0: return "Q4_0";
        case MVH_TYPE_Q8_0: return "Q8_0";
        case MVH_TYPE_Q6_K: return "Q6_K";
        case MVH_TYPE_NATIVE_Q4_0: return "native Q4_0";
        case MVH_TYPE_NATIVE_Q8_0: return "native Q8_0";
    }
    return "type-?";
}

// ggml_tensor_nbytes (src/gguf.cpp:82-105) for the accepted types; 0 = invalid
uint64_t tensor_nbytes(uint32_t t, uint64_t n) {
    switch (t) {
        case MVH_TYPE_F32: return n * 4;
        case MVH_TYPE_F16: return n * 2;
        case MVH_TYPE_Q4_0: return n % 32 ? 0 : n / 32 * 18;
        case MVH_TYPE_Q8_0: return n % 32 ? 0 : n / 32 * 34;
        case MVH_TYPE_Q6_K: return n % 256 ? 0 : n / 256 * 210;
        case MVH_TYPE_NATIVE_Q4_0: return n % 32 ? 0 : n / 32 * 20;
        case MVH_TYPE_NATIVE_Q8_0: return n % 32 ? 0 : n / 32 * 36;
    }
    return 0;
}

// is_ffn_tensor (src/gguf_kernels.cpp:50-54)
bool is_ffn(const std::string& n) {
    return n.find(".ffn_gate.") != std::string::npos || n.find(".ffn_up.") != std::string::npos ||
           n.find(".ffn_down.") != std::string::npos;
}

int grow(mvh_context* c, mvh_context::Buf& b, size_t bytes) {
    if (bytes <= b.cap) return MVH_OK;
    if (b.p) {
        MVH_HIP(hipStreamSynchronize(c->stream));
        MVH_HIP(hipFree(b.p));
        b.p = nullptr;
        b.cap = 0;
    }
    const size_t cap = std::max(bytes, static_cast<size_t>(1) << 20);
    if (hipMalloc(&b.p, cap) != hipSuccess) {
        (void)hipGetLastError();
        return fail(MVH_E_NOMEM, "device allocation of %zu bytes failed", cap);
    }
    b.cap = cap;
    return MVH_OK;
}

size_t up16(size_t n) { return (n + 15) & ~static_cast<size_t>(15); }

// Device view of an input: either the caller's device pointer or a staged copy.
int stage_in(mvh_context* c, mvh_context::Buf& b, const void* src, size_t bytes, int kind, const void** out) {
    if (kind == MVH_DEVICE) {
        *out = src;
        return MVH_OK;
    }
    if (kind != MVH_HOST) return fail(MVH_E_INVALID, "ptr_kind must be MVH_HOST or MVH_DEVICE");
    if (int rc = grow(c, b, bytes)) return rc;
    MVH_HIP(hipMemcpyAsync(b.p, src, bytes, hipMemcpyHostToDevice, c->stream));
    *out = b.p;
    return MVH_OK;
}

// fp32 activations: the kernels read them as 16-byte vectors, so a device
// pointer must be 16-byte aligned (host buffers are staged into aligned ones)
int stage_in_act(mvh_context* c, mvh_context::Buf& b, const float* x, size_t bytes, int kind, const void** out) {
    if (kind == MVH_DEVICE && (reinterpret_cast<uintptr_t>(x) & 15))
        return fail(MVH_E_INVALID, "device activations must be 16-byte aligned");
    return stage_in(c, b, x, bytes, kind, out);
}

int finish_out(mvh_context* c, void* host_dst, const void* dev_src, size_t bytes, int kind) {
    if (kind == MVH_DEVICE) return MVH_OK;
    MVH_HIP(hipMemcpyAsync(host_dst, dev_src, bytes, hipMemcpyDeviceToHost, c->stream));
    MVH_HIP(hipStreamSynchronize(c->stream));
    return MVH_OK;
}

// Q8 activation scratch: q [rows][cols] | d [rows][cols/32] | s [rows][cols/32]
struct ActView {
    int8_t* q;
    float* d;
    int* s;
};
size_t act_bytes(size_t rows, size_t cols) { return up16(rows * cols) + 2 * up16(rows * (cols / 32) * 4); }
ActView act_carve(void* base_p, size_t rows, size_t cols) {
    const size_t nq = up16(rows * cols), nd = up16(rows * (cols / 32) * 4);
    auto* base = static_cast<uint8_t*>(base_p);
    return ActView{reinterpret_cast<int8_t*>(base), reinterpret_cast<float*>(base + nq),
                   reinterpret_cast<int*>(base + nq + nd)};
}
int act_buffers(mvh_context* c, size_t rows, size_t cols, ActView* v) {
    if (int rc = grow(c, c->act, act_bytes(rows, cols))) return rc;
    *v = act_carve(c->act.p, rows, cols);
    return MVH_OK;
}
// Activation rows the FORCE_Q8 Q4_0 path of tensor_matmul_batch_v06 quantizes
// into: whole 16-token slabs in the MFMA GEMM's operand order, else one row per token.
size_t v06_act_rows(size_t batch, size_t cols) {
    return mvh::gemm_q4_0_mfma_ok(cols) ? mvh::q8_op_bytes(batch, cols) / cols : batch;
}

#define CHECK_CTX(c)                                                   \
    do {                                                               \
        if (!(c)) return fail(MVH_E_INVALID, "null context");          \
        MVH_HIP(hipSetDevice((c)->device));                            \
    } while (0)

namespace prof = memvanta::hip::prof;

// Times the device work of one tensor call for the kernel profiler (nothing
// when it is off): the start event goes in after the input staging, end()
// records the stop event before the output copy and waits for it.
class ProfSpan {
public:
    ProfSpan(mvh_context* c, const mvh_tensor* w, size_t batch) : name_(w->name), batch_(batch) {
        if (!prof::enabled()) return;
        rec_.emplace(c->stream);
        if (rec_->start() != hipSuccess) rec_.reset();
    }
    int end() {
        if (!rec_) return MVH_OK;
        hipError_t e = rec_->stop(name_, batch_);
        if (e == hipSuccess) e = rec_->flush();
        rec_.reset();
        return e == hipSuccess ? MVH_OK : fail(MVH_E_DEVICE, "profiler events: %s", hipGetErrorString(e));
    }

private:
    std::string name_;
    size_t batch_;
    std::optional<prof::Recorder> rec_;
};

// A call with nothing to launch still counts, as profile_add runs after the
// reference's empty loops.
int prof_empty(const mvh_tensor* w, size_t batch) {
    if (prof::enabled()) prof::add(w->name, batch, 0.0);
    return MVH_OK;
}

// Per-(token, row) fp32-activation dots with tensor_matmul_batch's dispatch.
int fp32_rows(mvh_context* c, const mvh_tensor* w, const float* xd, float* yd, size_t batch, const char* what) {
    const size_t cols = w->ne0, rows = w->ne1;
    const auto* W = static_cast<const uint8_t*>(w->d);
    switch (w->type) {
        case MVH_TYPE_Q4_0:
            if (cols % 32) return fail(MVH_E_SHAPE, "Q4_0 %s row not block aligned: %s", what, w->name.c_str());
            MVH_HIP(mvh::launch_gemv_q4_0_f32act(W, xd, yd, rows, cols, batch, c->stream));
            return MVH_OK;
        case MVH_TYPE_Q8_0:
            if (cols % 32) return fail(MVH_E_SHAPE, "Q8_0 %s row not block aligned: %s", what, w->name.c_str());
            MVH_HIP(mvh::launch_gemv_q8_0(W, xd, yd, rows, cols, batch, c->stream));
            return MVH_OK;
        case MVH_TYPE_Q6_K:
            if (cols % 256) return fail(MVH_E_SHAPE, "Q6_K %s row not block aligned: %s", what, w->name.c_str());
            MVH_HIP(mvh::launch_gemv_q6_k(W, xd, yd, rows, cols, batch, c->stream));
            return MVH_OK;
        case MVH_TYPE_F32:
            MVH_HIP(mvh::launch_gemv_f32(reinterpret_cast<const float*>(W), xd, yd, rows, cols, batch, c->stream));
            return MVH_OK;
        case MVH_TYPE_F16:
            MVH_HIP(mvh::launch_gemv_f16(reinterpret_cast<const uint16_t*>(W), xd, yd, rows, cols, batch, c->stream));
            return MVH_OK;
    }
    return fail(MVH_E_TYPE, "unsupported %s tensor type %s: %s", what, type_name(w->type), w->name.c_str());
}

int check_kv(const mvh_kv_cache* kv, size_t layer) {
    if (!kv) return fail(MVH_E_INVALID, "null KV cache");
    if (layer >= kv->n_layer) return fail(MVH_E_RANGE, "KV layer %zu out of range", layer);
    return MVH_OK;
}

int ensure_page(mvh_kv_cache* kv, size_t layer, size_t p) {
    const size_t slot = layer * kv->max_pages + p;
    if (kv->hk[slot]) return MVH_OK;
    uint8_t* slab = nullptr;
    if (!kv->pool.empty()) {
        slab = kv->pool.back();
        kv->pool.pop_back();
    } else if (hipMalloc(&slab, 2 * kv->page_stride()) != hipSuccess) {
        (void)hipGetLastError();
        return fail(MVH_E_NOMEM, "KV page allocation failed");
    }
    kv->hk[slot] = slab;
    kv->hv[slot] = slab + kv->page_stride();
    ++kv->live_pages;
    MVH_HIP(hipMemcpy(kv->dk + slot, &kv->hk[slot], sizeof(void*), hipMemcpyHostToDevice));
    MVH_HIP(hipMemcpy(kv->dv + slot, &kv->hv[slot], sizeof(void*), hipMemcpyHostToDevice));
    return MVH_OK;
}

}  // namespace

extern "C" {

const char* mvh_last_error(void) { return g_err.c_str(); }
int mvh_version(void) { return 1; }

void mvh_profile_enable(int enabled) { prof::enable(enabled != 0); }
void mvh_profile_reset(void) { prof::reset(); }

int mvh_profile_snapshot(mvh_profile_entry* out, size_t cap, size_t* n_total) {
    if (!n_total) return fail(MVH_E_INVALID, "null n_total");
    if (cap && !out) return fail(MVH_E_INVALID, "null out with cap > 0");
    const auto entries = prof::snapshot();
    *n_total = entries.size();
    for (size_t i = 0; i < entries.size() && i < cap; ++i) {
        const auto& e = entries[i];
        mvh_profile_entry& o = out[i];
        o.layer = e.layer;
        o.kind = e.kind;
        const size_t n = std::min(e.tensor.size(), sizeof o.tensor - 1);
        std::memcpy(o.tensor, e.tensor.data(), n);
        o.tensor[n] = '\0';
        o.calls = e.calls;
        o.batch = e.batch;
        o.ms = e.ms;
    }
    return MVH_OK;
}

const char* mvh_profile_kind_name(int kind) { return prof::kind_name(kind); }

int mvh_device_count(int* count) {
    if (!count) return fail(MVH_E_INVALID, "null count");
    MVH_HIP(hipGetDeviceCount(count));
    return MVH_OK;
}

int mvh_context_create(int device, mvh_context** out) {
    if (!out) return fail(MVH_E_INVALID, "null out");
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return fail(MVH_E_INVALID, "device %d out of range", device);
    MVH_HIP(hipSetDevice(device));
    {
        // the no-allocation entry point's scratch: its address on this device
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_dev[device]) {
            void* ptr = nullptr;
            const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !ptr)
                return fail(MVH_E_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                            hipGetErrorString(e));
            g_scratch_dev[device] = ptr;
        }
    }
    auto* c = new (std::nothrow) mvh_context;
    if (!c) return fail(MVH_E_NOMEM, "host allocation failed");
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(MVH_E_DEVICE, "hipStreamCreate failed");
    }
    *out = c;
    return MVH_OK;
}

int mvh_context_destroy(mvh_context* c) {
    if (!c) return MVH_OK;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (auto* b : {&c->act, &c->xin, &c->yout, &c->scores})
        if (b->p) (void)hipFree(b->p);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return MVH_OK;
}

int mvh_context_stream(mvh_context* c, void** stream) {
    if (!c || !stream) return fail(MVH_E_INVALID, "null argument");
    *stream = c->stream;
    return MVH_OK;
}

int mvh_context_synchronize(mvh_context* c) {
    CHECK_CTX(c);
    MVH_HIP(hipStreamSynchronize(c->stream));
    return MVH_OK;
}

static int make_tensor(mvh_context* c, const char* name, uint32_t type, uint64_t ne0, uint64_t ne1, uint64_t nbytes,
                       mvh_tensor** out) {
    if (!out) return fail(MVH_E_INVALID, "null out");
    *out = nullptr;
    const uint64_t want = tensor_nbytes(type, ne0 * ne1);
    if (type != MVH_TYPE_F32 && type != MVH_TYPE_F16 && type != MVH_TYPE_Q4_0 && type != MVH_TYPE_Q8_0 &&
        type != MVH_TYPE_Q6_K && type != MVH_TYPE_NATIVE_Q4_0 && type != MVH_TYPE_NATIVE_Q8_0)
        return fail(MVH_E_TYPE, "unsupported GGML type %u: %s", type, name ? name : "");
    if (!want || want != nbytes)
        return fail(MVH_E_SHAPE, "tensor byte size %llu does not match %s [%llu x %llu]: %s",
                    static_cast<unsigned long long>(nbytes), type_name(type), static_cast<unsigned long long>(ne1),
                    static_cast<unsigned long long>(ne0), name ? name : "");
    auto* t = new (std::nothrow) mvh_tensor;
    if (!t) return fail(MVH_E_NOMEM, "host allocation failed");
    t->device = c->device;
    t->name = name ? name : "";
    t->type = type;
    t->ne0 = ne0;
    t->ne1 = ne1;
    t->nbytes = nbytes;
    *out = t;
    return MVH_OK;
}

int mvh_tensor_upload(mvh_context* c, const char* name, uint32_t type, uint64_t ne0, uint64_t ne1,
                      const void* host_bytes, uint64_t nbytes, mvh_tensor** out) {
    CHECK_CTX(c);
    if (!host_bytes && nbytes) return fail(MVH_E_INVALID, "null tensor bytes");
    mvh_tensor* t = nullptr;
    if (int rc = make_tensor(c, name, type, ne0, ne1, nbytes, &t)) return rc;
    if (hipMalloc(&t->d, std::max<uint64_t>(nbytes, 16)) != hipSuccess) {
        (void)hipGetLastError();
        delete t;
        return fail(MVH_E_NOMEM, "device allocation of %llu bytes failed: %s", static_cast<unsigned long long>(nbytes),
                    name ? name : "");
    }
    t->owned = true;
    if (nbytes && hipMemcpy(t->d, host_bytes, nbytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(t->d);
        delete t;
        return fail(MVH_E_DEVICE, "tensor upload failed: %s", name ? name : "");
    }
    *out = t;
    return MVH_OK;
}

int mvh_tensor_wrap(mvh_context* c, const char* name, uint32_t type, uint64_t ne0, uint64_t ne1,
                    const void* device_bytes, uint64_t nbytes, mvh_tensor** out) {
    CHECK_CTX(c);
    if (!device_bytes) return fail(MVH_E_INVALID, "null device bytes");
    if (reinterpret_cast<uintptr_t>(device_bytes) & 15) return fail(MVH_E_INVALID, "device bytes must be 16-byte aligned");
    mvh_tensor* t = nullptr;
    if (int rc = make_tensor(c, name, type, ne0, ne1, nbytes, &t)) return rc;
    t->d = const_cast<void*>(device_bytes);
    t->owned = false;
    *out = t;
    return MVH_OK;
}

int mvh_tensor_free(mvh_tensor* t) {
    if (!t) return MVH_OK;
    if (t->owned && t->d) {
        (void)hipSetDevice(t->device);
        (void)hipFree(t->d);  // hipFree waits for work that may still read it
    }
    delete t;
    return MVH_OK;
}

int mvh_tensor_info(const mvh_tensor* t, uint32_t* type, uint64_t* ne0, uint64_t* ne1, uint64_t* nbytes,
                    const void** device_bytes) {
    if (!t) return fail(MVH_E_INVALID, "null tensor");
    if (type) *type = t->type;
    if (ne0) *ne0 = t->ne0;
    if (ne1) *ne1 = t->ne1;
    if (nbytes) *nbytes = t->nbytes;
    if (device_bytes) *device_bytes = t->d;
    return MVH_OK;
}

int mvh_quantize_q8(mvh_context* c, const float* x, size_t batch, size_t cols, int8_t* q, float* d, int kind) {
    CHECK_CTX(c);
    if (cols % 32) return fail(MVH_E_SHAPE, "Q8 activation quantization requires cols multiple of 32");
    if (!batch || !cols) return MVH_OK;
    if (!x || !q || !d) return fail(MVH_E_INVALID, "null argument");
    const void* xd = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, batch * cols * 4, kind, &xd)) return rc;
    ActView a;
    if (int rc = act_buffers(c, batch, cols, &a)) return rc;
    int8_t* qd = kind == MVH_DEVICE ? q : a.q;
    float* dd = kind == MVH_DEVICE ? d : a.d;
    MVH_HIP(mvh::launch_quantize_q8(static_cast<const float*>(xd), qd, dd, a.s, batch, cols, c->stream));
    if (kind == MVH_HOST) {
        MVH_HIP(hipMemcpyAsync(q, a.q, batch * cols, hipMemcpyDeviceToHost, c->stream));
        MVH_HIP(hipMemcpyAsync(d, a.d, batch * (cols / 32) * 4, hipMemcpyDeviceToHost, c->stream));
        MVH_HIP(hipStreamSynchronize(c->stream));
    }
    return MVH_OK;
}

static bool is_native(const mvh_tensor* w) {
    return w->type == MVH_TYPE_NATIVE_Q4_0 || w->type == MVH_TYPE_NATIVE_Q8_0;
}

int mvh_matvec(mvh_context* c, const mvh_tensor* w, const float* x, float* y, int kind) {
    CHECK_CTX(c);
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (is_native(w))
        return fail(MVH_E_TYPE, "unsupported matvec tensor type %s: %s", type_name(w->type), w->name.c_str());
    if (!x || !y) return fail(MVH_E_INVALID, "null x/y");
    const size_t cols = w->ne0, rows = w->ne1;
    if (!rows) return prof_empty(w, 1);
    const void* xd = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, cols * 4, kind, &xd)) return rc;
    float* yd = y;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, rows * 4)) return rc;
        yd = static_cast<float*>(c->yout.p);
    }
    ProfSpan span(c, w, 1);
    const auto* W = static_cast<const uint8_t*>(w->d);
    switch (w->type) {
        case MVH_TYPE_Q4_0: {
            if (cols % 32) return fail(MVH_E_SHAPE, "Q4_0 matrix row not block aligned: %s", w->name.c_str());
            if (mvh::gemv_q4_0_rows16_ok(cols)) {  // quantization fused into the GEMV
                MVH_HIP(mvh::launch_gemv_q4_0_rows16(W, static_cast<const float*>(xd), nullptr, nullptr, yd, rows,
                                                         cols, c->stream));
                break;
            }
            ActView a;
            if (int rc = act_buffers(c, 1, cols, &a)) return rc;
            MVH_HIP(mvh::launch_quantize_q8(static_cast<const float*>(xd), a.q, a.d, a.s, 1, cols, c->stream));
            MVH_HIP(mvh::launch_gemv_q4_0(W, a.q, a.d, yd, rows, cols, c->stream));
            break;
        }
        case MVH_TYPE_Q8_0:
        case MVH_TYPE_Q6_K:
        case MVH_TYPE_F32:
        case MVH_TYPE_F16:
            if (int rc = fp32_rows(c, w, static_cast<const float*>(xd), yd, 1, "matrix")) return rc;
            break;
        default:
            return fail(MVH_E_TYPE, "unsupported matvec tensor type %s: %s", type_name(w->type), w->name.c_str());
    }
    if (int rc = span.end()) return rc;
    return finish_out(c, y, yd, rows * 4, kind);
}

int mvh_matvec_q8(mvh_context* c, const mvh_tensor* w, const int8_t* q, const float* d, float* y, int kind) {
    CHECK_CTX(c);
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (!q || !d || !y) return fail(MVH_E_INVALID, "null q/d/y");
    if (w->type != MVH_TYPE_Q4_0)
        return fail(MVH_E_TYPE, "Q8-activation matvec needs a Q4_0 tensor, got %s: %s", type_name(w->type),
                    w->name.c_str());
    const size_t cols = w->ne0, rows = w->ne1, nb = cols / 32;
    if (cols % 32) return fail(MVH_E_SHAPE, "Q4_0 matrix row not block aligned: %s", w->name.c_str());
    if (!rows) return prof_empty(w, 1);
    const int8_t* qd = q;
    const float* dd = d;
    float* yd = y;
    if (kind == MVH_HOST) {
        ActView a;
        if (int rc = act_buffers(c, 1, cols, &a)) return rc;
        MVH_HIP(hipMemcpyAsync(a.q, q, cols, hipMemcpyHostToDevice, c->stream));
        MVH_HIP(hipMemcpyAsync(a.d, d, nb * 4, hipMemcpyHostToDevice, c->stream));
        if (int rc = grow(c, c->yout, rows * 4)) return rc;
        qd = a.q;
        dd = a.d;
        yd = static_cast<float*>(c->yout.p);
    } else if (kind != MVH_DEVICE) {
        return fail(MVH_E_INVALID, "ptr_kind must be MVH_HOST or MVH_DEVICE");
    } else if (reinterpret_cast<uintptr_t>(q) & 15) {
        return fail(MVH_E_INVALID, "device q must be 16-byte aligned");
    }
    ProfSpan span(c, w, 1);
    MVH_HIP(mvh::launch_gemv_q4_0(static_cast<const uint8_t*>(w->d), qd, dd, yd, rows, cols, c->stream));
    if (int rc = span.end()) return rc;
    return finish_out(c, y, yd, rows * 4, kind);
}

int mvh_matmul_batch(mvh_context* c, const mvh_tensor* w, const float* x, float* y, size_t batch, int kind) {
    CHECK_CTX(c);
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (is_native(w))
        return fail(MVH_E_TYPE, "unsupported batch matrix tensor type %s: %s", type_name(w->type), w->name.c_str());
    const size_t cols = w->ne0, rows = w->ne1;
    if (!batch || !rows) return prof_empty(w, batch);
    if (!x || !y) return fail(MVH_E_INVALID, "null x/y");
    const void* xd = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, batch * cols * 4, kind, &xd)) return rc;
    float* yd = y;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, batch * rows * 4)) return rc;
        yd = static_cast<float*>(c->yout.p);
    }
    ProfSpan span(c, w, batch);
    if (int rc = fp32_rows(c, w, static_cast<const float*>(xd), yd, batch, "batch matrix")) return rc;
    if (int rc = span.end()) return rc;
    return finish_out(c, y, yd, batch * rows * 4, kind);
}

// tensor_matmul_batch_v06 past its fallback checks (src/gguf_kernels.cpp:264-270),
// on device buffers: `act` is the Q8 activation scratch of the FORCE_Q8 Q4_0
// branch (v06_act_rows(batch, cols) rows), unused otherwise.
static int v06_device(mvh_context* c, const mvh_tensor* w, const float* xd, float* yd, size_t batch, int act_mode,
                      const ActView& a) {
    const size_t cols = w->ne0, rows = w->ne1, nb = cols / 32;
    const auto* W = static_cast<const uint8_t*>(w->d);
    if (act_mode == MVH_ACT_Q8) {
        if (w->type == MVH_TYPE_Q4_0) {
            const bool mfma = mvh::gemm_q4_0_mfma_ok(cols);  // int8 MFMA tiles, same per-block chain
            // the MFMA path takes the activations in its operand order (whole 16-token slabs)
            MVH_HIP(mvh::launch_quantize_q8(xd, a.q, a.d, a.s, batch, cols, c->stream, mfma));
            if (mfma) {
                MVH_HIP(mvh::launch_gemm_q4_0_q8_mfma(W, a.q, a.d, yd, rows, cols, batch, c->stream));
            } else {
                MVH_HIP(mvh::launch_gemv_q4_0(W, a.q, a.d, yd, rows, cols, c->stream, batch));
            }
        } else {
            MVH_HIP(mvh::launch_gemv_q8_0(W, xd, yd, rows, cols, batch, c->stream));
        }
    } else {
        // FFN tensors block 8 tokens (two batch4 calls), others 4; the tail
        // tokens use the per-token fp32 dot (src/gguf_kernels.cpp:268)
        const size_t step = is_ffn(w->name) ? 8 : 4;
        const size_t blocked = batch / step * step;
        MVH_HIP(mvh::launch_batch4_f32act(w->type, W, xd, yd, rows, cols, blocked, c->stream));
        if (blocked < batch) {
            if (int rc = fp32_rows(c, w, xd + blocked * cols, yd + blocked * rows, batch - blocked, "batch matrix"))
                return rc;
        }
    }
    return MVH_OK;
}

int mvh_matmul_batch_v06(mvh_context* c, const mvh_tensor* w, const float* x, float* y, size_t batch, int act_mode,
                         int kind) {
    CHECK_CTX(c);
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (act_mode != MVH_ACT_REF && act_mode != MVH_ACT_Q8) return fail(MVH_E_INVALID, "bad act_mode %d", act_mode);
    const size_t cols = w->ne0, rows = w->ne1;
    // fallback conditions of src/gguf_kernels.cpp:263
    if (batch < 2 || (w->type != MVH_TYPE_Q4_0 && w->type != MVH_TYPE_Q8_0) || cols % 32)
        return mvh_matmul_batch(c, w, x, y, batch, kind);
    if (!rows) return prof_empty(w, batch);
    if (!x || !y) return fail(MVH_E_INVALID, "null x/y");
    const void* xv = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, batch * cols * 4, kind, &xv)) return rc;
    const auto* xd = static_cast<const float*>(xv);
    float* yd = y;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, batch * rows * 4)) return rc;
        yd = static_cast<float*>(c->yout.p);
    }
    ProfSpan span(c, w, batch);
    ActView a{};
    if (act_mode == MVH_ACT_Q8 && w->type == MVH_TYPE_Q4_0)
        if (int rc = act_buffers(c, v06_act_rows(batch, cols), cols, &a)) return rc;
    if (int rc = v06_device(c, w, xd, yd, batch, act_mode, a)) return rc;
    if (int rc = span.end()) return rc;
    return finish_out(c, y, yd, batch * rows * 4, kind);
}

int mvh_matmul_batch_v06_noalloc(mvh_context* c, const mvh_tensor* w, const float* x, float* y, size_t batch,
                                 int act_mode) {
    CHECK_CTX(c);
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (act_mode != MVH_ACT_REF && act_mode != MVH_ACT_Q8) return fail(MVH_E_INVALID, "bad act_mode %d", act_mode);
    if (is_native(w))
        return fail(MVH_E_TYPE, "unsupported batch matrix tensor type %s: %s", type_name(w->type), w->name.c_str());
    const size_t cols = w->ne0, rows = w->ne1;
    if (!batch || !rows) return MVH_OK;
    if (!x || !y) return fail(MVH_E_INVALID, "null x/y");
    if (reinterpret_cast<uintptr_t>(x) & 15) return fail(MVH_E_INVALID, "device activations must be 16-byte aligned");
    // fallback conditions of src/gguf_kernels.cpp:263: tensor_matmul_batch's per-(token, row) dots
    if (batch < 2 || (w->type != MVH_TYPE_Q4_0 && w->type != MVH_TYPE_Q8_0) || cols % 32)
        return fp32_rows(c, w, x, y, batch, "batch matrix");
    ActView a{};
    if (act_mode == MVH_ACT_Q8 && w->type == MVH_TYPE_Q4_0) {
        const size_t need = act_bytes(v06_act_rows(batch, cols), cols);
        if (need > MVH_NOALLOC_SCRATCH_BYTES)
            return fail(MVH_E_RANGE,
                        "batch %zu x cols %zu needs %zu bytes of Q8 activation scratch, above the %u-byte static "
                        "scratch of mvh_matmul_batch_v06_noalloc",
                        batch, cols, need, static_cast<unsigned>(MVH_NOALLOC_SCRATCH_BYTES));
        void* base = g_scratch_dev[c->device];  // looked up when the context was created
        if (!base) return fail(MVH_E_DEVICE, "no scratch address for device %d", c->device);
        a = act_carve(base, v06_act_rows(batch, cols), cols);
    }
    return v06_device(c, w, x, y, batch, act_mode, a);
}

int mvh_read_row_f32(mvh_context* c, const mvh_tensor* w, size_t row, float* out, size_t cols, int kind) {
    CHECK_CTX(c);
    if (!w || !out) return fail(MVH_E_INVALID, "null argument");
    // the reference checks the shape first (src/gguf_kernels.cpp:226), then the type
    if (cols != w->ne0 || row >= w->ne1) return fail(MVH_E_RANGE, "tensor row shape mismatch: %s", w->name.c_str());
    if (is_native(w))
        return fail(MVH_E_TYPE, "unsupported embedding tensor type %s: %s", type_name(w->type), w->name.c_str());
    if (w->type == MVH_TYPE_Q6_K && w->ne0 % 256)
        return fail(MVH_E_SHAPE, "Q6_K embedding row not block aligned: %s", w->name.c_str());
    float* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, w->ne0 * 4)) return rc;
        od = static_cast<float*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_read_row(w->type, static_cast<const uint8_t*>(w->d), w->ne0, row, od, c->stream));
    return finish_out(c, out, od, w->ne0 * 4, kind);
}

int mvh_fp32_to_fp16(mvh_context* c, const float* x, uint16_t* out, size_t n, int kind) {
    CHECK_CTX(c);
    if (!n) return MVH_OK;
    if (!x || !out) return fail(MVH_E_INVALID, "null argument");
    const void* xd = nullptr;
    if (int rc = stage_in(c, c->xin, x, n * 4, kind, &xd)) return rc;
    uint16_t* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, n * 2)) return rc;
        od = static_cast<uint16_t*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_f2h(static_cast<const float*>(xd), od, n, c->stream));
    return finish_out(c, out, od, n * 2, kind);
}

int mvh_stream_read(mvh_context* c, const void* buf, size_t bytes, uint32_t* sink, size_t sink_words) {
    CHECK_CTX(c);
    if (!buf || !sink) return fail(MVH_E_INVALID, "null argument");
    if (bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15))
        return fail(MVH_E_INVALID, "buffer must be 16-byte aligned and a multiple of 16 bytes");
    MVH_HIP(mvh::launch_stream_read(buf, bytes, sink, sink_words, c->stream));
    return MVH_OK;
}

int mvh_argmax(mvh_context* c, const float* logits, size_t n, size_t rows, int* out, int kind) {
    CHECK_CTX(c);
    if (!n) return fail(MVH_E_INVALID, "empty logits");  // Sampler::sample's check
    if (!rows) return MVH_OK;
    if (!logits || !out) return fail(MVH_E_INVALID, "null argument");
    if (n > 0x7fffffff) return fail(MVH_E_RANGE, "logits row too long");
    const void* ld = nullptr;
    if (int rc = stage_in(c, c->xin, logits, rows * n * 4, kind, &ld)) return rc;
    int* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, rows * 4)) return rc;
        od = static_cast<int*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_argmax(static_cast<const float*>(ld), n, rows, od, nullptr, nullptr, c->stream));
    return finish_out(c, out, od, rows * 4, kind);
}

int mvh_fp16_to_fp32(mvh_context* c, const uint16_t* h, float* out, size_t n, int kind) {
    CHECK_CTX(c);
    if (!n) return MVH_OK;
    if (!h || !out) return fail(MVH_E_INVALID, "null argument");
    const void* hd = nullptr;
    if (int rc = stage_in(c, c->xin, h, n * 2, kind, &hd)) return rc;
    float* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, n * 4)) return rc;
        od = static_cast<float*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_h2f(static_cast<const uint16_t*>(hd), od, n, c->stream));
    return finish_out(c, out, od, n * 4, kind);
}

// ---- native block formats (src/quant.cpp, src/quant_kernels.cpp) ----

static int quantize_native(mvh_context* c, uint32_t type, const float* x, size_t n, void* blocks, int kind) {
    CHECK_CTX(c);
    const bool q4 = type == mvh::kNQ4_0;
    if (n % 32) return fail(MVH_E_SHAPE, q4 ? "q4_0 length must be multiple of 32" : "q8_0 length must be multiple of 32");
    if (!n) return MVH_OK;
    if (!x || !blocks) return fail(MVH_E_INVALID, "null argument");
    const size_t out_bytes = n / 32 * (q4 ? 20 : 36);
    const void* xd = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, n * 4, kind, &xd)) return rc;
    void* od = blocks;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, out_bytes)) return rc;
        od = c->yout.p;
    } else if (reinterpret_cast<uintptr_t>(blocks) & 3) {
        return fail(MVH_E_INVALID, "device blocks must be 4-byte aligned");
    }
    MVH_HIP(mvh::launch_quantize_native(type, static_cast<const float*>(xd), static_cast<uint8_t*>(od), n, c->stream));
    return finish_out(c, blocks, od, out_bytes, kind);
}

int mvh_quantize_q8_0(mvh_context* c, const float* x, size_t n, void* blocks, int kind) {
    return quantize_native(c, mvh::kNQ8_0, x, n, blocks, kind);
}

int mvh_quantize_q4_0(mvh_context* c, const float* x, size_t n, void* blocks, int kind) {
    return quantize_native(c, mvh::kNQ4_0, x, n, blocks, kind);
}

static int need_native(const mvh_tensor* w, uint32_t type, const char* fn) {
    if (!w) return fail(MVH_E_INVALID, "null tensor");
    if (w->type != type)
        return fail(MVH_E_TYPE, "%s needs a %s tensor, got %s: %s", fn, type_name(type), type_name(w->type),
                    w->name.c_str());
    return MVH_OK;
}

int mvh_matvec_q4_q8(mvh_context* c, const mvh_tensor* w, const void* xq, float* y, int kind) {
    CHECK_CTX(c);
    if (int rc = need_native(w, MVH_TYPE_NATIVE_Q4_0, "matvec_q4_q8")) return rc;
    const size_t cols = w->ne0, rows = w->ne1;
    if (cols % 32) return fail(MVH_E_SHAPE, "q4_q8 cols must be multiple of 32");
    if (!rows) return MVH_OK;
    if (!xq || !y) return fail(MVH_E_INVALID, "null xq/y");
    if (kind == MVH_DEVICE && (reinterpret_cast<uintptr_t>(xq) & 3))
        return fail(MVH_E_INVALID, "device xq must be 4-byte aligned");
    const void* xd = nullptr;
    if (int rc = stage_in(c, c->xin, xq, cols / 32 * 36, kind, &xd)) return rc;
    float* yd = y;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, rows * 4)) return rc;
        yd = static_cast<float*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_matvec_q4q8_native(static_cast<const uint8_t*>(w->d), static_cast<const uint8_t*>(xd), yd, rows,
                                           cols, c->stream));
    return finish_out(c, y, yd, rows * 4, kind);
}

static int native_f32act(mvh_context* c, const mvh_tensor* w, uint32_t type, const char* fn, const char* shape_err,
                         const float* x, float* y, size_t batch, int kind) {
    CHECK_CTX(c);
    if (int rc = need_native(w, type, fn)) return rc;
    const size_t cols = w->ne0, rows = w->ne1;
    if (cols % 32) return fail(MVH_E_SHAPE, "%s", shape_err);
    if (!rows || !batch) return MVH_OK;
    if (!x || !y) return fail(MVH_E_INVALID, "null x/y");
    const void* xd = nullptr;
    if (int rc = stage_in_act(c, c->xin, x, batch * cols * 4, kind, &xd)) return rc;
    float* yd = y;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, batch * rows * 4)) return rc;
        yd = static_cast<float*>(c->yout.p);
    }
    MVH_HIP(mvh::launch_gemv_native_f32act(type == MVH_TYPE_NATIVE_Q4_0 ? mvh::kNQ4_0 : mvh::kNQ8_0,
                                           static_cast<const uint8_t*>(w->d), static_cast<const float*>(xd), yd, rows,
                                           cols, batch, c->stream));
    return finish_out(c, y, yd, batch * rows * 4, kind);
}

int mvh_matmul_q4_0_batch(mvh_context* c, const mvh_tensor* w, const float* x, float* y, size_t batch, int kind) {
    return native_f32act(c, w, MVH_TYPE_NATIVE_Q4_0, "matmul_q4_0_batch", "q4_0 cols must be multiple of 32", x, y,
                         batch, kind);
}

int mvh_matvec_q4_0(mvh_context* c, const mvh_tensor* w, const float* x, float* y, int kind) {
    return native_f32act(c, w, MVH_TYPE_NATIVE_Q4_0, "matvec_q4_0", "q4_0 cols must be multiple of 32", x, y, 1, kind);
}

int mvh_matvec_q8_0(mvh_context* c, const mvh_tensor* w, const float* x, float* y, int kind) {
    return native_f32act(c, w, MVH_TYPE_NATIVE_Q8_0, "matvec_q8_0", "q8_0 cols must be multiple of 32", x, y, 1, kind);
}

int mvh_kv_parse_type(const char* s, int* type) {
    if (!s || !type) return fail(MVH_E_INVALID, "null argument");
    const std::string t = s;
    if (t == "f32") *type = MVH_KV_F32;
    else if (t == "f16") *type = MVH_KV_F16;
    else if (t == "q8" || t == "q8_0") *type = MVH_KV_Q8;
    else return fail(MVH_E_INVALID, "unknown KV cache type: %s", s);
    return MVH_OK;
}

const char* mvh_kv_type_name(int type) {
    switch (type) {
    case MVH_KV_F32: return "f32";
    case MVH_KV_F16: return "f16";
    case MVH_KV_Q8: return "q8";
    }
    return "?";
}

int mvh_kv_create(mvh_context* c, size_t n_layer, size_t kv_dim, size_t page_tokens, size_t max_tokens, int kv_type,
                  mvh_kv_cache** out) {
    CHECK_CTX(c);
    if (!out) return fail(MVH_E_INVALID, "null out");
    *out = nullptr;
    if (kv_type != MVH_KV_F32 && kv_type != MVH_KV_F16 && kv_type != MVH_KV_Q8)
        return fail(MVH_E_INVALID, "unknown KV cache type id %d", kv_type);
    if (!page_tokens) page_tokens = 128;  // PagedKVCache default (src/llama_model.cpp:19)
    if (!n_layer || !kv_dim || !max_tokens) return fail(MVH_E_INVALID, "KV cache needs layers, kv_dim and max_tokens");
    if (kv_dim % 8) return fail(MVH_E_SHAPE, "kv_dim must be a multiple of 8");
    if (max_tokens > 16000) return fail(MVH_E_RANGE, "max_tokens above 16000 is not supported");
    auto* kv = new (std::nothrow) mvh_kv_cache;
    if (!kv) return fail(MVH_E_NOMEM, "host allocation failed");
    kv->device = c->device;
    kv->type = kv_type;
    kv->n_layer = n_layer;
    kv->kv_dim = kv_dim;
    kv->page_tokens = page_tokens;
    kv->max_tokens = max_tokens;
    kv->max_pages = (max_tokens + page_tokens - 1) / page_tokens;
    const size_t n = n_layer * kv->max_pages;
    kv->hk.assign(n, nullptr);
    kv->hv.assign(n, nullptr);
    if (hipMalloc(&kv->dk, n * sizeof(void*)) != hipSuccess || hipMalloc(&kv->dv, n * sizeof(void*)) != hipSuccess) {
        (void)hipGetLastError();
        if (kv->dk) (void)hipFree(kv->dk);
        delete kv;
        return fail(MVH_E_NOMEM, "KV page table allocation failed");
    }
    MVH_HIP(hipMemcpy(kv->dk, kv->hk.data(), n * sizeof(void*), hipMemcpyHostToDevice));
    MVH_HIP(hipMemcpy(kv->dv, kv->hv.data(), n * sizeof(void*), hipMemcpyHostToDevice));
    *out = kv;
    return MVH_OK;
}

int mvh_kv_reset(mvh_kv_cache* kv) {
    if (!kv) return fail(MVH_E_INVALID, "null KV cache");
    MVH_HIP(hipSetDevice(kv->device));
    MVH_HIP(hipDeviceSynchronize());
    for (size_t i = 0; i < kv->hk.size(); ++i)
        if (kv->hk[i]) {
            kv->pool.push_back(kv->hk[i]);
            kv->hk[i] = kv->hv[i] = nullptr;
        }
    kv->live_pages = 0;
    const size_t n = kv->hk.size();
    MVH_HIP(hipMemcpy(kv->dk, kv->hk.data(), n * sizeof(void*), hipMemcpyHostToDevice));
    MVH_HIP(hipMemcpy(kv->dv, kv->hv.data(), n * sizeof(void*), hipMemcpyHostToDevice));
    return MVH_OK;
}

int mvh_kv_destroy(mvh_kv_cache* kv) {
    if (!kv) return MVH_OK;
    (void)hipSetDevice(kv->device);
    (void)hipDeviceSynchronize();
    for (auto* p : kv->hk)
        if (p) (void)hipFree(p);
    for (auto* p : kv->pool) (void)hipFree(p);
    (void)hipFree(kv->dk);
    (void)hipFree(kv->dv);
    delete kv;
    return MVH_OK;
}

int mvh_kv_bytes_allocated(const mvh_kv_cache* kv, size_t* bytes) {
    if (!kv || !bytes) return fail(MVH_E_INVALID, "null argument");
    *bytes = kv->live_pages * mvh::kv_page_pair_bytes_ref(kv->type, kv->page_tokens, kv->kv_dim);
    return MVH_OK;
}

int mvh_kv_type(const mvh_kv_cache* kv, int* type) {
    if (!kv || !type) return fail(MVH_E_INVALID, "null argument");
    *type = kv->type;
    return MVH_OK;
}

int mvh_kv_write(mvh_context* c, mvh_kv_cache* kv, size_t layer, size_t pos, size_t n_tokens, const float* k,
                 const float* v, int kind) {
    CHECK_CTX(c);
    if (int rc = check_kv(kv, layer)) return rc;
    if (!n_tokens) return MVH_OK;
    if (!k || !v) return fail(MVH_E_INVALID, "null k/v");
    if (pos + n_tokens > kv->max_tokens) return fail(MVH_E_RANGE, "context exhausted");
    for (size_t p = pos / kv->page_tokens; p <= (pos + n_tokens - 1) / kv->page_tokens; ++p)
        if (int rc = ensure_page(kv, layer, p)) return rc;
    const size_t bytes = n_tokens * kv->kv_dim * 4;
    const void* kd = nullptr;
    const void* vd = nullptr;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->xin, 2 * bytes)) return rc;
        MVH_HIP(hipMemcpyAsync(c->xin.p, k, bytes, hipMemcpyHostToDevice, c->stream));
        MVH_HIP(hipMemcpyAsync(static_cast<uint8_t*>(c->xin.p) + bytes, v, bytes, hipMemcpyHostToDevice, c->stream));
        kd = c->xin.p;
        vd = static_cast<uint8_t*>(c->xin.p) + bytes;
    } else {
        kd = k;
        vd = v;
    }
    const size_t base = layer * kv->max_pages;
    MVH_HIP(mvh::launch_kv_write(kv->type, kv->dk + base, kv->dv + base, static_cast<const float*>(kd),
                                 static_cast<const float*>(vd), kv->kv_dim, nullptr, pos, n_tokens, kv->kv_dim,
                                 kv->page_tokens, c->stream));
    if (kind == MVH_HOST) MVH_HIP(hipStreamSynchronize(c->stream));
    return MVH_OK;
}

int mvh_kv_read_row(mvh_context* c, const mvh_kv_cache* kv, size_t layer, size_t pos, int which, void* out,
                    float* scale) {
    CHECK_CTX(c);
    if (int rc = check_kv(kv, layer)) return rc;
    if (!out) return fail(MVH_E_INVALID, "null out");
    if (pos >= kv->max_tokens) return fail(MVH_E_RANGE, "KV position out of range");
    const size_t slot = layer * kv->max_pages + pos / kv->page_tokens, i = pos % kv->page_tokens;
    const uint8_t* page = which ? kv->hv[slot] : kv->hk[slot];
    if (!page) return fail(MVH_E_RANGE, which ? "KV value page missing" : "KV key page missing");
    const size_t eb = mvh::kv_elem_bytes(kv->type);
    MVH_HIP(hipStreamSynchronize(c->stream));
    MVH_HIP(hipMemcpy(out, page + i * kv->kv_dim * eb, kv->kv_dim * eb, hipMemcpyDeviceToHost));
    if (scale) {
        *scale = 1.0f;
        if (kv->type == MVH_KV_Q8)
            MVH_HIP(hipMemcpy(scale, page + mvh::kv_scale_offset(kv->page_tokens, kv->kv_dim) + 4 * i, 4,
                              hipMemcpyDeviceToHost));
    }
    return MVH_OK;
}

int mvh_attn_decode(mvh_context* c, const mvh_kv_cache* kv, size_t layer, const float* q, size_t pos, size_t n_head,
                    size_t n_head_kv, size_t head_dim, float* out, int kind) {
    CHECK_CTX(c);
    if (int rc = check_kv(kv, layer)) return rc;
    if (!q || !out) return fail(MVH_E_INVALID, "null q/out");
    if (!n_head || !n_head_kv || n_head % n_head_kv || !head_dim)
        return fail(MVH_E_SHAPE, "invalid Llama head configuration");
    if (head_dim % 8 || n_head_kv * head_dim > kv->kv_dim)
        return fail(MVH_E_SHAPE, "head_dim must be a multiple of 8 and n_head_kv*head_dim <= kv_dim");
    if (pos >= kv->max_tokens) return fail(MVH_E_RANGE, "context exhausted");
    for (size_t p = 0; p <= pos / kv->page_tokens; ++p)
        if (!kv->hk[layer * kv->max_pages + p]) return fail(MVH_E_RANGE, "KV key page missing");
    const size_t qn = n_head * head_dim;
    const void* qd = nullptr;
    if (int rc = stage_in(c, c->xin, q, qn * 4, kind, &qd)) return rc;
    float* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, qn * 4)) return rc;
        od = static_cast<float*>(c->yout.p);
    }
    if (int rc = grow(c, c->scores, n_head * (pos + 1) * 4)) return rc;
    const size_t base = layer * kv->max_pages;
    MVH_HIP(mvh::launch_attn_decode(kv->type, kv->dk + base, kv->dv + base, static_cast<const float*>(qd),
                                    static_cast<float*>(c->scores.p), od, pos, n_head, n_head_kv, head_dim,
                                    kv->kv_dim, kv->page_tokens, c->stream));
    return finish_out(c, out, od, qn * 4, kind);
}

int mvh_attn_batch(mvh_context* c, const mvh_kv_cache* kv, size_t layer, const float* q, size_t pos, size_t n_tokens,
                   size_t n_head, size_t n_head_kv, size_t head_dim, float* out, int kind) {
    CHECK_CTX(c);
    if (int rc = check_kv(kv, layer)) return rc;
    if (!n_tokens) return MVH_OK;
    if (!q || !out) return fail(MVH_E_INVALID, "null q/out");
    if (!n_head || !n_head_kv || n_head % n_head_kv || !head_dim)
        return fail(MVH_E_SHAPE, "invalid Llama head configuration");
    if (head_dim % 8 || n_head_kv * head_dim > kv->kv_dim)
        return fail(MVH_E_SHAPE, "head_dim must be a multiple of 8 and n_head_kv*head_dim <= kv_dim");
    if (pos + n_tokens > kv->max_tokens) return fail(MVH_E_RANGE, "context exhausted");
    const size_t last = pos + n_tokens - 1;
    for (size_t p = 0; p <= last / kv->page_tokens; ++p)
        if (!kv->hk[layer * kv->max_pages + p]) return fail(MVH_E_RANGE, "KV key page missing");
    const size_t qn = n_tokens * n_head * head_dim;
    const void* qd = nullptr;
    if (int rc = stage_in(c, c->xin, q, qn * 4, kind, &qd)) return rc;
    float* od = out;
    if (kind == MVH_HOST) {
        if (int rc = grow(c, c->yout, qn * 4)) return rc;
        od = static_cast<float*>(c->yout.p);
    }
    if (int rc = grow(c, c->scores, n_tokens * n_head * (last + 1) * 4)) return rc;
    const size_t base = layer * kv->max_pages;
    const float* qf = static_cast<const float*>(qd);
    float* sc = static_cast<float*>(c->scores.p);
    if (head_dim % 32 == 0)  // scores once per (token, head), V tiles shared by groups of 32 tokens
        MVH_HIP(mvh::launch_attn_prefill(kv->type, kv->dk + base, kv->dv + base, qf, n_head * head_dim, sc, od, nullptr,
                                         nullptr, false, nullptr, pos, last + 1, n_tokens, n_head, n_head_kv, head_dim,
                                         kv->kv_dim, kv->page_tokens, c->stream));
    else
        MVH_HIP(mvh::launch_attn(kv->type, kv->dk + base, kv->dv + base, qf, n_head * head_dim, sc, od, nullptr, pos,
                                 last + 1, n_tokens, n_head, n_head_kv, head_dim, kv->kv_dim, kv->page_tokens,
                                 c->stream));
    return finish_out(c, out, od, qn * 4, kind);
}

}  // extern "C"

namespace {
using ModelT = memvanta::hip::LlamaModel;
ModelT* M(mvh_model* m) { return reinterpret_cast<ModelT*>(m); }
const ModelT* M(const mvh_model* m) { return reinterpret_cast<const ModelT*>(m); }
template <class F>
int guarded(F&& f) {
    try {
        f();
        return MVH_OK;
    } catch (const std::exception& e) {
        const std::string w = e.what();
        const int code = w.find("out of range") != std::string::npos || w.find("exhausted") != std::string::npos
                             ? MVH_E_RANGE
                             : w.find("hip") != std::string::npos ? MVH_E_DEVICE : MVH_E_INVALID;
        return fail(code, "%s", w.c_str());
    }
}
}  // namespace

extern "C" {

int mvh_model_open(const char* path, int device, size_t ctx_override, size_t page_tokens, int kv_type, int act_mode,
                   size_t max_batch, mvh_model** out) {
    if (!path || !out) return fail(MVH_E_INVALID, "null argument");
    *out = nullptr;
    if (act_mode != MVH_ACT_REF && act_mode != MVH_ACT_Q8) return fail(MVH_E_INVALID, "bad act_mode %d", act_mode);
    if (kv_type != MVH_KV_F32 && kv_type != MVH_KV_F16 && kv_type != MVH_KV_Q8)
        return fail(MVH_E_INVALID, "unknown KV cache type id %d", kv_type);
    return guarded([&] {
        auto mode = act_mode == MVH_ACT_Q8 ? memvanta::hip::PrefillMode::Q8 : memvanta::hip::PrefillMode::Reference;
        *out = reinterpret_cast<mvh_model*>(
            new ModelT(path, device, ctx_override, page_tokens, kv_type, mode, max_batch));
    });
}

int mvh_model_kv_type(const mvh_model* m, int* type) {
    if (!m || !type) return fail(MVH_E_INVALID, "null argument");
    *type = M(m)->kv_type();
    return MVH_OK;
}

int mvh_model_close(mvh_model* m) {
    delete M(m);
    return MVH_OK;
}

int mvh_model_config(const mvh_model* m, size_t out[7]) {
    if (!m || !out) return fail(MVH_E_INVALID, "null argument");
    const auto& c = M(m)->config();
    out[0] = c.n_ctx;
    out[1] = c.n_embd;
    out[2] = c.n_ff;
    out[3] = c.n_layer;
    out[4] = c.n_head;
    out[5] = c.n_head_kv;
    out[6] = c.vocab;
    return MVH_OK;
}

int mvh_model_reset(mvh_model* m) {
    if (!m) return fail(MVH_E_INVALID, "null model");
    M(m)->reset();
    return MVH_OK;
}

int mvh_model_forward(mvh_model* m, int token, float* logits) {
    if (!m) return fail(MVH_E_INVALID, "null model");
    return guarded([&] {
        const auto& l = M(m)->forward(token, logits != nullptr);
        if (logits) std::memcpy(logits, l.data(), l.size() * sizeof(float));
    });
}

int mvh_model_prefill(mvh_model* m, const int* tokens, size_t n, size_t batch, float* logits) {
    if (!m || (!tokens && n)) return fail(MVH_E_INVALID, "null argument");
    return guarded([&] {
        std::vector<int> t(tokens, tokens + n);
        const auto& l = M(m)->prefill(t, batch, logits != nullptr);
        if (logits && n) std::memcpy(logits, l.data(), l.size() * sizeof(float));
    });
}

int mvh_model_generate_greedy(mvh_model* m, int token, size_t n, int* out_tokens, float* last_logits) {
    if (!m || (!out_tokens && n)) return fail(MVH_E_INVALID, "null argument");
    return guarded([&] {
        const auto ids = M(m)->generate_greedy(token, n);
        std::memcpy(out_tokens, ids.data(), n * sizeof(int));
        if (last_logits && n) {
            const auto& l = M(m)->logits();
            std::memcpy(last_logits, l.data(), l.size() * sizeof(float));
        }
    });
}

int mvh_model_position(const mvh_model* m, size_t* pos) {
    if (!m || !pos) return fail(MVH_E_INVALID, "null argument");
    *pos = M(m)->position();
    return MVH_OK;
}

int mvh_model_kv_bytes(const mvh_model* m, size_t* bytes) {
    if (!m || !bytes) return fail(MVH_E_INVALID, "null argument");
    *bytes = M(m)->kv_bytes_allocated();
    return MVH_OK;
}

int mvh_model_stream(mvh_model* m, void** stream) {
    if (!m || !stream) return fail(MVH_E_INVALID, "null argument");
    *stream = M(m)->stream();
    return MVH_OK;
}

}  // extern "C"
