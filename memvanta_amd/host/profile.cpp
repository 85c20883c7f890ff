// profile.cpp -- registry and event timing of the kernel profiler.
#include "profile.hpp"

#include <atomic>
#include <cerrno>
#include <climits>
#include <cstdlib>
#include <mutex>

namespace memvanta {
namespace hip {
namespace prof {

namespace {
std::atomic<bool> g_enabled{false};
std::mutex g_mu;
std::vector<Entry> g_entries;
}  // namespace

bool enabled() { return g_enabled.load(std::memory_order_relaxed); }
void enable(bool on) { g_enabled.store(on, std::memory_order_relaxed); }

void reset() {
    std::lock_guard<std::mutex> lock(g_mu);
    g_entries.clear();
}

std::vector<Entry> snapshot() {
    std::lock_guard<std::mutex> lock(g_mu);
    return g_entries;
}

const char* kind_name(int kind) {
    static const char* const names[] = {"q_proj", "k_proj", "v_proj", "o_proj", "ffn_gate",
                                        "ffn_up", "ffn_down", "output", "other"};
    return kind >= QProj && kind <= Other ? names[kind] : "other";
}

// classify_tensor (src/gguf_kernels.cpp:38-47): the first pattern that matches
int classify(const std::string& name) {
    static const struct {
        const char* pat;
        int kind;
    } rules[] = {{".attn_q.", QProj},   {".attn_k.", KProj},  {".attn_v.", VProj},     {".attn_output.", OProj},
                 {".ffn_gate.", FfnGate}, {".ffn_up.", FfnUp}, {".ffn_down.", FfnDown}};
    for (const auto& r : rules)
        if (name.find(r.pat) != std::string::npos) return r.kind;
    return name == "output.weight" ? Output : Other;
}

// tensor_layer (src/gguf_kernels.cpp:56-61): std::stoi of the text between
// "blk." and the next '.', -1 when stoi would throw or there is no such text
int layer_of(const std::string& name) {
    if (name.rfind("blk.", 0) != 0) return -1;
    const auto p = name.find('.', 4);
    if (p == std::string::npos) return -1;
    const std::string s = name.substr(4, p - 4);
    errno = 0;
    char* end = nullptr;
    const long v = std::strtol(s.c_str(), &end, 10);
    if (end == s.c_str() || errno == ERANGE || v < INT_MIN || v > INT_MAX) return -1;
    return static_cast<int>(v);
}

// profile_add (src/gguf_kernels.cpp:63-73): one call of `batch` tokens
void add(const std::string& tensor, std::size_t batch, double ms) {
    Entry e;
    e.layer = layer_of(tensor);
    e.kind = classify(tensor);
    e.tensor = tensor;
    e.calls = 1;
    e.batch = batch;
    e.ms = ms;
    std::lock_guard<std::mutex> lock(g_mu);
    for (auto& x : g_entries) {
        if (x.layer == e.layer && x.kind == e.kind && x.tensor == e.tensor && x.batch == e.batch) {
            x.calls += 1;
            x.ms += e.ms;
            return;
        }
    }
    g_entries.push_back(std::move(e));
}

Recorder::~Recorder() { discard(); }

hipError_t Recorder::start() {
    if (open_) (void)hipEventDestroy(open_);
    open_ = nullptr;
    hipError_t e = hipEventCreate(&open_);
    if (e == hipSuccess) e = hipEventRecord(open_, st_);
    return e;
}

hipError_t Recorder::stop(const std::string& tensor, std::size_t batch) {
    if (!open_) return hipErrorInvalidValue;
    hipEvent_t b{};
    hipError_t e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipEventRecord(b, st_);
    if (e != hipSuccess) {
        if (b) (void)hipEventDestroy(b);
        return e;
    }
    pending_.push_back({tensor, batch, open_, b});
    open_ = nullptr;
    return hipSuccess;
}

hipError_t Recorder::flush() {
    hipError_t err = hipSuccess;
    if (!pending_.empty()) err = hipEventSynchronize(pending_.back().b);
    for (auto& p : pending_) {
        float ms = 0.0f;
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, p.a, p.b);
        if (err == hipSuccess) add(p.tensor, p.batch, ms);
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    pending_.clear();
    return err;
}

void Recorder::discard() {
    for (auto& p : pending_) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    pending_.clear();
    if (open_) (void)hipEventDestroy(open_);
    open_ = nullptr;
}

}  // namespace prof
}  // namespace hip
}  // namespace memvanta
