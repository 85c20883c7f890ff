// profile.hpp -- the kernel profiler of the reference's tensor ops
// (enable_kernel_profiling / reset_kernel_profile / kernel_profile_snapshot /
// kernel_profile_kind_name, include/memvanta/gguf_kernels.hpp:11-23,
// src/gguf_kernels.cpp:34-73,:219-222), timed on the device.
//
// While enabled, each timed call (a C ABI matvec / matmul entry, or one GEMV /
// GEMM launch group of a model step) is bracketed by two HIP events on its
// stream; the elapsed time is added to the entry of its (layer, kind, tensor,
// batch), as profile_add aggregates it.  Layer and kind come from the tensor
// name by the reference's rules (tensor_layer, classify_tensor).  Process-wide
// and thread-safe, like the reference's registry.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <string>
#include <vector>

namespace memvanta {
namespace hip {
namespace prof {

enum Kind : int { QProj = 0, KProj, VProj, OProj, FfnGate, FfnUp, FfnDown, Output, Other };

struct Entry {
    int layer = -1;
    int kind = Other;
    std::string tensor;
    std::size_t calls = 0;
    std::size_t batch = 0;
    double ms = 0.0;
};

bool enabled();
void enable(bool on);
void reset();
std::vector<Entry> snapshot();
const char* kind_name(int kind);  // "q_proj" ... "other"; "other" for unknown values
int classify(const std::string& name);
int layer_of(const std::string& name);
void add(const std::string& tensor, std::size_t batch, double ms);

// Event pairs recorded on one stream; flush() waits for the last one and adds
// every pair's elapsed time to the registry.
class Recorder {
public:
    explicit Recorder(hipStream_t st) : st_(st) {}
    ~Recorder();
    Recorder(const Recorder&) = delete;
    Recorder& operator=(const Recorder&) = delete;
    // start / stop around the launches of one call; stop names the call
    hipError_t start();
    hipError_t stop(const std::string& tensor, std::size_t batch);
    hipError_t flush();
    void discard();  // drop pending pairs (error paths)

private:
    struct Pending {
        std::string tensor;
        std::size_t batch;
        hipEvent_t a, b;
    };
    hipStream_t st_;
    hipEvent_t open_{};
    std::vector<Pending> pending_;
};

}  // namespace prof
}  // namespace hip
}  // namespace memvanta
