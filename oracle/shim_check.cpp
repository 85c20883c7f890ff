// shim_check -- TEST INFRASTRUCTURE ONLY (never the product).
//
// Compiles the reference-side shim exactly as the integration guide prints it
// (extracted to _ref/gguf_kernels_hip.cpp by shim_build.py) against the
// reference's own headers, checks at compile time that every shim function
// has the signature of the reference function it replaces
// (include/memvanta/gguf_kernels.hpp:20-30), then, at run time, opens a GGUF
// with the reference's GgufFile and runs each named tensor through the
// reference's CPU kernels (_ref/libmvref.so) and through the shim
// (libmemvanta_hip.so on the GPU), printing one JSON line per comparison:
//   {"tensor": ..., "op": ..., "n": outputs, "mismatch": bit-unequal outputs,
//    "max_ulp": largest difference in units in the last place}
// or, where a side throws, both error texts; then the profiler entries the
// shim reports.
//
// usage: shim_check <file.gguf> <tensor name>...
#include "gguf_kernels_hip.cpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <type_traits>
#include <vector>

namespace mb = memvanta::hip_backend;
static_assert(std::is_same_v<decltype(&memvanta::tensor_read_row_f32), decltype(&mb::tensor_read_row_f32)>);
static_assert(std::is_same_v<decltype(&memvanta::tensor_matvec), decltype(&mb::tensor_matvec)>);
static_assert(std::is_same_v<decltype(&memvanta::tensor_matmul_batch), decltype(&mb::tensor_matmul_batch)>);
static_assert(std::is_same_v<decltype(&memvanta::tensor_matmul_batch_v06), decltype(&mb::tensor_matmul_batch_v06)>);
static_assert(std::is_same_v<decltype(&memvanta::enable_kernel_profiling), decltype(&mb::enable_kernel_profiling)>);
static_assert(std::is_same_v<decltype(&memvanta::reset_kernel_profile), decltype(&mb::reset_kernel_profile)>);
static_assert(std::is_same_v<decltype(&memvanta::kernel_profile_snapshot), decltype(&mb::kernel_profile_snapshot)>);
static_assert(std::is_same_v<decltype(&memvanta::kernel_profile_kind_name), decltype(&mb::kernel_profile_kind_name)>);

namespace {

// N(0,1)-like activations from a fixed xorshift stream, every 997th entry an
// outlier of +-20 (the activation distribution of the GEMV configuration)
std::vector<float> activations(std::size_t n, uint64_t seed) {
    std::vector<float> x(n);
    uint64_t s = seed * 0x9e3779b97f4a7c15ull + 1;
    auto next = [&] {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return static_cast<double>(s >> 11) * (1.0 / 9007199254740992.0);
    };
    for (std::size_t i = 0; i < n; ++i) {
        const double u1 = next() + 1e-12, u2 = next();
        x[i] = static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
        if (i % 997 == 13) x[i] = (i & 1) ? 20.0f : -20.0f;
    }
    return x;
}

int64_t ordered(float f) {
    int32_t i;
    std::memcpy(&i, &f, 4);
    return i < 0 ? static_cast<int64_t>(INT32_MIN) - i : i;
}

void report(const std::string& tensor, const char* op, const std::vector<float>& a, const std::vector<float>& b) {
    std::size_t mismatch = 0;
    int64_t max_ulp = 0;
    for (std::size_t i = 0; i < a.size(); ++i) {
        if (std::memcmp(&a[i], &b[i], 4) != 0) {
            ++mismatch;
            const int64_t d = std::llabs(ordered(a[i]) - ordered(b[i]));
            if (d > max_ulp) max_ulp = d;
        }
    }
    std::printf("{\"tensor\": \"%s\", \"op\": \"%s\", \"n\": %zu, \"mismatch\": %zu, \"max_ulp\": %lld}\n",
                tensor.c_str(), op, a.size(), mismatch, static_cast<long long>(max_ulp));
}

std::string error_of(const std::function<void()>& fn) {
    try {
        fn();
    } catch (const std::exception& e) {
        return e.what();
    }
    return "";
}

// runs both sides; equal error texts (both throwing) are a match too
void compare(const std::string& tensor, const char* op, std::vector<float>& want, std::vector<float>& got,
             const std::function<void()>& ref, const std::function<void()>& hip) {
    const std::string e_ref = error_of(ref), e_hip = error_of(hip);
    if (e_ref.empty() && e_hip.empty()) {
        report(tensor, op, want, got);
        return;
    }
    std::printf("{\"tensor\": \"%s\", \"op\": \"%s\", \"reference_error\": \"%s\", \"hip_error\": \"%s\"}\n",
                tensor.c_str(), op, e_ref.c_str(), e_hip.c_str());
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s <file.gguf> <tensor>...\n", argv[0]);
        return 2;
    }
    try {
        memvanta::GgufFile f(argv[1]);
        for (int a = 2; a < argc; ++a) {
            const std::string name = argv[a];
            const memvanta::GgufTensor& t = f.tensor(name);
            const std::size_t cols = t.ne(0), rows = t.ne(1);
            {
                const auto x = activations(cols, a);
                std::vector<float> want(rows), got(rows);
                compare(name, "tensor_matvec", want, got,
                        [&] { memvanta::tensor_matvec(f, t, x.data(), want.data(), 4, nullptr); },
                        [&] { mb::tensor_matvec(f, t, x.data(), got.data(), 4, nullptr); });
            }
            for (const char* mode : {"0", "1"}) {
                const std::size_t batch = 13;
                const auto x = activations(cols * batch, 100 + a);
                std::vector<float> want(rows * batch), got(rows * batch);
                setenv("MEMVANTA_FORCE_Q8_ACT", mode, 1);
                compare(name, mode[0] == '1' ? "tensor_matmul_batch_v06 FORCE_Q8" : "tensor_matmul_batch_v06", want,
                        got,
                        [&] { memvanta::tensor_matmul_batch_v06(f, t, x.data(), want.data(), batch, 4, nullptr); },
                        [&] { mb::tensor_matmul_batch_v06(f, t, x.data(), got.data(), batch, 4, nullptr); });
                unsetenv("MEMVANTA_FORCE_Q8_ACT");
            }
            {
                const std::size_t batch = 3;
                const auto x = activations(cols * batch, 200 + a);
                std::vector<float> want(rows * batch), got(rows * batch);
                compare(name, "tensor_matmul_batch", want, got,
                        [&] { memvanta::tensor_matmul_batch(f, t, x.data(), want.data(), batch, 4, nullptr); },
                        [&] { mb::tensor_matmul_batch(f, t, x.data(), got.data(), batch, 4, nullptr); });
            }
            {
                std::vector<float> want(cols), got(cols);
                compare(name, "tensor_read_row_f32", want, got,
                        [&] { memvanta::tensor_read_row_f32(f, t, rows - 1, want.data(), cols); },
                        [&] { mb::tensor_read_row_f32(f, t, rows - 1, got.data(), cols); });
                std::vector<float> wide(cols + 32), wide2(cols + 32);
                compare(name, "read_row_wrong_cols", wide, wide2,
                        [&] { memvanta::tensor_read_row_f32(f, t, 0, wide.data(), cols + 32); },
                        [&] { mb::tensor_read_row_f32(f, t, 0, wide2.data(), cols + 32); });
            }
        }
        // the profiler, through the shim and in the reference: two matvec calls per tensor; the
        // entries (tensor, layer, kind, calls, batch, in snapshot order) must agree
        auto profile = [&](const char* side, auto reset, auto enable, auto matvec, auto snapshot, auto kind_name) {
            reset();
            enable(true);
            for (int a = 2; a < argc; ++a) {
                const memvanta::GgufTensor& t = f.tensor(argv[a]);
                const auto x = activations(t.ne(0), 7);
                std::vector<float> y(t.ne(1));
                matvec(f, t, x.data(), y.data(), 4u, static_cast<memvanta::WorkerPool*>(nullptr));
                matvec(f, t, x.data(), y.data(), 4u, static_cast<memvanta::WorkerPool*>(nullptr));
            }
            enable(false);
            for (const auto& e : snapshot())
                std::printf("{\"op\": \"profile\", \"side\": \"%s\", \"tensor\": \"%s\", \"layer\": %d, "
                            "\"kind\": \"%s\", \"calls\": %zu, \"batch\": %zu}\n",
                            side, e.tensor.c_str(), e.layer, kind_name(e.kind), e.calls, e.batch);
        };
        profile("hip", mb::reset_kernel_profile, mb::enable_kernel_profiling, mb::tensor_matvec,
                mb::kernel_profile_snapshot, mb::kernel_profile_kind_name);
        profile("reference", memvanta::reset_kernel_profile, memvanta::enable_kernel_profiling,
                memvanta::tensor_matvec, memvanta::kernel_profile_snapshot, memvanta::kernel_profile_kind_name);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "shim_check: %s\n", e.what());
        return 1;
    }
    return 0;
}
