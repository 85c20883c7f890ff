// gguf.hpp -- read-only GGUF v2/v3 reader with the interface of MemVanta's
// GgufFile / GgufTensor (include/memvanta/gguf.hpp:37-82): tensors are
// borrowed byte ranges of a read-only mmap, dims in GGML order (ne0 = cols).
#pragma once
#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

namespace memvanta {
namespace hip {

enum class GgmlType : std::uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q6_K = 14 };

struct GgufTensor {
    std::string name;
    std::vector<std::uint64_t> dims;  // GGML order: ne0, ne1, ...
    std::uint32_t type{};
    std::uint64_t offset{};           // absolute file offset
    std::uint64_t nbytes{};
    std::uint64_t elements() const;
    std::uint64_t ne(std::size_t i) const { return i < dims.size() ? dims[i] : 1; }
};

class GgufFile {
public:
    explicit GgufFile(const std::string& path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const std::vector<GgufTensor>& tensors() const { return tensors_; }
    const GgufTensor& tensor(const std::string& name) const;
    bool has_tensor(const std::string& name) const;
    const std::byte* tensor_data(const GgufTensor& t) const { return data_ + t.offset; }
    std::optional<std::uint64_t> get_u64(const std::string& key) const;
    std::optional<double> get_f64(const std::string& key) const;
    std::optional<std::string> get_string(const std::string& key) const;

private:
    using Value = std::variant<std::uint64_t, std::int64_t, double, bool, std::string>;
    int fd_ = -1;
    const std::byte* data_ = nullptr;
    std::uint64_t size_ = 0;
    std::unordered_map<std::string, Value> meta_;  // scalar metadata only
    std::vector<GgufTensor> tensors_;
    std::unordered_map<std::string, std::size_t> index_;
};

// ggml_tensor_nbytes (src/gguf.cpp:82-105) for the types this backend reads
std::uint64_t tensor_nbytes(std::uint32_t type, std::uint64_t elements);
const char* type_name(std::uint32_t type);

}  // namespace hip
}  // namespace memvanta
