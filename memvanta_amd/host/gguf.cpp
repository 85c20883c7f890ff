// gguf.cpp -- GGUF reader (layout as parsed by src/gguf.cpp:121-136 of the
// reference: header, key/value metadata, tensor infos, data aligned to
// general.alignment, default 32).  Errors are std::runtime_error with the
// reference's messages.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <limits>
#include <stdexcept>

namespace memvanta {
namespace hip {
namespace {

class Cursor {
public:
    Cursor(const std::byte* p, std::uint64_t n) : p_(p), n_(n) {}
    std::uint64_t pos() const { return off_; }
    void need(std::uint64_t k) const {
        if (k > n_ || off_ > n_ - k) throw std::runtime_error("truncated GGUF");
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + off_, sizeof(T));
        off_ += sizeof(T);
        return v;
    }
    std::string str() {
        const auto len = get<std::uint64_t>();
        need(len);
        std::string s(reinterpret_cast<const char*>(p_ + off_), static_cast<std::size_t>(len));
        off_ += len;
        return s;
    }
    void skip(std::uint64_t k) {
        need(k);
        off_ += k;
    }

private:
    const std::byte* p_;
    std::uint64_t n_, off_ = 0;
};

// GGUF metadata value type ids
enum : std::uint32_t { U8 = 0, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARR, U64, I64, F64V };

std::uint64_t scalar_size(std::uint32_t t) {
    switch (t) {
        case U8: case I8: case BOOL: return 1;
        case U16: case I16: return 2;
        case U32: case I32: case F32V: return 4;
        case U64: case I64: case F64V: return 8;
    }
    throw std::runtime_error("unknown GGUF metadata type");
}

}  // namespace

std::uint64_t GgufTensor::elements() const {
    std::uint64_t n = 1;
    for (auto d : dims) {
        if (d && n > std::numeric_limits<std::uint64_t>::max() / d) throw std::runtime_error("tensor element overflow");
        n *= d;
    }
    return n;
}

std::uint64_t tensor_nbytes(std::uint32_t type, std::uint64_t n) {
    auto blocks = [&](std::uint64_t qk, std::uint64_t bs) {
        if (n % qk) throw std::runtime_error("quantized tensor element count is not block aligned");
        return n / qk * bs;
    };
    switch (type) {
        case 0: return n * 4;
        case 1: return n * 2;
        case 2: return blocks(32, 18);
        case 8: return blocks(32, 34);
        case 14: return blocks(256, 210);
    }
    throw std::runtime_error("unsupported GGML type for byte-size calculation: " + std::to_string(type));
}

const char* type_name(std::uint32_t t) {
    switch (t) {
        case 0: return "F32";
        case 1: return "F16";
        case 2: return "Q4_0";
        case 8: return "Q8_0";
        case 14: return "Q6_K";
    }
    return "type-?";
}

GgufFile::GgufFile(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("open failed: " + path);
    struct stat st {};
    if (fstat(fd_, &st) != 0 || st.st_size == 0) {
        ::close(fd_);
        throw std::runtime_error("empty file");
    }
    size_ = static_cast<std::uint64_t>(st.st_size);
    void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) {
        ::close(fd_);
        throw std::runtime_error("mmap failed");
    }
    data_ = static_cast<const std::byte*>(p);
    try {
        Cursor c(data_, size_);
        char magic[4];
        for (char& m : magic) m = static_cast<char>(c.get<std::uint8_t>());
        if (std::memcmp(magic, "GGUF", 4)) throw std::runtime_error("not a GGUF file");
        const auto version = c.get<std::uint32_t>();
        if (version < 2 || version > 3) throw std::runtime_error("unsupported GGUF version: " + std::to_string(version));
        const auto nt = c.get<std::uint64_t>(), nkv = c.get<std::uint64_t>();
        if (nt > 1000000 || nkv > 1000000) throw std::runtime_error("implausible GGUF counts");
        for (std::uint64_t i = 0; i < nkv; ++i) {
            auto key = c.str();
            const auto t = c.get<std::uint32_t>();
            switch (t) {
                case U8: meta_[key] = std::uint64_t{c.get<std::uint8_t>()}; break;
                case I8: meta_[key] = std::int64_t{c.get<std::int8_t>()}; break;
                case U16: meta_[key] = std::uint64_t{c.get<std::uint16_t>()}; break;
                case I16: meta_[key] = std::int64_t{c.get<std::int16_t>()}; break;
                case U32: meta_[key] = std::uint64_t{c.get<std::uint32_t>()}; break;
                case I32: meta_[key] = std::int64_t{c.get<std::int32_t>()}; break;
                case F32V: meta_[key] = double{c.get<float>()}; break;
                case BOOL: meta_[key] = c.get<std::uint8_t>() != 0; break;
                case STR: meta_[key] = c.str(); break;
                case U64: meta_[key] = c.get<std::uint64_t>(); break;
                case I64: meta_[key] = c.get<std::int64_t>(); break;
                case F64V: meta_[key] = c.get<double>(); break;
                case ARR: {  // arrays (tokenizer tables) are skipped
                    const auto et = c.get<std::uint32_t>();
                    const auto n = c.get<std::uint64_t>();
                    if (et == STR)
                        for (std::uint64_t j = 0; j < n; ++j) c.skip(c.get<std::uint64_t>());
                    else if (et == ARR)
                        throw std::runtime_error("nested GGUF arrays are unsupported");
                    else
                        c.skip(n * scalar_size(et));
                    break;
                }
                default: throw std::runtime_error("unknown GGUF metadata type");
            }
        }
        struct Info {
            std::string name;
            std::vector<std::uint64_t> dims;
            std::uint32_t type;
            std::uint64_t rel;
        };
        std::vector<Info> infos(static_cast<std::size_t>(nt));
        for (auto& inf : infos) {
            inf.name = c.str();
            const auto nd = c.get<std::uint32_t>();
            if (nd == 0 || nd > 4) throw std::runtime_error("invalid tensor dimensions");
            inf.dims.resize(nd);
            for (auto& d : inf.dims) d = c.get<std::uint64_t>();
            inf.type = c.get<std::uint32_t>();
            inf.rel = c.get<std::uint64_t>();
        }
        std::uint64_t align = get_u64("general.alignment").value_or(32);
        if (!align || (align & (align - 1))) throw std::runtime_error("invalid GGUF alignment");
        const std::uint64_t base = (c.pos() + align - 1) & ~(align - 1);
        tensors_.reserve(infos.size());
        for (auto& inf : infos) {
            GgufTensor t;
            t.name = std::move(inf.name);
            t.dims = std::move(inf.dims);
            t.type = inf.type;
            t.offset = base + inf.rel;
            try {
                t.nbytes = tensor_nbytes(t.type, t.elements());
            } catch (const std::exception&) {
                t.nbytes = 0;  // a type this backend does not read; rejected when used
            }
            if (t.offset > size_ || t.nbytes > size_ - t.offset)
                throw std::runtime_error("tensor out of file bounds: " + t.name);
            index_[t.name] = tensors_.size();
            tensors_.push_back(std::move(t));
        }
    } catch (...) {
        munmap(const_cast<std::byte*>(data_), size_);
        ::close(fd_);
        throw;
    }
}

GgufFile::~GgufFile() {
    if (data_) munmap(const_cast<std::byte*>(data_), size_);
    if (fd_ >= 0) ::close(fd_);
}

const GgufTensor& GgufFile::tensor(const std::string& name) const {
    auto it = index_.find(name);
    if (it == index_.end()) throw std::runtime_error("missing tensor: " + name);
    return tensors_[it->second];
}

bool GgufFile::has_tensor(const std::string& name) const { return index_.count(name) != 0; }

std::optional<std::uint64_t> GgufFile::get_u64(const std::string& k) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return {};
    if (auto p = std::get_if<std::uint64_t>(&it->second)) return *p;
    if (auto p = std::get_if<std::int64_t>(&it->second))
        if (*p >= 0) return static_cast<std::uint64_t>(*p);
    return {};
}

std::optional<double> GgufFile::get_f64(const std::string& k) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return {};
    if (auto p = std::get_if<double>(&it->second)) return *p;
    if (auto p = std::get_if<std::uint64_t>(&it->second)) return static_cast<double>(*p);
    if (auto p = std::get_if<std::int64_t>(&it->second)) return static_cast<double>(*p);
    return {};
}

std::optional<std::string> GgufFile::get_string(const std::string& k) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return {};
    if (auto p = std::get_if<std::string>(&it->second)) return *p;
    return {};
}

}  // namespace hip
}  // namespace memvanta
