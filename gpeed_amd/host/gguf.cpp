// GGUF v2/v3 reader (see gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace glm5 {
namespace gpu {

// ---------------------------------------------------------------- geometry

int dtype_block_size(DType t) {
    switch (t) {
        case DType::Q4_0: case DType::Q4_1: case DType::Q5_0: case DType::Q5_1:
        case DType::Q8_0: case DType::Q8_1: case DType::IQ4_NL:
            return 32;
        case DType::Q2_K: case DType::Q3_K: case DType::Q4_K: case DType::Q5_K: case DType::Q6_K:
        case DType::Q8_K: case DType::IQ2_XXS: case DType::IQ2_XS: case DType::IQ3_XXS: case DType::IQ1_S:
        case DType::IQ3_S: case DType::IQ2_S: case DType::IQ4_XS: case DType::IQ1_M: case DType::TQ1_0:
        case DType::TQ2_0:
            return 256;
        default:
            return 1;
    }
}

size_t dtype_type_size(DType t) {
    switch (t) {
        case DType::F32: case DType::I32: return 4;
        case DType::F16: case DType::BF16: case DType::I16: return 2;
        case DType::F64: case DType::I64: return 8;
        case DType::I8: return 1;
        case DType::Q4_0: return 18;
        case DType::Q4_1: return 20;
        case DType::Q5_0: return 22;
        case DType::Q5_1: return 24;
        case DType::Q8_0: return 34;
        case DType::Q8_1: return 36;
        case DType::Q2_K: return 84;
        case DType::Q3_K: return 110;
        case DType::Q4_K: return 144;
        case DType::Q5_K: return 176;
        case DType::Q6_K: return 210;
        case DType::Q8_K: return 292;
        case DType::IQ2_XXS: return 66;
        case DType::IQ2_XS: return 74;
        case DType::IQ2_S: return 82;
        case DType::IQ3_XXS: return 98;
        case DType::IQ3_S: return 110;
        case DType::IQ1_S: return 50;
        case DType::IQ1_M: return 56;
        case DType::IQ4_NL: return 18;
        case DType::IQ4_XS: return 136;
        case DType::TQ1_0: return 54;
        case DType::TQ2_0: return 66;
        default: return 0;
    }
}

size_t dtype_row_bytes(DType t, uint64_t n) {
    const size_t ts = dtype_type_size(t);
    const uint64_t bs = (uint64_t)dtype_block_size(t);
    if (ts == 0 || n % bs) return 0;
    return (size_t)(n / bs) * ts;
}

const char* dtype_name(DType t) {
    switch (t) {
        case DType::F32: return "F32"; case DType::F16: return "F16"; case DType::BF16: return "BF16";
        case DType::F64: return "F64"; case DType::I8: return "I8"; case DType::I16: return "I16";
        case DType::I32: return "I32"; case DType::I64: return "I64";
        case DType::Q4_0: return "Q4_0"; case DType::Q4_1: return "Q4_1"; case DType::Q5_0: return "Q5_0";
        case DType::Q5_1: return "Q5_1"; case DType::Q8_0: return "Q8_0"; case DType::Q8_1: return "Q8_1";
        case DType::Q2_K: return "Q2_K"; case DType::Q3_K: return "Q3_K"; case DType::Q4_K: return "Q4_K";
        case DType::Q5_K: return "Q5_K"; case DType::Q6_K: return "Q6_K"; case DType::Q8_K: return "Q8_K";
        case DType::IQ2_XXS: return "IQ2_XXS"; case DType::IQ2_XS: return "IQ2_XS"; case DType::IQ2_S: return "IQ2_S";
        case DType::IQ3_XXS: return "IQ3_XXS"; case DType::IQ3_S: return "IQ3_S"; case DType::IQ1_S: return "IQ1_S";
        case DType::IQ1_M: return "IQ1_M"; case DType::IQ4_NL: return "IQ4_NL"; case DType::IQ4_XS: return "IQ4_XS";
        case DType::TQ1_0: return "TQ1_0"; case DType::TQ2_0: return "TQ2_0";
        default: return "UNKNOWN";
    }
}

// ---------------------------------------------------------------- values

uint64_t GgufValue::as_u64() const {
    switch (type) {
        case GgufValueType::UINT8: case GgufValueType::UINT16: case GgufValueType::UINT32:
        case GgufValueType::UINT64: case GgufValueType::BOOL:
            return bits;
        case GgufValueType::INT8: return (uint64_t)(int64_t)(int8_t)bits;
        case GgufValueType::INT16: return (uint64_t)(int64_t)(int16_t)bits;
        case GgufValueType::INT32: return (uint64_t)(int64_t)(int32_t)bits;
        case GgufValueType::INT64: return bits;
        case GgufValueType::FLOAT32: case GgufValueType::FLOAT64: return (uint64_t)as_f64();
        default: throw std::runtime_error("GGUF: value is not numeric");
    }
}

int64_t GgufValue::as_i64() const { return (int64_t)as_u64(); }

double GgufValue::as_f64() const {
    if (type == GgufValueType::FLOAT32) {
        float f;
        const uint32_t u = (uint32_t)bits;
        std::memcpy(&f, &u, 4);
        return f;
    }
    if (type == GgufValueType::FLOAT64) {
        double d;
        std::memcpy(&d, &bits, 8);
        return d;
    }
    switch (type) {
        case GgufValueType::INT8: case GgufValueType::INT16: case GgufValueType::INT32: case GgufValueType::INT64:
            return (double)as_i64();
        default: return (double)as_u64();
    }
}

bool GgufValue::as_bool() const { return type == GgufValueType::BOOL ? bits != 0 : as_u64() != 0; }

const std::string& GgufValue::as_str() const {
    if (type != GgufValueType::STRING) throw std::runtime_error("GGUF: value is not a string");
    return str;
}

uint64_t TensorInfo::n_elements() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
}

uint64_t TensorInfo::n_rows() const { return dims.empty() || dims[0] == 0 ? 0 : n_elements() / dims[0]; }

uint64_t TensorInfo::row_bytes() const { return dims.empty() ? 0 : dtype_row_bytes(type, dims[0]); }

uint64_t TensorInfo::n_bytes() const { return row_bytes() * n_rows(); }

// ---------------------------------------------------------------- parsing

namespace {

// Sequential reads of the file from offset 0: straight from the mapping, or
// from a prefix read with pread and grown on demand. Every length is checked
// against the file size before it is used.
class Reader {
public:
    Reader(int fd, const uint8_t* map, uint64_t size) : fd_(fd), map_(map), size_(size) {}

    uint64_t pos() const { return pos_; }
    uint64_t left() const { return size_ - pos_; }

    const uint8_t* take(uint64_t n) {
        if (n > left()) throw std::runtime_error("GGUF: unexpected end of file");
        const uint64_t at = pos_;
        pos_ += n;
        if (map_) return map_ + at;
        if (pos_ > buf_.size()) grow(pos_);
        return buf_.data() + at;
    }
    template <typename T>
    T read() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string read_str() {
        const uint64_t n = read<uint64_t>();
        const uint8_t* p = take(n);
        return std::string(reinterpret_cast<const char*>(p), (size_t)n);
    }

private:
    void grow(uint64_t need) {
        uint64_t want = std::max<uint64_t>(need, std::max<uint64_t>(2 * buf_.size(), 1u << 20));
        want = std::min(want, size_);
        const size_t old = buf_.size();
        buf_.resize((size_t)want);
        size_t got = old;
        while (got < buf_.size()) {
            const ssize_t r = ::pread(fd_, buf_.data() + got, buf_.size() - got, (off_t)got);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) throw std::runtime_error("GGUF: short read of header");
            got += (size_t)r;
        }
    }

    int fd_;
    const uint8_t* map_;
    uint64_t size_;
    uint64_t pos_ = 0;
    std::vector<uint8_t> buf_;
};

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read little-endian

GgufValue read_value(Reader& r, GgufValueType type, int depth) {
    GgufValue v;
    v.type = type;
    switch (type) {
        case GgufValueType::UINT8: case GgufValueType::INT8: case GgufValueType::BOOL:
            v.bits = r.read<uint8_t>();
            break;
        case GgufValueType::UINT16: case GgufValueType::INT16: v.bits = r.read<uint16_t>(); break;
        case GgufValueType::UINT32: case GgufValueType::INT32: case GgufValueType::FLOAT32:
            v.bits = r.read<uint32_t>();
            break;
        case GgufValueType::UINT64: case GgufValueType::INT64: case GgufValueType::FLOAT64:
            v.bits = r.read<uint64_t>();
            break;
        case GgufValueType::STRING: v.str = r.read_str(); break;
        case GgufValueType::ARRAY: {
            if (depth > 8) throw std::runtime_error("GGUF: arrays nested too deep");
            v.array_type = static_cast<GgufValueType>(r.read<uint32_t>());
            const uint64_t n = r.read<uint64_t>();
            if (n > r.left()) throw std::runtime_error("GGUF: array longer than the file");
            v.array.reserve((size_t)n);
            for (uint64_t i = 0; i < n; ++i) v.array.push_back(read_value(r, v.array_type, depth + 1));
            break;
        }
        default: throw std::runtime_error("GGUF: bad value type");
    }
    return v;
}

}  // namespace

std::shared_ptr<GgufFile> GgufFile::open(const std::string& path) {
    std::shared_ptr<GgufFile> f(new GgufFile());
    f->path_ = path;
    f->parse();
    return f;
}

GgufFile::~GgufFile() {
    if (map_) ::munmap(const_cast<uint8_t*>(map_), (size_t)file_size_);
    if (fd_ >= 0) ::close(fd_);
}

void GgufFile::parse() {
    fd_ = ::open(path_.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw std::runtime_error("GGUF: cannot open " + path_);
    struct stat st {};
    if (::fstat(fd_, &st) != 0) throw std::runtime_error("GGUF: cannot stat " + path_);
    file_size_ = (uint64_t)st.st_size;
    if (file_size_ > 0) {
        void* p = ::mmap(nullptr, (size_t)file_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (p != MAP_FAILED) map_ = static_cast<const uint8_t*>(p);
    }
    Reader r(fd_, map_, file_size_);
    if (r.read<uint32_t>() != kMagic) throw std::runtime_error("GGUF: bad magic");
    version_ = r.read<uint32_t>();
    if (version_ < 2 || version_ > 3) throw std::runtime_error("GGUF: unsupported version");
    const uint64_t n_tensors = r.read<uint64_t>();
    const uint64_t n_kv = r.read<uint64_t>();
    if (n_tensors > r.left() || n_kv > r.left()) throw std::runtime_error("GGUF: counts larger than the file");

    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.read_str();
        const auto vt = static_cast<GgufValueType>(r.read<uint32_t>());
        GgufValue v = read_value(r, vt, 0);
        if (key == "general.alignment") {
            const uint64_t a = v.as_u64();
            if (a == 0 || a > (1u << 30) || (a & (a - 1))) throw std::runtime_error("GGUF: bad alignment");
            alignment_ = (uint32_t)a;
        }
        metadata_.emplace(std::move(key), std::move(v));  // a repeated key keeps its first value
    }

    tensors_.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo t;
        t.name = r.read_str();
        const uint32_t nd = r.read<uint32_t>();
        if (nd > 8) throw std::runtime_error("GGUF: tensor with more than 8 dimensions");
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d) t.dims[d] = r.read<uint64_t>();
        t.type = static_cast<DType>(r.read<uint32_t>());
        t.offset = r.read<uint64_t>();
        tensor_index_.emplace(t.name, tensors_.size());
        tensors_.push_back(std::move(t));
    }
    // the tensor data starts at the first alignment boundary after the infos
    data_offset_ = (r.pos() + alignment_ - 1) / alignment_ * alignment_;
    for (const TensorInfo& t : tensors_) {
        const uint64_t nb = t.n_bytes();
        if (nb && (t.offset > file_size_ || data_offset_ + t.offset + nb > file_size_))
            throw std::runtime_error("GGUF: tensor " + t.name + " runs past the end of " + path_);
    }
    if (map_) ::madvise(const_cast<uint8_t*>(map_), (size_t)file_size_, MADV_SEQUENTIAL);
}

const GgufValue* GgufFile::find(const std::string& key) const {
    auto it = metadata_.find(key);
    return it == metadata_.end() ? nullptr : &it->second;
}

const GgufValue& GgufFile::get(const std::string& key) const {
    const GgufValue* v = find(key);
    if (!v) throw std::runtime_error("GGUF: missing metadata key " + key);
    return *v;
}

std::vector<std::string> GgufFile::keys() const {
    std::vector<std::string> out;
    out.reserve(metadata_.size());
    for (const auto& kv : metadata_) out.push_back(kv.first);
    std::sort(out.begin(), out.end());
    return out;
}

const TensorInfo* GgufFile::find_tensor(const std::string& name) const {
    auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

void GgufFile::set_shard(int shard) {
    shard_ = shard;
    for (TensorInfo& t : tensors_) t.shard = shard;
}

void GgufFile::read_at(uint64_t offset, size_t bytes, void* dst) const {
    if (offset > file_size_ || data_offset_ + offset + bytes > file_size_)
        throw std::runtime_error("GGUF: short read of tensor data in " + path_);
    const uint64_t at = data_offset_ + offset;
    if (map_) {
        std::memcpy(dst, map_ + at, bytes);
        return;
    }
    uint8_t* d = static_cast<uint8_t*>(dst);
    size_t got = 0;
    while (got < bytes) {
        const ssize_t r = ::pread(fd_, d + got, bytes - got, (off_t)(at + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) throw std::runtime_error("GGUF: short read of tensor data in " + path_);
        got += (size_t)r;
    }
}

void GgufFile::read_tensor(const TensorInfo& t, void* dst) const {
    if (t.shard != shard_) throw std::runtime_error("GGUF: tensor belongs to a different shard");
    read_at(t.offset, (size_t)t.n_bytes(), dst);
}

// ---------------------------------------------------------------- model

void GgufModel::load(const std::vector<std::string>& paths) {
    files_.clear();
    tensor_map_.clear();
    tensor_names_.clear();
    for (size_t i = 0; i < paths.size(); ++i) {
        auto f = GgufFile::open(paths[i]);
        f->set_shard((int)i);
        files_.push_back(std::move(f));
    }
    for (const auto& f : files_)
        for (const TensorInfo& t : f->tensors())
            if (tensor_map_.emplace(t.name, &t).second) tensor_names_.push_back(t.name);
}

const GgufValue* GgufModel::find(const std::string& key) const {
    for (const auto& f : files_)
        if (const GgufValue* v = f->find(key)) return v;
    return nullptr;
}

std::vector<std::string> GgufModel::keys() const {
    return files_.empty() ? std::vector<std::string>{} : files_.front()->keys();
}

const TensorInfo* GgufModel::find_tensor(const std::string& name) const {
    auto it = tensor_map_.find(name);
    return it == tensor_map_.end() ? nullptr : it->second;
}

void GgufModel::read_tensor(const TensorInfo& t, void* dst) const { files_.at((size_t)t.shard)->read_tensor(t, dst); }

std::vector<std::string> GgufModel::discover_shards(const std::string& any_shard) {
    // <dir>/<prefix>-<i>-of-<n><ext>, i and n zero-padded to the same width
    const size_t slash = any_shard.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "" : any_shard.substr(0, slash + 1);
    const std::string base = any_shard.substr(dir.size());
    const size_t dot = base.rfind('.');
    const std::string stem = dot == std::string::npos ? base : base.substr(0, dot);
    const std::string ext = dot == std::string::npos ? "" : base.substr(dot);
    const size_t of = stem.rfind("-of-");
    if (of == std::string::npos || of == 0) return {any_shard};
    const size_t dash = stem.rfind('-', of - 1);
    if (dash == std::string::npos) return {any_shard};
    const std::string idx = stem.substr(dash + 1, of - dash - 1), total = stem.substr(of + 4);
    auto digits = [](const std::string& s) {
        return !s.empty() && std::all_of(s.begin(), s.end(), [](char c) { return c >= '0' && c <= '9'; });
    };
    if (!digits(idx) || !digits(total)) return {any_shard};
    const int n = std::stoi(total);
    std::vector<std::string> out;
    for (int i = 1; i <= n; ++i) {
        char num[32];
        std::snprintf(num, sizeof num, "%0*d", (int)idx.size(), i);
        out.push_back(dir + stem.substr(0, dash) + "-" + num + "-of-" + total + ext);
    }
    return out;
}

}  // namespace gpu
}  // namespace glm5
