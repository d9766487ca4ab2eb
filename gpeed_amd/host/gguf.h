// GGUF v2/v3 reader for the device-resident weight store.
//
// Mirrors the reference's loader interface (cpp/core/include/glm5/gguf.h:
// GgufValueType, GgufValue, TensorInfo, GgufFile, GgufModel with the same
// method names and meanings; parse order of cpp/core/src/gguf.cpp:135-187,
// byte reads of gguf.cpp:242-260) so a caller written against it switches
// by namespace. Differences, all on the host side of the hot path:
// * the file is memory-mapped on Linux as well (the reference maps only on
//   Windows, gguf.cpp:220-240), so payloads go from the page cache straight
//   into the host-to-device copy; without a mapping, reads use pread;
// * the header is parsed from the mapping (or from a prefix grown on
//   demand), with every length checked against the file size;
// * errors are std::runtime_error with the reference's "GGUF: ..." texts.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace glm5 {
namespace gpu {

// ggml tensor types (values are the GGUF file's type ids; cpp/core/include/
// glm5/common.h:10-45 lists the same ids).
enum class DType : uint32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9,
    Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15,
    IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23,
    I8 = 24, I16 = 25, I32 = 26, I64 = 27, F64 = 28, IQ1_M = 29, BF16 = 30, TQ1_0 = 34, TQ2_0 = 35,
};

// Elements per block (1 for scalar types), bytes per block (or per element),
// bytes of n elements (0 if the type's layout is unknown or n is not a whole
// number of blocks) -- the ggml format's geometry (quant.cpp:52-126).
int dtype_block_size(DType t);
size_t dtype_type_size(DType t);
size_t dtype_row_bytes(DType t, uint64_t n_elements);
const char* dtype_name(DType t);

enum class GgufValueType : uint32_t {
    UINT8 = 0, INT8 = 1, UINT16 = 2, INT16 = 3, UINT32 = 4, INT32 = 5, FLOAT32 = 6, BOOL = 7,
    STRING = 8, ARRAY = 9, UINT64 = 10, INT64 = 11, FLOAT64 = 12,
};

struct GgufValue {
    GgufValueType type = GgufValueType::UINT8;
    uint64_t bits = 0;                   // scalar payload, little-endian, zero-extended
    std::string str;                     // STRING
    GgufValueType array_type = GgufValueType::UINT8;
    std::vector<GgufValue> array;        // ARRAY

    bool is_array() const { return type == GgufValueType::ARRAY; }
    // Integer / float coercions of a scalar (throw for strings and arrays).
    uint64_t as_u64() const;
    int64_t as_i64() const;
    double as_f64() const;
    bool as_bool() const;
    const std::string& as_str() const;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;  // ggml order: dims[0] is the row length
    DType type = DType::F32;
    uint64_t offset = 0;         // from the start of the tensor-data section
    int shard = 0;

    uint64_t n_elements() const;
    uint64_t n_rows() const;     // n_elements / dims[0]
    uint64_t row_bytes() const;  // bytes of one row of dims[0] elements
    uint64_t n_bytes() const;    // row_bytes * n_rows
};

class GgufFile {
public:
    static std::shared_ptr<GgufFile> open(const std::string& path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const std::string& path() const { return path_; }
    uint32_t version() const { return version_; }
    uint32_t alignment() const { return alignment_; }
    uint64_t data_offset() const { return data_offset_; }
    uint64_t file_size() const { return file_size_; }
    size_t n_tensors() const { return tensors_.size(); }

    bool has(const std::string& key) const { return metadata_.count(key) != 0; }
    const GgufValue* find(const std::string& key) const;
    const GgufValue& get(const std::string& key) const;
    std::vector<std::string> keys() const;  // sorted

    const std::vector<TensorInfo>& tensors() const { return tensors_; }
    const TensorInfo* find_tensor(const std::string& name) const;
    void set_shard(int shard);

    // Copies `bytes` of the tensor-data section from `offset` into dst.
    void read_at(uint64_t offset, size_t bytes, void* dst) const;
    // The whole payload of t (n_bytes()).
    void read_tensor(const TensorInfo& t, void* dst) const;
    // Start of the tensor-data section in the mapping, or nullptr.
    const uint8_t* data_ptr() const { return map_ ? map_ + data_offset_ : nullptr; }

private:
    GgufFile() = default;
    void parse();

    std::string path_;
    int fd_ = -1;
    const uint8_t* map_ = nullptr;
    uint64_t file_size_ = 0;
    uint32_t version_ = 0;
    uint32_t alignment_ = 32;
    int shard_ = 0;
    uint64_t data_offset_ = 0;
    std::vector<TensorInfo> tensors_;
    std::unordered_map<std::string, size_t> tensor_index_;
    std::unordered_map<std::string, GgufValue> metadata_;
};

// One or more shards forming a model.
class GgufModel {
public:
    void load(const std::vector<std::string>& paths);
    const GgufValue* find(const std::string& key) const;
    const GgufFile& file(size_t i) const { return *files_.at(i); }
    const std::vector<std::shared_ptr<GgufFile>>& files() const { return files_; }
    std::vector<std::string> keys() const;
    const TensorInfo* find_tensor(const std::string& name) const;
    const std::vector<std::string>& tensor_names() const { return tensor_names_; }
    void read_tensor(const TensorInfo& t, void* dst) const;
    // "<prefix>-<i>-of-<n>.gguf" shards given any one of them (the path
    // itself when the name has no shard suffix).
    static std::vector<std::string> discover_shards(const std::string& any_shard);

private:
    std::vector<std::shared_ptr<GgufFile>> files_;
    std::unordered_map<std::string, const TensorInfo*> tensor_map_;
    std::vector<std::string> tensor_names_;
};

}  // namespace gpu
}  // namespace glm5
