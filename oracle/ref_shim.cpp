// C entry points over the reference's own CPU path, for oracle/_ref.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// the reference's unmodified cpp/core/src/{quant,gguf,weights}.cpp, read in
// place from the reference checkout, into oracle/_ref/libgpeed_ref*.so. The
// library is used to pin the plain-C oracle bit for bit and as the
// "reference" CPU baseline in bench.py. Nothing in the product loads it.
//
// WeightStore::matvec_quant / matmul_quant need a GgufModel, so ref_store_open
// writes the caller's payload as a one-tensor GGUF v3 file (the layout
// gguf.cpp:102-139 parses), loads it with GgufModel::load, pins it with
// WeightStore::pin_nonexpert (weights.cpp:70-84) so later calls read RAM, and
// removes the file.
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <unistd.h>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "glm5/common.h"
#include "glm5/gguf.h"
#include "glm5/quant.h"
#include "glm5/simd.h"
#include "glm5/weights.h"

namespace {

thread_local std::string g_err;

struct RefStore {
    glm5::GgufModel model;
    std::unique_ptr<glm5::WeightStore> store;
    std::string name;
};

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
    for (int i = 0; i < 4; ++i) b.push_back(static_cast<uint8_t>(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& b, uint64_t v) {
    for (int i = 0; i < 8; ++i) b.push_back(static_cast<uint8_t>(v >> (8 * i)));
}
void put_str(std::vector<uint8_t>& b, const std::string& s) {
    put_u64(b, s.size());
    b.insert(b.end(), s.begin(), s.end());
}

// JSON of what the reference loader parsed, in the schema of the product
// loader's dump (tests/cpp/host_check gguf-info), for a field-by-field
// comparison.
std::string jstr(const std::string& v) {
    std::string o = "\"";
    for (unsigned char c : v) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += (char)c;
        } else if (c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
        } else {
            o += (char)c;
        }
    }
    return o + "\"";
}

std::string jval(const glm5::GgufValue& v) {
    using T = glm5::GgufValueType;
    char buf[64];
    switch (v.type) {
        case T::STRING: return jstr(v.as_str());
        case T::ARRAY: {
            std::string o = "[";
            for (size_t i = 0; i < v.array.size(); ++i) o += (i ? "," : "") + jval(v.array[i]);
            return o + "]";
        }
        case T::FLOAT32: case T::FLOAT64: std::snprintf(buf, sizeof buf, "%.17g", v.as_f64()); return buf;
        case T::BOOL: return v.as_bool() ? "true" : "false";
        case T::INT8: case T::INT16: case T::INT32: case T::INT64:
            std::snprintf(buf, sizeof buf, "%lld", (long long)v.as_i64());
            return buf;
        default: std::snprintf(buf, sizeof buf, "%llu", (unsigned long long)v.as_u64()); return buf;
    }
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

int ref_dequantize(int dtype, const void* src, float* dst, uint64_t n) {
    try {
        glm5::dequantize(static_cast<glm5::DType>(dtype), src, dst, n);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int ref_dequantize_row(int dtype, const void* src, float* dst, uint64_t n) {
    try {
        glm5::dequantize_row(static_cast<glm5::DType>(dtype), src, dst, n);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

float ref_dot_f32(const float* a, const float* b, int n) { return glm5::dot_f32(a, b, n); }

void ref_axpy_f32(float* a, const float* b, float s, int n) { glm5::axpy_f32(a, b, s, n); }

// Registers `n_rows` rows of `in_dim` weights of type `dtype` (payload in
// GGUF row order) as tensor `name`. Returns a handle, or nullptr with
// ref_last_error().
void* ref_store_open_typed(const uint8_t* payload, uint64_t n_rows, int in_dim, int dtype, const char* name,
                           const char* tmpdir) {
    try {
        auto* h = new RefStore();
        h->name = name;
        const auto type = static_cast<glm5::DType>(dtype);
        const size_t rb = glm5::dtype_row_bytes(type, static_cast<uint64_t>(in_dim));
        const size_t bytes = rb * n_rows;
        std::vector<uint8_t> hdr;
        put_u32(hdr, 0x46554747u);  // "GGUF"
        put_u32(hdr, 3);
        put_u64(hdr, 1);  // tensors
        put_u64(hdr, 1);  // kv pairs
        put_str(hdr, "general.alignment");
        put_u32(hdr, 4);  // UINT32
        put_u32(hdr, 32);
        put_str(hdr, h->name);
        put_u32(hdr, 2);
        put_u64(hdr, static_cast<uint64_t>(in_dim));
        put_u64(hdr, n_rows);
        put_u32(hdr, static_cast<uint32_t>(type));
        put_u64(hdr, 0);
        while (hdr.size() % 32) hdr.push_back(0);
        std::string path = std::string(tmpdir ? tmpdir : "/tmp") + "/gpeed_ref_" +
                           std::to_string(::getpid()) + "_" +
                           std::to_string(reinterpret_cast<uintptr_t>(h)) + ".gguf";
        FILE* f = std::fopen(path.c_str(), "wb");
        if (!f) throw std::runtime_error("ref_store_open: cannot create " + path);
        std::fwrite(hdr.data(), 1, hdr.size(), f);
        std::fwrite(payload, 1, bytes, f);
        std::fclose(f);
        h->model.load({path});
        h->store = std::make_unique<glm5::WeightStore>(h->model, false);
        h->store->pin_nonexpert();
        std::remove(path.c_str());
        return h;
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

void* ref_store_open(const uint8_t* payload, uint64_t n_rows, int in_dim, const char* name, const char* tmpdir) {
    return ref_store_open_typed(payload, n_rows, in_dim, static_cast<int>(glm5::DType::IQ3_XXS), name, tmpdir);
}

int ref_store_resident_bytes(void* hp, uint64_t* out) {
    *out = static_cast<RefStore*>(hp)->store->resident_bytes();
    return 0;
}

int ref_store_matvec(void* hp, uint64_t row0, int in_dim, int out_dim, const float* x, float* dst) {
    try {
        auto* h = static_cast<RefStore*>(hp);
        h->store->matvec_quant(h->name, row0, in_dim, out_dim, x, dst);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int ref_store_matmul(void* hp, uint64_t row0, int in_dim, int out_dim, const float* X, int n_tok,
                     float* Y) {
    try {
        auto* h = static_cast<RefStore*>(hp);
        h->store->matmul_quant(h->name, row0, in_dim, out_dim, X, n_tok, Y);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

void ref_store_close(void* hp) { delete static_cast<RefStore*>(hp); }

// The reference loader's view of a GGUF model (GgufModel::load over the
// shards GgufModel::discover_shards finds), as JSON into out (len bytes);
// returns the JSON length, or -1 (message in ref_last_error).
long ref_gguf_dump(const char* path, char* out, size_t len) {
    try {
        glm5::GgufModel m;
        m.load(glm5::GgufModel::discover_shards(path));
        const glm5::GgufFile& f0 = m.file(0);
        std::string o = "{\"version\":" + std::to_string(f0.version()) +
                        ",\"data_offset\":" + std::to_string(f0.data_offset()) +
                        ",\"shards\":" + std::to_string(m.files().size()) + ",\"kv\":{";
        const auto keys = m.keys();
        for (size_t i = 0; i < keys.size(); ++i) {
            const glm5::GgufValue* v = m.find(keys[i]);
            o += (i ? "," : "") + jstr(keys[i]) + ":{\"type\":" + std::to_string((unsigned)v->type) +
                 ",\"array_type\":" + std::to_string((unsigned)v->array_type) + ",\"value\":" + jval(*v) + "}";
        }
        o += "},\"tensors\":[";
        const auto& names = m.tensor_names();
        for (size_t i = 0; i < names.size(); ++i) {
            const glm5::TensorInfo* t = m.find_tensor(names[i]);
            std::string dims;
            for (size_t d = 0; d < t->dims.size(); ++d) dims += (d ? "," : "") + std::to_string(t->dims[d]);
            const uint64_t rows = t->dims.empty() ? 0 : t->n_elements() / t->dims[0];
            o += std::string(i ? "," : "") + "{\"name\":" + jstr(t->name) + ",\"type\":" +
                 std::to_string((unsigned)t->type) + ",\"dims\":[" + dims + "],\"offset\":" +
                 std::to_string(t->offset) + ",\"shard\":" + std::to_string(t->shard) + ",\"n_bytes\":" +
                 std::to_string(t->row_bytes() * rows) + ",\"rows\":" + std::to_string(rows) + "}";
        }
        o += "]}";
        if (o.size() + 1 > len) {
            g_err = "ref_gguf_dump: buffer too small";
            return -1;
        }
        std::memcpy(out, o.c_str(), o.size() + 1);
        return (long)o.size();
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// GgufModel::read_tensor of one tensor into dst (len bytes at most).
long ref_gguf_read(const char* path, const char* name, void* dst, size_t len) {
    try {
        glm5::GgufModel m;
        m.load(glm5::GgufModel::discover_shards(path));
        const glm5::TensorInfo* t = m.find_tensor(name);
        if (!t) throw std::runtime_error(std::string("no tensor ") + name);
        const uint64_t rows = t->dims.empty() ? 0 : t->n_elements() / t->dims[0];
        const size_t n = (size_t)(t->row_bytes() * rows);
        if (n > len) throw std::runtime_error("ref_gguf_read: buffer too small");
        m.read_tensor(*t, dst);
        return (long)n;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// Threads the OpenMP regions of matvec_quant / matmul_quant will use (1 for
// the library built without -fopenmp, as the reference is on Linux).
int ref_openmp_threads() {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
