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

// Registers `n_rows` rows of `in_dim` IQ3_XXS weights (payload in GGUF row
// order) as tensor `name`. Returns a handle, or nullptr with ref_last_error().
void* ref_store_open(const uint8_t* payload, uint64_t n_rows, int in_dim, const char* name,
                     const char* tmpdir) {
    try {
        auto* h = new RefStore();
        h->name = name;
        const size_t rb = glm5::dtype_row_bytes(glm5::DType::IQ3_XXS, static_cast<uint64_t>(in_dim));
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
        put_u32(hdr, static_cast<uint32_t>(glm5::DType::IQ3_XXS));
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
