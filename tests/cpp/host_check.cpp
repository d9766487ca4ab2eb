// Drives the C++ host layer (gpeed_amd/host/glm5_gpu.h) for the GPU tests:
// reads raw inputs written by tests/test_gpu_host_cpp.py, calls the
// reference-signature entry points, writes the outputs back. The checks
// against the oracle happen in the Python test.
//
//   host_check kernels
//   host_check errors
//   host_check matmul <dir> <n_rows> <in_dim> <row0> <out_dim> <n_tok>
//       reads <dir>/w.bin, <dir>/x.bin; writes <dir>/y.bin (matvec_quant of
//       token 0) and <dir>/Y.bin (matmul_quant)
//   host_check moe <dir> <n_exp> <hidden> <inter> <n_tok> <top_k> <mode>
//       reads gate.bin up.bin down.bin x.bin logits.bin; writes Y.bin
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../gpeed_amd/host/glm5_gpu.h"

namespace {

std::vector<char> slurp(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("cannot open " + path);
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::vector<char> buf((size_t)n);
    if (n > 0 && std::fread(buf.data(), 1, (size_t)n, f) != (size_t)n) throw std::runtime_error("short read " + path);
    std::fclose(f);
    return buf;
}

void spit(const std::string& path, const void* p, size_t n) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, n, f) != n) throw std::runtime_error("cannot write " + path);
    std::fclose(f);
}

bool throws_with(const std::function<void()>& fn, const std::string& what) {
    try {
        fn();
    } catch (const std::runtime_error& e) {
        return std::string(e.what()).find(what) != std::string::npos;
    }
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const std::string mode = argc > 1 ? argv[1] : "";
        if (mode == "kernels") {
            const int n = glm5::cuda_device_count();
            const std::string name = glm5::cuda_device_name(0);
            std::vector<float> a(1000), b(1000), c(1000);
            for (int i = 0; i < 1000; ++i) {
                a[i] = 0.5f * i;
                b[i] = 1.0f - i;
            }
            glm5::cuda_add(a.data(), b.data(), c.data(), 1000);
            for (int i = 0; i < 1000; ++i)
                if (c[i] != a[i] + b[i]) throw std::runtime_error("cuda_add mismatch");
            std::printf("devices=%d name=%s add=ok\n", n, name.c_str());
            return 0;
        }
        if (mode == "errors") {
            glm5::gpu::WeightStore ws;
            std::vector<unsigned char> w(98 * 2 * 64, 0);
            ws.add("blk.0.ffn_up.weight", w.data(), 64, 512);
            std::vector<float> x(512, 1.0f), y(64);
            const bool a = throws_with([&] { ws.matvec_quant("nope", 0, 512, 64, x.data(), y.data()); },
                                       "weights: missing tensor nope");
            const bool b = throws_with([&] { ws.matvec_quant("blk.0.ffn_up.weight", 0, 500, 64, x.data(), y.data()); },
                                       "weights: row not block aligned for blk.0.ffn_up.weight");
            ws.matmul_quant("blk.0.ffn_up.weight", 0, 512, 64, x.data(), 0, y.data());  // n_tok <= 0: no-op
            ws.matvec_quant("blk.0.ffn_up.weight", 0, 512, 64, x.data(), y.data());
            bool zero = true;
            for (float v : y) zero = zero && v == 0.0f;  // all-zero weights
            std::printf("missing=%d unaligned=%d zero=%d\n", a, b, zero);
            return a && b && zero ? 0 : 1;
        }
        if (mode == "matmul" && argc == 8) {
            const std::string dir = argv[2];
            const uint64_t n_rows = std::strtoull(argv[3], nullptr, 10);
            const int in_dim = std::atoi(argv[4]), out_dim = std::atoi(argv[6]), n_tok = std::atoi(argv[7]);
            const uint64_t row0 = std::strtoull(argv[5], nullptr, 10);
            const std::vector<char> w = slurp(dir + "/w.bin"), x = slurp(dir + "/x.bin");
            glm5::gpu::WeightStore ws;
            ws.add("t", w.data(), n_rows, in_dim);
            std::vector<float> y((size_t)out_dim), Y((size_t)n_tok * out_dim);
            const float* X = reinterpret_cast<const float*>(x.data());
            ws.matvec_quant("t", row0, in_dim, out_dim, X, y.data());
            ws.matmul_quant("t", row0, in_dim, out_dim, X, n_tok, Y.data());
            spit(dir + "/y.bin", y.data(), y.size() * 4);
            spit(dir + "/Y.bin", Y.data(), Y.size() * 4);
            return 0;
        }
        if (mode == "moe" && argc == 9) {
            const std::string dir = argv[2];
            const int E = std::atoi(argv[3]), H = std::atoi(argv[4]), I = std::atoi(argv[5]);
            const int T = std::atoi(argv[6]), K = std::atoi(argv[7]), md = std::atoi(argv[8]);
            glm5::gpu::WeightStore ws;
            ws.add("gate", slurp(dir + "/gate.bin").data(), (uint64_t)E * I, H);
            ws.add("up", slurp(dir + "/up.bin").data(), (uint64_t)E * I, H);
            ws.add("down", slurp(dir + "/down.bin").data(), (uint64_t)E * H, I);
            const std::vector<char> x = slurp(dir + "/x.bin"), lg = slurp(dir + "/logits.bin");
            std::vector<float> Y((size_t)T * H);
            ws.moe_experts("gate", "up", "down", E, H, I, reinterpret_cast<const float*>(x.data()), T,
                           reinterpret_cast<const float*>(lg.data()), K, md, nullptr, md == 0 ? 2.5f : 1.0f, true,
                           10.0f, Y.data());
            spit(dir + "/Y.bin", Y.data(), Y.size() * 4);
            return 0;
        }
        std::fprintf(stderr, "usage: host_check kernels|errors|matmul ...|moe ...\n");
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "host_check: %s\n", e.what());
        return 1;
    }
}
