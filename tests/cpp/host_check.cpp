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
//   host_check dequant <dtype> <raw file> <n> <out>
//   host_check gguf-info <file>          (no device use)
//       the GGUF model (shards discovered from the name) as one JSON object
//   host_check gguf-read <file> <tensor> <out>   (no device use)
//       the tensor's payload bytes
//   host_check gguf-store <file> <script>
//       a WeightStore over the model, driven by the script's lines:
//         pin_nonexpert | pin_experts          prints "resident <bytes>"
//         readback <tensor> <out>              GGUF bytes from the HBM copy
//         matvec <tensor> <row0> <in> <out> <x> <y>
//         matmul <tensor> <row0> <in> <out> <n_tok> <X> <Y>
//         moe <gate> <up> <down> <E> <H> <I> <T> <K> <X> <logits> <Y>
//         heads <tensor> <row0> <in> <rows_per_head> <n_heads> <x> <y>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
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

std::string json_str(const std::string& v) {
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

std::string json_value(const glm5::gpu::GgufValue& v) {
    using T = glm5::gpu::GgufValueType;
    char buf[64];
    switch (v.type) {
        case T::STRING: return json_str(v.str);
        case T::ARRAY: {
            std::string o = "[";
            for (size_t i = 0; i < v.array.size(); ++i) o += (i ? "," : "") + json_value(v.array[i]);
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

void gguf_info(const std::string& path) {
    glm5::gpu::GgufModel m;
    m.load(glm5::gpu::GgufModel::discover_shards(path));
    const auto& f0 = m.file(0);
    std::printf("{\"version\":%u,\"alignment\":%u,\"data_offset\":%llu,\"shards\":%zu,\"kv\":{", f0.version(),
                f0.alignment(), (unsigned long long)f0.data_offset(), m.files().size());
    const auto keys = m.keys();
    for (size_t i = 0; i < keys.size(); ++i) {
        const auto* v = m.find(keys[i]);
        std::printf("%s%s:{\"type\":%u,\"array_type\":%u,\"value\":%s}", i ? "," : "", json_str(keys[i]).c_str(),
                    (unsigned)v->type, (unsigned)v->array_type, json_value(*v).c_str());
    }
    std::printf("},\"tensors\":[");
    const auto& names = m.tensor_names();
    for (size_t i = 0; i < names.size(); ++i) {
        const auto* t = m.find_tensor(names[i]);
        std::string dims;
        for (size_t d = 0; d < t->dims.size(); ++d) dims += (d ? "," : "") + std::to_string(t->dims[d]);
        std::printf("%s{\"name\":%s,\"type\":%u,\"type_name\":\"%s\",\"dims\":[%s],\"offset\":%llu,\"shard\":%d,"
                    "\"n_bytes\":%llu,\"rows\":%llu}",
                    i ? "," : "", json_str(t->name).c_str(), (unsigned)t->type, glm5::gpu::dtype_name(t->type),
                    dims.c_str(), (unsigned long long)t->offset, t->shard, (unsigned long long)t->n_bytes(),
                    (unsigned long long)t->n_rows());
    }
    std::printf("]}\n");
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
        if (mode == "moe-batch" && argc == 10) {  // the whole step, shared expert when sh == 1
            const std::string dir = argv[2];
            const int E = std::atoi(argv[3]), H = std::atoi(argv[4]), I = std::atoi(argv[5]);
            const int T = std::atoi(argv[6]), K = std::atoi(argv[7]), md = std::atoi(argv[8]);
            const bool sh = std::atoi(argv[9]) != 0;
            glm5::gpu::WeightStore ws;
            ws.add("gate", slurp(dir + "/gate.bin").data(), (uint64_t)E * I, H);
            ws.add("up", slurp(dir + "/up.bin").data(), (uint64_t)E * I, H);
            ws.add("down", slurp(dir + "/down.bin").data(), (uint64_t)E * H, I);
            if (sh) {
                ws.add("gate_sh", slurp(dir + "/gate_sh.bin").data(), (uint64_t)I, H);
                ws.add("up_sh", slurp(dir + "/up_sh.bin").data(), (uint64_t)I, H);
                ws.add("down_sh", slurp(dir + "/down_sh.bin").data(), (uint64_t)H, I);
            }
            const std::vector<char> x = slurp(dir + "/x.bin"), lg = slurp(dir + "/logits.bin");
            std::vector<float> Y((size_t)T * H);
            ws.moe_batch("gate", "up", "down", sh ? "gate_sh" : "", sh ? "up_sh" : "", sh ? "down_sh" : "", E, H, I,
                         reinterpret_cast<const float*>(x.data()), T, reinterpret_cast<const float*>(lg.data()), K,
                         md, nullptr, md == 0 ? 2.5f : 1.0f, true, 10.0f, Y.data());
            spit(dir + "/Y.bin", Y.data(), Y.size() * 4);
            return 0;
        }
        if (mode == "moe-router" && argc == 9) {  // the whole moe_batch from X: router product on the device too
            const std::string dir = argv[2];
            const int E = std::atoi(argv[3]), H = std::atoi(argv[4]), I = std::atoi(argv[5]);
            const int T = std::atoi(argv[6]), K = std::atoi(argv[7]), md = std::atoi(argv[8]);
            glm5::gpu::WeightStore ws;
            ws.add("blk.0.ffn_gate_inp.weight", slurp(dir + "/router.bin").data(), (uint64_t)E, H,
                   glm5::gpu::DType::F32);
            ws.add("gate", slurp(dir + "/gate.bin").data(), (uint64_t)E * I, H);
            ws.add("up", slurp(dir + "/up.bin").data(), (uint64_t)E * I, H);
            ws.add("down", slurp(dir + "/down.bin").data(), (uint64_t)E * H, I);
            ws.add("gate_sh", slurp(dir + "/gate_sh.bin").data(), (uint64_t)I, H);
            ws.add("up_sh", slurp(dir + "/up_sh.bin").data(), (uint64_t)I, H);
            ws.add("down_sh", slurp(dir + "/down_sh.bin").data(), (uint64_t)H, I);
            const std::vector<char> x = slurp(dir + "/x.bin");
            std::vector<float> Y((size_t)T * H);
            ws.moe_batch("blk.0.ffn_gate_inp.weight", "gate", "up", "down", "gate_sh", "up_sh", "down_sh", E, H, I,
                         reinterpret_cast<const float*>(x.data()), T, K, md, nullptr, md == 0 ? 2.5f : 1.0f, true,
                         10.0f, Y.data());
            spit(dir + "/Y.bin", Y.data(), Y.size() * 4);
            return 0;
        }
        if (mode == "dense-mlp" && argc == 6) {  // Model::dense_mlp / dense_mlp_batch on the device
            const std::string dir = argv[2];
            const int H = std::atoi(argv[3]), I = std::atoi(argv[4]), T = std::atoi(argv[5]);
            glm5::gpu::WeightStore ws;
            ws.add("gate", slurp(dir + "/gate.bin").data(), (uint64_t)I, H);
            ws.add("up", slurp(dir + "/up.bin").data(), (uint64_t)I, H);
            ws.add("down", slurp(dir + "/down.bin").data(), (uint64_t)H, I);
            const std::vector<char> x = slurp(dir + "/x.bin");
            std::vector<float> Y((size_t)T * H);
            ws.dense_mlp("gate", "up", "down", H, I, reinterpret_cast<const float*>(x.data()), T, 10.0f, Y.data());
            spit(dir + "/Y.bin", Y.data(), Y.size() * 4);
            return 0;
        }
        if (mode == "dequant" && argc == 6) {  // host-array dequantize (quant.h:18-22)
            const int dtype = std::atoi(argv[2]);
            const uint64_t n = std::strtoull(argv[4], nullptr, 10);
            const std::vector<char> raw = slurp(argv[3]);
            std::vector<float> out(n);
            glm5::gpu::dequantize(static_cast<glm5::gpu::DType>(dtype), raw.data(), out.data(), n);
            spit(argv[5], out.data(), out.size() * 4);
            return 0;
        }
        if (mode == "gguf-info" && argc == 3) {
            gguf_info(argv[2]);
            return 0;
        }
        if (mode == "gguf-read" && argc == 5) {
            glm5::gpu::GgufModel m;
            m.load(glm5::gpu::GgufModel::discover_shards(argv[2]));
            const auto* t = m.find_tensor(argv[3]);
            if (!t) throw std::runtime_error(std::string("no tensor ") + argv[3]);
            std::vector<char> buf((size_t)t->n_bytes());
            m.read_tensor(*t, buf.data());
            spit(argv[4], buf.data(), buf.size());
            return 0;
        }
        if (mode == "gguf-store" && argc == 4) {
            glm5::gpu::GgufModel m;
            m.load(glm5::gpu::GgufModel::discover_shards(argv[2]));
            glm5::gpu::WeightStore ws(m);
            std::ifstream script(argv[3]);
            std::string line;
            while (std::getline(script, line)) {
                std::istringstream in(line);
                std::string op;
                if (!(in >> op)) continue;
                if (op == "pin_nonexpert" || op == "pin_experts") {
                    const size_t b = op == "pin_nonexpert" ? ws.pin_nonexpert() : ws.pin_experts();
                    std::printf("resident %zu\n", b);
                } else if (op == "readback") {
                    std::string name, out;
                    in >> name >> out;
                    const auto* t = m.find_tensor(name);
                    if (!t) throw std::runtime_error("no tensor " + name);
                    std::vector<char> buf((size_t)t->n_bytes());
                    ws.read_resident(name, buf.data());
                    spit(out, buf.data(), buf.size());
                } else if (op == "matvec" || op == "matmul") {
                    std::string name, xf, yf;
                    uint64_t row0 = 0;
                    int in_dim = 0, out_dim = 0, n_tok = 1;
                    in >> name >> row0 >> in_dim >> out_dim;
                    if (op == "matmul") in >> n_tok;
                    in >> xf >> yf;
                    const std::vector<char> x = slurp(xf);
                    std::vector<float> y((size_t)n_tok * out_dim);
                    if (op == "matvec")
                        ws.matvec_quant(name, row0, in_dim, out_dim, reinterpret_cast<const float*>(x.data()), y.data());
                    else
                        ws.matmul_quant(name, row0, in_dim, out_dim, reinterpret_cast<const float*>(x.data()), n_tok,
                                        y.data());
                    spit(yf, y.data(), y.size() * 4);
                } else if (op == "heads") {
                    std::string name, xf, yf;
                    uint64_t row0 = 0;
                    int in_dim = 0, rph = 0, nh = 0;
                    in >> name >> row0 >> in_dim >> rph >> nh >> xf >> yf;
                    const std::vector<char> x = slurp(xf);
                    std::vector<float> y((size_t)rph * nh);
                    ws.matvec_heads(name, row0, in_dim, rph, nh, reinterpret_cast<const float*>(x.data()), y.data());
                    spit(yf, y.data(), y.size() * 4);
                } else if (op == "moe") {
                    std::string g, u, d, xf, lf, yf;
                    int E, H, I, T, K;
                    in >> g >> u >> d >> E >> H >> I >> T >> K >> xf >> lf >> yf;
                    const std::vector<char> x = slurp(xf), lg = slurp(lf);
                    std::vector<float> Y((size_t)T * H);
                    ws.moe_experts(g, u, d, E, H, I, reinterpret_cast<const float*>(x.data()), T,
                                   reinterpret_cast<const float*>(lg.data()), K, 1, nullptr, 1.0f, true, 10.0f, Y.data());
                    spit(yf, Y.data(), Y.size() * 4);
                } else {
                    throw std::runtime_error("bad script line: " + line);
                }
            }
            std::printf("resident %zu\n", ws.resident_bytes());
            return 0;
        }
        std::fprintf(stderr, "usage: host_check kernels|errors|matmul ...|moe ...|dequant ...|gguf-info|gguf-read|gguf-store\n");
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "host_check: %s\n", e.what());
        return 1;
    }
}
