// C++ host layer over the gpeed C ABI (see glm5_gpu.h).
#include "glm5_gpu.h"

#include <algorithm>
#include <climits>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/gpeed_iq3.h"

namespace glm5 {

namespace {

void check(int rc, const char* what) {
    if (rc != GPEED_OK) throw std::runtime_error(std::string(what) + ": " + gpeed_last_error());
}

constexpr int kH2D = 1, kD2H = 2;

}  // namespace

int cuda_device_count() { return gpeed_device_count(); }

std::string cuda_device_name(int index) {
    char buf[256];
    if (gpeed_device_name(index, buf, sizeof buf) != GPEED_OK) return "<none>";
    return buf;
}

void cuda_add(const float* a, const float* b, float* dst, int n) { check(gpeed_add_f32(a, b, dst, n), "cuda_add"); }

namespace gpu {

WeightStore::WeightStore() { check(gpeed_init(), "gpeed_init"); }

WeightStore::WeightStore(const GgufModel& model) : WeightStore() { model_ = &model; }

void WeightStore::pin(const std::string& name) {
    if (!model_) throw std::runtime_error("weights: no GGUF model attached for " + name);
    const TensorInfo* t = model_->find_tensor(name);
    if (!t) throw std::runtime_error("weights: missing tensor " + name);
    if (t->type != DType::IQ3_XXS)
        throw std::runtime_error(std::string("weights: ") + dtype_name(t->type) + " is not on the GPU path for " + name);
    if (t->dims.empty() || t->dims[0] > (uint64_t)INT32_MAX || t->dims[0] % 256)
        throw std::runtime_error("weights: row not block aligned for " + name);
    // straight from the file mapping when there is one, else through a host copy
    const GgufFile& f = model_->file((size_t)t->shard);
    std::vector<uint8_t> tmp;
    const void* src = f.data_ptr() ? static_cast<const void*>(f.data_ptr() + t->offset) : nullptr;
    if (!src) {
        tmp.resize((size_t)t->n_bytes());
        model_->read_tensor(*t, tmp.data());
        src = tmp.data();
    }
    add(name, src, t->n_rows(), (int)t->dims[0]);
}

size_t WeightStore::pin_matching(bool experts) {
    if (!model_) throw std::runtime_error("weights: no GGUF model attached");
    for (const std::string& name : model_->tensor_names()) {
        const bool is_expert = name.find("exps.weight") != std::string::npos;  // weights.cpp:72-73
        if (is_expert != experts || has(name)) continue;
        const TensorInfo* t = model_->find_tensor(name);
        if (!t || t->type != DType::IQ3_XXS || t->dims.empty() || t->dims[0] % 256) continue;
        pin(name);
    }
    return resident_bytes_;
}

size_t WeightStore::pin_nonexpert() { return pin_matching(false); }

size_t WeightStore::pin_experts() { return pin_matching(true); }

void WeightStore::read_resident(const std::string& name, void* dst) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("weights: missing tensor " + name);
    const Tensor& t = it->second;
    const size_t raw_bytes = gpeed_iq3xxs_row_bytes(t.in_dim) * t.n_rows;
    void* raw = nullptr;
    check(gpeed_malloc(&raw, raw_bytes), "malloc");
    int rc = gpeed_iq3xxs_untile(t.t64, t.n_rows, t.in_dim, raw, nullptr);
    if (rc == GPEED_OK) rc = gpeed_stream_sync(nullptr);
    if (rc == GPEED_OK) rc = gpeed_memcpy(dst, raw, raw_bytes, kD2H);
    (void)gpeed_free(raw);
    check(rc, "weights: read back");
}

WeightStore::~WeightStore() {
    for (auto& kv : tensors_) (void)gpeed_free(kv.second.t64);
    for (auto& kv : ws_) (void)gpeed_free(kv.second.p);
    for (Buffer* b : {&x_, &y_, &route_ws_, &moe_ws_, &logits_, &bias_, &eptr_, &tok_, &wt_})
        (void)gpeed_free(b->p);
}

void* WeightStore::scratch(Buffer& b, size_t bytes, bool init) {
    if (bytes > b.bytes) {
        check(gpeed_free(b.p), "free");
        b.p = nullptr;
        b.bytes = 0;
        bytes = (bytes + 255) / 256 * 256;
        check(gpeed_malloc(&b.p, bytes), "malloc");
        b.bytes = bytes;
        if (init) {
            check(gpeed_ws_init(b.p, bytes, nullptr), "workspace init");
            check(gpeed_stream_sync(nullptr), "sync");
        }
    }
    return b.p;
}

void WeightStore::check_ws(void* ws, const std::string& what) {
    if (gpeed_ws_status(ws, nullptr) != GPEED_OK)
        throw std::runtime_error(what + ": " + gpeed_last_error());
}

void WeightStore::add(const std::string& name, const void* gguf_rows, uint64_t n_rows, int in_dim) {
    const size_t rb = gpeed_iq3xxs_row_bytes(in_dim);
    if (rb == 0) throw std::runtime_error("weights: row not block aligned for " + name);
    const size_t raw_bytes = rb * n_rows;
    void* raw = nullptr;
    check(gpeed_malloc(&raw, raw_bytes), "malloc");
    Tensor t;
    t.n_rows = n_rows;
    t.in_dim = in_dim;
    t.bytes = gpeed_iq3xxs_t64_bytes(n_rows, in_dim);
    int rc = gpeed_memcpy(raw, gguf_rows, raw_bytes, kH2D);
    if (rc == GPEED_OK) rc = gpeed_malloc(&t.t64, t.bytes);
    if (rc == GPEED_OK) rc = gpeed_iq3xxs_tile(raw, n_rows, in_dim, t.t64, nullptr);
    if (rc == GPEED_OK) rc = gpeed_stream_sync(nullptr);
    (void)gpeed_free(raw);
    if (rc != GPEED_OK) {
        (void)gpeed_free(t.t64);
        check(rc, "weights: upload");
    }
    auto it = tensors_.find(name);
    if (it != tensors_.end()) {
        resident_bytes_ -= it->second.bytes;
        (void)gpeed_free(it->second.t64);
    }
    tensors_[name] = t;
    resident_bytes_ += t.bytes;
}

const WeightStore::Tensor& WeightStore::get(const std::string& name, int in_dim) {
    auto it = tensors_.find(name);
    if (it == tensors_.end() && model_ && model_->find_tensor(name) && in_dim % 256 == 0) {
        pin(name);  // first use of a tensor of the attached model
        it = tensors_.find(name);
    }
    if (it == tensors_.end()) throw std::runtime_error("weights: missing tensor " + name);
    if (in_dim % 256 != 0) throw std::runtime_error("weights: row not block aligned for " + name);
    return it->second;
}

void WeightStore::matvec_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* x,
                               float* dst) {
    if (out_dim <= 0) return;  // weights.cpp:88
    const Tensor& t = get(name, in_dim);
    const size_t xb = (size_t)in_dim * sizeof(float), yb = (size_t)out_dim * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    const size_t wsb = gpeed_iq3xxs_matvec_ws_bytes(in_dim, out_dim);
    if (wsb == 0) throw std::runtime_error("weights: unsupported shape for " + name);
    Buffer& wbuf = ws_[std::make_tuple(in_dim, out_dim)];
    void* ws = scratch(wbuf, wsb, true);
    check(gpeed_memcpy(xd, x, xb, kH2D), "weights: upload x");
    check(gpeed_iq3xxs_matvec(t.t64, t.n_rows, row0, in_dim, out_dim, static_cast<const float*>(xd),
                              static_cast<float*>(yd), ws, wbuf.bytes, nullptr),
          ("weights: matvec_quant " + name).c_str());
    check_ws(ws, "weights: matvec_quant " + name);
    check(gpeed_memcpy(dst, yd, yb, kD2H), "weights: download y");
}

void WeightStore::matmul_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* X,
                               int n_tok, float* Y) {
    if (n_tok <= 0 || out_dim <= 0) return;  // weights.cpp:88
    const Tensor& t = get(name, in_dim);
    const size_t xb = (size_t)n_tok * in_dim * sizeof(float), yb = (size_t)n_tok * out_dim * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    const size_t wsb = gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, n_tok);
    if (wsb == 0) throw std::runtime_error("weights: unsupported shape for " + name);
    Buffer& wbuf = ws_[std::make_tuple(in_dim, out_dim)];
    void* ws = scratch(wbuf, wsb, true);
    check(gpeed_memcpy(xd, X, xb, kH2D), "weights: upload x");
    check(gpeed_iq3xxs_matmul(t.t64, t.n_rows, row0, in_dim, out_dim, static_cast<const float*>(xd), n_tok,
                              static_cast<float*>(yd), ws, wbuf.bytes, nullptr),
          ("weights: matmul_quant " + name).c_str());
    check_ws(ws, "weights: matmul_quant " + name);
    check(gpeed_memcpy(Y, yd, yb, kD2H), "weights: download y");
}

void WeightStore::matvec_heads(const std::string& name, uint64_t row0, int in_dim, int rows_per_head, int n_heads,
                               const float* x, float* dst) {
    if (n_heads <= 0 || rows_per_head <= 0) return;
    const Tensor& t = get(name, in_dim);
    const int out_dim = rows_per_head * n_heads;
    const size_t xb = (size_t)n_heads * in_dim * sizeof(float), yb = (size_t)out_dim * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    const size_t wsb = gpeed_iq3xxs_gemv_ws_bytes(1, in_dim, out_dim, 1);
    if (wsb == 0) throw std::runtime_error("weights: unsupported shape for " + name);
    Buffer& wbuf = ws_[std::make_tuple(in_dim, out_dim)];
    void* ws = scratch(wbuf, std::max(wsb, gpeed_iq3xxs_matvec_ws_bytes(in_dim, out_dim)), true);
    check(gpeed_memcpy(xd, x, xb, kH2D), "weights: upload x");
    check(gpeed_iq3xxs_matvec_heads(t.t64, t.n_rows, row0, in_dim, rows_per_head, n_heads,
                                    static_cast<const float*>(xd), static_cast<float*>(yd), ws, wbuf.bytes, nullptr),
          ("weights: matvec_heads " + name).c_str());
    check_ws(ws, "weights: matvec_heads " + name);
    check(gpeed_memcpy(dst, yd, yb, kD2H), "weights: download y");
}

void WeightStore::moe_experts(const std::string& gate, const std::string& up, const std::string& down, int n_exp,
                              int hidden, int inter, const float* X, int n_tok, const float* logits, int top_k,
                              int mode, const float* bias, float routed_scale, bool norm_topk, float swiglu_limit,
                              float* Y) {
    if (n_tok <= 0) return;
    const Tensor& tg = get(gate, hidden);
    const Tensor& tu = get(up, hidden);
    const Tensor& td = get(down, inter);
    const size_t n_asg = (size_t)n_tok * top_k;
    void* lg = scratch(logits_, (size_t)n_tok * n_exp * sizeof(float), false);
    void* bd = bias ? scratch(bias_, (size_t)n_exp * sizeof(float), false) : nullptr;
    void* ep = scratch(eptr_, (size_t)(n_exp + 1) * sizeof(int), false);
    void* tk = scratch(tok_, n_asg * sizeof(int), false);
    void* wt = scratch(wt_, n_asg * sizeof(float), false);
    const size_t rwsb = gpeed_moe_route_ws_bytes(n_tok, n_exp, top_k);
    const size_t mwsb = gpeed_iq3xxs_moe_ws_bytes(n_tok, n_exp, top_k, hidden, inter);
    if (rwsb == 0 || mwsb == 0) throw std::runtime_error("moe: unsupported shape");
    void* rws = scratch(route_ws_, rwsb, false);
    void* mws = scratch(moe_ws_, mwsb, true);
    const size_t xb = (size_t)n_tok * hidden * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, xb, false);
    check(gpeed_memcpy(lg, logits, (size_t)n_tok * n_exp * sizeof(float), kH2D), "moe: upload logits");
    if (bias) check(gpeed_memcpy(bd, bias, (size_t)n_exp * sizeof(float), kH2D), "moe: upload bias");
    check(gpeed_memcpy(xd, X, xb, kH2D), "moe: upload x");
    check(gpeed_moe_route(static_cast<const float*>(lg), n_tok, n_exp, top_k, mode, static_cast<const float*>(bd),
                          routed_scale, norm_topk ? 1 : 0, static_cast<int*>(ep), static_cast<int*>(tk),
                          static_cast<float*>(wt), nullptr, rws, route_ws_.bytes, nullptr),
          "moe: route");
    check(gpeed_iq3xxs_moe_experts(tg.t64, tu.t64, td.t64, n_exp, hidden, inter, static_cast<const float*>(xd),
                                   n_tok, top_k, static_cast<const int*>(ep), static_cast<const int*>(tk),
                                   static_cast<const float*>(wt), swiglu_limit, static_cast<float*>(yd), mws,
                                   moe_ws_.bytes, nullptr),
          "moe: experts");
    check_ws(mws, "moe: experts");
    check(gpeed_memcpy(Y, yd, xb, kD2H), "moe: download y");
}

}  // namespace gpu
}  // namespace glm5
