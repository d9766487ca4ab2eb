// C++ host layer over the gpeed C ABI (see glm5_gpu.h).
#include "glm5_gpu.h"

#include <algorithm>
#include <climits>
#include <cstring>
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

void dequantize(DType t, const void* src, float* dst, uint64_t n) {
    const int bs = gpeed_dtype_block_size((int)t);
    if (bs == 0) throw std::runtime_error(std::string("dequantize: unimplemented type ") + dtype_name(t));
    if (n % (uint64_t)bs) throw std::runtime_error("dequantize: element count not a multiple of block size");
    if (n == 0) return;
    check(gpeed_init(), "gpeed_init");
    const size_t in_bytes = gpeed_dtype_row_bytes((int)t, n), out_bytes = (size_t)n * sizeof(float);
    void* s = nullptr;
    void* d = nullptr;
    int rc = gpeed_malloc(&s, in_bytes);
    if (rc == GPEED_OK) rc = gpeed_malloc(&d, out_bytes);
    if (rc == GPEED_OK) rc = gpeed_memcpy(s, src, in_bytes, kH2D);
    if (rc == GPEED_OK) rc = gpeed_dequantize((int)t, s, static_cast<float*>(d), n, nullptr);
    if (rc == GPEED_OK) rc = gpeed_stream_sync(nullptr);
    if (rc == GPEED_OK) rc = gpeed_memcpy(dst, d, out_bytes, kD2H);
    (void)gpeed_free(s);
    (void)gpeed_free(d);
    check(rc, "dequantize");
}

void dequantize_row(DType t, const void* src, float* dst, uint64_t n) { dequantize(t, src, dst, n); }

WeightStore::WeightStore() { check(gpeed_init(), "gpeed_init"); }

WeightStore::WeightStore(const GgufModel& model) : WeightStore() { model_ = &model; }

void WeightStore::pin(const std::string& name) {
    if (!model_) throw std::runtime_error("weights: no GGUF model attached for " + name);
    const TensorInfo* t = model_->find_tensor(name);
    if (!t) throw std::runtime_error("weights: missing tensor " + name);
    const int bs = gpeed_dtype_block_size((int)t->type);
    if (bs == 0)
        throw std::runtime_error(std::string("weights: ") + dtype_name(t->type) + " is not decoded for " + name);
    if (t->dims.empty() || t->dims[0] > (uint64_t)INT32_MAX || t->dims[0] % (uint64_t)bs || t->dims[0] % 32)
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
    add(name, src, t->n_rows(), (int)t->dims[0], t->type);
}

size_t WeightStore::pin_matching(bool experts) {
    if (!model_) throw std::runtime_error("weights: no GGUF model attached");
    for (const std::string& name : model_->tensor_names()) {
        const bool is_expert = name.find("exps.weight") != std::string::npos;  // weights.cpp:72-73
        if (is_expert != experts || has(name)) continue;
        const TensorInfo* t = model_->find_tensor(name);
        // as weights.cpp:74-76: F32 tensors and payloads under 4 KiB stay on
        // the host; so do types the kernels do not decode
        if (!t || t->type == DType::F32 || t->n_bytes() < 4096) continue;
        const int bs = gpeed_dtype_block_size((int)t->type);
        if (bs == 0 || t->dims.empty() || t->dims[0] % (uint64_t)bs || t->dims[0] % 32) continue;
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
    const size_t raw_bytes = gpeed_dtype_row_bytes(t.dtype, (uint64_t)t.in_dim) * t.n_rows;
    if (t.dtype != GPEED_DTYPE_IQ3_XXS) {  // kept as its GGUF rows
        check(gpeed_memcpy(dst, t.data, raw_bytes, kD2H), "weights: read back");
        return;
    }
    void* raw = nullptr;
    check(gpeed_malloc(&raw, raw_bytes), "malloc");
    int rc = gpeed_iq3xxs_untile(t.data, t.n_rows, t.in_dim, raw, nullptr);
    if (rc == GPEED_OK) rc = gpeed_stream_sync(nullptr);
    if (rc == GPEED_OK) rc = gpeed_memcpy(dst, raw, raw_bytes, kD2H);
    (void)gpeed_free(raw);
    check(rc, "weights: read back");
}

WeightStore::~WeightStore() {
    for (auto& kv : tensors_) (void)gpeed_free(kv.second.data);
    for (auto& kv : ws_) (void)gpeed_free(kv.second.p);
    for (Buffer* b : {&x_, &y_, &route_ws_, &moe_ws_, &batch_ws_, &logits_, &bias_, &eptr_, &tok_, &wt_})
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
    add(name, gguf_rows, n_rows, in_dim, DType::IQ3_XXS);
}

void WeightStore::add(const std::string& name, const void* gguf_rows, uint64_t n_rows, int in_dim, DType type) {
    const int bs = gpeed_dtype_block_size((int)type);
    if (bs == 0) throw std::runtime_error(std::string("weights: ") + dtype_name(type) + " is not decoded for " + name);
    const size_t rb = gpeed_dtype_row_bytes((int)type, in_dim > 0 ? (uint64_t)in_dim : 0);
    if (rb == 0 || in_dim % 32) throw std::runtime_error("weights: row not block aligned for " + name);
    const size_t raw_bytes = rb * n_rows;
    Tensor t;
    t.n_rows = n_rows;
    t.in_dim = in_dim;
    t.dtype = (int)type;
    int rc = GPEED_OK;
    if (type == DType::IQ3_XXS) {  // kept in the T64 layout
        void* raw = nullptr;
        check(gpeed_malloc(&raw, raw_bytes), "malloc");
        t.bytes = gpeed_iq3xxs_t64_bytes(n_rows, in_dim);
        rc = gpeed_memcpy(raw, gguf_rows, raw_bytes, kH2D);
        if (rc == GPEED_OK) rc = gpeed_malloc(&t.data, t.bytes);
        if (rc == GPEED_OK) rc = gpeed_iq3xxs_tile(raw, n_rows, in_dim, t.data, nullptr);
        if (rc == GPEED_OK) rc = gpeed_stream_sync(nullptr);
        (void)gpeed_free(raw);
    } else {  // kept as its GGUF rows
        t.bytes = raw_bytes;
        rc = gpeed_malloc(&t.data, t.bytes);
        if (rc == GPEED_OK) rc = gpeed_memcpy(t.data, gguf_rows, raw_bytes, kH2D);
    }
    if (rc != GPEED_OK) {
        (void)gpeed_free(t.data);
        check(rc, "weights: upload");
    }
    auto it = tensors_.find(name);
    if (it != tensors_.end()) {
        resident_bytes_ -= it->second.bytes;
        (void)gpeed_free(it->second.data);
    }
    tensors_[name] = t;
    resident_bytes_ += t.bytes;
}

const WeightStore::Tensor& WeightStore::get(const std::string& name, int in_dim) {
    auto it = tensors_.find(name);
    if (it == tensors_.end() && model_) {
        const TensorInfo* ti = model_->find_tensor(name);
        if (!ti) throw std::runtime_error("weights: missing tensor " + name);
        const int bs = gpeed_dtype_block_size((int)ti->type);
        if (bs == 0)
            throw std::runtime_error(std::string("weights: ") + dtype_name(ti->type) + " is not decoded for " + name);
        if (in_dim % bs != 0) throw std::runtime_error("weights: row not block aligned for " + name);
        pin(name);  // first use of a tensor of the attached model
        it = tensors_.find(name);
    }
    if (it == tensors_.end()) throw std::runtime_error("weights: missing tensor " + name);
    if (in_dim % gpeed_dtype_block_size(it->second.dtype) != 0)
        throw std::runtime_error("weights: row not block aligned for " + name);
    return it->second;
}

const WeightStore::Tensor& WeightStore::get_iq3(const std::string& name, int in_dim) {
    const Tensor& t = get(name, in_dim);
    if (t.dtype != GPEED_DTYPE_IQ3_XXS) throw std::runtime_error("weights: " + name + " is not IQ3_XXS");
    return t;
}

void WeightStore::matvec_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* x,
                               float* dst) {
    if (out_dim <= 0) return;  // weights.cpp:88
    const Tensor& t = get(name, in_dim);
    if (t.dtype != GPEED_DTYPE_IQ3_XXS) {
        rows_product(t, name, row0, in_dim, out_dim, x, 1, dst);
        return;
    }
    iq3_product(t, name, row0, in_dim, out_dim, x, 1, dst, "matvec_quant");
}

void WeightStore::matmul_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* X,
                               int n_tok, float* Y) {
    if (n_tok <= 0 || out_dim <= 0) return;  // weights.cpp:88
    const Tensor& t = get(name, in_dim);
    if (t.dtype != GPEED_DTYPE_IQ3_XXS) {
        rows_product(t, name, row0, in_dim, out_dim, X, n_tok, Y);
        return;
    }
    iq3_product(t, name, row0, in_dim, out_dim, X, n_tok, Y, "matmul_quant");
}

// The T64 products start on a 64-row tile. The reference takes any row0
// (weights.cpp:86-203), so a row0 inside a tile runs the product from the
// tile's first row (at most 63 rows more) and keeps rows row0.. of the
// result: the values of those rows are the same either way.
void WeightStore::iq3_product(const Tensor& t, const std::string& name, uint64_t row0, int in_dim, int out_dim,
                              const float* X, int n_tok, float* Y, const char* who) {
    const uint64_t shift = row0 % 64;
    if (row0 > t.n_rows || (uint64_t)out_dim > t.n_rows - row0)
        throw std::runtime_error(std::string("weights: ") + who + " rows outside " + name);
    const int out_a = out_dim + (int)shift;
    const size_t xb = (size_t)n_tok * in_dim * sizeof(float), yb = (size_t)n_tok * out_a * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    const size_t wsb = gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_a, n_tok);
    if (wsb == 0) throw std::runtime_error("weights: unsupported shape for " + name);
    Buffer& wbuf = ws_[std::make_tuple(in_dim, out_a)];
    void* ws = scratch(wbuf, wsb, true);
    check(gpeed_memcpy(xd, X, xb, kH2D), "weights: upload x");
    check(gpeed_iq3xxs_matmul(t.data, t.n_rows, row0 - shift, in_dim, out_a, static_cast<const float*>(xd), n_tok,
                              static_cast<float*>(yd), ws, wbuf.bytes, nullptr),
          (std::string("weights: ") + who + " " + name).c_str());
    check_ws(ws, std::string("weights: ") + who + " " + name);
    if (shift == 0) {
        check(gpeed_memcpy(Y, yd, yb, kD2H), "weights: download y");
        return;
    }
    std::vector<float> full((size_t)n_tok * out_a);
    check(gpeed_memcpy(full.data(), yd, yb, kD2H), "weights: download y");
    for (int tk = 0; tk < n_tok; ++tk)
        std::memcpy(Y + (size_t)tk * out_dim, full.data() + (size_t)tk * out_a + shift, (size_t)out_dim * sizeof(float));
}

void WeightStore::rows_product(const Tensor& t, const std::string& name, uint64_t row0, int in_dim, int out_dim,
                               const float* X, int n_tok, float* Y) {
    const size_t xb = (size_t)n_tok * in_dim * sizeof(float), yb = (size_t)n_tok * out_dim * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    check(gpeed_memcpy(xd, X, xb, kH2D), "weights: upload x");
    check(gpeed_matmul_rows(t.dtype, t.data, t.n_rows, row0, in_dim, out_dim, static_cast<const float*>(xd), n_tok,
                            static_cast<float*>(yd), nullptr),
          ("weights: product over " + name).c_str());
    check(gpeed_memcpy(Y, yd, yb, kD2H), "weights: download y");
}

void WeightStore::matvec_heads(const std::string& name, uint64_t row0, int in_dim, int rows_per_head, int n_heads,
                               const float* x, float* dst) {
    if (n_heads <= 0 || rows_per_head <= 0) return;
    const Tensor& t = get_iq3(name, in_dim);
    const int out_dim = rows_per_head * n_heads;
    const size_t xb = (size_t)n_heads * in_dim * sizeof(float), yb = (size_t)out_dim * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, yb, false);
    const size_t wsb = gpeed_iq3xxs_gemv_ws_bytes(1, in_dim, out_dim, 1);
    if (wsb == 0) throw std::runtime_error("weights: unsupported shape for " + name);
    Buffer& wbuf = ws_[std::make_tuple(in_dim, out_dim)];
    void* ws = scratch(wbuf, std::max(wsb, gpeed_iq3xxs_matvec_ws_bytes(in_dim, out_dim)), true);
    check(gpeed_memcpy(xd, x, xb, kH2D), "weights: upload x");
    check(gpeed_iq3xxs_matvec_heads(t.data, t.n_rows, row0, in_dim, rows_per_head, n_heads,
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
    const Tensor& tg = get_iq3(gate, hidden);
    const Tensor& tu = get_iq3(up, hidden);
    const Tensor& td = get_iq3(down, inter);
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
    check(gpeed_iq3xxs_moe_experts(tg.data, tu.data, td.data, n_exp, hidden, inter, static_cast<const float*>(xd),
                                   n_tok, top_k, static_cast<const int*>(ep), static_cast<const int*>(tk),
                                   static_cast<const float*>(wt), swiglu_limit, static_cast<float*>(yd), mws,
                                   moe_ws_.bytes, nullptr),
          "moe: experts");
    check_ws(mws, "moe: experts");
    check(gpeed_memcpy(Y, yd, xb, kD2H), "moe: download y");
}

void WeightStore::moe_batch(const std::string& router, const std::string& gate, const std::string& up,
                            const std::string& down, const std::string& gate_sh, const std::string& up_sh,
                            const std::string& down_sh, int n_exp, int hidden, int inter, const float* X, int n_tok,
                            int top_k, int mode, const float* bias, float routed_scale, bool norm_topk,
                            float swiglu_limit, float* Y) {
    if (n_tok <= 0) return;
    const Tensor& tr = get(router, hidden);
    if (tr.dtype != GPEED_DTYPE_F32) throw std::runtime_error("moe: router " + router + " is not F32");
    const size_t xb = (size_t)n_tok * hidden * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* lg = scratch(logits_, (size_t)n_tok * n_exp * sizeof(float), false);
    check(gpeed_memcpy(xd, X, xb, kH2D), "moe: upload x");
    check(gpeed_matmul_rows(tr.dtype, tr.data, tr.n_rows, 0, hidden, n_exp, static_cast<const float*>(xd), n_tok,
                            static_cast<float*>(lg), nullptr),
          ("moe: router product " + router).c_str());
    moe_batch_dev(gate, up, down, gate_sh, up_sh, down_sh, n_exp, hidden, inter, n_tok, top_k, mode, bias,
                  routed_scale, norm_topk, swiglu_limit, Y);
}

void WeightStore::moe_batch(const std::string& gate, const std::string& up, const std::string& down,
                            const std::string& gate_sh, const std::string& up_sh, const std::string& down_sh,
                            int n_exp, int hidden, int inter, const float* X, int n_tok, const float* logits,
                            int top_k, int mode, const float* bias, float routed_scale, bool norm_topk,
                            float swiglu_limit, float* Y) {
    if (n_tok <= 0) return;
    const size_t xb = (size_t)n_tok * hidden * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* lg = scratch(logits_, (size_t)n_tok * n_exp * sizeof(float), false);
    check(gpeed_memcpy(lg, logits, (size_t)n_tok * n_exp * sizeof(float), kH2D), "moe: upload logits");
    check(gpeed_memcpy(xd, X, xb, kH2D), "moe: upload x");
    moe_batch_dev(gate, up, down, gate_sh, up_sh, down_sh, n_exp, hidden, inter, n_tok, top_k, mode, bias,
                  routed_scale, norm_topk, swiglu_limit, Y);
}

void WeightStore::dense_mlp(const std::string& gate, const std::string& up, const std::string& down, int hidden,
                            int inter, const float* X, int n_tok, float swiglu_limit, float* Y) {
    if (n_tok <= 0) return;
    const Tensor& tg = get_iq3(gate, hidden);
    const Tensor& tu = get_iq3(up, hidden);
    const Tensor& td = get_iq3(down, inter);
    if (tg.n_rows < (uint64_t)inter || tu.n_rows < (uint64_t)inter || td.n_rows < (uint64_t)hidden)
        throw std::runtime_error("dense_mlp: tensor rows fewer than the shape");
    const size_t xb = (size_t)n_tok * hidden * sizeof(float);
    void* xd = scratch(x_, xb, false);
    void* yd = scratch(y_, xb, false);
    check(gpeed_memcpy(xd, X, xb, kH2D), "dense_mlp: upload x");
    void* ws = nullptr;
    if (n_tok == 1) {
        const size_t wsb = gpeed_iq3xxs_dense_mlp_ws_bytes(hidden, inter);
        if (wsb == 0) throw std::runtime_error("dense_mlp: unsupported shape");
        ws = scratch(mlp_ws_, wsb, true);
        check(gpeed_iq3xxs_dense_mlp(tg.data, tu.data, td.data, hidden, inter, static_cast<const float*>(xd),
                                     swiglu_limit, static_cast<float*>(yd), ws, mlp_ws_.bytes, nullptr),
              "dense_mlp");
    } else {
        const size_t wsb = gpeed_iq3xxs_mlp_gemm_ws_bytes(n_tok, hidden, inter, GPEED_X_F32, 0, nullptr);
        if (wsb == 0) throw std::runtime_error("dense_mlp: unsupported shape");
        ws = scratch(mlp_ws_, wsb, true);
        check(gpeed_iq3xxs_mlp_gemm(tg.data, tu.data, td.data, hidden, inter, xd, GPEED_X_F32, n_tok, swiglu_limit,
                                    static_cast<float*>(yd), 0, nullptr, nullptr, nullptr, ws, mlp_ws_.bytes,
                                    nullptr),
              "dense_mlp");
    }
    check_ws(ws, "dense_mlp");
    check(gpeed_memcpy(Y, yd, xb, kD2H), "dense_mlp: download y");
}

// The routed step from the logits and X already in the logits_ / x_
// buffers; Y to the host.
void WeightStore::moe_batch_dev(const std::string& gate, const std::string& up, const std::string& down,
                                const std::string& gate_sh, const std::string& up_sh, const std::string& down_sh,
                                int n_exp, int hidden, int inter, int n_tok, int top_k, int mode, const float* bias,
                                float routed_scale, bool norm_topk, float swiglu_limit, float* Y) {
    const Tensor& tg = get_iq3(gate, hidden);
    const Tensor& tu = get_iq3(up, hidden);
    const Tensor& td = get_iq3(down, inter);
    const bool shared = !gate_sh.empty();
    const void* sg = shared ? get_iq3(gate_sh, hidden).data : nullptr;
    const void* su = shared ? get_iq3(up_sh, hidden).data : nullptr;
    const void* sd = shared ? get_iq3(down_sh, inter).data : nullptr;
    const size_t wsb = gpeed_iq3xxs_moe_batch_ws_bytes(n_tok, n_exp, top_k, hidden, inter, shared ? 1 : 0);
    if (wsb == 0) throw std::runtime_error("moe: unsupported shape");
    void* ws = scratch(batch_ws_, wsb, true);
    void* lg = logits_.p;
    void* bd = bias ? scratch(bias_, (size_t)n_exp * sizeof(float), false) : nullptr;
    const size_t xb = (size_t)n_tok * hidden * sizeof(float);
    void* xd = x_.p;
    void* yd = scratch(y_, xb, false);
    if (bias) check(gpeed_memcpy(bd, bias, (size_t)n_exp * sizeof(float), kH2D), "moe: upload bias");
    check(gpeed_iq3xxs_moe_batch(static_cast<const float*>(lg), n_tok, n_exp, top_k, mode,
                                 static_cast<const float*>(bd), routed_scale, norm_topk ? 1 : 0, tg.data, tu.data,
                                 td.data, sg, su, sd, hidden, inter, static_cast<const float*>(xd), swiglu_limit,
                                 static_cast<float*>(yd), nullptr, nullptr, nullptr, ws, batch_ws_.bytes, nullptr),
          "moe: batch");
    check_ws(ws, "moe: batch");
    check(gpeed_memcpy(Y, yd, xb, kD2H), "moe: download y");
}

}  // namespace gpu
}  // namespace glm5
