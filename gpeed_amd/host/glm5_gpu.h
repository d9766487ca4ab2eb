// C++ host layer over the gpeed C ABI, with the reference's call signatures.
//
// * glm5::cuda_device_count / cuda_device_name / cuda_add keep the kernel
//   slot of cpp/kernels/include/glm5/kernels.h:7-11 (device_info.cu) and run
//   on the HIP device.
// * glm5::gpu::WeightStore keeps WeightStore::matvec_quant / matmul_quant
//   (cpp/core/include/glm5/weights.h:41-48, weights.cpp:86-203): same
//   arguments, host fp32 arrays in and out, synchronous, the same
//   std::runtime_error messages ("weights: missing tensor <name>",
//   "weights: row not block aligned for <name>"). Tensors are uploaded once
//   (add) and kept in HBM in the T64 layout.
// * WeightStore::moe_experts runs steps 1-3 of Model::moe_batch
//   (model_batch.cpp:165-262) from the router logits on the device.
//
// No HIP header is needed by users of this file; it links against
// libgpeed_iq3.so (include/gpeed_iq3.h).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <map>
#include <tuple>
#include <unordered_map>

#include "gguf.h"

namespace glm5 {

int cuda_device_count();
std::string cuda_device_name(int index);
// dst[i] = a[i] + b[i] over host arrays, computed on the device.
void cuda_add(const float* a, const float* b, float* dst, int n);

namespace gpu {

// dequantize / dequantize_row (quant.h:18-22) over host arrays, computed on
// the device: n weights of type t at src into dst, bit-exact with the
// reference, for F32, F16, BF16, Q8_0, Q2_K, Q3_K, Q6_K, IQ3_XXS, IQ3_S,
// IQ2_S and IQ4_XS. Throws the reference's messages ("dequantize:
// unimplemented type <name>", "dequantize: element count not a multiple of
// block size").
void dequantize(DType t, const void* src, float* dst, uint64_t n);
void dequantize_row(DType t, const void* src, float* dst, uint64_t n);

class WeightStore {
public:
    WeightStore();
    // A store that takes its tensors from a parsed GGUF model (the reference's
    // WeightStore(const GgufModel&), weights.cpp:10-11). pin_nonexpert /
    // pin_experts upload them; a product on an IQ3_XXS tensor not yet
    // resident uploads it first (where the reference would stream it from the
    // file, weights.cpp:94-107). The model must outlive the store.
    explicit WeightStore(const GgufModel& model);
    ~WeightStore();
    WeightStore(const WeightStore&) = delete;
    WeightStore& operator=(const WeightStore&) = delete;

    // Uploads n_rows GGUF IQ3_XXS rows of in_dim weights (host bytes) and
    // keeps their T64 copy in HBM (the role of pin_nonexpert,
    // weights.cpp:70-84). Replaces a tensor of the same name.
    void add(const std::string& name, const void* gguf_rows, uint64_t n_rows, int in_dim);
    // The same for a tensor of another decoded type, kept in HBM as its GGUF
    // rows (in_dim a multiple of the block size and of 32).
    void add(const std::string& name, const void* gguf_rows, uint64_t n_rows, int in_dim, DType type);
    bool has(const std::string& name) const { return tensors_.count(name) != 0; }
    size_t resident_bytes() const { return resident_bytes_; }

    // pin_nonexpert (weights.cpp:70-84) on the device: every tensor of the
    // attached model except the routed experts (names containing
    // "exps.weight"), F32 tensors and payloads under 4 KiB, as the
    // reference, uploaded once and kept in HBM (IQ3_XXS in the T64 layout,
    // the other decoded types as GGUF rows). Returns the bytes held in HBM.
    size_t pin_nonexpert();
    // The routed-expert tensors as well (the reference keeps them on disk; the
    // whole model fits in 288 GB of HBM). Returns the bytes held in HBM.
    size_t pin_experts();
    // Uploads one tensor of a decoded type of the attached model (rows =
    // n_elements / dims[0], so a 3-D expert tensor is
    // [n_exp * rows_per_expert, in_dim]).
    void pin(const std::string& name);
    // The GGUF bytes of a resident tensor, read back from its HBM copy
    // (n_rows * row_bytes into host memory at dst).
    void read_resident(const std::string& name, void* dst) const;

    // dst[j] = sum_i W[row0+j][i] * x[i], j < out_dim (weights.cpp:167-203):
    // one GEMV launch (IQ3_XXS), or the raw-row product for another type.
    void matvec_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* x,
                      float* dst);
    // Y[t][j] = sum_i W[row0+j][i] * X[t][i], t < n_tok (weights.cpp:86-165):
    // 8-token GEMV passes for decode-sized batches, the prefill GEMM (one
    // pass over W) from gpeed_iq3xxs_matmul_gemm_min_tok() tokens on.
    void matmul_quant(const std::string& name, uint64_t row0, int in_dim, int out_dim, const float* X,
                      int n_tok, float* Y);

    // The per-head absorbed projections of MLA attention (model.cpp:638-643,
    // 664-665) as one launch: for h < n_heads, dst[h*rows_per_head ..] =
    // rows row0 + h*rows_per_head .. of the tensor times x[h*in_dim ..]; the
    // same as n_heads matvec_quant calls. rows_per_head, row0 multiples of 64.
    void matvec_heads(const std::string& name, uint64_t row0, int in_dim, int rows_per_head, int n_heads,
                      const float* x, float* dst);

    // Model::dense_mlp (model.cpp:677-690; one token) and dense_mlp_batch
    // (model_batch.cpp:145-163; n_tok tokens) on the device: Y [n_tok][hidden]
    // = down(SwiGLU(gate X, up X)) with the reference's clamp (min(g, lim),
    // clamp(u, -lim, lim)), X [n_tok][hidden] and Y host arrays. gate / up
    // [inter][hidden] and down [hidden][inter] are IQ3_XXS tensors of the
    // store. One token: the two-launch dense GEMV (gpeed_iq3xxs_dense_mlp);
    // more: gpeed_iq3xxs_mlp_gemm.
    void dense_mlp(const std::string& gate, const std::string& up, const std::string& down, int hidden, int inter,
                   const float* X, int n_tok, float swiglu_limit, float* Y);

    // Model::moe_batch steps 1-3: router top_k over logits [n_tok][n_exp]
    // (mode 0: sigmoid + bias with routed_scale / norm_topk as the reference;
    // mode 1: softmax over the top_k), expert buckets, per-expert gate/up
    // (rows e*inter of gate/up), SwiGLU(limit), down (rows e*hidden), and
    // Y[t] = sum of the weighted expert outputs (overwritten).
    void moe_experts(const std::string& gate, const std::string& up, const std::string& down, int n_exp,
                     int hidden, int inter, const float* X, int n_tok, const float* logits, int top_k, int mode,
                     const float* bias, float routed_scale, bool norm_topk, float swiglu_limit, float* Y);
    // The whole of Model::moe_batch after the router product
    // (model_batch.cpp:174-280): moe_experts, plus, when gate_sh is not
    // empty, the shared expert (gate_sh / up_sh [inter, hidden], down_sh
    // [hidden, inter]) over every token added last, as add_f32 does. One
    // call of gpeed_iq3xxs_moe_batch (five launches).
    void moe_batch(const std::string& gate, const std::string& up, const std::string& down,
                   const std::string& gate_sh, const std::string& up_sh, const std::string& down_sh, int n_exp,
                   int hidden, int inter, const float* X, int n_tok, const float* logits, int top_k, int mode,
                   const float* bias, float routed_scale, bool norm_topk, float swiglu_limit, float* Y);
    // The whole of Model::moe_batch (model_batch.cpp:165-281) with step 1 on
    // the device too: the router product matmul_quant(router) (ffn_gate_inp,
    // model_batch.cpp:172; an F32 [n_exp, hidden] tensor of the store) of X,
    // whose logits are bitwise the reference's (dot_f32's own order), then
    // the routed step as the overload above. X goes up and Y comes down once.
    void moe_batch(const std::string& router, const std::string& gate, const std::string& up,
                   const std::string& down, const std::string& gate_sh, const std::string& up_sh,
                   const std::string& down_sh, int n_exp, int hidden, int inter, const float* X, int n_tok,
                   int top_k, int mode, const float* bias, float routed_scale, bool norm_topk, float swiglu_limit,
                   float* Y);

private:
    struct Tensor {
        void* data = nullptr;  // T64 copy (IQ3_XXS) or GGUF rows
        uint64_t n_rows = 0;
        int in_dim = 0;
        int dtype = 18;
        size_t bytes = 0;
    };
    struct Buffer {
        void* p = nullptr;
        size_t bytes = 0;
    };
    const Tensor& get(const std::string& name, int in_dim);
    const Tensor& get_iq3(const std::string& name, int in_dim);
    void moe_batch_dev(const std::string& gate, const std::string& up, const std::string& down,
                       const std::string& gate_sh, const std::string& up_sh, const std::string& down_sh, int n_exp,
                       int hidden, int inter, int n_tok, int top_k, int mode, const float* bias, float routed_scale,
                       bool norm_topk, float swiglu_limit, float* Y);
    void iq3_product(const Tensor& t, const std::string& name, uint64_t row0, int in_dim, int out_dim,
                     const float* X, int n_tok, float* Y, const char* who);
    void rows_product(const Tensor& t, const std::string& name, uint64_t row0, int in_dim, int out_dim,
                      const float* X, int n_tok, float* Y);
    void* scratch(Buffer& b, size_t bytes, bool init);
    // throws if a kernel flagged the workspace (waits for the stream)
    static void check_ws(void* ws, const std::string& what);

    size_t pin_matching(bool experts);

    const GgufModel* model_ = nullptr;
    std::unordered_map<std::string, Tensor> tensors_;
    size_t resident_bytes_ = 0;
    // One matvec / matmul workspace per (in_dim, out_dim), initialised when
    // it is made and grown when a call needs more; each launch leaves its
    // tickets at zero, and one sized for n_tok serves every smaller call.
    std::map<std::tuple<int, int>, Buffer> ws_;
    Buffer x_, y_, route_ws_, moe_ws_, batch_ws_, logits_, bias_, eptr_, tok_, wt_, mlp_ws_;
};

}  // namespace gpu
}  // namespace glm5
