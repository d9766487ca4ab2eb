/* CPU oracle for the IQ3_XXS dequantize-and-multiply path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * CPU algorithm, used as the correctness reference by tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py. Nothing in
 * the product (gpeed_amd/) links,
 * imports or calls it, and no product path falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root). How each function is pinned:
 *   orc_f16_to_f32       all 65,536 fp16 patterns vs numpy's float16 widening
 *   orc_sign_byte        all 128 entries vs the reference table (text) and the
 *                        even-parity closed form
 *   orc_iq3xxs_block     golden block fixtures, brute force over every
 *                        (grid, sign, scale) combination vs a closed form,
 *                        and bitwise vs oracle/_ref (the reference compiled
 *                        from source) when that library is built
 *   orc_dot_f32          bitwise vs oracle/_ref, and vs an fp64 dot within the
 *                        fp32 error bound
 *   orc_matvec/matmul    bitwise vs oracle/_ref's WeightStore::matvec_quant /
 *                        matmul_quant, and vs fp64 dense products
 *   orc_moe_route        brute-force re-derivation of top-k + integer
 *                        invariants of the stable bucket sort
 *   orc_moe_experts      vs an fp64 dense restatement of each expert FFN
 *   orc_moe_forward      one token, rank-order combine: vs an fp64
 *                        restatement, and vs orc_moe_batch at one token
 *   orc_moe_batch        route + experts + the shared expert: vs an fp64
 *                        dense restatement of the whole step (every expert
 *                        and the shared FFN)
 *   orc_dequant_block    (Q8_0, Q2_K, Q3_K, Q6_K, IQ2_S, IQ3_S, IQ4_XS)
 *                        bitwise vs oracle/_ref over random blocks and blocks
 *                        of special values, codebooks vs the reference
 *                        header, closed forms for single-code blocks
 *   orc_matmul_rows      bitwise vs oracle/_ref's WeightStore::matvec_quant /
 *                        matmul_quant on tensors of each type
 */
#ifndef GPEED_IQ3_ORACLE_H
#define GPEED_IQ3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type id of IQ3_XXS (common.h:27) and its geometry (quant.cpp:69,108). */
#define ORC_DTYPE_F32 0
#define ORC_DTYPE_F16 1
#define ORC_DTYPE_Q8_0 8
#define ORC_DTYPE_Q2_K 10
#define ORC_DTYPE_Q3_K 11
#define ORC_DTYPE_Q6_K 14
#define ORC_DTYPE_IQ3_XXS 18
#define ORC_DTYPE_IQ3_S 21
#define ORC_DTYPE_IQ2_S 22
#define ORC_DTYPE_IQ4_XS 23
#define ORC_DTYPE_BF16 30
#define ORC_QK_K 256
#define ORC_IQ3XXS_BLOCK_BYTES 98

#define ORC_OK 0
#define ORC_ERR_NOT_MULTIPLE (-1) /* quant.cpp:523-524 */
#define ORC_ERR_UNIMPLEMENTED (-2) /* quant.cpp:553-554 */
#define ORC_ERR_UNALIGNED_ROW (-3) /* weights.cpp:93-94 */

size_t orc_iq3xxs_row_bytes(uint64_t n_elements);

/* quant_oracle.c: the other block formats (quant.cpp:165-502) */
int orc_block_elems(int dtype);
int orc_block_bytes(int dtype);
size_t orc_row_bytes(int dtype, uint64_t n);
int orc_dequant_block(int dtype, const uint8_t* blk, float* y);
uint64_t orc_iq2s_grid(uint32_t i);
uint32_t orc_iq3s_grid(uint32_t i);
int orc_iq4nl_value(int i);
int orc_matmul_rows(int dtype, const uint8_t* w, uint64_t row0, int in_dim, int out_dim, const float* X,
                    int n_tok, float* Y, float* row_buf);
float orc_f16_to_f32(uint16_t h);
uint8_t orc_sign_byte(unsigned idx7);
uint32_t orc_grid_entry(unsigned idx);
void orc_iq3xxs_block(const uint8_t* blk, float* y);
int orc_dequantize(int dtype, const void* src, float* dst, uint64_t n);
float orc_dot_f32(const float* a, const float* b, int n);
void orc_axpy_f32(float* a, const float* b, float s, int n);

int orc_matvec_quant(const uint8_t* w, uint64_t row0, int in_dim, int out_dim,
                     const float* x, float* dst);
int orc_matmul_quant(const uint8_t* w, uint64_t row0, int in_dim, int out_dim,
                     const float* X, int n_tok, float* Y);

/* mode 0: the reference router (sigmoid + bias, top-k by choice, weights
 * score/sum*routed_scale). mode 1: softmax over the logits, renormalised over
 * the selected top-k. */
int orc_moe_route(const float* logits, int n_tok, int n_exp, int top_k, int mode,
                  const float* bias, float routed_scale, int norm_topk,
                  int* eptr, int* tok, float* wt, int* sel);
int orc_moe_experts(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                    int hidden, int inter, const float* X, int n_tok, int n_exp,
                    const int* eptr, const int* tok, const float* wt,
                    float swiglu_limit, float* Y);
int orc_dense_mlp(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                  int hidden, int inter, const float* X, int n_tok, float swiglu_limit,
                  float* Y);
int orc_moe_forward(const float* logits, int n_exp, int top_k, const float* bias, float routed_scale,
                    int norm_topk, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                    const uint8_t* w_gate_sh, const uint8_t* w_up_sh, const uint8_t* w_down_sh, int hidden,
                    int inter, const float* x, float swiglu_limit, float* y);
int orc_moe_batch(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                  float routed_scale, int norm_topk, const uint8_t* w_gate, const uint8_t* w_up,
                  const uint8_t* w_down, const uint8_t* w_gate_sh, const uint8_t* w_up_sh,
                  const uint8_t* w_down_sh, int hidden, int inter, const float* X, float swiglu_limit, float* Y);

#ifdef __cplusplus
}
#endif
#endif
