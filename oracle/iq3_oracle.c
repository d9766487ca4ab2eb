/* CPU oracle for the IQ3_XXS dequantize-and-multiply path.
 *
 * TEST INFRASTRUCTURE ONLY: the correctness reference for tests/, smoke() and bench.py's
 * cpu_baseline leg. The product never links or calls this file.
 *
 * Build with -ffp-contract=off and spell every fused multiply-add as fmaf():
 * the reference is C++ built with -mfma (CMakeLists.txt:44-46), and GCC
 * contracts a*b+c into an FMA by default for C++ even under -std=c++20, so
 * the scalar tails of dot_f32 / axpy_f32 (simd.h:30, 48) are fused there as
 * well as the explicit _mm256_fmadd_ps steps. Products without an add
 * (blk_iq3_xxs) are unaffected.
 */
#include "iq3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "iq3xxs_grid.h"

/* quant.cpp:119-126 (dtype_row_bytes for a 256-element, 98-byte block type). */
size_t orc_iq3xxs_row_bytes(uint64_t n) {
    if (n % ORC_QK_K) return 0;
    return (size_t)(n / ORC_QK_K) * ORC_IQ3XXS_BLOCK_BYTES;
}

/* quant.cpp:130-154: software fp16 -> fp32 with subnormals, inf and NaN
 * (NaN payload kept as man << 13). */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* normalise: shift the mantissa until the implicit bit appears */
            uint32_t e = 113; /* 127 - 15 + 1 */
            while (!(man & 0x400u)) {
                man <<= 1;
                --e;
            }
            bits = sign | (e << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (ex == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* iq3xxs_tables.h:61 (kSignsIq2xs): the 7 stored sign bits plus an eighth
 * bit that makes the byte's parity even. */
uint8_t orc_sign_byte(unsigned idx7) {
    unsigned v = idx7 & 127u, p = 0;
    for (unsigned t = v; t; t >>= 1) p ^= t & 1u;
    return (uint8_t)(v | (p << 7));
}

uint32_t orc_grid_entry(unsigned idx) { return oracle_iq3xxs_grid[idx & 255u]; }

static uint32_t rd_u32le(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}

/* quant.cpp:186-210 (blk_iq3_xxs). Layout of the 98-byte block:
 * [0,2) fp16 d; [2,66) qs[64] grid indices; [66,98) 8 LE u32 words, one per
 * 32-weight sub-block: bits 28..31 scale s, bits 7l..7l+6 sign index of
 * 8-weight group l. y[32ib+8l+j] = (d*(0.5+s)*0.5 * grid_j) * (+/-1). */
void orc_iq3xxs_block(const uint8_t* blk, float* y) {
    const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const uint8_t* qs = blk + 2;
    const uint8_t* ss = blk + 66;
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t aux = rd_u32le(ss + 4 * ib);
        const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; ++l) {
            const uint8_t sg = orc_sign_byte((aux >> (7 * l)) & 127u);
            const uint32_t g1 = oracle_iq3xxs_grid[qs[2 * l + 0]];
            const uint32_t g2 = oracle_iq3xxs_grid[qs[2 * l + 1]];
            for (int j = 0; j < 4; ++j) {
                y[j + 0] = db * (float)((g1 >> (8 * j)) & 255u) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
                y[j + 4] =
                    db * (float)((g2 >> (8 * j)) & 255u) * (((sg >> (j + 4)) & 1u) ? -1.0f : 1.0f);
            }
            y += 8;
        }
        qs += 8;
    }
}

/* quant.cpp:521-573 (dequantize_impl): F32, F16, BF16 and every block format
 * the reference decodes (quant.cpp:507-519). */
int orc_dequantize(int dtype, const void* src, float* dst, uint64_t n) {
    const uint8_t* p = (const uint8_t*)src;
    switch (dtype) {
        case ORC_DTYPE_F32:
            memcpy(dst, src, (size_t)n * 4);
            return ORC_OK;
        case ORC_DTYPE_F16:
            for (uint64_t i = 0; i < n; ++i)
                dst[i] = orc_f16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
            return ORC_OK;
        case ORC_DTYPE_BF16:
            for (uint64_t i = 0; i < n; ++i) {
                const uint32_t bits = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
                memcpy(dst + i, &bits, 4);
            }
            return ORC_OK;
        default: {
            /* quant.cpp:546-563: one block function per type over n / block */
            const int be = orc_block_elems(dtype), bb = orc_block_bytes(dtype);
            if (be <= 1) return ORC_ERR_UNIMPLEMENTED;
            if (n % (uint64_t)be) return ORC_ERR_NOT_MULTIPLE;
            for (uint64_t b = 0; b < n / (uint64_t)be; ++b) {
                const int rc = orc_dequant_block(dtype, p + b * (uint64_t)bb, dst + b * (uint64_t)be);
                if (rc) return rc;
            }
            return ORC_OK;
        }
    }
}

/* simd.h:12-37 (dot_f32, AVX2 path) in scalar form, same order: two 8-lane
 * FMA accumulators over 16-element strides (lanes i%16<8 -> a0, else a1), an
 * 8-element FMA step into a0, then (a0+a1), lo128+hi128, two horizontal adds,
 * and a fused multiply-add tail. */
float orc_dot_f32(const float* a, const float* b, int n) {
    float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        for (int l = 0; l < 8; ++l) {
            a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
            a1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
        }
    }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
    float s[8], lo[4];
    for (int l = 0; l < 8; ++l) s[l] = a0[l] + a1[l];
    for (int l = 0; l < 4; ++l) lo[l] = s[l] + s[l + 4];
    const float h0 = lo[0] + lo[1];
    const float h1 = lo[2] + lo[3];
    float acc = h0 + h1;
    for (; i < n; ++i) acc = fmaf(a[i], b[i], acc);
    return acc;
}

/* simd.h:40-50 (axpy_f32): a[i] = fma(s, b[i], a[i]) over 8-wide steps and
 * (contracted) over the tail. */
void orc_axpy_f32(float* a, const float* b, float s, int n) {
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) a[i + l] = fmaf(s, b[i + l], a[i + l]);
    for (; i < n; ++i) a[i] = fmaf(s, b[i], a[i]);
}

/* weights.cpp:167-203 (matvec_quant): for each output row j, dequantize row
 * row0+j of the payload and dot it with x. Single-threaded: the reference's
 * Linux build has no OpenMP (cpp/CMakeLists.txt:18-26), and the per-row
 * result does not depend on the thread count. */
int orc_matvec_quant(const uint8_t* w, uint64_t row0, int in_dim, int out_dim, const float* x,
                     float* dst) {
    if (in_dim % ORC_QK_K) return ORC_ERR_UNALIGNED_ROW;
    const size_t rb = orc_iq3xxs_row_bytes((uint64_t)in_dim);
    float* row = (float*)malloc(sizeof(float) * (size_t)in_dim);
    if (!row) return ORC_ERR_UNIMPLEMENTED;
    const uint8_t* src = w + row0 * rb;
    for (int j = 0; j < out_dim; ++j) {
        orc_dequantize(ORC_DTYPE_IQ3_XXS, src + rb * (size_t)j, row, (uint64_t)in_dim);
        dst[j] = orc_dot_f32(row, x, in_dim);
    }
    free(row);
    return ORC_OK;
}

/* weights.cpp:86-165 (matmul_quant). Both of its regimes (row-parallel for
 * X <= 16 MiB, 64-row blocked otherwise) compute
 * Y[t][j] = dot_f32(deq(W[row0+j]), X[t]); each row is dequantized once. */
int orc_matmul_quant(const uint8_t* w, uint64_t row0, int in_dim, int out_dim, const float* X,
                     int n_tok, float* Y) {
    if (n_tok <= 0 || out_dim <= 0) return ORC_OK; /* weights.cpp:88 */
    if (in_dim % ORC_QK_K) return ORC_ERR_UNALIGNED_ROW;
    const size_t rb = orc_iq3xxs_row_bytes((uint64_t)in_dim);
    float* row = (float*)malloc(sizeof(float) * (size_t)in_dim);
    if (!row) return ORC_ERR_UNIMPLEMENTED;
    const uint8_t* src = w + row0 * rb;
    for (int j = 0; j < out_dim; ++j) {
        orc_dequantize(ORC_DTYPE_IQ3_XXS, src + rb * (size_t)j, row, (uint64_t)in_dim);
        for (int t = 0; t < n_tok; ++t)
            Y[(size_t)t * out_dim + j] = orc_dot_f32(row, X + (size_t)t * in_dim, in_dim);
    }
    free(row);
    return ORC_OK;
}

/* model_batch.cpp:245-253 / model.cpp:683-688: silu(min(g,lim)) * clamp(u,-lim,lim)
 * with silu(x) = x / (1 + exp(-x)) (ops.h:17). std::min(g, lim) is
 * `lim < g ? lim : g` and std::clamp(u, lo, hi) is `u < lo ? lo : (hi < u ?
 * hi : u)`: a NaN g or u passes through both. */
static float swiglu1(float g, float u, float lim) {
    const float gi = lim < g ? lim : g;
    const float ui = u < -lim ? -lim : (lim < u ? lim : u);
    return (gi / (1.0f + expf(-gi))) * ui;
}

/* Rank test for top-k: a precedes b when its key is larger; equal keys keep
 * the lower expert id first. */
static int before(float ka, int a, float kb, int b) { return ka > kb || (ka == kb && a < b); }

/* model_batch.cpp:178-219 (moe_batch steps 1-2): per-token top-k, then a
 * stable bucket sort of the (token, k) assignments by expert.
 * mode 0 restates the reference router (model_batch.cpp:186-203):
 *   score = sigmoid(logit), choice = score + bias, top-k by choice,
 *   denom = 1e-20 + sum of the top-k scores (in rank order),
 *   w = score * (norm_topk ? routed_scale/denom : routed_scale).
 * mode 1 is softmax routing: top-k by logit, w = exp(l - lmax_topk) normalised
 * over the top-k (summed in rank order). */
int orc_moe_route(const float* logits, int n_tok, int n_exp, int top_k, int mode,
                  const float* bias, float routed_scale, int norm_topk, int* eptr, int* tok,
                  float* wt, int* sel) {
    if (top_k <= 0 || top_k > n_exp || n_exp > 1024) return ORC_ERR_UNIMPLEMENTED;
    float key[1024], score[1024];
    int idx[1024];
    int* cnt = (int*)calloc((size_t)n_exp, sizeof(int));
    int* asg_e = (int*)malloc(sizeof(int) * (size_t)n_tok * top_k + 1);
    float* asg_w = (float*)malloc(sizeof(float) * (size_t)n_tok * top_k + 1);
    for (int t = 0; t < n_tok; ++t) {
        const float* lg = logits + (size_t)t * n_exp;
        for (int e = 0; e < n_exp; ++e) {
            if (mode == 0) {
                score[e] = 1.0f / (1.0f + expf(-lg[e]));
                key[e] = score[e] + (bias ? bias[e] : 0.0f);
            } else {
                score[e] = lg[e];
                key[e] = lg[e];
            }
        }
        /* selection of the top_k largest keys, in rank order */
        for (int k = 0; k < top_k; ++k) {
            int best = -1;
            for (int e = 0; e < n_exp; ++e) {
                int taken = 0;
                for (int q = 0; q < k; ++q) taken |= idx[q] == e;
                if (taken) continue;
                if (best < 0 || before(key[e], e, key[best], best)) best = e;
            }
            idx[k] = best;
        }
        float w[1024];
        if (mode == 0) {
            float denom = 1e-20f;
            for (int k = 0; k < top_k; ++k) denom += score[idx[k]];
            const float inv = norm_topk ? routed_scale / denom : routed_scale;
            for (int k = 0; k < top_k; ++k) w[k] = score[idx[k]] * inv;
        } else {
            const float lmax = score[idx[0]];
            float denom = 0.0f;
            for (int k = 0; k < top_k; ++k) {
                w[k] = expf(score[idx[k]] - lmax);
                denom += w[k];
            }
            for (int k = 0; k < top_k; ++k) w[k] = w[k] / denom;
        }
        for (int k = 0; k < top_k; ++k) {
            asg_e[(size_t)t * top_k + k] = idx[k];
            asg_w[(size_t)t * top_k + k] = w[k];
            if (sel) sel[(size_t)t * top_k + k] = idx[k];
            ++cnt[idx[k]];
        }
    }
    int acc = 0;
    for (int e = 0; e < n_exp; ++e) {
        eptr[e] = acc;
        acc += cnt[e];
    }
    eptr[n_exp] = acc;
    /* stable bucket sort (model_batch.cpp:211-219): assignments in (token, k)
     * order are appended to their expert's bucket */
    for (int e = 0; e < n_exp; ++e) cnt[e] = eptr[e];
    for (int a = 0; a < n_tok * top_k; ++a) {
        const int e = asg_e[a];
        const int p = cnt[e]++;
        tok[p] = a / top_k;
        wt[p] = asg_w[a];
    }
    free(cnt);
    free(asg_e);
    free(asg_w);
    return ORC_OK;
}

/* model_batch.cpp:221-262 (moe_batch step 3): for every expert with tokens,
 * gather its rows of X, gate/up = matmul_quant at row0 = e*inter, SwiGLU
 * clamp, down = matmul_quant at row0 = e*hidden, then Y[t] += w * down in
 * expert-then-bucket order (axpy_f32). Y is overwritten (zeroed first). */
int orc_moe_experts(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int hidden,
                    int inter, const float* X, int n_tok, int n_exp, const int* eptr, const int* tok,
                    const float* wt, float swiglu_limit, float* Y) {
    const int H = hidden, I = inter;
    const int cap = eptr[n_exp] > 0 ? eptr[n_exp] : 1;
    float* Xg = (float*)malloc(sizeof(float) * (size_t)cap * H);
    float* Gg = (float*)malloc(sizeof(float) * (size_t)cap * I);
    float* Ug = (float*)malloc(sizeof(float) * (size_t)cap * I);
    float* Dg = (float*)malloc(sizeof(float) * (size_t)cap * H);
    int rc = ORC_OK;
    memset(Y, 0, sizeof(float) * (size_t)n_tok * H);
    for (int e = 0; e < n_exp && rc == ORC_OK; ++e) {
        const int lo = eptr[e], g = eptr[e + 1] - eptr[e];
        if (g == 0) continue;
        for (int i = 0; i < g; ++i)
            memcpy(Xg + (size_t)i * H, X + (size_t)tok[lo + i] * H, sizeof(float) * H);
        rc |= orc_matmul_quant(w_gate, (uint64_t)e * I, H, I, Xg, g, Gg);
        rc |= orc_matmul_quant(w_up, (uint64_t)e * I, H, I, Xg, g, Ug);
        for (int i = 0; i < g * I; ++i) Gg[i] = swiglu1(Gg[i], Ug[i], swiglu_limit);
        rc |= orc_matmul_quant(w_down, (uint64_t)e * H, I, H, Gg, g, Dg);
        for (int i = 0; i < g; ++i)
            orc_axpy_f32(Y + (size_t)tok[lo + i] * H, Dg + (size_t)i * H, wt[lo + i], H);
    }
    free(Xg);
    free(Gg);
    free(Ug);
    free(Dg);
    return rc;
}

/* model_batch.cpp:145-163 (dense_mlp_batch; model.cpp:677-690 is its n=1
 * case): gate/up matmul_quant at row0 0, SwiGLU clamp, down matmul_quant. */
int orc_dense_mlp(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int hidden,
                  int inter, const float* X, int n_tok, float swiglu_limit, float* Y) {
    const int H = hidden, I = inter;
    float* G = (float*)malloc(sizeof(float) * (size_t)n_tok * I);
    float* U = (float*)malloc(sizeof(float) * (size_t)n_tok * I);
    int rc = orc_matmul_quant(w_gate, 0, H, I, X, n_tok, G);
    rc |= orc_matmul_quant(w_up, 0, H, I, X, n_tok, U);
    for (int i = 0; i < n_tok * I; ++i) G[i] = swiglu1(G[i], U[i], swiglu_limit);
    rc |= orc_matmul_quant(w_down, 0, I, H, G, n_tok, Y);
    free(G);
    free(U);
    return rc;
}

/* model_batch.cpp:165-281 (moe_batch) from the router logits: router and
 * bucket sort (orc_moe_route), routed experts (orc_moe_experts), and, when
 * the shared-expert tensors are given (non-NULL), the shared expert over
 * every token (the dense FFN of orc_dense_mlp, model_batch.cpp:264-279)
 * added last with add_f32 (simd.h:53-62: a[i] += b[i]). */
int orc_moe_batch(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                  float routed_scale, int norm_topk, const uint8_t* w_gate, const uint8_t* w_up,
                  const uint8_t* w_down, const uint8_t* w_gate_sh, const uint8_t* w_up_sh,
                  const uint8_t* w_down_sh, int hidden, int inter, const float* X, float swiglu_limit, float* Y) {
    const size_t N = (size_t)n_tok * top_k;
    int* eptr = (int*)malloc(sizeof(int) * ((size_t)n_exp + 1));
    int* tok = (int*)malloc(sizeof(int) * (N ? N : 1));
    float* wt = (float*)malloc(sizeof(float) * (N ? N : 1));
    int rc = orc_moe_route(logits, n_tok, n_exp, top_k, mode, bias, routed_scale, norm_topk, eptr, tok, wt, NULL);
    if (rc == ORC_OK)
        rc = orc_moe_experts(w_gate, w_up, w_down, hidden, inter, X, n_tok, n_exp, eptr, tok, wt, swiglu_limit, Y);
    if (rc == ORC_OK && w_gate_sh) {
        float* sd = (float*)malloc(sizeof(float) * (size_t)n_tok * hidden);
        rc = orc_dense_mlp(w_gate_sh, w_up_sh, w_down_sh, hidden, inter, X, n_tok, swiglu_limit, sd);
        for (size_t i = 0; i < (size_t)n_tok * hidden; ++i) Y[i] += sd[i];
        free(sd);
    }
    free(eptr);
    free(tok);
    free(wt);
    return rc;
}

/* model.cpp:692-755 (moe_forward, one token): sigmoid scores ranked by score
 * + bias (the selection of orc_moe_route, mode 0), weights
 * (score / denom) * routed_scale (each step rounded, :715-724; without
 * norm_topk score * routed_scale), the experts in rank order, each
 * axpy_f32 into the output, then the shared expert (shared tensors
 * non-NULL) with add_f32. */
int orc_moe_forward(const float* logits, int n_exp, int top_k, const float* bias, float routed_scale,
                    int norm_topk, const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                    const uint8_t* w_gate_sh, const uint8_t* w_up_sh, const uint8_t* w_down_sh, int hidden,
                    int inter, const float* x, float swiglu_limit, float* y) {
    const int H = hidden, I = inter;
    if (top_k <= 0 || top_k > n_exp || n_exp > 1024) return ORC_ERR_UNIMPLEMENTED;
    int sel[32];
    float score[1024];
    if (top_k > 32) return ORC_ERR_UNIMPLEMENTED;
    int eptr[1025], tok[32];
    float wt[32];
    int rc = orc_moe_route(logits, 1, n_exp, top_k, 0, bias, routed_scale, norm_topk, eptr, tok, wt, sel);
    if (rc) return rc;
    for (int e = 0; e < n_exp; ++e) score[e] = 1.0f / (1.0f + expf(-logits[e]));
    float wsum[32], denom = 1e-20f;
    for (int k = 0; k < top_k; ++k) {
        wsum[k] = score[sel[k]];
        denom += wsum[k];
    }
    if (norm_topk)
        for (int k = 0; k < top_k; ++k) wsum[k] /= denom;
    for (int k = 0; k < top_k; ++k) wsum[k] *= routed_scale;
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* d = (float*)malloc(sizeof(float) * (size_t)H);
    memset(y, 0, sizeof(float) * (size_t)H);
    for (int k = 0; k < top_k && rc == ORC_OK; ++k) {
        const int e = sel[k];
        rc |= orc_matvec_quant(w_gate, (uint64_t)e * I, H, I, x, g);
        rc |= orc_matvec_quant(w_up, (uint64_t)e * I, H, I, x, u);
        for (int i = 0; i < I; ++i) g[i] = swiglu1(g[i], u[i], swiglu_limit);
        rc |= orc_matvec_quant(w_down, (uint64_t)e * H, I, H, g, d);
        orc_axpy_f32(y, d, wsum[k], H);
    }
    if (rc == ORC_OK && w_gate_sh) {
        rc |= orc_matvec_quant(w_gate_sh, 0, H, I, x, g);
        rc |= orc_matvec_quant(w_up_sh, 0, H, I, x, u);
        for (int i = 0; i < I; ++i) g[i] = swiglu1(g[i], u[i], swiglu_limit);
        rc |= orc_matvec_quant(w_down_sh, 0, I, H, g, d);
        for (int i = 0; i < H; ++i) y[i] += d[i];
    }
    free(g);
    free(u);
    free(d);
    return rc;
}
