/* CPU oracle for the other GGUF block formats of a UD-IQ3_XXS file.
 *
 * TEST INFRASTRUCTURE ONLY (see iq3_oracle.h): a plain-C restatement of the
 * reference's dequantizers, used as the correctness reference by tests/.
 * Nothing in the product links or calls it.
 *
 * Each format is restated element by element: orc_q_elem(dtype, blk, e)
 * returns element e of one block, with the reference's float operations in
 * the reference's order (quant.cpp is built without FP contraction, as
 * -std=c++20 implies, so every product and difference is rounded on its
 * own; this file is compiled with -ffp-contract=off for the same reason).
 * Byte positions follow the reference's pointer walks, rewritten as
 * closed-form offsets. Pinned bitwise against oracle/_ref (the reference's
 * quant.cpp compiled from source) over random and special-value blocks, and
 * the codebooks against the reference header's values.
 */
#include <math.h>
#include <string.h>

#include "iq3_oracle.h"
#include "../gpeed_amd/csrc/quant_grids.h"

static const uint16_t kIq2sPacked[1024] = {GPEED_IQ2S_PACKED};
static const uint16_t kIq3sPacked[512] = {GPEED_IQ3S_PACKED};
static const int8_t kIq4nl[16] = {GPEED_IQ4NL_VALUES};
static const uint8_t kIq2sLevels[3] = {GPEED_IQ2S_LEVELS};

static uint32_t u16le(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

/* byte j of IQ2_S grid entry i (quant_tables.h:15, packed encoding) */
static uint32_t iq2s_grid_byte(uint32_t i, int j) { return kIq2sLevels[(kIq2sPacked[i] >> (2 * j)) & 3]; }
/* byte j of IQ3_S grid entry i (quant_tables.h:275, packed encoding) */
static uint32_t iq3s_grid_byte(uint32_t i, int j) { return 2u * ((kIq3sPacked[i] >> (3 * j)) & 7u) + 1u; }

uint64_t orc_iq2s_grid(uint32_t i) {
    uint64_t v = 0;
    for (int j = 0; j < 8; ++j) v |= (uint64_t)iq2s_grid_byte(i, j) << (8 * j);
    return v;
}
uint32_t orc_iq3s_grid(uint32_t i) {
    uint32_t v = 0;
    for (int j = 0; j < 4; ++j) v |= iq3s_grid_byte(i, j) << (8 * j);
    return v;
}
int orc_iq4nl_value(int i) { return kIq4nl[i & 15]; }

/* quant.cpp:52-81 (dtype_block_size) and :83-114 (dtype_type_size), for the
 * types the reference decodes (quant.cpp:507-519 plus F32/F16/BF16). */
int orc_block_elems(int dtype) {
    switch (dtype) {
        case ORC_DTYPE_F32: case ORC_DTYPE_F16: case ORC_DTYPE_BF16: return 1;
        case ORC_DTYPE_Q8_0: return 32;
        case ORC_DTYPE_Q2_K: case ORC_DTYPE_Q3_K: case ORC_DTYPE_Q6_K: case ORC_DTYPE_IQ3_XXS:
        case ORC_DTYPE_IQ3_S: case ORC_DTYPE_IQ2_S: case ORC_DTYPE_IQ4_XS: return ORC_QK_K;
        default: return 0;
    }
}
int orc_block_bytes(int dtype) {
    switch (dtype) {
        case ORC_DTYPE_F32: return 4;
        case ORC_DTYPE_F16: case ORC_DTYPE_BF16: return 2;
        case ORC_DTYPE_Q8_0: return 34;
        case ORC_DTYPE_Q2_K: return 84;
        case ORC_DTYPE_Q3_K: return 110;
        case ORC_DTYPE_Q6_K: return 210;
        case ORC_DTYPE_IQ3_XXS: return 98;
        case ORC_DTYPE_IQ3_S: return 110;
        case ORC_DTYPE_IQ2_S: return 82;
        case ORC_DTYPE_IQ4_XS: return 136;
        default: return 0;
    }
}
/* quant.cpp:119-126 (dtype_row_bytes) */
size_t orc_row_bytes(int dtype, uint64_t n) {
    const int be = orc_block_elems(dtype);
    if (be == 0 || n % (uint64_t)be) return 0;
    return (size_t)(n / (uint64_t)be) * (size_t)orc_block_bytes(dtype);
}

/* quant.cpp:165-184 (blk_q8_0): d (fp16) then 32 int8 codes; y = d * q. */
static float q8_0_elem(const uint8_t* b, int e) {
    const float d = orc_f16_to_f32((uint16_t)u16le(b));
    return d * (float)(int8_t)b[2 + e];
}

/* quant.cpp:212-306 (blk_q6_K; the AVX2 and scalar paths agree): ql[128],
 * qh[64], int8 scales[16], d. Element e: half h = e/128, quarter q = e%128/32,
 * l = e%32; low nibble of ql[64h + l + 32(q&1)] (high nibble for q >= 2),
 * two bits (2q) of qh[32h + l]; scale sc[8h + l/16 + 2q]; y = (d*sc)*(v-32). */
static float q6_k_elem(const uint8_t* b, int e) {
    const int h = e >> 7, q = (e >> 5) & 3, l = e & 31;
    const uint32_t lo = b[64 * h + l + 32 * (q & 1)];
    const uint32_t nib = q >= 2 ? lo >> 4 : lo & 15u;
    const uint32_t hi = (b[128 + 32 * h + l] >> (2 * q)) & 3u;
    const int v = (int)(nib | (hi << 4)) - 32;
    const float d = orc_f16_to_f32((uint16_t)u16le(b + 208));
    const float dsc = d * (float)(int8_t)b[192 + 8 * h + (l >> 4) + 2 * q];
    return dsc * (float)v;
}

/* quant.cpp:309-335 (blk_q2_K): scales[16], qs[64], d, dmin. Element e:
 * h = e/128, j = e%128/32 (2-bit plane), s = e%32/16, l = e%16; scale byte
 * sc = scales[8h + 2j + s]; code (qs[32h + 16s + l] >> 2j) & 3;
 * y = (d*(sc&15))*code - dmin*(sc>>4). */
static float q2_k_elem(const uint8_t* b, int e) {
    const int h = e >> 7, j = (e >> 5) & 3, s = (e >> 4) & 1, l = e & 15;
    const uint32_t sc = b[8 * h + 2 * j + s];
    const uint32_t code = (b[16 + 32 * h + 16 * s + l] >> (2 * j)) & 3u;
    const float d = orc_f16_to_f32((uint16_t)u16le(b + 80));
    const float mn = orc_f16_to_f32((uint16_t)u16le(b + 82));
    const float dl = d * (float)(sc & 15u);
    const float ml = mn * (float)(sc >> 4);
    return dl * (float)code - ml;
}

/* The 6-bit scale k (0..15) of a Q3_K block, as quant.cpp:340-347 unpacks
 * the 12 scale bytes: low nibble from byte k (k < 8) or the high nibble of
 * byte k-8, top two bits from byte 8 + k%4 at bit 2*(k/4). */
static int q3_k_scale(const uint8_t* sb, int k) {
    const uint32_t low = k < 8 ? sb[k] & 15u : sb[k - 8] >> 4;
    const uint32_t top = (sb[8 + (k & 3)] >> (2 * (k >> 2))) & 3u;
    return (int)(int8_t)(uint8_t)(low | (top << 4));
}

/* quant.cpp:337-370 (blk_q3_K): hmask[32], qs[64], scales[12], d. Element
 * e: h, j, s, l as Q2_K; code (qs[32h + 16s + l] >> 2j) & 3, minus 4 when
 * bit 4h + j of hmask[16s + l] is clear; y = (d*(scale-32))*value. */
static float q3_k_elem(const uint8_t* b, int e) {
    const int h = e >> 7, j = (e >> 5) & 3, s = (e >> 4) & 1, l = e & 15;
    const int code = (int)((b[32 + 32 * h + 16 * s + l] >> (2 * j)) & 3u);
    const int hbit = (b[16 * s + l] >> (4 * h + j)) & 1;
    const float d = orc_f16_to_f32((uint16_t)u16le(b + 108));
    const float dl = d * (float)(q3_k_scale(b + 96, 8 * h + 2 * j + s) - 32);
    return dl * (float)(code - (hbit ? 0 : 4));
}

/* quant.cpp:186-210 (blk_iq3_xxs), through the existing block decoder. */

/* quant.cpp:373-418 (blk_iq2_s): d, qs[32] (grid low bytes), signs[32],
 * qh[8], scales[8]. Element e: group g = e/8 (l = g%4 inside sub-block
 * ib = g/4), j = e%8; index qs[g] | bits (2l, 2l+1) of qh[ib] as bits 8-9;
 * scale nibble (l < 2 low, else high) of scales[ib];
 * y = ((d*(0.5+s))*0.25) * grid_j * (bit j of signs[g] ? -1 : 1). */
static float iq2_s_elem(const uint8_t* b, int e) {
    const int g = e >> 3, ib = g >> 2, l = g & 3, j = e & 7;
    const uint32_t idx = (uint32_t)b[2 + g] | (((uint32_t)b[66 + ib] << (8 - 2 * l)) & 0x300u);
    const uint32_t nib = l < 2 ? b[74 + ib] & 15u : b[74 + ib] >> 4;
    const float d = orc_f16_to_f32((uint16_t)u16le(b));
    const float dl = d * (0.5f + (float)nib) * 0.25f;
    const float sign = ((b[34 + g] >> j) & 1) ? -1.0f : 1.0f;
    return dl * (float)iq2s_grid_byte(idx, j) * sign;
}

/* quant.cpp:421-482 (blk_iq3_s): d, qs[64], qh[8], signs[32], scales[4].
 * Element e: group g = e/8 of sub-block ib = g/4 (l = g%4), j = e%8;
 * grid index qs[8ib + 2l + j/4] with bit 8 from qh[ib] (bit 2l for j < 4,
 * bit 2l+1 otherwise); scale nibble of scales[ib/2] (low for even ib);
 * y = (d*(1+2s)) * grid * (bit j of signs[g] ? -1 : 1). */
static float iq3_s_elem(const uint8_t* b, int e) {
    const int g = e >> 3, ib = g >> 2, l = g & 3, j = e & 7, half = j >> 2;
    const uint32_t idx = (uint32_t)b[2 + 8 * ib + 2 * l + half] |
                         (((uint32_t)b[66 + ib] << (8 - 2 * l - half)) & 256u);
    const uint32_t nib = (ib & 1) ? b[106 + (ib >> 1)] >> 4 : b[106 + (ib >> 1)] & 15u;
    const float d = orc_f16_to_f32((uint16_t)u16le(b));
    const float db = d * (1.0f + 2.0f * (float)nib);
    const float sign = ((b[74 + g] >> j) & 1) ? -1.0f : 1.0f;
    return db * (float)iq3s_grid_byte(idx, j & 3) * sign;
}

/* quant.cpp:485-502 (blk_iq4_xs): d, scales_h (u16), scales_l[4], qs[128].
 * Element e: sub-block ib = e/32, i = e%32; 6-bit scale = nibble ib%2 of
 * scales_l[ib/2] | bits (2ib, 2ib+1) of scales_h << 4; code = low nibble of
 * qs[16ib + i] (i < 16) or high nibble of qs[16ib + i - 16];
 * y = (d*(ls-32)) * kvalues[code]. */
static float iq4_xs_elem(const uint8_t* b, int e) {
    const int ib = e >> 5, i = e & 31;
    const uint32_t sh = u16le(b + 2);
    const int ls = (int)(((b[4 + (ib >> 1)] >> (4 * (ib & 1))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
    const uint32_t q = b[8 + 16 * ib + (i & 15)];
    const uint32_t code = i < 16 ? q & 15u : q >> 4;
    const float d = orc_f16_to_f32((uint16_t)u16le(b));
    const float dl = d * (float)(ls - 32);
    return dl * (float)kIq4nl[code];
}

/* One block of a quantized type into y[orc_block_elems(dtype)]. */
int orc_dequant_block(int dtype, const uint8_t* blk, float* y) {
    const int n = orc_block_elems(dtype);
    switch (dtype) {
        case ORC_DTYPE_Q8_0: for (int e = 0; e < n; ++e) y[e] = q8_0_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_Q6_K: for (int e = 0; e < n; ++e) y[e] = q6_k_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_Q2_K: for (int e = 0; e < n; ++e) y[e] = q2_k_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_Q3_K: for (int e = 0; e < n; ++e) y[e] = q3_k_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_IQ2_S: for (int e = 0; e < n; ++e) y[e] = iq2_s_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_IQ3_S: for (int e = 0; e < n; ++e) y[e] = iq3_s_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_IQ4_XS: for (int e = 0; e < n; ++e) y[e] = iq4_xs_elem(blk, e); return ORC_OK;
        case ORC_DTYPE_IQ3_XXS: orc_iq3xxs_block(blk, y); return ORC_OK;
        default: return ORC_ERR_UNIMPLEMENTED;
    }
}

/* weights.cpp:86-165 / 167-203 (matmul_quant, matvec_quant) for any type
 * the reference decodes: each row dequantized (dequantize_row) and
 * Y[t][j] = dot_f32(row, X[t]). */
int orc_matmul_rows(int dtype, const uint8_t* w, uint64_t row0, int in_dim, int out_dim, const float* X,
                    int n_tok, float* Y, float* row_buf) {
    if (n_tok <= 0 || out_dim <= 0) return ORC_OK;
    const int be = orc_block_elems(dtype);
    if (be == 0) return ORC_ERR_UNIMPLEMENTED;
    if (in_dim % be) return ORC_ERR_UNALIGNED_ROW;
    const size_t rb = orc_row_bytes(dtype, (uint64_t)in_dim);
    const uint8_t* src = w + row0 * rb;
    for (int j = 0; j < out_dim; ++j) {
        const int rc = orc_dequantize(dtype, src + rb * (size_t)j, row_buf, (uint64_t)in_dim);
        if (rc) return rc;
        for (int t = 0; t < n_tok; ++t) Y[(size_t)t * out_dim + j] = orc_dot_f32(row_buf, X + (size_t)t * in_dim, in_dim);
    }
    return ORC_OK;
}
