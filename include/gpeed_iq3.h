/* gpeed_iq3.h - C ABI of the MI355X (gfx950) IQ3_XXS dequantize-and-multiply path.
 *
 * Plain C: device pointers, sizes and a stream handle (a hipStream_t passed
 * as void*; NULL = the default stream). No entry point throws or allocates
 * device memory on the compute path; each returns GPEED_OK or a negative
 * status (the C++ host layer turns these back into the reference's
 * std::runtime_error behaviour). Compute entry points are asynchronous on
 * `stream` unless stated otherwise.
 *
 * Citations name the reference interface each entry point replaces, with
 * paths relative to the reference repository root.
 */
#ifndef GPEED_IQ3_H
#define GPEED_IQ3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* gpeed_stream_t;

#define GPEED_OK 0
#define GPEED_ERR_INVALID (-1)        /* null pointer, negative size, bounds */
#define GPEED_ERR_NOT_MULTIPLE (-2)   /* n % 256 != 0            (quant.cpp:523-524) */
#define GPEED_ERR_UNALIGNED_ROW (-3)  /* in_dim % 256 != 0       (weights.cpp:93-94, 173-174) */
#define GPEED_ERR_UNIMPLEMENTED (-4)  /* dtype not on this path  (quant.cpp:553-554); caller falls back */
#define GPEED_ERR_HIP (-5)            /* a HIP runtime call failed (see gpeed_last_error) */
#define GPEED_ERR_LAYOUT (-6)         /* T64 operand addressed off a 64-row tile boundary */
#define GPEED_ERR_WORKSPACE (-7)      /* workspace missing or too small */
#define GPEED_ERR_NO_DEVICE (-8)      /* no HIP device visible */
#define GPEED_ERR_WS_STATE (-9)       /* a kernel flagged its workspace (gpeed_ws_status) */

/* Flags of a workspace's error word (gpeed_ws_status). */
#define GPEED_WS_TICKET 1u            /* a shared tile's ticket counted more arrivals than the tile has
                                       * parts: the workspace was not initialised, is shared by calls
                                       * that overlap, or was left by a call that flagged an error */
#define GPEED_WS_TIMEOUT 2u           /* a bounded wait for another workgroup's partial gave up (its
                                       * rows are wrong) */
#define GPEED_WS_BUCKETS 4u           /* expert buckets (eptr / tok) break the router's invariants */

#define GPEED_DTYPE_IQ3_XXS 18        /* common.h:27 */
/* the other types a UD-IQ3_XXS file holds (common.h:10-43) */
#define GPEED_DTYPE_F32 0
#define GPEED_DTYPE_F16 1
#define GPEED_DTYPE_Q8_0 8
#define GPEED_DTYPE_Q2_K 10
#define GPEED_DTYPE_Q3_K 11
#define GPEED_DTYPE_Q6_K 14
#define GPEED_DTYPE_IQ3_S 21
#define GPEED_DTYPE_IQ2_S 22
#define GPEED_DTYPE_IQ4_XS 23
#define GPEED_DTYPE_BF16 30

#define GPEED_X_F32 0                 /* activation element types of gpeed_iq3xxs_gemm */
#define GPEED_X_BF16 1

/* ---- device query / smoke (replaces kernels.h:7-11) --------------------- */

/* cuda_device_count (kernels.h:7, device_info.cu:12-16): 0 when none. */
int gpeed_device_count(void);
/* cuda_device_name (kernels.h:8, device_info.cu:18-22): writes the device
 * name (or "<none>") into buf, NUL-terminated. */
int gpeed_device_name(int index, char* buf, size_t len);
/* cuda_add (kernels.h:11, device_info.cu:24-38): dst = a + b for HOST
 * arrays; synchronous, stages through device memory like the reference. */
int gpeed_add_f32(const float* a, const float* b, float* dst, int n);

/* Reads the device attributes the launches are sized by (CU count) for the
 * current device. Called implicitly by the compute entry points; call it
 * once up front to keep the one-time query out of timed regions. */
int gpeed_init(void);
/* Message of the last failing call on this thread ("" if none). */
const char* gpeed_last_error(void);
/* Measurement aid, no reference counterpart: reads `bytes` from device
 * memory p (16-byte aligned, bytes a multiple of 16) once with out_words
 * (1..65535) workgroups of
 * 512 threads, each streaming a contiguous share in 16-byte loads; out[i]
 * receives a fold of what workgroup i read. Its duration is the plain
 * streaming-read time the GEMV is set against. */
int gpeed_stream_read(const void* p, size_t bytes, uint32_t* out, size_t out_words, gpeed_stream_t stream);

/* Device memory and copies for callers without HIP headers (the C++ host
 * layer; no reference counterpart: the reference keeps weights in host RAM,
 * weights.cpp:62-84). gpeed_memcpy kind: 1 host->device, 2 device->host,
 * 3 device->device; synchronous. gpeed_zero: device memset to 0 on stream. */
int gpeed_malloc(void** ptr, size_t bytes);
int gpeed_free(void* ptr);
int gpeed_memcpy(void* dst, const void* src, size_t bytes, int kind);
int gpeed_zero(void* ptr, size_t bytes, gpeed_stream_t stream);
int gpeed_stream_sync(gpeed_stream_t stream);

/* Launch timing for benchmarks (no reference counterpart): gpeed_prof_start
 * makes a pool of max_launches event pairs and times every following launch
 * of the hot kernels with events stamped by the dispatch itself (kernel
 * execution only); gpeed_prof_read stops timing, waits, and returns the
 * durations of the timed launches of one kind (0 = GEMV k_gemv_t64,
 * 1 = grouped GEMV, 2 = prefill GEMM) in launch order (up to max_n of them;
 * *n = how many there were). */
int gpeed_prof_start(int max_launches);
int gpeed_prof_read(int kind, float* durations_ms, int max_n, int* n);

/* ---- workspaces (no reference counterpart: the reference computes on the
 *      host with per-thread scratch, weights.cpp:100-107, 180-187) -------- */

/* Every workspace of the products below (GEMV, matvec / matmul, dense MLP,
 * GEMM, routed experts) starts with a 256-byte header whose first word
 * collects the GPEED_WS_* flags of the kernels that used it. A call returns
 * before its kernels run, so these conditions cannot be its status; they
 * stay in the header until gpeed_ws_status reads them. */

/* Waits for `stream`, then returns GPEED_OK if no kernel flagged ws since the
 * last check, else GPEED_ERR_WS_STATE (gpeed_last_error names the flags) and
 * clears the flags. After a flag, results written since the last check are
 * unreliable and the workspace must be initialised again. */
int gpeed_ws_status(void* ws, gpeed_stream_t stream);
/* Zero-fills ws[0..ws_bytes) with a fill kernel on `stream` (safe under graph
 * capture). Needed once for every new workspace (its header must start at
 * zero), and for GEMV, matvec / matmul and dense-MLP workspaces again after
 * a flagged error; those calls leave every word they count on at zero
 * again, for any shape the workspace is sized for. GEMM and routed-expert
 * kernels clear their own counters on every call. */
int gpeed_ws_init(void* ws, size_t ws_bytes, gpeed_stream_t stream);

/* ---- geometry (replaces quant.cpp:52-126 for IQ3_XXS) ------------------- */

/* dtype_row_bytes(IQ3_XXS, in_dim) (quant.cpp:119-126): 0 if in_dim % 256. */
size_t gpeed_iq3xxs_row_bytes(int64_t in_dim);
/* Bytes of the T64 (tiled) copy of an [n_rows, in_dim] IQ3_XXS tensor: the
 * GGUF size rounded up to whole 64-row tiles. */
size_t gpeed_iq3xxs_t64_bytes(uint64_t n_rows, int64_t in_dim);

/* ---- dequantize (replaces quant.h:18-22, quant.cpp:565-573) ------------- */

/* dequantize(DType, src, dst, n): dst[0..n) fp32 from the GGUF bytes at src
 * (device pointers; src 2-byte aligned, 4 for F32; dst 16-byte aligned), for
 * F32, F16, BF16, Q8_0, Q2_K, Q3_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S and IQ4_XS,
 * the types the reference decodes (quant.cpp:507-563). Bit-exact with the
 * reference (NaN payloads aside). Other dtypes return
 * GPEED_ERR_UNIMPLEMENTED, n not a multiple of the block size
 * GPEED_ERR_NOT_MULTIPLE (quant.cpp:523-524). */
int gpeed_dequantize(int dtype, const void* src, float* dst, uint64_t n, gpeed_stream_t stream);
/* dtype_block_size (quant.cpp:52-81) for the types above, else 0. */
int gpeed_dtype_block_size(int dtype);
/* dtype_row_bytes (quant.cpp:119-126) for the types above: 0 for another
 * type or when n is not a multiple of the block size. */
size_t gpeed_dtype_row_bytes(int dtype, uint64_t n);

/* ---- products over raw GGUF rows of any decoded type -------------------- */

/* matmul_quant / matvec_quant (weights.cpp:86-203) on a tensor kept in HBM
 * as its GGUF rows (n_rows rows of gpeed_dtype_row_bytes(dtype, in_dim)
 * bytes, device pointer, 2-byte aligned, 4 for F32): Y[t][j] = sum_i
 * W[row0 + j][i] * X[t][i] for t < n_tok, j < out_dim, with the weights
 * dequantized bit-exactly and fp32 accumulation. X [n_tok][in_dim] fp32
 * (16-byte aligned), Y [n_tok][out_dim] fp32. in_dim must be a multiple of
 * the block size and of 32, except for F32 rows, which take any length and
 * are multiplied in dot_f32's own order (simd.h:12-37): bitwise the
 * reference's products (the router's ffn_gate_inp, model_batch.cpp:172, so
 * its logits and the routing they give). No workspace. The IQ3_XXS entry
 * points above (T64 layout) are the fast path for IQ3_XXS; this one takes
 * every type. */
int gpeed_matmul_rows(int dtype, const void* w, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                      const float* X, int n_tok, float* Y, gpeed_stream_t stream);
/* Host-only (no reference counterpart): the expanded codebook the kernels
 * use for IQ2_S (1024 entries of 8 bytes), IQ3_S (512 of 4) or IQ3_XXS
 * (256 of 4), one entry per uint64. */
int gpeed_codebook(int dtype, uint64_t* out, size_t n);

/* ---- weight residency (replaces weights.cpp:62-84 pin_nonexpert/payload) */

/* Host-only layout introspection (no device use; no reference counterpart):
 * the 64 KiB replicated grid table the GEMV kernels build in LDS (32768 fp16
 * bit patterns; returns GPEED_ERR_INVALID if n < 32768), and the T64
 * sign/scale word made from a GGUF aux word. Lets CPU tests model the GPU
 * decode. */
int gpeed_t64_grid_table(uint16_t* out, size_t n);
uint32_t gpeed_t64_aux_word(uint32_t gguf_aux);

/* GGUF rows -> T64 copy (same bytes per weight, 64-row tiles) / back.
 * Done once at load time, in place of pinning the GGUF payload. */
int gpeed_iq3xxs_tile(const void* raw, uint64_t n_rows, int64_t in_dim, void* t64,
                      gpeed_stream_t stream);
int gpeed_iq3xxs_untile(const void* t64, uint64_t n_rows, int64_t in_dim, void* raw,
                        gpeed_stream_t stream);

/* ---- products (replace WeightStore::matvec_quant, weights.h:41-42,
 *      weights.cpp:167-203, and matmul_quant, weights.h:47-48,
 *      weights.cpp:86-165) ----------------------------------------------- */

/* Workspace bytes of gpeed_iq3xxs_matvec / gpeed_iq3xxs_matmul for up to
 * n_tok vectors (n_tok = 1 for matvec) on the current device. A workspace
 * sized for n_tok serves every call with fewer tokens and the same
 * (in_dim, out_dim), and matvec. Initialise it once (gpeed_ws_init). One
 * workspace per stream: calls that run concurrently must not share one. */
size_t gpeed_iq3xxs_matvec_ws_bytes(int64_t in_dim, int64_t out_dim);
size_t gpeed_iq3xxs_matmul_ws_bytes(int64_t in_dim, int64_t out_dim, int n_tok);
/* The same size for a device with num_cus compute units, computed on the
 * host without touching a device (sizing ahead of time, or on a machine
 * without the GPU). 0 for arguments the call would refuse. */
size_t gpeed_iq3xxs_matmul_ws_bytes_for(int64_t in_dim, int64_t out_dim, int n_tok, int num_cus);
/* Token count from which gpeed_iq3xxs_matmul runs the prefill GEMM (one pass
 * over W) instead of 8-token GEMV passes (one pass per 8 tokens). */
int gpeed_iq3xxs_matmul_gemm_min_tok(void);
/* dst[j] = sum_i W[row0+j][i] * x[i], j < out_dim, from the T64 copy of a
 * tensor with n_rows rows. row0 % 64 == 0. x, dst: fp32 device arrays (x
 * 16-byte aligned). One launch: the GEMV workgroups prepare the activation
 * blocks they use. */
int gpeed_iq3xxs_matvec(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                        const float* x, float* dst, void* ws, size_t ws_bytes,
                        gpeed_stream_t stream);
/* No counterpart in the reference: gpeed_iq3xxs_matvec for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc) and so bring no workspace either. The
 * same kernel and result, bit for bit; its tickets and partial sums live in
 * a fixed 4 MiB device array per GPU (set up by gpeed_init or the first
 * call on a device, held until the process ends). A shape whose launch
 * needs more than that is refused (GPEED_ERR_INVALID; the dense shapes up
 * to 12288 x 12288 fit). Every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU (other streams, other threads) race and
 * may give wrong rows; calls in order on one stream are safe. Allocates
 * nothing and calls no allocating routine. */
int gpeed_iq3xxs_matvec_noalloc(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                                const float* x, float* dst, gpeed_stream_t stream);
/* No counterpart in the reference (the status call of the entry point
 * above, for the same callers that cannot allocate): waits for `stream`,
 * then returns GPEED_OK if no kernel flagged this GPU's fixed scratch since
 * the last check, else GPEED_ERR_WS_STATE (gpeed_last_error names the
 * flags, as gpeed_ws_status) after zero-filling the whole array again, so
 * the next call starts clean. Results of calls since the last check are
 * unreliable when it reports a flag. Allocates nothing; not for use under
 * graph capture (it waits). */
int gpeed_iq3xxs_matvec_noalloc_status(gpeed_stream_t stream);
/* Test aid for the status call (no reference counterpart): writes one
 * 32-bit word at byte `offset` (a multiple of 4) of this GPU's fixed scratch,
 * synchronously. The scratch starts with the workspace header (error word at
 * 0), then at byte 256 one ticket word per 64-row tile of the last shape.
 * Allocates nothing. */
int gpeed_iq3xxs_matvec_noalloc_poke(size_t offset, uint32_t value);
/* Y[t][j] = sum_i W[row0+j][i] * X[t][i] for t < n_tok (X [n_tok][in_dim],
 * Y [n_tok][out_dim], fp32, row-major). Row t of Y is the matvec of X[t]
 * (weights.cpp:86-165 makes the same promise) up to fp32 summation order.
 * Below gpeed_iq3xxs_matmul_gemm_min_tok() tokens: GEMV passes of up to 8
 * tokens; from there on: the prefill GEMM with fp32 X (gpeed_iq3xxs_gemm),
 * so W is read once whatever n_tok. */
int gpeed_iq3xxs_matmul(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                        const float* X, int n_tok, float* Y, void* ws, size_t ws_bytes,
                        gpeed_stream_t stream);

/* Prefill GEMM: Y[t][j] = sum_i W[row0+j][i] * X[t][i] for t < n_tok, with
 * X [n_tok][in_dim] fp32 (x_dtype GPEED_X_F32) or bf16 (GPEED_X_BF16), Y fp32
 * [n_tok][out_dim]. W records are staged through LDS and decoded to exact
 * fp16 values of q*(2s+1) as MFMA operands; the block scale d/4 is applied
 * to each block's fp32 partial. The prefill-sized case of matmul_quant
 * (weights.cpp:86-165, model_batch.cpp:30-95 / 151-162). When the 128 x 192
 * result tiles fill fewer than half the device's CUs (few tokens or few
 * rows), K is split over workgroups and the partials are added in a fixed
 * order (bitwise repeatable). X 16-byte aligned; ws:
 * gpeed_iq3xxs_gemm_ws_bytes bytes for this device (initialised once for
 * its header: the X preparation clears the split-K tickets of every call);
 * calls on one ws must not overlap. W records are addressed with 32-bit
 * offsets: a tensor whose requested rows hold 4 GiB of records or more is
 * rejected (GPEED_ERR_INVALID). */
size_t gpeed_iq3xxs_gemm_ws_bytes(int64_t n_tok, int64_t in_dim, int64_t out_dim, int x_dtype);
int gpeed_iq3xxs_gemm(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim, const void* X,
                      int x_dtype, int n_tok, float* Y, void* ws, size_t ws_bytes, gpeed_stream_t stream);
/* The down projection of dense_mlp_batch (model_batch.cpp:145-163, SwiGLU
 * clamp as model_batch.cpp:245-253) as one GEMM: X[t] = silu(min(G[t],
 * limit)) * clamp(U[t], -limit, limit) for G, U fp32 [n_tok][in_dim], formed
 * while the fp16 images are prepared. ws: gpeed_iq3xxs_gemm_ws_bytes with
 * x_dtype GPEED_X_F32. */
int gpeed_iq3xxs_gemm_swiglu(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                             const float* G, const float* U, float limit, int n_tok, float* Y, void* ws,
                             size_t ws_bytes, gpeed_stream_t stream);
/* Two matmul_quant calls on the same X (kv_a and q_a, model_batch.cpp:62,72;
 * gate and up, model_batch.cpp:151-162) as one launch: X is prepared once
 * and the result tiles of both tensors share the grid, so neither product
 * waits for the other. Y_a [n_tok][out_a] from rows row0_a.. of w_a, Y_b
 * [n_tok][out_b] from w_b, each exactly as gpeed_iq3xxs_gemm would give it.
 * ws: gpeed_iq3xxs_gemm2_ws_bytes bytes (same rules as the GEMM's). */
size_t gpeed_iq3xxs_gemm2_ws_bytes(int64_t n_tok, int64_t in_dim, int64_t out_a, int64_t out_b, int x_dtype);
int gpeed_iq3xxs_gemm2(const void* w_a, uint64_t n_rows_a, uint64_t row0_a, int out_a, const void* w_b,
                       uint64_t n_rows_b, uint64_t row0_b, int out_b, int in_dim, const void* X, int x_dtype,
                       int n_tok, float* Y_a, float* Y_b, void* ws, size_t ws_bytes, gpeed_stream_t stream);
/* dense_mlp_batch (model_batch.cpp:145-163) over n_tok tokens as GEMMs:
 * Y [n_tok][hidden] = down(SwiGLU(gate X, up X)) with the SwiGLU clamp of
 * gpeed_iq3xxs_gemm_swiglu, for whole T64 tensors gate/up [inter][hidden] and
 * down [hidden][inter]. Up to n_extra = 2 more whole T64 tensors of the same
 * X (extra_w[i], extra_out[i] rows of hidden; extra_Y[i] [n_tok][extra_out[i]];
 * e.g. the latent projections kv_a, q_a of model_batch.cpp:62, 72, which the
 * reference runs as matmul_quant calls of their own) are computed in the
 * down launch: at up to 64 tokens of fp32 X it holds both problems, with K
 * splits that give every workgroup the same number of blocks, so those
 * products fill the CUs the down product leaves idle (elsewhere they are a
 * launch of their own). Four launches in all: X images, gate+up, SwiGLU
 * images, down (+ extra). Each output is as the GEMM entry points above give
 * it. ws: gpeed_iq3xxs_mlp_gemm_ws_bytes bytes (same rules as the GEMM's);
 * the gate/up rows are kept in it. */
size_t gpeed_iq3xxs_mlp_gemm_ws_bytes(int64_t n_tok, int64_t hidden, int64_t inter, int x_dtype, int n_extra,
                                      const int* extra_out);
int gpeed_iq3xxs_mlp_gemm(const void* w_gate, const void* w_up, const void* w_down, int hidden, int inter,
                          const void* X, int x_dtype, int n_tok, float swiglu_limit, float* Y, int n_extra,
                          const void* const* extra_w, const int* extra_out, float* const* extra_Y, void* ws,
                          size_t ws_bytes, gpeed_stream_t stream);

/* The two halves of the products, for callers that reuse one activation
 * across several tensors (gate and up of model.cpp:681-682) or fuse the
 * SwiGLU epilogue into the next product's input (model.cpp:683-689). A
 * "prepared activation" holds 1..8 fp32 vectors as the fp16 hi/lo MFMA
 * operand plus a power-of-two scale per 256 elements, in a caller-owned
 * device buffer of gpeed_iq3xxs_act_bytes(in_dim, n_tok) bytes (16-byte
 * aligned). The GEMV workspace (gpeed_iq3xxs_gemv_ws_bytes; initialised
 * once with gpeed_ws_init, one per stream) holds the tickets and partial
 * sums of row tiles that workgroups share; a workspace sized for n_tok
 * serves every call with fewer tokens on the same shape. */
size_t gpeed_iq3xxs_act_bytes(int64_t in_dim, int n_tok);
int gpeed_iq3xxs_prep_act(const float* x, int64_t in_dim, int n_tok, void* act, size_t act_bytes,
                          gpeed_stream_t stream);
/* act <- silu(min(g,limit)) * clamp(u,-limit,limit) over n_tok vectors of
 * n = in_dim elements (model.cpp:683-688, model_batch.cpp:245-253 with
 * swiglu_limit, model_config.h:70). */
int gpeed_iq3xxs_prep_swiglu(const float* g, const float* u, int64_t n, int n_tok, float limit,
                             void* act, size_t act_bytes, gpeed_stream_t stream);
size_t gpeed_iq3xxs_gemv_ws_bytes(int n_tensors, int64_t in_dim, int64_t out_dim, int n_tok);
/* dst[t][j] = sum_i W[row0+j][i] * x_t[i] for the n_tok (1..8) prepared
 * vectors; dst is [n_tok][out_dim]. */
int gpeed_iq3xxs_gemv_act(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                          const void* act, int n_tok, float* dst, void* ws, size_t ws_bytes,
                          gpeed_stream_t stream);
/* One fp32 vector x straight in: the GEMV workgroups prepare the activation
 * blocks they use themselves, so a product is one launch. gemv2_x: two same-shape
 * tensors (gate and up); gemv_swiglu: the input is silu(min(g,limit)) *
 * clamp(u,-limit,limit) computed in the kernel (the down projection of
 * model.cpp:683-689). ws as gpeed_iq3xxs_gemv_ws_bytes(n_tensors, in_dim,
 * out_dim, 1). */
int gpeed_iq3xxs_gemv_x(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim, const float* x,
                        float* dst, void* ws, size_t ws_bytes, gpeed_stream_t stream);
int gpeed_iq3xxs_gemv2_x(const void* w_a, const void* w_b, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                         const float* x, float* dst_a, float* dst_b, void* ws, size_t ws_bytes,
                         gpeed_stream_t stream);
int gpeed_iq3xxs_gemv_swiglu(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                             const float* g, const float* u, float limit, float* dst, void* ws, size_t ws_bytes,
                             gpeed_stream_t stream);
/* The per-head absorbed projections of MLA attention in one launch: for
 * head h < n_heads, dst[h*rows_per_head + j] = sum_i W[row0 + h*rows_per_head
 * + j][i] * x[h*in_dim + i], j < rows_per_head. These are the n_heads
 * matvec_quant calls with row0 = h * rows_per_head on each head's own
 * vector: attn_k_b at model.cpp:638-643 (rows h*kv_lora, in_dim qk_nope)
 * and attn_v_b at model.cpp:664-665 (rows h*v_head, in_dim kv_lora).
 * x [n_heads][in_dim], dst [n_heads][rows_per_head] fp32; rows_per_head and
 * row0 multiples of 64. ws: gpeed_iq3xxs_gemv_ws_bytes(1, in_dim,
 * n_heads * rows_per_head, 1) bytes, initialised once. */
int gpeed_iq3xxs_matvec_heads(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int rows_per_head,
                              int n_heads, const float* x, float* dst, void* ws, size_t ws_bytes,
                              gpeed_stream_t stream);
/* Model::dense_mlp (model.cpp:677-690) on the device without the
 * intermediate vectors: y = W_down (silu(min(g,limit)) * clamp(u,-limit,limit))
 * with g = W_gate x, u = W_up x. gate and up run together; the workgroup
 * that completes 64 rows of g and u writes their SwiGLU straight into the
 * down projection's prepared activation (one power-of-two scale per 64
 * values); the second launch multiplies it. The first launch also zero-fills
 * y, and the second adds the parts of its row tiles that several workgroups
 * share into y with atomic adds, so repeated calls agree to within the fp32
 * rounding of those two to four adds (their order varies); where y overlaps
 * x the parts are summed in a fixed order instead (bitwise repeatable).
 * gate/up are T64 copies of inter x hidden, down
 * of hidden x inter (rows from 0); hidden and inter multiples of 256. ws:
 * gpeed_iq3xxs_dense_mlp_ws_bytes bytes, initialised once with
 * gpeed_ws_init (every call leaves it ready for the next); one workspace per
 * stream. */
size_t gpeed_iq3xxs_dense_mlp_ws_bytes(int64_t hidden, int64_t inter);
int gpeed_iq3xxs_dense_mlp(const void* w_gate, const void* w_up, const void* w_down, int hidden, int inter,
                           const float* x, float limit, float* y, void* ws, size_t ws_bytes, gpeed_stream_t stream);
/* Two same-shape tensors against one prepared activation in one launch
 * (gate and up of model.cpp:681-682, or of the shared expert at 747-748);
 * ws sized for n_tensors = 2. */
int gpeed_iq3xxs_gemv2_act(const void* w_a, const void* w_b, uint64_t n_rows, uint64_t row0,
                           int in_dim, int out_dim, const void* act, int n_tok, float* dst_a,
                           float* dst_b, void* ws, size_t ws_bytes, gpeed_stream_t stream);

/* ---- routed experts (replace Model::moe_batch steps 1-3,
 *      model_batch.cpp:165-262) ------------------------------------------ */

/* Router on the device: per token t < n_tok the top_k of logits[t][0..n_exp)
 * (mode 0: the reference router, score = sigmoid(logit), ranked by score +
 * bias[e] (bias may be NULL), weight = score * routed_scale / (1e-20 + sum
 * of the top-k scores) if norm_topk else score * routed_scale,
 * model_batch.cpp:186-203; mode 1: ranked by logit, weight = softmax over
 * the top_k); equal keys rank the lower expert id first. Then the stable
 * bucket sort of the (token, k) assignments by expert (model_batch.cpp:
 * 205-219): eptr[n_exp+1] offsets, tok[n_tok*top_k] token of each bucket
 * slot, wt[...] its weight; sel[n_tok*top_k] (optional, may be NULL) the
 * ranked experts per token. All device arrays; integers equal the CPU's.
 * n_exp <= 1024, top_k <= 32. ws: gpeed_moe_route_ws_bytes bytes. */
size_t gpeed_moe_route_ws_bytes(int n_tok, int n_exp, int top_k);
int gpeed_moe_route(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                    float routed_scale, int norm_topk, int* eptr, int* tok, float* wt, int* sel, void* ws,
                    size_t ws_bytes, gpeed_stream_t stream);
/* Routed experts for n_tok tokens X [n_tok][hidden]: for every expert e with
 * tokens, gate/up = rows e*inter.. of w_gate / w_up (T64 copies of
 * [n_exp*inter, hidden] tensors, ffn_gate_exps / ffn_up_exps), SwiGLU with
 * swiglu_limit, down = rows e*hidden.. of w_down ([n_exp*hidden, inter],
 * ffn_down_exps); Y[t] = sum over the token's experts, in expert order, of
 * wt * down (Y overwritten; the shared expert is not included). hidden and
 * inter are multiples of 256; n_tok <= 8192. eptr/tok/wt as gpeed_moe_route
 * makes them: eptr[0] = 0, non-decreasing, eptr[n_exp] = n_tok*top_k, every
 * tok entry in [0, n_tok) and every token present top_k times. Buckets that
 * break these rules are not multiplied: Y is zero and the workspace's
 * GPEED_WS_BUCKETS flag is set. ws: gpeed_iq3xxs_moe_ws_bytes bytes
 * (initialised once for its header). */
size_t gpeed_iq3xxs_moe_ws_bytes(int n_tok, int n_exp, int top_k, int hidden, int inter);
int gpeed_iq3xxs_moe_experts(const void* w_gate, const void* w_up, const void* w_down, int n_exp, int hidden,
                             int inter, const float* X, int n_tok, int top_k, const int* eptr, const int* tok,
                             const float* wt, float swiglu_limit, float* Y, void* ws, size_t ws_bytes,
                             gpeed_stream_t stream);

/* The whole routed-expert step of Model::moe_batch from the router logits
 * (model_batch.cpp:174-280, steps 2-4; step 1's router product is a
 * matvec / matmul of ffn_gate_inp): the router and bucket sort of
 * gpeed_moe_route (mode, bias, routed_scale, norm_topk as there), the routed
 * experts of gpeed_iq3xxs_moe_experts, and, when w_gate_sh / w_up_sh /
 * w_down_sh are given (T64 copies of ffn_gate_shexp / ffn_up_shexp [inter,
 * hidden] and ffn_down_shexp [hidden, inter]; all three NULL for none), the
 * shared expert over every token, added last (add_f32,
 * model_batch.cpp:264-280): Y[t] = (sum over the token's experts, in expert
 * order, of wt * down) + shared[t]. Five launches. eptr / tok / wt
 * (optional device outputs, may be NULL) receive the routing as
 * gpeed_moe_route makes it. Limits as gpeed_moe_route and
 * gpeed_iq3xxs_moe_experts. ws: gpeed_iq3xxs_moe_batch_ws_bytes(...,
 * shared = 1 with a shared expert) bytes, initialised once for its header. */
size_t gpeed_iq3xxs_moe_batch_ws_bytes(int n_tok, int n_exp, int top_k, int hidden, int inter, int shared);
int gpeed_iq3xxs_moe_batch(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                           float routed_scale, int norm_topk, const void* w_gate, const void* w_up,
                           const void* w_down, const void* w_gate_sh, const void* w_up_sh, const void* w_down_sh,
                           int hidden, int inter, const float* X, float swiglu_limit, float* Y, int* eptr, int* tok,
                           float* wt, void* ws, size_t ws_bytes, gpeed_stream_t stream);

/* Checks expert buckets held in HOST memory against the invariants above
 * (what the reference's bucket sort, model_batch.cpp:205-219, produces):
 * GPEED_OK, or GPEED_ERR_INVALID with the first violation in
 * gpeed_last_error. For callers that build eptr / tok on the host. */
int gpeed_moe_check_buckets(const int* eptr, const int* tok, int n_exp, int n_tok, int top_k);

/* Same product as gpeed_iq3xxs_matvec straight from GGUF rows (no tiling;
 * any row0), one wavefront per row. */
int gpeed_iq3xxs_matvec_raw(const void* w_gguf, uint64_t n_rows, uint64_t row0, int in_dim,
                            int out_dim, const float* x, float* dst, gpeed_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
