// C ABI (include/gpeed_iq3.h) over the gfx950 kernels.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gpeed_iq3.h"
#include "iq3_common.h"
#include "iq3_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(GPEED_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::mutex g_init_mu;
struct DeviceState {
    int num_cus = 0;  // set once, read without the lock afterwards
};
DeviceState g_dev[kMaxDevices];

// Per-device launch parameters, read once per device.
int device_state(const DeviceState** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(GPEED_ERR_INVALID, "device index out of range");
    DeviceState& st = g_dev[dev];
    if (!__atomic_load_n(&st.num_cus, __ATOMIC_ACQUIRE)) {
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (!st.num_cus) {
            int cus = 0;
            e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
            __atomic_store_n(&st.num_cus, cus > 0 ? cus : 1, __ATOMIC_RELEASE);
        }
    }
    *out = &st;
    return GPEED_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Scratch of gpeed_iq3xxs_matvec_noalloc: a GEMV workspace (header, tickets,
// tagged partials) in a fixed device array, one copy per GPU that loads the
// library, held until the process ends. Host code never uses the array's
// name as an address: each device's copy is reached through the pointer
// hipGetSymbolAddress returned for it (g_noalloc[dev]).
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_noalloc_mu;
void* g_noalloc[kMaxDevices] = {};

// Zero-fills this device's copy of `scratch` (at p) on `s` and waits for
// the fill, so that a call from any stream afterwards sees it cleared.
int noalloc_clear(void* p, hipStream_t s) {
    hipError_t e = gpeed::launch_fill_zero(p, kNoAllocScratchBytes, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "clearing the no-allocation scratch");
}

// This device's copy of `scratch` (looked up once per device, with that
// device current), zero-filled on `s` the first time; the pointer is
// published only once the fill has completed. The first use cannot be on a
// stream under graph capture (its wait is not allowed there): gpeed_init
// does it ahead of time. No allocation.
int noalloc_scratch(int dev, hipStream_t s, void** out) {
    void* p = __atomic_load_n(&g_noalloc[dev], __ATOMIC_ACQUIRE);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_noalloc_mu);
        p = g_noalloc[dev];
        if (!p) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            hipError_t e = hipStreamIsCapturing(s, &cs);
            if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
            if (cs != hipStreamCaptureStatusNone)
                return fail(GPEED_ERR_INVALID,
                            "matvec_noalloc: first use on this device under graph capture; call gpeed_init first");
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
            const int rc = noalloc_clear(p, s);
            if (rc) return rc;
            __atomic_store_n(&g_noalloc[dev], p, __ATOMIC_RELEASE);
        }
    }
    *out = p;
    return GPEED_OK;
}

// Launch timing pool (see iq3_prof.h). One pool per process, guarded by a
// mutex; events are created on the device current at gpeed_prof_start.
struct ProfPool {
    std::mutex mu;
    bool on = false;
    std::vector<hipEvent_t> start, stop;
    std::vector<int> kind;
    size_t used = 0;
};
ProfPool g_prof;

}  // namespace

namespace gpeed {
bool prof_slot(int kind, hipEvent_t* a, hipEvent_t* b) {
    std::lock_guard<std::mutex> lk(g_prof.mu);
    if (!g_prof.on || g_prof.used >= g_prof.start.size()) return false;
    const size_t i = g_prof.used++;
    g_prof.kind[i] = kind;
    *a = g_prof.start[i];
    *b = g_prof.stop[i];
    return true;
}
}  // namespace gpeed

extern "C" {

const char* gpeed_last_error(void) { return g_err.c_str(); }

int gpeed_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(GPEED_ERR_INVALID, "malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return GPEED_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "hipMalloc");
}

int gpeed_free(void* ptr) {
    if (!ptr) return GPEED_OK;
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "hipFree");
}

int gpeed_memcpy(void* dst, const void* src, size_t bytes, int kind) {
    if (bytes == 0) return GPEED_OK;
    if (!dst || !src) return fail(GPEED_ERR_INVALID, "memcpy: null pointer");
    hipMemcpyKind k;
    switch (kind) {
        case 1: k = hipMemcpyHostToDevice; break;
        case 2: k = hipMemcpyDeviceToHost; break;
        case 3: k = hipMemcpyDeviceToDevice; break;
        default: return fail(GPEED_ERR_INVALID, "memcpy: kind must be 1, 2 or 3");
    }
    hipError_t e = hipMemcpy(dst, src, bytes, k);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "hipMemcpy");
}

int gpeed_zero(void* ptr, size_t bytes, gpeed_stream_t stream) {
    if (bytes == 0) return GPEED_OK;
    if (!ptr) return fail(GPEED_ERR_INVALID, "zero: null pointer");
    hipError_t e = hipMemsetAsync(ptr, 0, bytes, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "hipMemsetAsync");
}

int gpeed_stream_sync(gpeed_stream_t stream) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "hipStreamSynchronize");
}

int gpeed_prof_start(int max_launches) {
    if (max_launches < 1 || max_launches > (1 << 20)) return fail(GPEED_ERR_INVALID, "prof_start: bad pool size");
    std::lock_guard<std::mutex> lk(g_prof.mu);
    for (size_t i = 0; i < g_prof.start.size(); ++i) {
        (void)hipEventDestroy(g_prof.start[i]);
        (void)hipEventDestroy(g_prof.stop[i]);
    }
    g_prof.start.assign(max_launches, nullptr);
    g_prof.stop.assign(max_launches, nullptr);
    g_prof.kind.assign(max_launches, -1);
    for (int i = 0; i < max_launches; ++i) {
        hipError_t e = hipEventCreate(&g_prof.start[i]);
        if (e == hipSuccess) e = hipEventCreate(&g_prof.stop[i]);
        if (e != hipSuccess) {
            g_prof.start.resize(i);
            g_prof.stop.resize(i);
            g_prof.kind.resize(i);
            return hip_fail(e, "prof_start: hipEventCreate");
        }
    }
    g_prof.used = 0;
    g_prof.on = true;
    return GPEED_OK;
}

int gpeed_prof_read(int kind, float* durations_ms, int max_n, int* n) {
    if (!n) return fail(GPEED_ERR_INVALID, "prof_read: null count");
    std::lock_guard<std::mutex> lk(g_prof.mu);
    g_prof.on = false;
    int c = 0;
    for (size_t i = 0; i < g_prof.used; ++i) {
        if (g_prof.kind[i] != kind) continue;
        hipError_t e = hipEventSynchronize(g_prof.stop[i]);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, g_prof.start[i], g_prof.stop[i]);
        if (e != hipSuccess) return hip_fail(e, "prof_read");
        if (durations_ms && c < max_n) durations_ms[c] = ms;
        ++c;
    }
    *n = c;
    return GPEED_OK;
}

int gpeed_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int gpeed_device_name(int index, char* buf, size_t len) {
    if (!buf || len == 0) return fail(GPEED_ERR_INVALID, "gpeed_device_name: empty buffer");
    hipDeviceProp_t prop;
    const char* name = "<none>";
    if (hipGetDeviceProperties(&prop, index) == hipSuccess) name = prop.name;
    std::snprintf(buf, len, "%s", name);
    return GPEED_OK;
}

int gpeed_add_f32(const float* a, const float* b, float* dst, int n) {
    if (n <= 0) return GPEED_OK;
    if (!a || !b || !dst) return fail(GPEED_ERR_INVALID, "gpeed_add_f32: null pointer");
    float *da = nullptr, *db = nullptr, *dd = nullptr;
    const size_t bytes = (size_t)n * sizeof(float);
    hipError_t e = hipMalloc(&da, bytes);
    if (e == hipSuccess) e = hipMalloc(&db, bytes);
    if (e == hipSuccess) e = hipMalloc(&dd, bytes);
    if (e == hipSuccess) e = hipMemcpy(da, a, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = gpeed::launch_add(da, db, dd, n, nullptr);
    if (e == hipSuccess) e = hipMemcpy(dst, dd, bytes, hipMemcpyDeviceToHost);
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(dd);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gpeed_add_f32");
}

int gpeed_stream_read(const void* p, size_t bytes, uint32_t* out, size_t out_words, gpeed_stream_t stream) {
    if (bytes == 0) return GPEED_OK;
    if (!p || !out || !aligned(p, 16)) return fail(GPEED_ERR_INVALID, "stream_read: null or misaligned pointer");
    if (bytes % 16) return fail(GPEED_ERR_INVALID, "stream_read: bytes is not a multiple of 16");
    if (out_words == 0 || out_words > 65535) return fail(GPEED_ERR_INVALID, "stream_read: out_words outside [1, 65535]");
    hipError_t e = gpeed::launch_stream_read(static_cast<const uint8_t*>(p), bytes, out, (int)out_words,
                                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "stream_read launch");
}

int gpeed_init(void) {
    if (gpeed_device_count() <= 0) return fail(GPEED_ERR_NO_DEVICE, "no HIP device");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    // the no-allocation entry point's scratch for this device (cleared on the
    // null stream, waited for here so that no later call depends on it)
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    void* p = nullptr;
    rc = noalloc_scratch(dev, nullptr, &p);
    if (rc) return rc;
    e = hipStreamSynchronize(nullptr);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gpeed_init: hipStreamSynchronize");
}

int gpeed_ws_status(void* ws, gpeed_stream_t stream) {
    if (!ws || !aligned(ws, 16)) return fail(GPEED_ERR_INVALID, "ws_status: null or misaligned workspace");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t flags = 0;
    hipError_t e = hipMemcpyAsync(&flags, ws, sizeof flags, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "ws_status");
    if (flags == 0) return GPEED_OK;
    e = gpeed::launch_fill_zero(ws, 16, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "ws_status: clearing the flags");
    std::string msg = "ws_status: workspace flagged:";
    if (flags & gpeed::kWsTicket) msg += " ticket count past the parts of a tile (not initialised or shared)";
    if (flags & gpeed::kWsTimeout) msg += " a wait for another workgroup's partial gave up";
    if (flags & gpeed::kWsBuckets) msg += " expert buckets break the router's invariants";
    return fail(GPEED_ERR_WS_STATE, msg);
}

int gpeed_ws_init(void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    if (ws_bytes == 0) return GPEED_OK;
    if (!ws || !aligned(ws, 16) || ws_bytes % 16)
        return fail(GPEED_ERR_INVALID, "ws_init: workspace null, not 16-byte aligned or not a multiple of 16 bytes");
    hipError_t e = gpeed::launch_fill_zero(ws, ws_bytes, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "ws_init launch");
}

int gpeed_moe_check_buckets(const int* eptr, const int* tok, int n_exp, int n_tok, int top_k) {
    if (!eptr || (!tok && n_tok > 0)) return fail(GPEED_ERR_INVALID, "moe_check_buckets: null pointer");
    if (n_exp < 1 || top_k < 1 || n_tok < 0) return fail(GPEED_ERR_INVALID, "moe_check_buckets: bad sizes");
    const long long n = (long long)n_tok * top_k;
    if (eptr[0] != 0) return fail(GPEED_ERR_INVALID, "moe_check_buckets: eptr[0] != 0");
    for (int e = 0; e < n_exp; ++e)
        if (eptr[e + 1] < eptr[e])
            return fail(GPEED_ERR_INVALID, "moe_check_buckets: eptr decreases at expert " + std::to_string(e));
    if (eptr[n_exp] != n) return fail(GPEED_ERR_INVALID, "moe_check_buckets: eptr[n_exp] != n_tok * top_k");
    std::vector<int> cnt((size_t)n_tok, 0);
    for (long long p = 0; p < n; ++p) {
        const int t = tok[p];
        if (t < 0 || t >= n_tok)
            return fail(GPEED_ERR_INVALID, "moe_check_buckets: tok[" + std::to_string(p) + "] out of range");
        ++cnt[(size_t)t];
    }
    for (int t = 0; t < n_tok; ++t)
        if (cnt[(size_t)t] != top_k)
            return fail(GPEED_ERR_INVALID, "moe_check_buckets: token " + std::to_string(t) + " appears " +
                                               std::to_string(cnt[(size_t)t]) + " times, not top_k");
    return GPEED_OK;
}

size_t gpeed_iq3xxs_row_bytes(int64_t in_dim) {
    if (in_dim <= 0 || in_dim % gpeed::kQK) return 0;
    return gpeed::iq3_row_bytes(in_dim);
}

size_t gpeed_iq3xxs_t64_bytes(uint64_t n_rows, int64_t in_dim) {
    if (in_dim <= 0 || in_dim % gpeed::kQK) return 0;
    return gpeed::t64_bytes(n_rows, in_dim);
}

int gpeed_dtype_block_size(int dtype) { return gpeed::rows_block_elems(dtype); }

size_t gpeed_dtype_row_bytes(int dtype, uint64_t n) {
    const int be = gpeed::rows_block_elems(dtype);
    if (be == 0 || n % (uint64_t)be) return 0;
    return (size_t)(n / (uint64_t)be) * gpeed::rows_block_bytes(dtype);
}

int gpeed_dequantize(int dtype, const void* src, float* dst, uint64_t n, gpeed_stream_t stream) {
    const int be = gpeed::rows_block_elems(dtype);
    if (be == 0) return fail(GPEED_ERR_UNIMPLEMENTED, "dequantize: unimplemented type " + std::to_string(dtype));
    if (n % (uint64_t)be)
        return fail(GPEED_ERR_NOT_MULTIPLE, "dequantize: element count not a multiple of block size");
    if (n == 0) return GPEED_OK;
    if (!src || !dst) return fail(GPEED_ERR_INVALID, "dequantize: null pointer");
    const size_t src_align = dtype == GPEED_DTYPE_F32 ? 4 : 2;
    if (!aligned(src, src_align) || !aligned(dst, 16))
        return fail(GPEED_ERR_INVALID, "dequantize: src must be element-aligned (2 bytes, F32 4) and dst 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = dtype == GPEED_DTYPE_IQ3_XXS
                       ? gpeed::launch_dequant_raw(static_cast<const uint8_t*>(src), dst, n, s)
                       : gpeed::launch_dequant_rows(dtype, static_cast<const uint8_t*>(src), dst, n, s);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "dequantize launch");
}

int gpeed_matmul_rows(int dtype, const void* w, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                      const float* X, int n_tok, float* Y, gpeed_stream_t stream) {
    if (n_tok <= 0 || out_dim <= 0) return GPEED_OK;  // weights.cpp:88
    const int be = gpeed::rows_block_elems(dtype);
    if (be == 0) return fail(GPEED_ERR_UNIMPLEMENTED, "matmul_rows: unimplemented type " + std::to_string(dtype));
    // the block formats' kernels walk rows in 32-weight runs; F32 rows (in
    // dot_f32's order) take any length, as the reference does (weights.cpp:92-94)
    if (in_dim <= 0 || in_dim % be || (dtype != GPEED_DTYPE_F32 && in_dim % 32))
        return fail(GPEED_ERR_UNALIGNED_ROW, "matmul_rows: row not block aligned (and a multiple of 32)");
    if (in_dim > (1 << 28) || n_tok > (1 << 24)) return fail(GPEED_ERR_INVALID, "matmul_rows: size too large");
    if (!w || !X || !Y) return fail(GPEED_ERR_INVALID, "matmul_rows: null pointer");
    if (row0 > n_rows || (uint64_t)out_dim > n_rows - row0)
        return fail(GPEED_ERR_INVALID, "matmul_rows: rows [row0, row0 + out_dim) outside the tensor");
    if (!aligned(w, dtype == GPEED_DTYPE_F32 ? 4 : 2) || !aligned(X, 16) || !aligned(Y, 4))
        return fail(GPEED_ERR_INVALID, "matmul_rows: w element-aligned, X 16-byte and Y 4-byte aligned");
    const size_t rb = gpeed_dtype_row_bytes(dtype, (uint64_t)in_dim);
    hipError_t e = gpeed::launch_matmul_rows(dtype, static_cast<const uint8_t*>(w), rb, row0, in_dim, out_dim, X,
                                             n_tok, Y, static_cast<hipStream_t>(stream));
    // (the type is known here, so the only invalid value left is a row
    // length whose per-wavefront row group passes the 2 GiB offset range)
    if (e == hipErrorInvalidValue)
        return fail(GPEED_ERR_INVALID, "matmul_rows: rows too long (one wavefront's rows exceed 2 GiB)");
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "matmul_rows launch");
}

int gpeed_codebook(int dtype, uint64_t* out, size_t n) {
    const size_t len = dtype == GPEED_DTYPE_IQ2_S ? 1024 : dtype == GPEED_DTYPE_IQ3_S ? 512
                                                      : dtype == GPEED_DTYPE_IQ3_XXS ? 256 : 0;
    if (len == 0) return fail(GPEED_ERR_UNIMPLEMENTED, "codebook: no grid for this type");
    if (!out || n < len) return fail(GPEED_ERR_INVALID, "codebook: buffer too small");
    for (size_t i = 0; i < len; ++i)
        out[i] = dtype == GPEED_DTYPE_IQ2_S ? gpeed::rows_iq2s_grid((int)i)
                 : dtype == GPEED_DTYPE_IQ3_S ? gpeed::rows_iq3s_grid((int)i)
                                              : gpeed::kIq3xxsGrid[i];
    return GPEED_OK;
}

int gpeed_t64_grid_table(uint16_t* out, size_t n) {
    if (!out || n < (size_t)gpeed::kGridTableBytes / 2)
        return fail(GPEED_ERR_INVALID, "t64_grid_table: buffer smaller than 32768 entries");
    gpeed::build_grid_table(out);
    return GPEED_OK;
}

uint32_t gpeed_t64_aux_word(uint32_t gguf_aux) { return gpeed::aux_to_t64(gguf_aux); }

static int check_tile_args(const void* a, const void* b, int64_t in_dim, const char* who) {
    if (in_dim <= 0 || in_dim % gpeed::kQK)
        return fail(GPEED_ERR_UNALIGNED_ROW, std::string(who) + ": row not block aligned");
    if (in_dim / gpeed::kQK > (1 << 24)) return fail(GPEED_ERR_INVALID, std::string(who) + ": in_dim too large");
    if (!a || !b) return fail(GPEED_ERR_INVALID, std::string(who) + ": null pointer");
    return GPEED_OK;
}

int gpeed_iq3xxs_tile(const void* raw, uint64_t n_rows, int64_t in_dim, void* t64,
                      gpeed_stream_t stream) {
    if (n_rows == 0) return GPEED_OK;
    int rc = check_tile_args(raw, t64, in_dim, "tile");
    if (rc) return rc;
    if (!aligned(raw, 2) || !aligned(t64, 16))
        return fail(GPEED_ERR_INVALID, "tile: raw must be 2-byte and t64 16-byte aligned");
    hipError_t e = gpeed::launch_tile(static_cast<const uint8_t*>(raw), n_rows, (int)in_dim,
                                      static_cast<uint8_t*>(t64), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "tile launch");
}

int gpeed_iq3xxs_untile(const void* t64, uint64_t n_rows, int64_t in_dim, void* raw,
                        gpeed_stream_t stream) {
    if (n_rows == 0) return GPEED_OK;
    int rc = check_tile_args(t64, raw, in_dim, "untile");
    if (rc) return rc;
    if (!aligned(raw, 2) || !aligned(t64, 16))
        return fail(GPEED_ERR_INVALID, "untile: raw must be 2-byte and t64 16-byte aligned");
    hipError_t e = gpeed::launch_untile(static_cast<const uint8_t*>(t64), n_rows, (int)in_dim,
                                        static_cast<uint8_t*>(raw), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "untile launch");
}

static bool dims_ok(int64_t in_dim) { return in_dim > 0 && in_dim % gpeed::kQK == 0 && in_dim <= (1 << 28); }
static size_t align256(size_t b) { return (b + 255) / 256 * 256; }
constexpr int kMaxTok = 8;

size_t gpeed_iq3xxs_act_bytes(int64_t in_dim, int n_tok) {
    if (!dims_ok(in_dim) || n_tok < 1 || n_tok > kMaxTok) return 0;
    return gpeed::act_bytes((int)in_dim, n_tok);
}

size_t gpeed_iq3xxs_gemv_ws_bytes(int n_tensors, int64_t in_dim, int64_t out_dim, int n_tok) {
    if (!dims_ok(in_dim) || out_dim <= 0 || out_dim > (1 << 30) || n_tensors < 1 || n_tensors > 2 ||
        n_tok < 1 || n_tok > kMaxTok)
        return 0;
    return gpeed::kWsHeader + gpeed::gemv_ws_bytes(n_tensors, (int)in_dim, (int)out_dim, n_tok);
}

// From this many tokens matmul runs the prefill GEMM (W read once) instead of
// ceil(n_tok / 8) GEMV passes (W read once per pass). Measured on MI355X over
// the 576..12288-row shapes of the decode mix and the dense MLP: from 9
// tokens (two GEMV passes) the GEMM is faster on every one of them.
constexpr int kMatmulGemmMinTok = 9;

int gpeed_iq3xxs_matmul_gemm_min_tok(void) { return kMatmulGemmMinTok; }

// Layout of a matvec / matmul workspace:
//   [0, kWsHeader)        header (error word)
//   [kWsHeader, front)    GEMV tickets and tagged partials, indexed so that a
//                         region sized for 8 tokens covers every token count
//   [front, ...)          per-call scratch: prepared activations of an 8-token
//                         pass, or the prefill GEMM's images and partials
// The front region of a matvec workspace is sized for one token; a matmul
// workspace's for 8, and its tail for the largest need of any token count
// up to the one it was sized for, so one buffer serves them all.
static size_t matmul_front(int64_t in_dim, int64_t out_dim, int n_tok) {
    return gpeed::kWsHeader + align256(gpeed::gemv_ws_bytes(1, (int)in_dim, (int)out_dim, n_tok));
}

static size_t matmul_tail(int64_t in_dim, int64_t out_dim, int n_tok, int num_cus) {
    if (n_tok < 2) return 0;
    size_t t = align256(gpeed::act_bytes((int)in_dim, n_tok < kMaxTok ? n_tok : kMaxTok));
    if (n_tok >= kMatmulGemmMinTok) {
        // matmul hands the GEMM fp32 X, which it tiles by 64 tokens at every
        // size. The split-K count (so the partials) depends only on the
        // token tile count and is not monotonic in it, while the images grow
        // with the tokens: the largest need of one tile count is at its last
        // token count, so every count's need is covered by taking the maximum
        // over the last count of each tile count below n_tok and n_tok
        // itself (the split count follows rounds of workgroups over the CUs,
        // so a larger tile count may split again).
        auto g = [&](int m) {
            return align256(gpeed::gemm_ws_bytes(m, (int)out_dim, (int)in_dim, 0, num_cus));
        };
        size_t best = g(n_tok);
        const int bm = gpeed::gemm_tile_m(n_tok, 0);
        for (int m = bm; m < n_tok; m += bm) {
            if (m < kMatmulGemmMinTok) continue;
            best = std::max(best, g(m));
        }
        t = std::max(t, best);
    }
    return t;
}

static size_t matmul_ws_bytes_cus(int64_t in_dim, int64_t out_dim, int n_tok, int num_cus) {
    if (n_tok < 1 || n_tok > (1 << 20) || !dims_ok(in_dim) || out_dim <= 0 || out_dim > (1 << 24)) return 0;
    if (n_tok == 1) return matmul_front(in_dim, out_dim, 1);
    return matmul_front(in_dim, out_dim, kMaxTok) + matmul_tail(in_dim, out_dim, n_tok, num_cus);
}

size_t gpeed_iq3xxs_matmul_ws_bytes(int64_t in_dim, int64_t out_dim, int n_tok) {
    if (n_tok < 1 || n_tok > (1 << 20) || !dims_ok(in_dim) || out_dim <= 0 || out_dim > (1 << 24)) return 0;
    if (n_tok == 1) return matmul_front(in_dim, out_dim, 1);
    const DeviceState* st = nullptr;
    if (device_state(&st)) return 0;
    return matmul_ws_bytes_cus(in_dim, out_dim, n_tok, st->num_cus);
}

size_t gpeed_iq3xxs_matmul_ws_bytes_for(int64_t in_dim, int64_t out_dim, int n_tok, int num_cus) {
    if (num_cus < 1 || num_cus > (1 << 16)) return 0;
    return matmul_ws_bytes_cus(in_dim, out_dim, n_tok, num_cus);
}

size_t gpeed_iq3xxs_matvec_ws_bytes(int64_t in_dim, int64_t out_dim) {
    return gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, 1);
}

static int check_mv_args(const void* w, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                         const void* x, const float* dst, const char* who) {
    if (in_dim <= 0 || in_dim % gpeed::kQK)
        return fail(GPEED_ERR_UNALIGNED_ROW, std::string(who) + ": row not block aligned");
    if (!dims_ok(in_dim) || out_dim > (1 << 30)) return fail(GPEED_ERR_INVALID, std::string(who) + ": size too large");
    if (!w || !x || !dst) return fail(GPEED_ERR_INVALID, std::string(who) + ": null pointer");
    if (row0 > n_rows || (uint64_t)out_dim > n_rows - row0)
        return fail(GPEED_ERR_INVALID, std::string(who) + ": rows out of range");
    return GPEED_OK;
}

static int check_act(const void* act, size_t act_bytes, int64_t in_dim, int n_tok, const char* who) {
    if (in_dim <= 0 || in_dim % gpeed::kQK)
        return fail(GPEED_ERR_UNALIGNED_ROW, std::string(who) + ": row not block aligned");
    if (!dims_ok(in_dim)) return fail(GPEED_ERR_INVALID, std::string(who) + ": in_dim too large");
    if (n_tok < 1 || n_tok > kMaxTok) return fail(GPEED_ERR_INVALID, std::string(who) + ": n_tok outside 1..8");
    if (!act || act_bytes < gpeed::act_bytes((int)in_dim, n_tok) || !aligned(act, 16))
        return fail(GPEED_ERR_WORKSPACE,
                    std::string(who) + ": activation buffer missing, misaligned or too small");
    return GPEED_OK;
}

int gpeed_iq3xxs_prep_act(const float* x, int64_t in_dim, int n_tok, void* act, size_t act_bytes,
                          gpeed_stream_t stream) {
    int rc = check_act(act, act_bytes, in_dim, n_tok, "prep_act");
    if (rc) return rc;
    if (!x || !aligned(x, 16)) return fail(GPEED_ERR_INVALID, "prep_act: x null or not 16-byte aligned");
    hipError_t e = gpeed::launch_prep_act(x, (int)in_dim, n_tok, static_cast<uint8_t*>(act),
                                          static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "prep_act launch");
}

int gpeed_iq3xxs_prep_swiglu(const float* g, const float* u, int64_t n, int n_tok, float limit, void* act,
                             size_t act_bytes, gpeed_stream_t stream) {
    int rc = check_act(act, act_bytes, n, n_tok, "prep_swiglu");
    if (rc) return rc;
    if (!g || !u || !aligned(g, 16) || !aligned(u, 16))
        return fail(GPEED_ERR_INVALID, "prep_swiglu: g/u null or not 16-byte aligned");
    hipError_t e = gpeed::launch_prep_swiglu(g, u, limit, (int)n, n_tok, static_cast<uint8_t*>(act),
                                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "prep_swiglu launch");
}

static int gemv_n(const void* const* w, float* const* dst, int n_tensors, uint64_t n_rows, uint64_t row0,
                  int in_dim, int out_dim, const void* act, int n_tok, void* ws, size_t ws_bytes,
                  gpeed_stream_t stream) {
    if (out_dim <= 0) return GPEED_OK;
    for (int i = 0; i < n_tensors; ++i) {
        int rc = check_mv_args(w[i], n_rows, row0, in_dim, out_dim, act, dst[i], "gemv");
        if (rc) return rc;
        if (!aligned(w[i], 16)) return fail(GPEED_ERR_INVALID, "gemv: T64 weights must be 16-byte aligned");
    }
    if (n_tok < 1 || n_tok > kMaxTok) return fail(GPEED_ERR_INVALID, "gemv: n_tok outside 1..8");
    if (!aligned(act, 16)) return fail(GPEED_ERR_WORKSPACE, "gemv: activation misaligned");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "gemv: row0 must be a multiple of 64 on the T64 layout");
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::kWsHeader + gpeed::gemv_ws_bytes(n_tensors, in_dim, out_dim, n_tok))
        return fail(GPEED_ERR_WORKSPACE, "gemv: workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    const uint8_t* wp[2] = {static_cast<const uint8_t*>(w[0]),
                            static_cast<const uint8_t*>(w[n_tensors > 1 ? 1 : 0])};
    float* yp[2] = {dst[0], dst[n_tensors > 1 ? 1 : 0]};
    hipError_t e = gpeed::launch_gemv_t64(wp, yp, n_tensors, in_dim, row0, out_dim, n_tok,
                                          static_cast<const uint8_t*>(act),
                                          static_cast<uint8_t*>(ws) + gpeed::kWsHeader, static_cast<uint32_t*>(ws),
                                          st->num_cus, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gemv launch");
}

int gpeed_iq3xxs_gemv_act(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                          const void* act, int n_tok, float* dst, void* ws, size_t ws_bytes,
                          gpeed_stream_t stream) {
    const void* w[1] = {w_t64};
    float* d[1] = {dst};
    return gemv_n(w, d, 1, n_rows, row0, in_dim, out_dim, act, n_tok, ws, ws_bytes, stream);
}

int gpeed_iq3xxs_gemv2_act(const void* w_a, const void* w_b, uint64_t n_rows, uint64_t row0,
                           int in_dim, int out_dim, const void* act, int n_tok, float* dst_a,
                           float* dst_b, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    const void* w[2] = {w_a, w_b};
    float* d[2] = {dst_a, dst_b};
    return gemv_n(w, d, 2, n_rows, row0, in_dim, out_dim, act, n_tok, ws, ws_bytes, stream);
}

static int gemv_x_n(const void* const* w, float* const* dst, int n_tensors, uint64_t n_rows, uint64_t row0,
                    int in_dim, int out_dim, const float* x, const float* x2, float lim, void* ws, size_t ws_bytes,
                    gpeed_stream_t stream, const char* who) {
    if (out_dim <= 0) return GPEED_OK;
    for (int i = 0; i < n_tensors; ++i) {
        int rc = check_mv_args(w[i], n_rows, row0, in_dim, out_dim, x, dst[i], who);
        if (rc) return rc;
        if (!aligned(w[i], 16)) return fail(GPEED_ERR_INVALID, std::string(who) + ": T64 weights must be 16-byte aligned");
    }
    if (!aligned(x, 16) || (x2 && !aligned(x2, 16)))
        return fail(GPEED_ERR_INVALID, std::string(who) + ": input not 16-byte aligned");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, std::string(who) + ": row0 must be a multiple of 64 on the T64 layout");
    if (!ws || !aligned(ws, 256) || ws_bytes < gpeed::kWsHeader + gpeed::gemv_ws_bytes(n_tensors, in_dim, out_dim, 1))
        return fail(GPEED_ERR_WORKSPACE, std::string(who) + ": workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    const uint8_t* wp[2] = {static_cast<const uint8_t*>(w[0]), static_cast<const uint8_t*>(w[n_tensors > 1 ? 1 : 0])};
    float* yp[2] = {dst[0], dst[n_tensors > 1 ? 1 : 0]};
    hipError_t e = gpeed::launch_gemv_x(wp, yp, n_tensors, in_dim, row0, out_dim, x, x2, lim,
                                        static_cast<uint8_t*>(ws) + gpeed::kWsHeader, static_cast<uint32_t*>(ws),
                                        st->num_cus, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, std::string(who + std::string(" launch")).c_str());
}

int gpeed_iq3xxs_gemv_x(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim, const float* x,
                        float* dst, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    const void* w[1] = {w_t64};
    float* d[1] = {dst};
    return gemv_x_n(w, d, 1, n_rows, row0, in_dim, out_dim, x, nullptr, 0.0f, ws, ws_bytes, stream, "gemv_x");
}

int gpeed_iq3xxs_gemv2_x(const void* w_a, const void* w_b, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                         const float* x, float* dst_a, float* dst_b, void* ws, size_t ws_bytes,
                         gpeed_stream_t stream) {
    const void* w[2] = {w_a, w_b};
    float* d[2] = {dst_a, dst_b};
    return gemv_x_n(w, d, 2, n_rows, row0, in_dim, out_dim, x, nullptr, 0.0f, ws, ws_bytes, stream, "gemv2_x");
}

int gpeed_iq3xxs_gemv_swiglu(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                             const float* g, const float* u, float limit, float* dst, void* ws, size_t ws_bytes,
                             gpeed_stream_t stream) {
    if (!u) return fail(GPEED_ERR_INVALID, "gemv_swiglu: null u");
    const void* w[1] = {w_t64};
    float* d[1] = {dst};
    return gemv_x_n(w, d, 1, n_rows, row0, in_dim, out_dim, g, u, limit, ws, ws_bytes, stream, "gemv_swiglu");
}

int gpeed_iq3xxs_matvec_heads(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int rows_per_head,
                              int n_heads, const float* x, float* dst, void* ws, size_t ws_bytes,
                              gpeed_stream_t stream) {
    if (n_heads <= 0 || rows_per_head <= 0) return GPEED_OK;
    if (rows_per_head % gpeed::kTileRows || row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "matvec_heads: rows_per_head and row0 must be multiples of 64");
    if ((int64_t)rows_per_head * n_heads > (1 << 30)) return fail(GPEED_ERR_INVALID, "matvec_heads: too many rows");
    const int out_dim = rows_per_head * n_heads;
    int rc = check_mv_args(w_t64, n_rows, row0, in_dim, out_dim, x, dst, "matvec_heads");
    if (rc) return rc;
    if (!aligned(w_t64, 16) || !aligned(x, 16))
        return fail(GPEED_ERR_INVALID, "matvec_heads: weights and x must be 16-byte aligned");
    if ((int64_t)n_heads * in_dim * 4 >= ((int64_t)1 << 31))
        return fail(GPEED_ERR_INVALID, "matvec_heads: inputs of 2 GiB or more");
    if (!ws || !aligned(ws, 256) || ws_bytes < gpeed::kWsHeader + gpeed::gemv_ws_bytes(1, in_dim, out_dim, 1))
        return fail(GPEED_ERR_WORKSPACE, "matvec_heads: workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    const hipError_t e = gpeed::launch_gemv_heads(static_cast<const uint8_t*>(w_t64), in_dim, row0, rows_per_head,
                                                  n_heads, x, dst, static_cast<uint8_t*>(ws) + gpeed::kWsHeader,
                                                  static_cast<uint32_t*>(ws), st->num_cus,
                                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "matvec_heads launch");
}

size_t gpeed_iq3xxs_dense_mlp_ws_bytes(int64_t hidden, int64_t inter) {
    if (hidden <= 0 || inter <= 0 || hidden % gpeed::kQK || inter % gpeed::kQK || hidden > (1 << 24) ||
        inter > (1 << 24))
        return 0;
    return gpeed::dense_mlp_ws_bytes((int)hidden, (int)inter);
}

int gpeed_iq3xxs_dense_mlp(const void* w_gate, const void* w_up, const void* w_down, int hidden, int inter,
                           const float* x, float limit, float* y, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    if (!w_gate || !w_up || !w_down || !x || !y) return fail(GPEED_ERR_INVALID, "dense_mlp: null pointer");
    const size_t need = gpeed_iq3xxs_dense_mlp_ws_bytes(hidden, inter);
    if (need == 0) return fail(GPEED_ERR_NOT_MULTIPLE, "dense_mlp: hidden and inter must be positive multiples of 256");
    if (!aligned(w_gate, 16) || !aligned(w_up, 16) || !aligned(w_down, 16) || !aligned(x, 16))
        return fail(GPEED_ERR_INVALID, "dense_mlp: weights and x must be 16-byte aligned");
    if (!ws || !aligned(ws, 256) || ws_bytes < need)
        return fail(GPEED_ERR_WORKSPACE, "dense_mlp: workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    const hipError_t e = gpeed::launch_dense_mlp(
        static_cast<const uint8_t*>(w_gate), static_cast<const uint8_t*>(w_up), static_cast<const uint8_t*>(w_down),
        hidden, inter, x, limit, y, static_cast<uint8_t*>(ws), st->num_cus, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "dense_mlp launch");
}

int gpeed_iq3xxs_matmul(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                        const float* X, int n_tok, float* Y, void* ws, size_t ws_bytes,
                        gpeed_stream_t stream) {
    if (n_tok <= 0 || out_dim <= 0) return GPEED_OK;  // weights.cpp:88
    if (n_tok == 1) return gpeed_iq3xxs_matvec(w_t64, n_rows, row0, in_dim, out_dim, X, Y, ws, ws_bytes, stream);
    int rc = check_mv_args(w_t64, n_rows, row0, in_dim, out_dim, X, Y, "matmul");
    if (rc) return rc;
    if (n_tok > (1 << 20)) return fail(GPEED_ERR_INVALID, "matmul: n_tok too large");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "matmul: row0 must be a multiple of 64 on the T64 layout");
    if (!aligned(w_t64, 16) || !aligned(X, 16)) return fail(GPEED_ERR_INVALID, "matmul: misaligned operand");
    const size_t need = gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, n_tok);
    if (!ws || !aligned(ws, 256) || ws_bytes < need)
        return fail(GPEED_ERR_WORKSPACE, "matmul: workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    uint8_t* base = static_cast<uint8_t*>(ws);
    uint32_t* err = static_cast<uint32_t*>(ws);
    uint8_t* tail = base + matmul_front(in_dim, out_dim, kMaxTok);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* w = static_cast<const uint8_t*>(w_t64);
    if (n_tok >= kMatmulGemmMinTok) {
        // one pass over W for all tokens (model_batch.cpp:30-95, 151-162 at
        // prefill chunk sizes)
        const hipError_t e = gpeed::launch_gemm(w, row0, in_dim, out_dim, X, 0, n_tok, Y, tail, err, st->num_cus, s);
        if (e == hipErrorInvalidValue) return fail(GPEED_ERR_INVALID, "matmul: tensor slice of 4 GiB or more");
        return e == hipSuccess ? GPEED_OK : hip_fail(e, "matmul gemm launch");
    }
    const uint8_t* wp[2] = {w, w};
    for (int t0 = 0; t0 < n_tok; t0 += kMaxTok) {
        const int nt = n_tok - t0 < kMaxTok ? n_tok - t0 : kMaxTok;
        float* yp[2] = {Y + (size_t)t0 * out_dim, Y + (size_t)t0 * out_dim};
        hipError_t e = gpeed::launch_prep_act(X + (size_t)t0 * in_dim, in_dim, nt, tail, s);
        if (e == hipSuccess)
            e = gpeed::launch_gemv_t64(wp, yp, 1, in_dim, row0, out_dim, nt, tail, base + gpeed::kWsHeader, err,
                                       st->num_cus, s);
        if (e != hipSuccess) return hip_fail(e, "matmul gemv launch");
    }
    return GPEED_OK;
}

int gpeed_iq3xxs_matvec(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                        const float* x, float* dst, void* ws, size_t ws_bytes,
                        gpeed_stream_t stream) {
    // one launch (activation prepared inside the GEMV), on the front region
    // of a matvec / matmul workspace
    if (out_dim <= 0) return GPEED_OK;  // weights.cpp:88
    if (in_dim <= 0 || in_dim % gpeed::kQK) return fail(GPEED_ERR_UNALIGNED_ROW, "matvec: row not block aligned");
    if (!dims_ok(in_dim)) return fail(GPEED_ERR_INVALID, "matvec: size too large");
    const size_t need = gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, 1);
    if (!ws || !aligned(ws, 256) || ws_bytes < need)
        return fail(GPEED_ERR_WORKSPACE, "matvec: workspace missing, misaligned or too small");
    return gpeed_iq3xxs_gemv_x(w_t64, n_rows, row0, in_dim, out_dim, x, dst, ws, need, stream);
}

int gpeed_iq3xxs_matvec_noalloc(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                                const float* x, float* dst, gpeed_stream_t stream) {
    if (out_dim <= 0) return GPEED_OK;  // weights.cpp:88
    int rc = check_mv_args(w_t64, n_rows, row0, in_dim, out_dim, x, dst, "matvec_noalloc");
    if (rc) return rc;
    if (!aligned(w_t64, 16) || !aligned(x, 16))
        return fail(GPEED_ERR_INVALID, "matvec_noalloc: weights and x must be 16-byte aligned");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "matvec_noalloc: row0 must be a multiple of 64 on the T64 layout");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    const size_t need =
        gpeed::kWsHeader + gpeed::gemv_ws_bytes_planned(1, in_dim, out_dim, 1, st->num_cus, gpeed::kPlanPrep);
    if (need > kNoAllocScratchBytes)
        return fail(GPEED_ERR_INVALID, "matvec_noalloc: this shape needs " + std::to_string(need) +
                                           " bytes of scratch, more than the fixed " +
                                           std::to_string(kNoAllocScratchBytes));
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    void* sp = nullptr;
    rc = noalloc_scratch(dev, s, &sp);
    if (rc) return rc;
    const uint8_t* wp[2] = {static_cast<const uint8_t*>(w_t64), static_cast<const uint8_t*>(w_t64)};
    float* yp[2] = {dst, dst};
    e = gpeed::launch_gemv_x(wp, yp, 1, in_dim, row0, out_dim, x, nullptr, 0.0f,
                             static_cast<uint8_t*>(sp) + gpeed::kWsHeader, static_cast<uint32_t*>(sp), st->num_cus,
                             s);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "matvec_noalloc launch");
}

int gpeed_iq3xxs_matvec_noalloc_status(gpeed_stream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(GPEED_ERR_INVALID, "device index out of range");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    void* sp = nullptr;
    int rc = noalloc_scratch(dev, s, &sp);
    if (rc) return rc;
    uint32_t flags = 0;
    e = hipMemcpyAsync(&flags, sp, sizeof flags, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "matvec_noalloc_status");
    if (flags == 0) return GPEED_OK;
    // a flagged call may have left tickets and tagged partials behind: the
    // whole array starts again from zero
    rc = noalloc_clear(sp, s);
    if (rc) return rc;
    std::string msg = "matvec_noalloc_status: scratch flagged:";
    if (flags & gpeed::kWsTicket) msg += " ticket count past the parts of a tile (calls overlapped)";
    if (flags & gpeed::kWsTimeout) msg += " a wait for another workgroup's partial gave up";
    return fail(GPEED_ERR_WS_STATE, msg + "; cleared");
}

int gpeed_iq3xxs_matvec_noalloc_poke(size_t offset, uint32_t value) {
    if (offset % 4 || offset + 4 > kNoAllocScratchBytes)
        return fail(GPEED_ERR_INVALID, "matvec_noalloc_poke: offset not a word inside the scratch");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(GPEED_ERR_INVALID, "device index out of range");
    void* sp = nullptr;
    const int rc = noalloc_scratch(dev, nullptr, &sp);
    if (rc) return rc;
    e = hipMemcpy(static_cast<uint8_t*>(sp) + offset, &value, sizeof value, hipMemcpyHostToDevice);
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "matvec_noalloc_poke");
}

size_t gpeed_moe_route_ws_bytes(int n_tok, int n_exp, int top_k) {
    if (n_tok < 1 || n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp) return 0;
    return gpeed::moe_route_ws_bytes(n_tok, top_k);
}

int gpeed_moe_route(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                    float routed_scale, int norm_topk, int* eptr, int* tok, float* wt, int* sel, void* ws,
                    size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0) return GPEED_OK;
    if (n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp)
        return fail(GPEED_ERR_UNIMPLEMENTED, "moe_route: needs 1 <= top_k <= min(32, n_exp), n_exp <= 1024");
    if (mode != 0 && mode != 1) return fail(GPEED_ERR_INVALID, "moe_route: mode must be 0 (sigmoid) or 1 (softmax)");
    if ((int64_t)n_tok * top_k > (1 << 24)) return fail(GPEED_ERR_INVALID, "moe_route: too many assignments");
    if (!logits || !eptr || !tok || !wt) return fail(GPEED_ERR_INVALID, "moe_route: null pointer");
    if (!ws || !aligned(ws, 256) || ws_bytes < gpeed::moe_route_ws_bytes(n_tok, top_k))
        return fail(GPEED_ERR_WORKSPACE, "moe_route: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_moe_route(logits, n_tok, n_exp, top_k, mode, bias, routed_scale, norm_topk, eptr,
                                           tok, wt, sel, static_cast<uint8_t*>(ws),
                                           static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "moe_route launch");
}

size_t gpeed_iq3xxs_moe_ws_bytes(int n_tok, int n_exp, int top_k, int hidden, int inter) {
    if (n_tok < 1 || n_tok > 8192 || n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp) return 0;
    if (!dims_ok(hidden) || !dims_ok(inter)) return 0;
    return gpeed::moe_ws_bytes(n_tok, n_exp, top_k, hidden, inter);
}

int gpeed_iq3xxs_moe_experts(const void* w_gate, const void* w_up, const void* w_down, int n_exp, int hidden,
                             int inter, const float* X, int n_tok, int top_k, const int* eptr, const int* tok,
                             const float* wt, float swiglu_limit, float* Y, void* ws, size_t ws_bytes,
                             gpeed_stream_t stream) {
    if (n_tok <= 0) return GPEED_OK;
    if (hidden <= 0 || hidden % gpeed::kQK || inter <= 0 || inter % gpeed::kQK)
        return fail(GPEED_ERR_UNALIGNED_ROW, "moe_experts: row not block aligned");
    if (!dims_ok(hidden) || !dims_ok(inter)) return fail(GPEED_ERR_INVALID, "moe_experts: size too large");
    if (n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp)
        return fail(GPEED_ERR_UNIMPLEMENTED, "moe_experts: needs 1 <= top_k <= min(32, n_exp), n_exp <= 1024");
    if (n_tok > 8192) return fail(GPEED_ERR_INVALID, "moe_experts: at most 8192 tokens per call");
    if (!w_gate || !w_up || !w_down || !X || !eptr || !tok || !wt || !Y)
        return fail(GPEED_ERR_INVALID, "moe_experts: null pointer");
    if (!aligned(w_gate, 16) || !aligned(w_up, 16) || !aligned(w_down, 16) || !aligned(X, 16) || !aligned(Y, 16))
        return fail(GPEED_ERR_INVALID, "moe_experts: weights, X and Y must be 16-byte aligned");
    if (!ws || !aligned(ws, 256) || ws_bytes < gpeed::moe_ws_bytes(n_tok, n_exp, top_k, hidden, inter))
        return fail(GPEED_ERR_WORKSPACE, "moe_experts: workspace missing, misaligned or too small");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    hipError_t e = gpeed::launch_moe_experts(
        static_cast<const uint8_t*>(w_gate), static_cast<const uint8_t*>(w_up), static_cast<const uint8_t*>(w_down),
        n_exp, hidden, inter, X, n_tok, top_k, eptr, tok, wt, swiglu_limit, Y, static_cast<uint8_t*>(ws),
        st->num_cus, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "moe_experts launch");
}

size_t gpeed_iq3xxs_moe_batch_ws_bytes(int n_tok, int n_exp, int top_k, int hidden, int inter, int shared) {
    if (n_tok < 1 || n_tok > 8192 || n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp) return 0;
    if ((int64_t)n_tok * top_k > (1 << 24)) return 0;
    if (!dims_ok(hidden) || !dims_ok(inter)) return 0;
    const DeviceState* st = nullptr;
    if (device_state(&st)) return 0;
    return gpeed::moe_batch_ws_bytes(n_tok, n_exp, top_k, hidden, inter, shared ? 1 : 0, st->num_cus);
}

int gpeed_iq3xxs_moe_batch(const float* logits, int n_tok, int n_exp, int top_k, int mode, const float* bias,
                           float routed_scale, int norm_topk, const void* w_gate, const void* w_up,
                           const void* w_down, const void* w_gate_sh, const void* w_up_sh, const void* w_down_sh,
                           int hidden, int inter, const float* X, float swiglu_limit, float* Y, int* eptr, int* tok,
                           float* wt, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0) return GPEED_OK;
    if (hidden <= 0 || hidden % gpeed::kQK || inter <= 0 || inter % gpeed::kQK)
        return fail(GPEED_ERR_UNALIGNED_ROW, "moe_batch: row not block aligned");
    if (!dims_ok(hidden) || !dims_ok(inter)) return fail(GPEED_ERR_INVALID, "moe_batch: size too large");
    if (n_exp < 1 || n_exp > 1024 || top_k < 1 || top_k > 32 || top_k > n_exp)
        return fail(GPEED_ERR_UNIMPLEMENTED, "moe_batch: needs 1 <= top_k <= min(32, n_exp), n_exp <= 1024");
    if (mode != 0 && mode != 1) return fail(GPEED_ERR_INVALID, "moe_batch: mode must be 0 (sigmoid) or 1 (softmax)");
    if (n_tok > 8192) return fail(GPEED_ERR_INVALID, "moe_batch: at most 8192 tokens per call");
    if (!logits || !w_gate || !w_up || !w_down || !X || !Y) return fail(GPEED_ERR_INVALID, "moe_batch: null pointer");
    const bool sh = w_gate_sh || w_up_sh || w_down_sh;
    if (sh && !(w_gate_sh && w_up_sh && w_down_sh))
        return fail(GPEED_ERR_INVALID, "moe_batch: give all three shared-expert tensors or none");
    for (const void* p : {w_gate, w_up, w_down, (const void*)X, (const void*)Y, w_gate_sh, w_up_sh, w_down_sh})
        if (p && !aligned(p, 16)) return fail(GPEED_ERR_INVALID, "moe_batch: weights, X and Y must be 16-byte aligned");
    const DeviceState* st = nullptr;
    int rc = device_state(&st);
    if (rc) return rc;
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::moe_batch_ws_bytes(n_tok, n_exp, top_k, hidden, inter, sh ? 1 : 0, st->num_cus))
        return fail(GPEED_ERR_WORKSPACE, "moe_batch: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_moe_batch(
        logits, n_tok, n_exp, top_k, mode, bias, routed_scale, norm_topk, static_cast<const uint8_t*>(w_gate),
        static_cast<const uint8_t*>(w_up), static_cast<const uint8_t*>(w_down), static_cast<const uint8_t*>(w_gate_sh),
        static_cast<const uint8_t*>(w_up_sh), static_cast<const uint8_t*>(w_down_sh), hidden, inter, X, swiglu_limit,
        Y, eptr, tok, wt, static_cast<uint8_t*>(ws), st->num_cus, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "moe_batch launch");
}

size_t gpeed_iq3xxs_gemm_ws_bytes(int64_t n_tok, int64_t in_dim, int64_t out_dim, int x_dtype) {
    if (n_tok < 1 || n_tok > (1 << 20) || !dims_ok(in_dim) || out_dim < 1 || out_dim > (1 << 24) ||
        (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16))
        return 0;
    const DeviceState* st = nullptr;
    if (device_state(&st)) return 0;
    return gpeed::kWsHeader +
           gpeed::gemm_ws_bytes((int)n_tok, (int)out_dim, (int)in_dim, x_dtype == GPEED_X_BF16, st->num_cus);
}

int gpeed_iq3xxs_gemm(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim, const void* X,
                      int x_dtype, int n_tok, float* Y, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0 || out_dim <= 0) return GPEED_OK;  // weights.cpp:88
    int rc = check_mv_args(w_t64, n_rows, row0, in_dim, out_dim, X, Y, "gemm");
    if (rc) return rc;
    if (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16) return fail(GPEED_ERR_INVALID, "gemm: x_dtype");
    if (n_tok > (1 << 20)) return fail(GPEED_ERR_INVALID, "gemm: n_tok too large");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "gemm: row0 must be a multiple of 64 on the T64 layout");
    if (!aligned(w_t64, 16) || !aligned(X, 16)) return fail(GPEED_ERR_INVALID, "gemm: misaligned operand");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::kWsHeader + gpeed::gemm_ws_bytes(n_tok, out_dim, in_dim, x_dtype == GPEED_X_BF16, st->num_cus))
        return fail(GPEED_ERR_WORKSPACE, "gemm: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_gemm(static_cast<const uint8_t*>(w_t64), row0, in_dim, out_dim, X,
                                      x_dtype == GPEED_X_BF16, n_tok, Y, static_cast<uint8_t*>(ws) + gpeed::kWsHeader,
                                      static_cast<uint32_t*>(ws), st->num_cus, static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue) return fail(GPEED_ERR_INVALID, "gemm: tensor slice of 4 GiB or more");
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gemm launch");
}

size_t gpeed_iq3xxs_gemm2_ws_bytes(int64_t n_tok, int64_t in_dim, int64_t out_a, int64_t out_b, int x_dtype) {
    if (n_tok < 1 || n_tok > (1 << 20) || !dims_ok(in_dim) || out_a < 0 || out_b < 0 || out_a + out_b < 1 ||
        out_a > (1 << 24) || out_b > (1 << 24) || (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16))
        return 0;
    const DeviceState* st = nullptr;
    if (device_state(&st)) return 0;
    return gpeed::kWsHeader + gpeed::gemm2_ws_bytes((int)n_tok, (int)out_a, (int)out_b, (int)in_dim,
                                                    x_dtype == GPEED_X_BF16, st->num_cus);
}

int gpeed_iq3xxs_gemm2(const void* w_a, uint64_t n_rows_a, uint64_t row0_a, int out_a, const void* w_b,
                       uint64_t n_rows_b, uint64_t row0_b, int out_b, int in_dim, const void* X, int x_dtype,
                       int n_tok, float* Y_a, float* Y_b, void* ws, size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0 || (out_a <= 0 && out_b <= 0)) return GPEED_OK;  // weights.cpp:88
    if (out_a <= 0 || out_b <= 0) {  // one tensor left: the ordinary GEMM
        const bool a = out_a > 0;
        return gpeed_iq3xxs_gemm(a ? w_a : w_b, a ? n_rows_a : n_rows_b, a ? row0_a : row0_b, in_dim,
                                 a ? out_a : out_b, X, x_dtype, n_tok, a ? Y_a : Y_b, ws, ws_bytes, stream);
    }
    int rc = check_mv_args(w_a, n_rows_a, row0_a, in_dim, out_a, X, Y_a, "gemm2");
    if (rc) return rc;
    rc = check_mv_args(w_b, n_rows_b, row0_b, in_dim, out_b, X, Y_b, "gemm2");
    if (rc) return rc;
    if (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16) return fail(GPEED_ERR_INVALID, "gemm2: x_dtype");
    if (n_tok > (1 << 20)) return fail(GPEED_ERR_INVALID, "gemm2: n_tok too large");
    if (row0_a % gpeed::kTileRows || row0_b % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "gemm2: row0 must be a multiple of 64 on the T64 layout");
    if (!aligned(w_a, 16) || !aligned(w_b, 16) || !aligned(X, 16))
        return fail(GPEED_ERR_INVALID, "gemm2: misaligned operand");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::kWsHeader +
                       gpeed::gemm2_ws_bytes(n_tok, out_a, out_b, in_dim, x_dtype == GPEED_X_BF16, st->num_cus))
        return fail(GPEED_ERR_WORKSPACE, "gemm2: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_gemm2(static_cast<const uint8_t*>(w_a), row0_a, out_a,
                                       static_cast<const uint8_t*>(w_b), row0_b, out_b, in_dim, X,
                                       x_dtype == GPEED_X_BF16, n_tok, Y_a, Y_b,
                                       static_cast<uint8_t*>(ws) + gpeed::kWsHeader, static_cast<uint32_t*>(ws),
                                       st->num_cus, static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue) return fail(GPEED_ERR_INVALID, "gemm2: tensor slice of 4 GiB or more");
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gemm2 launch");
}

int gpeed_iq3xxs_gemm_swiglu(const void* w_t64, uint64_t n_rows, uint64_t row0, int in_dim, int out_dim,
                             const float* G, const float* U, float limit, int n_tok, float* Y, void* ws,
                             size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0 || out_dim <= 0) return GPEED_OK;
    int rc = check_mv_args(w_t64, n_rows, row0, in_dim, out_dim, G, Y, "gemm_swiglu");
    if (rc) return rc;
    if (!U) return fail(GPEED_ERR_INVALID, "gemm_swiglu: null pointer");
    if (n_tok > (1 << 20)) return fail(GPEED_ERR_INVALID, "gemm_swiglu: n_tok too large");
    if (row0 % gpeed::kTileRows)
        return fail(GPEED_ERR_LAYOUT, "gemm_swiglu: row0 must be a multiple of 64 on the T64 layout");
    if (!aligned(w_t64, 16) || !aligned(G, 16) || !aligned(U, 16))
        return fail(GPEED_ERR_INVALID, "gemm_swiglu: misaligned operand");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::kWsHeader + gpeed::gemm_ws_bytes(n_tok, out_dim, in_dim, 0, st->num_cus))
        return fail(GPEED_ERR_WORKSPACE, "gemm_swiglu: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_gemm(static_cast<const uint8_t*>(w_t64), row0, in_dim, out_dim, G, 0, n_tok, Y,
                                      static_cast<uint8_t*>(ws) + gpeed::kWsHeader, static_cast<uint32_t*>(ws),
                                      st->num_cus, static_cast<hipStream_t>(stream), U, limit);
    if (e == hipErrorInvalidValue) return fail(GPEED_ERR_INVALID, "gemm_swiglu: tensor slice of 4 GiB or more");
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "gemm_swiglu launch");
}

size_t gpeed_iq3xxs_mlp_gemm_ws_bytes(int64_t n_tok, int64_t hidden, int64_t inter, int x_dtype, int n_extra,
                                      const int* extra_out) {
    if (n_tok < 1 || n_tok > (1 << 20) || !dims_ok(hidden) || !dims_ok(inter) || hidden > (1 << 24) ||
        inter > (1 << 24) || (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16) || n_extra < 0 || n_extra > 2 ||
        (n_extra > 0 && !extra_out))
        return 0;
    const int e1 = n_extra > 0 ? extra_out[0] : 0, e2 = n_extra > 1 ? extra_out[1] : 0;
    if (e1 < 0 || e2 < 0 || e1 > (1 << 24) || e2 > (1 << 24)) return 0;
    const DeviceState* st = nullptr;
    if (device_state(&st)) return 0;
    return gpeed::kWsHeader + gpeed::mlp_gemm_ws_bytes((int)hidden, (int)inter, (int)n_tok,
                                                       x_dtype == GPEED_X_BF16, e1, e2, st->num_cus);
}

int gpeed_iq3xxs_mlp_gemm(const void* w_gate, const void* w_up, const void* w_down, int hidden, int inter,
                          const void* X, int x_dtype, int n_tok, float swiglu_limit, float* Y, int n_extra,
                          const void* const* extra_w, const int* extra_out, float* const* extra_Y, void* ws,
                          size_t ws_bytes, gpeed_stream_t stream) {
    if (n_tok <= 0) return GPEED_OK;  // weights.cpp:88
    int rc = check_mv_args(w_gate, (uint64_t)inter, 0, hidden, inter, X, Y, "mlp_gemm");
    if (!rc) rc = check_mv_args(w_up, (uint64_t)inter, 0, hidden, inter, X, Y, "mlp_gemm");
    if (!rc) rc = check_mv_args(w_down, (uint64_t)hidden, 0, inter, hidden, X, Y, "mlp_gemm");
    if (rc) return rc;
    if (x_dtype != GPEED_X_F32 && x_dtype != GPEED_X_BF16) return fail(GPEED_ERR_INVALID, "mlp_gemm: x_dtype");
    if (n_tok > (1 << 20)) return fail(GPEED_ERR_INVALID, "mlp_gemm: n_tok too large");
    if (n_extra < 0 || n_extra > 2 || (n_extra > 0 && (!extra_w || !extra_out || !extra_Y)))
        return fail(GPEED_ERR_INVALID, "mlp_gemm: extra tensors (0 to 2, with their outputs)");
    const void* ew[2] = {nullptr, nullptr};
    int eo[2] = {0, 0};
    float* ey[2] = {nullptr, nullptr};
    for (int i = 0; i < n_extra; ++i) {
        if (extra_out[i] <= 0) continue;  // nothing to compute
        rc = check_mv_args(extra_w[i], (uint64_t)extra_out[i], 0, hidden, extra_out[i], X, extra_Y[i], "mlp_gemm");
        if (rc) return rc;
        if (!aligned(extra_w[i], 16)) return fail(GPEED_ERR_INVALID, "mlp_gemm: misaligned operand");
        ew[i] = extra_w[i];
        eo[i] = extra_out[i];
        ey[i] = extra_Y[i];
    }
    if (!aligned(w_gate, 16) || !aligned(w_up, 16) || !aligned(w_down, 16) || !aligned(X, 16))
        return fail(GPEED_ERR_INVALID, "mlp_gemm: misaligned operand");
    const DeviceState* st = nullptr;
    rc = device_state(&st);
    if (rc) return rc;
    if (!ws || !aligned(ws, 256) ||
        ws_bytes < gpeed::kWsHeader + gpeed::mlp_gemm_ws_bytes(hidden, inter, n_tok, x_dtype == GPEED_X_BF16,
                                                                eo[0], eo[1], st->num_cus))
        return fail(GPEED_ERR_WORKSPACE, "mlp_gemm: workspace missing, misaligned or too small");
    hipError_t e = gpeed::launch_mlp_gemm(
        static_cast<const uint8_t*>(w_gate), static_cast<const uint8_t*>(w_up), static_cast<const uint8_t*>(w_down),
        hidden, inter, X, x_dtype == GPEED_X_BF16, n_tok, swiglu_limit, Y, static_cast<const uint8_t*>(ew[0]), eo[0],
        ey[0], static_cast<const uint8_t*>(ew[1]), eo[1], ey[1], static_cast<uint8_t*>(ws) + gpeed::kWsHeader,
        static_cast<uint32_t*>(ws), st->num_cus, static_cast<hipStream_t>(stream));
    if (e == hipErrorInvalidValue) return fail(GPEED_ERR_INVALID, "mlp_gemm: tensor of 4 GiB or more");
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "mlp_gemm launch");
}

int gpeed_iq3xxs_matvec_raw(const void* w_gguf, uint64_t n_rows, uint64_t row0, int in_dim,
                            int out_dim, const float* x, float* dst, gpeed_stream_t stream) {
    if (out_dim <= 0) return GPEED_OK;
    int rc = check_mv_args(w_gguf, n_rows, row0, in_dim, out_dim, x, dst, "matvec_raw");
    if (rc) return rc;
    if (!aligned(w_gguf, 2) || !aligned(x, 16))
        return fail(GPEED_ERR_INVALID, "matvec_raw: w must be 2-byte and x 16-byte aligned");
    hipError_t e = gpeed::launch_matvec_raw(static_cast<const uint8_t*>(w_gguf), in_dim, row0, out_dim,
                                            x, dst, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GPEED_OK : hip_fail(e, "matvec_raw launch");
}

}  // extern "C"
