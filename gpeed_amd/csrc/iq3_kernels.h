// Kernel launchers shared between the .hip translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gpeed {

// quant.cpp:186-210 over n/256 raw GGUF blocks -> fp32 (bit-exact).
hipError_t launch_dequant_raw(const uint8_t* src, float* dst, unsigned long long n, hipStream_t s);
// GGUF rows -> T16 (tiled) and back. n_rows rows of in_dim weights.
hipError_t launch_tile(const uint8_t* raw, unsigned long long n_rows, int in_dim, uint8_t* t16,
                       hipStream_t s);
hipError_t launch_untile(const uint8_t* t16, unsigned long long n_rows, int in_dim, uint8_t* raw,
                         hipStream_t s);
// fp32 activations [n_tok][in_dim] -> fp16 hi/lo A-operand layout with a
// power-of-two scale per token (xscale[t] = 2^-e_t).
hipError_t launch_prep_x(const float* x, int n_tok, int in_dim, uint32_t* x16, float* xscale,
                         hipStream_t s);
size_t prep_x_bytes(int n_tok, int in_dim);
// Same layout for h = silu(min(g,lim)) * clamp(u,-lim,lim) (SwiGLU epilogue).
hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int n_tok, int in_dim,
                              uint32_t* x16, float* xscale, hipStream_t s);
// y[j] = sum_k W[row0+j][k] x[k] from the T16 payload (one token).
hipError_t launch_matvec_t16(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const uint32_t* x16, const float* xscale, float* y,
                             const void* sign_table, hipStream_t s);
// Same product straight from GGUF rows (VALU decode, no repacking).
hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* dst, int n, hipStream_t s);

}  // namespace gpeed
