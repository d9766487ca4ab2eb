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
// Prepared activation ("act"): for each 256-element block, the fp16 hi/lo
// MFMA A operand of the block scaled by a power of two (1 KiB), then one fp32
// unscale per block. act_bytes() is its size, rounded to 256 bytes.
size_t act_bytes(int in_dim);
hipError_t launch_prep_act(const float* x, int in_dim, uint8_t* act, hipStream_t s);
// Same for h = silu(min(g,lim)) * clamp(u,-lim,lim) (SwiGLU epilogue).
hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int in_dim, uint8_t* act,
                              hipStream_t s);
// y_i[j] = sum_k W_i[row0+j][k] x[k] over the T16 payloads of n_tensors
// (1 or 2) same-shape tensors sharing one prepared activation.
hipError_t launch_matvec_t16(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                             unsigned long long row0, int out_dim, const uint8_t* act,
                             const void* grid_table, int num_cus, hipStream_t s);
// Same product straight from GGUF rows (VALU decode, no repacking).
hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* dst, int n, hipStream_t s);

}  // namespace gpeed
