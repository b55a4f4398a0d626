// Internal definitions shared by the HIP translation units of the BitLinear
// backend (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

// Activation workspace written by the quantizer for each token (row of
// act_row_bytes(K) bytes, 256-byte aligned):
//   [0, 4*S)            int32 sum of the token's int8 values per 1024-column
//                       slice (S = ceil(K/1024)), used for w = code - 1
//   [nib_off, +K)       split-nibble copy for the v_dot8 GEMV: per 16 columns
//                       four dwords {lo4(even cols), lo4(odd), hi4(even),
//                       hi4(odd)}; nibble n of "even" is column 2n
//   [perm_off, +K)      int8 copy for the MFMA GEMM: per 16 columns, byte
//                       4k+b holds column 4b+k (the order in which a packed
//                       dword decodes to four int8 dwords)
namespace bm {

constexpr int kSlice = 1024;  // scalar T-MAC block: 256 groups of 4 columns

__host__ __device__ inline int slices_of(int K) { return (K + kSlice - 1) / kSlice; }
__host__ __device__ inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
__host__ __device__ inline size_t act_nib_off(int K) { return align_up((size_t)slices_of(K) * 4, 64); }
__host__ __device__ inline size_t act_perm_off(int K) { return act_nib_off(K) + align_up((size_t)K, 64); }
__host__ __device__ inline size_t act_row_bytes(int K) {
  return align_up(act_perm_off(K) + align_up((size_t)K, 64), 256);
}

}  // namespace bm

#define BM_HIP_CHECK_RET(expr, ret)                                            \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      bm_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),     \
                   __FILE__, __LINE__);                                        \
      return ret;                                                              \
    }                                                                          \
  } while (0)

extern "C" void bm_set_error(const char *fmt, ...);

// Kernel launchers (bm_kernels.hip).  All return hipSuccess or the launch
// error; shapes are validated by the callers.
namespace bm {

// nibbles = false leaves the split-nibble part of the workspace unwritten
// (for products that read only the permuted bytes: product_reads_nibbles);
// fast = true sums the squares as a pairwise tree for n = 1024, 2048, 4096
// (fast mode; other n keep the sequential sum)
hipError_t launch_quantize(const float *x, int M, int n, int x_stride,
                           const float *gamma, float *x_norm, int8_t *xq,
                           int quant_stride, float *scale_x, uint8_t *act,
                           hipStream_t s, bool nibbles = true, bool fast = false);
hipError_t launch_prep_i8(const int8_t *xq, int M, int ldx, int K, uint8_t *act, bool nib,
                          hipStream_t s);
// Output modes of the products: fp32 store, fp32 accumulate (out += o, the
// residual add of src/model.c:1214-1215, 1139-1142), exact int32 totals.
enum { MODE_STORE = 0, MODE_ACC = 1, MODE_I32 = 2 };

// fp32 output with the scalar 1024-column epilogue; inv[m] computed from
// scale_x[m] and w_scale (unused for MODE_I32)
hipError_t launch_product(const uint8_t *act, const float *scale_x, int M,
                          const uint8_t *packed, int N, int K, float w_scale,
                          bool canonical, void *out, int mode, hipStream_t s);
// int8 activations straight into the few-token MFMA product (exact int32
// totals, no workspace): hipErrorNotSupported unless the product takes that
// kernel and every row of xq starts on 16 bytes
hipError_t launch_small_i8(const int8_t *xq, int M, int ldx, int K, const uint8_t *packed, int N,
                           bool canonical, int32_t *out, hipStream_t s);
bool product_needs_generic(int M, int K);
bool product_reads_nibbles(int M, int N, int K);
hipError_t launch_generic(const int8_t *xq, int ldx, const float *scale_x,
                          int M, const uint8_t *packed, int N, int K,
                          float w_scale, void *out, int mode, hipStream_t s);
hipError_t launch_rms_norm(const float *x, int n, const float *gamma,
                           float *out, float *max_out, hipStream_t s);
hipError_t launch_canonicalize(uint8_t *p, size_t bytes, hipStream_t s);
// x[i] += o[i] for i < n, one fp32 rounding each (the residual connection,
// src/model.c:1140-1142)
hipError_t launch_residual_add(float *x, const float *o, size_t n, hipStream_t s);

// Host -> device copy of caller memory through the library's own pinned
// staging (bm_runtime.hip); enqueued on s, complete once s is.
hipError_t upload(void *dst, const void *src, size_t bytes, hipStream_t s);

// One BitLinear call (RMSNorm + int8 + GEMV, canonical weights) on mapped
// host memory in a single launch of dropin_blocks(N, K) blocks
// (bm_decode.hip): x, out, and the copies xn (normalized input) and xq
// (int8 input) are mapped host buffers; block b writes seq to the
// host-mapped word flags[b] once its results are visible to the host.
// Needs rows_fit(K).
bool rows_fit(int K);
int dropin_blocks(int N, int K);
hipError_t launch_dropin(const float *x, int K, const float *gamma, const uint8_t *W, int N,
                         float w_scale, float *out, float *xn, int8_t *xq, unsigned *flags,
                         unsigned seq, hipStream_t s);
// One BitLinear call of one token on device memory in a single launch of
// the same kernel (canonical weights): out, the int8 input xq and scale_x.
hipError_t launch_rows_dev(const float *x, int K, const float *gamma, const uint8_t *W, int N,
                           float w_scale, float *out, int8_t *xq, float *scale_x, hipStream_t s);
// int8-input products with exact int32 totals, one launch, no workspace:
// each block row (token) turns its int8 values into split nibbles itself.
bool rows_i8_fit(int K);
hipError_t launch_rows_i8(const int8_t *xq, int M, int ldx, int K, const uint8_t *W, int N,
                          bool canonical, int32_t *out, hipStream_t s);

}  // namespace bm
