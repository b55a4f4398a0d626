// Device helpers shared by the kernel translation units.
#pragma once

#include "bm_common.h"
#include "bm_fp.h"

namespace bm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// 16-byte streaming load (nontemporal: weights are read once per pass)
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const v4i v = __builtin_nontemporal_load((const v4i*)p);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

__device__ __forceinline__ uint32_t canon_codes(uint32_t p) {
  // field 11 -> 10: clear the low bit where both bits are set
  return p - (((p >> 1) & p) & 0x55555555u);
}

// ---------------------------------------------------------------------------
// Activation workspace writers
// ---------------------------------------------------------------------------

// 16 int8 values of columns 16g..16g+15 -> split nibbles + permuted int8
__device__ __forceinline__ void write_act_group(uint8_t* __restrict__ act_row, int K, int g,
                                                const int (&q)[16]) {
  uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int xe = q[2 * n], xo = q[2 * n + 1];
    le |= (uint32_t)(xe & 15) << (4 * n);
    lo |= (uint32_t)(xo & 15) << (4 * n);
    he |= (uint32_t)((xe >> 4) & 15) << (4 * n);
    ho |= (uint32_t)((xo >> 4) & 15) << (4 * n);
  }
  uint4 nib = make_uint4(le, lo, he, ho);
  *(uint4*)(act_row + act_nib_off(K) + 16 * (size_t)g) = nib;
  uint32_t pm[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    pm[k] = (uint32_t)(q[k] & 255) | ((uint32_t)(q[4 + k] & 255) << 8) |
            ((uint32_t)(q[8 + k] & 255) << 16) | ((uint32_t)(q[12 + k] & 255) << 24);
  }
  *(uint4*)(act_row + act_perm_off(K) + 16 * (size_t)g) = make_uint4(pm[0], pm[1], pm[2], pm[3]);
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float inv_scale_of(float scale_x, float w_scale) {
  return cr_divf(1.0f, __fmul_rn(scale_x, w_scale));  // src/kernel.c:391
}

}  // namespace bm
