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

// 16 int8 values of columns 16g..16g+15 -> split nibbles (unless nib is
// false: the MFMA products read only the permuted bytes) + permuted int8
__device__ __forceinline__ void write_act_group(uint8_t* __restrict__ act_row, int K, int g,
                                                const int (&q)[16], bool nib = true) {
  if (nib) {
  uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int xe = q[2 * n], xo = q[2 * n + 1];
    le |= (uint32_t)(xe & 15) << (4 * n);
    lo |= (uint32_t)(xo & 15) << (4 * n);
    he |= (uint32_t)((xe >> 4) & 15) << (4 * n);
    ho |= (uint32_t)((xo >> 4) & 15) << (4 * n);
  }
  *(uint4*)(act_row + act_nib_off(K) + 16 * (size_t)g) = make_uint4(le, lo, he, ho);
  }
  uint32_t pm[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    pm[k] = (uint32_t)(q[k] & 255) | ((uint32_t)(q[4 + k] & 255) << 8) |
            ((uint32_t)(q[8 + k] & 255) << 16) | ((uint32_t)(q[12 + k] & 255) << 24);
  }
  *(uint4*)(act_row + act_perm_off(K) + 16 * (size_t)g) = make_uint4(pm[0], pm[1], pm[2], pm[3]);
}

// Cross-lane reductions on DPP (no LDS round trips).  All 64 lanes must be
// active.  Within a 16-lane row: quad_perm [1,0,3,2] and [2,3,0,1] give
// every lane its quad's value, row_half_mirror pairs the two quads of each
// half row, row_mirror the two half rows.  Rows are then combined through
// scalar reads of lanes 0, 16, 32, 48.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

// sum over the 16 lanes of each row, in every lane of the row
__device__ __forceinline__ int row_sum_i32(int v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}

__device__ __forceinline__ float row_max_f32(float v) {
  v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
  return v;
}

__device__ __forceinline__ float lane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// sum / max over the wave, in every lane
__device__ __forceinline__ int wave_sum_i32(int v) {
  v = row_sum_i32(v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = row_max_f32(v);
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// A T-lane row team (T = 16, 32, 64; 16 lanes = one 1024-column slice)
// holding one weight row: reduce each lane's partial x.code over its 16-lane
// slice, subtract the slice's sum of x, and fold the team's slices into the
// fp32 output in slice order (src/kernel.c:255-256, 407-425).
template <int T>
__device__ __forceinline__ float row_finish(int part, int xs_slice, int p_index, int n_slices,
                                            float inv, float o, int unit_base) {
  part = row_sum_i32(part);
  const float f = __fmul_rn((float)(part - xs_slice), inv);
  if constexpr (T == 16) {
    if (p_index < n_slices) o = __fadd_rn(o, f);
  } else {
    // the team's rows (16-lane slices) in order: rows unit_base/16 ..
    const float r[4] = {lane_f32(f, 0), lane_f32(f, 16), lane_f32(f, 32), lane_f32(f, 48)};
#pragma unroll
    for (int q = 0; q < T / 16; ++q) {
      const float fq = T == 64 ? r[q] : (unit_base == 0 ? r[q] : r[2 + q]);
      if (p_index * (T / 16) + q < n_slices) o = __fadd_rn(o, fq);
    }
  }
  return o;
}

// the same team's exact int32 total (x.w over the team's columns)
template <int T>
__device__ __forceinline__ int row_total_i32(int part, int xs_slice, int unit_base) {
  const int t = row_sum_i32(part) - xs_slice;
  if constexpr (T == 16) {
    return t;
  } else {
    const int r[4] = {__builtin_amdgcn_readlane(t, 0), __builtin_amdgcn_readlane(t, 16),
                      __builtin_amdgcn_readlane(t, 32), __builtin_amdgcn_readlane(t, 48)};
    if constexpr (T == 64) return (r[0] + r[1]) + (r[2] + r[3]);
    return unit_base == 0 ? r[0] + r[1] : r[2] + r[3];
  }
}

// ---------------------------------------------------------------------------
// Sum of squares in the four sequential chains (src/kernel.c:77-89)
// ---------------------------------------------------------------------------
// chains held in registers (K/64 = E in {16, 32, 64}): lanes 16j..16j+15 of
// wave 0 own chain j in segments of E consecutive elements; each lane adds
// its segment to the running sum, which then moves one lane up the 16-lane
// row (DPP row_shr:1).  After 16 rounds lane 16j+15 holds chain j's sum.
// ---------------------------------------------------------------------------
// Fast mode (opt-in, not the reference's bits): the sum of squares as one
// balanced pairwise tree over the columns -- 16 consecutive columns per
// leaf group, (((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)))+..., then the groups
// pairwise in index order -- in place of the four sequential chains.  The
// same tree in every kernel that offers the mode, so a token's prefill and
// decode normalize alike.  (The reduction class of the Metal backend's
// rms_norm_quantize, src/metal/bm_shaders.metal:40-60, not its order.)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sq_tree16(const float4 (&v)[4]) {
  float t[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    t[k] = __fadd_rn(__fadd_rn(__fmul_rn(v[k].x, v[k].x), __fmul_rn(v[k].y, v[k].y)),
                     __fadd_rn(__fmul_rn(v[k].z, v[k].z), __fmul_rn(v[k].w, v[k].w)));
  return __fadd_rn(__fadd_rn(t[0], t[1]), __fadd_rn(t[2], t[3]));
}

// pairwise over the 16 lanes of each row (every butterfly step adds two
// equal-sized halves, so all lanes of the row hold the same bits), then the
// four rows pairwise: the tree over the wave's 64 leaf groups
__device__ __forceinline__ float wave_tree_f32(float v) {
  v = __fadd_rn(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
  v = __fadd_rn(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
  v = __fadd_rn(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
  v = __fadd_rn(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
  return __fadd_rn(__fadd_rn(lane_f32(v, 0), lane_f32(v, 16)),
                   __fadd_rn(lane_f32(v, 32), lane_f32(v, 48)));
}

// the tree's top levels over the G wave sums (1024 columns each)
template <int G>
__device__ __forceinline__ float tree_top(const float* w) {
  if constexpr (G == 1) return w[0];
  if constexpr (G == 2) return __fadd_rn(w[0], w[1]);
  return __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
}

__host__ __device__ inline bool chain_in_regs(int K) { return K == 1024 || K == 2048 || K == 4096; }
__host__ __device__ inline int sq_stride_of(int K) { return K / 4 + 68; }

template <int E>
__device__ __forceinline__ float chain_regs(const float* __restrict__ sq, int stride, int lane) {
  const int j = lane >> 4, seg = lane & 15;
  const float* __restrict__ src = sq + j * stride + seg * (E + 4);
  float v[E];
#pragma unroll
  for (int u = 0; u < E / 4; ++u) {
    const float4 t = *(const float4*)(src + 4 * u);
    v[4 * u] = t.x;
    v[4 * u + 1] = t.y;
    v[4 * u + 2] = t.z;
    v[4 * u + 3] = t.w;
  }
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int k = 0; k < E; ++k) s = __fadd_rn(s, v[k]);
    if (r < 15)
      s = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(s), __float_as_int(s), 0x111,
                                                     0xf, 0xf, false));
  }
  return s;
}

__device__ __forceinline__ float inv_scale_of(float scale_x, float w_scale) {
  return cr_divf(1.0f, __fmul_rn(scale_x, w_scale));  // src/kernel.c:391
}

}  // namespace bm
