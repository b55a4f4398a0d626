// gfx950 kernels of the ternary BitLinear hot path.
//
// Numerics (parity mode, the only mode): every kernel reproduces the
// reference's scalar path bit for bit (src/kernel.c:72-129, 346-448):
//   * sum of squares in four interleaved sequential fp32 chains, combined
//     ((s0+s1)+s2)+s3, tail added last (src/kernel.c:77-89);
//   * rms = 1/sqrtf(sum/n + 1e-6f), out = (x*rms)*w, no FMA contraction
//     (the file is built with -ffp-contract=off and uses __f*_rn);
//   * int8 = clamp((int)(v + (v >= 0 ? .5f : -.5f)), -128, 127);
//   * int32 totals per 1024-column block, fp32 out += total*inv_scale in
//     block order, then the K % 4 remainder (src/kernel.c:255-256, 407-447).
// Ternary decode: code = bits, w = min(code - 1, 1) (src/quantization.c:
// 27-31).  Kernels compute x.w = x.code - sum(x) with code in {0,1,2}; a
// code 11 is rewritten to 10 first (same value) unless the caller promises
// canonical weights.
#include <type_traits>

#include "bm_common.h"
#include "bm_dev.h"

namespace bm {

// ---------------------------------------------------------------------------
// Quantizer: one 256-thread block per token
// ---------------------------------------------------------------------------
constexpr int QT = 256;
constexpr int QTILE = 4096;  // elements per pass of the sequential chains

__global__ __launch_bounds__(QT) void k_quantize(const float* __restrict__ x, int n, int x_stride,
                                                 const float* __restrict__ gamma,
                                                 float* __restrict__ x_norm,
                                                 int8_t* __restrict__ xq, int quant_stride,
                                                 float* __restrict__ scale_out,
                                                 float* __restrict__ max_out,
                                                 uint8_t* __restrict__ act, size_t act_stride) {
  __shared__ __attribute__((aligned(16))) float sq[4][QTILE / 4 + 4];
  __shared__ float s_chain[4];
  __shared__ float s_rms;
  __shared__ float s_wmax[QT / 64];

  const int m = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const float* __restrict__ xr = x + (size_t)m * x_stride;
  const int n4 = n & ~3;

  // (1) four sequential chains over x[4i+j]^2, one lane each
  float chain = 0.0f;
  for (int t0 = 0; t0 < n4; t0 += QTILE) {
    const int cnt = min(QTILE, n4 - t0);
    for (int i = tid; i < cnt; i += QT) {
      const float v = xr[t0 + i];
      sq[i & 3][i >> 2] = __fmul_rn(v, v);
    }
    __syncthreads();
    if (tid < 4) {
      const float* c = sq[tid];
      const int len = cnt >> 2;
      int i = 0;
      for (; i + 8 <= len; i += 8) {
        const float4 a = *(const float4*)(c + i);
        const float4 b = *(const float4*)(c + i + 4);
        chain = __fadd_rn(chain, a.x);
        chain = __fadd_rn(chain, a.y);
        chain = __fadd_rn(chain, a.z);
        chain = __fadd_rn(chain, a.w);
        chain = __fadd_rn(chain, b.x);
        chain = __fadd_rn(chain, b.y);
        chain = __fadd_rn(chain, b.z);
        chain = __fadd_rn(chain, b.w);
      }
      for (; i < len; ++i) chain = __fadd_rn(chain, c[i]);
    }
    __syncthreads();
  }
  if (tid < 4) s_chain[tid] = chain;
  __syncthreads();
  if (tid == 0) {
    float sum = __fadd_rn(__fadd_rn(__fadd_rn(s_chain[0], s_chain[1]), s_chain[2]), s_chain[3]);
    for (int i = n4; i < n; ++i) sum = __fadd_rn(sum, __fmul_rn(xr[i], xr[i]));
    s_rms = cr_divf(1.0f, cr_sqrtf(__fadd_rn(cr_divf(sum, (float)n), 1e-6f)));
  }
  __syncthreads();
  const float rms = s_rms;

  // (2) max |(x*rms)*w| over the row (exact in any order)
  float mx = 0.0f;
  for (int i = tid; i < n; i += QT) {
    const float v = __fmul_rn(__fmul_rn(xr[i], rms), gamma[i]);
    mx = fmaxf(mx, fabsf(v));
  }
  mx = wave_max_f32(mx);
  if (lane == 0) s_wmax[wave] = mx;
  __syncthreads();
  float max_abs = s_wmax[0];
#pragma unroll
  for (int w = 1; w < QT / 64; ++w) max_abs = fmaxf(max_abs, s_wmax[w]);

  const float scale_x = cr_divf(127.0f, __fadd_rn(max_abs, 1e-5f));
  if (tid == 0) {
    if (scale_out) scale_out[m] = scale_x;
    if (max_out) max_out[m] = max_abs;
  }

  // (3) normalized values, int8, activation workspace; thread = 16 columns
  uint8_t* __restrict__ arow = act ? act + (size_t)m * act_stride : nullptr;
  const int n_groups = (n + 15) >> 4;
  for (int g0 = 0; g0 < n_groups; g0 += QT) {
    const int g = g0 + tid;
    int q[16];
    int qsum = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int c = 16 * g + j;
      int iv = 0;
      if (c < n) {
        const float v = __fmul_rn(__fmul_rn(xr[c], rms), gamma[c]);
        if (x_norm) x_norm[(size_t)m * n + c] = v;
        const float t = __fmul_rn(v, scale_x);
        const float r = __fadd_rn(t, t >= 0.0f ? 0.5f : -0.5f);
        iv = (int)r;
        iv = iv > 127 ? 127 : (iv < -128 ? -128 : iv);
        if (xq) xq[(size_t)m * quant_stride + c] = (int8_t)iv;
      }
      q[j] = iv;
      qsum += iv;
    }
    if (arow) {
      if (g < n_groups) write_act_group(arow, n, g, q);
      // 64 groups = one 1024-column slice = one wave of this pass
      const int s = wave_sum_i32(g < n_groups ? qsum : 0);
      const int slice = (g0 >> 6) + wave;
      if (lane == 0 && slice < slices_of(n)) ((int*)arow)[slice] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// Quantizer for n = 1024 * G (G in {1, 2, 4}): one wave per token, four
// tokens per block (two at G = 4), no block barriers.  Lane l keeps the 16-column groups
// l + 64i in registers; the squares pass through the wave's own LDS region
// once to reach the four-chain layout; everything else is register work.
// Same numerics as k_quantize.
// ---------------------------------------------------------------------------
// tokens (waves) per block: four, two at n = 4096 (LDS <= 64 KiB per block)
__host__ __device__ inline int quantize_wave_tpb(int n) { return n >= 4096 ? 2 : 4; }
__host__ __device__ inline size_t quantize_wave_lds(int n) {
  return (size_t)quantize_wave_tpb(n) * 4 * (size_t)sq_stride_of(n) * sizeof(float);
}

template <int G>
__global__ __launch_bounds__(G == 4 ? 128 : 256) void k_quantize_wave(const float* __restrict__ x, int M,
                                                       int x_stride,
                                                       const float* __restrict__ gamma,
                                                       float* __restrict__ x_norm,
                                                       int8_t* __restrict__ xq, int quant_stride,
                                                       float* __restrict__ scale_out,
                                                       uint8_t* __restrict__ act,
                                                       size_t act_stride, bool nib,
                                                       bool fast) {
  constexpr int K = 1024 * G, E = K / 64;
  extern __shared__ __attribute__((aligned(16))) float lds_sq[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = blockIdx.x * (G == 4 ? 2 : 4) + wave;
  if (m >= M) return;  // whole waves only; nothing below waits for other waves
  const int stride = sq_stride_of(K);
  float* __restrict__ sq = lds_sq + (size_t)wave * 4 * stride;
  const float* __restrict__ xr = x + (size_t)m * x_stride;

  float4 xv[G][4], gv[G][4];
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) xv[i][k] = ((const float4*)xr)[4 * (lane + 64 * i) + k];
  // gamma is read after the sum of squares (the same rows for every token,
  // so they come from L2): during the chains its registers stay free, which
  // lets two waves share a SIMD at n = 4096 and four at n = 2048
  auto load_gamma = [&]() {
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) gv[i][k] = ((const float4*)gamma)[4 * (lane + 64 * i) + k];
  };
  float sum;
  if (fast) {
    // the pairwise tree: leaf group lane + 64 i, then the G wave sums
    float w[G];
#pragma unroll
    for (int i = 0; i < G; ++i) w[i] = wave_tree_f32(sq_tree16(xv[i]));
    sum = tree_top<G>(w);
  } else {
    // column 16g + 4k + j is element 4g + k of chain j (segments of E padded
    // by 4 floats)
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int e = 4 * (lane + 64 * i);
      const int pe = e + 4 * (e / E);
      const float4* v = xv[i];
      *(float4*)&sq[pe] = make_float4(__fmul_rn(v[0].x, v[0].x), __fmul_rn(v[1].x, v[1].x),
                                      __fmul_rn(v[2].x, v[2].x), __fmul_rn(v[3].x, v[3].x));
      *(float4*)&sq[stride + pe] = make_float4(__fmul_rn(v[0].y, v[0].y), __fmul_rn(v[1].y, v[1].y),
                                               __fmul_rn(v[2].y, v[2].y), __fmul_rn(v[3].y, v[3].y));
      *(float4*)&sq[2 * stride + pe] =
          make_float4(__fmul_rn(v[0].z, v[0].z), __fmul_rn(v[1].z, v[1].z),
                      __fmul_rn(v[2].z, v[2].z), __fmul_rn(v[3].z, v[3].z));
      *(float4*)&sq[3 * stride + pe] =
          make_float4(__fmul_rn(v[0].w, v[0].w), __fmul_rn(v[1].w, v[1].w),
                      __fmul_rn(v[2].w, v[2].w), __fmul_rn(v[3].w, v[3].w));
    }
    // one wave's LDS operations complete in order; the fences keep the
    // compiler from moving the reads above the writes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float cs = chain_regs<E>(sq, stride, lane);
    const float s0 = lane_f32(cs, 15), s1 = lane_f32(cs, 31);
    const float s2 = lane_f32(cs, 47), s3 = lane_f32(cs, 63);
    sum = __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
  }
  load_gamma();
  // sum / K with K a power of two: an exact scaling, rounded like the division
  const float rms = cr_divf(1.0f, cr_sqrtf(__fadd_rn(__fmul_rn(sum, 1.0f / K), 1e-6f)));

  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 v = xv[i][k];
      const float4 g4 = gv[i][k];
      xv[i][k] = make_float4(__fmul_rn(__fmul_rn(v.x, rms), g4.x), __fmul_rn(__fmul_rn(v.y, rms), g4.y),
                             __fmul_rn(__fmul_rn(v.z, rms), g4.z), __fmul_rn(__fmul_rn(v.w, rms), g4.w));
      if (x_norm) ((float4*)(x_norm + (size_t)m * K))[4 * (lane + 64 * i) + k] = xv[i][k];
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xv[i][k].x), fabsf(xv[i][k].y)),
                           fmaxf(fabsf(xv[i][k].z), fabsf(xv[i][k].w))));
    }
  mx = wave_max_f32(mx);
  const float scale_x = cr_divf(127.0f, __fadd_rn(mx, 1e-5f));
  if (lane == 0 && scale_out) scale_out[m] = scale_x;

  uint8_t* __restrict__ arow = act ? act + (size_t)m * act_stride : nullptr;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + 64 * i;
    int q[16];
    int qsum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float vv[4] = {xv[i][k].x, xv[i][k].y, xv[i][k].z, xv[i][k].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float t = __fmul_rn(vv[j], scale_x);
        int iv = (int)__fadd_rn(t, t >= 0.0f ? 0.5f : -0.5f);
        iv = iv > 127 ? 127 : (iv < -128 ? -128 : iv);
        q[4 * k + j] = iv;
        qsum += iv;
      }
    }
    if (xq) {
      int8_t* dst = xq + (size_t)m * quant_stride + 16 * g;
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = (uint32_t)(q[4 * k] & 255) | ((uint32_t)(q[4 * k + 1] & 255) << 8) |
               ((uint32_t)(q[4 * k + 2] & 255) << 16) | ((uint32_t)(q[4 * k + 3] & 255) << 24);
      if (((uintptr_t)dst & 15) == 0) {
        *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) dst[j] = (int8_t)q[j];
      }
    }
    if (arow) write_act_group(arow, K, g, q, nib);
    const int ssum = wave_sum_i32(qsum);  // groups 64i .. 64i+63 = slice i
    if (arow && lane == 0) ((int*)arow)[i] = ssum;
  }
}

// int8 activations given directly (stress shape): workspace only.  A row
// that starts on 16 bytes is read 16 bytes per thread; NIB: also the split
// nibbles, which only the per-token GEMV kernels read
template <bool NIB>
__global__ __launch_bounds__(QT) void k_prep_i8(const int8_t* __restrict__ xq, int ldx, int K,
                                                uint8_t* __restrict__ act, size_t act_stride) {
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int8_t* __restrict__ xr = xq + (size_t)m * ldx;
  uint8_t* __restrict__ arow = act + (size_t)m * act_stride;
  const int n_groups = (K + 15) >> 4;
  const bool vec = ((uintptr_t)xr & 15) == 0;
  for (int g0 = 0; g0 < n_groups; g0 += QT) {
    const int g = g0 + tid;
    int q[16];
    int qsum = 0;
    if (vec && 16 * g + 15 < K) {
      const int4 v = *(const int4*)(xr + 16 * g);
      const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) q[j] = (int)(int8_t)(w[j >> 2] >> (8 * (j & 3)));
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int c = 16 * g + j;
        q[j] = c < K ? (int)xr[c] : 0;
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) qsum += q[j];
    if (g < n_groups) write_act_group(arow, K, g, q, NIB);
    const int s = wave_sum_i32(g < n_groups ? qsum : 0);
    const int slice = (g0 >> 6) + wave;
    if (lane == 0 && slice < slices_of(K)) ((int*)arow)[slice] = s;
  }
}


// ---------------------------------------------------------------------------
// Decode GEMV (v_dot8 on split nibbles).  K % 64 == 0, K <= 64*64*P.
//   T lanes per row (16/32/64), each lane owns 64 columns (16 packed bytes)
//   per pass; P passes cover K.  16 consecutive lanes = one 1024-column
//   slice, reduced with xor shuffles inside the 16-lane group.
//   Each wave owns GW consecutive row groups (64/T rows each) and issues
//   all of their weight loads before the first dot product, so a wave keeps
//   GW KiB (T=32) in flight and never waits on its own stores.
// ---------------------------------------------------------------------------
template <int T, int P, int GW, bool CANON, int MODE>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ act, size_t act_stride,
                                              const float* __restrict__ scale_x,
                                              const uint8_t* __restrict__ W, int N, int K,
                                              float w_scale, float* __restrict__ out,
                                              int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  constexpr int RPW = 64 / T;  // rows per wave per row group
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int n_rg = (N + RPW - 1) / RPW;
  const int rg0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GW;
  if (rg0 >= n_rg) return;
  const int chunks = K >> 6;
  const size_t wstride = (size_t)(K >> 2);

  const uint8_t* __restrict__ arow = act + (size_t)m * act_stride;
  const int* __restrict__ ssum = (const int*)arow;
  const uint4* __restrict__ anib = (const uint4*)(arow + act_nib_off(K));

  // activations of this lane's chunks: 4 groups x {le, lo, he, ho}
  uint32_t xa[P][16];
  int xs[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * T + u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint4 v = j < chunks ? anib[4 * j + g] : make_uint4(0, 0, 0, 0);
      xa[p][4 * g + 0] = v.x;
      xa[p][4 * g + 1] = v.y;
      xa[p][4 * g + 2] = v.z;
      xa[p][4 * g + 3] = v.w;
    }
    // lane groups past the last slice hold no columns: their total is 0
    const int slice = (p * T + u) / 16;
    xs[p] = slice < slices_of(K) ? ssum[slice] : 0;
  }

  // weights of all GW row groups.  Rows past N reread row N-1 and are never
  // stored; lanes past the last chunk read the last chunk, which meets zero
  // activations.
  uint4 wv[GW][P];
#pragma unroll
  for (int i = 0; i < GW; ++i) {
    const int r = min((rg0 + i) * RPW + sub, N - 1);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = min(p * T + u, chunks - 1);
      wv[i][p] = load_stream16(W + (size_t)r * wstride + 16 * (size_t)j);
    }
  }
  const float inv = I32 ? 0.0f : inv_scale_of(scale_x[m], w_scale);

  float o[GW];
  int tot[GW];
#pragma unroll
  for (int i = 0; i < GW; ++i) {
    o[i] = 0.0f;
    tot[i] = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint32_t w4[4] = {wv[i][p].x, wv[i][p].y, wv[i][p].z, wv[i][p].w};
      uint32_t al = 0;
      int ah = 0;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t pw = CANON ? w4[d] : canon_codes(w4[d]);
        const uint32_t lo = pw & 0x33333333u;
        const uint32_t hi = (pw >> 2) & 0x33333333u;
        al = __builtin_amdgcn_udot8(lo, xa[p][4 * d + 0], al, false);
        al = __builtin_amdgcn_udot8(hi, xa[p][4 * d + 1], al, false);
        ah = __builtin_amdgcn_sdot8((int)lo, (int)xa[p][4 * d + 2], ah, false);
        ah = __builtin_amdgcn_sdot8((int)hi, (int)xa[p][4 * d + 3], ah, false);
      }
      const int part = ah * 16 + (int)al;
      if (I32)
        tot[i] += row_total_i32<T>(part, xs[p], unit_base);
      else
        o[i] = row_finish<T>(part, xs[p], p, slices_of(K), inv, o[i], unit_base);
    }
  }
  if (u == 0) {
#pragma unroll
    for (int i = 0; i < GW; ++i) {
      const int row = (rg0 + i) * RPW + sub;
      if (rg0 + i < n_rg && row < N) {
        if (I32)
          out_i32[(size_t)m * N + row] = tot[i];
        else
          out[(size_t)m * N + row] = MODE == 1 ? __fadd_rn(out[(size_t)m * N + row], o[i]) : o[i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Few-token GEMV (2 <= M < 32): the k_gemv row layout, but each wave loads
// its weight rows once and applies them to every token in turn.  A token's
// activations (split nibbles + slice sums) are staged in LDS for the whole
// block, double-buffered through registers one token ahead.  K <= 8192.
// ---------------------------------------------------------------------------
constexpr int kMtMaxK = 8192, kMtMaxM = 32;

template <int T, int P, int GW, bool CANON, int MODE>
__global__ __launch_bounds__(256) void k_gemv_mt(const uint8_t* __restrict__ act,
                                                 size_t act_stride,
                                                 const float* __restrict__ scale_x, int M,
                                                 const uint8_t* __restrict__ W, int N, int K,
                                                 float w_scale, float* __restrict__ out,
                                                 int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  constexpr int RPW = 64 / T;
  constexpr int SU = kMtMaxK / 16 / 256;  // staged uint4 per thread per token
  __shared__ uint4 s_nib[2][kMtMaxK / 16];
  __shared__ int s_sl[2][kMtMaxK / 1024];
  __shared__ float s_inv[kMtMaxM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int n_rg = (N + RPW - 1) / RPW;
  const int rg0 = (blockIdx.x * 4 + wave) * GW;
  const int chunks = K >> 6, n_groups16 = K >> 4, n_sl = slices_of(K);
  const size_t wstride = (size_t)(K >> 2);
  const size_t nib_off = act_nib_off(K);

  if (tid < M) s_inv[tid] = I32 ? 0.0f : inv_scale_of(scale_x[tid], w_scale);

  // this wave's weights, once
  uint4 wv[GW][P];
#pragma unroll
  for (int i = 0; i < GW; ++i) {
    const int r = min((rg0 + i) * RPW + sub, N - 1);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = min(p * T + u, chunks - 1);
      wv[i][p] = load_stream16(W + (size_t)r * wstride + 16 * (size_t)j);
    }
  }

  // token m's activations: global -> registers -> LDS buffer m & 1
  uint4 st_nib[SU];
  int st_sl = 0;
  auto fetch = [&](int m) __attribute__((always_inline)) {
    const uint8_t* __restrict__ arow = act + (size_t)min(m, M - 1) * act_stride;
#pragma unroll
    for (int k = 0; k < SU; ++k) {
      const int g = tid + 256 * k;
      st_nib[k] = g < n_groups16 ? ((const uint4*)(arow + nib_off))[g] : make_uint4(0, 0, 0, 0);
    }
    st_sl = tid < n_sl ? ((const int*)arow)[tid] : 0;
  };
  auto put = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < SU; ++k) {
      const int g = tid + 256 * k;
      if (g < n_groups16) s_nib[buf][g] = st_nib[k];
    }
    if (tid < n_sl) s_sl[buf][tid] = st_sl;
  };

  fetch(0);
  put(0);
  fetch(1);
  __syncthreads();
  for (int m = 0; m < M; ++m) {
    const int buf = m & 1;
    uint32_t xa[P][16];
    int xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint4 v = j < chunks ? s_nib[buf][4 * j + g] : make_uint4(0, 0, 0, 0);
        xa[p][4 * g + 0] = v.x;
        xa[p][4 * g + 1] = v.y;
        xa[p][4 * g + 2] = v.z;
        xa[p][4 * g + 3] = v.w;
      }
      const int slice = (p * T + u) / 16;
      xs[p] = slice < n_sl ? s_sl[buf][slice] : 0;
    }
    const float inv = s_inv[m];
    if (rg0 < n_rg) {
#pragma unroll
      for (int i = 0; i < GW; ++i) {
        float o = 0.0f;
        int tot = 0;
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const uint32_t w4[4] = {wv[i][p].x, wv[i][p].y, wv[i][p].z, wv[i][p].w};
          uint32_t al = 0;
          int ah = 0;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t pw = CANON ? w4[d] : canon_codes(w4[d]);
            const uint32_t lo = pw & 0x33333333u;
            const uint32_t hi = (pw >> 2) & 0x33333333u;
            al = __builtin_amdgcn_udot8(lo, xa[p][4 * d + 0], al, false);
            al = __builtin_amdgcn_udot8(hi, xa[p][4 * d + 1], al, false);
            ah = __builtin_amdgcn_sdot8((int)lo, (int)xa[p][4 * d + 2], ah, false);
            ah = __builtin_amdgcn_sdot8((int)hi, (int)xa[p][4 * d + 3], ah, false);
          }
          const int part = ah * 16 + (int)al;
          if (I32)
            tot += row_total_i32<T>(part, xs[p], unit_base);
          else
            o = row_finish<T>(part, xs[p], p, n_sl, inv, o, unit_base);
        }
        const int row = (rg0 + i) * RPW + sub;
        if (u == 0 && rg0 + i < n_rg && row < N) {
          const size_t at = (size_t)m * N + row;
          if (I32)
            out_i32[at] = tot;
          else
            out[at] = MODE == 1 ? __fadd_rn(out[at], o) : o;
        }
      }
    }
    put(buf ^ 1);  // token m+1 into the buffer token m-1 used
    fetch(m + 2);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Few-token product on int8 MFMA (2 <= M <= 256, K % 128 == 0; up to 16
// tokens at K <= 8192 go to k_gemm_few below instead): block row
// y takes tokens 32y .. 32y+31, the 32 rows of v_mfma_i32_32x32x32_i8's A
// operand (rows past M are not stored); 32 weight rows are its B operand.
// A block of 8 waves owns GPB groups of 32 weight rows; the WPG waves of a
// group split its 1024-column slices.  Each wave loads a slice's packed
// weights and the tokens' permuted int8 (cache-resident: every block reads
// them) with coalesced loads, regroups them for the MFMA lanes through its
// own LDS, decodes the weights in registers, and leaves the exact int32
// x.code per (slice, token, row) in LDS; the block then folds the slices in
// order, each as (x.code - sum x) / (scale_x * w_scale) with one rounding
// (src/kernel.c:255-256, 407-425).  Lane (j, h) covers columns
// 128t + 64h + 16q .. in step q of each 128-column block t.
// ---------------------------------------------------------------------------
constexpr int kSmMaxM = 32, kSmMaxSlices = 16;  // K <= 16384
constexpr int kSmMaxTokens = 256;  // up to 8 token tiles of 32 in one launch

__host__ __device__ inline int sm_wpg(int n_slices) {  // waves per row group: a power of two
  return n_slices >= 8 ? 8 : (n_slices >= 4 ? 4 : (n_slices >= 2 ? 2 : 1));
}

// 16 int8 values in column order -> the MFMA operand order of the
// activation workspace (byte 4k+b = column 4b+k): a 4x4 byte transpose
__device__ __forceinline__ v4i transpose_4x4_bytes(v4i c) {
  const uint32_t c0 = c[0], c1 = c[1], c2 = c[2], c3 = c[3];
  // v_perm_b32 selector bytes: 0..3 = bytes of the second operand, 4..7 of
  // the first
  const uint32_t t0 = __builtin_amdgcn_perm(c1, c0, 0x05010400u);  // c0.0 c1.0 c0.1 c1.1
  const uint32_t t1 = __builtin_amdgcn_perm(c3, c2, 0x05010400u);  // c2.0 c3.0 c2.1 c3.1
  const uint32_t t2 = __builtin_amdgcn_perm(c1, c0, 0x07030602u);  // c0.2 c1.2 c0.3 c1.3
  const uint32_t t3 = __builtin_amdgcn_perm(c3, c2, 0x07030602u);  // c2.2 c3.2 c2.3 c3.3
  return v4i{(int)__builtin_amdgcn_perm(t1, t0, 0x05040100u), (int)__builtin_amdgcn_perm(t1, t0, 0x07060302u),
             (int)__builtin_amdgcn_perm(t3, t2, 0x05040100u), (int)__builtin_amdgcn_perm(t3, t2, 0x07060302u)};
}

// Fold of a few-token block: slice s's exact int32 x.code of (token m, row
// r) is part[(s * TS + m) * rows_b + r]; each slice's term is
// (x.code - sum x) / (scale_x * w_scale), exact int32 before the one
// rounding, added in slice order (src/kernel.c:255-256, 407-425).
// Thread -> (token, row) pairs of the block's rows.
template <int MODE, int TS>
__device__ __forceinline__ void small_fold(const float* __restrict__ s_part,
                                           const int (*s_sx)[kSmMaxSlices],
                                           const float* __restrict__ s_inv, int M, int rows_b,
                                           int N, int n_slices, float* __restrict__ out,
                                           int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  for (int i = threadIdx.x; i < M * rows_b; i += blockDim.x) {
    const int m = i / rows_b, r = i % rows_b;
    const int row = blockIdx.x * rows_b + r;
    if (row >= N) continue;
    float o = 0.0f;
    int tot = 0;
    for (int sl = 0; sl < n_slices; ++sl) {
      const int t = __float_as_int(s_part[((size_t)sl * TS + m) * rows_b + r]) - s_sx[m][sl];
      if (I32)
        tot += t;
      else
        o = __fadd_rn(o, __fmul_rn((float)t, s_inv[m]));
    }
    const size_t at = (size_t)m * N + row;
    if (I32)
      out_i32[at] = tot;
    else
      out[at] = MODE == 1 ? __fadd_rn(out[at], o) : o;
  }
}

// RAW: act is the callers' int8 activations themselves (row stride
// act_stride, rows on 16 bytes, int32 outputs): each wave puts its chunks in
// operand order and sums its slice's values (sdot4 against ones) itself, so
// no preparation launch and no workspace are needed.
template <bool CANON, int MODE, int MT8, bool RAW>
__global__ __launch_bounds__(512) void k_gemm_small(const uint8_t* __restrict__ act,
                                                    size_t act_stride,
                                                    const float* __restrict__ scale_x, int M,
                                                    const uint8_t* __restrict__ W, int N, int K,
                                                    float w_scale, float* __restrict__ out,
                                                    int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  // token tile blockIdx.y: tokens 32y .. 32y+31, of which the first 8 * MT8
  // are loaded (the tile's rows past M repeat its last token; their results
  // are never stored)
  const int m_base = blockIdx.y * kSmMaxM;
  act += (size_t)m_base * act_stride;
  if (!I32) scale_x += m_base;
  if (I32)
    out_i32 += (size_t)m_base * N;
  else
    out += (size_t)m_base * N;
  M = min(kSmMaxM, M - m_base);
  extern __shared__ __attribute__((aligned(16))) float s_part[];  // [slice][32 tokens][GPB*32 rows]
  __shared__ int s_sx[kSmMaxM][kSmMaxSlices];
  __shared__ float s_inv[kSmMaxM];
  __shared__ __attribute__((aligned(16))) uint8_t s_tA[8][32 * 128];  // per wave: one step of A
  __shared__ __attribute__((aligned(16))) uint8_t s_tB[8][32 * 128];  // per wave: 4 steps of B
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j32 = lane & 31, h = lane >> 5;
  const int n_slices = slices_of(K);
  const int wpg = sm_wpg(n_slices), gpb = 8 / wpg, spw = (n_slices + wpg - 1) / wpg;
  const int rows_b = 32 * gpb;
  const size_t wstride = (size_t)(K >> 2);
  const size_t perm = RAW ? 0 : act_perm_off(K);
  static_assert(!RAW || MODE == 2, "raw int8 activations: int32 outputs only");

  // Every global load below is unconditional (indices clamped into the
  // buffers; values that are not needed are never used): a load inside a
  // branch makes the compiler wait for all outstanding loads at its first
  // use, so the first step would wait for the whole slice.  The slice sums
  // of x and the scales are needed only by the fold: loaded first, into
  // registers, and put in LDS after the products.
  const int e_sx = min(tid, kSmMaxM * n_slices - 1);
  const int sx_m = e_sx / n_slices, sx_sl = e_sx % n_slices;
  int sx_v = 0;
  if constexpr (!RAW) sx_v = ((const int*)(act + (size_t)min(sx_m, M - 1) * act_stride))[sx_sl];
  float sc_v = 0.0f;
  if constexpr (!I32) sc_v = scale_x[min(tid & (kSmMaxM - 1), M - 1)];

  const int g = wave / wpg;                       // row group in the block
  const int n0 = (blockIdx.x * gpb + g) * 32;     // its first weight row
  const int cr = lane >> 3, cc = lane & 7;
  uint8_t* __restrict__ tA = s_tA[wave];
  uint8_t* __restrict__ tB = s_tB[wave];
  // 16-byte chunk c of row r (128-byte rows), XOR-swizzled by r % 8 so that
  // 16 rows read at one chunk index hit distinct banks
  auto swz = [](int r, int c) __attribute__((always_inline)) { return r * 128 + 16 * (c ^ (r & 7)); };
  auto wave_lds_sync = []() __attribute__((always_inline)) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  const int sl0 = (wave % wpg) * spw, sl1 = min(n_slices, sl0 + spw);
  for (int sl = sl0; sl < sl1; ++sl) {
    const int kb0 = sl * kSlice, kb1 = min(K, kb0 + kSlice);
    v16i acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0;
    // The whole slice's operands are requested before the first MFMA, in a
    // coalesced order (lane l: row l/8 + 8i, 16-byte chunk l%8 of a 128-byte
    // run), then moved to the MFMA lanes through the wave's own LDS.
    const int nst = (kb1 - kb0) >> 7;  // 128-column blocks, <= 8
    const int wb = (kb1 - kb0) >> 2;   // packed bytes of the slice per row
    // Issued in the order the steps use them (B of steps 0-3, A of step 0,
    // ..., B of steps 4-7, A of step 4, ...), held there by scheduling
    // barriers: completion waits count loads in issue order, so a step
    // waits only for its own operands and those issued before them.
    v4i ca[kSlice / 128][MT8], cb[kSlice / 512][4];
#pragma unroll
    for (int t = 0; t < kSlice / 128; ++t) {
      if (t % 4 == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = min(n0 + cr + 8 * i, N - 1);
          cb[t / 4][i] = *(const v4i*)(W + (size_t)r * wstride + (kb0 >> 2) +
                                       min(32 * t + 16 * cc, wb - 16));
        }
      }
#pragma unroll
      for (int i = 0; i < MT8; ++i)
        ca[t][i] = *(const v4i*)(act + (size_t)min(cr + 8 * i, M - 1) * act_stride + perm + kb0 +
                                 128 * min(t, nst - 1) + 16 * cc);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Every step runs (a branch around a step would pull its loads into
    // the branch); the steps past a short last slice multiply zero codes.
    // Software-pipelined: a step's operands are read from LDS into
    // registers one step ahead, so the wave's LDS buffers are free again as
    // soon as those reads complete; each turn issues step t's MFMAs first,
    // then stages step t+1 (its loads' wait, the write to LDS, the read
    // back) while they run.
    int xs[MT8];
#pragma unroll
    for (int i = 0; i < MT8; ++i) xs[i] = 0;
    auto stage_write = [&](int t) __attribute__((always_inline)) {
      if constexpr (RAW) {
#pragma unroll
        for (int i = 0; i < MT8; ++i) {
          const v4i c = ca[t][i];
          int sum = 0;
#pragma unroll
          for (int d = 0; d < 4; ++d) sum = __builtin_amdgcn_sdot4(c[d], 0x01010101, sum, false);
          xs[i] += t < nst ? sum : 0;
          ca[t][i] = transpose_4x4_bytes(c);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < MT8) *(v4i*)(tA + swz(cr + 8 * i, cc)) = ca[t][i];
        if (t % 4 == 0) *(v4i*)(tB + swz(cr + 8 * i, cc)) = cb[t / 4][i];
      }
    };
    uint4 bwv[2];
    v4i aov[2][4];
    auto stage_read = [&](int t) __attribute__((always_inline)) {
      bwv[t & 1] = *(const uint4*)(tB + swz(j32, 2 * (t % 4) + h));
      if (t >= nst) bwv[t & 1] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) aov[t & 1][q] = *(const v4i*)(tA + swz(j32, 4 * h + q));
    };
    stage_write(0);
    wave_lds_sync();
    stage_read(0);
    wave_lds_sync();  // the reads are done before the next step's writes
#pragma unroll
    for (int t = 0; t < kSlice / 128; ++t) {
      const uint4 bw = bwv[t & 1];
      const uint32_t w4[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pw = CANON ? w4[q] : canon_codes(w4[q]);
        v4i bo;
        bo[0] = (int)(pw & 0x03030303u);
        bo[1] = (int)((pw >> 2) & 0x03030303u);
        bo[2] = (int)((pw >> 4) & 0x03030303u);
        bo[3] = (int)((pw >> 6) & 0x03030303u);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(aov[t & 1][q], bo, acc, 0, 0, 0);
      }
      if (t + 1 < kSlice / 128) {
        stage_write(t + 1);
        wave_lds_sync();
        stage_read(t + 1);
        wave_lds_sync();
      }
    }
    if constexpr (RAW) {
      // the slice's sum of x for token cr + 8i: over the 8 lanes cr*8 .. +7
#pragma unroll
      for (int i = 0; i < MT8; ++i) {
        int v = xs[i];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        v += __shfl_xor(v, 4);
        if (cc == 0) s_sx[cr + 8 * i][sl] = v;
      }
    }
    // acc element v: token 8(v/4) + 4h + v%4, weight row j32; the exact
    // int32 x.code of the slice (rows of A past 8 MT8 hold stale bytes and
    // only reach tokens that are never stored)
    float* __restrict__ part = s_part + (size_t)sl * kSmMaxM * rows_b;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = 8 * (v >> 2) + 4 * h + (v & 3);
      part[m * rows_b + g * 32 + j32] = __int_as_float(acc[v]);
    }
  }
  if (!RAW && tid < kSmMaxM * n_slices) s_sx[sx_m][sx_sl] = sx_v;
  if (!I32 && tid < kSmMaxM) s_inv[tid] = inv_scale_of(sc_v, w_scale);
  __syncthreads();
  small_fold<MODE, kSmMaxM>(s_part, s_sx, s_inv, M, rows_b, N, n_slices, out, out_i32);
}

// ---------------------------------------------------------------------------
// Up to 16 tokens on v_mfma_i32_16x16x64_i8.  The block layout is
// k_gemm_small's: 8 waves, GPB groups of 32 weight rows, the WPG waves of a
// group splitting the group's 1024-column slices, the slices folded in order
// at the end.  In a slice, lane l (i = l % 16, g = l / 16) owns columns
// 256 s + 64 g .. +63 of super-step s (s = 0..3); MFMA q of the super-step
// multiplies columns 16 q .. 16 q + 15 of that run (the A and B lanes of one
// index cover the same columns; D lane l element v is token 4 g + v, row
// l % 16).  The weights are loaded straight into those lanes (16 packed
// bytes of rows i and 16 + i per super-step); the slice's activations are
// loaded coalesced (8 lanes per 128-byte run of a token), put in the wave's
// own LDS once, and read back in lane order.  Every global load is issued
// before the first MFMA, activations first, then weights in super-step
// order, unconditionally (columns past a short last slice read in-bounds
// bytes and multiply zero codes).  RAW: int8 activations from the caller's
// rows, put in operand order with a 4x4 byte transpose and summed per slice
// with v_dot4 against ones.  MT8: 8-token groups loaded (1 for M <= 8; the
// A rows of tokens not loaded hold stale LDS bytes and reach only tokens
// that are never stored).  STREAM: nontemporal weight loads, for matrices of
// 8 MB and more (K = N = 8192 at M = 16: 7.9 against 8.2 us per call with
// the weights cold; plain loads are faster on smaller matrices and whenever
// the weights are still cached).
// ---------------------------------------------------------------------------
constexpr int kFewM = 16;  // tokens of k_gemm_few
// K <= 8192: the per-wave activation slices (128 KB) and the slice results
// (16 KB at most) fit the 160 KB of LDS
constexpr int kFewMaxSlices = 8;
inline bool few_stream(int N, int K) { return (size_t)N * (size_t)(K / 4) >= ((size_t)8 << 20); }
__host__ __device__ inline size_t few_lds(int K) {  // dynamic LDS: the slice results
  const int n_slices = slices_of(K);
  return (size_t)n_slices * kFewM * 32 * (8 / sm_wpg(n_slices)) * sizeof(float);
}

template <bool CANON, int MODE, int MT8, bool RAW, bool STREAM>
__global__ __launch_bounds__(512) void k_gemm_few(const uint8_t* __restrict__ act,
                                                  size_t act_stride,
                                                  const float* __restrict__ scale_x, int M,
                                                  const uint8_t* __restrict__ W, int N, int K,
                                                  float w_scale, float* __restrict__ out,
                                                  int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  static_assert(!RAW || MODE == 2, "raw int8 activations: int32 outputs only");
  extern __shared__ __attribute__((aligned(16))) float s_part[];  // [slice][16 tokens][GPB*32 rows]
  __shared__ int s_sx[kSmMaxM][kSmMaxSlices];
  __shared__ float s_inv[kSmMaxM];
  __shared__ __attribute__((aligned(16))) uint8_t s_x[8][kFewM * kSlice];  // per wave: a slice of x
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int cr = lane >> 3, cc = lane & 7;
  const int n_slices = slices_of(K);
  const int wpg = sm_wpg(n_slices), gpb = 8 / wpg, spw = (n_slices + wpg - 1) / wpg;
  const int rows_b = 32 * gpb;
  const size_t wstride = (size_t)(K >> 2);
  const size_t perm = RAW ? 0 : act_perm_off(K);

  // fold inputs (slice sums of x, scales): loaded first, into registers
  const int e_sx = min(tid, kFewM * n_slices - 1);
  const int sx_m = e_sx / n_slices, sx_sl = e_sx % n_slices;
  int sx_v = 0;
  if constexpr (!RAW) sx_v = ((const int*)(act + (size_t)min(sx_m, M - 1) * act_stride))[sx_sl];
  float sc_v = 0.0f;
  if constexpr (!I32) sc_v = scale_x[min(tid & (kFewM - 1), M - 1)];

  const int grp = wave / wpg;
  const int n0 = (blockIdx.x * gpb + grp) * 32;
  const uint8_t* __restrict__ x0 = act + (size_t)min(cr, M - 1) * act_stride + perm;
  const uint8_t* __restrict__ x1 = act + (size_t)min(cr + 8, M - 1) * act_stride + perm;
  const uint8_t* __restrict__ w0 = W + (size_t)min(n0 + li, N - 1) * wstride;
  const uint8_t* __restrict__ w1 = W + (size_t)min(n0 + 16 + li, N - 1) * wstride;
  uint8_t* __restrict__ tx = s_x[wave];
  // 16-byte chunk c of token r's 1024-byte row, XOR-swizzled by r so that
  // the 16 tokens read at one chunk index hit distinct banks
  auto xpos = [](int r, int c) __attribute__((always_inline)) { return r * kSlice + 16 * (c ^ r); };
  auto wave_lds_sync = []() __attribute__((always_inline)) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  const int sl0 = (wave % wpg) * spw, sl1 = min(n_slices, sl0 + spw);
  for (int sl = sl0; sl < sl1; ++sl) {
    const int kb0 = sl * kSlice, ncols = min(K, kb0 + kSlice) - kb0;  // a multiple of 128
    const int nst = ncols >> 7;
    v4i xa[8][MT8];
    uint4 wv[4][2];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int c = kb0 + 128 * min(t, nst - 1) + 16 * cc;
      xa[t][0] = *(const v4i*)(x0 + c);
      if constexpr (MT8 == 2) xa[t][1] = *(const v4i*)(x1 + c);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int c = kb0 + min(256 * st + 64 * lg, ncols - 64);
      if constexpr (STREAM) {
        wv[st][0] = load_stream16(w0 + (c >> 2));
        wv[st][1] = load_stream16(w1 + (c >> 2));
      } else {
        wv[st][0] = *(const uint4*)(w0 + (c >> 2));
        wv[st][1] = *(const uint4*)(w1 + (c >> 2));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the slice's activations into the wave's LDS, in operand order
    int xs0 = 0, xs1 = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int i = 0; i < MT8; ++i) {
        v4i a = xa[t][i];
        if constexpr (RAW) {
          int sum = 0;
#pragma unroll
          for (int d = 0; d < 4; ++d) sum = __builtin_amdgcn_sdot4(a[d], 0x01010101, sum, false);
          (i == 0 ? xs0 : xs1) += t < nst ? sum : 0;
          a = transpose_4x4_bytes(a);
        }
        *(v4i*)(tx + xpos(cr + 8 * i, 8 * t + cc)) = a;
      }
    }
    // the weights' decode stays below the writes: hoisted above them, it
    // would make the writes wait for the weight loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RAW) {
      // token cr's (and cr + 8's) slice sum: over the 8 lanes cr*8 .. +7
      xs0 += __shfl_xor(xs0, 1);
      xs0 += __shfl_xor(xs0, 2);
      xs0 += __shfl_xor(xs0, 4);
      xs1 += __shfl_xor(xs1, 1);
      xs1 += __shfl_xor(xs1, 2);
      xs1 += __shfl_xor(xs1, 4);
      if (cc == 0) {
        s_sx[cr][sl] = xs0;
        s_sx[cr + 8][sl] = xs1;
      }
    }
    wave_lds_sync();
    v4i acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bool valid = 256 * st + 64 * lg < ncols;
      const uint32_t b0[4] = {wv[st][0].x, wv[st][0].y, wv[st][0].z, wv[st][0].w};
      const uint32_t b1[4] = {wv[st][1].x, wv[st][1].y, wv[st][1].z, wv[st][1].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4i a = *(const v4i*)(tx + xpos(li, 16 * st + 4 * lg + q));
        const uint32_t p0 = valid ? (CANON ? b0[q] : canon_codes(b0[q])) : 0u;
        const uint32_t p1 = valid ? (CANON ? b1[q] : canon_codes(b1[q])) : 0u;
        const v4i o0 = {(int)(p0 & 0x03030303u), (int)((p0 >> 2) & 0x03030303u),
                        (int)((p0 >> 4) & 0x03030303u), (int)((p0 >> 6) & 0x03030303u)};
        const v4i o1 = {(int)(p1 & 0x03030303u), (int)((p1 >> 2) & 0x03030303u),
                        (int)((p1 >> 4) & 0x03030303u), (int)((p1 >> 6) & 0x03030303u)};
        acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, o0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, o1, acc1, 0, 0, 0);
      }
      // the next super-step's decode stays below these MFMAs, so that each
      // super-step waits only for its own weights
      __builtin_amdgcn_sched_barrier(0);
    }
    wave_lds_sync();  // the reads are done before the next slice's writes
    float* __restrict__ part = s_part + (size_t)sl * kFewM * rows_b;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * lg + v;
      part[m * rows_b + grp * 32 + li] = __int_as_float(acc0[v]);
      part[m * rows_b + grp * 32 + 16 + li] = __int_as_float(acc1[v]);
    }
  }
  if (!RAW && tid < kFewM * n_slices) s_sx[sx_m][sx_sl] = sx_v;
  if (!I32 && tid < kFewM) s_inv[tid] = inv_scale_of(sc_v, w_scale);
  __syncthreads();
  small_fold<MODE, kFewM>(s_part, s_sx, s_inv, M, rows_b, N, n_slices, out, out_i32);
}

// ---------------------------------------------------------------------------
// Generic product for any K (K % 64 != 0 or very long rows): one wave per
// row, plain int8 activations, 1024-column slices then the K % 4 remainder.
// ---------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void k_generic(const int8_t* __restrict__ xq, int ldx,
                                                 const float* __restrict__ scale_x,
                                                 const uint8_t* __restrict__ W, int N, int K,
                                                 float w_scale, float* __restrict__ out,
                                                 int32_t* __restrict__ out_i32) {
  constexpr bool I32 = MODE == 2;
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= N) return;  // whole wave leaves together
  const int8_t* __restrict__ xr = xq + (size_t)m * ldx;
  const uint8_t* __restrict__ row = W + (size_t)r * ((K + 3) / 4);
  const int n_groups = K / 4;
  const float inv = I32 ? 0.0f : inv_scale_of(scale_x[m], w_scale);
  float o = 0.0f;
  int tot = 0;
  for (int g0 = 0; g0 < n_groups; g0 += 256) {
    const int g1 = min(g0 + 256, n_groups);
    int part = 0;
    for (int g = g0 + lane; g < g1; g += 64) {
      const uint32_t b = row[g];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int w = (int)((b >> (2 * j)) & 3u) - 1;
        w = w > 1 ? 1 : w;
        part += w * (int)xr[4 * g + j];
      }
    }
    part = wave_sum_i32(part);
    if (I32)
      tot += part;
    else
      o = __fadd_rn(o, __fmul_rn((float)part, inv));
  }
  if (4 * n_groups < K) {
    int rem = 0;
    const uint32_t b = row[n_groups];
    for (int c = 4 * n_groups; c < K; ++c) {
      int w = (int)((b >> (2 * (c & 3))) & 3u) - 1;
      w = w > 1 ? 1 : w;
      rem += w * (int)xr[c];
    }
    if (I32)
      tot += rem;
    else
      o = __fadd_rn(o, __fmul_rn((float)rem, inv));
  }
  if (lane == 0) {
    if (I32)
      out_i32[(size_t)m * N + r] = tot;
    else
      out[(size_t)m * N + r] = MODE == 1 ? __fadd_rn(out[(size_t)m * N + r], o) : o;
  }
}

// ---------------------------------------------------------------------------
// Prefill / batched GEMM on int8 MFMA (v_mfma_i32_32x32x32_i8).
//   A block of WM x WN waves owns a (32 MT WM) x (32 NTW WN) output tile;
//   each wave MT x NTW MFMA tiles of 32 x 32.  K runs in stages
//   of BK = 256 columns (128 when K is an odd multiple of 128) through an
//   LDS ring of NBUF stages: A (the tile's rows of permuted int8
//   activations) and B (the tile's weight rows, BK/4 packed bytes each) go
//   straight from global memory into LDS (global_load_lds_dwordx4: each
//   lane's 16 bytes land at the instruction's LDS base + 16 * lane, so the
//   swizzle is applied to the global side), NBUF stages ahead of their use;
//   each wave waits for its own loads of the next stage (vmcnt) and one
//   barrier per stage publishes it.  Operands are read one 32-deep step
//   ahead of their MFMAs, so the LDS latency hides behind the current
//   step.  LDS serves a 16-byte read for 16 lanes per cycle from 64 banks:
//   A's 16-byte chunks are XOR-swizzled by row (row/2 mod 8 for 8 chunks
//   per row, row mod 16 for 16) and B's chunks by column, so the operand
//   reads of 16 consecutive rows hit 16 different bank groups.
//   Lane (j = lane%32, h = lane/32) covers columns kb + (BK/2) h + 16 s ..
//   in step s, for A and B alike; its packed weight dword of step s decodes
//   to the four int8 operand dwords (codes 0, 1, 2 as they are).  Each
//   1024-column slice's accumulators start from -(slice sum of x) as the
//   C operand of the slice's first MFMA (w = code - 1), and are folded into
//   fp32 in slice order at its end (src/kernel.c:255-256, 407-425).
// ---------------------------------------------------------------------------
constexpr int GBK = 128;         // K granularity of the MFMA GEMM
constexpr int GMAX_SLICES = 16;  // K <= 16384

// Output tile of a block.  Workgroups go to the 8 XCDs round robin
// (block b on XCD b % 8), each XCD with its own L2: every XCD is given one
// contiguous run of tiles, walked in groups of 8 tile rows so that the
// blocks resident at once share their A rows and weight columns in L2.
__device__ __forceinline__ void gemm_tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nb = tiles_m * tiles_n;
  const int xcd = b % 8, local = b / 8;
  const int per = nb / 8, extra = nb % 8;
  const int t = xcd * per + min(xcd, extra) + local;
  constexpr int G = 8;
  const int g = t / (G * tiles_n);
  const int rows = min(G, tiles_m - g * G);
  const int r = t - g * G * tiles_n;
  tm = g * G + r % rows;
  tn = r / rows;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16 bytes per lane from sbase + voff into LDS at lds_base + 16 * lane.
// The compiler does not see the LDS write: completion is awaited with
// wait_vm and published with a barrier.
__device__ __forceinline__ void lds_load16(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(
                   __builtin_amdgcn_readfirstlane(lds_base)),
               "v"(voff), "s"(sbase));
}
// wait until at most N of this wave's vector memory operations are pending
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
template <int NCH>
__device__ __forceinline__ int gemm_a_swz(int r) {
  return NCH == 8 ? ((r >> 1) & 7) : (r & 15);
}
template <int NBC>
__device__ __forceinline__ int gemm_b_swz(int n) {
  return NBC == 2 ? ((n >> 3) & 1) : ((n >> 2) & 3);
}

template <bool CANON, int MODE, int MT, int NTW, int WM, int WN, int NBUF, int OCC, int BK>
__global__ __launch_bounds__(64 * WM * WN, OCC) void k_gemm(const uint8_t* __restrict__ act,
                                                      size_t act_stride,
                                                      const float* __restrict__ scale_x, int M,
                                                      const uint8_t* __restrict__ W, int N, int K,
                                                      float w_scale, float* __restrict__ out,
                                                      int32_t* __restrict__ out_i32, int ldo) {
  static_assert(BK == 128 || BK == 256, "stage depth");
  constexpr bool I32 = MODE == 2;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int BM = 32 * MT * WM, BN = 32 * NTW * WN;
  constexpr int NCH = BK / 16, BB = BK / 4, NBC = BB / 16;  // A chunks per row; B bytes, chunks per column
  constexpr int NQ = BK / 32;                                 // 32-deep steps per stage
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BB;
  static_assert((A_BYTES / 16) % NT == 0 && (B_BYTES / 16) % NT == 0, "stage chunks per thread");
  constexpr int NA = A_BYTES / 16 / NT, NB = B_BYTES / 16 / NT, PER = NA + NB;
  constexpr int SPS = kSlice / BK;  // stages per slice
  __shared__ __attribute__((aligned(16))) uint8_t sA[NBUF][A_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sB[NBUF][B_BYTES];
  __shared__ __attribute__((aligned(16))) int s_sx[GMAX_SLICES][BM];
  __shared__ __attribute__((aligned(16))) float s_inv[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / WN, wn = w % WN;
  const int j32 = lane & 31, h = lane >> 5;
  int tm, tn;
  gemm_tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const size_t wstride = (size_t)(K >> 2);
  const int n_sl = slices_of(K);
  const int n_st = K / BK;

  // each thread's stage loads: LDS slot s = (i NW + w) 64 + lane of A
  // (row s / NCH, position s % NCH) and of B (column s / NBC); rows and
  // columns past M / N reload the last one
  uint32_t a_off[NA], b_off[NB];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int s = (i * NW + w) * 64 + lane;
    const int row = s / NCH, c = (s % NCH) ^ gemm_a_swz<NCH>(row);
    a_off[i] = (uint32_t)((min(m0 + row, M - 1) - m0) * act_stride) + 16 * c;
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int s = (i * NW + w) * 64 + lane;
    const int col = s / NBC, c = (s % NBC) ^ gemm_b_swz<NBC>(col);
    b_off[i] = (uint32_t)((min(n0 + col, N - 1) - n0) * wstride) + 16 * c;
  }
  const uint8_t* a_base = act + (size_t)m0 * act_stride + act_perm_off(K);
  const uint8_t* b_base = W + (size_t)n0 * wstride;
  auto issue = [&](int st) __attribute__((always_inline)) {
    const int buf = st % NBUF;
    const uint8_t* ab = a_base + (size_t)st * BK;
    const uint8_t* bb = b_base + (size_t)st * BB;
#pragma unroll
    for (int i = 0; i < NA; ++i) lds_load16(ab, a_off[i], lds_addr(&sA[buf][(i * NW + w) * 1024]));
#pragma unroll
    for (int i = 0; i < NB; ++i) lds_load16(bb, b_off[i], lds_addr(&sB[buf][(i * NW + w) * 1024]));
  };

  // per-row slice sums of x and 1/(scale_x * w_scale)
  for (int i = tid; i < BM * n_sl; i += NT) {
    const int r = i % BM, sl = i / BM;
    const int row = min(m0 + r, M - 1);
    s_sx[sl][r] = ((const int*)(act + (size_t)row * act_stride))[sl];
  }
  if (tid < BM) {
    const int row = min(m0 + tid, M - 1);
    s_inv[tid] = I32 ? 0.0f : inv_scale_of(scale_x[row], w_scale);
  }

  v4i fa[2][MT];     // A operands of the current and the next step
  uint4 fb[2][NTW];  // packed B of four steps
  auto read_a = [&](int st, int q, v4i (&d)[MT]) __attribute__((always_inline)) {
    const uint8_t* cA = sA[st % NBUF];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = (wm * MT + mt) * 32 + j32;
      d[mt] = *(const v4i*)(cA + r * BK + 16 * (((NCH / 2) * h + q) ^ gemm_a_swz<NCH>(r)));
    }
  };
  auto read_b = [&](int st, int u, uint4 (&d)[NTW]) __attribute__((always_inline)) {
    const uint8_t* cB = sB[st % NBUF];
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int col = (wn * NTW + nt) * 32 + j32;
      d[nt] = *(const uint4*)(cB + col * BB + 16 * (((NBC / 2) * h + u) ^ gemm_b_swz<NBC>(col)));
    }
  };

  v16i acc[MT][NTW];
  float o[MT][NTW][16];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NTW; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        acc[a][b][v] = 0;
        o[a][b][v] = 0.0f;
      }

  // stages 0 .. NBUF-1 in flight, stage 0 published
#pragma unroll
  for (int i = 0; i < NBUF; ++i)
    if (i < n_st) issue(i);
  {
    const int later = min(NBUF - 1, n_st - 1);
    if (later >= 3) wait_vm<3 * PER>();
    else if (later == 2) wait_vm<2 * PER>();
    else if (later == 1) wait_vm<PER>();
    else wait_vm<0>();
  }
  __syncthreads();
  read_a(0, 0, fa[0]);
  read_b(0, 0, fb[0]);

  auto stage = [&](int st, auto pb_c) __attribute__((always_inline)) {
    // NQ = 4: fb[PB] holds the stage's B and the next stage's goes to
    // fb[PB ^ 1]; NQ = 8: fb[0] and fb[1] hold steps 0..3 and 4..7
    constexpr int PB = NQ == 4 ? decltype(pb_c)::value : 0;
    const bool first = I32 ? st == 0 : st % SPS == 0;
    const int sl = st / SPS;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (q < NQ - 1) {
        read_a(st, q + 1, fa[(q + 1) & 1]);
        if (NQ == 8 && q == 3) read_b(st, 1, fb[1]);
      } else if (st + 1 < n_st) {
        // publish stage st+1 (this wave's loads, then the barrier), refill
        // the buffer of stage st, read the next stage's first operands
        const int later = min(NBUF - 2, n_st - 2 - st);
        if (later >= 2) wait_vm<2 * PER>();
        else if (later == 1) wait_vm<PER>();
        else wait_vm<0>();
        __syncthreads();
        if (st + NBUF < n_st) issue(st + NBUF);
        read_a(st + 1, 0, fa[0]);
        read_b(st + 1, 0, fb[NQ == 4 ? PB ^ 1 : 0]);
      }
      v4i bop[NTW];
      const int cb = NQ == 4 ? PB : q / 4;
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const uint4 bw = fb[cb][nt];
        const uint32_t w4[4] = {bw.x, bw.y, bw.z, bw.w};
        const uint32_t pw = CANON ? w4[q & 3] : canon_codes(w4[q & 3]);
        bop[nt][0] = (int)(pw & 0x03030303u);
        bop[nt][1] = (int)((pw >> 2) & 0x03030303u);
        bop[nt][2] = (int)((pw >> 4) & 0x03030303u);
        bop[nt][3] = (int)((pw >> 6) & 0x03030303u);
      }
      const v4i (&aq)[MT] = fa[q & 1];
      if (q == 0 && first) {
        // accumulators start at -(slice sum of x) of their rows (I32: of all slices)
        v16i c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            // rows 8g + 4h + (0..3) of the MFMA tile: elements 4g .. 4g+3
            const int r0 = (wm * MT + mt) * 32 + 8 * g + 4 * h;
            int4 sx4;
            if (I32) {
              sx4 = make_int4(0, 0, 0, 0);
              for (int s2 = 0; s2 < n_sl; ++s2) {
                const int4 t4 = *(const int4*)&s_sx[s2][r0];
                sx4.x += t4.x;
                sx4.y += t4.y;
                sx4.z += t4.z;
                sx4.w += t4.w;
              }
            } else {
              sx4 = *(const int4*)&s_sx[sl][r0];
            }
            c[mt][4 * g + 0] = -sx4.x;
            c[mt][4 * g + 1] = -sx4.y;
            c[mt][4 * g + 2] = -sx4.z;
            c[mt][4 * g + 3] = -sx4.w;
          }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq[mt], bop[nt], c[mt], 0, 0, 0);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
            acc[mt][nt] =
                __builtin_amdgcn_mfma_i32_32x32x32_i8(aq[mt], bop[nt], acc[mt][nt], 0, 0, 0);
      }
      if constexpr (NTW == 2) {
        // 128 x 256 tiles (two B operands per step): the step's weight decode
        // first, then its four MFMAs each followed by one LDS read of the
        // next step's operands (M=4096, K=N=8192: 1-5 % faster per product
        // over two boxes, 247-253 against 249-255 us on one; on the other
        // tile shapes the same order measured 1-3 % slower, so they keep the
        // compiler's)
        if (q < NQ - 1) {
          __builtin_amdgcn_sched_group_barrier(0x002, 4 * NTW, 0);
#pragma unroll
          for (int i = 0; i < MT * NTW; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
      }
    }
    if (!I32 && (st % SPS == SPS - 1 || st + 1 == n_st)) {
      // the slice's fp32 term, added in slice order (the first to 0)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float inv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 in4 = *(const float4*)&s_inv[(wm * MT + mt) * 32 + 8 * g + 4 * h];
          inv[4 * g + 0] = in4.x;
          inv[4 * g + 1] = in4.y;
          inv[4 * g + 2] = in4.z;
          inv[4 * g + 3] = in4.w;
        }
        if (sl == 0) {
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              o[mt][nt][v] = __fadd_rn(0.0f, __fmul_rn((float)acc[mt][nt][v], inv[v]));
        } else {
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              o[mt][nt][v] = __fadd_rn(o[mt][nt][v], __fmul_rn((float)acc[mt][nt][v], inv[v]));
        }
      }
    }
  };

  int st = 0;
  for (; st + 2 <= n_st; st += 2) {
    stage(st, std::integral_constant<int, 0>());
    stage(st + 1, std::integral_constant<int, 1>());
  }
  if (st < n_st) stage(st, std::integral_constant<int, 0>());

  if (I32) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[mt][nt][v] = __int_as_float(acc[mt][nt][v]);
  }

  if (MODE == 1 && !I32) {
    // residual add: every residual load in flight before the first add (a
    // guarded load + add + store per element waits out one load latency per
    // element); rows and columns past M / N read the last one and store nothing
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int n = min(n0 + (wn * NTW + nt) * 32 + j32, N - 1);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = min(m0 + (wm * MT + mt) * 32 + 8 * (v >> 2) + 4 * h + (v & 3), M - 1);
          o[mt][nt][v] = __fadd_rn(out[(size_t)r * ldo + n], o[mt][nt][v]);
        }
      }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int n = n0 + (wn * NTW + nt) * 32 + j32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = m0 + (wm * MT + mt) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (r < M && n < N) {
          if (I32)
            out_i32[(size_t)r * ldo + n] = __float_as_int(o[mt][nt][v]);
          else
            out[(size_t)r * ldo + n] = o[mt][nt][v];
        }
      }
    }
}

__global__ void k_canonicalize(uint32_t* __restrict__ p, size_t n_words) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n_words;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = canon_codes(p[i]);
}

__global__ void k_residual_add(float* __restrict__ x, const float* __restrict__ o, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    x[i] = __fadd_rn(x[i], o[i]);
}

__global__ void k_canonicalize_tail(uint8_t* __restrict__ p, size_t n) {
  const size_t i = threadIdx.x;
  if (i < n) p[i] = (uint8_t)canon_codes(p[i]);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
hipError_t launch_quantize(const float* x, int M, int n, int x_stride, const float* gamma,
                           float* x_norm, int8_t* xq, int quant_stride, float* scale_x,
                           uint8_t* act, hipStream_t s, bool nibbles, bool fast) {
  if (M <= 0) return hipSuccess;
  // one wave per token when the rows allow 16-byte loads of whole groups
  const bool aligned = ((uintptr_t)x % 16 == 0) && (x_stride % 4 == 0) &&
                       ((uintptr_t)gamma % 16 == 0) && (!x_norm || (uintptr_t)x_norm % 16 == 0);
  if (aligned && (n == 1024 || n == 2048 || n == 4096)) {
    const int tpb = quantize_wave_tpb(n);
    const dim3 grid((M + tpb - 1) / tpb), block(64 * tpb);
    const size_t lds = quantize_wave_lds(n);
    if (n == 1024)
      hipLaunchKernelGGL(k_quantize_wave<1>, grid, block, lds, s, x, M, x_stride, gamma, x_norm,
                         xq, quant_stride, scale_x, act, act_row_bytes(n), nibbles, fast);
    else if (n == 2048)
      hipLaunchKernelGGL(k_quantize_wave<2>, grid, block, lds, s, x, M, x_stride, gamma, x_norm,
                         xq, quant_stride, scale_x, act, act_row_bytes(n), nibbles, fast);
    else
      hipLaunchKernelGGL(k_quantize_wave<4>, grid, block, lds, s, x, M, x_stride, gamma, x_norm,
                         xq, quant_stride, scale_x, act, act_row_bytes(n), nibbles, fast);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_quantize, dim3(M), dim3(QT), 0, s, x, n, x_stride, gamma, x_norm, xq,
                     quant_stride, scale_x, (float*)nullptr, act, act_row_bytes(n));
  return hipGetLastError();
}

hipError_t launch_residual_add(float* x, const float* o, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_residual_add, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256),
                     0, s, x, o, n);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, int n, const float* gamma, float* out, float* max_out,
                           hipStream_t s) {
  hipLaunchKernelGGL(k_quantize, dim3(1), dim3(QT), 0, s, x, n, n, gamma, out, (int8_t*)nullptr,
                     0, (float*)nullptr, max_out, (uint8_t*)nullptr, (size_t)0);
  return hipGetLastError();
}

hipError_t launch_prep_i8(const int8_t* xq, int M, int ldx, int K, uint8_t* act, bool nib,
                          hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (nib)
    hipLaunchKernelGGL(k_prep_i8<true>, dim3(M), dim3(QT), 0, s, xq, ldx, K, act,
                       act_row_bytes(K));
  else
    hipLaunchKernelGGL(k_prep_i8<false>, dim3(M), dim3(QT), 0, s, xq, ldx, K, act,
                       act_row_bytes(K));
  return hipGetLastError();
}

// rows per wave: as many as keep >= 8 waves per CU busy (256 CUs)
template <int T, int P, bool CANON, int MODE>
static hipError_t gemv_t(const uint8_t* act, const float* scale_x, int M, const uint8_t* W, int N,
                         int K, float w_scale, void* out, hipStream_t s) {
  constexpr int RPW = 64 / T;
  const long long n_rg = (N + RPW - 1) / RPW;
  const long long want = 8LL * 256 * 4 / (M < 4 ? M : 4);  // waves wanted in all
  auto go = [&](auto gw) {
    constexpr int GW = decltype(gw)::value;
    const long long waves = (n_rg + GW - 1) / GW;
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    hipLaunchKernelGGL((k_gemv<T, P, GW, CANON, MODE>), dim3(blocks, M), dim3(256), 0, s, act,
                       act_row_bytes(K), scale_x, W, N, K, w_scale, (float*)out, (int32_t*)out);
    return hipGetLastError();
  };
  // (16 groups per wave measured slower than 8: fewer waves fit per SIMD)
  if (n_rg >= 8 * want) return go(std::integral_constant<int, 8>());
  if (n_rg >= 4 * want) return go(std::integral_constant<int, 4>());
  if (n_rg >= 2 * want) return go(std::integral_constant<int, 2>());
  return go(std::integral_constant<int, 1>());
}

template <int T, int P, bool CANON, int MODE>
static hipError_t gemv_mt_t(const uint8_t* act, const float* scale_x, int M, const uint8_t* W,
                            int N, int K, float w_scale, void* out, hipStream_t s) {
  constexpr int RPW = 64 / T;
  constexpr int GW = P == 1 ? 8 : 4;
  const long long n_rg = (N + RPW - 1) / RPW;
  const long long waves = (n_rg + GW - 1) / GW;
  hipLaunchKernelGGL((k_gemv_mt<T, P, GW, CANON, MODE>), dim3((unsigned)((waves + 3) / 4)),
                     dim3(256), 0, s, act, act_row_bytes(K), scale_x, M, W, N, K, w_scale,
                     (float*)out, (int32_t*)out);
  return hipGetLastError();
}

template <bool CANON, int MODE>
static hipError_t gemv_dispatch(const uint8_t* act, const float* scale_x, int M, const uint8_t* W,
                                int N, int K, float w_scale, void* out, hipStream_t s) {
  if (M >= 2 && M <= kMtMaxM && K <= kMtMaxK) {
    if (K <= 1024) return gemv_mt_t<16, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
    if (K <= 2048) return gemv_mt_t<32, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
    if (K <= 4096) return gemv_mt_t<64, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
    return gemv_mt_t<64, 2, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  }
  if (K <= 1024) return gemv_t<16, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  if (K <= 2048) return gemv_t<32, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  if (K <= 4096) return gemv_t<64, 1, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  if (K <= 8192) return gemv_t<64, 2, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  return gemv_t<64, 4, CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
}

// Tile shape per product: the one with the least estimated time.  With n
// the tiles of the busiest CU (ceil(tiles / 256)), a shape's time is
// modelled as (K/1024 + 0.5) (a + b (n - 1)) us: a is one tile alone on its
// CU, b each further tile sharing it.  Fitted to the measured times of three
// shapes at M = 129..4096, K = 1024..8192 (14 products): 64 x 64 a = 3.0,
// b = 1.2; 64 x 128 a = 3.7, b = 2.1; 128 x 256 a = 7.0, b = 8.8; the
// estimate picks the fastest shape or one within 7 % of it on all 14.
// Tiles of 4096 outputs run as 32 x 128 (4 waves of 32 x 32, four blocks
// per CU), which measured 2-11 % faster than 64 x 64 on the seven products
// the estimate gives them (M = 300..1536, K = 1024..4096), and also replace
// 64 x 128 tiles that would leave CUs idle (at most one per CU): M = 1024,
// K = 4096 -> 2048 in 14.0 us against 15.6; with more tiles they lose
// (M = 1024, K = 2048 -> 8384: 27.5 against 26.4 us).  Where 64 x 128 tiles
// come two per CU, 64 x 256 tiles (8 waves of 64 x 32, one block per CU)
// read each activation tile once instead of twice and measured 3-8 %
// faster on seven such products (M = 2048, K = 4096 -> 2048: 22.1 against
// 23.1 us); at more tiles per CU they lose (M = 2048, K = 2048 -> 8512:
// 53.6 against 45.3 us).  128 x 256 tiles win only at long K or many tiles
// per CU (K >= 8192: 3-15 % faster than 64 x 128 on six products; M = 4096,
// K = 4096 -> 8192, four tiles per CU: 5 %) and lost 3-19 % on the four
// shorter products the estimate gave them (M = 1600..2560, K = 2048, 4096),
// so they are considered only there.  All but 64 x 128 take K % 256 == 0.
constexpr int kCUs = 256;
enum { GEMM_32x128 = 0, GEMM_64x128 = 1, GEMM_128x256 = 2, GEMM_64x256 = 3 };
static int gemm_shape(int M, int N, int K) {
  struct Cand {
    int shape, bm, bn;
    double a, b;
  };
  const Cand cands[3] = {{GEMM_32x128, 64, 64, 3.0, 1.2},  // fitted on 64 x 64 tiles
                         {GEMM_64x128, 64, 128, 3.7, 2.1},
                         {GEMM_128x256, 128, 256, 7.0, 8.8}};
  int best = GEMM_64x128;
  double best_t = 1e300;
  for (const Cand& c : cands) {
    if (c.shape != GEMM_64x128 && K % 256 != 0) continue;
    const long long tiles = (long long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    const long long n = (tiles + kCUs - 1) / kCUs;
    if (c.shape == GEMM_128x256 && K < 8192 && n < 4) continue;
    const double t = (K / 1024.0 + 0.5) * (c.a + c.b * (double)(n - 1));
    if (t < best_t) {
      best_t = t;
      best = c.shape;
    }
  }
  const long long tiles64x128 = (long long)((M + 63) / 64) * ((N + 127) / 128);
  if (best == GEMM_64x128 && K % 256 == 0 && tiles64x128 <= 2 * kCUs)
    best = tiles64x128 <= kCUs ? GEMM_32x128 : GEMM_64x256;
  return best;
}

// stage depth 256 when K allows, else 128 (DEEP_ONLY shapes: 256 only); the
// LDS ring holds two 256-deep stages or three 128-deep ones
template <bool CANON, int MODE, int MT, int NTW, int WM, int WN, int OCC, bool DEEP_ONLY = false>
static void gemm_launch_tile(const uint8_t* act, const float* scale_x, int M, const uint8_t* W,
                             int N, int K, float w_scale, void* out, int ldo, hipStream_t s) {
  constexpr int BM = 32 * MT * WM, BN = 32 * NTW * WN;
  const dim3 grid((unsigned)((M + BM - 1) / BM * ((N + BN - 1) / BN)));
  if (DEEP_ONLY || K % 256 == 0)
    hipLaunchKernelGGL((k_gemm<CANON, MODE, MT, NTW, WM, WN, 2, OCC, 256>), grid,
                       dim3(64 * WM * WN), 0, s, act, act_row_bytes(K), scale_x, M, W, N, K,
                       w_scale, (float*)out, (int32_t*)out, ldo);
  else if constexpr (!DEEP_ONLY)
    hipLaunchKernelGGL((k_gemm<CANON, MODE, MT, NTW, WM, WN, 3, OCC, 128>), grid,
                       dim3(64 * WM * WN), 0, s, act, act_row_bytes(K), scale_x, M, W, N, K,
                       w_scale, (float*)out, (int32_t*)out, ldo);
}

template <bool CANON, int MODE>
static hipError_t gemm_t(const uint8_t* act, const float* scale_x, int M, const uint8_t* W, int N,
                         int K, float w_scale, void* out, hipStream_t s) {
  const int shape = gemm_shape(M, N, K);
  // 128 x 256: 2 x 4 waves of 64 x 64; 64 x 128: 1 x 4 waves of 64 x 32 (half
  // the B decode per MFMA of 2 x 2 waves of 32 x 64, 2-5 % faster);
  // 64 x 256: 1 x 8 waves of 64 x 32; 32 x 128: 1 x 4 waves of 32 x 32
  if (shape == GEMM_128x256)
    gemm_launch_tile<CANON, MODE, 2, 2, 2, 4, 1, true>(act, scale_x, M, W, N, K, w_scale, out, N,
                                                       s);
  else if (shape == GEMM_64x128)
    gemm_launch_tile<CANON, MODE, 2, 1, 1, 4, 3>(act, scale_x, M, W, N, K, w_scale, out, N, s);
  else if (shape == GEMM_64x256)
    gemm_launch_tile<CANON, MODE, 2, 1, 1, 8, 2, true>(act, scale_x, M, W, N, K, w_scale, out, N,
                                                       s);
  else
    gemm_launch_tile<CANON, MODE, 1, 1, 1, 4, 4, true>(act, scale_x, M, W, N, K, w_scale, out, N,
                                                       s);
  return hipGetLastError();
}

// blocks of one k_gemm_small (or k_gemm_few) launch
static long long small_blocks(int M, int N, int K) {
  const int gpb = 8 / sm_wpg(slices_of(K));
  return (long long)((N + 32 * gpb - 1) / (32 * gpb)) * ((M + kSmMaxM - 1) / kSmMaxM);
}

// which kernel serves a product of this shape: 0 generic, 1 GEMV per token,
// 2 MFMA GEMM, 3 few-token MFMA (k_gemm_few for up to 16 tokens at
// K <= 8192, else k_gemm_small).  Few tokens: up to 32 always; up to 256
// while one launch fits one block per CU, where it measured faster than the
// 128-row GEMM tiles (K=4096 -> 2048: 9-11 us against 23 us at M = 32-256;
// K=2048 -> 8384: 9.5 us against 14 us at M = 32, 64)
static int product_path(int M, int N, int K) {
  if (K % 64 != 0 || K > 16384) return 0;
  if (M >= 2 && K % 128 == 0 &&
      (M <= kSmMaxM || (M <= kSmMaxTokens && small_blocks(M, N, K) <= 256)))
    return 3;
  if (M >= 32 && K % GBK == 0) return 2;
  return 1;
}

template <bool CANON, int MODE>
static hipError_t product_t(const uint8_t* act, const float* scale_x, int M, const uint8_t* W,
                            int N, int K, float w_scale, void* out, hipStream_t s) {
  const int path = product_path(M, N, K);
  if (path == 2) return gemm_t<CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
  if (path == 3) {
    const int n_slices = slices_of(K), gpb = 8 / sm_wpg(n_slices);
    const dim3 grid((N + 32 * gpb - 1) / (32 * gpb), (M + kSmMaxM - 1) / kSmMaxM);
    const size_t lds = (size_t)n_slices * kSmMaxM * 32 * gpb * sizeof(float);
    if (M <= kFewM && n_slices <= kFewMaxSlices) {
      const bool big = few_stream(N, K);
      const size_t fl = few_lds(K), ab = act_row_bytes(K);
      if (M <= 8 && big)
        hipLaunchKernelGGL((k_gemm_few<CANON, MODE, 1, false, true>), grid, dim3(512), fl, s, act,
                           ab, scale_x, M, W, N, K, w_scale, (float*)out, (int32_t*)out);
      else if (M <= 8)
        hipLaunchKernelGGL((k_gemm_few<CANON, MODE, 1, false, false>), grid, dim3(512), fl, s, act,
                           ab, scale_x, M, W, N, K, w_scale, (float*)out, (int32_t*)out);
      else if (big)
        hipLaunchKernelGGL((k_gemm_few<CANON, MODE, 2, false, true>), grid, dim3(512), fl, s, act,
                           ab, scale_x, M, W, N, K, w_scale, (float*)out, (int32_t*)out);
      else
        hipLaunchKernelGGL((k_gemm_few<CANON, MODE, 2, false, false>), grid, dim3(512), fl, s, act,
                           ab, scale_x, M, W, N, K, w_scale, (float*)out, (int32_t*)out);
      return hipGetLastError();
    }
    // 8-token groups of A that a block loads: what its tile of up to 32
    // tokens needs
    if (M <= 8)
      hipLaunchKernelGGL((k_gemm_small<CANON, MODE, 1, false>), grid, dim3(512), lds, s, act,
                         act_row_bytes(K), scale_x, M, W, N, K, w_scale, (float*)out,
                         (int32_t*)out);
    else if (M <= 16)
      hipLaunchKernelGGL((k_gemm_small<CANON, MODE, 2, false>), grid, dim3(512), lds, s, act,
                         act_row_bytes(K), scale_x, M, W, N, K, w_scale, (float*)out,
                         (int32_t*)out);
    else
      hipLaunchKernelGGL((k_gemm_small<CANON, MODE, 4, false>), grid, dim3(512), lds, s, act,
                         act_row_bytes(K), scale_x, M, W, N, K, w_scale, (float*)out,
                         (int32_t*)out);
    return hipGetLastError();
  }
  return gemv_dispatch<CANON, MODE>(act, scale_x, M, W, N, K, w_scale, out, s);
}

template <bool CANON, int MT8>
static void small_i8_t(dim3 grid, size_t lds, const int8_t* xq, int M, int ldx, int K,
                       const uint8_t* W, int N, int32_t* out, hipStream_t s) {
  hipLaunchKernelGGL((k_gemm_small<CANON, MODE_I32, MT8, true>), grid, dim3(512), lds, s,
                     (const uint8_t*)xq, (size_t)ldx, (const float*)nullptr, M, W, N, K, 0.0f,
                     (float*)nullptr, out);
}

template <bool CANON, int MT8>
static void few_i8_t(dim3 grid, int K, const int8_t* xq, int M, int ldx, const uint8_t* W, int N,
                     int32_t* out, hipStream_t s) {
  if (few_stream(N, K))
    hipLaunchKernelGGL((k_gemm_few<CANON, MODE_I32, MT8, true, true>), grid, dim3(512),
                       few_lds(K), s, (const uint8_t*)xq, (size_t)ldx, (const float*)nullptr, M,
                       W, N, K, 0.0f, (float*)nullptr, out);
  else
    hipLaunchKernelGGL((k_gemm_few<CANON, MODE_I32, MT8, true, false>), grid, dim3(512),
                       few_lds(K), s, (const uint8_t*)xq, (size_t)ldx, (const float*)nullptr, M,
                       W, N, K, 0.0f, (float*)nullptr, out);
}

hipError_t launch_small_i8(const int8_t* xq, int M, int ldx, int K, const uint8_t* packed, int N,
                           bool canonical, int32_t* out, hipStream_t s) {
  if (product_path(M, N, K) != 3 || ((uintptr_t)xq & 15) != 0 || ldx % 16 != 0)
    return hipErrorNotSupported;
  const int n_slices = slices_of(K), gpb = 8 / sm_wpg(n_slices);
  const dim3 grid((N + 32 * gpb - 1) / (32 * gpb), (M + kSmMaxM - 1) / kSmMaxM);
  const size_t lds = (size_t)n_slices * kSmMaxM * 32 * gpb * sizeof(float);
  if (M <= kFewM && n_slices <= kFewMaxSlices) {
    if (canonical) {
      if (M <= 8) few_i8_t<true, 1>(grid, K, xq, M, ldx, packed, N, out, s);
      else few_i8_t<true, 2>(grid, K, xq, M, ldx, packed, N, out, s);
    } else {
      if (M <= 8) few_i8_t<false, 1>(grid, K, xq, M, ldx, packed, N, out, s);
      else few_i8_t<false, 2>(grid, K, xq, M, ldx, packed, N, out, s);
    }
    return hipGetLastError();
  }
  const int mt8 = M <= 8 ? 1 : (M <= 16 ? 2 : 4);
  if (canonical) {
    if (mt8 == 1) small_i8_t<true, 1>(grid, lds, xq, M, ldx, K, packed, N, out, s);
    else if (mt8 == 2) small_i8_t<true, 2>(grid, lds, xq, M, ldx, K, packed, N, out, s);
    else small_i8_t<true, 4>(grid, lds, xq, M, ldx, K, packed, N, out, s);
  } else {
    if (mt8 == 1) small_i8_t<false, 1>(grid, lds, xq, M, ldx, K, packed, N, out, s);
    else if (mt8 == 2) small_i8_t<false, 2>(grid, lds, xq, M, ldx, K, packed, N, out, s);
    else small_i8_t<false, 4>(grid, lds, xq, M, ldx, K, packed, N, out, s);
  }
  return hipGetLastError();
}

hipError_t launch_product(const uint8_t* act, const float* scale_x, int M, const uint8_t* packed,
                          int N, int K, float w_scale, bool canonical, void* out, int mode,
                          hipStream_t s) {
  if (product_path(M, N, K) == 0) return hipErrorInvalidValue;  // caller uses launch_generic
  if (canonical) {
    if (mode == MODE_I32) return product_t<true, 2>(act, scale_x, M, packed, N, K, w_scale, out, s);
    if (mode == MODE_ACC) return product_t<true, 1>(act, scale_x, M, packed, N, K, w_scale, out, s);
    return product_t<true, 0>(act, scale_x, M, packed, N, K, w_scale, out, s);
  }
  if (mode == MODE_I32) return product_t<false, 2>(act, scale_x, M, packed, N, K, w_scale, out, s);
  if (mode == MODE_ACC) return product_t<false, 1>(act, scale_x, M, packed, N, K, w_scale, out, s);
  return product_t<false, 0>(act, scale_x, M, packed, N, K, w_scale, out, s);
}

bool product_needs_generic(int M, int K) { return product_path(M, 1, K) == 0; }

bool product_reads_nibbles(int M, int N, int K) {
  const int path = product_path(M, N, K);
  return path != 2 && path != 3;
}

hipError_t launch_generic(const int8_t* xq, int ldx, const float* scale_x, int M,
                          const uint8_t* packed, int N, int K, float w_scale, void* out, int mode,
                          hipStream_t s) {
  dim3 grid((N + 3) / 4, M);
  float* of = (float*)out;
  int32_t* oi = (int32_t*)out;
  if (mode == MODE_I32)
    hipLaunchKernelGGL(k_generic<2>, grid, dim3(256), 0, s, xq, ldx, scale_x, packed, N, K,
                       w_scale, of, oi);
  else if (mode == MODE_ACC)
    hipLaunchKernelGGL(k_generic<1>, grid, dim3(256), 0, s, xq, ldx, scale_x, packed, N, K,
                       w_scale, of, oi);
  else
    hipLaunchKernelGGL(k_generic<0>, grid, dim3(256), 0, s, xq, ldx, scale_x, packed, N, K,
                       w_scale, of, oi);
  return hipGetLastError();
}

hipError_t launch_canonicalize(uint8_t* p, size_t bytes, hipStream_t s) {
  const size_t words = bytes / 4;
  if (words) {
    int blocks = (int)((words + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_canonicalize, dim3(blocks), dim3(256), 0, s, (uint32_t*)p, words);
  }
  if (bytes % 4)
    hipLaunchKernelGGL(k_canonicalize_tail, dim3(1), dim3(64), 0, s, p + 4 * words, bytes % 4);
  return hipGetLastError();
}

}  // namespace bm
