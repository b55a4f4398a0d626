// Fused single-token decode kernels (bs = 1).
//
// A decoded token runs, per layer,
//   k_rows_fused  in_proj: quantize x (block prologue) + GEMV over the
//                 layer's in_proj rows, stored on the device per head as
//                 [z (hd) | x (hd) | B | C | dt]
//   k_ssm_heads   the SSM step of every channel (src/kernel.c:34-70)
//   k_rows_fused  out_proj: quantize y + GEMV, residual add fused into the
//                 store (src/model.c:1214-1215)
// then the LM head (k_rows_fused with the final RMSNorm in front,
// src/model.c:1225, 1259-1261, and a per-block greedy candidate) and
// k_pick, which finishes the greedy choice (src/model.c:143-154), advances
// the step state and writes the next token's embedding.
//
// Every block recomputes the RMSNorm/int8 prologue of its input.  Its
// critical path is the sequential sum of squares (four fp32 chains,
// src/kernel.c:77-89): the chains run from registers of one wave, one
// dependent add per element, while the block's weight rows are already in
// flight.  All elementwise prologue work runs on register-resident copies of
// the input.  Kernel boundaries order the phases; no grid-wide fences.
#include <type_traits>

#include "bm_dev.h"
#include "bm_libm.h"

namespace bm {

// control words shared with bm_model.hip.  CTL_DONE: 0 steps always run,
// 1 armed (generate with stop_on_eos), 2 the end token was picked: every
// later step leaves the state, the activations, the logits and the
// bookkeeping untouched, so the state stops where the reference's loop
// stops (src/main.c:473-500)
// (CTL_DONE beside CTL_POS: k_inproj_ssm reads both with one 8-byte load)
enum { CTL_POS = 0, CTL_DONE = 1, CTL_STEP = 2, CTL_HCOUNT = 3, CTL_TOKEN = 4 };
constexpr int kDoneArmed = 1, kDoneStopped = 2;

__device__ __forceinline__ bool is_end_token(int t) { return t == 50256 || t == 0; }
constexpr int kHist = 256;

__device__ __forceinline__ float silu_r(float x) {
  return cr_divf(x, __fadd_rn(1.0f, libm::expf_glibc(-x)));
}

__device__ __forceinline__ float softplus_r(float x) {
  if (x > 20.0f) return x;
  return libm::logf_glibc(__fadd_rn(1.0f, libm::expf_glibc(x)));
}

// ---------------------------------------------------------------------------
// Sum of squares: four sequential chains
// ---------------------------------------------------------------------------

// other K: one lane per chain over LDS, two 32-value buffers alternating
__device__ __forceinline__ void add32(float& s, const float4 (&b)[8]) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    s = __fadd_rn(s, b[u].x);
    s = __fadd_rn(s, b[u].y);
    s = __fadd_rn(s, b[u].z);
    s = __fadd_rn(s, b[u].w);
  }
}

__device__ __forceinline__ void load32(float4 (&b)[8], const float* __restrict__ c) {
#pragma unroll
  for (int u = 0; u < 8; ++u) b[u] = *(const float4*)(c + 4 * u);
}

__device__ __forceinline__ float chain_lds(const float* __restrict__ c, int len) {
  float s = 0.0f;
  int i = 0;
  if (len >= 64) {
    float4 A[8], B[8];
    load32(A, c);
    for (; i + 64 <= len; i += 64) {
      load32(B, c + i + 32);
      add32(s, A);
      if (i + 96 <= len) load32(A, c + i + 64);
      add32(s, B);
    }
  }
  for (; i < len; ++i) s = __fadd_rn(s, c[i]);
  return s;
}

// ---------------------------------------------------------------------------
// Block prologue on register-resident input
//   thread t owns float4 chunks c = t + i*blockDim.x (i < C), i.e. columns
//   4c..4c+3; K % 64 == 0
// ---------------------------------------------------------------------------
template <int C>
__device__ __forceinline__ void stage_load(float4 (&st)[C], const float* __restrict__ src, int K) {
  const int n4 = K >> 2;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = threadIdx.x + i * blockDim.x;
    st[i] = c < n4 ? ((const float4*)src)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

struct Lds {
  float* sq;      // [4][stride] squares, chain-major (padded per segment)
  uint32_t* nib;  // [K/4] split-nibble activations
  int8_t* q8;     // [K] int8 activations
  int* slices;    // [S] sum of int8 per 1024-column slice
  float* bc;      // [32] broadcast words
  int stride;
};

__host__ __device__ inline size_t lds_bytes(int K) {
  return 16 * (size_t)sq_stride_of(K) + 2 * (size_t)K + 4 * (size_t)((K + 1023) / 1024) + 16 + 128;
}

__device__ __forceinline__ Lds lds_carve(uint8_t* base, int K) {
  Lds l;
  l.stride = sq_stride_of(K);
  l.sq = (float*)base;
  l.nib = (uint32_t*)(l.sq + 4 * l.stride);
  l.q8 = (int8_t*)(l.nib + K / 4);
  l.slices = (int*)(l.q8 + K);
  l.bc = (float*)(l.slices + (K + 1023) / 1024 + 4);
  return l;
}

// rms = 1/sqrtf(sum_sq/K + 1e-6f) with the sequential four-chain sum
// (src/kernel.c:77-91)
template <int C>
__device__ float pro_rms(const float4 (&xv)[C], int K, const Lds& l) {
  const int tid = threadIdx.x, nt = blockDim.x, n4 = K >> 2;
  const bool regs = chain_in_regs(K);
  const int E = K >> 6;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = tid + i * nt;
    if (c < n4) {
      const int e = c + (regs ? 4 * (c / E) : 0);
      l.sq[e] = __fmul_rn(xv[i].x, xv[i].x);
      l.sq[l.stride + e] = __fmul_rn(xv[i].y, xv[i].y);
      l.sq[2 * l.stride + e] = __fmul_rn(xv[i].z, xv[i].z);
      l.sq[3 * l.stride + e] = __fmul_rn(xv[i].w, xv[i].w);
    }
  }
  __syncthreads();
  if (tid < 64) {
    float cs = 0.0f;
    if (regs) {
      if (K == 1024)
        cs = chain_regs<16>(l.sq, l.stride, tid);
      else if (K == 2048)
        cs = chain_regs<32>(l.sq, l.stride, tid);
      else
        cs = chain_regs<64>(l.sq, l.stride, tid);
    } else if ((tid & 15) == 15) {
      cs = chain_lds(l.sq + (tid >> 4) * l.stride, n4);
    }
    // lanes 15, 31, 47, 63 hold the chain sums: ((s0+s1)+s2)+s3
    const float s0 = __shfl(cs, 15, 64), s1 = __shfl(cs, 31, 64);
    const float s2 = __shfl(cs, 47, 64), s3 = __shfl(cs, 63, 64);
    if (tid == 0) {
      const float sum = __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
      l.bc[0] = cr_divf(1.0f, cr_sqrtf(__fadd_rn(cr_divf(sum, (float)K), 1e-6f)));
    }
  }
  __syncthreads();
  return l.bc[0];
}

__device__ __forceinline__ float4 scale4(const float4& x, float rms, const float4& g) {
  return make_float4(__fmul_rn(__fmul_rn(x.x, rms), g.x), __fmul_rn(__fmul_rn(x.y, rms), g.y),
                     __fmul_rn(__fmul_rn(x.z, rms), g.z), __fmul_rn(__fmul_rn(x.w, rms), g.w));
}

// round half away from zero and clamp (src/kernel.c:115-125): t + 0.5 with
// t's sign (copysign gives -0.5 only for t < 0 or t = -0, where t >= 0 ?
// 0.5 : -0.5 would give +0.5 for -0; both then truncate to 0), one med3
__device__ __forceinline__ int q8i_of(float v, float scale_x) {
  const float t = __fmul_rn(v, scale_x);
  const int iv = (int)__fadd_rn(t, __builtin_copysignf(0.5f, t));
  return iv > 127 ? 127 : (iv < -128 ? -128 : iv);
}
__device__ __forceinline__ uint32_t q8_of(float v, float scale_x) {
  return (uint32_t)(q8i_of(v, scale_x) & 255);
}

// int8 quantization of (x*rms)*gamma (src/kernel.c:93-128, 358-386) into the
// split-nibble layout + slice sums; returns scale_x.
template <int C>
__device__ float pro_quant(const float4 (&xv)[C], const float4 (&gv)[C], float rms, int K,
                           const Lds& l, float* __restrict__ xn_out = nullptr,
                           int8_t* __restrict__ xq_out = nullptr) {
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6, n4 = K >> 2;
  float4 v[C];
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    v[i] = scale4(xv[i], rms, gv[i]);
    if (tid + i * nt < n4) {
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
      if (xn_out) ((float4*)xn_out)[tid + i * nt] = v[i];
    }
  }
  mx = wave_max_f32(mx);
  if (lane == 0) l.bc[8 + wave] = mx;
  __syncthreads();
  float max_abs = 0.0f;
  for (int w = 0; w < (nt >> 6); ++w) max_abs = fmaxf(max_abs, l.bc[8 + w]);
  const float scale_x = cr_divf(127.0f, __fadd_rn(max_abs, 1e-5f));
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = tid + i * nt;
    if (c < n4) {
      const uint32_t q4 = q8_of(v[i].x, scale_x) | (q8_of(v[i].y, scale_x) << 8) |
                          (q8_of(v[i].z, scale_x) << 16) | (q8_of(v[i].w, scale_x) << 24);
      ((uint32_t*)l.q8)[c] = q4;
      if (xq_out) ((uint32_t*)xq_out)[c] = q4;
    }
  }
  __syncthreads();
  // 16 columns per thread from one 16-byte LDS read -> split nibbles
  const int n_groups = K >> 4;
  for (int g0 = 0; g0 < n_groups; g0 += nt) {
    const int g = g0 + tid;
    int qsum = 0;
    if (g < n_groups) {
      const uint4 raw = *(const uint4*)(l.q8 + 16 * g);
      const uint32_t wds[4] = {raw.x, raw.y, raw.z, raw.w};
      int q[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        q[j] = (int)(int8_t)(wds[j >> 2] >> (8 * (j & 3)));
        qsum += q[j];
      }
      uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        le |= (uint32_t)(q[2 * n] & 15) << (4 * n);
        lo |= (uint32_t)(q[2 * n + 1] & 15) << (4 * n);
        he |= (uint32_t)((q[2 * n] >> 4) & 15) << (4 * n);
        ho |= (uint32_t)((q[2 * n + 1] >> 4) & 15) << (4 * n);
      }
      *(uint4*)(l.nib + 4 * g) = make_uint4(le, lo, he, ho);
    }
    const int s = wave_sum_i32(qsum);  // one wave = 64 groups = one slice
    const int slice = (g0 >> 6) + wave;
    if (lane == 0 && slice < slices_of(K)) l.slices[slice] = s;
  }
  __syncthreads();
  return scale_x;
}

// ---------------------------------------------------------------------------
// Prologue for K = 1024 * G (G in {1, 2, 4}): every thread of the block owns
// 4G consecutive columns (float4s G*t .. G*t+G-1) in registers for the whole
// prologue, so all four waves share the scaling and packing work whatever K
// is; the R = 4/G threads of a 16-column group sit in consecutive lanes.
// The squares go through LDS once to reach the chain layout, wave 0 runs the
// chains, and the int8 values are packed straight from registers.  Returns
// scale_x.
//   PRENORM: x first becomes (x * rms(x)) * g_pre (the final norm).
// ---------------------------------------------------------------------------
template <int G>
__device__ __forceinline__ void put_squares(const float4 (&v)[G], const Lds& l) {
  constexpr int E = 1024 * G / 64;
  // column 4e + j is element e of chain j (segments of E elements padded by
  // 4 floats); the thread's elements G*t .. G*t+G-1 lie in one segment
  const int e = G * (int)threadIdx.x;
  const int pe = e + 4 * (e / E);
#pragma unroll
  for (int k = 0; k < G; ++k) {
    l.sq[pe + k] = __fmul_rn(v[k].x, v[k].x);
    l.sq[l.stride + pe + k] = __fmul_rn(v[k].y, v[k].y);
    l.sq[2 * l.stride + pe + k] = __fmul_rn(v[k].z, v[k].z);
    l.sq[3 * l.stride + pe + k] = __fmul_rn(v[k].w, v[k].w);
  }
}

// rms = 1/sqrtf(sum/K + 1e-6f) from the squares in LDS; wave 0 runs the
// chains, the result is broadcast through LDS (src/kernel.c:77-91); the
// other waves run `idle` meanwhile
struct NoWork {
  __device__ void operator()() const {}
};

template <int G, typename F = NoWork>
__device__ __forceinline__ float chain_rms(const Lds& l, F&& idle = NoWork{}) {
  constexpr int K = 1024 * G, E = K / 64;
  __syncthreads();
  if (threadIdx.x >= 64) {
    idle();
  } else {
    const float cs = chain_regs<E>(l.sq, l.stride, threadIdx.x);
    const float s0 = lane_f32(cs, 15), s1 = lane_f32(cs, 31);
    const float s2 = lane_f32(cs, 47), s3 = lane_f32(cs, 63);
    if (threadIdx.x == 0) {
      const float sum = __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
      // sum / K with K a power of two: an exact scaling, rounded like the
      // division
      l.bc[0] = cr_divf(1.0f, cr_sqrtf(__fadd_rn(__fmul_rn(sum, 1.0f / K), 1e-6f)));
    }
  }
  __syncthreads();
  return l.bc[0];
}

// the thread's columns of the input and of the norm weights, loaded at
// kernel entry (before the weight rows, so that the prologue's first wait
// covers these loads only)
template <int G, bool PRENORM>
struct SplitIn {
  float4 xv[G], gv[G], gp[PRENORM ? G : 1];
};

template <int G, bool PRENORM>
__device__ __forceinline__ void split_load(SplitIn<G, PRENORM>& in, const float* __restrict__ x,
                                           const float* __restrict__ g_pre,
                                           const float* __restrict__ g) {
  const int c4 = G * (int)threadIdx.x;
#pragma unroll
  for (int k = 0; k < G; ++k) {
    in.xv[k] = ((const float4*)x)[c4 + k];
    in.gv[k] = ((const float4*)g)[c4 + k];
    if constexpr (PRENORM) in.gp[k] = ((const float4*)g_pre)[c4 + k];
  }
}

// fast mode: 1/rms from the pairwise tree (one block barrier).  A 16-column
// leaf is ((q0 + q1) + (q2 + q3)) over its four float4s; the thread holds G
// of them, and the first butterfly steps of the wave tree finish the leaf
// across its R = 4/G lanes, the rest pair the leaves in index order.
template <int G>
__device__ __forceinline__ float fast_rms(const float4 (&xv)[G], const Lds& l) {
  constexpr int K = 1024 * G;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float t[G];
#pragma unroll
  for (int k = 0; k < G; ++k)
    t[k] = __fadd_rn(__fadd_rn(__fmul_rn(xv[k].x, xv[k].x), __fmul_rn(xv[k].y, xv[k].y)),
                     __fadd_rn(__fmul_rn(xv[k].z, xv[k].z), __fmul_rn(xv[k].w, xv[k].w)));
  float part;
  if constexpr (G == 4)
    part = __fadd_rn(__fadd_rn(t[0], t[1]), __fadd_rn(t[2], t[3]));
  else if constexpr (G == 2)
    part = __fadd_rn(t[0], t[1]);
  else
    part = t[0];
  const float w = wave_tree_f32(part);
  if (lane == 0) l.bc[12 + wave] = w;
  __syncthreads();
  const float s = tree_top<4>(l.bc + 12);
  return cr_divf(1.0f, cr_sqrtf(__fadd_rn(__fmul_rn(s, 1.0f / K), 1e-6f)));
}

// idle: work for waves 1.. while wave 0 runs the first chain (the first
// fast-mode tree has no such window: they run it at once)
template <int G, bool PRENORM, typename F = NoWork>
__device__ float split_prologue(SplitIn<G, PRENORM>& in, const Lds& l, bool fast,
                                float* __restrict__ xn_out = nullptr,
                                int8_t* __restrict__ xq_out = nullptr, F&& idle = NoWork{}) {
  constexpr int R = 4 / G, CPT = 4 * G;  // threads per 16-column group, columns per thread
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c4 = G * tid;
  float4 (&xv)[G] = in.xv;
  const float4 (&gv)[G] = in.gv;
  const float4 (&gp)[PRENORM ? G : 1] = in.gp;
  float rms;
  if (fast) {
    if (threadIdx.x >= 64) idle();
    rms = fast_rms<G>(xv, l);
  } else {
    put_squares<G>(xv, l);
    if constexpr (!std::is_same<std::decay_t<F>, NoWork>::value) {
      // waves 1.. issue their rows during the chain: the other inputs are
      // passed through an empty asm first (which waits for them now), so
      // that their uses after the chain depend on this point and not on
      // loads that the compiler, not knowing how many rows were issued in
      // between, would otherwise wait for with all of the rows
#pragma unroll
      for (int k = 0; k < G; ++k) {
        asm volatile("" : "+v"(xv[k].x), "+v"(xv[k].y), "+v"(xv[k].z), "+v"(xv[k].w));
        asm volatile("" : "+v"(in.gv[k].x), "+v"(in.gv[k].y), "+v"(in.gv[k].z), "+v"(in.gv[k].w));
        if constexpr (PRENORM)
          asm volatile("" : "+v"(in.gp[k].x), "+v"(in.gp[k].y), "+v"(in.gp[k].z), "+v"(in.gp[k].w));
      }
    }
    rms = chain_rms<G>(l, idle);
  }
  if constexpr (PRENORM) {
    // final_feat = (x * rms) * norm_f (src/model.c:1225, src/kernel.c:93-103)
#pragma unroll
    for (int k = 0; k < G; ++k) xv[k] = scale4(xv[k], rms, gp[k]);
    if (fast) {
      __syncthreads();  // the first tree's sums are read before they are replaced
      rms = fast_rms<G>(xv, l);
    } else {
      put_squares<G>(xv, l);
      rms = chain_rms<G>(l);
    }
  }
  // int8 quantization (src/kernel.c:93-128, 358-386)
  float mx = 0.0f;
#pragma unroll
  for (int k = 0; k < G; ++k) {
    xv[k] = scale4(xv[k], rms, gv[k]);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xv[k].x), fabsf(xv[k].y)),
                         fmaxf(fabsf(xv[k].z), fabsf(xv[k].w))));
    if (xn_out) ((float4*)xn_out)[c4 + k] = xv[k];
  }
  mx = wave_max_f32(mx);
  if (lane == 0) l.bc[8 + wave] = mx;
  __syncthreads();
  const float max_abs = fmaxf(fmaxf(l.bc[8], l.bc[9]), fmaxf(l.bc[10], l.bc[11]));
  const float scale_x = cr_divf(127.0f, __fadd_rn(max_abs, 1e-5f));
  int q[CPT];
#pragma unroll
  for (int k = 0; k < G; ++k) {
    const float vv[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) q[4 * k + j] = q8i_of(vv[j], scale_x);
  }
  // this thread's nibbles of its group's four split-nibble words: columns
  // 2n (even) and 2n+1 (odd) of the group are nibble n; the thread's
  // columns start at 16-column offset CPT * (tid % R)
  const int n0 = (CPT / 2) * (tid % R);
  uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
  for (int n = 0; n < CPT / 2; ++n) {
    const int sh = 4 * (n0 + n);
    le |= (uint32_t)(q[2 * n] & 15) << sh;
    lo |= (uint32_t)(q[2 * n + 1] & 15) << sh;
    he |= (uint32_t)((q[2 * n] >> 4) & 15) << sh;
    ho |= (uint32_t)((q[2 * n + 1] >> 4) & 15) << sh;
  }
  if constexpr (R >= 2) {  // the group's R lanes are adjacent: OR their parts
    le |= (uint32_t)dpp_mov<0xB1>((int)le);
    lo |= (uint32_t)dpp_mov<0xB1>((int)lo);
    he |= (uint32_t)dpp_mov<0xB1>((int)he);
    ho |= (uint32_t)dpp_mov<0xB1>((int)ho);
  }
  if constexpr (R == 4) {
    le |= (uint32_t)dpp_mov<0x4E>((int)le);
    lo |= (uint32_t)dpp_mov<0x4E>((int)lo);
    he |= (uint32_t)dpp_mov<0x4E>((int)he);
    ho |= (uint32_t)dpp_mov<0x4E>((int)ho);
  }
  if (tid % R == 0) *(uint4*)(l.nib + 4 * (tid / R)) = make_uint4(le, lo, he, ho);
  if (xq_out) {
    uint32_t b[G];
#pragma unroll
    for (int k = 0; k < G; ++k)
      b[k] = (uint32_t)(q[4 * k] & 255) | (uint32_t)(q[4 * k + 1] & 255) << 8 |
             (uint32_t)(q[4 * k + 2] & 255) << 16 | (uint32_t)(q[4 * k + 3] & 255) << 24;
    if constexpr (G == 4)
      *(uint4*)(xq_out + CPT * tid) = make_uint4(b[0], b[1], b[2], b[3]);
    else if constexpr (G == 2)
      *(uint2*)(xq_out + CPT * tid) = make_uint2(b[0], b[1]);
    else
      *(uint32_t*)(xq_out + CPT * tid) = b[0];
  }
  // no slice sums here: the GEMV lanes take their share of each slice's sum
  // of x from the nibbles they read (lane_sums)
  __syncthreads();
  return scale_x;
}

// ---------------------------------------------------------------------------
// GEMV pieces
// ---------------------------------------------------------------------------

// x.code over one lane's 64 columns (16 packed bytes, split-nibble act)
__device__ __forceinline__ int dot64(uint4 w, const uint32_t (&xa)[16]) {
  const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
  uint32_t al = 0;
  int ah = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t lo = w4[d] & 0x33333333u;
    const uint32_t hi = (w4[d] >> 2) & 0x33333333u;
    al = __builtin_amdgcn_udot8(lo, xa[4 * d + 0], al, false);
    al = __builtin_amdgcn_udot8(hi, xa[4 * d + 1], al, false);
    ah = __builtin_amdgcn_sdot8((int)lo, (int)xa[4 * d + 2], ah, false);
    ah = __builtin_amdgcn_sdot8((int)hi, (int)xa[4 * d + 3], ah, false);
  }
  return ah * 16 + (int)al;
}

// reduce a lane partial over its 16-lane slice group, subtract the slice's
// sum of x, fold the slices of the T-lane row team in order into fp32
// (src/kernel.c:255-256, 407-425)
template <int P, int T, bool READ_SL = true>
__device__ __forceinline__ void load_lane_act(const Lds& l, int K, int u, uint32_t (&xa)[P][16],
                                              int (&xsl)[P]) {
  const int chunks = K >> 6;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * T + u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 v = j < chunks ? *(const uint4*)(l.nib + 16 * j + 4 * g) : make_uint4(0, 0, 0, 0);
      xa[p][4 * g + 0] = v.x;
      xa[p][4 * g + 1] = v.y;
      xa[p][4 * g + 2] = v.z;
      xa[p][4 * g + 3] = v.w;
    }
    const int sl = (p * T + u) >> 4;
    xsl[p] = READ_SL && sl < slices_of(K) ? l.slices[sl] : 0;
  }
}

// The lane's share of its slice's sum of x: its 64 columns from the split
// nibbles it holds (x = lo + 16 hi, lo unsigned, hi signed).  Subtracted
// from the lane's partial x.code before the 16-lane reduction, it makes the
// slice total x.code - sum(x) (w = code - 1) without a reduction of x in
// the prologue; exact in int32 either way.
template <int P>
__device__ __forceinline__ void lane_sums(const uint32_t (&xa)[P][16], int (&xs)[P]) {
  constexpr uint32_t ones = 0x11111111u;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint32_t al = 0;
    int ah = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      al = __builtin_amdgcn_udot8(xa[p][4 * g + 0], ones, al, false);
      al = __builtin_amdgcn_udot8(xa[p][4 * g + 1], ones, al, false);
      ah = __builtin_amdgcn_sdot8((int)xa[p][4 * g + 2], (int)ones, ah, false);
      ah = __builtin_amdgcn_sdot8((int)xa[p][4 * g + 3], (int)ones, ah, false);
    }
    xs[p] = ah * 16 + (int)al;
  }
}

// ---------------------------------------------------------------------------
// Quantize + GEMV over a slice of rows, 256 threads per block.
//   PRENORM: the input first goes through RMSNorm(gamma_pre) -- the
//            reference's final norm -- then the BitLinear's own norm
//   MODE:    0 store, 1 accumulate (residual)
//   PICK:    1: each block also writes its first-max row (value, index);
//            2: the rows are stored multiplied by 1/temp (the sampler's
//               temperature, src/model.c:160-166) and each block writes the
//               max of what it stored under `x > m` from -1e30f
//   DROP:    a single call on mapped host memory (x in, out, and block 0's
//            copies of the normalized and int8 input out): each block
//            stages its rows in LDS, writes them as one contiguous run of
//            write-through stores and then writes dr.seq to its own
//            host-mapped word dr.flags[block], which the caller polls
//            instead of synchronizing the stream (no device-wide counter:
//            atomics on one word serialize across the XCDs, ~70 ns per
//            block; system-scope atomics on a host word, ~1 us each)
// ---------------------------------------------------------------------------
struct DropOut {
  float* xn;        // normalized input, written by block 0 (or null)
  int8_t* xq;       // int8 input, written by block 0 (or null)
  unsigned* flags;  // DROP: host-mapped completion words, one per block;
                    // LM head: the step's CTL_DONE word (or null)
  unsigned seq;
  float* scale;     // scale_x, written by block 0 (or null)
};

// FASTC: 0 = the fast argument decides at run time; 1 / 2 = parity / fast
// mode fixed at compile time (the LM head: with both prologues in one kernel
// the compiler's merge of the two paths made waves 1.. wait for all the rows
// they issue during the first chain before the second norm could start)
template <int T, int P, int NPF, int C, bool PRENORM, int MODE, int PICK, bool WP,
          bool DROP = false, int FASTC = 0>
__global__ __launch_bounds__(256) void k_rows_fused(const float* __restrict__ x, int K,
                                                    const float* __restrict__ gamma_pre,
                                                    const float* __restrict__ gamma,
                                                    const uint8_t* __restrict__ W, int N,
                                                    float w_scale, float* __restrict__ out,
                                                    float* __restrict__ part_v,
                                                    int* __restrict__ part_i, float temp,
                                                    int fast, DropOut dr) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int RPW = 64 / T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int G = (N + RPW - 1) / RPW;
  const int per = G / (int)gridDim.x, extra = G % (int)gridDim.x, b = blockIdx.x;
  const int g0 = b * per + min(b, extra);
  const int g1 = g0 + per + (b < extra ? 1 : 0);
  const size_t wstride = (size_t)(K >> 2);
  const int chunks = K >> 6;

  // the input vectors first (the prologue waits for them), then the weights
  float4 sx[WP ? 1 : C], sg[WP ? 1 : C], sg2[PRENORM && !WP ? C : 1];
  SplitIn<C, PRENORM> sin;
  if constexpr (WP) {
    split_load<C, PRENORM>(sin, x, gamma_pre, gamma);
  } else {
    stage_load<C>(sx, x, K);
    stage_load<C>(sg, PRENORM ? gamma_pre : gamma, K);
    if constexpr (PRENORM) stage_load<C>(sg2, gamma, K);
  }
  // the LM head of a stopped decode (CTL_DONE, passed in dr.flags, which
  // only the DROP form uses otherwise) stores nothing (the word is a scalar
  // load the wave waits for: ~0.1 us, once per token); the out_proj of such
  // a step needs no test, its input y is zero (k_inproj_ssm).  DropOut keeps
  // its size: one more pointer in it (376 -> 384 bytes of kernel arguments)
  // made every out_proj launch 0.19 us slower
  bool stopped = false;
  if constexpr (PRENORM) stopped = dr.flags && *(const int*)dr.flags == kDoneStopped;

  // The row loads are unconditional, with indices clamped into the tensor:
  // a load inside a branch makes the compiler wait for all outstanding
  // loads where the prologue first reads x, so the chains would start only
  // once most of the rows had arrived.  What a lane loads past its row
  // (j >= chunks) meets zero activations, and groups past the block's are
  // skipped, so nothing else needs masking.  Streaming loads: with the
  // out_proj and LM head rows read this way (the in_proj rows already
  // were) the 1B decode step measured 0.2937-0.2944 ms against 0.3000-
  // 0.3009 ms; with plain loads 0.308, and with only one of the two kinds
  // streaming 0.300 (LM head) or 0.305 (out_proj).
  uint4 wv[NPF][P];
  auto load_rows = [&]() {
#pragma unroll
    for (int it = 0; it < NPF; ++it) {
      const int r = min((g0 + wave + 4 * it) * RPW + sub, N - 1);
#pragma unroll
      for (int p = 0; p < P; ++p)
        wv[it][p] = load_stream16(W + (size_t)r * wstride + 16 * min(p * T + u, chunks - 1));
    }
  };
  // The LM head streams more weight bytes than the memory pipeline takes
  // at once, so issuing a wave's loads stalls that wave until most of them
  // have arrived: there the waves issue their rows once the input's squares
  // are in LDS (waves 1.. while wave 0 runs the first chain, wave 0 after
  // the prologue), so the chains start at once.
  constexpr bool defer_rows = PRENORM && WP;
  if (!defer_rows) load_rows();

  // MODE 1: the residual values of the prefetched rows, read now so that
  // the final x += o does not wait for them
  float resid[NPF];
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int r = (g0 + wave + 4 * it) * RPW + sub;
    resid[it] = (MODE == 1 && u == 0 && g0 + wave + 4 * it < g1 && r < N) ? out[r] : 0.0f;
  }

  const Lds l = lds_carve(lds, K);
  float* const xn_out = b == 0 ? dr.xn : nullptr;
  int8_t* const xq_out = b == 0 ? dr.xq : nullptr;
  float scale_x;
  if constexpr (WP) {
    if constexpr (defer_rows)
      scale_x = split_prologue<C, PRENORM>(sin, l, FASTC == 0 ? fast != 0 : FASTC == 2, xn_out,
                                           xq_out, load_rows);
    else
      scale_x = split_prologue<C, PRENORM>(sin, l, FASTC == 0 ? fast != 0 : FASTC == 2, xn_out,
                                           xq_out);
  } else {
    float rms = pro_rms<C>(sx, K, l);
    if constexpr (PRENORM) {
      // final_feat = (x * rms) * norm_f (src/model.c:1225, src/kernel.c:93-103)
#pragma unroll
      for (int i = 0; i < C; ++i) sx[i] = scale4(sx[i], rms, sg[i]);
      rms = pro_rms<C>(sx, K, l);
      scale_x = pro_quant<C>(sx, sg2, rms, K, l, xn_out, xq_out);
    } else {
      scale_x = pro_quant<C>(sx, sg, rms, K, l, xn_out, xq_out);
    }
  }
  if (defer_rows && wave == 0) load_rows();
  if (b == 0 && tid == 0 && dr.scale) *dr.scale = scale_x;
  const float inv = inv_scale_of(scale_x, w_scale);
  uint32_t xa[P][16];
  int xsl[P], xsd[P];  // slice sums (after the reduction) or lane shares (before it)
  load_lane_act<P, T, !WP>(l, K, u, xa, xsl);
  if constexpr (WP) {
    lane_sums<P>(xa, xsd);
  } else {
#pragma unroll
    for (int p = 0; p < P; ++p) xsd[p] = 0;
  }

  float best_v = PICK == 2 ? -1e30f : -1e9f;
  int best_i = 0x7fffffff;
  const float inv_temp = PICK == 2 ? cr_divf(1.0f, temp) : 1.0f;
  // DROP: the block's rows [r0, r0 + rows) go to LDS first (the squares'
  // area, free after the prologue; a block owns at most 4 * NPF * RPW rows)
  const int r0 = g0 * RPW;
  auto emit = [&](int r, float o, float res) {
    if (u == 0 && r < N && !stopped) {
      if (PICK == 2) o = __fmul_rn(o, inv_temp);
      if (DROP)
        l.sq[r - r0] = o;
      else if (MODE == 1)
        out[r] = __fadd_rn(res, o);
      else
        out[r] = o;
      if (PICK && o > best_v) {  // rows ascend per lane: first max kept
        best_v = o;
        best_i = r;
      }
    }
  };
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = g0 + wave + 4 * it;
    if (grp < g1) {  // uniform per wave
      float o = 0.0f;
#pragma unroll
      for (int p = 0; p < P; ++p)
        o = row_finish<T>(dot64(wv[it][p], xa[p]) - xsd[p], xsl[p], p, slices_of(K), inv, o,
                           unit_base);
      emit(grp * RPW + sub, o, resid[it]);
    }
  }
  for (int grp = g0 + wave + 4 * NPF; grp < g1; grp += 4) {  // beyond the prefetch
    const int r = grp * RPW + sub;
    float o = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      const uint4 w = (r < N && j < chunks) ? *(const uint4*)(W + (size_t)r * wstride + 16 * j)
                                            : make_uint4(0, 0, 0, 0);
      o = row_finish<T>(dot64(w, xa[p]) - xsd[p], xsl[p], p, slices_of(K), inv, o, unit_base);
    }
    emit(r, o, MODE == 1 && u == 0 && r < N ? out[r] : 0.0f);
  }

  if constexpr (DROP) {
    __syncthreads();
    const int r_end = min(g1 * RPW, N);
    // system-scope stores go through to host memory (nothing of them stays
    // in L2), so each thread only waits for its own stores to complete
    // before the barrier; an L2 write-back per wave (a system release
    // fence) costs ~35 ns per block at 786 blocks.  A barrier alone does
    // not wait for the other waves' stores.  Block 0 also wrote the copies
    // of the input with plain stores in the prologue: its threads take the
    // full release fence.
    for (int r = r0 + tid; r < r_end; r += blockDim.x)
      __hip_atomic_store(out + r, l.sq[r - r0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (b == 0)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
    else
      __asm__ __volatile__("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
      __hip_atomic_store(dr.flags + b, dr.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }

  if constexpr (PICK == 2) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(best_v, o, 64);
      if (ov > best_v) best_v = ov;
    }
    if (lane == 0) l.bc[16 + wave] = best_v;
    __syncthreads();
    if (tid == 0 && !stopped) {
      for (int k = 1; k < 4; ++k)
        if (l.bc[16 + k] > best_v) best_v = l.bc[16 + k];
      part_v[blockIdx.x] = best_v;
    }
  } else if constexpr (PICK == 1) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(best_v, o, 64);
      const int oi = __shfl_xor(best_i, o, 64);
      if (ov > best_v || (ov == best_v && oi < best_i)) {
        best_v = ov;
        best_i = oi;
      }
    }
    if (lane == 0) {
      l.bc[16 + wave] = best_v;
      ((int*)l.bc)[20 + wave] = best_i;
    }
    __syncthreads();
    if (tid == 0 && !stopped) {
      for (int k = 1; k < 4; ++k) {
        const float v = l.bc[16 + k];
        const int i = ((int*)l.bc)[20 + k];
        if (v > best_v || (v == best_v && i < best_i)) {
          best_v = v;
          best_i = i;
        }
      }
      part_v[blockIdx.x] = best_v;
      part_i[blockIdx.x] = best_i;
    }
  }
}

// ---------------------------------------------------------------------------
// int8-input product of one token per block row (blockIdx.y = token), exact
// int32 totals x.w (src/kernel.c:159-316 on given int8 activations): the
// row layout of k_rows_fused, with the token's int8 values turned into
// split nibbles in LDS by the block itself, so there is no preparation
// launch and no workspace; each GEMV lane subtracts its own columns' sum of
// x (lane_sums) before the row reduction.  The token's values are loaded
// before the weight rows (vector-memory waits complete in issue order, so
// the conversion would otherwise wait for every weight byte).  K % 64 == 0,
// K <= 64 T P <= 8192.
// ---------------------------------------------------------------------------
// 16 int8 values (bytes of d, column c = byte c) -> the split-nibble group
// {lo4 of the even columns, lo4 of the odd, hi4 of the even, hi4 of the
// odd}, nibble n of "even" = column 2n: byte gathers instead of per-nibble
// shifts
__device__ __forceinline__ uint4 split_nibbles16(uint4 d) {
  const uint32_t L[4] = {d.x & 0x0F0F0F0Fu, d.y & 0x0F0F0F0Fu, d.z & 0x0F0F0F0Fu,
                         d.w & 0x0F0F0F0Fu};
  const uint32_t H[4] = {(d.x >> 4) & 0x0F0F0F0Fu, (d.y >> 4) & 0x0F0F0F0Fu,
                         (d.z >> 4) & 0x0F0F0F0Fu, (d.w >> 4) & 0x0F0F0F0Fu};
  // bytes {a.b0, a.b2, b.b0, b.b2} (even) or {a.b1, a.b3, b.b1, b.b3} (odd),
  // then byte pairs merged into nibble pairs and the merged bytes gathered
  auto pack = [](const uint32_t (&v)[4], uint32_t sel) __attribute__((always_inline)) {
    const uint32_t e01 = __builtin_amdgcn_perm(v[1], v[0], sel);
    const uint32_t e23 = __builtin_amdgcn_perm(v[3], v[2], sel);
    const uint32_t t01 = e01 | (e01 >> 4), t23 = e23 | (e23 >> 4);
    return __builtin_amdgcn_perm(t23, t01, 0x06040200u);
  };
  // v_perm_b32 selector bytes: 0..3 = bytes of the second operand, 4..7 of
  // the first
  return make_uint4(pack(L, 0x06040200u), pack(L, 0x07050301u), pack(H, 0x06040200u),
                    pack(H, 0x07050301u));
}

__device__ __forceinline__ int dot64c(uint4 w, const uint32_t (&xa)[16]) {
  return dot64(make_uint4(canon_codes(w.x), canon_codes(w.y), canon_codes(w.z), canon_codes(w.w)),
               xa);
}

template <int T, int P, int NPF, bool CANON, bool XVEC, int NW>
__global__ __launch_bounds__(64 * NW) void k_rows_i8(const int8_t* __restrict__ xq, int ldx, int K,
                                                 const uint8_t* __restrict__ W, int N,
                                                 int32_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint32_t nib[];  // [K / 4 + 4]
  constexpr int RPW = 64 / T;
  constexpr int XG = (512 + 64 * NW - 1) / (64 * NW);  // 16-column groups per thread: K / 16 <= 512
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int G = (N + RPW - 1) / RPW;
  const int per = G / (int)gridDim.x, extra = G % (int)gridDim.x, b = blockIdx.x;
  const int g0 = b * per + min(b, extra);
  const int g1 = g0 + per + (b < extra ? 1 : 0);
  const int m = blockIdx.y;
  const size_t wstride = (size_t)(K >> 2);
  const int chunks = K >> 6, n_groups = K >> 4;

  // The token's int8 values first (16 columns per group), then the weight
  // rows.  Every load is issued unconditionally (indices clamped into the
  // buffers, unused values replaced by zeros afterwards): a load inside a
  // branch makes the compiler wait for all outstanding loads at the branch's
  // end, so the conversion of x would wait for every weight byte instead of
  // running while the rows are in flight.
  const int8_t* __restrict__ xr = xq + (size_t)m * ldx;
  uint4 xv[XG];
#pragma unroll
  for (int i = 0; i < XG; ++i) {
    const int g = min(tid + i * (int)blockDim.x, n_groups - 1);
    if constexpr (XVEC) {
      xv[i] = *(const uint4*)(xr + 16 * g);
    } else {
      uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 16; ++j) wd[j >> 2] |= (uint32_t)(uint8_t)xr[16 * g + j] << (8 * (j & 3));
      xv[i] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
  }

  uint4 wv[NPF][P];
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = g0 + wave + NW * it;
    const int r = grp * RPW + sub;
    const int rc = min(r, N - 1);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      const uint4 w = load_stream16(W + (size_t)rc * wstride + 16 * min(j, chunks - 1));
      wv[it][p] = (grp < g1 && r < N && j < chunks) ? w : make_uint4(0, 0, 0, 0);
    }
  }

  // split nibbles of the token's values into LDS (groups past K go to a
  // spare slot, so that the stores, and with them the loads, stay
  // unconditional)
#pragma unroll
  for (int i = 0; i < XG; ++i) {
    const int g = min(tid + i * (int)blockDim.x, n_groups);
    *(uint4*)(nib + 4 * g) = split_nibbles16(xv[i]);
  }
  __syncthreads();

  uint32_t xa[P][16];
  int xsd[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * T + u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 v = j < chunks ? *(const uint4*)(nib + 16 * j + 4 * g) : make_uint4(0, 0, 0, 0);
      xa[p][4 * g + 0] = v.x;
      xa[p][4 * g + 1] = v.y;
      xa[p][4 * g + 2] = v.z;
      xa[p][4 * g + 3] = v.w;
    }
  }
  lane_sums<P>(xa, xsd);

  // int32 totals: the lane's passes first, then one row reduction
  auto total = [&](const uint4 (&w)[P]) __attribute__((always_inline)) {
    int part = 0;
#pragma unroll
    for (int p = 0; p < P; ++p)
      part += (CANON ? dot64(w[p], xa[p]) : dot64c(w[p], xa[p])) - xsd[p];
    return row_total_i32<T>(part, 0, unit_base);
  };
  int32_t* __restrict__ orow = out + (size_t)m * N;
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = g0 + wave + NW * it;
    if (grp < g1) {  // uniform per wave
      const int t = total(wv[it]);
      const int r = grp * RPW + sub;
      if (u == 0 && r < N) orow[r] = t;
    }
  }
  for (int grp = g0 + wave + NW * NPF; grp < g1; grp += NW) {  // beyond the prefetch
    const int r = grp * RPW + sub;
    uint4 w[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      w[p] = (r < N && j < chunks) ? load_stream16(W + (size_t)r * wstride + 16 * j)
                                   : make_uint4(0, 0, 0, 0);
    }
    const int t = total(w);
    if (u == 0 && r < N) orow[r] = t;
  }
}

// ---------------------------------------------------------------------------
// in_proj + SSM step in one kernel.  Block (head h, channel group q) owns
// kCB channels of the head: it computes their z and x rows and the head's
// B, C, dt rows (each block of a head recomputes these three), then runs the
// SSM step of its channels (src/kernel.c:34-70) from the values in LDS.
// The per-head row layout of the weights is [z (hd) | x (hd) | B | C | dt].
// ---------------------------------------------------------------------------
constexpr int kCB = 16;              // channels per block
constexpr int kRowsCB = 2 * kCB + 3;  // weight rows per block

struct SsmArgs {
  const float* dt_bias;
  const float* A;
  const float* cw;  // [4][di]
  const float* cb;
  float* cs;        // [3][di] ring
  float* ssm;
  const float* D;
  float* y;
  const int* ctl;
  int hd, di;
};

template <int T, int P, int NPF, int C, bool WP, bool GATED>
__global__ __launch_bounds__(256) void k_inproj_ssm(const float* __restrict__ x, int K,
                                                    const float* __restrict__ gamma,
                                                    const uint8_t* __restrict__ W, float w_scale,
                                                    SsmArgs a, int fast) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float s_proj[kRowsCB];
  constexpr int RPW = 64 / T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int hd = a.hd, groups_per_head = hd / kCB;
  const int h = blockIdx.x / groups_per_head, q = blockIdx.x % groups_per_head;
  const size_t wstride = (size_t)(K >> 2);
  const int chunks = K >> 6;
  const int n_groups = (kRowsCB + RPW - 1) / RPW;
  // weight row of local row r
  auto wrow = [&](int r) {
    const int base = h * (2 * hd + 3);
    if (r < kCB) return base + q * kCB + r;
    if (r < 2 * kCB) return base + hd + q * kCB + (r - kCB);
    return base + 2 * hd + (r - 2 * kCB);
  };

  // the ring position first (nothing waits for it until the SSM step), the
  // input vector next (the prologue waits for it), then the weights
  int pos;
  bool stopped = false;  // GATED: a stopped decode leaves the state as it is
  if constexpr (GATED) {
    const int2 pos_done = *(const int2*)a.ctl;  // CTL_POS, CTL_DONE
    pos = pos_done.x;
    stopped = pos_done.y == kDoneStopped;
  } else {
    pos = a.ctl[CTL_POS];
  }
  float4 sx[WP ? 1 : C], sg[WP ? 1 : C];
  SplitIn<C, false> sin;
  if constexpr (WP) {
    split_load<C, false>(sin, x, nullptr, gamma);
  } else {
    stage_load<C>(sx, x, K);
    stage_load<C>(sg, gamma, K);
  }

  uint4 wv[NPF][P];
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = wave + 4 * it;
    const int r = min(grp * RPW + sub, kRowsCB - 1);
    const size_t roff = (size_t)wrow(r) * wstride;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = min(p * T + u, chunks - 1);
      wv[it][p] = load_stream16(W + roff + 16 * j);
    }
  }

  // SSM inputs of this thread's channel (threads 0..kCB-1), fetched while the
  // prologue runs: all three ring slots, so that no address waits for pos
  const int c = tid < kCB ? tid : 0;
  const int idx = h * hd + q * kCB + c;
  const float ring0 = a.cs[idx], ring1 = a.cs[(size_t)a.di + idx];
  const float ring2 = a.cs[2 * (size_t)a.di + idx];
  const float cw0 = a.cw[idx], cw1 = a.cw[a.di + idx], cw2 = a.cw[2 * a.di + idx];
  const float cw3 = a.cw[3 * a.di + idx], cbias = a.cb[idx], st0 = a.ssm[idx], Dc = a.D[idx];
  const float dtb = a.dt_bias[h], Ah = a.A[h];

  const Lds l = lds_carve(lds, K);
  float scale_x;
  if constexpr (WP) {
    scale_x = split_prologue<C, false>(sin, l, fast != 0);
  } else {
    const float rms = pro_rms<C>(sx, K, l);
    scale_x = pro_quant<C>(sx, sg, rms, K, l);
  }
  const float inv = inv_scale_of(scale_x, w_scale);
  uint32_t xa[P][16];
  int xsl[P], xsd[P];  // slice sums (after the reduction) or lane shares (before it)
  load_lane_act<P, T, !WP>(l, K, u, xa, xsl);
  if constexpr (WP) {
    lane_sums<P>(xa, xsd);
  } else {
#pragma unroll
    for (int p = 0; p < P; ++p) xsd[p] = 0;
  }

#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = wave + 4 * it;
    if (grp < n_groups) {  // uniform per wave
      float o = 0.0f;
#pragma unroll
      for (int p = 0; p < P; ++p)
        o = row_finish<T>(dot64(wv[it][p], xa[p]) - xsd[p], xsl[p], p, slices_of(K), inv, o,
                           unit_base);
      const int r = grp * RPW + sub;
      if (u == 0 && r < kRowsCB) s_proj[r] = o;
    }
  }
  __syncthreads();

  // scalar_ssm_inner for the block's channels (src/kernel.c:34-70), its
  // three independent transcendental parts on three waves at once: wave 0
  // the conv and silu(conv) of each channel, wave 1 silu(z), wave 2 the
  // head's softplus and decay; then wave 0 forms the state and y
  __shared__ float s_tail[2 * kCB + 2];
  if (wave == 0 && lane < kCB) {
    // taps in age order from the ring position (src/block.c:107)
    const float tap0 = pos == 0 ? ring0 : (pos == 1 ? ring1 : ring2);
    const float tap1 = pos == 0 ? ring1 : (pos == 1 ? ring2 : ring0);
    const float tap2 = pos == 0 ? ring2 : (pos == 1 ? ring0 : ring1);
    const float xin = s_proj[kCB + c];
    float conv = __fadd_rn(cbias, __fmul_rn(tap0, cw0));
    conv = __fadd_rn(conv, __fmul_rn(tap1, cw1));
    conv = __fadd_rn(conv, __fmul_rn(tap2, cw2));
    conv = __fadd_rn(conv, __fmul_rn(xin, cw3));
    if (!stopped) a.cs[(size_t)pos * a.di + idx] = xin;  // the oldest tap is overwritten
    s_tail[c] = silu_r(conv);
  } else if (wave == 1 && lane < kCB) {
    s_tail[kCB + lane] = silu_r(s_proj[lane]);
  } else if (wave == 2 && lane == 0) {
    const float dt_val = softplus_r(__fadd_rn(s_proj[2 * kCB + 2], dtb));
    s_tail[2 * kCB] = dt_val;
    s_tail[2 * kCB + 1] = libm::expf_glibc(__fmul_rn(Ah, dt_val));
  }
  __syncthreads();
  if (tid < kCB && stopped) {
    // a stopped step: the state stays, and y = 0 makes the out_proj that
    // follows add exactly +0 to x (RMSNorm of zeros, int8 zeros, zero totals)
    a.y[idx] = 0.0f;
  } else if (tid < kCB) {
    const float dt_val = s_tail[2 * kCB], decay = s_tail[2 * kCB + 1];
    const float Bdt = __fmul_rn(s_proj[2 * kCB], dt_val);
    const float C_val = s_proj[2 * kCB + 1];
    const float xact = s_tail[c];
    const float st = __fadd_rn(__fmul_rn(st0, decay), __fmul_rn(xact, Bdt));
    a.ssm[idx] = st;
    a.y[idx] = __fmul_rn(__fadd_rn(__fmul_rn(st, C_val), __fmul_rn(xact, Dc)), s_tail[kCB + c]);
  }
}

// ---------------------------------------------------------------------------
// SSM step, one block per head, one thread per channel.  proj holds the
// in_proj outputs per head as [z (hd) | x (hd) | B | C | dt].
// ---------------------------------------------------------------------------
__global__ void k_ssm_heads(const float* __restrict__ proj, int hd, int di,
                            const float* __restrict__ dt_bias, const float* __restrict__ A,
                            const float* __restrict__ cw, const float* __restrict__ cb,
                            float* __restrict__ cs, float* __restrict__ ssm,
                            const float* __restrict__ D, float* __restrict__ y,
                            const int* __restrict__ ctl) {
  const int h = blockIdx.x, c = blockIdx.y * blockDim.x + threadIdx.x;
  if (c >= hd) return;
  const float* __restrict__ ph = proj + (size_t)h * (2 * hd + 3);
  const int idx = h * hd + c;
  if (ctl[CTL_DONE] == kDoneStopped) {  // a stopped decode keeps its state; y = 0 (see
    y[idx] = 0.0f;                       // k_inproj_ssm)
    return;
  }
  const int pos = ctl[CTL_POS];
  const int t1 = pos + 1 < 3 ? pos + 1 : pos - 2;
  const int t2 = pos + 2 < 3 ? pos + 2 : pos - 1;
  const float dt_val = softplus_r(__fadd_rn(ph[2 * hd + 2], dt_bias[h]));
  const float decay = libm::expf_glibc(__fmul_rn(A[h], dt_val));
  const float Bdt = __fmul_rn(ph[2 * hd], dt_val);
  const float C_val = ph[2 * hd + 1];
  const float xin = ph[hd + c];
  float* c0 = cs + (size_t)pos * di;
  float conv = __fadd_rn(cb[idx], __fmul_rn(c0[idx], cw[idx]));
  conv = __fadd_rn(conv, __fmul_rn(cs[(size_t)t1 * di + idx], cw[di + idx]));
  conv = __fadd_rn(conv, __fmul_rn(cs[(size_t)t2 * di + idx], cw[2 * di + idx]));
  conv = __fadd_rn(conv, __fmul_rn(xin, cw[3 * di + idx]));
  c0[idx] = xin;  // the oldest tap is overwritten (cs_write == cs0)
  const float xa = silu_r(conv);
  const float st = __fadd_rn(__fmul_rn(ssm[idx], decay), __fmul_rn(xa, Bdt));
  ssm[idx] = st;
  y[idx] = __fmul_rn(__fadd_rn(__fmul_rn(st, C_val), __fmul_rn(xa, D[idx])), silu_r(ph[c]));
}

// ---------------------------------------------------------------------------
// Greedy pick over the LM-head blocks' candidates (block order = row order,
// so "greater, or equal with a lower index" keeps the first maximum), then
// the step bookkeeping and x = embed[token] (src/model.c:1195-1202).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pick(const float* __restrict__ part_v,
                                              const int* __restrict__ part_i, int n_parts,
                                              int* __restrict__ ctl, int* __restrict__ hist,
                                              int* __restrict__ out_tokens,
                                              const float* __restrict__ embed, int dm,
                                              float* __restrict__ x) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ int s_tok;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the step counters, read while the candidates load (nothing else in the
  // step writes them)
  const int step = tid == 0 ? ctl[CTL_STEP] : 0;
  const int hcount = tid == 0 ? ctl[CTL_HCOUNT] : 0;
  const int pos = tid == 0 ? ctl[CTL_POS] : 0;
  const int done = tid == 0 ? ctl[CTL_DONE] : 0;
  float bv = -1e9f;
  int bi = 0x7fffffff;
  // the first 4 * 256 candidates in one round of loads (indices clamped,
  // unconditional: a load in a branch would make the first comparison wait
  // for the loads of every turn), the rest in turns
  constexpr int PU = 4;
  float pv[PU];
  int pi[PU];
#pragma unroll
  for (int u = 0; u < PU; ++u) {
    const int b = min(tid + 256 * u, n_parts - 1);
    pv[u] = part_v[b];
    pi[u] = part_i[b];
  }
#pragma unroll
  for (int u = 0; u < PU; ++u)
    if (tid + 256 * u < n_parts && (pv[u] > bv || (pv[u] == bv && pi[u] < bi))) {
      bv = pv[u];
      bi = pi[u];
    }
  for (int b = tid + 256 * PU; b < n_parts; b += blockDim.x) {
    const float v = part_v[b];
    const int i = part_i[b];
    if (v > bv || (v == bv && i < bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < 4; ++k)
      if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) {
        bv = sv[k];
        bi = si[k];
      }
    const int best = bi == 0x7fffffff ? 0 : bi;
    if (done != kDoneStopped) {  // a stopped decode changes nothing
      if (out_tokens) out_tokens[step] = best;
      ctl[CTL_STEP] = step + 1;
      ctl[CTL_TOKEN] = best;
      hist[hcount % kHist] = best;
      ctl[CTL_HCOUNT] = hcount + 1;
      ctl[CTL_POS] = pos + 1 < 3 ? pos + 1 : 0;  // src/block.c:107
      if (done == kDoneArmed && is_end_token(best)) ctl[CTL_DONE] = kDoneStopped;
    }
    s_tok = done == kDoneStopped ? -1 : best;
  }
  __syncthreads();
  const int tok = s_tok;
  if (tok < 0) return;
  const float* __restrict__ row = embed + (size_t)tok * dm;
  if (dm % 4 == 0 && dm <= 4 * 4 * 256) {
    // every load of the row in flight before the first store (16-byte
    // rows: the embedding table and x are 256-byte aligned, dm % 4 == 0)
    float4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = tid + 256 * k;
      v[k] = 4 * i < dm ? ((const float4*)row)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = tid + 256 * k;
      if (4 * i < dm) ((float4*)x)[i] = v[k];
    }
  } else {
    for (int i = tid; i < dm; i += blockDim.x) x[i] = row[i];
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

// blocks such that each of the 4 waves owns at most NPF row groups
template <int NPF>
static int rows_blocks(int N, int K) {
  const int rpw = K <= 1024 ? 4 : (K <= 2048 ? 2 : 1);
  const int G = (N + rpw - 1) / rpw;
  int b = (G + 4 * NPF - 1) / (4 * NPF);
  return b < 1 ? 1 : b;
}

template <int NPF, bool PRENORM, int MODE, int PICK, bool DROP = false>
static hipError_t rows_t(const float* x, int K, const float* gpre, const float* g,
                         const uint8_t* W, int N, float w_scale, float* out, float* pv, int* pi,
                         hipStream_t s, float temp = 1.0f, DropOut dr = DropOut{},
                         bool fast = false) {
  const size_t lds = lds_bytes(K);
  const dim3 grid(rows_blocks<NPF>(N, K)), block(256);
  if (K % 64 != 0) return hipErrorInvalidValue;
  if constexpr (PRENORM && !DROP) {
    // the LM head: parity and fast mode as separate kernels
    if (K == 1024 || K == 2048) {
      if (K == 1024 && fast)
        hipLaunchKernelGGL((k_rows_fused<16, 1, NPF, 1, PRENORM, MODE, PICK, true, DROP, 2>), grid,
                           block, lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, 1, dr);
      else if (K == 1024)
        hipLaunchKernelGGL((k_rows_fused<16, 1, NPF, 1, PRENORM, MODE, PICK, true, DROP, 1>), grid,
                           block, lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, 0, dr);
      else if (fast)
        hipLaunchKernelGGL((k_rows_fused<32, 1, NPF, 2, PRENORM, MODE, PICK, true, DROP, 2>), grid,
                           block, lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, 1, dr);
      else
        hipLaunchKernelGGL((k_rows_fused<32, 1, NPF, 2, PRENORM, MODE, PICK, true, DROP, 1>), grid,
                           block, lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, 0, dr);
      return hipGetLastError();
    }
  }
  if (K == 1024)
    hipLaunchKernelGGL((k_rows_fused<16, 1, NPF, 1, PRENORM, MODE, PICK, true, DROP>), grid, block, lds,
                       s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K == 2048)
    hipLaunchKernelGGL((k_rows_fused<32, 1, NPF, 2, PRENORM, MODE, PICK, true, DROP>), grid, block, lds,
                       s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K == 4096)
    hipLaunchKernelGGL((k_rows_fused<64, 1, NPF, 4, PRENORM, MODE, PICK, true, DROP>), grid, block, lds,
                       s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K <= 1024)
    hipLaunchKernelGGL((k_rows_fused<16, 1, NPF, 1, PRENORM, MODE, PICK, false, DROP>), grid, block,
                       lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K <= 2048)
    hipLaunchKernelGGL((k_rows_fused<32, 1, NPF, 2, PRENORM, MODE, PICK, false, DROP>), grid, block,
                       lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K <= 4096)
    hipLaunchKernelGGL((k_rows_fused<64, 1, NPF, 4, PRENORM, MODE, PICK, false, DROP>), grid, block,
                       lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else if (K <= 8192)
    hipLaunchKernelGGL((k_rows_fused<64, 2, NPF, 8, PRENORM, MODE, PICK, false, DROP>), grid, block,
                       lds, s, x, K, gpre, g, W, N, w_scale, out, pv, pi, temp, (int)fast, dr);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// proj = BitLinear(x) over the per-head in_proj rows
hipError_t launch_inproj(const float* x, int K, const float* gamma, const uint8_t* W, int N,
                         float w_scale, float* proj, hipStream_t s, bool fast) {
  return rows_t<4, false, 0, 0>(x, K, nullptr, gamma, W, N, w_scale, proj, nullptr, nullptr,
                                    s, 1.0f, DropOut{}, fast);
}

// x += BitLinear(y)  (out_proj with the residual add)
hipError_t launch_outproj(const float* y, int K, const float* gamma, const uint8_t* W, int N,
                          float w_scale, float* x, hipStream_t s, bool fast) {
  return rows_t<2, false, 1, 0>(y, K, nullptr, gamma, W, N, w_scale, x, nullptr, nullptr, s,
                                1.0f, DropOut{}, fast);
}

bool inproj_ssm_fits(int K, int hd) { return K % 64 == 0 && K <= 8192 && hd % kCB == 0; }

// the shapes the fused row kernels (in_proj, out_proj, LM head) cover
bool rows_fit(int K) { return K % 64 == 0 && K <= 8192; }

int dropin_blocks(int N, int K) { return rows_blocks<4>(N, K); }

hipError_t launch_dropin(const float* x, int K, const float* gamma, const uint8_t* W, int N,
                         float w_scale, float* out, float* xn, int8_t* xq, unsigned* flags,
                         unsigned seq, hipStream_t s) {
  if (!rows_fit(K) || N < 1) return hipErrorInvalidValue;
  return rows_t<4, false, 0, 0, true>(x, K, nullptr, gamma, W, N, w_scale, out, nullptr, nullptr,
                                      s, 1.0f, DropOut{xn, xq, flags, seq, nullptr});
}

hipError_t launch_rows_dev(const float* x, int K, const float* gamma, const uint8_t* W, int N,
                           float w_scale, float* out, int8_t* xq, float* scale_x, hipStream_t s) {
  if (!rows_fit(K) || N < 1) return hipErrorInvalidValue;
  return rows_t<4, false, 0, 0>(x, K, nullptr, gamma, W, N, w_scale, out, nullptr, nullptr, s,
                                1.0f, DropOut{nullptr, xq, nullptr, 0, scale_x});
}

bool rows_i8_fit(int K) { return K % 64 == 0 && K <= 8192; }  // K / 16 <= 2 * 256 groups

template <int T, int P, int NPF, int NW = 4>
static hipError_t rows_i8_t(const int8_t* xq, int M, int ldx, int K, const uint8_t* W, int N,
                            bool canonical, int32_t* out, hipStream_t s) {
  const int rpw = 64 / T;
  const int G = (N + rpw - 1) / rpw;
  const dim3 grid((unsigned)max(1, (G + NW * NPF - 1) / (NW * NPF)), (unsigned)M), block(64 * NW);
  const size_t lds = (size_t)K + 16;  // K / 4 dwords of split nibbles + a spare group
  // every token's row starts on 16 bytes: 16-byte loads of x
  const bool xvec = ((uintptr_t)xq & 15) == 0 && (M == 1 || ldx % 16 == 0);
  if (canonical && xvec)
    hipLaunchKernelGGL((k_rows_i8<T, P, NPF, true, true, NW>), grid, block, lds, s, xq, ldx, K, W,
                       N, out);
  else if (canonical)
    hipLaunchKernelGGL((k_rows_i8<T, P, NPF, true, false, NW>), grid, block, lds, s, xq, ldx, K,
                       W, N, out);
  else if (xvec)
    hipLaunchKernelGGL((k_rows_i8<T, P, NPF, false, true, NW>), grid, block, lds, s, xq, ldx, K,
                       W, N, out);
  else
    hipLaunchKernelGGL((k_rows_i8<T, P, NPF, false, false, NW>), grid, block, lds, s, xq, ldx, K,
                       W, N, out);
  return hipGetLastError();
}

hipError_t launch_rows_i8(const int8_t* xq, int M, int ldx, int K, const uint8_t* W, int N,
                          bool canonical, int32_t* out, hipStream_t s) {
  if (!rows_i8_fit(K) || N < 1 || M < 1) return hipErrorInvalidValue;
  if (K <= 1024) return rows_i8_t<16, 1, 4>(xq, M, ldx, K, W, N, canonical, out, s);
  if (K <= 2048) return rows_i8_t<32, 1, 4>(xq, M, ldx, K, W, N, canonical, out, s);
  if (K <= 4096) return rows_i8_t<64, 1, 4>(xq, M, ldx, K, W, N, canonical, out, s);
  // K = N = 8192, M = 1 (stress shape, weights cold, per call with launch
  // gaps): 5.8 us with four row groups per wave (512 blocks of 4 waves);
  // 6.0 with two (1024 blocks), 6.3 with five or eight, 6.4 with one;
  // 6.1-6.9 with blocks of 8 or 16 waves, 6.4-8.7 with blocks of 2
  return rows_i8_t<64, 2, 4>(xq, M, ldx, K, W, N, canonical, out, s);
}

// in_proj + SSM for every head: y (and the states) updated in one launch
template <bool GATED>
static hipError_t inproj_ssm_t(const float* x, int K, const float* gamma, const uint8_t* W,
                               float w_scale, const SsmArgs& args, const dim3& grid,
                               size_t lds, hipStream_t s, bool fast) {
  const dim3 block(256);
  if (K == 1024)
    hipLaunchKernelGGL((k_inproj_ssm<16, 1, 3, 1, true, GATED>), grid, block, lds, s, x, K, gamma,
                       W, w_scale, args, (int)fast);
  else if (K == 2048)
    hipLaunchKernelGGL((k_inproj_ssm<32, 1, 5, 2, true, GATED>), grid, block, lds, s, x, K, gamma,
                       W, w_scale, args, (int)fast);
  else if (K == 4096)
    hipLaunchKernelGGL((k_inproj_ssm<64, 1, 9, 4, true, GATED>), grid, block, lds, s, x, K, gamma,
                       W, w_scale, args, (int)fast);
  else if (K <= 1024)
    hipLaunchKernelGGL((k_inproj_ssm<16, 1, 3, 1, false, GATED>), grid, block, lds, s, x, K,
                       gamma, W, w_scale, args, (int)fast);
  else if (K <= 2048)
    hipLaunchKernelGGL((k_inproj_ssm<32, 1, 5, 2, false, GATED>), grid, block, lds, s, x, K,
                       gamma, W, w_scale, args, (int)fast);
  else if (K <= 4096)
    hipLaunchKernelGGL((k_inproj_ssm<64, 1, 9, 4, false, GATED>), grid, block, lds, s, x, K,
                       gamma, W, w_scale, args, (int)fast);
  else
    hipLaunchKernelGGL((k_inproj_ssm<64, 2, 9, 8, false, GATED>), grid, block, lds, s, x, K,
                       gamma, W, w_scale, args, (int)fast);
  return hipGetLastError();
}

// gated: the kernel reads the done word (CTL_DONE) and, once stopped, leaves
// the state as it is (the step graph of a generate with stop_on_eos)
hipError_t launch_inproj_ssm(const float* x, int K, const float* gamma, const uint8_t* W,
                             float w_scale, int nh, int hd, const float* dt_bias, const float* A,
                             const float* cw, const float* cb, float* cs, float* ssm,
                             const float* D, float* y, const int* ctl, hipStream_t s,
                             bool fast, bool gated) {
  if (!inproj_ssm_fits(K, hd)) return hipErrorInvalidValue;
  const SsmArgs args{dt_bias, A, cw, cb, cs, ssm, D, y, ctl, hd, nh * hd};
  const dim3 grid(nh * (hd / kCB));
  const size_t lds = lds_bytes(K);
  return gated ? inproj_ssm_t<true>(x, K, gamma, W, w_scale, args, grid, lds, s, fast)
               : inproj_ssm_t<false>(x, K, gamma, W, w_scale, args, grid, lds, s, fast);
}

hipError_t launch_ssm_heads(const float* proj, int nh, int hd, const float* dt_bias,
                            const float* A, const float* cw, const float* cb, float* cs,
                            float* ssm, const float* D, float* y, const int* ctl, hipStream_t s) {
  // a block row per head, 256 channels per block
  const int threads = hd < 256 ? (hd + 63) / 64 * 64 : 256;
  hipLaunchKernelGGL(k_ssm_heads, dim3(nh, (hd + threads - 1) / threads), dim3(threads), 0, s,
                     proj, hd, nh * hd, dt_bias, A, cw, cb, cs, ssm, D, y, ctl);
  return hipGetLastError();
}

// LM head: logits = BitLinear(RMSNorm(x; norm_f); lm_head), plus per-block
// greedy candidates when pick is set
constexpr int kLmNpf = 16;  // row groups per wave in the LM head
int lm_head_blocks(int N, int K) { return rows_blocks<kLmNpf>(N, K); }

// pick: 0 logits only, 1 with the blocks' greedy candidates (part_v,
// part_i), 2 logits times 1/temp with the blocks' maxima (part_v)
hipError_t launch_lm_head(const float* x, int K, const float* norm_f, const float* lm_norm,
                          const uint8_t* W, int N, float w_scale, float* logits, int pick,
                          float temp, float* part_v, int* part_i, hipStream_t s, bool fast,
                          const int* gate) {
  DropOut dr{};
  dr.flags = (unsigned*)gate;
  if (pick == 1)
    return rows_t<kLmNpf, true, 0, 1>(x, K, norm_f, lm_norm, W, N, w_scale, logits, part_v, part_i,
                                      s, 1.0f, dr, fast);
  if (pick == 2)
    return rows_t<kLmNpf, true, 0, 2>(x, K, norm_f, lm_norm, W, N, w_scale, logits, part_v, nullptr,
                                      s, temp, dr, fast);
  return rows_t<kLmNpf, true, 0, 0>(x, K, norm_f, lm_norm, W, N, w_scale, logits, nullptr, nullptr,
                                    s, 1.0f, dr, fast);
}

hipError_t launch_pick(const float* part_v, const int* part_i, int n_parts, int* ctl, int* hist,
                       int* out_tokens, const float* embed, int dm, float* x, hipStream_t s) {
  hipLaunchKernelGGL(k_pick, dim3(1), dim3(256), 0, s, part_v, part_i, n_parts, ctl, hist,
                     out_tokens, embed, dm, x);
  return hipGetLastError();
}

}  // namespace bm
