// Fused single-token decode kernels (bs = 1).
//
// A decoded token runs 2 kernels per layer plus one for the LM head:
//   k_inproj_ssm   one block per SSM head: quantize x (block prologue),
//                  GEMV over the head's 2*hd+3 in_proj rows (stored
//                  contiguously on the device), then the head's SSM step
//                  (src/kernel.c:34-70) straight from LDS; writes y.
//   k_rows_fused   quantize the input (block prologue), GEMV over a slice of
//                  rows; used for out_proj with the residual add fused
//                  (src/model.c:1214-1215) and for the LM head with the final
//                  RMSNorm in front (src/model.c:1225, 1259-1261) and the
//                  greedy pick at the end (src/model.c:143-154): the last
//                  block to finish reduces the per-block maxima.
// Every block recomputes the RMSNorm/absmax prologue of its input; the
// sequential sum of squares (four chains, src/kernel.c:77-89) is the
// critical path, so its LDS reads are software-pipelined 32 deep and the
// block's first weight loads are issued before it.
#include "bm_dev.h"
#include "bm_libm.h"

namespace bm {

// control words shared with bm_model.hip
enum { CTL_POS = 0, CTL_TOKEN = 1, CTL_STEP = 2, CTL_HCOUNT = 3, CTL_TICKET = 4 };
constexpr int kHist = 256;

__device__ __forceinline__ float silu_r(float x) {
  return cr_divf(x, __fadd_rn(1.0f, libm::expf_glibc(-x)));
}

__device__ __forceinline__ float softplus_r(float x) {
  if (x > 20.0f) return x;
  return libm::logf_glibc(__fadd_rn(1.0f, libm::expf_glibc(x)));
}

// Sequential fp32 sum of c[0..len) (one lane), loads pipelined 32 ahead.
__device__ __forceinline__ float chain_lds(const float* __restrict__ c, int len) {
  float s = 0.0f;
  int i = 0;
  if (len >= 32) {
    float4 cur[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = *(const float4*)(c + 4 * u);
    for (; i + 32 <= len; i += 32) {
      float4 nxt[8];
      const bool more = i + 64 <= len;
      if (more) {
#pragma unroll
        for (int u = 0; u < 8; ++u) nxt[u] = *(const float4*)(c + i + 32 + 4 * u);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        s = __fadd_rn(s, cur[u].x);
        s = __fadd_rn(s, cur[u].y);
        s = __fadd_rn(s, cur[u].z);
        s = __fadd_rn(s, cur[u].w);
      }
      if (more) {
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      }
    }
  }
  for (; i < len; ++i) s = __fadd_rn(s, c[i]);
  return s;
}

// LDS layout of the quantization prologue for an input of K columns
struct Prologue {
  float* xs;        // [K]   input, then (PRENORM) the normalized feature
  float* sq;        // [4][K/4 + 4]  squares, chain-major
  uint32_t* nib;    // [K/4] split-nibble activations (4 dwords per 16 cols)
  int* slices;      // [S]   sum of int8 values per 1024-column slice
  float* bc;        // [8]   broadcast words
  int sq_stride;
};

__host__ __device__ inline size_t prologue_lds_bytes(int K) {
  const size_t sqs = (size_t)(K / 4 + 4);
  return 4 * (size_t)K + 16 * sqs + (size_t)K + 4 * (size_t)((K + 1023) / 1024) + 64 + 64;
}

__device__ __forceinline__ Prologue prologue_carve(uint8_t* lds, int K) {
  Prologue p;
  p.sq_stride = K / 4 + 4;
  p.sq = (float*)lds;
  p.xs = p.sq + 4 * p.sq_stride;
  p.nib = (uint32_t*)(p.xs + K);
  p.slices = (int*)(p.nib + K / 4);
  p.bc = (float*)(p.slices + (K + 1023) / 1024 + 4);
  return p;
}

// sum of squares of p.xs via the four chains -> rms (src/kernel.c:77-91)
__device__ __forceinline__ float prologue_rms(const Prologue& p, int K) {
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int i = tid; i < K; i += nt) {
    const float v = p.xs[i];
    p.sq[(i & 3) * p.sq_stride + (i >> 2)] = __fmul_rn(v, v);
  }
  __syncthreads();
  if (tid < 4) p.bc[1 + tid] = chain_lds(p.sq + tid * p.sq_stride, K >> 2);
  __syncthreads();
  if (tid == 0) {
    float sum = __fadd_rn(__fadd_rn(__fadd_rn(p.bc[1], p.bc[2]), p.bc[3]), p.bc[4]);
    p.bc[0] = cr_divf(1.0f, cr_sqrtf(__fadd_rn(cr_divf(sum, (float)K), 1e-6f)));
  }
  __syncthreads();
  return p.bc[0];
}

// Quantization prologue of scalar_bitlinear_forward (src/kernel.c:356-391)
// over an input already in p.xs; fills p.nib and p.slices, returns scale_x.
// K % 64 == 0, blockDim.x a multiple of 64.
__device__ float prologue_quant(const Prologue& p, int K, const float* __restrict__ gamma,
                                float rms) {
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
  float mx = 0.0f;
  for (int i = tid; i < K; i += nt)
    mx = fmaxf(mx, fabsf(__fmul_rn(__fmul_rn(p.xs[i], rms), gamma[i])));
  mx = wave_max_f32(mx);
  if (lane == 0) p.bc[8 + wave] = mx;  // bc has room: carved 64 bytes after slices
  __syncthreads();
  float max_abs = 0.0f;
  for (int w = 0; w < (nt >> 6); ++w) max_abs = fmaxf(max_abs, p.bc[8 + w]);
  const float scale_x = cr_divf(127.0f, __fadd_rn(max_abs, 1e-5f));
  const int n_groups = K >> 4;
  for (int g0 = 0; g0 < n_groups; g0 += nt) {
    const int g = g0 + tid;
    int qsum = 0;
    if (g < n_groups) {
      int q[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int c = 16 * g + j;
        const float v = __fmul_rn(__fmul_rn(p.xs[c], rms), gamma[c]);
        const float t = __fmul_rn(v, scale_x);
        int iv = (int)__fadd_rn(t, t >= 0.0f ? 0.5f : -0.5f);
        iv = iv > 127 ? 127 : (iv < -128 ? -128 : iv);
        q[j] = iv;
        qsum += iv;
      }
      uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        le |= (uint32_t)(q[2 * n] & 15) << (4 * n);
        lo |= (uint32_t)(q[2 * n + 1] & 15) << (4 * n);
        he |= (uint32_t)((q[2 * n] >> 4) & 15) << (4 * n);
        ho |= (uint32_t)((q[2 * n + 1] >> 4) & 15) << (4 * n);
      }
      *(uint4*)(p.nib + 4 * g) = make_uint4(le, lo, he, ho);
    }
    const int s = wave_sum_i32(qsum);  // one wave = 64 groups = one slice
    const int slice = (g0 >> 6) + wave;
    if (lane == 0 && slice < slices_of(K)) p.slices[slice] = s;
  }
  __syncthreads();
  return scale_x;
}

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

// Row dot product finish: reduce a lane partial over its 16-lane slice
// group, subtract the slice's sum of x, fold the slices of the T-lane row
// team in slice order into fp32 (src/kernel.c:255-256, 407-425).
template <int T>
__device__ __forceinline__ float row_finish(int part, int xs_slice, int p_index, int n_slices,
                                            float inv, float o, int unit_base) {
  part += __shfl_xor(part, 8, 64);
  part += __shfl_xor(part, 4, 64);
  part += __shfl_xor(part, 2, 64);
  part += __shfl_xor(part, 1, 64);
  const float f = __fmul_rn((float)(part - xs_slice), inv);
#pragma unroll
  for (int q = 0; q < T / 16; ++q) {
    const float fq = __shfl(f, unit_base + 16 * q, 64);
    if (p_index * (T / 16) + q < n_slices) o = __fadd_rn(o, fq);
  }
  return o;
}

// lane activations of the chunks it owns: nib groups 4j..4j+3
template <int P, int T>
__device__ __forceinline__ void load_lane_act(const Prologue& pr, int K, int u,
                                              uint32_t (&xa)[P][16], int (&xsl)[P]) {
  const int chunks = K >> 6;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * T + u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 v = j < chunks ? *(const uint4*)(pr.nib + 16 * j + 4 * g) : make_uint4(0, 0, 0, 0);
      xa[p][4 * g + 0] = v.x;
      xa[p][4 * g + 1] = v.y;
      xa[p][4 * g + 2] = v.z;
      xa[p][4 * g + 3] = v.w;
    }
    const int sl = (p * T + u) >> 4;
    xsl[p] = sl < slices_of(K) ? pr.slices[sl] : 0;
  }
}

// ---------------------------------------------------------------------------
// in_proj GEMV + SSM step, one block per head.
//   rows of head h in the device copy: [z (hd) | x (hd) | B | C | dt]
// ---------------------------------------------------------------------------
template <int T, int P, int NPF>
__global__ __launch_bounds__(1024) void k_inproj_ssm(
    const float* __restrict__ x, int K, const float* __restrict__ gamma,
    const uint8_t* __restrict__ W, float w_scale, int hd, int di, const float* __restrict__ dt_bias,
    const float* __restrict__ A, const float* __restrict__ cw, const float* __restrict__ cb,
    float* __restrict__ cs, float* __restrict__ ssm, const float* __restrict__ D,
    float* __restrict__ y, const int* __restrict__ ctl) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int RPW = 64 / T;
  const int h = blockIdx.x;
  const int rows = 2 * hd + 3;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int n_groups = (rows + RPW - 1) / RPW;
  const size_t wstride = (size_t)(K >> 2);
  const uint8_t* __restrict__ Wh = W + (size_t)h * rows * wstride;
  const int chunks = K >> 6;

  // weight prefetch: this wave's first NPF row groups
  uint4 wv[NPF][P];
#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int r = (wave + it * nwaves) * RPW + sub;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      wv[it][p] = (r < rows && j < chunks) ? *(const uint4*)(Wh + (size_t)r * wstride + 16 * j)
                                           : make_uint4(0, 0, 0, 0);
    }
  }

  Prologue pr = prologue_carve(lds, K);
  float* pj = (float*)(lds + prologue_lds_bytes(K));  // [rows] projections of this head
  for (int i = tid; i < K; i += blockDim.x) pr.xs[i] = x[i];
  const float rms = prologue_rms(pr, K);
  const float scale_x = prologue_quant(pr, K, gamma, rms);
  const float inv = inv_scale_of(scale_x, w_scale);

  uint32_t xa[P][16];
  int xsl[P];
  load_lane_act<P, T>(pr, K, u, xa, xsl);

#pragma unroll
  for (int it = 0; it < NPF; ++it) {
    const int grp = wave + it * nwaves;
    const int r = grp * RPW + sub;
    if (grp < n_groups) {  // uniform per wave
      float o = 0.0f;
#pragma unroll
      for (int p = 0; p < P; ++p)
        o = row_finish<T>(dot64(wv[it][p], xa[p]), xsl[p], p, slices_of(K), inv, o, unit_base);
      if (u == 0 && r < rows) pj[r] = o;
    }
  }
  // groups past the prefetched ones (none at the model shapes)
  for (int grp = wave + NPF * nwaves; grp < n_groups; grp += nwaves) {
    const int r = grp * RPW + sub;
    float o = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      const uint4 w = (r < rows && j < chunks) ? *(const uint4*)(Wh + (size_t)r * wstride + 16 * j)
                                               : make_uint4(0, 0, 0, 0);
      o = row_finish<T>(dot64(w, xa[p]), xsl[p], p, slices_of(K), inv, o, unit_base);
    }
    if (u == 0 && r < rows) pj[r] = o;
  }
  __syncthreads();

  // SSM step for the hd channels of this head (src/kernel.c:46-69)
  if (tid < hd) {
    const int c = tid, idx = h * hd + c;
    const int pos = ctl[CTL_POS];
    const int t1 = pos + 1 < 3 ? pos + 1 : pos - 2;
    const int t2 = pos + 2 < 3 ? pos + 2 : pos - 1;
    const float dt_val = softplus_r(__fadd_rn(pj[2 * hd + 2], dt_bias[h]));
    const float decay = libm::expf_glibc(__fmul_rn(A[h], dt_val));
    const float Bdt = __fmul_rn(pj[2 * hd], dt_val);
    const float C_val = pj[2 * hd + 1];
    const float xin = pj[hd + c];
    float* c0 = cs + (size_t)pos * di;
    float conv = __fadd_rn(cb[idx], __fmul_rn(c0[idx], cw[idx]));
    conv = __fadd_rn(conv, __fmul_rn(cs[(size_t)t1 * di + idx], cw[di + idx]));
    conv = __fadd_rn(conv, __fmul_rn(cs[(size_t)t2 * di + idx], cw[2 * di + idx]));
    conv = __fadd_rn(conv, __fmul_rn(xin, cw[3 * di + idx]));
    c0[idx] = xin;
    const float xa_ = silu_r(conv);
    const float st = __fadd_rn(__fmul_rn(ssm[idx], decay), __fmul_rn(xa_, Bdt));
    ssm[idx] = st;
    y[idx] = __fmul_rn(__fadd_rn(__fmul_rn(st, C_val), __fmul_rn(xa_, D[idx])), silu_r(pj[c]));
  }
}

// ---------------------------------------------------------------------------
// Quantize + GEMV over a slice of rows, 256 threads per block.
//   PRENORM: input first goes through RMSNorm(norm_f) (the reference's final
//            norm), then the BitLinear's own norm.
//   MODE:    0 store, 1 accumulate (residual)
//   ARGMAX:  greedy pick over all rows; the last block finishes the step
// ---------------------------------------------------------------------------
struct StepIO {
  int* ctl;
  int* hist;
  int* out_tokens;
  float* part_v;  // [gridDim.x]
  int* part_i;
  const float* embed;  // next token's embedding row goes to x_next
  float* x_next;
  int dm;
};

template <int T, int P, bool PRENORM, int MODE, bool ARGMAX>
__global__ __launch_bounds__(256) void k_rows_fused(const float* __restrict__ x, int K,
                                                    const float* __restrict__ gamma_pre,
                                                    const float* __restrict__ gamma,
                                                    const uint8_t* __restrict__ W, int N,
                                                    float w_scale, float* __restrict__ out,
                                                    StepIO io) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int RPW = 64 / T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int u = lane % T, sub = lane / T, unit_base = sub * T;
  const int G = (N + RPW - 1) / RPW;
  const int g0 = (int)((long long)blockIdx.x * G / gridDim.x);
  const int g1 = (int)((long long)(blockIdx.x + 1) * G / gridDim.x);
  const size_t wstride = (size_t)(K >> 2);
  const int chunks = K >> 6;

  // prefetch the first row group of this wave
  uint4 w[P];
  {
    const int r = (g0 + wave) * RPW + sub;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      w[p] = (g0 + wave < g1 && r < N && j < chunks)
                 ? *(const uint4*)(W + (size_t)r * wstride + 16 * j)
                 : make_uint4(0, 0, 0, 0);
    }
  }

  Prologue pr = prologue_carve(lds, K);
  for (int i = tid; i < K; i += blockDim.x) pr.xs[i] = x[i];
  float rms = prologue_rms(pr, K);
  if (PRENORM) {
    // final_feat = (x * rms) * norm_f  (src/model.c:1225, src/kernel.c:93-103)
    for (int i = tid; i < K; i += blockDim.x)
      pr.xs[i] = __fmul_rn(__fmul_rn(pr.xs[i], rms), gamma_pre[i]);
    __syncthreads();
    rms = prologue_rms(pr, K);
  }
  const float scale_x = prologue_quant(pr, K, gamma, rms);
  const float inv = inv_scale_of(scale_x, w_scale);
  uint32_t xa[P][16];
  int xsl[P];
  load_lane_act<P, T>(pr, K, u, xa, xsl);

  float best_v = -1e9f;
  int best_i = 0x7fffffff;
  for (int grp = g0 + wave; grp < g1; grp += 4) {
    const int r = grp * RPW + sub;
    // next group's weights while this one computes
    uint4 wn[P];
    const int rn = (grp + 4) * RPW + sub;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = p * T + u;
      wn[p] = (grp + 4 < g1 && rn < N && j < chunks)
                  ? *(const uint4*)(W + (size_t)rn * wstride + 16 * j)
                  : make_uint4(0, 0, 0, 0);
    }
    float o = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p)
      o = row_finish<T>(dot64(w[p], xa[p]), xsl[p], p, slices_of(K), inv, o, unit_base);
    if (u == 0 && r < N) {
      if (MODE == 1)
        out[r] = __fadd_rn(out[r], o);
      else
        out[r] = o;
      if (ARGMAX && o > best_v) {  // rows ascend per lane: first max kept
        best_v = o;
        best_i = r;
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) w[p] = wn[p];
  }

  if (ARGMAX) {
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int s_last;
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
      sv[wave] = best_v;
      si[wave] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
      for (int k = 1; k < 4; ++k)
        if (sv[k] > best_v || (sv[k] == best_v && si[k] < best_i)) {
          best_v = sv[k];
          best_i = si[k];
        }
      io.part_v[blockIdx.x] = best_v;
      io.part_i[blockIdx.x] = best_i;
      __threadfence();
      const int t = atomicAdd(io.ctl + CTL_TICKET, 1);
      s_last = (t == (int)gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    // last block: reduce the per-block candidates (block order = row order)
    float bv = -1e9f;
    int bi = 0x7fffffff;
    for (int b = tid; b < (int)gridDim.x; b += blockDim.x) {
      const float v = io.part_v[b];
      const int i = io.part_i[b];
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
    __syncthreads();
    if (lane == 0) {
      sv[wave] = bv;
      si[wave] = bi;
    }
    __syncthreads();
    __shared__ int s_tok;
    if (tid == 0) {
      for (int k = 1; k < 4; ++k)
        if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) {
          bv = sv[k];
          bi = si[k];
        }
      const int best = bi == 0x7fffffff ? 0 : bi;
      int* ctl = io.ctl;
      const int step = ctl[CTL_STEP];
      if (io.out_tokens) io.out_tokens[step] = best;
      ctl[CTL_STEP] = step + 1;
      ctl[CTL_TOKEN] = best;
      io.hist[ctl[CTL_HCOUNT] % kHist] = best;
      ctl[CTL_HCOUNT] += 1;
      ctl[CTL_POS] = ctl[CTL_POS] + 1 < 3 ? ctl[CTL_POS] + 1 : 0;  // src/block.c:107
      ctl[CTL_TICKET] = 0;
      s_tok = best;
    }
    __syncthreads();
    // next step's input: x = embed[token] (src/model.c:1195-1202)
    const int tok = s_tok;
    for (int i = tid; i < io.dm; i += blockDim.x)
      io.x_next[i] = io.embed[(size_t)tok * io.dm + i];
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
hipError_t launch_inproj_ssm(const float* x, int K, const float* gamma, const uint8_t* W,
                             float w_scale, int nh, int hd, const float* dt_bias,
                             const float* A, const float* cw, const float* cb, float* cs,
                             float* ssm, const float* D, float* y, const int* ctl,
                             hipStream_t s) {
  const int di = nh * hd;
  const size_t lds = prologue_lds_bytes(K) + 4 * (size_t)(2 * hd + 3) + 16;
  const dim3 grid(nh), block(1024);
  if (K <= 1024)
    hipLaunchKernelGGL((k_inproj_ssm<16, 1, 3>), grid, block, lds, s, x, K, gamma, W, w_scale,
                       hd, di, dt_bias, A, cw, cb, cs, ssm, D, y, ctl);
  else if (K <= 2048)
    hipLaunchKernelGGL((k_inproj_ssm<32, 1, 5>), grid, block, lds, s, x, K, gamma, W, w_scale,
                       hd, di, dt_bias, A, cw, cb, cs, ssm, D, y, ctl);
  else if (K <= 4096)
    hipLaunchKernelGGL((k_inproj_ssm<64, 1, 9>), grid, block, lds, s, x, K, gamma, W, w_scale,
                       hd, di, dt_bias, A, cw, cb, cs, ssm, D, y, ctl);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <bool PRENORM, int MODE, bool ARGMAX>
static hipError_t rows_fused_t(const float* x, int K, const float* gpre, const float* g,
                               const uint8_t* W, int N, float w_scale, float* out, StepIO io,
                               int blocks, hipStream_t s) {
  const size_t lds = prologue_lds_bytes(K);
  if (K <= 1024)
    hipLaunchKernelGGL((k_rows_fused<16, 1, PRENORM, MODE, ARGMAX>), dim3(blocks), dim3(256),
                       lds, s, x, K, gpre, g, W, N, w_scale, out, io);
  else if (K <= 2048)
    hipLaunchKernelGGL((k_rows_fused<32, 1, PRENORM, MODE, ARGMAX>), dim3(blocks), dim3(256),
                       lds, s, x, K, gpre, g, W, N, w_scale, out, io);
  else if (K <= 4096)
    hipLaunchKernelGGL((k_rows_fused<64, 1, PRENORM, MODE, ARGMAX>), dim3(blocks), dim3(256),
                       lds, s, x, K, gpre, g, W, N, w_scale, out, io);
  else if (K <= 8192)
    hipLaunchKernelGGL((k_rows_fused<64, 2, PRENORM, MODE, ARGMAX>), dim3(blocks), dim3(256),
                       lds, s, x, K, gpre, g, W, N, w_scale, out, io);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// out (+)= BitLinear(x) over N rows; blocks chosen for the row count
hipError_t launch_rows_fused(const float* x, int K, const float* gamma, const uint8_t* W, int N,
                             float w_scale, float* out, bool accumulate, hipStream_t s) {
  StepIO io{};
  const int rpw = K <= 1024 ? 4 : (K <= 2048 ? 2 : 1);
  int blocks = (N / rpw + 7) / 8;  // ~2 row groups per wave
  if (blocks > 256) blocks = 256;
  if (blocks < 1) blocks = 1;
  if (accumulate)
    return rows_fused_t<false, 1, false>(x, K, nullptr, gamma, W, N, w_scale, out, io, blocks, s);
  return rows_fused_t<false, 0, false>(x, K, nullptr, gamma, W, N, w_scale, out, io, blocks, s);
}

// LM head: RMSNorm(norm_f) + BitLinear(lm_head) -> logits, then (argmax)
// the greedy step bookkeeping and the next token's embedding
hipError_t launch_lm_head(const float* x, int K, const float* norm_f, const float* lm_norm,
                          const uint8_t* W, int N, float w_scale, float* logits, bool argmax,
                          int* ctl, int* hist, int* out_tokens, float* part_v, int* part_i,
                          const float* embed, float* x_next, int blocks, hipStream_t s) {
  StepIO io{ctl, hist, out_tokens, part_v, part_i, embed, x_next, K};
  if (argmax)
    return rows_fused_t<true, 0, true>(x, K, norm_f, lm_norm, W, N, w_scale, logits, io, blocks,
                                       s);
  return rows_fused_t<true, 0, false>(x, K, norm_f, lm_norm, W, N, w_scale, logits, io, blocks,
                                      s);
}

size_t decode_prologue_lds(int K) { return prologue_lds_bytes(K); }

}  // namespace bm
