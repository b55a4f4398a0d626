// Device-resident BitMamba model: the reference's model_load /
// model_prefill / model_forward_step (src/model.c:477-1314, src/block.c)
// with every activation kept in HBM.
//
// Per decoded token the device runs, without a host round trip, per layer
//   k_rows_fused (quantize x + in_proj GEMV) -> k_ssm_heads (SSM step) ->
//   k_rows_fused (quantize y + out_proj GEMV accumulated into x)
// then the LM head (RMSNorm(norm_f) + quantize + GEMV, each block keeping
// its greedy candidate) and k_pick (greedy choice, bookkeeping, embedding of
// the next token); with a repetition penalty the LM head is followed by
// k_penalty, k_argmax_step and k_embed instead.  The sequence is captured
// once into a hipGraph and replayed; the current token, conv ring position,
// step counter and history live in device memory.
// Numerics are those of the scalar reference path, bit for bit.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "bm_bit2.h"
#include "bm_common.h"
#include "bm_fp.h"
#include "bm_hip.h"
#include "bm_libm.h"

namespace bm {

// control block in device memory
// CTL_DONE: 0 steps always run, 1 armed (generate with stop_on_eos), 2 the
// end token was picked: later steps change nothing (bm_decode.hip)
enum { CTL_POS = 0, CTL_DONE = 1, CTL_STEP = 2, CTL_HCOUNT = 3, CTL_TOKEN = 4, CTL_WORDS = 8 };
constexpr int kDoneArmed = 1, kDoneStopped = 2;
constexpr int kHistory = 256;  // HISTORY_MAX (src/main.c:19)

__device__ __forceinline__ float silu_ref(float x) {
  // x / (1.0f + expf(-x))  (src/bitmamba.h:234-237)
  return cr_divf(x, __fadd_rn(1.0f, libm::expf_glibc(-x)));
}

__device__ __forceinline__ float softplus_ref(float x) {
  // x > 20 ? x : logf(1.0f + expf(x))  (src/bitmamba.h:238-243)
  if (x > 20.0f) return x;
  return libm::logf_glibc(__fadd_rn(1.0f, libm::expf_glibc(x)));
}

// Prefill SSM (ssm_batch_worker, src/block.c:127-160) in three phases.  Of
// scalar_ssm_inner's per-token work (src/kernel.c:34-70) only the state
// update st = st * decay + xa * (B * dt) and y = (st * C + xa * D) * silu(z)
// depend on the previous token; dt, decay, the depthwise conv over the
// token's three predecessors, silu and the products with B * dt and D do
// not.  Phase 1 computes those for a chunk of tokens with one thread per
// (channel, 4-token quad); phase 2 runs the recurrence, one thread per
// channel; phase 3 forms y from each token's state, again in parallel.
// Every value is the same fp32 expression, in the same order, as in the
// token-serial loop, so the results are bit for bit those of that loop.
// proj holds the in_proj outputs in the device's per-head order: head h
// occupies [h*(2hd+3), (h+1)*(2hd+3)) of a token's row as
// [z (hd) | x (hd) | B | C | dt].
constexpr int kSsmChunk = 1024;  // tokens per pass of the three phases
// Phase values of a chunk of nt tokens, in nq = ceil(nt / 4) token quads.
// The recurrence reads and writes per channel four tokens at a time, so its
// planes keep a quad's four values together:
//   XBDT  xa * B * dt   [nqa][di][4]   (phase 1 -> 2)
//   ST    the state after each token [nqa][di][4]   (phase 2 -> 3)
//   DECAY exp(A * dt)   [nh][nqa * 4]  (phase 1 -> 2)
// and the rest per (token, channel) or (token, head):
//   XAD   xa * D  [nt][di]   (phase 1 -> 3; phase 3 takes silu(z) itself,
//         which balances the two: phase 1 is VALU-bound, phase 3 memory-bound)
//   C     [nt][nh]                         (phase 1 -> 3)
// The recurrence runs without conditions over nqr quads (nq rounded up to
// whole pairs of its Q-quad buffers): tokens past nt carry decay 1 and
// xa * B * dt = -0, which leave every state value, zeros' signs included,
// as it is.  Its last prefetch reads Q quads further (nqa = nqr + Q).
constexpr int kScanQ = 8, kScanQSmall = 4;
__host__ __device__ inline int scan_q(int nq) { return nq <= 2 * kScanQSmall ? kScanQSmall : kScanQ; }
struct PreLayout {
  int nq, nqr, nqa;
  size_t xbdt, st, decay, xad, c, total;  // float offsets
};
__host__ __device__ inline PreLayout pre_layout(int nt, int di, int nh) {
  PreLayout L;
  L.nq = (nt + 3) / 4;
  const int q = scan_q(L.nq);
  L.nqr = (L.nq + 2 * q - 1) / (2 * q) * (2 * q);
  L.nqa = L.nqr + q;
  const size_t ch = (size_t)di, nq4 = (size_t)L.nqa * 4;
  L.xbdt = 0;
  L.st = L.xbdt + nq4 * ch;
  L.decay = L.st + nq4 * ch;  // float4 reads: every offset up to here is a multiple of 4
  L.xad = L.decay + (size_t)nh * nq4;
  L.c = L.xad + (size_t)nt * ch;
  L.total = L.c + (size_t)nt * nh;
  return L;
}

// Phase 1, one block per (256 channels, token quad) over the nqr quads:
// the head values (dt, decay, B * dt) once per (token, head) of the block,
// then per channel the conv over the quad's window of inputs, silu and the
// products; tokens past the chunk get the recurrence's identity values
__global__ __launch_bounds__(256) void k_ssm_prep(const float* __restrict__ proj, int pd, int t0,
                                                  int nt, int di, int nh, int hd,
                                                  const float* __restrict__ dt_bias,
                                                  const float* __restrict__ A,
                                                  const float* __restrict__ cw,
                                                  const float* __restrict__ cb,
                                                  const float* __restrict__ cs,
                                                  const float* __restrict__ D,
                                                  const int* __restrict__ ctl,
                                                  float* __restrict__ pre) {
  __shared__ float s_bdt[4][256];
  const PreLayout PL = pre_layout(nt, di, nh);
  const int idx = blockIdx.x * blockDim.x + threadIdx.x, q = blockIdx.y, tq = 4 * q;
  // the heads this block's channels belong to: h_first .. h_first + nhb - 1
  const int h_first = (blockIdx.x * blockDim.x) / hd;
  const int nhb = min(di - 1, (int)(blockIdx.x * blockDim.x + blockDim.x) - 1) / hd - h_first + 1;
  // the channel's inputs first, so that their loads are in flight while the
  // head threads run the softplus / exp chains below
  const bool live = idx < di;
  const int ci = live ? idx : di - 1;
  const int h = ci / hd, c = ci - h * hd;
  const size_t xoff = (size_t)h * (2 * hd + 3) + hd + c;
  const int pos0 = ctl[CTL_POS];
  // inputs of tokens tq-3 .. tq+3 of the chunk: from the batch, or from the
  // conv ring for the three tokens before the prompt (x_{-j} sits at ring
  // position pos0 + 3 - j); past the chunk's end: unused
  float xv[7];
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    const int tp = tq - 3 + k, tg = t0 + tp;
    xv[k] = tp >= nt ? 0.0f
            : tg >= 0 ? proj[(size_t)tg * pd + xoff]
                      : cs[(size_t)((pos0 + 3 + tg) % 3) * di + ci];
  }
  const float w0 = cw[ci], w1 = cw[di + ci], w2 = cw[2 * di + ci], w3 = cw[3 * di + ci];
  const float bias = cb[ci], Dv = D[ci];
  for (int w = threadIdx.x; w < 4 * nhb; w += blockDim.x) {
    const int e = w / nhb, hb = w - e * nhb, t = tq + e, h = h_first + hb;
    float decay = 1.0f;
    if (t < nt) {
      const float* __restrict__ ph = proj + (size_t)(t0 + t) * pd + (size_t)h * (2 * hd + 3);
      const float dt_val = softplus_ref(__fadd_rn(ph[2 * hd + 2], dt_bias[h]));
      s_bdt[e][hb] = __fmul_rn(ph[2 * hd], dt_val);
      decay = libm::expf_glibc(__fmul_rn(A[h], dt_val));
      pre[PL.c + (size_t)t * nh + h] = ph[2 * hd + 1];
    }
    pre[PL.decay + (size_t)h * PL.nqa * 4 + t] = decay;
  }
  __syncthreads();
  if (!live) return;
  float xb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = tq + e;
    xb[e] = -0.0f;
    if (t < nt) {
      float conv = __fadd_rn(bias, __fmul_rn(xv[e], w0));
      conv = __fadd_rn(conv, __fmul_rn(xv[e + 1], w1));
      conv = __fadd_rn(conv, __fmul_rn(xv[e + 2], w2));
      conv = __fadd_rn(conv, __fmul_rn(xv[e + 3], w3));
      const float xa = silu_ref(conv);
      xb[e] = __fmul_rn(xa, s_bdt[e][h - h_first]);
      const size_t at = (size_t)t * di + idx;
      pre[PL.xad + at] = __fmul_rn(xa, Dv);
    }
  }
  reinterpret_cast<float4*>(pre + PL.xbdt)[(size_t)q * di + idx] =
      make_float4(xb[0], xb[1], xb[2], xb[3]);
}

// Phase 2 for the chunk's tokens: the state recurrence alone, one thread per
// channel, a quad of tokens per load, two buffers of Q quads in flight and
// no branch in the loop, so loads wait only for their own buffer.  The last
// chunk (n_total > 0) also leaves the conv ring as the token loop would: the
// inputs of the last three tokens at their ring positions.
template <int Q>
__global__ __launch_bounds__(64) void k_ssm_scan(float* __restrict__ pre, int nt, int di, int nh,
                                                 float* __restrict__ ssm,
                                                 const float* __restrict__ proj, int pd, int hd,
                                                 float* __restrict__ cs,
                                                 const int* __restrict__ ctl, int n_total) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= di) return;
  const PreLayout PL = pre_layout(nt, di, nh);
  const int h = idx / hd;
  const float4* __restrict__ xbq = reinterpret_cast<const float4*>(pre + PL.xbdt) + idx;
  const float4* __restrict__ decq =
      reinterpret_cast<const float4*>(pre + PL.decay + (size_t)h * PL.nqa * 4);
  float4* __restrict__ stq = reinterpret_cast<float4*>(pre + PL.st) + idx;
  float st = ssm[idx];
  float4 dec[2][Q], xb[2][Q];
  auto fetch = [&](int buf, int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      dec[buf][j] = decq[qb + j];
      xb[buf][j] = xbq[(size_t)(qb + j) * di];
    }
  };
  auto run = [&](int buf, int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const float4 d = dec[buf][j], x = xb[buf][j];
      float4 o;
      st = __fadd_rn(__fmul_rn(st, d.x), x.x);
      o.x = st;
      st = __fadd_rn(__fmul_rn(st, d.y), x.y);
      o.y = st;
      st = __fadd_rn(__fmul_rn(st, d.z), x.z);
      o.z = st;
      st = __fadd_rn(__fmul_rn(st, d.w), x.w);
      o.w = st;
      stq[(size_t)(qb + j) * di] = o;
    }
  };
  // the scheduler barriers keep each buffer's loads ahead of the other's
  // updates, as written
  fetch(0, 0);
  for (int qb = 0; qb < PL.nqr; qb += 2 * Q) {
    fetch(1, qb + Q);
    __builtin_amdgcn_sched_barrier(0);
    run(0, qb);
    __builtin_amdgcn_sched_barrier(0);
    fetch(0, qb + 2 * Q);  // past nqr on the last pass: read, not used
    __builtin_amdgcn_sched_barrier(0);
    run(1, qb + Q);
    __builtin_amdgcn_sched_barrier(0);
  }
  ssm[idx] = st;
  if (n_total > 0) {
    const int c = idx - h * hd;
    const int pos0 = ctl[CTL_POS];
    for (int k = max(0, n_total - 3); k < n_total; ++k)
      cs[(size_t)((pos0 + k) % 3) * di + idx] =
          proj[(size_t)k * pd + (size_t)h * (2 * hd + 3) + hd + c];
  }
}

// Phase 3, one thread per (channel, token quad): y = (st * C + xa * D) *
// silu(z) with st the state phase 2 left after each token
__global__ __launch_bounds__(256) void k_ssm_out(const float* __restrict__ pre,
                                                 const float* __restrict__ proj, int pd, int t0,
                                                 int nt, int di, int nh, int hd,
                                                 float* __restrict__ y) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x, q = blockIdx.y;
  if (idx >= di) return;
  const PreLayout PL = pre_layout(nt, di, nh);
  const int h = idx / hd;
  const size_t zoff = (size_t)h * (2 * hd + 3) + (idx - h * hd);
  const float4 s4 = reinterpret_cast<const float4*>(pre + PL.st)[(size_t)q * di + idx];
  const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 4 * q + e;
    if (t < nt) {
      const size_t at = (size_t)t * di + idx;
      y[(size_t)(t0 + t) * di + idx] =
          __fmul_rn(__fadd_rn(__fmul_rn(sv[e], pre[PL.c + (size_t)t * nh + h]), pre[PL.xad + at]),
                    silu_ref(proj[(size_t)(t0 + t) * pd + zoff]));
    }
  }
}

__global__ void k_advance_pos(int* ctl, int n) {
  if (threadIdx.x == 0 && blockIdx.x == 0) ctl[CTL_POS] = (ctl[CTL_POS] + n) % 3;
}

// a decode run's steps count from 0 (the tokens buffer is filled from its
// start) and always run (a continuation after an end token goes on from it)
__global__ void k_restart_steps(int* ctl) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    ctl[CTL_STEP] = 0;
    ctl[CTL_DONE] = 0;
  }
}

// x[t] = embed[tok[t]]; out-of-range ids read row 0 (src/model.c:1116-1122)
__global__ void k_embed(const float* __restrict__ embed, int dm, int vocab,
                        const int* __restrict__ toks, float* __restrict__ x) {
  const int t = blockIdx.y;
  int tok = toks[t];
  if (tok < 0 || tok >= vocab) tok = 0;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dm; i += gridDim.x * blockDim.x)
    x[(size_t)t * dm + i] = embed[(size_t)tok * dm + i];
}

// A_precomp = -expf(A_log) (src/model.c:786-792)
__global__ void k_neg_exp(const float* __restrict__ a, float* __restrict__ out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = -libm::expf_glibc(a[i]);
}

// Repetition penalty over the distinct tokens of the last kHistory
// (src/model.c:1272-1305).  Each distinct token is scaled once, so the
// entries can be processed in parallel.
__global__ void k_penalty(float* __restrict__ logits, int vocab, const int* __restrict__ hist,
                          const int* __restrict__ ctl, float penalty) {
  if (ctl[CTL_DONE] == kDoneStopped) return;  // the logits stay those of the end token's step
  const int count = ctl[CTL_HCOUNT];
  const int len = count < kHistory ? count : kHistory;
  const int j = threadIdx.x;
  if (j >= len) return;
  const int base = count - len;
  const int past = hist[(base + j) % kHistory];
  if (past < 0 || past >= vocab) return;
  for (int i = 0; i < j; ++i)
    if (hist[(base + i) % kHistory] == past) return;  // not the first occurrence
  if (past == 50256 || past == 198 || past == 628 || past == 13) return;
  if (!(penalty > 0.0f)) return;
  const float v = logits[past];
  logits[past] = v > 0 ? cr_divf(v, penalty) : __fmul_rn(v, penalty);
}

// Greedy pick: first index of the maximum, starting from best = 0 and
// max = -1e9 (src/model.c:143-154).  Then bookkeeping for the next step.
__global__ __launch_bounds__(1024) void k_argmax_step(const float* __restrict__ logits, int vocab,
                                                       int* __restrict__ ctl,
                                                       int* __restrict__ hist,
                                                       int* __restrict__ out_tokens) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float bv = -1e9f;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < vocab; i += blockDim.x) {
    const float v = logits[i];
    if (v > bv) {  // ascending i per thread: first max kept
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) {
        bv = sv[w];
        bi = si[w];
      }
    const int best = bi == 0x7fffffff ? 0 : bi;
    if (ctl[CTL_DONE] == kDoneStopped) return;  // a stopped decode changes nothing
    const int step = ctl[CTL_STEP];
    if (out_tokens) out_tokens[step] = best;
    ctl[CTL_STEP] = step + 1;
    ctl[CTL_TOKEN] = best;
    hist[ctl[CTL_HCOUNT] % kHistory] = best;
    ctl[CTL_HCOUNT] += 1;
    ctl[CTL_POS] = ctl[CTL_POS] + 1 < 3 ? ctl[CTL_POS] + 1 : 0;  // src/block.c:107
    if (ctl[CTL_DONE] == kDoneArmed && (best == 50256 || best == 0)) ctl[CTL_DONE] = kDoneStopped;
  }
}

hipError_t launch_inproj(const float* x, int K, const float* gamma, const uint8_t* W, int N,
                         float w_scale, float* proj, hipStream_t s, bool fast);
hipError_t launch_outproj(const float* y, int K, const float* gamma, const uint8_t* W, int N,
                          float w_scale, float* x, hipStream_t s, bool fast);
bool inproj_ssm_fits(int K, int hd);
hipError_t launch_inproj_ssm(const float* x, int K, const float* gamma, const uint8_t* W,
                             float w_scale, int nh, int hd, const float* dt_bias, const float* A,
                             const float* cw, const float* cb, float* cs, float* ssm,
                             const float* D, float* y, const int* ctl, hipStream_t s,
                             bool fast, bool gated = false);
hipError_t launch_ssm_heads(const float* proj, int nh, int hd, const float* dt_bias,
                            const float* A, const float* cw, const float* cb, float* cs,
                            float* ssm, const float* D, float* y, const int* ctl, hipStream_t s);
int lm_head_blocks(int N, int K);
hipError_t launch_lm_head(const float* x, int K, const float* norm_f, const float* lm_norm,
                          const uint8_t* W, int N, float w_scale, float* logits, int pick,
                          float temp, float* part_v, int* part_i, hipStream_t s, bool fast,
                          const int* gate = nullptr);
hipError_t launch_pick(const float* part_v, const int* part_i, int n_parts, int* ctl, int* hist,
                       int* out_tokens, const float* embed, int dm, float* x, hipStream_t s);
size_t sample_scratch_bytes(int V);
hipError_t launch_sample(float* logits, int V, float temp, float min_p, float top_p, int top_k,
                         uint64_t* rng_state, void* scratch, const float* pmax, int npart,
                         int* ctl, int* hist, int* out_tokens, const float* embed, int dm,
                         float* x, hipStream_t s, bool gated = false);

}  // namespace bm

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct Layer {
  float *in_norm, *conv_wt, *conv_b, *dt_bias, *A, *D, *out_norm;
  uint8_t *in_proj, *out_proj;
  float in_scale, out_scale;
};

}  // namespace

struct bm_hip_model {
  int vocab = 0, dm = 0, nl = 0, nh = 0, di = 0, hd = 0, pd = 0;
  hipStream_t stream = nullptr;
  void* arena = nullptr;  // every weight, 256-byte aligned sub-buffers
  size_t arena_bytes = 0;
  float* embed = nullptr;
  float *norm_f = nullptr, *lm_norm = nullptr;
  uint8_t* lm_head = nullptr;
  float lm_scale = 1.0f;
  std::vector<Layer> L;
  // state
  float *conv_state = nullptr, *ssm_state = nullptr;
  int *ctl = nullptr, *hist = nullptr, *out_tokens = nullptr;
  int out_cap = 0;
  // decode scratch
  float *x = nullptr, *proj = nullptr, *y = nullptr, *feat = nullptr, *logits = nullptr;
  float* part_v = nullptr;  // per-block greedy candidates of the LM head
  int* part_i = nullptr;
  int lm_blocks = 0;
  float* scale = nullptr;
  uint8_t* act = nullptr;
  int8_t* xq = nullptr;
  // prefill scratch (grow on demand)
  float *px = nullptr, *pproj = nullptr, *py = nullptr, *pscale = nullptr;
  float* ppre = nullptr;  // prefill SSM phase-1 values of a chunk (pre_layout)
  uint8_t* pact = nullptr;
  int8_t* pxq = nullptr;
  int* ptok = nullptr;
  int pcap = 0;
  // sampler (src/model.c:132-361): temp < 0.05 is greedy
  float temp = 0.0f, min_p = 0.0f, top_p = 1.0f;
  int top_k = 0;
  uint64_t* rng = nullptr;      // XorShift64* state (src/utils.c:117-134)
  void* samp_scratch = nullptr;
  // captured decode step, and kGraphSteps of them in one graph
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph_n = nullptr;
  hipGraphExec_t exec_n = nullptr;
  float graph_penalty = 1.0f;
  bool graph_with_out = false;
  float graph_samp[4] = {0.0f, 0.0f, 1.0f, 0.0f};
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // BM_HIP_NO_GRAPH=1: enqueue each step's kernels directly instead of
  // replaying the captured graph (for tools that cannot trace graphs)
  bool no_graph = false;
  // fast mode (bm_hip_model_set_fast): sums of squares as a pairwise tree
  bool fast = false, graph_fast = false;
  // the step graph of a generate with stop_on_eos: its kernels read the
  // done word (CTL_DONE) and change nothing once the end token is picked
  bool gated = false, graph_gated = false;
};

namespace {

#define MCHECK(expr)                                                                     \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess) {                                                              \
      bm_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,       \
                   __LINE__);                                                            \
      return -1;                                                                         \
    }                                                                                    \
  } while (0)

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// quantize + product of one BitLinear on M rows (src/kernel.c:346-448)
int bitlinear(bm_hip_model* m, const float* x, int M, int K, const float* norm,
              const uint8_t* W, int N, float scale, void* out, int mode, uint8_t* act,
              float* sc, int8_t* xq, hipStream_t s) {
  const bool generic = bm::product_needs_generic(M, K);
  MCHECK(bm::launch_quantize(x, M, K, K, norm, nullptr, generic ? xq : nullptr, K, sc,
                             generic ? nullptr : act, s, bm::product_reads_nibbles(M, N, K),
                             m->fast));
  if (generic)
    MCHECK(bm::launch_generic(xq, K, sc, M, W, N, K, scale, out, mode, s));
  else
    MCHECK(bm::launch_product(act, sc, M, W, N, K, scale, true, out, mode, s));
  return 0;
}


// The kernels of one decode step, enqueued on s.  m->x already holds the
// embedding of the current token.  Widths the fused row kernels do not cover
// (d_model % 64 != 0, more than 8192 columns) take the generic quantize +
// product kernels instead, with the same results.
int enqueue_step(bm_hip_model* m, hipStream_t s, float penalty, bool write_out) {
  const int dm = m->dm, di = m->di;
  const bool rows_dm = bm::rows_fit(dm), rows_di = bm::rows_fit(di);
  for (int l = 0; l < m->nl; ++l) {
    const Layer& Ly = m->L[l];
    float* cs = m->conv_state + (size_t)l * 3 * di;
    float* ss = m->ssm_state + (size_t)l * di;
    // block_step, unfused branch (src/block.c:361-371), then the residual
    if (bm::inproj_ssm_fits(dm, m->hd)) {
      MCHECK(bm::launch_inproj_ssm(m->x, dm, Ly.in_norm, Ly.in_proj, Ly.in_scale, m->nh, m->hd,
                                   Ly.dt_bias, Ly.A, Ly.conv_wt, Ly.conv_b, cs, ss, Ly.D, m->y,
                                   m->ctl, s, m->fast, m->gated));
    } else {
      if (rows_dm) {
        MCHECK(bm::launch_inproj(m->x, dm, Ly.in_norm, Ly.in_proj, m->pd, Ly.in_scale, m->proj,
                                 s, m->fast));
      } else if (bitlinear(m, m->x, 1, dm, Ly.in_norm, Ly.in_proj, m->pd, Ly.in_scale, m->proj,
                           bm::MODE_STORE, m->act, m->scale, m->xq, s)) {
        return -1;
      }
      MCHECK(bm::launch_ssm_heads(m->proj, m->nh, m->hd, Ly.dt_bias, Ly.A, Ly.conv_wt,
                                  Ly.conv_b, cs, ss, Ly.D, m->y, m->ctl, s));
    }
    if (rows_di) {
      MCHECK(bm::launch_outproj(m->y, di, Ly.out_norm, Ly.out_proj, dm, Ly.out_scale, m->x, s,
                                m->fast));
    } else if (bitlinear(m, m->y, 1, di, Ly.out_norm, Ly.out_proj, dm, Ly.out_scale, m->x,
                         bm::MODE_ACC, m->act, m->scale, m->xq, s)) {
      return -1;
    }
  }
  const bool sampled = !(m->temp < 0.05f);  // src/model.c:143-144
  // the fused LM head: greedy candidates per block, or (sampled without a
  // penalty) logits x 1/temp with the blocks' maxima
  const bool fused_pick = rows_dm && penalty == 1.0f && !sampled;  // x / 1.0f == x * 1.0f == x
  const bool fused_scale = rows_dm && penalty == 1.0f && sampled;
  if (rows_dm) {
    MCHECK(bm::launch_lm_head(m->x, dm, m->norm_f, m->lm_norm, m->lm_head, m->vocab,
                              m->lm_scale, m->logits, fused_pick ? 1 : (fused_scale ? 2 : 0),
                              m->temp, m->part_v, m->part_i, s, m->fast,
                              m->gated ? m->ctl + bm::CTL_DONE : nullptr));
  } else {
    // rms_norm(norm_f), then BitLinear with lm_head.norm (src/model.c:1225, 1259-1261)
    MCHECK(bm::launch_rms_norm(m->x, dm, m->norm_f, m->feat, m->scale + 8, s));
    if (bitlinear(m, m->feat, 1, dm, m->lm_norm, m->lm_head, m->vocab, m->lm_scale, m->logits,
                  bm::MODE_STORE, m->act, m->scale, m->xq, s))
      return -1;
  }
  int* out = write_out ? m->out_tokens : nullptr;
  if (sampled) {
    if (penalty != 1.0f) {
      hipLaunchKernelGGL(bm::k_penalty, dim3(1), dim3(bm::kHistory), 0, s, m->logits, m->vocab,
                         m->hist, m->ctl, penalty);
      MCHECK(hipGetLastError());
    }
    MCHECK(bm::launch_sample(m->logits, m->vocab, m->temp, m->min_p, m->top_p, m->top_k, m->rng,
                             m->samp_scratch, fused_scale ? m->part_v : nullptr,
                             fused_scale ? m->lm_blocks : 0, m->ctl, m->hist, out, m->embed, dm,
                             m->x, s, m->gated));
  } else if (fused_pick) {
    MCHECK(bm::launch_pick(m->part_v, m->part_i, m->lm_blocks, m->ctl, m->hist, out, m->embed, dm,
                           m->x, s));
  } else {
    hipLaunchKernelGGL(bm::k_penalty, dim3(1), dim3(bm::kHistory), 0, s, m->logits, m->vocab,
                       m->hist, m->ctl, penalty);
    MCHECK(hipGetLastError());
    hipLaunchKernelGGL(bm::k_argmax_step, dim3(1), dim3(1024), 0, s, m->logits, m->vocab, m->ctl,
                       m->hist, out);
    MCHECK(hipGetLastError());
    hipLaunchKernelGGL(bm::k_embed, dim3((dm + 255) / 256, 1), dim3(256), 0, s, m->embed, dm,
                       m->vocab, m->ctl + bm::CTL_TOKEN, m->x);
    MCHECK(hipGetLastError());
  }
  return 0;
}

void drop_graphs(bm_hip_model* m) {
  if (m->exec) (void)hipGraphExecDestroy(m->exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  if (m->exec_n) (void)hipGraphExecDestroy(m->exec_n);
  if (m->graph_n) (void)hipGraphDestroy(m->graph_n);
  m->exec = m->exec_n = nullptr;
  m->graph = m->graph_n = nullptr;
}

// decode steps per replay of the multi-step graph: one graph launch per
// kGraphSteps tokens instead of one per token (every step reads its
// position, token and counters from the control block on the device, so
// replaying this graph equals kGraphSteps replays of the one-step graph)
constexpr int kGraphSteps = 8;

int ensure_graph(bm_hip_model* m, float penalty, bool write_out) {
  if (m->no_graph) {
    m->graph_penalty = penalty;
    m->graph_with_out = write_out;
    return 0;
  }
  const float samp[4] = {m->temp, m->min_p, m->top_p, (float)m->top_k};
  if (m->exec && m->graph_penalty == penalty && m->graph_with_out == write_out &&
      m->graph_fast == m->fast && m->graph_gated == m->gated &&
      memcmp(samp, m->graph_samp, sizeof(samp)) == 0)
    return 0;
  drop_graphs(m);
  for (int multi = 0; multi < 2; ++multi) {
    MCHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = 0;
    for (int i = 0; i < (multi ? kGraphSteps : 1) && rc == 0; ++i)
      rc = enqueue_step(m, m->stream, penalty, write_out);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc != 0) {
      if (g) (void)hipGraphDestroy(g);
      drop_graphs(m);
      return -1;
    }
    MCHECK(e);
    (multi ? m->graph_n : m->graph) = g;
    MCHECK(hipGraphInstantiate(multi ? &m->exec_n : &m->exec, g, nullptr, nullptr, 0));
  }
  m->graph_penalty = penalty;
  m->graph_with_out = write_out;
  m->graph_fast = m->fast;
  m->graph_gated = m->gated;
  memcpy(m->graph_samp, samp, sizeof(samp));
  return 0;
}

int ensure_prefill(bm_hip_model* m, int n) {
  if (n <= m->pcap) return 0;
  // free the old buffers and forget them first, so that a failed
  // allocation below leaves no stale pointer and no capacity behind
  m->pcap = 0;
  for (void** p : {(void**)&m->px, (void**)&m->pproj, (void**)&m->py, (void**)&m->pscale,
                   (void**)&m->pact, (void**)&m->pxq, (void**)&m->ptok, (void**)&m->ppre}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  const size_t K = (size_t)(m->di > m->dm ? m->di : m->dm);
  MCHECK(hipMalloc(&m->px, (size_t)n * m->dm * 4));
  MCHECK(hipMalloc(&m->pproj, (size_t)n * m->pd * 4));
  MCHECK(hipMalloc(&m->py, (size_t)n * m->di * 4));
  MCHECK(hipMalloc(&m->pscale, (size_t)n * 4));
  MCHECK(hipMalloc(&m->pact, (size_t)n * bm::act_row_bytes((int)K)));
  MCHECK(hipMalloc(&m->pxq, (size_t)n * K));
  MCHECK(hipMalloc(&m->ptok, (size_t)n * 4));
  MCHECK(hipMalloc(&m->ppre,
                   bm::pre_layout(n < bm::kSsmChunk ? n : bm::kSsmChunk, m->di, m->nh).total * 4));
  m->pcap = n;  // only once every buffer exists
  return 0;
}

void model_release(bm_hip_model* m) {
  if (!m) return;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  drop_graphs(m);
  for (void* p : {(void*)m->arena, (void*)m->conv_state, (void*)m->ssm_state, (void*)m->ctl,
                  (void*)m->hist, (void*)m->out_tokens, (void*)m->x, (void*)m->proj,
                  (void*)m->y, (void*)m->feat, (void*)m->logits, (void*)m->scale,
                  (void*)m->part_v, (void*)m->part_i, (void*)m->rng, m->samp_scratch,
                  (void*)m->act, (void*)m->xq, (void*)m->px, (void*)m->pproj, (void*)m->py,
                  (void*)m->pscale, (void*)m->pact, (void*)m->pxq, (void*)m->ptok,
                  (void*)m->ppre})
    if (p) (void)hipFree(p);
  if (m->ev0) (void)hipEventDestroy(m->ev0);
  if (m->ev1) (void)hipEventDestroy(m->ev1);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int load_into(bm_hip_model* m, const bm_bit2_view_t& v) {
  m->vocab = v.vocab;
  m->dm = v.d_model;
  m->nl = v.n_layers;
  m->nh = v.n_heads;
  m->di = 2 * v.d_model;
  m->hd = m->di / m->nh;
  m->pd = 2 * m->di + 3 * m->nh;
  const int dm = m->dm, di = m->di, nh = m->nh;
  MCHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  const char* ng = getenv("BM_HIP_NO_GRAPH");
  m->no_graph = ng && ng[0] == '1';
  MCHECK(hipEventCreate(&m->ev0));
  MCHECK(hipEventCreate(&m->ev1));

  // arena layout
  auto packed_bytes = [](const bm_bit2_tensor_t* t) {
    return (size_t)t->rows * (size_t)((t->cols + 3) / 4);
  };
  size_t total = up256((size_t)m->vocab * dm * 4) + 2 * up256((size_t)dm * 4) +
                 up256(packed_bytes(&v.tensors[v.n_tensors - 1]));
  for (int l = 0; l < m->nl; ++l) {
    total += up256(packed_bytes(bm_bit2_layer(&v, l, BM_L_IN_PROJ))) +
             up256(packed_bytes(bm_bit2_layer(&v, l, BM_L_OUT_PROJ)));
    total += up256((size_t)dm * 4) + up256((size_t)4 * di * 4) + 3 * up256((size_t)di * 4) +
             2 * up256((size_t)nh * 4) + up256((size_t)di * 4);
  }
  total += up256((size_t)nh * 4);  // A_log staging
  MCHECK(hipMalloc(&m->arena, total));
  m->arena_bytes = total;
  uint8_t* cur = (uint8_t*)m->arena;
  auto take = [&](size_t bytes) {
    uint8_t* p = cur;
    cur += up256(bytes);
    return p;
  };
  auto put_f = [&](const bm_bit2_tensor_t* t, size_t count) -> float* {
    float* d = (float*)take(count * 4);
    if (bm::upload(d, t->data, count * 4, m->stream) != hipSuccess) return nullptr;
    return d;
  };
  auto put_w = [&](const bm_bit2_tensor_t* t) -> uint8_t* {
    const size_t b = packed_bytes(t);
    uint8_t* d = take(b);
    if (bm::upload(d, t->packed, b, m->stream) != hipSuccess) return nullptr;
    if (bm::launch_canonicalize(d, b, m->stream) != hipSuccess) return nullptr;
    return d;
  };
  // in_proj rows regrouped per head: [z_h | x_h | B_h | C_h | dt_h] (the
  // reference's order is [z | x | B | C | dt], src/block.c:54-58)
  std::vector<uint8_t> perm;
  auto put_w_heads = [&](const bm_bit2_tensor_t* t) -> uint8_t* {
    const size_t rb = (size_t)((t->cols + 3) / 4);
    perm.resize((size_t)t->rows * rb);
    const int hd = m->hd, rows_h = 2 * hd + 3;
    for (int h = 0; h < nh; ++h) {
      uint8_t* dst = perm.data() + (size_t)h * rows_h * rb;
      memcpy(dst, t->packed + (size_t)h * hd * rb, hd * rb);
      memcpy(dst + hd * rb, t->packed + (size_t)(di + h * hd) * rb, hd * rb);
      memcpy(dst + 2 * hd * rb, t->packed + (size_t)(2 * di + h) * rb, rb);
      memcpy(dst + (2 * hd + 1) * rb, t->packed + (size_t)(2 * di + nh + h) * rb, rb);
      memcpy(dst + (2 * hd + 2) * rb, t->packed + (size_t)(2 * di + 2 * nh + h) * rb, rb);
    }
    uint8_t* d = take(perm.size());
    if (bm::upload(d, perm.data(), perm.size(), m->stream) != hipSuccess) return nullptr;
    if (bm::launch_canonicalize(d, perm.size(), m->stream) != hipSuccess) return nullptr;
    if (hipStreamSynchronize(m->stream) != hipSuccess) return nullptr;
    return d;
  };
  m->embed = put_f(&v.tensors[0], (size_t)m->vocab * dm);
  const bm_bit2_tensor_t* fin = &v.tensors[1 + BM_L_COUNT * m->nl];
  m->norm_f = put_f(&fin[0], dm);
  m->lm_norm = put_f(&fin[1], dm);
  m->lm_head = put_w(&fin[2]);
  m->lm_scale = fin[2].scale;
  if (!m->embed || !m->norm_f || !m->lm_norm || !m->lm_head) {
    bm_set_error("upload failed");
    return -1;
  }
  float* alog = (float*)take((size_t)nh * 4);
  std::vector<float> wt((size_t)4 * di);
  m->L.resize(m->nl);
  for (int l = 0; l < m->nl; ++l) {
    Layer& Ly = m->L[l];
    const bm_bit2_tensor_t* t = bm_bit2_layer(&v, l, 0);
    Ly.in_norm = put_f(&t[BM_L_IN_NORM], dm);
    Ly.in_proj = put_w_heads(&t[BM_L_IN_PROJ]);
    Ly.in_scale = t[BM_L_IN_PROJ].scale;
    // conv1d weight [channel][tap] -> [tap][channel] (src/model.c:794-805)
    for (int tap = 0; tap < 4; ++tap)
      for (int ch = 0; ch < di; ++ch) {
        float w;
        memcpy(&w, (const uint8_t*)t[BM_L_CONV_W].data + ((size_t)ch * 4 + tap) * 4, 4);
        wt[(size_t)tap * di + ch] = w;
      }
    Ly.conv_wt = (float*)take((size_t)4 * di * 4);
    MCHECK(hipMemcpy(Ly.conv_wt, wt.data(), (size_t)4 * di * 4, hipMemcpyHostToDevice));
    Ly.conv_b = put_f(&t[BM_L_CONV_B], di);
    Ly.dt_bias = put_f(&t[BM_L_DT_BIAS], nh);
    MCHECK(bm::upload(alog, t[BM_L_A_LOG].data, (size_t)nh * 4, m->stream));
    Ly.A = (float*)take((size_t)nh * 4);
    hipLaunchKernelGGL(bm::k_neg_exp, dim3((nh + 255) / 256), dim3(256), 0, m->stream, alog,
                       Ly.A, nh);
    MCHECK(hipGetLastError());
    MCHECK(hipStreamSynchronize(m->stream));
    Ly.D = put_f(&t[BM_L_D], di);
    Ly.out_norm = put_f(&t[BM_L_OUT_NORM], di);
    Ly.out_proj = put_w(&t[BM_L_OUT_PROJ]);
    Ly.out_scale = t[BM_L_OUT_PROJ].scale;
    if (!Ly.in_norm || !Ly.in_proj || !Ly.conv_b || !Ly.dt_bias || !Ly.D || !Ly.out_norm ||
        !Ly.out_proj) {
      bm_set_error("upload failed");
      return -1;
    }
  }
  // state + scratch
  MCHECK(hipMalloc(&m->conv_state, (size_t)m->nl * 3 * di * 4));
  MCHECK(hipMalloc(&m->ssm_state, (size_t)m->nl * di * 4));
  MCHECK(hipMemset(m->conv_state, 0, (size_t)m->nl * 3 * di * 4));
  MCHECK(hipMemset(m->ssm_state, 0, (size_t)m->nl * di * 4));
  MCHECK(hipMalloc(&m->ctl, bm::CTL_WORDS * 4));
  MCHECK(hipMemset(m->ctl, 0, bm::CTL_WORDS * 4));
  MCHECK(hipMalloc(&m->hist, bm::kHistory * 4));
  MCHECK(hipMemset(m->hist, 0, bm::kHistory * 4));
  MCHECK(hipMalloc(&m->x, (size_t)dm * 4));
  MCHECK(hipMalloc(&m->proj, (size_t)m->pd * 4));
  MCHECK(hipMalloc(&m->y, (size_t)di * 4));
  MCHECK(hipMalloc(&m->feat, (size_t)dm * 4));
  MCHECK(hipMalloc(&m->logits, (size_t)m->vocab * 4));
  m->lm_blocks = bm::lm_head_blocks(m->vocab, dm);
  MCHECK(hipMalloc(&m->part_v, (size_t)m->lm_blocks * 4));
  MCHECK(hipMalloc(&m->part_i, (size_t)m->lm_blocks * 4));
  MCHECK(hipMalloc(&m->scale, 64));
  MCHECK(hipMalloc(&m->rng, sizeof(uint64_t)));
  {
    const uint64_t seed0 = 0x853c49e6748fea9bULL;  // src/utils.c:119
    MCHECK(hipMemcpy(m->rng, &seed0, sizeof(seed0), hipMemcpyHostToDevice));
  }
  MCHECK(hipMalloc(&m->samp_scratch, bm::sample_scratch_bytes(m->vocab)));
  // the sampler's histogram and block counter start cleared
  MCHECK(hipMemset(m->samp_scratch, 0, bm::sample_scratch_bytes(m->vocab)));
  MCHECK(hipMalloc(&m->act, bm::act_row_bytes(di > dm ? di : dm)));
  MCHECK(hipMalloc(&m->xq, (size_t)(di > dm ? di : dm)));
  MCHECK(hipDeviceSynchronize());
  return 0;
}

int set_ctl(bm_hip_model* m, int token, const int* history, int history_len, int done = 0) {
  int h[bm::kHistory];
  const int len = history_len < bm::kHistory ? history_len : bm::kHistory;
  for (int j = 0; j < len; ++j) h[j] = history[history_len - len + j];
  int ctl[bm::CTL_WORDS];
  MCHECK(hipMemcpyAsync(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost, m->stream));
  MCHECK(hipStreamSynchronize(m->stream));
  ctl[bm::CTL_TOKEN] = token;
  ctl[bm::CTL_STEP] = 0;
  ctl[bm::CTL_HCOUNT] = len;
  ctl[bm::CTL_DONE] = done;
  MCHECK(hipMemcpyAsync(m->ctl, ctl, sizeof(ctl), hipMemcpyHostToDevice, m->stream));
  if (len) MCHECK(hipMemcpyAsync(m->hist, h, (size_t)len * 4, hipMemcpyHostToDevice, m->stream));
  hipLaunchKernelGGL(bm::k_embed, dim3((m->dm + 255) / 256, 1), dim3(256), 0, m->stream,
                     m->embed, m->dm, m->vocab, m->ctl + bm::CTL_TOKEN, m->x);
  MCHECK(hipGetLastError());
  MCHECK(hipStreamSynchronize(m->stream));
  return 0;
}

// the step graphs write the picked tokens here: room for at least 4096
// (16 KB), so that a longer generation than the first one does not have to
// capture the graphs again
int ensure_out(bm_hip_model* m, int n) {
  if (n <= m->out_cap) return 0;
  if (m->out_tokens) (void)hipFree(m->out_tokens);
  m->out_tokens = nullptr;
  m->out_cap = 0;
  drop_graphs(m);  // the captured graphs refer to the old buffer
  const int cap = n > 4096 ? n : 4096;
  MCHECK(hipMalloc(&m->out_tokens, (size_t)cap * 4));
  m->out_cap = cap;
  return 0;
}

// n_steps decode steps back to back on the model stream, timed with events
int run_steps(bm_hip_model* m, int n_steps, double* decode_ms) {
  MCHECK(hipEventRecord(m->ev0, m->stream));
  int i = 0;
  if (!m->no_graph)
    for (; i + kGraphSteps <= n_steps; i += kGraphSteps) MCHECK(hipGraphLaunch(m->exec_n, m->stream));
  for (; i < n_steps; ++i) {
    if (m->no_graph) {
      if (enqueue_step(m, m->stream, m->graph_penalty, m->graph_with_out)) return -1;
    } else {
      MCHECK(hipGraphLaunch(m->exec, m->stream));
    }
  }
  MCHECK(hipEventRecord(m->ev1, m->stream));
  MCHECK(hipEventSynchronize(m->ev1));
  float ms = 0.0f;
  MCHECK(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  if (decode_ms) *decode_ms = ms;
  return 0;
}

}  // namespace

extern "C" bm_hip_model_t* bm_hip_model_load(const void* image, size_t size) {
  if (!bm_hip_init()) return nullptr;
  bm_bit2_view_t v;
  const int rc = bm_bit2_parse(image, size, &v);
  if (rc != 0) {
    bm_set_error(rc == -1 ? "malformed BIT2 image" : "BIT2 shapes rejected by the loader");
    return nullptr;
  }
  bm_hip_model* m = new bm_hip_model();
  const int ok = load_into(m, v);
  bm_bit2_view_free(&v);
  if (ok != 0) {
    model_release(m);
    return nullptr;
  }
  return m;
}

extern "C" void bm_hip_model_free(bm_hip_model_t* m) { model_release(m); }

extern "C" int bm_hip_model_config(const bm_hip_model_t* m, int which) {
  switch (which) {
    case 0: return m->vocab;
    case 1: return m->dm;
    case 2: return m->nl;
    case 3: return m->nh;
    default: return m->di;
  }
}

extern "C" int bm_hip_model_reset(bm_hip_model_t* m) {
  MCHECK(hipMemsetAsync(m->conv_state, 0, (size_t)m->nl * 3 * m->di * 4, m->stream));
  MCHECK(hipMemsetAsync(m->ssm_state, 0, (size_t)m->nl * m->di * 4, m->stream));
  MCHECK(hipMemsetAsync(m->ctl, 0, bm::CTL_WORDS * 4, m->stream));
  MCHECK(hipStreamSynchronize(m->stream));
  return 0;
}

extern "C" int bm_hip_model_prefill(bm_hip_model_t* m, const int32_t* tokens, int n) {
  if (n <= 0) return 0;
  if (ensure_prefill(m, n)) return -1;
  hipStream_t s = m->stream;
  const int dm = m->dm, di = m->di;
  MCHECK(hipMemcpyAsync(m->ptok, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s));
  hipLaunchKernelGGL(bm::k_embed, dim3((dm + 255) / 256, n), dim3(256), 0, s, m->embed, dm,
                     m->vocab, m->ptok, m->px);
  MCHECK(hipGetLastError());
  for (int l = 0; l < m->nl; ++l) {
    const Layer& Ly = m->L[l];
    // block_step_batch (src/block.c:378-447): batched in_proj, the SSM in
    // three phases per chunk of tokens (k_ssm_prep, k_ssm_scan, k_ssm_out),
    // batched out_proj, then x += out (src/model.c:1139-1142)
    if (bitlinear(m, m->px, n, dm, Ly.in_norm, Ly.in_proj, m->pd, Ly.in_scale, m->pproj,
                  bm::MODE_STORE, m->pact, m->pscale, m->pxq, s))
      return -1;
    float* cs = m->conv_state + (size_t)l * 3 * di;
    for (int t0 = 0; t0 < n; t0 += bm::kSsmChunk) {
      const int nt = n - t0 < bm::kSsmChunk ? n - t0 : bm::kSsmChunk;
      const bm::PreLayout PL = bm::pre_layout(nt, di, m->nh);
      hipLaunchKernelGGL(bm::k_ssm_prep, dim3((di + 255) / 256, PL.nqr), dim3(256), 0, s,
                         m->pproj, m->pd, t0, nt, di, m->nh, m->hd, Ly.dt_bias, Ly.A,
                         Ly.conv_wt, Ly.conv_b, cs, Ly.D, m->ctl, m->ppre);
      MCHECK(hipGetLastError());
      auto scan = bm::scan_q(PL.nq) == bm::kScanQ ? bm::k_ssm_scan<bm::kScanQ>
                                                  : bm::k_ssm_scan<bm::kScanQSmall>;
      hipLaunchKernelGGL(scan, dim3((di + 63) / 64), dim3(64), 0, s, m->ppre, nt, di, m->nh,
                         m->ssm_state + (size_t)l * di, m->pproj, m->pd, m->hd, cs, m->ctl,
                         t0 + nt == n ? n : 0);
      MCHECK(hipGetLastError());
      hipLaunchKernelGGL(bm::k_ssm_out, dim3((di + 255) / 256, PL.nq), dim3(256), 0, s, m->ppre,
                         m->pproj, m->pd, t0, nt, di, m->nh, m->hd, m->py);
      MCHECK(hipGetLastError());
    }
    if (bitlinear(m, m->py, n, di, Ly.out_norm, Ly.out_proj, dm, Ly.out_scale, m->px,
                  bm::MODE_ACC, m->pact, m->pscale, m->pxq, s))
      return -1;
  }
  hipLaunchKernelGGL(bm::k_advance_pos, dim3(1), dim3(64), 0, s, m->ctl, n);
  MCHECK(hipGetLastError());
  MCHECK(hipStreamSynchronize(s));
  return 0;
}

extern "C" int bm_hip_model_step(bm_hip_model_t* m, int token, const int* history,
                                 int history_len, float penalty) {
  if (token < 0 || token >= m->vocab) return 0;  // src/model.c:1188-1193
  m->gated = false;
  if (set_ctl(m, token, history, history_len)) return -1;
  if (enqueue_step(m, m->stream, penalty, false)) return -1;
  int ctl[bm::CTL_WORDS];
  MCHECK(hipMemcpyAsync(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost, m->stream));
  MCHECK(hipStreamSynchronize(m->stream));
  return ctl[bm::CTL_TOKEN];
}

extern "C" int bm_hip_model_set_sampler(bm_hip_model_t* m, float temp, float min_p, float top_p,
                                        int top_k) {
  m->temp = temp;
  m->min_p = min_p;
  m->top_p = top_p;
  m->top_k = top_k;
  return 0;
}

extern "C" int bm_hip_model_set_fast(bm_hip_model_t* m, int on) {
  m->fast = on != 0;
  return 0;
}

// One kernel of the decode step launched `reps` times back to back on the
// model's stream, timed with events on that stream: which 0 = layer's
// in_proj + SSM step, 1 = layer's out_proj (+ residual), 2 = the LM head
// (greedy candidates).  Changes the recurrent state and the activations.
extern "C" int bm_hip_model_time_kernel(bm_hip_model_t* m, int which, int layer, int reps,
                                        float* avg_us) {
  if (!m || !avg_us || reps < 1 || which < 0 || which > 2 || layer < -1 || layer >= m->nl) {
    bm_set_error("bm_hip_model_time_kernel: bad arguments");
    return -1;
  }
  const int dm = m->dm, di = m->di;
  if (!bm::inproj_ssm_fits(dm, m->hd) || !bm::rows_fit(di) || !bm::rows_fit(dm)) {
    bm_set_error("bm_hip_model_time_kernel: the model's widths take the generic kernels");
    return -1;
  }
  hipStream_t s = m->stream;
  int next = 0;  // layer == -1: the layers in turn, as a decode step reads them
  auto launch = [&]() -> hipError_t {
    const int li = layer >= 0 ? layer : next;
    next = next + 1 == m->nl ? 0 : next + 1;
    const Layer& Ly = m->L[li];
    float* cs = m->conv_state + (size_t)li * 3 * di;
    float* ss = m->ssm_state + (size_t)li * di;
    if (which == 0)
      return bm::launch_inproj_ssm(m->x, dm, Ly.in_norm, Ly.in_proj, Ly.in_scale, m->nh, m->hd,
                                   Ly.dt_bias, Ly.A, Ly.conv_wt, Ly.conv_b, cs, ss, Ly.D, m->y,
                                   m->ctl, s, m->fast);
    if (which == 1)
      return bm::launch_outproj(m->y, di, Ly.out_norm, Ly.out_proj, dm, Ly.out_scale, m->x, s,
                                m->fast);
    return bm::launch_lm_head(m->x, dm, m->norm_f, m->lm_norm, m->lm_head, m->vocab, m->lm_scale,
                              m->logits, 1, m->temp, m->part_v, m->part_i, s, m->fast);
  };
  hipEvent_t e0 = nullptr, e1 = nullptr;
  MCHECK(hipEventCreate(&e0));
  MCHECK(hipEventCreate(&e1));
  hipError_t e = launch();
  if (e == hipSuccess) e = launch();  // warm
  if (e == hipSuccess) e = hipEventRecord(e0, s);
  for (int i = 0; i < reps && e == hipSuccess; ++i) e = launch();
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  MCHECK(e);
  *avg_us = ms * 1000.0f / (float)reps;
  return 0;
}

extern "C" int bm_hip_model_seed(bm_hip_model_t* m, uint64_t seed) {
  const uint64_t s = seed ? seed : 0x853c49e6748fea9bULL;  // rng_seed (src/utils.c:121-124)
  MCHECK(hipMemcpyAsync(m->rng, &s, sizeof(s), hipMemcpyHostToDevice, m->stream));
  MCHECK(hipStreamSynchronize(m->stream));
  return 0;
}

// --- recurrent state files (state_save / state_load, src/chat.c:1160-1271) ---
// BMST image: u32 magic "BMST", n_layers, d_inner, d_conv; then per layer
// conv_state [(d_conv-1) * d_inner] floats, ssm_state [d_inner] floats and
// the int conv_pos.  The device model keeps one ring position for all
// layers (they advance together), so an image whose layers disagree on it is
// rejected.
namespace {
constexpr uint32_t kStateMagic = 0x424D5354;  // src/chat.h:14-15
constexpr int kDConv = 4;                     // BM_CONV_KERNEL
}  // namespace

extern "C" size_t bm_hip_model_state_bytes(const bm_hip_model_t* m) {
  return 16 + (size_t)m->nl * ((size_t)(kDConv - 1) * m->di * 4 + (size_t)m->di * 4 + 4);
}

extern "C" int bm_hip_model_state_save(const bm_hip_model_t* m, void* out, size_t len) {
  const size_t need = bm_hip_model_state_bytes(m);
  if (!out || len < need) {
    bm_set_error("state_save: buffer of %zu bytes, %zu needed", len, need);
    return -1;
  }
  const size_t conv = (size_t)(kDConv - 1) * m->di, lay = conv * 4 + (size_t)m->di * 4 + 4;
  std::vector<float> cs((size_t)m->nl * conv), ss((size_t)m->nl * m->di);
  int ctl[bm::CTL_WORDS];
  MCHECK(hipStreamSynchronize(m->stream));
  MCHECK(hipMemcpy(cs.data(), m->conv_state, cs.size() * 4, hipMemcpyDeviceToHost));
  MCHECK(hipMemcpy(ss.data(), m->ssm_state, ss.size() * 4, hipMemcpyDeviceToHost));
  MCHECK(hipMemcpy(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost));
  uint8_t* p = (uint8_t*)out;
  const uint32_t hdr[4] = {kStateMagic, (uint32_t)m->nl, (uint32_t)m->di, (uint32_t)kDConv};
  memcpy(p, hdr, 16);
  for (int l = 0; l < m->nl; ++l) {
    uint8_t* q = p + 16 + (size_t)l * lay;
    memcpy(q, cs.data() + (size_t)l * conv, conv * 4);
    memcpy(q + conv * 4, ss.data() + (size_t)l * m->di, (size_t)m->di * 4);
    memcpy(q + conv * 4 + (size_t)m->di * 4, &ctl[bm::CTL_POS], 4);
  }
  return (int)need;
}

extern "C" int bm_hip_model_state_load(bm_hip_model_t* m, const void* in, size_t len) {
  const uint8_t* p = (const uint8_t*)in;
  uint32_t hdr[4];
  if (!in || len < 16) {
    bm_set_error("state_load: short header");
    return -1;
  }
  memcpy(hdr, p, 16);
  if (hdr[0] != kStateMagic) {
    bm_set_error("state_load: invalid magic");
    return -1;
  }
  if ((int)hdr[1] != m->nl || (int)hdr[2] != m->di || (int)hdr[3] != kDConv) {
    bm_set_error("state_load: dimensions mismatch (layers=%u/%d, d_inner=%u/%d, d_conv=%u/%d)",
                 hdr[1], m->nl, hdr[2], m->di, hdr[3], kDConv);
    return -1;
  }
  const size_t conv = (size_t)(kDConv - 1) * m->di, lay = conv * 4 + (size_t)m->di * 4 + 4;
  std::vector<float> cs((size_t)m->nl * conv), ss((size_t)m->nl * m->di);
  int pos = -1;
  const char* why = nullptr;
  for (int l = 0; l < m->nl && !why; ++l) {
    if (16 + (size_t)(l + 1) * lay > len) {
      why = "truncated";
      break;
    }
    const uint8_t* q = p + 16 + (size_t)l * lay;
    memcpy(cs.data() + (size_t)l * conv, q, conv * 4);
    memcpy(ss.data() + (size_t)l * m->di, q + conv * 4, (size_t)m->di * 4);
    int cp;
    memcpy(&cp, q + conv * 4 + (size_t)m->di * 4, 4);
    if (cp < 0 || cp >= kDConv - 1)
      why = "invalid conv_pos";
    else if (l > 0 && cp != pos)
      why = "layers at different conv positions";
    pos = cp;
  }
  if (why) {
    // the reference resets the state after a bad layer (src/chat.c:1246-1265)
    bm_set_error("state_load: %s", why);
    if (bm_hip_model_reset(m)) return -1;
    return -1;
  }
  int ctl[bm::CTL_WORDS];
  MCHECK(hipStreamSynchronize(m->stream));
  MCHECK(hipMemcpy(m->conv_state, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  MCHECK(hipMemcpy(m->ssm_state, ss.data(), ss.size() * 4, hipMemcpyHostToDevice));
  MCHECK(hipMemcpy(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost));
  ctl[bm::CTL_POS] = pos;
  MCHECK(hipMemcpy(m->ctl, ctl, sizeof(ctl), hipMemcpyHostToDevice));
  return 0;
}

extern "C" int bm_hip_model_logits(const bm_hip_model_t* m, float* out) {
  MCHECK(hipMemcpyAsync(out, m->logits, (size_t)m->vocab * 4, hipMemcpyDeviceToHost, m->stream));
  MCHECK(hipStreamSynchronize(m->stream));
  return 0;
}

extern "C" int bm_hip_model_layer_state(const bm_hip_model_t* m, int layer, float* conv_state,
                                        float* ssm_state) {
  int ctl[bm::CTL_WORDS];
  MCHECK(hipMemcpy(conv_state, m->conv_state + (size_t)layer * 3 * m->di, (size_t)3 * m->di * 4,
                   hipMemcpyDeviceToHost));
  MCHECK(hipMemcpy(ssm_state, m->ssm_state + (size_t)layer * m->di, (size_t)m->di * 4,
                   hipMemcpyDeviceToHost));
  MCHECK(hipMemcpy(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost));
  return ctl[bm::CTL_POS];
}

extern "C" int bm_hip_model_set_layer_state(bm_hip_model_t* m, int layer, const float* conv_state,
                                            const float* ssm_state, int conv_pos) {
  if (layer < 0 || layer >= m->nl || conv_pos < 0 || conv_pos > 2 || !conv_state || !ssm_state) {
    bm_set_error("set_layer_state: invalid arguments (layer=%d conv_pos=%d)", layer, conv_pos);
    return -1;
  }
  MCHECK(hipStreamSynchronize(m->stream));
  MCHECK(hipMemcpy(m->conv_state + (size_t)layer * 3 * m->di, conv_state, (size_t)3 * m->di * 4,
                   hipMemcpyHostToDevice));
  MCHECK(hipMemcpy(m->ssm_state + (size_t)layer * m->di, ssm_state, (size_t)m->di * 4,
                   hipMemcpyHostToDevice));
  int ctl[bm::CTL_WORDS];
  MCHECK(hipMemcpy(ctl, m->ctl, sizeof(ctl), hipMemcpyDeviceToHost));
  ctl[bm::CTL_POS] = conv_pos;
  MCHECK(hipMemcpy(m->ctl, ctl, sizeof(ctl), hipMemcpyHostToDevice));
  return 0;
}

extern "C" int bm_hip_model_generate(bm_hip_model_t* m, const int32_t* prompt, int n_prompt,
                                     int n_steps, float penalty, int stop_on_eos,
                                     int32_t* out_tokens, double* decode_ms) {
  if (n_prompt <= 0 || n_steps < 0) {
    bm_set_error("generate: empty prompt");
    return -1;
  }
  // src/main.c:451-500: prefill all but the last prompt token, history =
  // the prompt, then greedy steps from the last prompt token
  if (n_prompt > 1 && bm_hip_model_prefill(m, prompt, n_prompt - 1)) return -1;
  // stop_on_eos: the step that picks the end token is the last that changes
  // anything (src/main.c:498-500), for widths whose every step kernel reads
  // the done word (the fused row kernels); other widths run all n_steps
  const bool fused = bm::inproj_ssm_fits(m->dm, m->hd) && bm::rows_fit(m->di) &&
                     bm::rows_fit(m->dm);
  m->gated = stop_on_eos && fused;
  if (set_ctl(m, prompt[n_prompt - 1], prompt, n_prompt, m->gated ? bm::kDoneArmed : 0))
    return -1;
  if (ensure_out(m, n_steps > 0 ? n_steps : 1)) return -1;
  if (ensure_graph(m, penalty, true)) return -1;
  if (run_steps(m, n_steps, decode_ms)) return -1;
  MCHECK(hipMemcpy(out_tokens, m->out_tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost));
  int n = n_steps;
  if (stop_on_eos)
    for (int i = 0; i < n_steps; ++i)
      if (out_tokens[i] == 50256 || out_tokens[i] == 0) {
        n = i + 1;
        break;
      }
  return n;
}

extern "C" int bm_hip_model_decode(bm_hip_model_t* m, int n_steps, float penalty,
                                   double* decode_ms) {
  // continues from the current device state (token, history, position)
  m->gated = false;
  if (ensure_out(m, n_steps > 0 ? n_steps : 1)) return -1;
  if (ensure_graph(m, penalty, true)) return -1;
  // on the device, in stream order: no host copy of the control words
  hipLaunchKernelGGL(bm::k_restart_steps, dim3(1), dim3(64), 0, m->stream, m->ctl);
  MCHECK(hipGetLastError());
  return run_steps(m, n_steps, decode_ms);
}

extern "C" int bm_hip_model_tokens(const bm_hip_model_t* m, int32_t* out, int n) {
  if (n > m->out_cap) n = m->out_cap;
  MCHECK(hipMemcpy(out, m->out_tokens, (size_t)n * 4, hipMemcpyDeviceToHost));
  return n;
}

// Diagnostic: evaluates the device scalar functions of the SSM path and the
// norms: fn 0 expf, 1 logf, 2 the division of each even/odd pair of inputs
// (both orders: out[i] = in[i] / in[i ^ 1]), 3 silu, 4 sqrt.
namespace bm {
__global__ void k_libm_eval(int fn, const float* __restrict__ in, float* __restrict__ out,
                            size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float v = in[i];
    float r;
    if (fn == 0)
      r = libm::expf_glibc(v);
    else if (fn == 1)
      r = libm::logf_glibc(v);
    else if (fn == 2)
      r = cr_divf(v, in[(i ^ 1) < n ? (i ^ 1) : i]);
    else if (fn == 3)
      r = silu_ref(v);
    else
      r = cr_sqrtf(v);
    out[i] = r;
  }
}
}  // namespace bm

extern "C" int bm_hip_libm_eval_dev(int fn, const float* in, float* out, size_t n, void* stream) {
  if (!bm_hip_init()) return -1;
  if (fn < 0 || fn > 4) {
    bm_set_error("bm_hip_libm_eval_dev: fn must be 0..4");
    return -1;
  }
  int blocks = (int)((n + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(bm::k_libm_eval, dim3(blocks), dim3(256), 0, (hipStream_t)stream, fn, in,
                     out, n);
  MCHECK(hipGetLastError());
  return 0;
}
