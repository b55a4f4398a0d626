// Device sampler: the reference's sample_advanced (src/model.c:132-361) with
// filter_and_sample (src/model.c:67-127) and the XorShift64* generator
// (src/utils.c:117-140), bit for bit.
//
// The O(V) passes are spread over kFront blocks, each owning a contiguous
// segment of the vocabulary:
//   k_samp_scale  temperature scaling in place and the segment's max logit
//                 (or the LM head does both, with its own blocks' maxima);
//   k_samp_hist   with the global max, the 128-bucket histogram (global
//                 atomics of per-block counts) and the segment's
//                 "pre-candidates" in index order: the logits at or above the
//                 lowest threshold the extraction can use (the histogram's
//                 last bucket, or the min_p threshold), a superset of the
//                 candidates.
// k_sample then runs the rest on one 1024-thread block: the cutoff bucket,
// the candidates filtered from the pre-candidate lists in order, selection,
// softmax, sorting and the draw, the step bookkeeping and the next token's
// embedding.  (Pass 2 and this in one kernel, with a block counter and
// device-scope fences handing over to the last block, measured 32 us per
// token against about 14 for the two launches.)
// The steps whose result depends on their order stay sequential on one
// thread, in the reference's order: the heap selections (their array order
// feeds the sums), every double sum, and the CDF walk.  Sorting is stable
// like glibc's qsort (a merge sort for these sizes), keyed on the value.
// Float-to-int bucket indices follow x86 cvttss2si (out of range -> INT_MIN).
#include "bm_common.h"
#include "bm_dev.h"
#include "bm_libm.h"

namespace bm {

struct SampleParams {
  float temp, min_p, top_p;
  int top_k;
};

struct Cand {  // token_prob_t (src/bitmamba.h:98-102)
  int id;
  float val;
};

namespace {

constexpr int kThreads = 1024;
constexpr int kBuckets = 128;      // HIST_BUCKETS (src/model.c:131)
constexpr int kPartial = 256;      // PARTIAL_K (src/model.c:319)
constexpr int kStage = 4096;       // candidates staged in LDS per serial pass
constexpr int kCtlPos = 0, kCtlDone = 1, kCtlStep = 2, kCtlHcount = 3, kCtlToken = 4;
constexpr int kDoneArmed = 1, kDoneStopped = 2;  // the done word (bm_decode.hip)

// a decode stopped at its end token: the front kernels (given the done
// word only in a gated step graph) return at once; k_sample and
// k_sample_greedy skip their stores at the end
__device__ __forceinline__ bool step_stopped(const int* ctl) {
  return ctl && __builtin_amdgcn_readfirstlane(ctl[kCtlDone]) == kDoneStopped;
}
constexpr int kHist = 256;
constexpr int kFront = 64;          // blocks of the O(V) passes (one wave of partials)
constexpr int kFrontThreads = 256;
static_assert(kFront % (kThreads / 64) == 0, "whole pre-candidate lists per wave");
constexpr int kMaxVocab = 256000;  // MAX_VOCAB of the loader (src/bitmamba.h:55)

// vocabulary segment of each front block: a multiple of 4 entries
__host__ __device__ __forceinline__ int front_seg(int V) { return ((V + kFront - 1) / kFront + 3) & ~3; }

// scratch: probs[V], pre[kFront * seg] (also the radix sort's second
// buffer), pmax[kFront], pcnt[kFront], hist[kBuckets].  hist is zero
// between calls: k_samp_scale clears it, and so does k_sample after use.
struct Scratch {
  Cand* probs;
  Cand* pre;
  float* pmax;
  int* pcnt;
  int* hist;
};
__host__ __device__ __forceinline__ Scratch scratch_of(void* base, int V) {
  Scratch s;
  s.probs = (Cand*)base;
  s.pre = s.probs + V;
  s.pmax = (float*)(s.pre + (size_t)kFront * front_seg(V));
  s.pcnt = (int*)(s.pmax + kFront);
  s.hist = s.pcnt + kFront;
  return s;
}

// where the token goes: with ctl, the step bookkeeping of k_argmax_step and
// (with embed) the next token's embedding row into x; without, out_tokens[0]
struct StepIO {
  int* ctl;
  int* hist;
  int* out_tokens;
  const float* embed;
  int dm;
  float* x;
};

constexpr int kCandLds = 512;      // candidates kept in LDS when they fit
constexpr int kListsPerWave = kFront / (kThreads / 64);

struct Smem {
  unsigned radix[16 * kThreads];  // sort_large: per-thread digit counts, then offsets
  Cand stage[kStage];
  Cand cand[kCandLds];
  Cand sel[kPartial];
  Cand sorted[kPartial];
  unsigned scan[kThreads];
  float fred[kThreads / 64];
  int ired[kThreads / 64];
  int iwork[8];
  float fwork[8];
};

__device__ __forceinline__ uint64_t rng_next(uint64_t& s) {
  uint64_t x = s;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  s = x;
  return x * 0x2545F4914F6CDD1DULL;
}

__device__ __forceinline__ float rng_float(uint64_t& s) {
  return __fmul_rn((float)(rng_next(s) >> 11), 1.0f / 9007199254740992.0f);
}

// (int)f as x86-64 cvttss2si computes it
__device__ __forceinline__ int cvtt_x86(float f) {
  return (f >= -2147483648.0f && f < 2147483648.0f) ? (int)f : (int)0x80000000;
}

// max of n partial maxima under `x > m` from -1e30f; called by whole waves
__device__ __forceinline__ float front_max(const float* __restrict__ pmax, int n) {
  const int lane = threadIdx.x & 63;
  float v = -1e30f;
  // the first 8 * 64 maxima in one round of loads (indices clamped,
  // unconditional: loads in the loop would each wait for the one before)
  constexpr int FU = 8;
  float w[FU];
#pragma unroll
  for (int u = 0; u < FU; ++u) w[u] = pmax[min(lane + 64 * u, n - 1)];
#pragma unroll
  for (int u = 0; u < FU; ++u)
    if (lane + 64 * u < n && w[u] > v) v = w[u];
  for (int i = lane + 64 * FU; i < n; i += 64) {
    const float x = pmax[i];
    if (x > v) v = x;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    if (w > v) v = w;
  }
  return __shfl(v, 0, 64);
}

// min_p threshold before the softmax (src/model.c:168-176)
__device__ __forceinline__ float min_p_threshold(float max_logit, float min_p) {
  if (min_p >= 1.0f) return max_logit;
  if (min_p > 0.0f) return __fadd_rn(max_logit, libm::logf_glibc(min_p));
  return -1e30f;
}

__device__ __forceinline__ int effective_k(int top_k) {
  return (top_k > 0 && top_k <= 256) ? top_k : 0;  // src/model.c:168-170
}

__device__ __forceinline__ float bucket_scale_of() {
  return cr_divf((float)(kBuckets - 1), 20.0f);  // src/model.c:182
}

// extraction threshold for a cutoff bucket (src/model.c:208-213).  It does
// not increase with the cutoff, so cutoff kBuckets-1 gives the lowest.
__device__ __forceinline__ float extract_threshold(float max_logit, float min_p_thresh,
                                                   int cutoff) {
  const float bucket_thresh =
      __fsub_rn(max_logit, cr_divf((float)(cutoff + 1), bucket_scale_of()));
  return bucket_thresh > min_p_thresh ? bucket_thresh : min_p_thresh;
}

// p[i..i+3] with zeros at and past `end`; p is 16-byte aligned, i % 4 == 0
__device__ __forceinline__ float4 load4(const float* __restrict__ p, int i, int end) {
  if (i + 4 <= end) return *(const float4*)(p + i);
  float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (i < end) r.x = p[i];
  if (i + 1 < end) r.y = p[i + 1];
  if (i + 2 < end) r.z = p[i + 2];
  return r;
}

__device__ __forceinline__ void heap_sift_down(Cand* h, int n, int i) {
  while (true) {
    int smallest = i;
    const int l = 2 * i + 1, r = 2 * i + 2;
    if (l < n && h[l].val < h[smallest].val) smallest = l;
    if (r < n && h[r].val < h[smallest].val) smallest = r;
    if (smallest == i) break;
    const Cand t = h[i];
    h[i] = h[smallest];
    h[smallest] = t;
    i = smallest;
  }
}

// block-wide max of v under `x > m` from -1e30f (NaN never wins)
__device__ float block_max(float v, Smem& sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    if (w > v) v = w;
  }
  if (lane == 0) sm.fred[wave] = v;
  __syncthreads();
  float m = -1e30f;
  for (int w = 0; w < kThreads / 64; ++w)
    if (sm.fred[w] > m) m = sm.fred[w];
  __syncthreads();
  return m;
}

// exclusive scan of one count per thread; returns this thread's offset,
// total in *total
__device__ unsigned block_scan(unsigned c, Smem& sm, unsigned* total) {
  sm.scan[threadIdx.x] = c;
  __syncthreads();
  for (int o = 1; o < kThreads; o <<= 1) {
    const unsigned add = threadIdx.x >= (unsigned)o ? sm.scan[threadIdx.x - o] : 0u;
    __syncthreads();
    sm.scan[threadIdx.x] += add;
    __syncthreads();
  }
  const unsigned incl = sm.scan[threadIdx.x];
  *total = sm.scan[kThreads - 1];
  __syncthreads();
  return incl - c;
}

// the candidates (i, v) with v >= thr in ascending i, from the front
// blocks' pre-candidate lists (each in index order, the blocks' segments
// ascending; pc: this wave's list lengths).  Wave w takes lists
// kListsPerWave * w .. + kListsPerWave - 1 and writes after the waves before
// it: into sm.cand when they all fit, else to `spill`.  Returns the count,
// the array in *out.
__device__ int gather(const Scratch& sc, const int (&pc)[kListsPerWave], int seg, float thr,
                      Cand* spill, Cand** out, Smem& sm) {
  constexpr int NW = kThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int cnt = 0;
  // the first 64 entries of every list in one round of loads (index 0 of
  // an empty list is in bounds: a segment holds at least 4), kept for the
  // second pass; the rest in turns
  Cand first[kListsPerWave];
#pragma unroll
  for (int j = 0; j < kListsPerWave; ++j)
    first[j] = (sc.pre + (size_t)(wave * kListsPerWave + j) * seg)[min(lane, max(pc[j], 1) - 1)];
#pragma unroll
  for (int j = 0; j < kListsPerWave; ++j) {
    const Cand* src = sc.pre + (size_t)(wave * kListsPerWave + j) * seg;
    cnt += lane < pc[j] && first[j].val >= thr;
    for (int i = lane + 64; i < pc[j]; i += 64) cnt += src[i].val >= thr;
  }
  cnt = wave_sum_i32(cnt);
  if (lane == 0) sm.ired[wave] = cnt;
  __syncthreads();
  int off = 0, total = 0;
  for (int w = 0; w < NW; ++w) {
    const int c = sm.ired[w];
    off += w < wave ? c : 0;
    total += c;
  }
  __syncthreads();
  Cand* dst = total <= kCandLds ? sm.cand : spill;
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int j = 0; j < kListsPerWave; ++j) {
    const Cand* src = sc.pre + (size_t)(wave * kListsPerWave + j) * seg;
    for (int i0 = 0; i0 < pc[j]; i0 += 64) {
      const int i = i0 + lane;
      Cand x{0, 0.0f};
      if (i0 == 0)
        x = first[j];
      else if (i < pc[j])
        x = src[i];
      const bool h = i < pc[j] && x.val >= thr;
      const uint64_t m = __ballot(h);
      if (h) dst[off + __popcll(m & below)] = x;
      off += __popcll(m);
    }
  }
  __syncthreads();
  *out = dst;
  return total;
}

// the sequential scan `best = 0, best_v = init; if (logits[i] > best_v) ...`
// over i = 0 .. V-1: init = logits[0] in the pruned-everything guards
// (src/model.c:225-233, 285-291), -1e9f in the greedy branch
// (src/model.c:144-154).  A later value wins only when strictly greater, so
// NaNs never win.  Returned to every thread.
__device__ int argmax_scan(const float* __restrict__ logits, int V, float init, Smem& sm) {
  float bv = init;
  int bi = 0;
  for (int i = threadIdx.x; i < V; i += kThreads) {
    const float v = logits[i];
    if (v > bv) {  // ascending i per thread: the first maximum stays
      bv = v;
      bi = i;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
    sm.fred[wave] = bv;
    sm.ired[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w)
      if (sm.fred[w] > bv || (sm.fred[w] == bv && sm.ired[w] < bi)) {
        bv = sm.fred[w];
        bi = sm.ired[w];
      }
    sm.iwork[0] = bi;
  }
  __syncthreads();
  const int best = sm.iwork[0];
  __syncthreads();
  return best;
}

// stable descending order of n <= kPartial candidates: src -> dst
__device__ void sort_small(const Cand* src, Cand* dst, int n) {
  const int i = threadIdx.x;
  if (i < n) {
    const float v = src[i].val;
    int r = 0;
    for (int j = 0; j < n; ++j) {
      const float w = src[j].val;
      r += (w > v) || (w == v && j < i);
    }
    dst[r] = src[i];
  }
  __syncthreads();
}

// key of a float for an ascending radix order that puts larger values first
__device__ __forceinline__ uint32_t desc_key(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}

// stable descending sort of n candidates in global memory (LSD radix, 4-bit
// digits, each thread a contiguous run); the result ends in `a`
__device__ void sort_large(Cand* a, Cand* b, int n, Smem& sm) {
  unsigned* cnt = sm.radix;  // [16][kThreads]
  const int per = (n + kThreads - 1) / kThreads;
  const int i0 = threadIdx.x * per, i1 = min(n, i0 + per);
  Cand* src = a;
  Cand* dst = b;
  for (int shift = 0; shift < 32; shift += 4) {
    unsigned c[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) c[d] = 0;
    for (int i = i0; i < i1; ++i) ++c[(desc_key(src[i].val) >> shift) & 15];
#pragma unroll
    for (int d = 0; d < 16; ++d) cnt[d * kThreads + threadIdx.x] = c[d];
    __syncthreads();
    // exclusive offsets in (digit, thread) order: thread t scans its 16
    // entries t*16 .. t*16+15 of the flattened array, then the partials
    unsigned part = 0;
    for (int e = 0; e < 16; ++e) part += cnt[threadIdx.x * 16 + e];
    unsigned total;
    unsigned base = block_scan(part, sm, &total);
    unsigned own[16];
    for (int e = 0; e < 16; ++e) own[e] = cnt[threadIdx.x * 16 + e];
    __syncthreads();
    // rewrite the counts as exclusive offsets
    for (int e = 0; e < 16; ++e) {
      cnt[threadIdx.x * 16 + e] = base;
      base += own[e];
    }
    __syncthreads();
    unsigned off[16];
#pragma unroll
    for (int d = 0; d < 16; ++d) off[d] = cnt[d * kThreads + threadIdx.x];
    for (int i = i0; i < i1; ++i) {
      const Cand x = src[i];
      const int d = (desc_key(x.val) >> shift) & 15;
      dst[off[d]++] = x;
    }
    __syncthreads();
    Cand* t = src;
    src = dst;
    dst = t;
  }
  // 8 passes: the sorted run is back in `a`
}

// filter_and_sample (src/model.c:67-127) with min_p = 0.  Its three walks
// over c (top_p cut, renormalising sum, CDF) are sequential in the
// reference's order on thread 0; the block stages c through LDS.  The token
// is valid in thread 0.
__device__ int filter_and_sample(const Cand* __restrict__ c, int n, float top_p, int top_k,
                                 uint64_t& rng, Smem& sm) {
  // stage chunk [c0, c0 + m) of c into sm.stage
  auto stage = [&](int c0, int m) __attribute__((always_inline)) {
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += kThreads) sm.stage[i] = c[c0 + i];
    __syncthreads();
  };
  if (top_p < 1.0f) {
    double cs = 0.0;
    int cut = n;
    for (int c0 = 0; c0 < n; c0 += kStage) {
      const int m = min(kStage, n - c0);
      stage(c0, m);
      if (threadIdx.x == 0 && cut == n)
        for (int i = 0; i < m; ++i) {
          cs += (double)sm.stage[i].val;
          if (cs >= (double)top_p) {
            cut = c0 + i + 1;
            break;
          }
        }
      if (threadIdx.x == 0) sm.iwork[2] = cut;
      __syncthreads();
      cut = sm.iwork[2];
      if (cut != n) break;
    }
    n = cut;
  }
  if (top_k > 0 && top_k < n) n = top_k;
  double new_sum = 0.0;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int m = min(kStage, n - c0);
    stage(c0, m);
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) new_sum += (double)sm.stage[i].val;
  }
  float r = 0.0f;
  if (threadIdx.x == 0) r = __fmul_rn(rng_float(rng), (float)new_sum);
  double cdf = 0.0;
  int token = -1;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int m = min(kStage, n - c0);
    stage(c0, m);
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) {
        cdf += (double)sm.stage[i].val;
        if ((double)r < cdf) {
          token = sm.stage[i].id;
          break;
        }
      }
    if (threadIdx.x == 0) sm.iwork[3] = token;
    __syncthreads();
    token = sm.iwork[3];
    if (token >= 0) break;
  }
  if (token < 0) {
    stage(n - 1, 1);
    token = sm.stage[0].id;
  }
  __syncthreads();
  return token;
}

// the entries of c[0..m) (m <= kStage) whose value is above `root`, in
// order, into sm.stage; returns their count.  Wave w takes entries
// 256w .. 256w+255, four per lane.
__device__ int stage_above(const Cand* __restrict__ c, int m, float root, Smem& sm) {
  constexpr int NW = kThreads / 64, PER = kStage / NW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  Cand x[PER / 64];
  uint64_t mk[PER / 64];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < PER / 64; ++j) {
    const int i = wave * PER + 64 * j + lane;
    bool h = false;
    if (i < m) {
      x[j] = c[i];
      h = x[j].val > root;
    }
    mk[j] = __ballot(h);
    cnt += __popcll(mk[j]);
  }
  if (lane == 0) sm.ired[wave] = cnt;
  __syncthreads();
  int off = 0, total = 0;
  for (int w = 0; w < NW; ++w) {
    const int cw = sm.ired[w];
    off += w < wave ? cw : 0;
    total += cw;
  }
#pragma unroll
  for (int j = 0; j < PER / 64; ++j) {
    if ((mk[j] >> lane) & 1ull) sm.stage[off + __popcll(mk[j] & below)] = x[j];
    off += __popcll(mk[j]);
  }
  __syncthreads();
  return total;
}

// min-heap selection of the k largest of c[0..n) (src/model.c:238-250,
// 322-337), one thread; c is global memory, staged through LDS.  The root
// never decreases (a replacement is larger than the old root, and after the
// sift the root is the replacement or a child that was not below the old
// root), so entries not above the root when their chunk is staged would be
// passed over and are not staged.
__device__ void heap_select(const Cand* __restrict__ c, int n, int k, Cand* heap, Smem& sm) {
  for (int i = threadIdx.x; i < k; i += kThreads) heap[i] = c[i];
  __syncthreads();
  if (threadIdx.x == 0)
    for (int i = k / 2 - 1; i >= 0; --i) heap_sift_down(heap, k, i);
  for (int c0 = k; c0 < n; c0 += kStage) {
    const int m = min(kStage, n - c0);
    __syncthreads();
    const int kept = stage_above(c + c0, m, heap[0].val, sm);
    if (threadIdx.x == 0)
      for (int i = 0; i < kept; ++i)
        if (sm.stage[i].val > heap[0].val) {
          heap[0] = sm.stage[i];
          heap_sift_down(heap, k, 0);
        }
  }
  __syncthreads();
}

// sum of (double) c[0..n).val in order, one thread, staged through LDS
__device__ double ordered_sum(const Cand* __restrict__ c, int n, Smem& sm) {
  double s = 0.0;
  for (int c0 = 0; c0 < n; c0 += kStage) {
    const int m = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += kThreads) sm.stage[i] = c[c0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) s += (double)sm.stage[i].val;
  }
  __syncthreads();
  return s;
}

// the generator state back, then the step bookkeeping of k_argmax_step
// (or, without ctl, the token alone); one thread
// the step counters, read by thread 0 when the kernel starts (nothing else
// in the step writes them) so that the bookkeeping at its end waits for no
// load
struct CtlSnap {
  int step = 0, hcount = 0, pos = 0, done = 0;
};
__device__ __forceinline__ CtlSnap ctl_snap(const StepIO& io) {
  CtlSnap c;
  if (threadIdx.x == 0 && io.ctl) {
    c.step = io.ctl[kCtlStep];
    c.hcount = io.ctl[kCtlHcount];
    c.pos = io.ctl[kCtlPos];
    c.done = io.ctl[kCtlDone];
  }
  return c;
}

__device__ void finish_step(int token, uint64_t rng, uint64_t* rng_state, const StepIO& io,
                            const CtlSnap& c) {
  *rng_state = rng;
  if (!io.ctl) {
    io.out_tokens[0] = token;
    return;
  }
  int* ctl = io.ctl;
  if (io.out_tokens) io.out_tokens[c.step] = token;
  ctl[kCtlStep] = c.step + 1;
  ctl[kCtlToken] = token;
  io.hist[c.hcount % kHist] = token;
  ctl[kCtlHcount] = c.hcount + 1;
  ctl[kCtlPos] = c.pos + 1 < 3 ? c.pos + 1 : 0;  // src/block.c:107
  if (c.done == kDoneArmed && (token == 50256 || token == 0)) ctl[kCtlDone] = kDoneStopped;
}

// the next token's embedding row (src/model.c:1116-1122), whole block
__device__ void embed_next(int token, const StepIO& io) {
  if (!io.ctl || !io.embed) return;
  const float* __restrict__ row = io.embed + (size_t)token * io.dm;
  for (int i = threadIdx.x; i < io.dm; i += kThreads) io.x[i] = row[i];
}

}  // namespace

// Front pass 1: logits[i] *= 1/temp over the block's segment and the
// segment's max under `x > m` from -1e30f (src/model.c:160-166).  Block 0
// also clears the histogram and the block counter of pass 2.  (The LM head
// can do this pass itself, with its own blocks' maxima.)
__global__ __launch_bounds__(kFrontThreads) void k_samp_scale(float* __restrict__ logits, int V,
                                                              float temp, void* scratch,
                                                              const int* ctl) {
  __shared__ float red[kFrontThreads / 64];
  if (step_stopped(ctl)) return;
  const Scratch sc = scratch_of(scratch, V);
  const int seg = front_seg(V);
  const int i0 = min(V, (int)blockIdx.x * seg), i1 = min(V, i0 + seg);
  if (blockIdx.x == 0 && threadIdx.x < kBuckets) sc.hist[threadIdx.x] = 0;
  const float inv_temp = cr_divf(1.0f, temp);
  float mx = -1e30f;
  for (int i = i0 + 4 * (int)threadIdx.x; i < i1; i += 4 * kFrontThreads) {
    const float4 q = load4(logits, i, i1);
    float v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __fmul_rn(v[e], inv_temp);
      if (i + e < i1 && v[e] > mx) mx = v[e];
    }
    if (i + 4 <= i1) {
      *(float4*)(logits + i) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < i1) logits[i + e] = v[e];
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float w = __shfl_xor(mx, o, 64);
    if (w > mx) mx = w;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFrontThreads / 64; ++w)
      if (red[w] > mx) mx = red[w];
    sc.pmax[blockIdx.x] = mx;
  }
}

// Front pass 2, kFront blocks: with the global max (of the npart partial
// maxima in pmax), each block adds its segment's counts to the 128-bucket
// histogram over logits >= the min_p threshold (src/model.c:180-194) and
// writes its pre-candidates: (i, logits[i]) with logits[i] >= the lowest
// extraction threshold, in index order, to pre[block * seg ..].
__global__ __launch_bounds__(kFrontThreads) void k_samp_hist(const float* __restrict__ logits,
                                                             int V, SampleParams p,
                                                             void* scratch,
                                                             const float* __restrict__ pmax,
                                                             int npart, const int* ctl) {
  constexpr int NW = kFrontThreads / 64;
  __shared__ int bhist[kBuckets];
  __shared__ int wcnt[NW];
  if (step_stopped(ctl)) return;
  const Scratch sc = scratch_of(scratch, V);
  const int seg = front_seg(V);
  const int i0 = min(V, (int)blockIdx.x * seg), i1 = min(V, i0 + seg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float4 q = load4(logits, i0 + 4 * (int)threadIdx.x, i1);  // before the max: independent
  const float max_logit = front_max(pmax, npart);
  const float min_p_thresh = min_p_threshold(max_logit, p.min_p);
  const int eff_k = effective_k(p.top_k);
  const bool use_hist = eff_k > 0;
  const float bucket_scale = bucket_scale_of();
  const float pre_thresh =
      use_hist ? extract_threshold(max_logit, min_p_thresh, kBuckets - 1) : min_p_thresh;
  if (threadIdx.x < kBuckets) bhist[threadIdx.x] = 0;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
  Cand* pre = sc.pre + (size_t)blockIdx.x * seg;
  int last = 0, off = 0;
  // the segment in rows of 4 * kFrontThreads entries (one row up to 65536
  // vocabulary entries), each compacted in index order after the last
  for (int i = i0 + 4 * (int)threadIdx.x, first = 1; i - 4 * (int)threadIdx.x < i1;
       i += 4 * kFrontThreads, first = 0) {
    const float4 qr = first ? q : load4(logits, i, i1);
    const float v[4] = {qr.x, qr.y, qr.z, qr.w};
    bool h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = i + e < i1;
      if (use_hist && in && v[e] >= min_p_thresh) {
        int b = cvtt_x86(__fmul_rn(__fsub_rn(max_logit, v[e]), bucket_scale));
        if (b >= kBuckets) b = kBuckets - 1;
        if (b < 0) b = 0;
        // the last bucket (20 or more below the max) takes most of the
        // vocabulary without a min_p threshold: counted in a register
        if (b == kBuckets - 1)
          ++last;
        else
          atomicAdd(&bhist[b], 1);
      }
      h[e] = in && v[e] >= pre_thresh;
    }
    // order-preserving compaction: lanes in order, then the waves
    uint64_t m[4];
    int wn = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m[e] = __ballot(h[e]);
      wn += __popcll(m[e]);
    }
    if (lane == 0) wcnt[wave] = wn;
    __syncthreads();
    int base = off, row = 0;
    for (int w = 0; w < NW; ++w) {
      base += w < wave ? wcnt[w] : 0;
      row += wcnt[w];
    }
    __syncthreads();
    int pos = base;
#pragma unroll
    for (int e = 0; e < 4; ++e) pos += __popcll(m[e] & below);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (h[e]) pre[pos++] = Cand{i + e, v[e]};
    off += row;
  }
  if (use_hist) {
    last = wave_sum_i32(last);
    if (lane == 0 && last) atomicAdd(&bhist[kBuckets - 1], last);
    __syncthreads();
    if (threadIdx.x < kBuckets && bhist[threadIdx.x])
      atomicAdd(&sc.hist[threadIdx.x], bhist[threadIdx.x]);
  }
  if (threadIdx.x == 0) sc.pcnt[blockIdx.x] = off;
}

// The rest of sample_advanced on one 1024-thread block, after the two front
// passes: the cutoff bucket, the candidates filtered from the pre-candidate
// lists in order, selection, softmax, sorting and the draw; then the step
// bookkeeping and the next token's embedding (StepIO).  Leaves the
// histogram cleared for the next call.
__global__ __launch_bounds__(1024) void k_sample(const float* __restrict__ logits, int V,
                                                 SampleParams p, uint64_t* __restrict__ rng_state,
                                                 void* scratch, const float* __restrict__ pmax,
                                                 int npart, StepIO io) {
  __shared__ Smem sm;
  const Scratch sc = scratch_of(scratch, V);
  const int seg = front_seg(V);
  // every load that does not depend on another goes out first
  const CtlSnap cs = ctl_snap(io);
  const int wave = threadIdx.x >> 6;
  int hc0 = 0, hc1 = 0;
  if (threadIdx.x < 64) {
    hc0 = sc.hist[2 * threadIdx.x];
    hc1 = sc.hist[2 * threadIdx.x + 1];
  }
  int pc[kListsPerWave];
#pragma unroll
  for (int j = 0; j < kListsPerWave; ++j) pc[j] = sc.pcnt[wave * kListsPerWave + j];
  uint64_t rng = *rng_state;
  const float max_logit = front_max(pmax, npart);
  const float min_p_thresh = min_p_threshold(max_logit, p.min_p);
  const int eff_k = effective_k(p.top_k);
  int token = 0;
  Cand* probs = sc.probs;
  Cand* probs2 = sc.pre;  // free once the candidates are gathered
  if (eff_k > 0) {
    // the cutoff bucket (src/model.c:196-213): first bucket whose running
    // count reaches k; lane l of wave 0 holds buckets 2l, 2l+1
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      const int c0 = hc0, c1 = hc1;
      int run = c0 + c1;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int up = __shfl_up(run, o, 64);
        if (l >= o) run += up;
      }
      const int before = run - (c0 + c1);
      const bool at0 = before + c0 >= eff_k, at1 = !at0 && run >= eff_k;
      const uint64_t hit = __ballot(at0 || at1);
      int cutoff = kBuckets - 1;
      if (hit) {
        const int first = __ffsll((unsigned long long)hit) - 1;
        const int a0 = __shfl(at0 ? 1 : 0, first, 64);
        cutoff = 2 * first + (a0 ? 0 : 1);
      }
      if (l == 0) sm.fwork[0] = extract_threshold(max_logit, min_p_thresh, cutoff);
    }
    __syncthreads();
    const float extract_thresh = sm.fwork[0];
    int n = gather(sc, pc, seg, extract_thresh, sc.probs, &probs, sm);
    if (n == 0) {
      token = argmax_scan(logits, V, logits[0], sm);
    } else {
      // top-k by a min-heap when there are more candidates (src/model.c:236-251)
      if (n > eff_k) {
        heap_select(probs, n, eff_k, sm.sel, sm);
        n = eff_k;
      } else {
        for (int i = threadIdx.x; i < n; i += kThreads) sm.sel[i] = probs[i];
        __syncthreads();
      }
      // softmax on the survivors (src/model.c:253-266)
      float lm = -1e30f;
      if ((int)threadIdx.x < n) lm = sm.sel[threadIdx.x].val;
      const float local_max = block_max(lm, sm);
      if ((int)threadIdx.x < n)
        sm.sel[threadIdx.x].val = libm::expf_glibc(__fsub_rn(sm.sel[threadIdx.x].val, local_max));
      __syncthreads();
      if (threadIdx.x == 0) {
        double sum_exp = 0.0;
        for (int i = 0; i < n; ++i) sum_exp += (double)sm.sel[i].val;
        sm.fwork[1] = cr_divf(1.0f, (float)sum_exp);
      }
      __syncthreads();
      const float inv_sum = sm.fwork[1];
      if ((int)threadIdx.x < n) sm.sel[threadIdx.x].val = __fmul_rn(sm.sel[threadIdx.x].val, inv_sum);
      __syncthreads();
      const Cand* src = sm.sel;
      if (p.top_p < 1.0f) {  // src/model.c:268-274
        sort_small(sm.sel, sm.sorted, n);
        src = sm.sorted;
      }
      token = filter_and_sample(src, n, p.top_p, 0, rng, sm);
    }
  } else {
    // no top-k: every candidate over the min_p threshold (src/model.c:278-300)
    int n = gather(sc, pc, seg, min_p_thresh, sc.probs, &probs, sm);
    if (n == 0) {
      token = argmax_scan(logits, V, logits[0], sm);
    } else {
      for (int i = threadIdx.x; i < n; i += kThreads)
        probs[i].val = libm::expf_glibc(__fsub_rn(probs[i].val, max_logit));
      __syncthreads();
      const double sum_exp = ordered_sum(probs, n, sm);
      if (threadIdx.x == 0) sm.fwork[1] = cr_divf(1.0f, (float)sum_exp);
      __syncthreads();
      const float inv_sum = sm.fwork[1];
      for (int i = threadIdx.x; i < n; i += kThreads) probs[i].val = __fmul_rn(probs[i].val, inv_sum);
      __syncthreads();
      bool done = false;
      if (p.top_p >= 1.0f && (p.top_k <= 0 || p.top_k >= n)) {  // src/model.c:306-307
        // order-independent: the candidates stay in index order
        token = filter_and_sample(probs, n, p.top_p, p.top_k, rng, sm);
        done = true;
      }
      if (!done && p.top_p < 1.0f && n > kPartial) {  // src/model.c:313-343
        heap_select(probs, n, kPartial, sm.sel, sm);
        sort_small(sm.sel, sm.sorted, kPartial);
        if (threadIdx.x == 0) {
          double cs = 0.0;
          int hit = 0;
          for (int i = 0; i < kPartial; ++i) {
            cs += (double)sm.sorted[i].val;
            if (cs >= (double)p.top_p) {
              hit = 1;
              break;
            }
          }
          sm.iwork[1] = hit;
        }
        __syncthreads();
        done = sm.iwork[1] != 0;
        __syncthreads();
        if (done) {
          // sm.sorted is read through the staging buffer
          for (int i = threadIdx.x; i < kPartial; i += kThreads) sm.sel[i] = sm.sorted[i];
          __syncthreads();
          token = filter_and_sample(sm.sel, kPartial, p.top_p, p.top_k, rng, sm);
        }
      }
      if (!done) {  // full sort (src/model.c:345-347)
        sort_large(probs, probs2, n, sm);
        token = filter_and_sample(probs, n, p.top_p, p.top_k, rng, sm);
      }
    }
  }

  // the token to every thread, the step, the next embedding; leave the
  // histogram cleared for the next call
  if (threadIdx.x == 0) {
    sm.iwork[4] = token;
    sm.iwork[5] = cs.done == kDoneStopped;
  }
  __syncthreads();
  token = sm.iwork[4];
  if (!sm.iwork[5]) {  // a stopped decode changes nothing
    if (threadIdx.x == 0) finish_step(token, rng, rng_state, io, cs);
    embed_next(token, io);
  }
  if (threadIdx.x < kBuckets) sc.hist[threadIdx.x] = 0;
}

// greedy (src/model.c:143-154): logits untouched, the generator state kept
__global__ __launch_bounds__(1024) void k_sample_greedy(const float* __restrict__ logits, int V,
                                                        uint64_t* __restrict__ rng_state,
                                                        StepIO io) {
  __shared__ Smem sm;
  const CtlSnap cs = ctl_snap(io);
  const int token = argmax_scan(logits, V, -1e9f, sm);
  if (threadIdx.x == 0) sm.iwork[5] = cs.done == kDoneStopped;
  __syncthreads();
  if (sm.iwork[5]) return;  // a stopped decode changes nothing
  if (threadIdx.x == 0) finish_step(token, *rng_state, rng_state, io, cs);
  embed_next(token, io);
}

size_t sample_scratch_bytes(int V) {
  if (V < 1) return 0;
  return ((size_t)V + (size_t)kFront * front_seg(V)) * sizeof(Cand) +
         (2 * kFront + kBuckets) * sizeof(int);
}

// pmax/npart: the maxima of logits already scaled by 1/temp (the LM head's
// scaled mode), or nullptr to scale here.  With ctl, the step bookkeeping
// and, with embed, the next embedding row into x[dm]; without, the token to
// out_tokens[0].
hipError_t launch_sample(float* logits, int V, float temp, float min_p, float top_p, int top_k,
                         uint64_t* rng_state, void* scratch, const float* pmax, int npart,
                         int* ctl, int* hist, int* out_tokens, const float* embed, int dm,
                         float* x, hipStream_t s, bool gated) {
  if (V < 1 || V > kMaxVocab) return hipErrorInvalidValue;
  if ((uintptr_t)logits % 16) return hipErrorInvalidValue;  // float4 passes
  const SampleParams p{temp, min_p, top_p, top_k};
  const StepIO io{ctl, hist, out_tokens, embed, dm, x};
  if (temp < 0.05f) {
    hipLaunchKernelGGL(k_sample_greedy, dim3(1), dim3(kThreads), 0, s, logits, V, rng_state, io);
    return hipGetLastError();
  }
  if (!pmax) {
    hipLaunchKernelGGL(k_samp_scale, dim3(kFront), dim3(kFrontThreads), 0, s, logits, V, temp,
                       scratch, gated ? (const int*)ctl : nullptr);
    pmax = scratch_of(scratch, V).pmax;
    npart = kFront;
  }
  hipLaunchKernelGGL(k_samp_hist, dim3(kFront), dim3(kFrontThreads), 0, s, logits, V, p, scratch,
                     pmax, npart, gated ? (const int*)ctl : nullptr);
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(kThreads), 0, s, logits, V, p, rng_state, scratch,
                     pmax, npart, io);
  return hipGetLastError();
}

}  // namespace bm

extern "C" size_t bm_hip_sample_workspace_bytes(int vocab) { return bm::sample_scratch_bytes(vocab); }

extern "C" int bm_hip_sample_advanced(float* logits, int vocab, float temp, float min_p,
                                      float top_p, int top_k, uint64_t* rng, void* workspace,
                                      int32_t* token_out, void* stream) {
  if (!logits || !rng || !workspace || !token_out) {
    bm_set_error("sample_advanced: null pointer");
    return -1;
  }
  const hipError_t e =
      bm::launch_sample(logits, vocab, temp, min_p, top_p, top_k, rng, workspace, nullptr, 0,
                        nullptr, nullptr, token_out, nullptr, 0, nullptr, (hipStream_t)stream,
                        false);
  if (e != hipSuccess) {
    bm_set_error("sample_advanced: %s (vocab %d, logits %p; vocab 1..256000, 16-byte aligned logits)",
                 hipGetErrorString(e), vocab, (void*)logits);
    return -1;
  }
  return 0;
}
