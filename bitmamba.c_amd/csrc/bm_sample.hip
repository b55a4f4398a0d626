// Device sampler: the reference's sample_advanced (src/model.c:132-361) with
// filter_and_sample (src/model.c:67-127) and the XorShift64* generator
// (src/utils.c:117-140), bit for bit, in one 1024-thread block per token.
//
// The O(V) passes run on the whole block: temperature scaling and the max
// logit, the 128-bucket histogram, candidate extraction in ascending index
// order (a block-wide scan), the exponentials and rescaling, and a stable
// radix sort where the reference sorts every candidate.  The steps whose
// result depends on their order stay sequential on one thread, in the
// reference's order: the heap selections (their array order feeds the
// sums), every double sum, and the CDF walk.  Sorting is stable like
// glibc's qsort (a merge sort for these sizes), keyed on the value.
// Float-to-int bucket indices follow x86 cvttss2si (out of range -> INT_MIN).
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
constexpr int kCtlPos = 0, kCtlToken = 1, kCtlStep = 2, kCtlHcount = 3;
constexpr int kHist = 256;

struct Smem {
  Cand stage[kStage];
  Cand sel[kPartial];
  Cand sorted[kPartial];
  int hist[kBuckets];
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

// candidates (i, logits[i]) with logits[i] >= thr, ascending i
__device__ int extract(const float* __restrict__ logits, int V, float thr, Cand* __restrict__ out,
                       Smem& sm) {
  const int per = (V + kThreads - 1) / kThreads;
  const int i0 = threadIdx.x * per, i1 = min(V, i0 + per);
  unsigned c = 0;
  for (int i = i0; i < i1; ++i) c += logits[i] >= thr;
  unsigned total;
  unsigned o = block_scan(c, sm, &total);
  for (int i = i0; i < i1; ++i) {
    const float v = logits[i];
    if (v >= thr) out[o++] = Cand{i, v};
  }
  __syncthreads();
  return (int)total;
}

// first index of the maximum, starting from index 0 (src/model.c:225-233,
// 285-291): a later value wins only when strictly greater, so a NaN at index
// 0 is never beaten and NaNs elsewhere never win.  Returned to every thread.
__device__ int argmax_from0(const float* __restrict__ logits, int V, Smem& sm) {
  float bv = logits[0];
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
  unsigned short* cnt = (unsigned short*)sm.stage;  // [16][kThreads]
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
    for (int d = 0; d < 16; ++d) cnt[d * kThreads + threadIdx.x] = (unsigned short)c[d];
    __syncthreads();
    // exclusive offsets in (digit, thread) order: thread t scans its 16
    // entries t*16 .. t*16+15 of the flattened array, then the partials
    unsigned part = 0;
    for (int e = 0; e < 16; ++e) part += cnt[threadIdx.x * 16 + e];
    unsigned total;
    unsigned base = block_scan(part, sm, &total);
    unsigned short own[16];
    for (int e = 0; e < 16; ++e) own[e] = cnt[threadIdx.x * 16 + e];
    __syncthreads();
    // rewrite the counts as exclusive offsets (they fit: n <= 65535 is
    // checked by the caller)
    for (int e = 0; e < 16; ++e) {
      cnt[threadIdx.x * 16 + e] = (unsigned short)base;
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

// min-heap selection of the k largest of c[0..n) (src/model.c:238-250,
// 322-337), one thread; c is global memory, staged through LDS
__device__ void heap_select(const Cand* __restrict__ c, int n, int k, Cand* heap, Smem& sm) {
  for (int i = threadIdx.x; i < k; i += kThreads) heap[i] = c[i];
  __syncthreads();
  if (threadIdx.x == 0)
    for (int i = k / 2 - 1; i >= 0; --i) heap_sift_down(heap, k, i);
  for (int c0 = k; c0 < n; c0 += kStage) {
    const int m = min(kStage, n - c0);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += kThreads) sm.stage[i] = c[c0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i)
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

}  // namespace

// One sampling step plus the step bookkeeping of k_argmax_step.  `logits`
// is scaled in place by 1/temp like the reference's.  `probs`/`probs2`:
// V candidates each of scratch.
__global__ __launch_bounds__(1024) void k_sample(float* __restrict__ logits, int V,
                                                 SampleParams p, uint64_t* __restrict__ rng_state,
                                                 Cand* __restrict__ probs, Cand* __restrict__ probs2,
                                                 int* __restrict__ ctl, int* __restrict__ hist,
                                                 int* __restrict__ out_tokens) {
  __shared__ Smem sm;
  uint64_t rng = *rng_state;
  int token = 0;

  // temperature and the max logit (src/model.c:160-166)
  const float inv_temp = cr_divf(1.0f, p.temp);
  float mx = -1e30f;
  for (int i = threadIdx.x; i < V; i += kThreads) {
    const float v = __fmul_rn(logits[i], inv_temp);
    logits[i] = v;
    if (v > mx) mx = v;
  }
  __syncthreads();
  const float max_logit = block_max(mx, sm);
  // min_p threshold before the softmax (src/model.c:172-176)
  float min_p_thresh = -1e30f;
  if (p.min_p >= 1.0f)
    min_p_thresh = max_logit;
  else if (p.min_p > 0.0f)
    min_p_thresh = __fadd_rn(max_logit, libm::logf_glibc(p.min_p));
  const int eff_k = (p.top_k > 0 && p.top_k <= 256) ? p.top_k : 0;

  if (eff_k > 0) {
    // bucket histogram and its cutoff (src/model.c:181-214)
    for (int b = threadIdx.x; b < kBuckets; b += kThreads) sm.hist[b] = 0;
    __syncthreads();
    const float bucket_scale = cr_divf((float)(kBuckets - 1), 20.0f);
    for (int i = threadIdx.x; i < V; i += kThreads) {
      const float v = logits[i];
      if (v >= min_p_thresh) {
        int b = cvtt_x86(__fmul_rn(__fsub_rn(max_logit, v), bucket_scale));
        if (b >= kBuckets) b = kBuckets - 1;
        if (b < 0) b = 0;
        atomicAdd(&sm.hist[b], 1);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int accum = 0, cutoff = kBuckets - 1;
      for (int b = 0; b < kBuckets; ++b) {
        accum += sm.hist[b];
        if (accum >= eff_k) {
          cutoff = b;
          break;
        }
      }
      const float bucket_thresh = __fsub_rn(max_logit, cr_divf((float)(cutoff + 1), bucket_scale));
      sm.fwork[0] = bucket_thresh > min_p_thresh ? bucket_thresh : min_p_thresh;
    }
    __syncthreads();
    const float extract_thresh = sm.fwork[0];
    int n = extract(logits, V, extract_thresh, probs, sm);
    if (n == 0) {
      token = argmax_from0(logits, V, sm);
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
    int n = extract(logits, V, min_p_thresh, probs, sm);
    if (n == 0) {
      token = argmax_from0(logits, V, sm);
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

  if (threadIdx.x == 0) {
    *rng_state = rng;
    const int step = ctl[kCtlStep];
    if (out_tokens) out_tokens[step] = token;
    ctl[kCtlStep] = step + 1;
    ctl[kCtlToken] = token;
    hist[ctl[kCtlHcount] % kHist] = token;
    ctl[kCtlHcount] += 1;
    ctl[kCtlPos] = ctl[kCtlPos] + 1 < 3 ? ctl[kCtlPos] + 1 : 0;  // src/block.c:107
  }
}

size_t sample_scratch_bytes(int V) { return 2 * (size_t)V * sizeof(Cand); }

hipError_t launch_sample(float* logits, int V, float temp, float min_p, float top_p, int top_k,
                         uint64_t* rng_state, void* scratch, int* ctl, int* hist, int* out_tokens,
                         hipStream_t s) {
  if (V < 1 || V > 65535) return hipErrorInvalidValue;  // 16-bit radix offsets
  Cand* probs = (Cand*)scratch;
  const SampleParams p{temp, min_p, top_p, top_k};
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(kThreads), 0, s, logits, V, p, rng_state, probs,
                     probs + V, ctl, hist, out_tokens);
  return hipGetLastError();
}

}  // namespace bm
