// Prefill / batched ternary GEMM on int8 MFMA, two K-groups per block.
//
// Semantics: scalar_bitlinear_forward_batch (src/kernel.c:322-338) per
// token, i.e. per output the int32 totals of each 1024-column block folded
// into fp32 in block order, out = 0; out += (float)total * inv_scale
// (src/kernel.c:255-256, 391, 407-425); or the exact int32 total (stress
// shape).  Bit-exact: the int32 sums are exact whatever their order, and the
// fp32 fold keeps the reference's order.
//
// Weights come in the MFMA tile layout written by k_tile_weights: for each
// run of 32 weight rows and each 128-column stage, 1 KB holding the rows'
// 32 packed bytes of the stage one after the other, so that a wave reads a
// 32-row x 128-column operand block as one contiguous kilobyte (full cache
// lines; the row-major image would give 32 bytes of each 128-byte line per
// stage).  Codes 11 are rewritten to 10 (same value, src/quantization.c:
// 27-31) while tiling, so the kernel uses w = code - 1 with code in {0,1,2}.
//
// Block: 512 threads = two K-groups of four waves.  Group g takes columns
// [g*K/2, (g+1)*K/2) of every dot product; the four waves of a group take
// 32*BT output columns each of the block's 64 x 128*BT tile (wave tile
// 64 x 32*BT, 2 x BT MFMA tiles of v_mfma_i32_32x32x32_i8).  Two waves per
// SIMD (one of each group), so one wave's VALU work (weight decode, slice
// folds) overlaps the other's MFMAs.  A wave keeps only the int32
// accumulators of its own K range (plus, for K = 3072/4096, one register per
// output of the range's first part), which is what lets a wave own 32*BT
// columns: keeping the fp32 running sum of all of K beside the accumulators
// would halve the tile.
//
// Per 128-column stage: the group's 256 threads load the activation stage
// (64 rows x 128 permuted int8, act_perm_off layout) three stages ahead into
// registers and write it to one of three LDS buffers a stage before use;
// each wave loads its weight blocks two stages ahead straight into registers
// (no LDS: no other wave of the group reads them).  Lane (j, h) of a wave
// covers columns 64h + 16q .. +15 of the stage in step q, for the activation
// and the weight operand alike.
//
// At the end group 1 hands its per-output values to group 0 through LDS:
// the int32 partial total of a 1024-column block that the split point cuts
// (added to group 0's partial before the block's fp32 term is formed), and
// the fp32 terms of its whole blocks; group 0 folds them in block order.
#include "bm_common.h"
#include "bm_dev.h"

namespace bm {

size_t tiled_bytes(int N, int K) {
  return (size_t)((N + 31) / 32) * (size_t)(K / 128) * 1024;
}

// one thread per 16 output bytes
__global__ void k_tile_weights(const uint8_t* __restrict__ W, int N, int K, int canonical,
                               uint8_t* __restrict__ T, size_t n16) {
  const int stages = K / 128;
  const size_t wstride = (size_t)(K / 4);
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t off = i * 16;
    const size_t tile = off / ((size_t)stages * 1024);
    const size_t rem = off - tile * (size_t)stages * 1024;
    const int st = (int)(rem >> 10), r = (int)((rem & 1023) >> 5), b = (int)(rem & 31);
    const size_t row = tile * 32 + r;
    v4i v;
    if (row < (size_t)N) {
      v = *(const v4i*)(W + row * wstride + (size_t)st * 32 + b);
      if (!canonical) {
        v.x = (int)canon_codes((uint32_t)v.x);
        v.y = (int)canon_codes((uint32_t)v.y);
        v.z = (int)canon_codes((uint32_t)v.z);
        v.w = (int)canon_codes((uint32_t)v.w);
      }
    } else {
      v = v4i{0x55555555, 0x55555555, 0x55555555, 0x55555555};  // code 01: weight 0
    }
    *(v4i*)(T + off) = v;
  }
}

hipError_t launch_tile_weights(const uint8_t* W, int N, int K, bool canonical, uint8_t* T,
                               hipStream_t s) {
  if (K % 128 != 0 || N <= 0 || ((uintptr_t)W & 15) || ((uintptr_t)T & 15))
    return hipErrorInvalidValue;
  const size_t n16 = tiled_bytes(N, K) / 16;
  int blocks = (int)((n16 + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_tile_weights, dim3(blocks), dim3(256), 0, s, W, N, K, canonical ? 1 : 0,
                     T, n16);
  return hipGetLastError();
}

namespace {

constexpr int KG_TM = 64;          // tile rows
constexpr int KG_STAGE = 128;      // columns per stage
constexpr int KG_ABUF = KG_TM * KG_STAGE;  // bytes of one activation stage
constexpr int KG_MAX_SLICES = 16;  // K <= 16384
constexpr int kKgBlocks = 256;     // persistent grid: one block per CU

// Split of K between the two groups and the 1024-column blocks each group
// covers (host-side plan, passed by value).
struct KgPlan {
  int n_st;       // stages per group
  int ks;         // first column of group 1 (K / 2)
  int seg_end0;   // group 0: stage after which its first block ends (n_st: one part)
  int seg_end1;   // group 1: the same
  int mid;        // ks is inside a 1024-column block
  int n_slices;   // blocks of K
  int ex;         // values per output handed from group 1 to group 0
};

// Output tile of a block: workgroups go to the 8 XCDs round robin (block b
// on XCD b % 8), each XCD with its own L2.  Every XCD gets one contiguous run
// of tiles, walked in groups of 8 tile rows so that the blocks resident at
// once share activation rows and weight columns in L2.
__device__ __forceinline__ void kg_tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
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

__device__ __forceinline__ void decode4(uint32_t pw, v4i& b) {
  b[0] = (int)(pw & 0x03030303u);
  b[1] = (int)((pw >> 2) & 0x03030303u);
  b[2] = (int)((pw >> 4) & 0x03030303u);
  b[3] = (int)((pw >> 6) & 0x03030303u);
}

template <int BT, bool HAS_O>
struct KgLds {
  static constexpr int A_BYTES = 2 * 3 * KG_ABUF;  // activation stages of both groups
  // hand-over pass: 4 waves x [mt][nt][v][lane] words
  static constexpr int PASS_BYTES = 4 * 2 * BT * 16 * 64 * 4;
  // finished output tile, row-major with a 16-byte pad per row
  static constexpr int PITCH = 128 * BT * 4 + 16;
  static constexpr int OUT_BYTES = KG_TM * PITCH;
  static constexpr int R_BYTES = PASS_BYTES > OUT_BYTES ? PASS_BYTES : OUT_BYTES;
  static constexpr int MAIN = A_BYTES + R_BYTES;
};

// Persistent: one 512-thread block per CU walks the tiles blockIdx.x,
// blockIdx.x + gridDim.x, ...  A finished tile's outputs go to LDS and are
// written to memory during the first stages of the block's next tile, so
// that the CUs' stores spread over the kernel instead of coming in one burst
// at the end of each round of tiles (the fp32 output is as large as the
// operands).
template <int MODE, int BT, bool HAS_O>
__global__ __launch_bounds__(512) void k_gemm_kg(const uint8_t* __restrict__ act,
                                                 size_t act_stride,
                                                 const float* __restrict__ scale_x, int M,
                                                 const uint8_t* __restrict__ Wt, int N, int K,
                                                 float w_scale, float* __restrict__ out,
                                                 int32_t* __restrict__ out_i32, KgPlan plan) {
  constexpr bool I32 = MODE == MODE_I32;
  constexpr int TN = 128 * BT;
  using L = KgLds<BT, HAS_O>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::MAIN];
  __shared__ __attribute__((aligned(16))) int s_sx[2][KG_MAX_SLICES][KG_TM];
  __shared__ __attribute__((aligned(16))) float s_inv[2][KG_TM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave >> 2, wn = wave & 3, gt = tid & 255;
  const int j32 = lane & 31, h = lane >> 5;
  const int tiles_m = (M + KG_TM - 1) / KG_TM, tiles_n = (N + TN - 1) / TN;
  const int n_tiles = tiles_m * tiles_n;
  const size_t perm = act_perm_off(K);
  const int n_st = plan.n_st;
  const int k0 = grp * plan.ks;
  const int stages_all = K / KG_STAGE;
  const int n_wtiles = (N + 31) / 32;
  uint8_t* __restrict__ sA = smem + grp * 3 * KG_ABUF;
  uint8_t* __restrict__ sR = smem + L::A_BYTES;

  int m0 = 0, n0 = 0, wtile0 = 0;
  auto set_tile = [&](int t) __attribute__((always_inline)) {
    int tm, tn;
    kg_tile_of(t, tiles_m, tiles_n, tm, tn);
    m0 = tm * KG_TM;
    n0 = tn * TN;
    wtile0 = (n0 >> 5) + wn * BT;
  };
  // per-row values of the tile (int32 sum of x per 1024-column block, and
  // 1/(scale_x * w_scale)) into registers; up to 16 blocks x 64 rows
  int rv_sx0 = 0, rv_sx1 = 0;
  float rv_inv = 0.0f;
  auto rows_fetch = [&]() __attribute__((always_inline)) {
    const int n = KG_TM * plan.n_slices;
    if (tid < n) {
      const int row = min(m0 + (tid % KG_TM), M - 1);
      rv_sx0 = ((const int*)(act + (size_t)row * act_stride))[tid / KG_TM];
    }
    if (tid + 512 < n) {
      const int row = min(m0 + ((tid + 512) % KG_TM), M - 1);
      rv_sx1 = ((const int*)(act + (size_t)row * act_stride))[(tid + 512) / KG_TM];
    }
    if (!I32 && tid < KG_TM) rv_inv = inv_scale_of(scale_x[min(m0 + tid, M - 1)], w_scale);
  };
  auto rows_put = [&](int b) __attribute__((always_inline)) {
    const int n = KG_TM * plan.n_slices;
    if (tid < n) s_sx[b][tid / KG_TM][tid % KG_TM] = rv_sx0;
    if (tid + 512 < n) s_sx[b][(tid + 512) / KG_TM][(tid + 512) % KG_TM] = rv_sx1;
    if (tid < KG_TM) s_inv[b][tid] = rv_inv;
  };

  // activation stage: chunk c = gt + 256 i is row c / 8, 16-byte chunk c % 8;
  // rows past M reread the last row, stages past the group's range the last
  auto load_a = [&](int st, v4i (&r)[2]) __attribute__((always_inline)) {
    const int kb = k0 + min(st, n_st - 1) * KG_STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = gt + 256 * i;
      const int row = min(m0 + (c >> 3), M - 1);
      r[i] = *(const v4i*)(act + (size_t)row * act_stride + perm + kb + 16 * (c & 7));
    }
  };
  // 16-byte chunks XOR-swizzled by row/2: the operand reads of 16
  // consecutive rows hit 16 different bank groups
  auto store_a = [&](int buf, const v4i (&r)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = gt + 256 * i;
      const int row = c >> 3;
      *(v4i*)(sA + buf * KG_ABUF + row * KG_STAGE + 16 * ((c & 7) ^ ((row >> 1) & 7))) = r[i];
    }
  };
  // weight blocks of the wave's BT row runs; runs past N reread the last
  auto load_b = [&](int st, v4i (&r)[BT]) __attribute__((always_inline)) {
    const int sg = (k0 >> 7) + min(st, n_st - 1);
#pragma unroll
    for (int nt = 0; nt < BT; ++nt) {
      const int t = min(wtile0 + nt, n_wtiles - 1);
      r[nt] = *(const v4i*)(Wt + ((size_t)t * stages_all + sg) * 1024 + j32 * 32 + h * 16);
    }
  };

  // Per-row values of the lane's outputs: element v of MFMA tile mt is row
  // 32 mt + 8 (v / 4) + 4 h + v % 4 of the tile, so each (mt, v / 4) is one
  // 16-byte read of four consecutive rows.
  auto rows_i = [&](const int* __restrict__ tab, int mt, int (&r)[16])
                    __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int4 q = *(const int4*)(tab + 32 * mt + 8 * g + 4 * h);
      r[4 * g] = q.x;
      r[4 * g + 1] = q.y;
      r[4 * g + 2] = q.z;
      r[4 * g + 3] = q.w;
    }
  };
  auto rows_f = [&](const float* __restrict__ tab, int mt, float (&r)[16])
                    __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 q = *(const float4*)(tab + 32 * mt + 8 * g + 4 * h);
      r[4 * g] = q.x;
      r[4 * g + 1] = q.y;
      r[4 * g + 2] = q.z;
      r[4 * g + 3] = q.w;
    }
  };
  // fp32 term of an int32 block total: (float)(total - sum x) * inv_scale
  auto term = [](int t, int sx, float inv) __attribute__((always_inline)) {
    return __fmul_rn((float)(t - sx), inv);
  };

  v16i acc[2][BT];
  float o[HAS_O ? 2 : 1][HAS_O ? BT : 1][16];
  int rb = 0;  // s_sx / s_inv buffer of the current tile

  // end of the first part of a group's range (HAS_O only): group 0 folds the
  // block's fp32 term into o; group 1 keeps the term, or the raw partial
  // total when the split point cuts the block
  auto first_part_end = [&]() __attribute__((always_inline)) {
    if constexpr (HAS_O) {
      const int slice = k0 >> 10;
      const bool keep_raw = grp == 1 && plan.mid;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        if (keep_raw) {
#pragma unroll
          for (int nt = 0; nt < BT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[mt][nt][v] = __int_as_float(acc[mt][nt][v]);
        } else {
          int sx[16];
          float inv[16];
          rows_i(s_sx[rb][slice], mt, sx);
          rows_f(s_inv[rb], mt, inv);
#pragma unroll
          for (int nt = 0; nt < BT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const float f = term(acc[mt][nt][v], sx[v], inv[v]);
              // o is +0 before: fl(+0 + f) = f, the reference's out = 0; out += f
              o[mt][nt][v] = grp == 0 ? __fadd_rn(o[mt][nt][v], f) : f;
            }
        }
#pragma unroll
        for (int nt = 0; nt < BT; ++nt)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0;
      }
    }
  };
  const int seg_end = grp == 0 ? plan.seg_end0 : plan.seg_end1;

  // Writes out the finished tile held in LDS (rows sm0.., columns sn0..):
  // 16-byte chunks c = tid + 512 i, row c / (TN / 4), columns 4 (c % (TN / 4))
  // onwards, for the chunk slots [c_lo, c_hi) of each thread.
  constexpr int CPT = KG_TM * TN / 4 / 512;  // chunks per thread
  const bool vec_out = (N % 4) == 0;
  auto drain = [&](int sm0, int sn0, int c_lo, int c_hi) __attribute__((always_inline)) {
    for (int i = c_lo; i < c_hi; ++i) {
      const int c = tid + 512 * i;
      const int row = c / (TN / 4), c4 = c % (TN / 4);
      const int r = sm0 + row, n = sn0 + 4 * c4;
      if (r >= M || n >= N) continue;
      const v4i v = *(const v4i*)(sR + row * L::PITCH + 16 * c4);
      const size_t idx = (size_t)r * N + n;
      if (vec_out && n + 3 < N) {
        if constexpr (I32) {
          *(v4i*)(out_i32 + idx) = v;
        } else if constexpr (MODE == MODE_ACC) {
          float4 a = *(const float4*)(out + idx);
          a.x = __fadd_rn(a.x, __int_as_float(v.x));
          a.y = __fadd_rn(a.y, __int_as_float(v.y));
          a.z = __fadd_rn(a.z, __int_as_float(v.z));
          a.w = __fadd_rn(a.w, __int_as_float(v.w));
          *(float4*)(out + idx) = a;
        } else {
          *(v4i*)(out + idx) = v;
        }
      } else {
        const int e_n = min(4, N - n);
        for (int e = 0; e < e_n; ++e) {
          if constexpr (I32)
            out_i32[idx + e] = v[e];
          else if constexpr (MODE == MODE_ACC)
            out[idx + e] = __fadd_rn(out[idx + e], __int_as_float(v[e]));
          else
            out[idx + e] = __int_as_float(v[e]);
        }
      }
    }
  };
  // the previous tile's outputs go out over the first stages of this one
  const int d_stages = min(n_st, 4);
  const int d_per = (CPT + d_stages - 1) / d_stages;
  int sm0 = 0, sn0 = 0;
  bool staged = false;

  // one stage: X holds activation stage st+1 (to LDS now), Y stage st+2 (in
  // flight), Z receives stage st+3; P holds the weights of stage st, Q those
  // of st+1, R receives st+2.  Order: the stage's eight operand reads from
  // LDS first, then the LDS writes and global loads of later stages, then
  // the four steps, each step's MFMAs next to the decode of the next step's
  // weights (scheduling fences keep the compiler from sinking the loads to
  // the stage's end or splitting the operand reads per step).
  auto body = [&](int st, v4i (&X)[2], v4i (&Y)[2], v4i (&Z)[2], v4i (&P)[BT], v4i (&Q)[BT],
                  v4i (&R)[BT]) __attribute__((always_inline)) {
    (void)Y;
    (void)Q;
    const uint8_t* __restrict__ cA = sA + (st % 3) * KG_ABUF;
    v4i aop[2][4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int r = mt * 32 + j32;
        aop[mt][q] = *(const v4i*)(cA + r * KG_STAGE + 16 * ((4 * h + q) ^ ((r >> 1) & 7)));
      }
    __builtin_amdgcn_sched_barrier(0);
    store_a((st + 1) % 3, X);
    load_b(st + 2, R);
    load_a(st + 3, Z);
    if (staged && st < d_stages) drain(sm0, sn0, st * d_per, min(CPT, (st + 1) * d_per));
    __builtin_amdgcn_sched_barrier(0);
    v4i bop[2][BT];
#pragma unroll
    for (int nt = 0; nt < BT; ++nt) decode4((uint32_t)P[nt][0], bop[0][nt]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < 3) {
#pragma unroll
        for (int nt = 0; nt < BT; ++nt) decode4((uint32_t)P[nt][q + 1], bop[(q + 1) & 1][nt]);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < BT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[mt][q], bop[q & 1][nt],
                                                             acc[mt][nt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (HAS_O && st + 1 == seg_end && seg_end < n_st) first_part_end();
    __syncthreads();
  };

  // hand-over area: [wave][mt][nt][v][lane] words of one pass
  int32_t* __restrict__ ex = (int32_t*)sR;
  auto ex_at = [&](int mt, int nt, int v) __attribute__((always_inline)) {
    return (((wn * 2 + mt) * BT + nt) * 16 + v) * 64 + lane;
  };
  const int n_ex = plan.ex;
  const int last = (K - 1) >> 10, last0 = (plan.ks - 1) >> 10;

  int tile = blockIdx.x;
  set_tile(tile);
  rows_fetch();
  v4i A0[2], A1[2], A2[2], B0[BT], B1[BT], B2[BT];
  load_a(0, A0);
  load_b(0, B0);
  load_a(1, A1);
  load_b(1, B1);
  load_a(2, A2);
  rows_put(0);
  for (;;) {
    store_a(0, A0);
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < BT; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][b][v] = 0;
    if constexpr (HAS_O) {
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < BT; ++b)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[a][b][v] = 0.0f;
    }
    __syncthreads();
    // three stages per turn so that each register set keeps its registers
    int st = 0;
    for (; st + 3 <= n_st; st += 3) {
      body(st, A1, A2, A0, B0, B1, B2);
      body(st + 1, A2, A0, A1, B1, B2, B0);
      body(st + 2, A0, A1, A2, B2, B0, B1);
    }
    if (st < n_st) body(st, A1, A2, A0, B0, B1, B2);
    if (st + 1 < n_st) body(st + 1, A2, A0, A1, B1, B2, B0);
    // every wave passed the last stage's barrier: the activation buffers,
    // and (drained in the first stages) the output area, are free

    const int cm0 = m0, cn0 = n0;
    const int next = tile + (int)gridDim.x;
    const bool more = next < n_tiles;

    // hand-over from group 1 to group 0, one or two passes.  Group 0 keeps
    // its running result in the accumulator registers (fp32 bits, or the
    // int32 total).
    if (grp == 0 && !I32 && !plan.mid) {
      // group 0's blocks end on the split point: fold its last block now
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        int sx[16];
        float inv[16];
        rows_i(s_sx[rb][last0], mt, sx);
        rows_f(s_inv[rb], mt, inv);
#pragma unroll
        for (int nt = 0; nt < BT; ++nt)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            acc[mt][nt][v] = __float_as_int(
                __fadd_rn(HAS_O ? o[mt][nt][v] : 0.0f, term(acc[mt][nt][v], sx[v], inv[v])));
      }
    }
    for (int e = 0; e < n_ex; ++e) {
      if (grp == 1) {
        // pass e: the kept first-part value, else the range's last part:
        // its raw int32 total (int32 outputs, or a range inside one block)
        // or its block's fp32 term
        const bool kept = HAS_O && n_ex == 2 && e == 0;
        const bool raw = I32 || (n_ex == 1 && plan.mid);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          if (kept) {
            if constexpr (HAS_O) {
#pragma unroll
              for (int nt = 0; nt < BT; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                  ex[ex_at(mt, nt, v)] = __float_as_int(o[mt][nt][v]);
            }
          } else if (raw) {
#pragma unroll
            for (int nt = 0; nt < BT; ++nt)
#pragma unroll
              for (int v = 0; v < 16; ++v) ex[ex_at(mt, nt, v)] = acc[mt][nt][v];
          } else {
            int sx[16];
            float inv[16];
            rows_i(s_sx[rb][last], mt, sx);
            rows_f(s_inv[rb], mt, inv);
#pragma unroll
            for (int nt = 0; nt < BT; ++nt)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                ex[ex_at(mt, nt, v)] = __float_as_int(term(acc[mt][nt][v], sx[v], inv[v]));
          }
        }
      }
      __syncthreads();
      if (grp == 0) {
        const bool split = !I32 && plan.mid && e == 0;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          int sx[16];
          float inv[16];
          if constexpr (I32) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sx[v] = 0;
            for (int sl = 0; sl < plan.n_slices; ++sl) {
              int t[16];
              rows_i(s_sx[rb][sl], mt, t);
#pragma unroll
              for (int v = 0; v < 16; ++v) sx[v] += t[v];
            }
#pragma unroll
            for (int nt = 0; nt < BT; ++nt)
#pragma unroll
              for (int v = 0; v < 16; ++v) acc[mt][nt][v] += ex[ex_at(mt, nt, v)] - sx[v];
          } else if (split) {
            // the split block: both partial totals, then its fp32 term
            rows_i(s_sx[rb][last0], mt, sx);
            rows_f(s_inv[rb], mt, inv);
#pragma unroll
            for (int nt = 0; nt < BT; ++nt)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                acc[mt][nt][v] = __float_as_int(
                    __fadd_rn(HAS_O ? o[mt][nt][v] : 0.0f,
                              term(acc[mt][nt][v] + ex[ex_at(mt, nt, v)], sx[v], inv[v])));
          } else {
#pragma unroll
            for (int nt = 0; nt < BT; ++nt)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                acc[mt][nt][v] = __float_as_int(__fadd_rn(__int_as_float(acc[mt][nt][v]),
                                                          __int_as_float(ex[ex_at(mt, nt, v)])));
          }
        }
      }
      __syncthreads();
    }
    // the finished tile into the output area, row-major
    if (grp == 0) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < BT; ++nt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int row = 32 * mt + 8 * (v >> 2) + 4 * h + (v & 3);
            const int col = (wn * BT + nt) * 32 + j32;
            *(int*)(sR + row * L::PITCH + 4 * col) = acc[mt][nt][v];
          }
    }
    sm0 = cm0;
    sn0 = cn0;
    staged = true;
    if (!more) break;
    // the next tile's first stages (issuing them before the hand-over, to
    // hide their latency, runs out of registers at two waves per SIMD)
    set_tile(next);
    rows_fetch();
    load_a(0, A0);
    load_b(0, B0);
    load_a(1, A1);
    load_b(1, B1);
    load_a(2, A2);
    tile = next;
    rb ^= 1;
    rows_put(rb);
  }
  __syncthreads();
  drain(sm0, sn0, 0, CPT);
}

// host plan; false if the shape is outside what the kernel covers
bool kg_plan(int K, int mode, KgPlan& p, bool& has_o) {
  if (K % 256 != 0 || K < 256 || K > 16384) return false;
  p.n_slices = slices_of(K);
  p.ks = K / 2;
  p.n_st = p.ks / KG_STAGE;
  p.mid = p.ks % kSlice != 0;
  if (mode == MODE_I32) {
    p.seg_end0 = p.seg_end1 = p.n_st;
    p.ex = 1;
    has_o = false;
    return true;
  }
  const int parts0 = (p.ks - 1) / kSlice + 1;
  const int parts1 = (K - 1) / kSlice - p.ks / kSlice + 1;
  if (parts0 > 2 || parts1 > 2) return false;
  p.seg_end0 = parts0 == 2 ? kSlice / KG_STAGE : p.n_st;
  p.seg_end1 = parts1 == 2 ? ((p.ks / kSlice + 1) * kSlice - p.ks) / KG_STAGE : p.n_st;
  p.ex = parts1;
  has_o = parts0 == 2 || parts1 == 2;
  return true;
}

template <int MODE, int BT, bool HAS_O>
hipError_t kg_launch(const uint8_t* act, const float* scale_x, int M, const uint8_t* Wt, int N,
                     int K, float w_scale, void* out, const KgPlan& p, hipStream_t s) {
  const long long tiles =
      (long long)((M + KG_TM - 1) / KG_TM) * ((N + 128 * BT - 1) / (128 * BT));
  const dim3 grid((unsigned)(tiles < kKgBlocks ? tiles : kKgBlocks));
  hipLaunchKernelGGL((k_gemm_kg<MODE, BT, HAS_O>), grid, dim3(512), 0, s, act, act_row_bytes(K),
                     scale_x, M, Wt, N, K, w_scale, (float*)out, (int32_t*)out, p);
  return hipGetLastError();
}

// rounds of resident blocks (one per CU) weighted by the tile's work
double kg_cost(int M, int N, int BT) {
  const long long tiles = (long long)((M + KG_TM - 1) / KG_TM) * ((N + 128 * BT - 1) / (128 * BT));
  return (double)((tiles + 255) / 256) * BT;
}

template <int MODE>
hipError_t kg_mode(const uint8_t* act, const float* scale_x, int M, const uint8_t* Wt, int N,
                   int K, float w_scale, void* out, hipStream_t s) {
  KgPlan p;
  bool has_o = false;
  if (!kg_plan(K, MODE, p, has_o)) return hipErrorInvalidValue;
  if (has_o) return kg_launch<MODE, 2, true>(act, scale_x, M, Wt, N, K, w_scale, out, p, s);
  if (kg_cost(M, N, 3) <= kg_cost(M, N, 2))
    return kg_launch<MODE, 3, false>(act, scale_x, M, Wt, N, K, w_scale, out, p, s);
  return kg_launch<MODE, 2, false>(act, scale_x, M, Wt, N, K, w_scale, out, p, s);
}

}  // namespace

bool gemm_tiled_supported(int M, int K, int mode) {
  KgPlan p;
  bool has_o;
  return M >= 1 && kg_plan(K, mode, p, has_o);
}

hipError_t launch_gemm_tiled(const uint8_t* act, const float* scale_x, int M,
                             const uint8_t* tiled, int N, int K, float w_scale, void* out,
                             int mode, hipStream_t s) {
  if (mode == MODE_I32) return kg_mode<MODE_I32>(act, scale_x, M, tiled, N, K, w_scale, out, s);
  if (mode == MODE_ACC) return kg_mode<MODE_ACC>(act, scale_x, M, tiled, N, K, w_scale, out, s);
  return kg_mode<MODE_STORE>(act, scale_x, M, tiled, N, K, w_scale, out, s);
}

}  // namespace bm
