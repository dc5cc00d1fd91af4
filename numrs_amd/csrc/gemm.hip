// fp32 MFMA GEMMs for matmul_backward (dA = dC @ B^T, dB = A^T @ dC) and the
// forward products, on gfx950 (CDNA4).
//
// One generic tile routine computes C[P,Q] (+)= X[P,R] @ Y[R,Q] where each
// operand is either "R-contiguous" (the reduction index is the fast one in
// memory: X[p*ld + r], Y[q*ld + r]) or "P/Q-contiguous" (X[r*ld + p],
// Y[r*ld + q]).  The four layouts cover every product on the path:
//   dA = dC @ B^T   X = dC (R-contig), Y = B   (R-contig)   [NT]
//   dB = A^T @ dC   X = A  (P-contig), Y = dC  (Q-contig)   [TN]
//   C  = A @ B      X = A  (R-contig), Y = B   (Q-contig)   [NN]
//   y  = x @ W^T    X = x  (R-contig), Y = W   (R-contig)   [NT]
//
// Work decomposition
//   * Workgroup tile 128(P) x 128(Q), 256 threads = 4 wave64s in a 2x2 grid,
//     each wave owns a 64x64 sub-tile = 2x2 blocks of v_mfma_f32_32x32x2f32
//     (16 accumulator VGPRs per block per lane).
//   * Reduction tile BR = 32, double-buffered in LDS, one barrier per tile; the
//     next tile's global loads are in flight while the MFMAs of the current
//     one run.  Each tile's MFMA sums start from zero and are added into
//     fp32 running totals (two-level accumulation, for accuracy).
//   * 226 VGPRs, no scratch, 2 waves per SIMD (launch bounds 256 x 2): LDS
//     (72 KiB per workgroup) allows two workgroups per CU.
//   * An MFMA 32x32x2 consumes, per lane l = 32*h + c, X[p=c][r=h] and
//     Y[r=h][q=c].  Eight consecutive reduction indices are fed to four
//     MFMAs as r = 4h + j (j = 0..3): an R-contiguous operand then gives each
//     lane four consecutive floats (one ds_read_b128 from a [p][r] LDS tile of
//     row stride 36 floats, conflict-free), and a P-contiguous operand gives
//     four ds_read_b32 from a [r][p] tile whose lanes read consecutive words.
//     Neither layout is transposed on its way into LDS.
//   * XCD-aware ordering: gfx950 dispatches workgroup b to XCD b % 8; the
//     logical tile index is permuted so each XCD owns a contiguous 4 x 8 patch
//     of tiles and its private L2 sees the operand rows/columns it reuses.
//   * matmul_backward launches dA and dB tiles in ONE grid.
//   * Aligned products with at least one 256 x 128 tile per CU take the
//     streamed large-tile path further down (DMA ring, one workgroup per CU).
//   * Split-K for products with few output tiles and long reductions (the
//     weight gradients X^T dY of Linear layers): each split writes a plain
//     partial, splitk_reduce adds them in split order -- deterministic.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kBP = 128;                 // tile extent along P and along Q
constexpr int kBR = 32;                  // reduction tile
constexpr int kThreads = 256;
constexpr int kRcStride = kBR + 4;       // [p][r] tile row stride (floats)
constexpr int kPcStride = kBP + 8;       // [r][p] tile row stride (floats)
constexpr int kTileFloats = kBP * kRcStride;  // 4608 >= kBR * kPcStride = 4352
constexpr int kGroupRows = 4;            // tile rows per raster group

struct Gemm {
  const float *X;
  const float *Y;
  float *C;
  int64_t ldx, ldy, ldc;
  // Batch z = zo * binner + zi addresses X + zo*bsx + zi*bsx2 (same for Y, C):
  // one level covers plain batches, two levels cover head-interleaved
  // layouts such as [batch, seq, heads, dim].
  int64_t bsx, bsy, bsc;
  int64_t bsx2, bsy2, bsc2;
  int binner;
  int P, Q, R;
  int tiles_p, tiles_q;
  int accumulate;
  float alpha;  // C = alpha * X@Y (+ C)
  // Split-K: with splits > 1 the reduction is cut into `splits` ranges of
  // whole k-tiles; range s writes its plain partial product to
  // partial + s*P*Q (row stride Q) and splitk_reduce forms alpha*sum (+C).
  int splits;
  int ktiles_per_split;
  float *partial;
  // Optional bias added per output column after alpha: C = alpha*X@Y + bias[q]
  // (+ C); the Linear forward's "+ b" folded into the product's epilogue.
  const float *bias;
  // Tiny kernel only: X entries whose `xmask` entry (same layout and
  // offsets as X) is not > 0 read as zero (ReLU backward applied on load).
  const float *xmask;
  // Activation applied last in the epilogue (batch-1 products): kActRelu
  // (x.max(0)) or kActGelu (exact erf); with `pre` the value before it is
  // stored there too (row stride ldc), for the activation's backward.
  int act;
  float *pre;
  // Optional residual added after the bias: C = alpha*X@Y + bias[q] +
  // res[p*ldr + q] (+ C) -- the "x + Linear(a)" of a residual block folded
  // into the product's epilogue (batch-1 products).
  const float *res;
  int64_t ldr;
  // Split products reduced inside their own launch: per output tile, eight
  // arrival counters (one per sub-block of TP/8 rows); null otherwise.
  unsigned *arrive;
};

// Epilogue activations: the ReLU forward kernel's x.max(0) and the unary
// kernel's exact-erf GELU, value for value.
constexpr int kActRelu = 1, kActGelu = 2;
__device__ __forceinline__ float act_value(int act, float v) {
  return act == kActRelu ? fmaxf(v, 0.0f) : numrs_hip::gelu_erf(v);
}

// Loads one 128 x 32 operand tile from global memory into registers
// (4 x float4 per thread) with zero fill outside [0,P) x [0,R).
template <bool RC, bool VEC>
struct TileLoad {
  f4 v[4];

  __device__ __forceinline__ void load(const float *__restrict__ base, int64_t ld, int p0, int r0,
                                       int P, int R, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + kThreads * i;
      int p, r;
      if (RC) {
        p = idx >> 3;
        r = (idx & 7) * 4;
      } else {
        r = idx >> 5;
        p = (idx & 31) * 4;
      }
      const int gp = p0 + p, gr = r0 + r;
      if (VEC) {
        // Extents are multiples of 4, so a float4 is wholly in or out.
        const bool in = RC ? (gp < P && gr < R) : (gr < R && gp < P);
        const float *src = RC ? base + (int64_t)gp * ld + gr : base + (int64_t)gr * ld + gp;
        v[i] = in ? *reinterpret_cast<const f4 *>(src) : f4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool in = RC ? (gp < P && gr + e < R) : (gr < R && gp + e < P);
          const float *src =
              RC ? base + (int64_t)gp * ld + gr + e : base + (int64_t)gr * ld + gp + e;
          v[i][e] = in ? *src : 0.f;
        }
      }
    }
  }

  __device__ __forceinline__ void store(float *__restrict__ lds, int tid) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + kThreads * i;
      if (RC) {
        *reinterpret_cast<f4 *>(lds + (idx >> 3) * kRcStride + (idx & 7) * 4) = v[i];
      } else {
        *reinterpret_cast<f4 *>(lds + (idx >> 5) * kPcStride + (idx & 31) * 4) = v[i];
      }
    }
  }
};

// Four reduction-consecutive operand values for MFMA group g at lane (h, c).
template <bool RC>
__device__ __forceinline__ f4 frag(const float *__restrict__ lds, int pbase, int c, int h, int g) {
  if (RC) {
    return *reinterpret_cast<const f4 *>(lds + (pbase + c) * kRcStride + 8 * g + 4 * h);
  } else {
    f4 f;
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = lds[(8 * g + 4 * h + j) * kPcStride + pbase + c];
    return f;
  }
}

// ACT: the epilogue applies d.act (separate instantiation, as for the
// streamed tiles).
template <bool XRC, bool YRC, bool VEC, bool ACT = false>
__device__ __forceinline__ void gemm_tile(const Gemm &d, int tile, int batch, float *smem) {
  // Split-K: consecutive logical tiles are the k-ranges of one output tile.
  const int split = tile % d.splits;
  tile /= d.splits;
  // Raster order: groups of kGroupRows tile-rows, column-major inside a group.
  const int per_group = kGroupRows * d.tiles_q;
  const int gidx = tile / per_group;
  const int first_p = gidx * kGroupRows;
  const int rows_in_group = min(d.tiles_p - first_p, kGroupRows);
  const int in_group = tile - gidx * per_group;
  const int tp = first_p + in_group % rows_in_group;
  const int tq = in_group / rows_in_group;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wp = wave >> 1, wq = wave & 1;
  const int c = lane & 31, h = lane >> 5;
  const int p0 = tp * kBP, q0 = tq * kBP;

  const int64_t zo = batch / d.binner, zi = batch - zo * d.binner;
  const float *__restrict__ X = d.X + zo * d.bsx + zi * d.bsx2;
  const float *__restrict__ Y = d.Y + zo * d.bsy + zi * d.bsy2;
  float *__restrict__ C = d.C + zo * d.bsc + zi * d.bsc2;

  float *xs0 = smem, *xs1 = smem + kTileFloats;
  float *ys0 = smem + 2 * kTileFloats, *ys1 = smem + 3 * kTileFloats;

  f16v acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};

  TileLoad<XRC, VEC> lx;
  TileLoad<YRC, VEC> ly;
  const int nk_all = (d.R + kBR - 1) / kBR;
  const int kt_begin = split * d.ktiles_per_split;
  const int nk = max(0, min(nk_all - kt_begin, d.ktiles_per_split));
  const int r_begin = kt_begin * kBR;

  lx.load(X, d.ldx, p0, r_begin, d.P, d.R, tid);
  ly.load(Y, d.ldy, q0, r_begin, d.Q, d.R, tid);
  lx.store(xs0, tid);
  ly.store(ys0, tid);
  __syncthreads();

  // Two-level accumulation: the MFMAs of one reduction tile accumulate from
  // zero, and the tile sums are added into running totals with VALU adds.  A
  // single MFMA accumulator chain over all of R carries a partial sum that
  // grows like sqrt(R), and its per-step rounding error with it; restarting
  // per tile keeps the MFMA partials small (error is 4x below numrs's own
  // sequential fp32 loop at R = 2048).
  f16v tot00 = {}, tot01 = {}, tot10 = {}, tot11 = {};
  for (int kt = 0; kt < nk; ++kt) {
    acc00 = f16v{};
    acc01 = f16v{};
    acc10 = f16v{};
    acc11 = f16v{};
    const bool more = kt + 1 < nk;
    if (more) {
      lx.load(X, d.ldx, p0, r_begin + (kt + 1) * kBR, d.P, d.R, tid);
      ly.load(Y, d.ldy, q0, r_begin + (kt + 1) * kBR, d.Q, d.R, tid);
    }
    const float *xl = (kt & 1) ? xs1 : xs0;
    const float *yl = (kt & 1) ? ys1 : ys0;
#pragma unroll
    for (int g = 0; g < kBR / 8; ++g) {
      const f4 a0 = frag<XRC>(xl, wp * 64, c, h, g);
      const f4 a1 = frag<XRC>(xl, wp * 64 + 32, c, h, g);
      const f4 b0 = frag<YRC>(yl, wq * 64, c, h, g);
      const f4 b1 = frag<YRC>(yl, wq * 64 + 32, c, h, g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc00 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b0[j], acc00, 0, 0, 0);
        acc01 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[j], b1[j], acc01, 0, 0, 0);
        acc10 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b0[j], acc10, 0, 0, 0);
        acc11 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[j], b1[j], acc11, 0, 0, 0);
      }
    }
    if (more) {
      lx.store((kt & 1) ? xs0 : xs1, tid);
      ly.store((kt & 1) ? ys0 : ys1, tid);
    }
    tot00 += acc00;
    tot01 += acc01;
    tot10 += acc10;
    tot11 += acc11;
    __syncthreads();
  }
  acc00 = tot00;
  acc01 = tot01;
  acc10 = tot10;
  acc11 = tot11;

  // 32x32 accumulator layout: lane (h, c), register i holds
  // row 8*(i/4) + 4*h + (i%4), column c.
  const f16v *accs[4] = {&acc00, &acc01, &acc10, &acc11};
  // Residual and bias values are all loaded before the first store (res or
  // bias may alias C as far as the compiler knows, which would otherwise
  // order each load after the previous store).
  float bq[2];
#pragma unroll
  for (int bj = 0; bj < 2; ++bj) {
    const int q = q0 + wq * 64 + bj * 32 + c;
    bq[bj] = d.splits == 1 && d.bias != nullptr && q < d.Q ? d.bias[q] : 0.0f;
  }
  f16v rv[4];
  if (d.splits == 1 && d.res != nullptr) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int bi = blk >> 1, bj = blk & 1;
      const int q = q0 + wq * 64 + bj * 32 + c;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int p = p0 + wp * 64 + bi * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        rv[blk][i] = p < d.P && q < d.Q ? d.res[(int64_t)p * d.ldr + q] : 0.0f;
      }
    }
  }
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int bi = blk >> 1, bj = blk & 1;
    const int q = q0 + wq * 64 + bj * 32 + c;
    const f16v &a = *accs[blk];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int p = p0 + wp * 64 + bi * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (p < d.P && q < d.Q) {
        if (d.splits > 1) {
          d.partial[((int64_t)split * d.P + p) * d.Q + q] = a[i];
        } else {
          float *dst = C + (int64_t)p * d.ldc + q;
          float v = d.alpha * a[i];
          if (d.bias != nullptr) v = v + bq[bj];
          if (d.res != nullptr) v = v + rv[blk][i];
          v = d.accumulate ? *dst + v : v;
          if constexpr (ACT) {
            if (d.pre != nullptr) d.pre[(int64_t)p * d.ldc + q] = v;
            v = act_value(d.act, v);
          }
          *dst = v;
        }
      }
    }
  }
}

// One split product's reduction: C = alpha * sum_s partial[s] (+ bias[q])
// (+ C), partial s at partial + s*n with row stride Q.
struct SplitSet {
  const float *partial;
  float *C;
  const float *bias;
  int64_t ldc, n;
  int Q, splits, acc;
  float alpha;
  int act;     // activation applied last (Gemm::act)
  float *pre;  // optional pre-activation output (row stride ldc)
  const float *res;  // residual added after the bias (row stride ldr)
  int64_t ldr;
  int kahan;  // the splits added as a compensated (Kahan) sum, in the same order
};

// Column sums out[c] (+)= sum_r g[r ldg + c] of a [rows, cols] block in one
// pass (the Linear backward's bias gradient, carried by the launch that
// reduces the weight gradient's splits).  A workgroup owns eight columns
// (two float4 groups; cols % 4 == 0, a last group past the end is skipped)
// and 128 row classes: thread k reads chunk k % 2 of rows k / 2, k / 2 + 128,
// ... and adds them in order, 16 loads in flight; the 128 class sums of a
// column are then added through LDS in a fixed order (32 sums of four
// consecutive classes, then those 32 in order) -- deterministic.  Two lanes
// read 32 contiguous bytes of a row (four columns per workgroup, one lane
// per row, measured 12.3 against 9.6 us for [4096, 1536]).  Consecutive
// column groups run on one XCD, so the workgroups that share a cache line
// read it through the same L2.
struct ColSum {
  const float *g;
  float *out;
  int64_t rows, cols, ldg;
  int acc;
  const float *mask;  // tiny kernel only (see tiny_colsum)
};
constexpr int kColSumCols = 8;
constexpr int kColSumLanes = kColSumCols / 4;       // lanes reading one row's columns
constexpr int kColSumClasses = 256 / kColSumLanes;  // row classes of a workgroup

// Column groups of a [., cols] block.
__host__ __device__ inline int64_t colsum_groups(int64_t cols) { return (cols + kColSumCols - 1) / kColSumCols; }

// Threads past the first 256 of a larger workgroup only meet the barriers.
__device__ __forceinline__ void colsum_block(const ColSum &c, int64_t blk) {
  __shared__ f4 red[256];
  const int k = threadIdx.x;
  const int j = k % kColSumLanes, rc = k / kColSumLanes;  // column chunk, row class
  const float *p = c.g + blk * kColSumCols + 4 * j;
  const bool live = k < 256 && blk * kColSumCols + 4 * j < c.cols;
  f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t r0 = rc; live && r0 < c.rows; r0 += kColSumClasses * 16) {
    f4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t r = r0 + kColSumClasses * u;
      v[u] = r < c.rows ? *reinterpret_cast<const f4 *>(p + r * c.ldg) : f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) s += v[u];
  }
  if (k < 256) red[k] = s;  // k = kColSumLanes * class + chunk
  __syncthreads();
  // 64 partials: chunk t % lanes, classes 4 (t / lanes) .. + 3, added in order
  f4 t = {0.0f, 0.0f, 0.0f, 0.0f};
  if (k < 64) {
    const int jj = k % kColSumLanes, g = k / kColSumLanes;
    t = ((red[kColSumLanes * (4 * g) + jj] + red[kColSumLanes * (4 * g + 1) + jj]) +
         red[kColSumLanes * (4 * g + 2) + jj]) +
        red[kColSumLanes * (4 * g + 3) + jj];
  }
  __syncthreads();
  if (k < 64) red[k] = t;
  __syncthreads();
  const int64_t gc = blk * kColSumCols + k;
  if (k < kColSumCols && gc < c.cols) {
    const int jj = k / 4, e = k % 4;
    float u = 0.0f;
    for (int g = 0; g < 64 / kColSumLanes; ++g) u += red[kColSumLanes * g + jj][e];
    c.out[gc] = c.acc ? c.out[gc] + u : u;
  }
}

// Workgroup b of a launch row of n workgroups (hardware ids go to the eight
// XCDs in turn, n % 8 == 0) -> column group, so that XCD x owns groups
// [x m/8, (x+1) m/8) of the m groups; -1 for a workgroup with no group.
__device__ __forceinline__ int64_t colsum_group(int b, int n, int64_t m) {
  if ((n & 7) != 0 || (m & 7) != 0) return b < m ? b : -1;
  const int64_t idx = b >> 3;
  return idx < (m >> 3) ? (b & 7) * (m >> 3) + idx : -1;
}

// Adds the splits' values v[0..n) to the running sum s in split order, plain
// or compensated (kahan): the operations of splitk_reduce's loop, for the
// reductions made inside a product's launch (Fused).
template <class V, int N>
__device__ __forceinline__ void add_splits(int kahan, V &s, V &comp, const V (&v)[N], int n) {
  if (kahan) {
#pragma unroll
    for (int u = 0; u < N; ++u)
      if (u < n) {
        const V y = v[u] - comp;
        const V t = s + y;
        comp = (t - s) - y;
        s = t;
      }
  } else {
#pragma unroll
    for (int u = 0; u < N; ++u)
      if (u < n) s += v[u];
  }
}

// The end of a split reduction at C[p, q..]: alpha, bias, residual,
// accumulate, activation (pre-activation stored first) -- splitk_reduce's
// epilogue, operation for operation.  Takes the set's fields one by one (a
// reference to a kernel argument, once inlined, had fields copied to private
// memory).  splitk_reduce keeps its own copy of this arithmetic: with these
// helpers inlined its set selection was promoted to LDS.
template <class V>
__device__ __forceinline__ void finish_split(float *C, int64_t ldc, const float *bias,
                                             const float *res, int64_t ldr, int acc, float alpha,
                                             int act, float *pre, int64_t p, int64_t q, V s) {
  V *dst = reinterpret_cast<V *>(C + p * ldc + q);
  V v = alpha * s;
  if (bias != nullptr) v = v + *reinterpret_cast<const V *>(bias + q);
  if (res != nullptr) v = v + *reinterpret_cast<const V *>(res + p * ldr + q);
  v = acc ? *dst + v : v;
  if (act) {
    if (pre != nullptr) *reinterpret_cast<V *>(pre + p * ldc + q) = v;
    if constexpr (std::is_same<V, f4>::value) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act_value(act, v[e]);
    } else {
      v = act_value(act, v);
    }
  }
  *dst = v;
}
#define NRS_FINISH_SPLIT(d, p, q, s) \
  finish_split((d).C, (d).ldc, (d).bias, (d).res, (d).ldr, (d).acc, (d).alpha, (d).act, (d).pre, p, q, s)

// Splits are added in order s = 0, 1, ... (deterministic); the loads of a
// batch of splits are issued before its ordered adds.  With column sums
// (has_cs), row y = 0 of the grid computes them and rows 1, 2, 3 reduce the
// sets; otherwise rows 0, 1, 2 reduce the sets.  The column sums (one
// long strided walk per workgroup) go first so that they are dispatched
// before, and overlap, the short split reductions.  VEC: four consecutive
// elements of one row per thread (Q, ldc and the pointers 16-byte aligned).
template <bool VEC>
__global__ void __launch_bounds__(256) splitk_reduce(SplitSet s0, SplitSet s1, SplitSet s2,
                                                     ColSum cs, int has_cs) {
  if (has_cs && blockIdx.y == 0) {
    const int64_t grp = colsum_group(blockIdx.x, gridDim.x, colsum_groups(cs.cols));
    if (grp >= 0) colsum_block(cs, grp);
    return;
  }
  const int y = (int)blockIdx.y - has_cs;
  const SplitSet &d = y == 0 ? s0 : y == 1 ? s1 : s2;
  typedef typename std::conditional<VEC, f4, float>::type V;
  constexpr int kW = VEC ? 4 : 1;
  constexpr int kBatch = VEC ? 4 : 8;
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * kW;
  if (e >= d.n) return;
  V s = V{}, comp = V{};
  for (int k0 = 0; k0 < d.splits; k0 += kBatch) {
    V v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < d.splits) v[u] = *reinterpret_cast<const V *>(d.partial + (k0 + u) * d.n + e);
    if (d.kahan) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k0 + u < d.splits) {
          const V y = v[u] - comp;
          const V t = s + y;
          comp = (t - s) - y;
          s = t;
        }
    } else {
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k0 + u < d.splits) s += v[u];
    }
  }
  const int64_t p = e / d.Q, q = e - p * d.Q;
  V *dst = reinterpret_cast<V *>(d.C + p * d.ldc + q);
  V v = d.alpha * s;
  if (d.bias != nullptr) v = v + *reinterpret_cast<const V *>(d.bias + q);
  if (d.res != nullptr) v = v + *reinterpret_cast<const V *>(d.res + p * d.ldr + q);
  v = d.acc ? *dst + v : v;
  if (d.act) {
    if (d.pre != nullptr) *reinterpret_cast<V *>(d.pre + p * d.ldc + q) = v;
    if constexpr (VEC) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act_value(d.act, v[e]);
    } else {
      v = act_value(d.act, v);
    }
  }
  *dst = v;
}

// Maps the hardware workgroup id to a logical tile so that XCD k (which
// receives ids k, k+8, k+16, ...) owns logical tiles [k*n/8, (k+1)*n/8).
__device__ __forceinline__ int xcd_tile(int b, int n) {
  if ((n & 7) != 0) return b;
  return (b & 7) * (n >> 3) + (b >> 3);
}

template <bool XRC, bool YRC, bool VEC, bool ACT = false>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(Gemm d) {
  __shared__ __attribute__((aligned(16))) float smem[4 * kTileFloats];
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  gemm_tile<XRC, YRC, VEC, ACT>(d, tile, blockIdx.y, smem);
}

// Two products in one grid: logical tiles [0, tiles_a) belong to `a`, the
// rest to `b`.  matmul_backward: dA = dC B^T (NT) with dB = A^T dC (TN);
// the Linear backward: dx = g W (NN) with dW = g^T x (TN).
template <bool XRC_A, bool YRC_A, bool VEC>
__global__ void __launch_bounds__(kThreads, 2) gemm_pair_kernel(Gemm a, Gemm b, int tiles_a) {
  __shared__ __attribute__((aligned(16))) float smem[4 * kTileFloats];
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  if (tile < tiles_a)
    gemm_tile<XRC_A, YRC_A, VEC>(a, tile, blockIdx.y, smem);
  else
    gemm_tile<false, false, VEC>(b, tile - tiles_a, blockIdx.y, smem);
}

template <bool VEC>
__global__ void __launch_bounds__(kThreads, 2) matmul_backward_kernel(Gemm da, Gemm db, int tiles_a) {
  __shared__ __attribute__((aligned(16))) float smem[4 * kTileFloats];
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  if (tile < tiles_a)
    gemm_tile<true, true, VEC>(da, tile, blockIdx.y, smem);
  else
    gemm_tile<false, false, VEC>(db, tile - tiles_a, blockIdx.y, smem);
}

// ---------------------------------------------------------------------------
// Streamed large-tile path, for aligned products with at least one output
// tile per CU (matmul_backward at 2048^2 and up).
//   * Workgroup tile 256(P) x 128(Q), one workgroup per CU with eight waves
//     (two per SIMD); each wave owns 64 x 64 = 2 x 2 MFMA blocks.
//   * Operands go global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging, no ds_write) into a three-stage ring of 48 KiB stages: the
//     tile used at step kt was issued right after the barrier that ended
//     step kt-3's reads, two tiles ahead.  One barrier per reduction tile.
//   * A DMA instruction writes 1 KiB contiguously, so the LDS layouts are
//     XOR-swizzled instead of padded: an R-contiguous tile is [p][32] with
//     16-byte chunk c stored at c ^ ((p & 7) ^ ((p >> 3) & 1)); a
//     P-contiguous tile is [32][EXT] with column bit 5 flipped on rows whose
//     bit 2 is set.  Both keep the fragment reads free of bank conflicts.
//   * Two-level accumulation with the MFMA partials added into the running
//     totals every three reduction tiles (96 reduction steps).
//   * A small-tile variant (128 x 64, 24 KiB stages, two workgroups per CU,
//     each wave 64 x 32 = 2 x 1 MFMA blocks) serves products whose output is
//     too small to give every CU a large tile's worth of work; the split
//     planner picks the tile and the split-K ranges per product.
// Requires P % TP == 0, Q % TQ == 0, R % 32 == 0 and vec_ok operands.
// ---------------------------------------------------------------------------
constexpr int kSP = 256, kSQ = 128;  // large workgroup tile
constexpr int kHP = 128, kHQ = 64;   // small workgroup tile
constexpr int kMP = 64, kMQ = 64;    // mini workgroup tile (batched products, up to 3 per CU)
// Wide workgroup tile: eight waves of 32 x 96 (three MFMA blocks each), for
// single products with both operands reduction-contiguous whose outputs are
// a multiple of 192 wide -- the packed q/k/v projection's [4096, 1536] is
// exactly 256 of them, one round on 256 CUs, where its 768 small tiles need
// a round and a half.
constexpr int kWP = 128, kWQ = 192;
// Streamed tile shapes, as the planners name them.
constexpr int kShapeLarge = 0, kShapeSmall = 1, kShapeMini = 2;
template <int TP, int TQ, int NW = 4>
struct StreamCfg {
  static constexpr int kStageX = TP * kBR;  // floats per X stage
  static constexpr int kStageY = TQ * kBR;  // floats per Y stage
  // DMA instructions (1 KiB each) per wave per reduction tile
  static constexpr int kDma = (TP + TQ) * kBR / 256 / NW;
  // waves form an (NW/2) x 2 grid; each owns kWP x TQ/2 outputs
  static constexpr int kWP = TP / (NW / 2);
  static constexpr int kBI = kWP / 32, kBJ = TQ / 64;  // 32 x 32 MFMA blocks per wave
};

using numrs_hip::lds_dma16;
using numrs_hip::wait_vm;

static_assert(wait_vm(0) == 0x3f70 && wait_vm(12) == 0x3f7c && wait_vm(24) == 0x7f78,
              "vmcnt immediate encoding");
static_assert(2 * StreamCfg<kSP, kSQ>::kDma < 64, "vmcnt is 6 bits");

// Three LDS stages per tile size, as distinct objects so that every stage
// address folds to a constant (the DMA's M0 value is then a scalar move).
__shared__ __attribute__((aligned(1024))) float g_sx0[StreamCfg<kSP, kSQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_sy0[StreamCfg<kSP, kSQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_sx1[StreamCfg<kSP, kSQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_sy1[StreamCfg<kSP, kSQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_sx2[StreamCfg<kSP, kSQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_sy2[StreamCfg<kSP, kSQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_hx0[StreamCfg<kHP, kHQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_hy0[StreamCfg<kHP, kHQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_hx1[StreamCfg<kHP, kHQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_hy1[StreamCfg<kHP, kHQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_hx2[StreamCfg<kHP, kHQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_hy2[StreamCfg<kHP, kHQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_wx0[StreamCfg<kWP, kWQ, 8>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_wy0[StreamCfg<kWP, kWQ, 8>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_wx1[StreamCfg<kWP, kWQ, 8>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_wy1[StreamCfg<kWP, kWQ, 8>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_wx2[StreamCfg<kWP, kWQ, 8>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_wy2[StreamCfg<kWP, kWQ, 8>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_mx0[StreamCfg<kMP, kMQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_my0[StreamCfg<kMP, kMQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_mx1[StreamCfg<kMP, kMQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_my1[StreamCfg<kMP, kMQ>::kStageY];
__shared__ __attribute__((aligned(1024))) float g_mx2[StreamCfg<kMP, kMQ>::kStageX];
__shared__ __attribute__((aligned(1024))) float g_my2[StreamCfg<kMP, kMQ>::kStageY];

__device__ __forceinline__ int rc_swizzle(int p) { return (p & 7) ^ ((p >> 3) & 1); }

// This wave's share of the EXT/8 DMA instructions for one EXT x 32 operand
// tile (each instruction: 64 lanes x 16 bytes = 1 KiB of LDS at stage byte
// address lds + 1024 m), NW waves per workgroup.  The per-lane source
// offsets do not change along the reduction: stream_offsets computes them
// once, in bytes from the tile's uniform base (row p0 for an R-contiguous
// operand, column p0 otherwise, at reduction tile 0), and stream_issue adds
// the reduction tile to the base.
template <int EXT, int NW>
struct StreamSlots {
  static constexpr int kPerWave = EXT / (8 * NW);
  static_assert(kPerWave >= 1 && kPerWave * 8 * NW == EXT, "DMA split across waves");
  uint32_t off[kPerWave];
};

template <bool RC, int EXT, int NW>
__device__ __forceinline__ void stream_offsets(StreamSlots<EXT, NW> &sl, int64_t ld, int wave,
                                               int lane) {
#pragma unroll
  for (int i = 0; i < StreamSlots<EXT, NW>::kPerWave; ++i) {
    const int m = wave * StreamSlots<EXT, NW>::kPerWave + i;
    if (RC) {  // 8 rows of 32 floats per instruction
      const int p = 8 * m + (lane >> 3);
      const int k = (lane & 7) ^ rc_swizzle(p);
      sl.off[i] = (uint32_t)(4 * ((int64_t)p * ld + 4 * k));
    } else {  // 1024 / (4 EXT) rows of EXT floats per instruction
      constexpr int kChunks = EXT / 4;
      const int r = m * (64 / kChunks) + lane / kChunks;
      const int lc = (lane % kChunks) ^ (((r >> 2) & 1) << 3);
      sl.off[i] = (uint32_t)(4 * ((int64_t)r * ld + 4 * lc));
    }
  }
}

// base: the operand's uniform tile base advanced to the reduction tile;
// lds: the stage's byte address; wave_u: the wave index as a uniform value.
template <int EXT, int NW>
__device__ __forceinline__ void stream_issue(const StreamSlots<EXT, NW> &sl, const float *base,
                                             uint32_t lds, uint32_t wave_u) {
  constexpr int kPerWave = StreamSlots<EXT, NW>::kPerWave;
#pragma unroll
  for (int i = 0; i < kPerWave; ++i)
    lds_dma16(base, sl.off[i], lds + 1024u * (wave_u * kPerWave + i));
}

// Fragment of MFMA group g (reduction indices 8g + 4h + j) for rows
// pb + c of a swizzled tile; same lane contract as frag().
template <bool RC, int EXT>
__device__ __forceinline__ f4 stream_frag(const float *lds, int pb, int c, int h, int g) {
  if (RC) {
    const int p = pb + c;
    const int cp = (2 * g + h) ^ rc_swizzle(p);
    return *reinterpret_cast<const f4 *>(lds + p * 32 + cp * 4);
  } else {
    f4 f;
    const int col = (pb + c) ^ (h << 5);
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = lds[(8 * g + 4 * h + j) * EXT + col];
    return f;
  }
}

template <int BI, int BJ>
struct StreamFrags {
  f4 a[BI], b[BJ];
};

template <bool XRC, bool YRC, int TP, int TQ, int NW>
__device__ __forceinline__ void stream_read(
    StreamFrags<StreamCfg<TP, TQ, NW>::kBI, StreamCfg<TP, TQ, NW>::kBJ> &f, const float *xl,
    const float *yl, int wp, int wq, int c, int h, int g) {
  using Cfg = StreamCfg<TP, TQ, NW>;
#pragma unroll
  for (int i = 0; i < Cfg::kBI; ++i)
    f.a[i] = stream_frag<XRC, TP>(xl, wp * Cfg::kWP + 32 * i, c, h, g);
#pragma unroll
  for (int j = 0; j < Cfg::kBJ; ++j)
    f.b[j] = stream_frag<YRC, TQ>(yl, wq * (TQ / 2) + 32 * j, c, h, g);
}

// Output tile (tp, tq) of logical tile `tile`: tiles run in groups of
// kGroupRows tile rows, column by column within a group.
__device__ __forceinline__ void tile_rc(int tiles_p, int tiles_q, int tile, int &tp, int &tq) {
  const int per_group = kGroupRows * tiles_q;
  const int gidx = tile / per_group;
  const int first_p = gidx * kGroupRows;
  const int rows_in_group = min(tiles_p - first_p, kGroupRows);
  const int in_group = tile - gidx * per_group;
  tp = first_p + in_group % rows_in_group;
  tq = in_group / rows_in_group;
}

// ACT: the epilogue applies d.act (and stores d.pre); a separate
// instantiation, so products without an activation keep the plain epilogue.
// FUSE (the fused launches of Fused, whose split products carry d.arrive):
// returns -1, or, for a split whose partial completed the arrivals at some of
// its tile's sub-blocks, (output tile << 8) | mask of those sub-blocks, which
// the caller then reduces.  Without FUSE, -1.
template <bool XRC, bool YRC, int TP, int TQ, int NW = 4, bool ACT = false, bool FUSE = false>
__device__ __forceinline__ int stream_tile(const Gemm &d, int tile, int batch) {
  using Cfg = StreamCfg<TP, TQ, NW>;
  constexpr int kBI = Cfg::kBI, kBJ = Cfg::kBJ, kDma = Cfg::kDma;
  // Split-K: consecutive logical tiles are the k-ranges of one output tile
  // (the planner leaves no range empty).
  const int split = tile % d.splits;
  tile /= d.splits;
  int tp, tq;
  tile_rc(d.tiles_p, d.tiles_q, tile, tp, tq);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wp = wave >> 1, wq = wave & 1;
  const int c = lane & 31, h = lane >> 5;
  const int p0 = tp * TP, q0 = tq * TQ;

  const int64_t zo = batch / d.binner, zi = batch - zo * d.binner;
  const float *__restrict__ X = d.X + zo * d.bsx + zi * d.bsx2;
  const float *__restrict__ Y = d.Y + zo * d.bsy + zi * d.bsy2;
  float *__restrict__ C = d.C + zo * d.bsc + zi * d.bsc2;
  int64_t ldc = d.ldc;
  const int kt0 = split * d.ktiles_per_split;
  const int nk = min(d.R / kBR - kt0, d.ktiles_per_split);
  X += XRC ? (int64_t)kt0 * kBR : (int64_t)kt0 * kBR * d.ldx;
  Y += YRC ? (int64_t)kt0 * kBR : (int64_t)kt0 * kBR * d.ldy;
  const bool part = d.splits > 1;
  if (part) {  // plain partial product, row stride Q; splitk_reduce finishes
    C = d.partial + (int64_t)split * d.P * d.Q;
    ldc = d.Q;
  }

  float *x0, *x1, *x2, *y0, *y1, *y2;
  if constexpr (TP == kSP) {
    x0 = g_sx0, x1 = g_sx1, x2 = g_sx2;
    y0 = g_sy0, y1 = g_sy1, y2 = g_sy2;
  } else if constexpr (TQ == kWQ) {
    static_assert(XRC && YRC, "wide tiles: reduction-contiguous operands only");
    x0 = g_wx0, x1 = g_wx1, x2 = g_wx2;
    y0 = g_wy0, y1 = g_wy1, y2 = g_wy2;
  } else if constexpr (TP == kHP) {
    x0 = g_hx0, x1 = g_hx1, x2 = g_hx2;
    y0 = g_hy0, y1 = g_hy1, y2 = g_hy2;
  } else {
    x0 = g_mx0, x1 = g_mx1, x2 = g_mx2;
    y0 = g_my0, y1 = g_my1, y2 = g_my2;
  }

  // DMA sources: uniform tile bases (advanced by xstep / ystep floats per
  // reduction tile) plus per-lane byte offsets fixed for the whole reduction.
  const float *Xb = X + (XRC ? (int64_t)p0 * d.ldx : (int64_t)p0);
  const float *Yb = Y + (YRC ? (int64_t)q0 * d.ldy : (int64_t)q0);
  const int64_t xstep = XRC ? kBR : (int64_t)kBR * d.ldx;
  const int64_t ystep = YRC ? kBR : (int64_t)kBR * d.ldy;
  StreamSlots<TP, NW> xs;
  StreamSlots<TQ, NW> ys;
  stream_offsets<XRC>(xs, d.ldx, wave, lane);
  stream_offsets<YRC>(ys, d.ldy, wave, lane);
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Stage byte addresses in LDS: the low 32 bits of a generic pointer into
  // the shared aperture are its LDS offset.
  auto lds_addr = [](const float *p) { return (uint32_t)(uintptr_t)p; };
  auto issue = [&](int t, const float *xl, const float *yl) {
    stream_issue<TP, NW>(xs, Xb + t * xstep, lds_addr(xl), wave_u);
    stream_issue<TQ, NW>(ys, Yb + t * ystep, lds_addr(yl), wave_u);
  };

  // Prologue: tiles 0, 1, 2 into stages 0, 1, 2; wait for tile 0.
  issue(0, x0, y0);
  if (nk > 1) issue(1, x1, y1);
  if (nk > 2) {
    issue(2, x2, y2);
    __builtin_amdgcn_s_waitcnt(wait_vm(2 * kDma));  // tile 0 landed, 1 and 2 may fly
  } else if (nk > 1) {
    __builtin_amdgcn_s_waitcnt(wait_vm(kDma));
  } else {
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
  }
  __syncthreads();

  f16v acc[kBI][kBJ], tot[kBI][kBJ];
#pragma unroll
  for (int i = 0; i < kBI; ++i)
#pragma unroll
    for (int j = 0; j < kBJ; ++j) {
      acc[i][j] = f16v{};
      tot[i][j] = f16v{};
    }
  StreamFrags<kBI, kBJ> cur, nxt;
  stream_read<XRC, YRC, TP, TQ, NW>(cur, x0, y0, wp, wq, c, h, 0);

  // One reduction tile kt held in (xl, yl); (xn, yn) holds tile kt+1.  Group
  // g's MFMAs run while group g+1's fragments load; before the last group
  // the barrier ends this tile's reads, tile kt+3 is issued into (xl, yl)
  // and tile kt+1's first fragments are read.  The flags (compile-time, so
  // the stages stay distinct objects for the waitcnt model) say whether
  // tile kt+1 exists, whether tile kt+2 is still in flight, and whether
  // tile kt+3 exists.
  auto step = [&](auto next_t, auto two_t, auto issue_t, int kt, float *xl, float *yl, float *xn,
                  float *yn) {
    constexpr bool kNext = decltype(next_t)::value;
    constexpr bool kTwo = decltype(two_t)::value;
    constexpr bool kIssue = decltype(issue_t)::value;
#pragma unroll
    for (int g = 0; g < kBR / 8; ++g) {
      if (g < kBR / 8 - 1) {
        stream_read<XRC, YRC, TP, TQ, NW>(nxt, xl, yl, wp, wq, c, h, g + 1);
        __builtin_amdgcn_sched_barrier(0);
      } else if (kNext) {
        if (kTwo)
          __builtin_amdgcn_s_waitcnt(wait_vm(kDma));  // tile kt+1 landed, kt+2 may fly
        else
          __builtin_amdgcn_s_waitcnt(wait_vm(0));
        __syncthreads();
        if (kIssue) {
          issue(kt + 3, xl, yl);
        }
        stream_read<XRC, YRC, TP, TQ, NW>(nxt, xn, yn, wp, wq, c, h, 0);
      }
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int i = 0; i < kBI; ++i)
#pragma unroll
          for (int j = 0; j < kBJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[i][sl], cur.b[j][sl], acc[i][j],
                                                            0, 0, 0);
      cur = nxt;
    }
  };
  auto flush = [&]() {
#pragma unroll
    for (int i = 0; i < kBI; ++i)
#pragma unroll
      for (int j = 0; j < kBJ; ++j) {
        tot[i][j] += acc[i][j];
        acc[i][j] = f16v{};
      }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  int kt = 0;
  for (; kt + 5 < nk; kt += 3) {
    step(T_{}, T_{}, T_{}, kt, x0, y0, x1, y1);
    step(T_{}, T_{}, T_{}, kt + 1, x1, y1, x2, y2);
    step(T_{}, T_{}, T_{}, kt + 2, x2, y2, x0, y0);
    flush();
  }
  // The last 1..5 tiles (kt is a multiple of 3, so tile kt sits in stage 0).
  switch (nk - kt) {
    case 5:
      step(T_{}, T_{}, T_{}, kt, x0, y0, x1, y1);
      step(T_{}, T_{}, T_{}, kt + 1, x1, y1, x2, y2);
      step(T_{}, T_{}, F_{}, kt + 2, x2, y2, x0, y0);
      step(T_{}, F_{}, F_{}, kt + 3, x0, y0, x1, y1);
      step(F_{}, F_{}, F_{}, kt + 4, x1, y1, x2, y2);
      break;
    case 4:
      step(T_{}, T_{}, T_{}, kt, x0, y0, x1, y1);
      step(T_{}, T_{}, F_{}, kt + 1, x1, y1, x2, y2);
      step(T_{}, F_{}, F_{}, kt + 2, x2, y2, x0, y0);
      step(F_{}, F_{}, F_{}, kt + 3, x0, y0, x1, y1);
      break;
    case 3:
      step(T_{}, T_{}, F_{}, kt, x0, y0, x1, y1);
      step(T_{}, F_{}, F_{}, kt + 1, x1, y1, x2, y2);
      step(F_{}, F_{}, F_{}, kt + 2, x2, y2, x0, y0);
      break;
    case 2:
      step(T_{}, F_{}, F_{}, kt, x0, y0, x1, y1);
      step(F_{}, F_{}, F_{}, kt + 1, x1, y1, x2, y2);
      break;
    default:
      step(F_{}, F_{}, F_{}, kt, x0, y0, x1, y1);
      break;
  }
  flush();

  // Residual values are all loaded (into the dead MFMA partials) before the
  // first store: res may alias C, which would otherwise order each load
  // after the previous store.
  const bool with_res = !part && d.res != nullptr;
  if (with_res) {
#pragma unroll
    for (int bi = 0; bi < kBI; ++bi)
#pragma unroll
      for (int bj = 0; bj < kBJ; ++bj) {
        const int q = q0 + wq * (TQ / 2) + bj * 32 + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int p = p0 + wp * Cfg::kWP + bi * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          acc[bi][bj][i] = d.res[(int64_t)p * d.ldr + q];
        }
      }
  }
  float bq[kBJ];  // this lane's bias columns, also read before any store
#pragma unroll
  for (int bj = 0; bj < kBJ; ++bj)
    bq[bj] = !part && d.bias != nullptr ? d.bias[q0 + wq * (TQ / 2) + bj * 32 + c] : 0.0f;
#pragma unroll
  for (int bi = 0; bi < kBI; ++bi)
#pragma unroll
    for (int bj = 0; bj < kBJ; ++bj) {
      const int q = q0 + wq * (TQ / 2) + bj * 32 + c;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int p = p0 + wp * Cfg::kWP + bi * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        float *dst = C + (int64_t)p * ldc + q;
        if (part) {
          if constexpr (FUSE)
            numrs_hip::st_dev(dst, tot[bi][bj][i]);  // read by another workgroup
          else
            *dst = tot[bi][bj][i];
        } else {
          float v = d.alpha * tot[bi][bj][i];
          if (d.bias != nullptr) v = v + bq[bj];
          if (with_res) v = v + acc[bi][bj][i];
          v = d.accumulate ? *dst + v : v;
          if constexpr (ACT) {
            if (d.pre != nullptr) d.pre[(int64_t)p * ldc + q] = v;
            v = act_value(d.act, v);
          }
          *dst = v;
        }
      }
    }
  if constexpr (!FUSE) {
    return -1;
  } else {
  if (!part) return -1;
  // Arrival: every lane's partial stores acknowledged at device scope, the
  // block met; then one counter per sub-block of this tile.  splits + 1
  // arrivals in all (the splits and the sub-block's reducer workgroup); the
  // last one reduces and sets the counter back to zero.
  __shared__ int s_arrived;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < 64) {
    bool last = false;
    if (threadIdx.x < 8) {
      unsigned *ctr = d.arrive + (int64_t)tile * 8 + threadIdx.x;
      last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)d.splits;
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const unsigned long long m = __ballot(last);
    if (threadIdx.x == 0) s_arrived = (int)(m & 0xffu);
  }
  __syncthreads();
  const int mask = s_arrived;
  return mask != 0 ? (tile << 8) | mask : -1;
  }
}

// Large tiles run eight waves (two per SIMD, 64 x 64 outputs each): while
// one wave waits at the stage barrier or on its fragment reads, the other's
// MFMAs issue (measured 3-4% faster than four waves of 128 x 64 at 2048^3).
constexpr int kBigWaves = 8;
constexpr int kBigThreads = 64 * kBigWaves;

// ---------------------------------------------------------------------------
// Split products reduced inside their own launch.  A batch-1 streamed launch
// of products a and b may end its grid with tail workgroups after the n_units
// product workgroups:
//   * one reducer per (split product, output tile, sub-block of TP/8 rows);
//   * (padding to the next multiple of eight hardware ids, so that the
//     column sums start on XCD 0 as in splitk_reduce);
//   * the column sums `cs`, as splitk_reduce's grid row 0 forms them;
//   * an independent split set `extra` (row partials of an earlier kernel),
//     NT float4 groups per workgroup.
// Each split of a tile stores its partial with device-scope (write-through)
// stores, waits until they are acknowledged, and then adds one to the
// arrival counter of each of the tile's eight sub-blocks; each reducer adds
// one to its own.  Of the splits + 1 arrivals, the last reduces the
// sub-block -- normally the reducer, which is dispatched after every product
// workgroup; a split that arrives after it does the work itself -- and sets
// the counter back to zero, so the counters are zero again for the next
// launch (and for each replay of a recorded graph).  No workgroup waits for
// another.  The partials are read at device scope, added in split order by
// add_splits and finished by finish_split: the bits of splitk_reduce.
// Order of the grid: with exactly one product split (and both unit counts
// multiples of 8), the split units come first (each XCD its share), then the
// tail, then the unsplit units -- workgroups are dispatched in hardware-id
// order, so the reductions run on the CUs the splits free while the unsplit
// tiles still run elsewhere; otherwise the product units in xcd_tile's order
// and the tail after them.
struct Fused {
  int n_units;               // product workgroups; 0: not a fused launch
  int n_tail;                // tail workgroups (a multiple of 8 when first_n > 0)
  int first_n, first_base, rest_base;  // unit order (first_n = 0: xcd_tile)
  SplitSet set[2];           // the reductions of products a and b (splits 0: none)
  int tiles_p[2], tiles_q[2];
  unsigned *count[2];        // arrival counters, 8 per output tile
  int sub[2];                // reducer workgroups per set (8 per output tile)
  int pad;                   // idle tail workgroups before the column sums
  ColSum cs;
  int cs_wgs;                // column-sum workgroups (a multiple of 8 when the groups are)
  SplitSet extra;
  int extra_wgs;
};

// Hardware id b -> product unit, or -1 - (tail index).
__device__ __forceinline__ int fused_unit(int b, const Fused &f) {
  if (f.first_n <= 0) return b < f.n_units ? xcd_tile(b, f.n_units) : -1 - (b - f.n_units);
  if (b < f.first_n) return f.first_base + (b & 7) * (f.first_n >> 3) + (b >> 3);
  if (b < f.first_n + f.n_tail) return -1 - (b - f.first_n);
  const int r = b - f.first_n - f.n_tail;  // r % 8 == b % 8: n_first and n_tail are multiples of 8
  return f.rest_base + (r & 7) * ((f.n_units - f.first_n) >> 3) + (r >> 3);
}

// Sub-block j of output tile `tile` of a split set: NT threads, each a float4
// group of the sub-block's TP/8 rows x TQ columns per pass.
template <int TP, int TQ, int NT>
__device__ __forceinline__ void fused_reduce_sub(const SplitSet &d, int tiles_p, int tiles_q, int tile, int j) {
  int tp, tq;
  tile_rc(tiles_p, tiles_q, tile, tp, tq);
  constexpr int kRows = TP / 8, kC4 = TQ / 4, kF4 = kRows * kC4;
  constexpr int kPass = (kF4 + NT - 1) / NT;  // float4 groups per thread
  constexpr int kBatch = 8;                  // splits loaded together
  const __amdgpu_buffer_rsrc_t rs = numrs_hip::dev_rsrc(d.partial, (int64_t)d.splits * d.n * 4);
  int64_t p[kPass], q[kPass], e[kPass];
  f4 s[kPass], comp[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int f = threadIdx.x + i * NT;
    const int r = f / kC4, c4 = f - r * kC4;
    p[i] = (int64_t)tp * TP + j * kRows + r;
    q[i] = (int64_t)tq * TQ + 4 * c4;
    e[i] = p[i] * d.Q + q[i];
    s[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    comp[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  for (int k0 = 0; k0 < d.splits; k0 += kBatch) {
    f4 v[kPass][kBatch];
#pragma unroll
    for (int i = 0; i < kPass; ++i)
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k0 + u < d.splits && threadIdx.x + i * NT < kF4)
          v[i][u] = numrs_hip::ld_dev4(rs, (int)(4 * ((k0 + u) * d.n + e[i])));
#pragma unroll
    for (int i = 0; i < kPass; ++i) add_splits(d.kahan, s[i], comp[i], v[i], d.splits - k0);
  }
#pragma unroll
  for (int i = 0; i < kPass; ++i)
    if (threadIdx.x + i * NT < kF4) NRS_FINISH_SPLIT(d, p[i], q[i], s[i]);
}

// The sub-blocks in `mask` of the output tile in `r` (stream_tile's return).
template <int TP, int TQ, int NT>
__device__ __forceinline__ void fused_reduce_mask(const Fused &f, int set, int r) {
  const int tile = r >> 8;
  for (int j = 0; j < 8; ++j)
    if ((r >> j) & 1) fused_reduce_sub<TP, TQ, NT>(f.set[set], f.tiles_p[set], f.tiles_q[set], tile, j);
}

// A reducer's arrival: true for the last of the splits + 1 arrivals.
__device__ __forceinline__ bool fused_arrive(unsigned *ctr, int splits) {
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    const bool last =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)splits;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  return s_last != 0;
}

// Tail workgroup u (hardware id n_units + u).
template <int TP, int TQ, int NT>
__device__ __forceinline__ void fused_tail(const Fused &f, int u) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (u < f.sub[k]) {
      if (fused_arrive(f.count[k] + u, f.set[k].splits))
        fused_reduce_sub<TP, TQ, NT>(f.set[k], f.tiles_p[k], f.tiles_q[k], u >> 3, u & 7);
      return;
    }
    u -= f.sub[k];
  }
  if (u < f.pad) return;
  u -= f.pad;
  if (u < f.cs_wgs) {
    const int64_t grp = colsum_group(u, f.cs_wgs, colsum_groups(f.cs.cols));
    if (grp >= 0) colsum_block(f.cs, grp);
    return;
  }
  u -= f.cs_wgs;
  if (u < f.extra_wgs) {
    const SplitSet &d = f.extra;
    const int64_t e = ((int64_t)u * NT + threadIdx.x) * 4;
    if (e < d.n) {
      f4 s = {0.0f, 0.0f, 0.0f, 0.0f}, comp = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k0 = 0; k0 < d.splits; k0 += 4) {
        f4 v[4];
#pragma unroll
        for (int w = 0; w < 4; ++w)
          if (k0 + w < d.splits) v[w] = *reinterpret_cast<const f4 *>(d.partial + (k0 + w) * d.n + e);
        add_splits(d.kahan, s, comp, v, d.splits - k0);
      }
      const int64_t p = e / d.Q, q = e - p * d.Q;
      NRS_FINISH_SPLIT(d, p, q, s);
    }
  }
}

// A pair kernel's body: the fused tail, or product a's tiles [0, tiles_a)
// then product b's (with a fused launch's reductions for sets 0 and 1).
template <bool XA, bool YA, int TP, int TQ, int NW, int NT, bool FUSE>
__device__ __forceinline__ void pair_body(const Gemm &a, const Gemm &b, int tiles_a, const Fused &f,
                                          int tile, int batch) {
  if (tile < tiles_a) {
    const int r = stream_tile<XA, YA, TP, TQ, NW, false, FUSE>(a, tile, batch);
    if constexpr (FUSE)
      if (r >= 0) fused_reduce_mask<TP, TQ, NT>(f, 0, r);
  } else {
    const int r = stream_tile<false, false, TP, TQ, NW, false, FUSE>(b, tile - tiles_a, batch);
    if constexpr (FUSE)
      if (r >= 0) fused_reduce_mask<TP, TQ, NT>(f, 1, r);
  }
}

template <bool XRC, bool YRC, bool ACT = false>
__global__ void __launch_bounds__(kBigThreads, 1) gemm_stream_kernel(Gemm d) {
  stream_tile<XRC, YRC, kSP, kSQ, kBigWaves, ACT>(d, xcd_tile(blockIdx.x, gridDim.x),
                                                  blockIdx.y);
}

template <bool ACT = false>
__global__ void __launch_bounds__(kBigThreads, 1) gemm_stream_wide(Gemm d) {
  stream_tile<true, true, kWP, kWQ, 8, ACT>(d, xcd_tile(blockIdx.x, gridDim.x), blockIdx.y);
}

template <bool XRC, bool YRC, bool ACT = false>
__global__ void __launch_bounds__(kThreads, 2) gemm_stream_small(Gemm d) {
  stream_tile<XRC, YRC, kHP, kHQ, 4, ACT>(d, xcd_tile(blockIdx.x, gridDim.x), blockIdx.y);
}

// Mini tiles (64 x 64, 16 KiB stages, three workgroups per CU, each wave one
// 32 x 32 MFMA block) for batched products whose 128 x 64 tiles would leave
// CUs idle, such as attention's per-head [256, 64] products at C4.
template <bool XRC, bool YRC>
__global__ void __launch_bounds__(kThreads, 3) gemm_stream_mini(Gemm d) {
  stream_tile<XRC, YRC, kMP, kMQ>(d, xcd_tile(blockIdx.x, gridDim.x), blockIdx.y);
}

// Pairs on the streamed path, logical tiles [0, tiles_a) for the first
// product.  matmul_backward: dA = dC B^T (NT) with dB = A^T dC (TN); the
// Linear backward: dx = g W (NN) with dW = g^T x (TN).
// A pair kernel's workgroup: with f.n_units != 0 (batch 1) a fused launch,
// whose hardware ids past n_units are tail workgroups and whose product units
// follow fused_unit's order; otherwise xcd_tile's (plain) or
// xcd_tile_batch's (BATCHED) order.  False for a tail workgroup, which has
// then done its work.
template <int TP, int TQ, int NT, bool BATCHED, bool FUSE>
__device__ __forceinline__ bool pair_unit(const Fused &f, int &tile, int &batch);

// FUSE: the fused launches' instantiation (Fused); the others keep the plain
// epilogue and order.
template <bool XA, bool YA, int TP, int TQ, int NW, int NT, bool BATCHED, bool FUSE>
__device__ __forceinline__ void pair_kernel_body(const Gemm &a, const Gemm &b, int tiles_a,
                                                 const Fused &f) {
  int tile, batch;
  if (!pair_unit<TP, TQ, NT, BATCHED, FUSE>(f, tile, batch)) return;
  // uniform by construction; said so, so that the DMA bases stay scalar
  tile = __builtin_amdgcn_readfirstlane(tile);
  batch = __builtin_amdgcn_readfirstlane(batch);
  pair_body<XA, YA, TP, TQ, NW, NT, FUSE>(a, b, tiles_a, f, tile, batch);
}

template <bool FUSE>
__global__ void __launch_bounds__(kBigThreads, 1)
    matmul_backward_stream(Gemm a, Gemm b, int tiles_a, Fused f) {
  pair_kernel_body<true, true, kSP, kSQ, kBigWaves, kBigThreads, false, FUSE>(a, b, tiles_a, f);
}

template <bool FUSE>
__global__ void __launch_bounds__(kThreads, 2)
    matmul_backward_stream_small(Gemm a, Gemm b, int tiles_a, Fused f) {
  pair_kernel_body<true, true, kHP, kHQ, 4, kThreads, false, FUSE>(a, b, tiles_a, f);
}

template <bool FUSE>
__global__ void __launch_bounds__(kBigThreads, 1)
    linear_backward_stream(Gemm a, Gemm b, int tiles_a, Fused f) {
  pair_kernel_body<true, false, kSP, kSQ, kBigWaves, kBigThreads, false, FUSE>(a, b, tiles_a, f);
}

template <bool FUSE>
__global__ void __launch_bounds__(kThreads, 2)
    linear_backward_stream_small(Gemm a, Gemm b, int tiles_a, Fused f) {
  pair_kernel_body<true, false, kHP, kHQ, 4, kThreads, false, FUSE>(a, b, tiles_a, f);
}

__global__ void __launch_bounds__(kThreads, 3) matmul_backward_stream_mini(Gemm da, Gemm db,
                                                                           int tiles_a) {
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  if (tile < tiles_a)
    stream_tile<true, true, kMP, kMQ>(da, tile, blockIdx.y);
  else
    stream_tile<false, false, kMP, kMQ>(db, tile - tiles_a, blockIdx.y);
}

__global__ void __launch_bounds__(kThreads, 3) linear_backward_stream_mini(Gemm dx, Gemm dw,
                                                                           int tiles_a) {
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  if (tile < tiles_a)
    stream_tile<true, false, kMP, kMQ>(dx, tile, blockIdx.y);
  else
    stream_tile<false, false, kMP, kMQ>(dw, tile - tiles_a, blockIdx.y);
}

// Maps the hardware workgroup (x fastest, XCD = linear id % 8) to a logical
// (tile, batch) so that XCD k owns the batch-major logical range
// [k*nb/8, (k+1)*nb/8): the tiles of one batch entry, which share operand
// panels, then run on one XCD and share its L2.
__device__ __forceinline__ void xcd_tile_batch(int &tile, int &batch) {
  const int nx = gridDim.x, nb = nx * gridDim.y, lin = blockIdx.x + nx * blockIdx.y;
  if ((nb & 7) != 0) {
    tile = xcd_tile(blockIdx.x, nx);
    batch = blockIdx.y;
    return;
  }
  const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
  tile = logical % nx;
  batch = logical / nx;
}

// Two transposed-left products in one launch (attention's dV = P^T dO with
// dK = alpha dS^T Q): both TN.
template <int TP, int TQ, int NT, bool BATCHED, bool FUSE>
__device__ __forceinline__ bool pair_unit(const Fused &f, int &tile, int &batch) {
  if constexpr (FUSE) {
    const int u = fused_unit(blockIdx.x, f);
    if (u < 0) {
      fused_tail<TP, TQ, NT>(f, -1 - u);
      return false;
    }
    tile = u;
    batch = 0;
  } else if (BATCHED) {
    xcd_tile_batch(tile, batch);
  } else {
    tile = xcd_tile(blockIdx.x, gridDim.x);
    batch = blockIdx.y;
  }
  return true;
}

template <bool FUSE>
__global__ void __launch_bounds__(kBigThreads, 1) tn_pair_stream(Gemm a, Gemm b, int tiles_a, Fused f) {
  pair_kernel_body<false, false, kSP, kSQ, kBigWaves, kBigThreads, true, FUSE>(a, b, tiles_a, f);
}

template <bool FUSE>
__global__ void __launch_bounds__(kThreads, 2) tn_pair_stream_small(Gemm a, Gemm b, int tiles_a,
                                                                    Fused f) {
  pair_kernel_body<false, false, kHP, kHQ, 4, kThreads, true, FUSE>(a, b, tiles_a, f);
}

__global__ void __launch_bounds__(kThreads, 3) tn_pair_stream_mini(Gemm a, Gemm b, int tiles_a) {
  int tile, batch;
  xcd_tile_batch(tile, batch);
  if (tile < tiles_a)
    stream_tile<false, false, kMP, kMQ>(a, tile, batch);
  else
    stream_tile<false, false, kMP, kMQ>(b, tile - tiles_a, batch);
}

int tiles(int64_t n) { return (int)((n + kBP - 1) / kBP); }

// Split-K plan for one product: a grid under 256 workgroups leaves most of
// the 256 CUs idle (a [512,512] weight gradient over 4096 tokens is 16
// tiles), so the reduction is split until the product has ~256 workgroups,
// keeping at least 8 k-tiles (256 reduction steps) per split.  Products of
// at most four output tiles (C1's layers: [64,784] x [784,128] is one tile
// over 25 k-tiles) split down to single k-tiles: their partials are small,
// and a lone workgroup walks its k-tiles one after another at about 3 us
// each on MI355X, against one splitk_reduce launch of about 4 us.  Batched
// products already fill the grid through their batch dimension.  The split
// count is recomputed from the k-tiles per split, so no range is empty.
int plan_splits(const Gemm &g, int64_t batch) {
  const int64_t t = (int64_t)g.tiles_p * g.tiles_q;
  const int nk = (g.R + kBR - 1) / kBR;
  if (batch != 1 || t >= 256) return 1;
  int64_t s = (256 + t - 1) / t;
  if (t <= 4 && nk >= 3) {
    s = std::min<int64_t>(s, nk);
  } else {
    if (nk < 16) return 1;
    s = std::min<int64_t>(s, nk / 8);
  }
  s = std::min<int64_t>(s, 32);
  if (s <= 1) return 1;
  const int64_t per = (nk + s - 1) / s;
  return (int)((nk + per - 1) / per);
}

void apply_splits(Gemm &g, int splits, float *partial) {
  const int nk = (g.R + kBR - 1) / kBR;
  g.splits = splits;
  g.ktiles_per_split = (nk + splits - 1) / splits;
  g.partial = partial;
}

// Whether the column sums of g [rows, cols] (row stride ldg) can ride in the
// split-reduce launch: float4 column groups and at most 8192 rows (a
// workgroup walks every row of its 16 columns).
bool colsum_fits(const float *g, int64_t rows, int64_t cols, int64_t ldg) {
  return cols % 4 == 0 && ldg % 4 == 0 && numrs_hip::aligned16(g) && rows <= 8192 &&
         cols / kColSumCols <= 0x7ffffff0;
}

// Reduces the split products among a and b (either may be null or unsplit)
// with one launch, which also forms the column sums `cs` when given and
// reduces the set `extra` (then the launch is made even when nothing was
// split).
int reduce_splits(numrs_hip_ctx *ctx, const Gemm *a, const Gemm *b, const ColSum *cs = nullptr,
                  const SplitSet *extra = nullptr) {
  const Gemm *g[2];
  int m = 0;
  if (a != nullptr && a->splits > 1) g[m++] = a;
  if (b != nullptr && b->splits > 1) g[m++] = b;
  if (m == 0 && cs == nullptr && extra == nullptr) return NUMRS_HIP_OK;
  SplitSet set[3] = {};
  bool vec = true;
  int64_t most = 0;
  for (int i = 0; i < m; ++i) {
    const Gemm &d = *g[i];
    set[i] = SplitSet{d.partial, d.C, d.bias, d.ldc, (int64_t)d.P * d.Q, d.Q, d.splits,
                      d.accumulate, d.alpha, d.act, d.pre, d.res, d.ldr};
  }
  if (extra != nullptr) set[m++] = *extra;
  for (int i = 0; i < m; ++i) {
    const SplitSet &d = set[i];
    vec = vec && d.Q % 4 == 0 && d.ldc % 4 == 0 && numrs_hip::aligned16(d.C) &&
          numrs_hip::aligned16(d.partial) && (d.bias == nullptr || numrs_hip::aligned16(d.bias)) &&
          (d.res == nullptr || (numrs_hip::aligned16(d.res) && d.ldr % 4 == 0)) &&
          (d.pre == nullptr || numrs_hip::aligned16(d.pre));
    most = std::max(most, d.n);
  }
  for (int i = m; i < 3; ++i) set[i] = set[0];
  int64_t blocks = (most / (vec ? 4 : 1) + 255) / 256;
  ColSum c{};
  const int has_cs = cs != nullptr ? 1 : 0;
  if (cs != nullptr) {
    c = *cs;
    blocks = std::max<int64_t>(blocks, colsum_groups(c.cols));
    blocks = (blocks + 7) & ~int64_t{7};  // whole rounds of the eight XCDs
  }
  if (blocks > 0x7fffffff)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "splitk_reduce: too large");
  dim3 grid((unsigned)std::max<int64_t>(blocks, 1), (unsigned)(m + has_cs));
  if (vec)
    splitk_reduce<true><<<grid, 256, 0, ctx->stream>>>(set[0], set[1], set[2], c, has_cs);
  else
    splitk_reduce<false><<<grid, 256, 0, ctx->stream>>>(set[0], set[1], set[2], c, has_cs);
  return numrs_hip::check_launch(ctx, "splitk_reduce");
}

// Vector (float4) loads need 16-byte aligned bases, leading dimensions and
// contiguous extents that are multiples of 4.
bool vec_ok(const Gemm &d, bool xrc, bool yrc) {
  auto ok = [](const void *p, int64_t ld, int64_t bs, int64_t bs2, int64_t contig) {
    return numrs_hip::aligned16(p) && (ld & 3) == 0 && (bs & 3) == 0 && (bs2 & 3) == 0 &&
           (contig & 3) == 0;
  };
  return ok(d.X, d.ldx, d.bsx, d.bsx2, xrc ? d.R : d.P) &&
         ok(d.Y, d.ldy, d.bsy, d.bsy2, yrc ? d.R : d.Q);
}

// ---------------------------------------------------------------------------
// Tiny products (a small batch's MLP layers: [64,784] x [784,128],
// [64,128] x [128,10] and their gradients).  128 x 128 tiles would leave all
// but a few CUs idle and walk the reduction serially, so a workgroup owns one
// 16 x 16 output block and its eight waves split the reduction: wave w takes
// the 16-wide reduction steps w, w + 8, ..., four v_mfma_f32_16x16x4f32 per
// step, with operands loaded straight from global memory (L2 serves the reuse
// across blocks); the eight partial blocks are then added in wave order
// through LDS -- deterministic.  One launch carries up to two products (a
// gradient pair) and the column sums of a bias gradient.
//   MFMA 16x16x4 lane contract (lane l = 16 g + i): A row i at reduction slot
//   g; B reduction slot g at column i; D column i, rows 4g + v (v = 0..3).
//   Reduction index k = 16 s + 4 g + j feeds MFMA j of step s at slot g, for
//   A and B alike.
constexpr int kTinyWaves = 8;
constexpr int kTinyThreads = 64 * kTinyWaves;
// Reduction steps per load batch and wave: 8 (143 VGPRs, one workgroup per
// CU) for reductions over 512, else 4 (79 VGPRs, three per CU).
constexpr int kTinyUBig = 8, kTinyUSmall = 4;
constexpr int kTinyColsumCols = 64;
constexpr int kTinyColsumRows = 8192;
constexpr int64_t kTinyMacs = int64_t{1} << 24;
constexpr int kTinyMaxR = 4096;  // at most four load batches per wave

// FUSE (batch 1, d.arrive set for a split product): a split stores its
// partial at device scope and arrives at its output block's counter; the
// last of the block's splits adds the block's partials in split order with
// splitk_reduce's arithmetic (add_splits, finish_split) and sets the counter
// back to zero -- no reduce launch, and no workgroup waits for another.
template <bool XRC, bool YRC, int U, bool FUSE = false>
__device__ __forceinline__ void tiny_tile(const Gemm &d, int tile, int batch) {
  // Split-K: consecutive logical blocks are the k-ranges of one output block.
  const int split = tile % d.splits;
  tile /= d.splits;
  const int tq_n = (d.Q + 15) >> 4;
  const int tp = tile / tq_n, tq = tile - tp * tq_n;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int p = tp * 16 + i, q = tq * 16 + i;
  const int64_t zo = batch / d.binner, zi = batch - zo * d.binner;
  const float *__restrict__ X = d.X + zo * d.bsx + zi * d.bsx2;
  const float *__restrict__ Y = d.Y + zo * d.bsy + zi * d.bsy2;
  float *__restrict__ C = d.C + zo * d.bsc + zi * d.bsc2;
  const float *__restrict__ M = d.xmask != nullptr ? d.xmask + zo * d.bsx + zi * d.bsx2 : nullptr;
  const bool pin = p < d.P, qin = q < d.Q;
  // This split's 16-wide reduction steps [s_lo, steps); k-tiles are 32 wide.
  const int s_lo = split * d.ktiles_per_split * 2;
  const int steps = min((d.R + 15) >> 4, s_lo + d.ktiles_per_split * 2);
  // Byte offsets from the (wave-uniform) operand bases fit in 32 bits
  // (tiny_fits), so each load needs one VGPR of address.
  const char *Xc = reinterpret_cast<const char *>(X), *Yc = reinterpret_cast<const char *>(Y);
  const char *Mc = reinterpret_cast<const char *>(M);
  const uint32_t ldx4 = 4u * (uint32_t)d.ldx, ldy4 = 4u * (uint32_t)d.ldy;
  const uint32_t xo = XRC ? (uint32_t)p * ldx4 : 4u * (uint32_t)p;  // reduction index 0
  const uint32_t yo = YRC ? (uint32_t)q * ldy4 : 4u * (uint32_t)q;
  const uint32_t xk = XRC ? 4u : ldx4, yk = YRC ? 4u : ldy4;  // bytes per reduction index
  auto ld = [](const char *base, uint32_t off) {
    return *reinterpret_cast<const float *>(base + off);
  };
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = s_lo + w; s0 < steps; s0 += kTinyWaves * U) {
    f4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + kTinyWaves * u;  // wave-uniform
      if (s < steps) {
        const int k = 16 * s + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool kin = k + j < d.R;
          const uint32_t xoff = xo + (uint32_t)(k + j) * xk;
          a[u][j] = pin && kin ? ld(Xc, xoff) : 0.0f;
          if (Mc != nullptr) a[u][j] = pin && kin && ld(Mc, xoff) > 0.0f ? a[u][j] : 0.0f;
          b[u][j] = qin && kin ? ld(Yc, yo + (uint32_t)(k + j) * yk) : 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s0 + kTinyWaves * u < steps)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][j], b[u][j], acc, 0, 0, 0);
  }
  __shared__ float part[kTinyWaves][256];
#pragma unroll
  for (int v = 0; v < 4; ++v) part[w][(4 * g + v) * 16 + i] = acc[v];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int t = threadIdx.x;
    float s = part[0][t];
#pragma unroll
    for (int ww = 1; ww < kTinyWaves; ++ww) s += part[ww][t];
    const int pp = tp * 16 + (t >> 4), qq = tq * 16 + (t & 15);
    if (pp < d.P && qq < d.Q && d.splits > 1) {
      float *dst = d.partial + ((int64_t)split * d.P + pp) * d.Q + qq;
      if constexpr (FUSE)
        numrs_hip::st_dev(dst, s);  // read by the block's last split
      else
        *dst = s;  // splitk_reduce finishes
    } else if (pp < d.P && qq < d.Q) {
      float *dst = C + (int64_t)pp * d.ldc + qq;
      float v = d.alpha * s;
      if (d.bias != nullptr) v = v + d.bias[qq];
      if (d.res != nullptr) v = v + d.res[(int64_t)pp * d.ldr + qq];
      v = d.accumulate ? *dst + v : v;
      if (d.act) {
        if (d.pre != nullptr) d.pre[(int64_t)pp * d.ldc + qq] = v;
        v = act_value(d.act, v);
      }
      *dst = v;
    }
  }
  if constexpr (FUSE) {
    if (d.splits > 1) {
      __shared__ int s_last;
      __builtin_amdgcn_s_waitcnt(0);  // this lane's partial stores acknowledged
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned *ctr = d.arrive + tile;
        const bool last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          (unsigned)(d.splits - 1);
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last ? 1 : 0;
      }
      __syncthreads();
      if (s_last != 0 && threadIdx.x < 256) {
        const int t = threadIdx.x;
        const int pp = tp * 16 + (t >> 4), qq = tq * 16 + (t & 15);
        if (pp < d.P && qq < d.Q) {
          const int64_t n = (int64_t)d.P * d.Q, e = (int64_t)pp * d.Q + qq;
          const __amdgpu_buffer_rsrc_t rs = numrs_hip::dev_rsrc(d.partial, (int64_t)d.splits * n * 4);
          float sum = 0.0f, comp = 0.0f;
          for (int k0 = 0; k0 < d.splits; k0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
              if (k0 + u < d.splits) v[u] = numrs_hip::ld_dev1(rs, (int)(4 * ((k0 + u) * n + e)));
            add_splits(0, sum, comp, v, d.splits - k0);
          }
          finish_split(C, d.ldc, d.bias, d.res, d.ldr, d.accumulate, d.alpha, d.act, d.pre,
                       (int64_t)pp, (int64_t)qq, sum);
        }
      }
    }
  }
}

// Column sums of a small bias gradient: 64 columns per workgroup, thread
// (class k, column c) adds rows k, k + 8, ... in order, and the eight class
// sums are added in class order.  With `mask` (same layout as g), entries
// whose mask is not > 0 count as zero.
__device__ __forceinline__ void tiny_colsum(const ColSum &c, int blk) {
  __shared__ float red[kTinyWaves][kTinyColsumCols];
  const int cl = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t col = (int64_t)blk * kTinyColsumCols + cl;
  float s = 0.0f;
  if (col < c.cols) {
    if (c.mask != nullptr) {
#pragma unroll 8
      for (int64_t r = k; r < c.rows; r += kTinyWaves) {
        const int64_t idx = r * c.ldg + col;
        s += c.mask[idx] > 0.0f ? c.g[idx] : 0.0f;
      }
    } else {
#pragma unroll 8
      for (int64_t r = k; r < c.rows; r += kTinyWaves) s += c.g[r * c.ldg + col];
    }
  }
  red[k][cl] = s;
  __syncthreads();
  if (threadIdx.x < kTinyColsumCols && col < c.cols) {
    float t = red[0][cl];
#pragma unroll
    for (int kk = 1; kk < kTinyWaves; ++kk) t += red[kk][cl];
    c.out[col] = c.acc ? c.out[col] + t : t;
  }
}

// Workgroups [0, tiles_a) form product a (layout XA, YA), the next tiles_b
// product b (TN), the rest (batch 0 only) the column sums cs.
template <bool XA, bool YA, int U, bool FUSE = false>
__global__ void __launch_bounds__(kTinyThreads) tiny_gemm_kernel(Gemm a, Gemm b, int tiles_a,
                                                                 int tiles_b, ColSum cs) {
  const int t = blockIdx.x;
  if (t < tiles_a)
    tiny_tile<XA, YA, U, FUSE>(a, t, blockIdx.y);
  else if (t < tiles_a + tiles_b)
    tiny_tile<false, false, U, FUSE>(b, t - tiles_a, blockIdx.y);
  else if (blockIdx.y == 0)
    tiny_colsum(cs, t - tiles_a - tiles_b);
}

int64_t tiny_tiles(const Gemm &g) { return (int64_t)((g.P + 15) / 16) * ((g.Q + 15) / 16); }

bool tiny_fits(const Gemm &g, int64_t batch) {
  // Each operand's byte extent under either layout stays below 2^31 (the
  // kernel's 32-bit load offsets).
  auto span = [](int64_t ext, int64_t other, int64_t ld) {
    return 4 * std::max((ext - 1) * ld + other, (other - 1) * ld + ext) < (int64_t{1} << 31);
  };
  return g.splits == 1 && g.R <= kTinyMaxR && (int64_t)g.P * g.Q * g.R * batch <= kTinyMacs &&
         span(g.P, g.R, g.ldx) && span(g.Q, g.R, g.ldy);
}

// Split-K for tiny products with few output blocks and a long reduction
// (the first MLP layer: 32 blocks over 784): blocks x splits fill the CUs,
// each split keeping at least four 32-wide k-tiles (a 16-wide step per
// wave); splitk_reduce then adds the splits in order.  A lone workgroup
// per CU streaming a long reduction is bound by its outstanding loads.
int tiny_split(int64_t cus, int64_t blocks, int R) {
  const int64_t kt = (R + kBR - 1) / kBR;
  int64_t sp = std::min<int64_t>({(cus + blocks - 1) / blocks, kt / 4, 32});
  if (sp <= 1) return 1;
  const int64_t per = (kt + sp - 1) / sp;
  return (int)((kt + per - 1) / per);
}

// One launch of the tiny kernel: product a (layout xa, ya), optionally a TN
// product b, and (batch 1) the column sums cs; then the split reduction
// when a batch-1 product was split.
int launch_tiny(numrs_hip_ctx *ctx, const Gemm &a_in, bool xa, bool ya, const Gemm *b_in,
                int64_t batch, const ColSum *cs) {
  Gemm a = a_in, bb = b_in != nullptr ? *b_in : a_in;
  const Gemm *b = b_in != nullptr ? &bb : nullptr;
  int64_t ta = tiny_tiles(a), tb = b != nullptr ? tiny_tiles(*b) : 0;
  const int64_t tc = cs != nullptr ? (cs->cols + kTinyColsumCols - 1) / kTinyColsumCols : 0;
  if (ta + tb + tc > 0x7fffffff || batch < 1 || batch > 65535 || (cs != nullptr && batch != 1))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "tiny_gemm: bad launch shape");
  int sa = 1, sb = 1;
  if (batch == 1) {
    const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    sa = tiny_split(cus, ta + tb, a.R);
    if (b != nullptr) sb = tiny_split(cus, ta + tb, b->R);
  }
  // Split products reduce inside this launch (tiny_tile's FUSE) unless the
  // context asks for the separate launch; offsets of the partials at device
  // scope are 32-bit.
  bool fuse = false;
  if (sa > 1 || sb > 1) {
    const size_t na = sa > 1 ? (size_t)sa * a.P * a.Q : 0;
    const size_t nb = sb > 1 ? (size_t)sb * bb.P * bb.Q : 0;
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (na + nb) * sizeof(float), &ws)) return rc;
    float *base = static_cast<float *>(ws);
    if (sa > 1) apply_splits(a, sa, base);
    if (sb > 1) apply_splits(bb, sb, base + na);
    fuse = ctx->split_reduce_mode == NUMRS_HIP_SPLIT_REDUCE_FUSED && 4 * (na + nb) < (size_t{1} << 31);
    if (fuse) {
      unsigned *cnt = nullptr;
      if (int rc = numrs_hip::arrival_counters(ctx, (size_t)(ta + tb), &cnt)) return rc;
      if (sa > 1) a.arrive = cnt;
      if (sb > 1) bb.arrive = cnt + ta;
    }
    ta *= sa;
    tb *= sb;
  }
  const dim3 grid((unsigned)(ta + tb + tc), (unsigned)batch);
  const ColSum c = cs != nullptr ? *cs : ColSum{};
  const int most_r = std::max(a.R, b != nullptr ? b->R : 0);
  auto go = [&](auto U, auto fuse_t) {
    constexpr int kU = decltype(U)::value;
    constexpr bool kF = decltype(fuse_t)::value;
    if (xa && ya)
      tiny_gemm_kernel<true, true, kU, kF><<<grid, kTinyThreads, 0, ctx->stream>>>(a, bb, (int)ta,
                                                                                    (int)tb, c);
    else if (xa)
      tiny_gemm_kernel<true, false, kU, kF><<<grid, kTinyThreads, 0, ctx->stream>>>(a, bb, (int)ta,
                                                                                     (int)tb, c);
    else if (ya)
      tiny_gemm_kernel<false, true, kU, kF><<<grid, kTinyThreads, 0, ctx->stream>>>(a, bb, (int)ta,
                                                                                     (int)tb, c);
    else
      tiny_gemm_kernel<false, false, kU, kF><<<grid, kTinyThreads, 0, ctx->stream>>>(a, bb, (int)ta,
                                                                                      (int)tb, c);
  };
  if (fuse)
    go(std::integral_constant<int, kTinyUSmall>{}, std::true_type{});
  else if (most_r > 16 * kTinyWaves * kTinyUSmall && sa == 1 && sb == 1)
    go(std::integral_constant<int, kTinyUBig>{}, std::false_type{});
  else
    go(std::integral_constant<int, kTinyUSmall>{}, std::false_type{});
  if (int rc = numrs_hip::check_launch(ctx, "tiny_gemm_kernel")) return rc;
  if (fuse) return NUMRS_HIP_OK;
  return reduce_splits(ctx, sa > 1 ? &a : nullptr, sb > 1 ? &bb : nullptr);
}

// The streamed path takes whole TP x TQ output tiles and whole reduction
// tiles of 16-byte aligned operands.
// The DMA's per-lane source offsets are 32-bit byte offsets of at most
// 256 rows from the tile base, so leading dimensions stay below 2^22 floats.
bool stream_fits(const Gemm &g, bool xrc, bool yrc, int tp, int tq) {
  constexpr int64_t kMaxLd = int64_t(1) << 22;
  return g.P % tp == 0 && g.Q % tq == 0 && g.R % kBR == 0 && g.R > 0 && vec_ok(g, xrc, yrc) &&
         g.ldx < kMaxLd && g.ldy < kMaxLd;
}

int shape_tp(int shape) { return shape == kShapeLarge ? kSP : shape == kShapeSmall ? kHP : kMP; }
int shape_tq(int shape) { return shape == kShapeLarge ? kSQ : shape == kShapeSmall ? kHQ : kMQ; }

Gemm as_stream(Gemm g, int shape) {
  g.tiles_p = g.P / shape_tp(shape);
  g.tiles_q = g.Q / shape_tq(shape);
  g.splits = 1;
  g.ktiles_per_split = g.R / kBR;
  g.partial = nullptr;
  return g;
}

// Split plan for the streamed path (batch 1).  Model, fitted to MI355X
// timings of both tile shapes over reduction lengths 1..128 tiles: a grid of
// W workgroups puts n = ceil(W / CUs) on the busiest CU.  Large tiles run one
// at a time, each costing T tile steps (T = its reduction tiles) plus a fixed
// cost (pipeline fill, epilogue, launch); small tiles run two at a time per
// CU, slower per step than a small tile alone.  A split product also writes
// and re-reads its fp32 partials (8 bytes per element per split) and launches
// a reduce.  Candidate per-workgroup reduction lengths T are ceil(k / s) for
// s = 1..32 of either product; each product is cut into ceil(k / T) ranges of
// equal length (at most 32 ranges, none empty) and the smallest estimate
// wins, ties going to fewer workgroups.  Product b is absent when tb == 0.
// A small tile alone on a CU runs a step in 0.9 us since the asm DMA ring
// (2048 -> 512 forward over 4096 rows, 256 tiles, one per CU: 66.4 us
// unsplit against 71.8 us split in two and reduced).
constexpr double kLargeTileUs = 4.22, kLargeFixedUs = 18.0;
// Wide tiles (kWP x kWQ, one per CU): a reduction step and the fixed cost
// as measured for [4096, K] x [K, 1536] over K = 128..2048 on MI355X (a
// step in 2.5-2.7 us, 9-15 us besides).
constexpr double kWideTileUs = 2.6, kWideFixedUs = 12.0;
constexpr double kSmallPairUs = 2.3, kSmallAloneUs = 0.9, kSmallFixedUs = 7.0;
constexpr double kPartialBytesPerUs = 6.0e6;

double stream_wave_us(bool small, int64_t n, int64_t T) {
  if (!small) return (double)n * ((double)T * kLargeTileUs + kLargeFixedUs);
  return (double)(n / 2) * ((double)T * kSmallPairUs + kSmallFixedUs) +
         (double)(n % 2) * ((double)T * kSmallAloneUs + kSmallFixedUs);
}

struct StreamPlan {
  bool small;
  int sa, sb;
  double t;
};

int stream_cut(int64_t k, int64_t T) {
  const int64_t s = std::min<int64_t>((k + T - 1) / T, 32);
  const int64_t per = (k + s - 1) / s;
  return (int)((k + per - 1) / per);
}

StreamPlan plan_shape(int64_t cus, int64_t ta, int64_t ka, int64_t pqa, int64_t tb, int64_t kb,
                      int64_t pqb, bool small) {
  cus = std::max<int64_t>(cus, 1);
  StreamPlan best{false, 1, 1, 0.0};
  int64_t best_w = 0;
  bool first = true;
  for (int cand = 0; cand < 64; ++cand) {
    const int64_t k = cand < 32 ? ka : kb;
    if (cand >= 32 && tb == 0) break;
    const int64_t T = (k + (cand & 31)) / ((cand & 31) + 1);
    if (T < 1) continue;
    const int sa = stream_cut(ka, T), sb = tb ? stream_cut(kb, T) : 1;
    const int64_t la = (ka + sa - 1) / sa, lb = tb ? (kb + sb - 1) / sb : 0;
    const int64_t w = ta * sa + tb * sb;
    double t = stream_wave_us(small, (w + cus - 1) / cus, std::max(la, lb));
    if (sa > 1) t += 8.0 * sa * pqa / kPartialBytesPerUs + 2.0;
    if (sb > 1) t += 8.0 * sb * pqb / kPartialBytesPerUs + 2.0;
    if (first || t < best.t || (t == best.t && w < best_w)) {
      first = false;
      best = {small, sa, sb, t};
      best_w = w;
    }
  }
  return best;
}

// Streamed-path plan for a batch-1 product a, or a pair with the TN product b
// in the same grid: picks the tile shape and the split-K ranges.  False when
// neither shape fits both products, or when the work is under four large
// tile steps per CU (the 128 x 128 path is then as good).
bool plan_streamed(numrs_hip_ctx *ctx, const Gemm &a, bool xa, bool ya, const Gemm *b,
                   StreamPlan *pl) {
  const double flops = 2.0 * a.P * a.Q * a.R + (b ? 2.0 * b->P * b->Q * b->R : 0.0);
  if (flops < 4.0 * ctx->num_cus * (2.0 * kSP * kSQ * kBR)) return false;
  bool any = false;
  for (int small = 0; small < 2; ++small) {
    const int tp = small ? kHP : kSP, tq = small ? kHQ : kSQ;
    if (!stream_fits(a, xa, ya, tp, tq) || (b && !stream_fits(*b, false, false, tp, tq))) continue;
    const int64_t ta = (int64_t)(a.P / tp) * (a.Q / tq), ka = a.R / kBR;
    const int64_t tb = b ? (int64_t)(b->P / tp) * (b->Q / tq) : 0, kb = b ? b->R / kBR : 0;
    if ((ta + tb) * 32 > 0x7fffffff) continue;  // grid of at most 32 splits per tile
    const StreamPlan c = plan_shape(ctx->num_cus, ta, ka, (int64_t)a.P * a.Q, tb, kb,
                                    b ? (int64_t)b->P * b->Q : 0, small != 0);
    if (!any || c.t < pl->t) *pl = c;
    any = true;
  }
  return any;
}

// Stream descriptors for a plan, with split products pointed at the
// context's workspace.
int stream_prepare(numrs_hip_ctx *ctx, const StreamPlan &pl, Gemm &ga, Gemm *gb) {
  ga = as_stream(ga, pl.small);
  if (gb != nullptr) *gb = as_stream(*gb, pl.small);
  const size_t na = pl.sa > 1 ? (size_t)pl.sa * ga.P * ga.Q : 0;
  const size_t nb = gb != nullptr && pl.sb > 1 ? (size_t)pl.sb * gb->P * gb->Q : 0;
  if (na + nb == 0) return NUMRS_HIP_OK;
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (na + nb) * sizeof(float), &ws)) return rc;
  float *base = static_cast<float *>(ws);
  if (na) apply_splits(ga, pl.sa, base);
  if (nb) apply_splits(*gb, pl.sb, base + na);
  return NUMRS_HIP_OK;
}

int64_t stream_grid(const Gemm &g) { return (int64_t)g.tiles_p * g.tiles_q * g.splits; }

SplitSet split_set(const Gemm &d) {
  return SplitSet{d.partial, d.C, d.bias, d.ldc, (int64_t)d.P * d.Q, d.Q, d.splits,
                  d.accumulate, d.alpha, d.act, d.pre, d.res, d.ldr, 0};
}

// splitk_reduce's float4 conditions for a set.
bool split_set_vec(const SplitSet &d) {
  return d.Q % 4 == 0 && d.ldc % 4 == 0 && numrs_hip::aligned16(d.C) &&
         numrs_hip::aligned16(d.partial) && (d.bias == nullptr || numrs_hip::aligned16(d.bias)) &&
         (d.res == nullptr || (numrs_hip::aligned16(d.res) && d.ldr % 4 == 0)) &&
         (d.pre == nullptr || numrs_hip::aligned16(d.pre));
}

// The fused form (see Fused) of a batch-1 streamed launch of a and b with
// the column sums cs and the set extra: fills f (marking the split products'
// tiles with their arrival counters) and the tail's workgroup count.  Leaves
// f.n_units = 0 -- the launch is then followed by splitk_reduce -- when there
// is nothing to reduce, or when a split set is not float4-addressable or its
// partials exceed the 32-bit device-scope offsets.
int fuse_plan(numrs_hip_ctx *ctx, int nt, Gemm &a, Gemm &b, const ColSum *cs,
              const SplitSet *extra, Fused &f, int64_t &tail) {
  f = Fused{};
  tail = 0;
  const bool sa = a.splits > 1, sb = b.splits > 1;
  if (!sa && !sb && cs == nullptr && extra == nullptr) return NUMRS_HIP_OK;
  if (ctx->split_reduce_mode != NUMRS_HIP_SPLIT_REDUCE_FUSED) return NUMRS_HIP_OK;
  const SplitSet s0 = sa ? split_set(a) : SplitSet{}, s1 = sb ? split_set(b) : SplitSet{};
  auto fits = [](const SplitSet &d) {
    return split_set_vec(d) && (int64_t)d.splits * d.n * 4 < (int64_t{1} << 31);
  };
  if ((sa && !fits(s0)) || (sb && !fits(s1)) || (extra != nullptr && !split_set_vec(*extra)))
    return NUMRS_HIP_OK;
  const int64_t na = stream_grid(a), nb = stream_grid(b);
  const int64_t ta = sa ? (int64_t)a.tiles_p * a.tiles_q : 0;
  const int64_t tb = sb ? (int64_t)b.tiles_p * b.tiles_q : 0;
  unsigned *cnt = nullptr;
  if (ta + tb > 0)
    if (int rc = numrs_hip::arrival_counters(ctx, (size_t)(8 * (ta + tb)), &cnt)) return rc;
  f.n_units = (int)(na + nb);
  if (sa != sb && na % 8 == 0 && nb % 8 == 0) {
    f.first_n = (int)(sa ? na : nb);
    f.first_base = sa ? 0 : (int)na;
    f.rest_base = sa ? (int)na : 0;
  }
  f.set[0] = s0;
  f.set[1] = s1;
  f.tiles_p[0] = a.tiles_p, f.tiles_q[0] = a.tiles_q;
  f.tiles_p[1] = b.tiles_p, f.tiles_q[1] = b.tiles_q;
  f.count[0] = sa ? cnt : nullptr;
  f.count[1] = sb ? cnt + 8 * ta : nullptr;
  f.sub[0] = (int)(8 * ta);
  f.sub[1] = (int)(8 * tb);
  a.arrive = f.count[0];
  b.arrive = f.count[1];
  const int64_t h = f.n_units + f.sub[0] + f.sub[1];
  if (cs != nullptr) {
    f.pad = (int)((8 - h % 8) % 8);
    f.cs = *cs;
    f.cs_wgs = (int)colsum_groups(cs->cols);
  }
  if (extra != nullptr) {
    f.extra = *extra;
    f.extra_wgs = (int)((extra->n / 4 + nt - 1) / nt);
  }
  tail = f.sub[0] + f.sub[1] + f.pad + f.cs_wgs + f.extra_wgs;
  if (f.first_n > 0) tail = (tail + 7) & ~int64_t{7};  // the unsplit units keep their XCDs
  f.n_tail = (int)tail;
  return NUMRS_HIP_OK;
}

// Streamed pair kernels by operand layout: dA = dC B^T with dB = A^T dC,
// dx = g W with dW = g^T x, and two transposed-left products.
enum PairKind { kPairMatmulBwd = 0, kPairLinearBwd = 1, kPairTN = 2 };

// One batch-1 launch of a streamed pair (tile shape `small`) with its split
// reductions, the column sums cs and the set extra in the same grid where
// fuse_plan allows; otherwise followed by splitk_reduce.  Only 128 x 64
// grids that fill every workgroup slot fuse: inside the C4 step the fused
// 256 x 128 launches measured slower than the product plus splitk_reduce (the
// reducers, which can only take a CU that a 148 KiB product workgroup has
// left, run behind the last product tiles), the 128 x 64 ones faster; and
// where the product leaves slots free (the LSTM weight gradients: 256 units)
// the reducers start at once, arrive before the splits, and the last split of
// each tile then reduces all of its sub-blocks alone (C5's pairs 82 + 59 us
// against 80 + 57 with the separate launch).
int launch_stream_pair(numrs_hip_ctx *ctx, PairKind kind, bool small, Gemm sa, Gemm sb,
                       const ColSum *cs, const SplitSet *extra, const char *who) {
  Fused f{};
  int64_t tail = 0;
  const int64_t slots = 2 * std::max<int64_t>(ctx->num_cus, 1);  // two 128 x 64 workgroups per CU
  if (small && stream_grid(sa) + stream_grid(sb) >= slots)
    if (int rc = fuse_plan(ctx, kThreads, sa, sb, cs, extra, f, tail)) return rc;
  const int64_t na = stream_grid(sa), total = na + stream_grid(sb) + tail;
  if (total > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: too large", who);
  const dim3 grid((unsigned)total, 1);
  const int ta = (int)na;
  auto go = [&](auto fuse_t) {
    constexpr bool kF = decltype(fuse_t)::value;
    switch (kind) {
      case kPairMatmulBwd:
        if (small)
          matmul_backward_stream_small<kF><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        else
          matmul_backward_stream<kF><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        break;
      case kPairLinearBwd:
        if (small)
          linear_backward_stream_small<kF><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        else
          linear_backward_stream<kF><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        break;
      default:
        if (small)
          tn_pair_stream_small<kF><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        else
          tn_pair_stream<kF><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, ta, f);
        break;
    }
  };
  if (f.n_units != 0)
    go(std::true_type{});
  else
    go(std::false_type{});
  if (int rc = numrs_hip::check_launch(ctx, who)) return rc;
  if (f.n_units != 0) return NUMRS_HIP_OK;
  return reduce_splits(ctx, &sa, &sb, cs, extra);
}

// Tile shape for a batched product (or a pair sharing the grid): no split-K,
// so the shape whose tiles fill the CUs with the smaller modelled time;
// false when neither shape fits or gives at least one tile per CU.
// Mini tiles run up to three per CU: a round of k of them (k = 1..3) costs
// T steps at the k-way rate plus a fixed cost.
constexpr double kMiniUs[4] = {0.0, 0.9, 1.25, 1.7}, kMiniFixedUs = 6.0;

double mini_wave_us(int64_t n, int64_t T) {
  double t = (double)(n / 3) * ((double)T * kMiniUs[3] + kMiniFixedUs);
  if (n % 3) t += (double)T * kMiniUs[n % 3] + kMiniFixedUs;
  return t;
}

bool pick_batched_stream(numrs_hip_ctx *ctx, const Gemm &a, bool xa, bool ya, const Gemm *b,
                         int64_t batch, int *shape_out) {
  bool any = false;
  double best = 0.0;
  const int64_t cus = std::max(ctx->num_cus, 1);
  for (int shape = kShapeLarge; shape <= kShapeMini; ++shape) {
    const int tp = shape_tp(shape), tq = shape_tq(shape);
    if (!stream_fits(a, xa, ya, tp, tq) || (b && !stream_fits(*b, false, false, tp, tq))) continue;
    const int64_t t = (int64_t)(a.P / tp) * (a.Q / tq) + (b ? (int64_t)(b->P / tp) * (b->Q / tq) : 0);
    if (t * batch < cus || t > 0x7fffffff) continue;
    const int64_t T = std::max<int64_t>(a.R, b ? b->R : 0) / kBR;
    const int64_t n = (t * batch + cus - 1) / cus;
    const double est = shape == kShapeMini ? mini_wave_us(n, T)
                                           : stream_wave_us(shape == kShapeSmall, n, T);
    if (!any || est < best) {
      best = est;
      *shape_out = shape;
    }
    any = true;
  }
  return any;
}

int check_dims(numrs_hip_ctx *ctx, const char *who, int64_t batch, int64_t M, int64_t K,
               int64_t N) {
  if (batch < 0 || M < 0 || K < 0 || N < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative dimension", who);
  const int64_t lim = (int64_t)1 << 30;
  if (M >= lim || K >= lim || N >= lim || batch >= 65536)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: dimension too large", who);
  return NUMRS_HIP_OK;
}

Gemm make(const float *X, const float *Y, float *C, int64_t ldx, int64_t ldy, int64_t ldc,
          int64_t bsx, int64_t bsy, int64_t bsc, int64_t P, int64_t Q, int64_t R, int acc) {
  Gemm g;
  g.X = X;
  g.Y = Y;
  g.C = C;
  g.ldx = ldx;
  g.ldy = ldy;
  g.ldc = ldc;
  g.bsx = bsx;
  g.bsy = bsy;
  g.bsc = bsc;
  g.bsx2 = g.bsy2 = g.bsc2 = 0;
  g.binner = 1;
  g.alpha = 1.0f;
  g.splits = 1;
  g.ktiles_per_split = (int)((R + kBR - 1) / kBR);
  g.partial = nullptr;
  g.bias = nullptr;
  g.xmask = nullptr;
  g.act = 0;
  g.pre = nullptr;
  g.res = nullptr;
  g.ldr = 0;
  g.arrive = nullptr;
  g.P = (int)P;
  g.Q = (int)Q;
  g.R = (int)R;
  g.tiles_p = tiles(P);
  g.tiles_q = tiles(Q);
  g.accumulate = acc;
  return g;
}

// Zero-length reduction: C = 0 (or unchanged when accumulating).
int zero_output(numrs_hip_ctx *ctx, float *C, int64_t count, int acc) {
  if (acc || count == 0) return NUMRS_HIP_OK;
  return numrs_hip_fill(ctx, C, count, 0.0f);
}

template <bool XRC, bool YRC>
int launch_one(numrs_hip_ctx *ctx, Gemm g, int64_t batch) {
  const int64_t n_tiles = (int64_t)g.tiles_p * g.tiles_q;
  if (n_tiles == 0 || batch == 0) return NUMRS_HIP_OK;
  if (tiny_fits(g, batch)) return launch_tiny(ctx, g, XRC, YRC, nullptr, batch, nullptr);
  StreamPlan pl;
  if (batch == 1 && plan_streamed(ctx, g, XRC, YRC, nullptr, &pl)) {
    if constexpr (XRC && YRC) {
      // the wide tile where it fits and its modelled time beats the plan's
      const int64_t cus = std::max<int64_t>(ctx->num_cus, 1);
      if (g.P % kWP == 0 && g.Q % kWQ == 0 && vec_ok(g, true, true) && g.ldx < (int64_t{1} << 22) &&
          g.ldy < (int64_t{1} << 22)) {
        const int64_t tw = (int64_t)(g.P / kWP) * (g.Q / kWQ);
        const double t = (double)((tw + cus - 1) / cus) * ((g.R / kBR) * kWideTileUs + kWideFixedUs);
        if (t < pl.t && tw <= 0x7fffffff) {
          Gemm sg = g;
          sg.tiles_p = g.P / kWP;
          sg.tiles_q = g.Q / kWQ;
          sg.splits = 1;
          sg.ktiles_per_split = g.R / kBR;
          sg.partial = nullptr;
          const dim3 grid((unsigned)tw, 1);
          if (sg.act)
            gemm_stream_wide<true><<<grid, kBigThreads, 0, ctx->stream>>>(sg);
          else
            gemm_stream_wide<false><<<grid, kBigThreads, 0, ctx->stream>>>(sg);
          return numrs_hip::check_launch(ctx, "gemm_stream_wide");
        }
      }
    }
    Gemm sg = g;
    if (int rc = stream_prepare(ctx, pl, sg, nullptr)) return rc;
    const dim3 grid((unsigned)stream_grid(sg), 1);
    if (sg.act && sg.splits == 1) {  // activation in the tile epilogue (the Linear forward)
      if constexpr (XRC && YRC) {
        if (pl.small)
          gemm_stream_small<true, true, true><<<grid, kThreads, 0, ctx->stream>>>(sg);
        else
          gemm_stream_kernel<true, true, true><<<grid, kBigThreads, 0, ctx->stream>>>(sg);
      } else {
        return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "gemm: activation on a non-NT product");
      }
    } else if (pl.small) {
      gemm_stream_small<XRC, YRC><<<grid, kThreads, 0, ctx->stream>>>(sg);
    } else {
      gemm_stream_kernel<XRC, YRC><<<grid, kBigThreads, 0, ctx->stream>>>(sg);
    }
    if (int rc = numrs_hip::check_launch(ctx, "gemm_stream_kernel")) return rc;
    return reduce_splits(ctx, &sg, nullptr);
  }
  int shape = kShapeLarge;
  if (batch > 1 && pick_batched_stream(ctx, g, XRC, YRC, nullptr, batch, &shape)) {
    const Gemm sg = as_stream(g, shape);
    dim3 grid((unsigned)stream_grid(sg), (unsigned)batch);
    if (shape == kShapeMini)
      gemm_stream_mini<XRC, YRC><<<grid, kThreads, 0, ctx->stream>>>(sg);
    else if (shape == kShapeSmall)
      gemm_stream_small<XRC, YRC><<<grid, kThreads, 0, ctx->stream>>>(sg);
    else
      gemm_stream_kernel<XRC, YRC><<<grid, kBigThreads, 0, ctx->stream>>>(sg);
    return numrs_hip::check_launch(ctx, "gemm_stream_kernel");
  }
  const int splits = plan_splits(g, batch);
  if (splits > 1) {
    void *ws = nullptr;
    const size_t bytes = (size_t)splits * g.P * g.Q * sizeof(float);
    if (int rc = numrs_hip::workspace(ctx, bytes, &ws)) return rc;
    apply_splits(g, splits, static_cast<float *>(ws));
  }
  if (n_tiles * splits > 0x7fffffff)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "gemm: too many tiles");
  dim3 grid((unsigned)(n_tiles * splits), (unsigned)batch);
  if (g.act && g.splits == 1) {  // activation in the tile epilogue (the Linear forward)
    if constexpr (XRC && YRC) {
      if (vec_ok(g, XRC, YRC))
        gemm_kernel<true, true, true, true><<<grid, kThreads, 0, ctx->stream>>>(g);
      else
        gemm_kernel<true, true, false, true><<<grid, kThreads, 0, ctx->stream>>>(g);
    } else {
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "gemm: activation on a non-NT product");
    }
  } else if (vec_ok(g, XRC, YRC)) {
    gemm_kernel<XRC, YRC, true><<<grid, kThreads, 0, ctx->stream>>>(g);
  } else {
    gemm_kernel<XRC, YRC, false><<<grid, kThreads, 0, ctx->stream>>>(g);
  }
  if (int rc = numrs_hip::check_launch(ctx, "gemm_kernel")) return rc;
  return reduce_splits(ctx, &g, nullptr);
}

int gemm_dispatch(numrs_hip_ctx *ctx, const Gemm &g, int64_t batch, bool xrc, bool yrc) {
  if (xrc && yrc) return launch_one<true, true>(ctx, g, batch);
  if (xrc && !yrc) return launch_one<true, false>(ctx, g, batch);
  if (!xrc && yrc) return launch_one<false, true>(ctx, g, batch);
  return launch_one<false, false>(ctx, g, batch);
}

int matmul_backward_impl(numrs_hip_ctx *ctx, const float *dC, const float *A, const float *B,
                         float *dA, float *dB, int64_t batch, int64_t M, int64_t K, int64_t N,
                         int64_t sa, int64_t sb, int64_t sc, int acc) {
  const char *who = "numrs_hip_matmul_backward";
  int rc = check_dims(ctx, who, batch, M, K, N);
  if (rc) return rc;
  if (dA == nullptr && dB == nullptr) return NUMRS_HIP_OK;
  if (batch == 0 || M == 0 || K == 0 || N == 0) {
    // Empty operands (0-byte buffers may be NULL): dA is reduced over N and dB
    // over M, so an empty reduction dimension gives zero gradients.
    for (int64_t b = 0; b < batch; ++b) {
      if (dA && M * K > 0) rc = zero_output(ctx, dA + b * sa, M * K, acc);
      if (!rc && dB && K * N > 0) rc = zero_output(ctx, dB + b * sb, K * N, acc);
      if (rc) return rc;
    }
    return NUMRS_HIP_OK;
  }
  if (dC == nullptr || (dA != nullptr && B == nullptr) || (dB != nullptr && A == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input pointer", who);
  // dA[M,K] = dC[M,N] @ B[K,N]^T : P=M, Q=K, R=N, X=dC (ld N), Y=B (ld N)
  Gemm ga = make(dC, B, dA, N, N, K, sc, sb, sa, M, K, N, acc);
  // dB[K,N] = A[M,K]^T @ dC[M,N] : P=K, Q=N, R=M, X=A (ld K), Y=dC (ld N)
  Gemm gb = make(A, dC, dB, K, N, N, sa, sc, sb, K, N, M, acc);
  if (dA == nullptr) return gemm_dispatch(ctx, gb, batch, false, false);
  if (dB == nullptr) return gemm_dispatch(ctx, ga, batch, true, true);
  if (tiny_fits(ga, batch) && tiny_fits(gb, batch))
    return launch_tiny(ctx, ga, true, true, &gb, batch, nullptr);
  StreamPlan pl;
  if (batch == 1 && plan_streamed(ctx, ga, true, true, &gb, &pl)) {
    Gemm sa = ga, sb = gb;
    if (int rc2 = stream_prepare(ctx, pl, sa, &sb)) return rc2;
    return launch_stream_pair(ctx, kPairMatmulBwd, pl.small, sa, sb, nullptr, nullptr,
                              "matmul_backward_stream");
  }
  int shape = kShapeLarge;
  if (batch > 1 && pick_batched_stream(ctx, ga, true, true, &gb, batch, &shape)) {
    const Gemm sa = as_stream(ga, shape), sb = as_stream(gb, shape);
    const int64_t ta = stream_grid(sa), tb = stream_grid(sb);
    dim3 grid((unsigned)(ta + tb), (unsigned)batch);
    if (shape == kShapeMini)
      matmul_backward_stream_mini<<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta);
    else if (shape == kShapeSmall)
      matmul_backward_stream_small<false><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    else
      matmul_backward_stream<false><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    return numrs_hip::check_launch(ctx, "matmul_backward_stream");
  }
  const int sa_ = plan_splits(ga, batch), sb_ = plan_splits(gb, batch);
  if (sa_ > 1 || sb_ > 1) {
    const size_t na = sa_ > 1 ? (size_t)sa_ * ga.P * ga.Q : 0;
    const size_t nb = sb_ > 1 ? (size_t)sb_ * gb.P * gb.Q : 0;
    void *ws = nullptr;
    if (int rc2 = numrs_hip::workspace(ctx, (na + nb) * sizeof(float), &ws)) return rc2;
    float *base = static_cast<float *>(ws);
    if (sa_ > 1) apply_splits(ga, sa_, base);
    if (sb_ > 1) apply_splits(gb, sb_, base + na);
  }
  const int64_t ta = (int64_t)ga.tiles_p * ga.tiles_q * sa_;
  const int64_t tb = (int64_t)gb.tiles_p * gb.tiles_q * sb_;
  if (ta + tb > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: too large", who);
  dim3 grid((unsigned)(ta + tb), (unsigned)batch);
  if (vec_ok(ga, true, true) && vec_ok(gb, false, false))
    matmul_backward_kernel<true><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
  else
    matmul_backward_kernel<false><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
  if (int rc2 = numrs_hip::check_launch(ctx, "matmul_backward_kernel")) return rc2;
  return reduce_splits(ctx, &ga, &gb);
}

int matmul_impl(numrs_hip_ctx *ctx, const float *A, const float *B, float *C, int64_t batch,
                int64_t M, int64_t K, int64_t N, int64_t sa, int64_t sb, int64_t sc, int ta,
                int tb, int acc) {
  const char *who = "numrs_hip_matmul";
  int rc = check_dims(ctx, who, batch, M, K, N);
  if (rc) return rc;
  if (batch == 0 || M == 0 || N == 0) return NUMRS_HIP_OK;
  if (C == nullptr || ((A == nullptr || B == nullptr) && K > 0))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (K == 0) {
    for (int64_t b = 0; b < batch; ++b)
      if ((rc = zero_output(ctx, C + b * sc, M * N, acc))) return rc;
    return NUMRS_HIP_OK;
  }
  // op(A)[M,K]: R-contiguous unless transposed (stored [K,M]).
  const bool xrc = !ta;
  const int64_t ldx = ta ? M : K;
  // op(B)[K,N]: Q-contiguous unless transposed (stored [N,K], R-contiguous).
  const bool yrc = tb != 0;
  const int64_t ldy = tb ? K : N;
  Gemm g = make(A, B, C, ldx, ldy, N, sa, sb, sc, M, N, K, acc);
  return gemm_dispatch(ctx, g, batch, xrc, yrc);
}

int gemm_general(numrs_hip_ctx *ctx, const float *A, int64_t lda, const float *B, int64_t ldb,
                 float *C, int64_t ldc, int64_t M, int64_t K, int64_t N, int ta, int tb,
                 float alpha, int acc, int64_t batch, int64_t binner, int64_t sao, int64_t sai,
                 int64_t sbo, int64_t sbi, int64_t sco, int64_t sci) {
  const char *who = "numrs_hip_gemm";
  int rc = check_dims(ctx, who, batch, M, K, N);
  if (rc) return rc;
  if (binner < 1 || binner > batch + (batch == 0))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: batch_inner %lld", who, (long long)binner);
  if (lda < 0 || ldb < 0 || ldc < N || sao < 0 || sai < 0 || sbo < 0 || sbi < 0 || sco < 0 ||
      sci < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: bad leading dimension or stride", who);
  if (lda < (ta ? M : K) || ldb < (tb ? K : N))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: leading dimension too small", who);
  if (batch == 0 || M == 0 || N == 0) return NUMRS_HIP_OK;
  if (C == nullptr || ((A == nullptr || B == nullptr) && K > 0))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  Gemm g = make(A, B, C, lda, ldb, ldc, sao, sbo, sco, M, N, K, acc);
  g.bsx2 = sai;
  g.bsy2 = sbi;
  g.bsc2 = sci;
  g.binner = (int)binner;
  g.alpha = alpha;
  if (K == 0) {
    if (acc) return NUMRS_HIP_OK;
    if (ldc != N || binner != 1 || sco != M * N)
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: empty reduction into a strided C", who);
    return numrs_hip_fill(ctx, C, batch * M * N, 0.0f);
  }
  return gemm_dispatch(ctx, g, batch, !ta, tb != 0);
}

// Launches a (first, TN-second) product pair in one grid with per-product
// split-K; `first_nt` selects the NT (matmul_backward dA) or NN (Linear dx)
// layout of the first product.  Either product may be absent (C == null).
// `cs` (optional): column sums that the pair's launch forms too -- the tiny
// kernel's own workgroups, or the split-reduce launch (a launch of its own
// when neither product is split) where colsum_fits; *cs_done says whether
// they were formed.
int launch_pair(numrs_hip_ctx *ctx, Gemm ga, Gemm gb, bool first_nt, const char *who,
                const ColSum *cs_in = nullptr, bool *cs_done = nullptr) {
  const bool has_a = ga.C != nullptr, has_b = gb.C != nullptr;
  if (cs_done != nullptr) *cs_done = false;
  if ((has_a || has_b) && (!has_a || tiny_fits(ga, 1)) && (!has_b || tiny_fits(gb, 1)) &&
      (cs_in == nullptr || cs_in->rows <= kTinyColsumRows)) {
    if (cs_done != nullptr) *cs_done = cs_in != nullptr;
    if (has_a) return launch_tiny(ctx, ga, true, first_nt, has_b ? &gb : nullptr, 1, cs_in);
    return launch_tiny(ctx, gb, false, false, nullptr, 1, cs_in);
  }
  const ColSum *cs = cs_in != nullptr && cs_in->mask == nullptr &&
                             colsum_fits(cs_in->g, cs_in->rows, cs_in->cols, cs_in->ldg)
                         ? cs_in
                         : nullptr;
  if (cs_done != nullptr) *cs_done = cs != nullptr;
  if (!has_a && !has_b) return cs ? reduce_splits(ctx, nullptr, nullptr, cs) : NUMRS_HIP_OK;
  if (!has_a || !has_b) {
    if (int rc = has_a ? gemm_dispatch(ctx, ga, 1, true, first_nt)
                       : gemm_dispatch(ctx, gb, 1, false, false))
      return rc;
    return cs ? reduce_splits(ctx, nullptr, nullptr, cs) : NUMRS_HIP_OK;
  }
  StreamPlan pl;
  if (plan_streamed(ctx, ga, true, first_nt, &gb, &pl)) {
    Gemm sa = ga, sb = gb;
    if (int rc = stream_prepare(ctx, pl, sa, &sb)) return rc;
    return launch_stream_pair(ctx, first_nt ? kPairMatmulBwd : kPairLinearBwd, pl.small, sa, sb,
                              cs, nullptr, who);
  }
  // Joint split plan, balanced by work: the pair shares one grid, and a
  // workgroup's time is its number of reduction tiles.  The weight gradient
  // (long reduction over tokens) next to dx (short reduction over features)
  // would otherwise leave a few long workgroups running alone -- Linear
  // 2048 -> 512 over 4096 tokens: 512 dx tiles of 16 k-tiles and 64 dW tiles
  // of 128.  Each product is cut so that no workgroup holds more than the
  // larger of (a) the shorter product's reduction and (b) the average work
  // per workgroup slot (two per CU), keeping at least 8 k-tiles per split.
  int sa_ = 1, sb_ = 1;
  {
    const int64_t ta0 = (int64_t)ga.tiles_p * ga.tiles_q, tb0 = (int64_t)gb.tiles_p * gb.tiles_q;
    const int64_t ka = (ga.R + kBR - 1) / kBR, kb = (gb.R + kBR - 1) / kBR;
    const int64_t slots = 2 * (int64_t)(ctx->num_cus > 0 ? ctx->num_cus : 256);
    const int64_t avg = (ta0 * ka + tb0 * kb + slots - 1) / slots;
    const int64_t target = std::max<int64_t>({std::min(ka, kb), avg, 8});
    auto splits_for = [&](int64_t nk) {
      int64_t sp = (nk + target - 1) / target;
      return (int)std::max<int64_t>(1, std::min<int64_t>({sp, nk / 8, 32}));
    };
    sa_ = splits_for(ka);
    sb_ = splits_for(kb);
  }
  if (sa_ > 1 || sb_ > 1) {
    const size_t na = sa_ > 1 ? (size_t)sa_ * ga.P * ga.Q : 0;
    const size_t nb = sb_ > 1 ? (size_t)sb_ * gb.P * gb.Q : 0;
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (na + nb) * sizeof(float), &ws)) return rc;
    float *base = static_cast<float *>(ws);
    if (sa_ > 1) apply_splits(ga, sa_, base);
    if (sb_ > 1) apply_splits(gb, sb_, base + na);
  }
  const int64_t ta = (int64_t)ga.tiles_p * ga.tiles_q * sa_;
  const int64_t tb = (int64_t)gb.tiles_p * gb.tiles_q * sb_;
  if (ta + tb > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: too large", who);
  dim3 grid((unsigned)(ta + tb), 1);
  const bool vec = vec_ok(ga, true, first_nt) && vec_ok(gb, false, false);
  if (first_nt) {
    if (vec) gemm_pair_kernel<true, true, true><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
    else gemm_pair_kernel<true, true, false><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
  } else {
    if (vec) gemm_pair_kernel<true, false, true><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
    else gemm_pair_kernel<true, false, false><<<grid, kThreads, 0, ctx->stream>>>(ga, gb, (int)ta);
  }
  if (int rc = numrs_hip::check_launch(ctx, "gemm_pair_kernel")) return rc;
  return reduce_splits(ctx, &ga, &gb, cs);
}

}  // namespace

int numrs_hip::gemm_nn_tn_pair(numrs_hip_ctx *ctx, BatchedMat X, BatchedMat Y1, BatchedOut C1,
                               BatchedMat Y2, BatchedOut C2, int64_t M, int64_t K, int64_t N,
                               float alpha, int accumulate, int64_t batch, int64_t binner) {
  const char *who = "gemm_nn_tn_pair";
  if (int rc = check_dims(ctx, who, batch, M, K, N)) return rc;
  if (binner < 1 || binner > std::max<int64_t>(batch, 1))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: batch_inner %lld", who, (long long)binner);
  if (batch == 0 || N == 0 || (C1.p == nullptr && C2.p == nullptr)) return NUMRS_HIP_OK;
  // C1[M,N] = X[M,K] Y1[K,N]: P=M, Q=N, R=K, X reduction-contiguous.
  Gemm ga = make(X.p, Y1.p, C1.p, X.ld, Y1.ld, C1.ld, X.so, Y1.so, C1.so, M, N, K, accumulate);
  // C2[K,N] = X^T Y2[M,N]: P=K, Q=N, R=M, X output-contiguous.
  Gemm gb = make(X.p, Y2.p, C2.p, X.ld, Y2.ld, C2.ld, X.so, Y2.so, C2.so, K, N, M, accumulate);
  ga.bsx2 = X.si, ga.bsy2 = Y1.si, ga.bsc2 = C1.si;
  gb.bsx2 = X.si, gb.bsy2 = Y2.si, gb.bsc2 = C2.si;
  ga.binner = gb.binner = (int)binner;
  ga.alpha = gb.alpha = alpha;
  if (M == 0 || K == 0) {
    // an empty reduction leaves zeros (or the accumulated values)
    for (int64_t z = 0; z < batch && !accumulate; ++z) {
      const int64_t zo = z / binner, zi = z - zo * binner;
      if (C1.p && M > 0)
        for (int64_t r = 0; r < M; ++r)
          if (int rc = numrs_hip_fill(ctx, C1.p + zo * C1.so + zi * C1.si + r * C1.ld, N, 0.0f))
            return rc;
      if (C2.p && K > 0)
        for (int64_t r = 0; r < K; ++r)
          if (int rc = numrs_hip_fill(ctx, C2.p + zo * C2.so + zi * C2.si + r * C2.ld, N, 0.0f))
            return rc;
    }
    return NUMRS_HIP_OK;
  }
  if (X.p == nullptr || (C1.p && Y1.p == nullptr) || (C2.p && Y2.p == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  if (C1.p == nullptr) return gemm_dispatch(ctx, gb, batch, false, false);
  if (C2.p == nullptr) return gemm_dispatch(ctx, ga, batch, true, false);
  if (batch == 1) return launch_pair(ctx, ga, gb, false, who);
  if (tiny_fits(ga, batch) && tiny_fits(gb, batch))
    return launch_tiny(ctx, ga, true, false, &gb, batch, nullptr);
  int shape = kShapeLarge;
  if (pick_batched_stream(ctx, ga, true, false, &gb, batch, &shape)) {
    const Gemm sa = as_stream(ga, shape), sb = as_stream(gb, shape);
    const int64_t ta = stream_grid(sa), tb = stream_grid(sb);
    dim3 grid((unsigned)(ta + tb), (unsigned)batch);
    if (shape == kShapeMini)
      linear_backward_stream_mini<<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta);
    else if (shape == kShapeSmall)
      linear_backward_stream_small<false><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    else
      linear_backward_stream<false><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    return numrs_hip::check_launch(ctx, who);
  }
  if (int rc = gemm_dispatch(ctx, ga, batch, true, false)) return rc;
  return gemm_dispatch(ctx, gb, batch, false, false);
}

int numrs_hip::gemm_tn_pair(numrs_hip_ctx *ctx, BatchedMat X1, BatchedMat Y1, BatchedOut C1,
                            float alpha1, BatchedMat X2, BatchedMat Y2, BatchedOut C2,
                            float alpha2, int64_t M, int64_t K, int64_t N, int accumulate,
                            int64_t batch, int64_t binner) {
  const char *who = "gemm_tn_pair";
  if (int rc = check_dims(ctx, who, batch, M, K, N)) return rc;
  if (binner < 1 || binner > std::max<int64_t>(batch, 1))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: batch_inner %lld", who, (long long)binner);
  if (batch == 0 || N == 0 || K == 0 || (C1.p == nullptr && C2.p == nullptr)) return NUMRS_HIP_OK;
  if ((C1.p && (X1.p == nullptr || Y1.p == nullptr)) || (C2.p && (X2.p == nullptr || Y2.p == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  // C[K,N] = alpha X^T Y with X [M,K], Y [M,N]: P=K, Q=N, R=M, both operands
  // output-contiguous.
  auto tn = [&](BatchedMat X, BatchedMat Y, BatchedOut C, float alpha) {
    Gemm g = make(X.p, Y.p, C.p, X.ld, Y.ld, C.ld, X.so, Y.so, C.so, K, N, M, accumulate);
    g.bsx2 = X.si, g.bsy2 = Y.si, g.bsc2 = C.si;
    g.binner = (int)binner;
    g.alpha = alpha;
    return g;
  };
  if (M == 0) {  // an empty reduction leaves zeros (or the accumulated values)
    for (int64_t z = 0; z < batch && !accumulate; ++z) {
      const int64_t zo = z / binner, zi = z - zo * binner;
      for (const BatchedOut *C : {&C1, &C2})
        if (C->p)
          for (int64_t r = 0; r < K; ++r)
            if (int rc = numrs_hip_fill(ctx, C->p + zo * C->so + zi * C->si + r * C->ld, N, 0.0f))
              return rc;
    }
    return NUMRS_HIP_OK;
  }
  const Gemm ga = C1.p ? tn(X1, Y1, C1, alpha1) : Gemm{}, gb = C2.p ? tn(X2, Y2, C2, alpha2) : Gemm{};
  if (C1.p == nullptr) return gemm_dispatch(ctx, gb, batch, false, false);
  if (C2.p == nullptr) return gemm_dispatch(ctx, ga, batch, false, false);
  if (batch > 1 && tiny_fits(ga, batch) && tiny_fits(gb, batch))
    return launch_tiny(ctx, ga, false, false, &gb, batch, nullptr);
  int shape = kShapeLarge;
  if (batch > 1 && pick_batched_stream(ctx, ga, false, false, &gb, batch, &shape)) {
    const Gemm sa = as_stream(ga, shape), sb = as_stream(gb, shape);
    const int64_t ta = stream_grid(sa), tb = stream_grid(sb);
    dim3 grid((unsigned)(ta + tb), (unsigned)batch);
    if (shape == kShapeMini)
      tn_pair_stream_mini<<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta);
    else if (shape == kShapeSmall)
      tn_pair_stream_small<false><<<grid, kThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    else
      tn_pair_stream<false><<<grid, kBigThreads, 0, ctx->stream>>>(sa, sb, (int)ta, Fused{});
    return numrs_hip::check_launch(ctx, who);
  }
  if (int rc = gemm_dispatch(ctx, ga, batch, false, false)) return rc;
  return gemm_dispatch(ctx, gb, batch, false, false);
}

int numrs_hip::gemm_tn2_colsum(numrs_hip_ctx *ctx, const float *X, int64_t ldx, int64_t M,
                               int64_t K, const float *Y1, int64_t ldy1, int64_t N1, float *C1,
                               int acc1, const float *Y2, int64_t ldy2, int64_t N2, float *C2,
                               int acc2, float *db, int acc_db, const float *db_part,
                               int64_t db_rows) {
  const char *who = "gemm_tn2_colsum";
  if (int rc = check_dims(ctx, who, 1, M, K, std::max(N1, N2))) return rc;
  if (X == nullptr || C1 == nullptr || C2 == nullptr || Y1 == nullptr || Y2 == nullptr ||
      M <= 0 || K <= 0 || N1 <= 0 || N2 <= 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null or empty operand", who);
  // C[K,N] = X^T Y with X [M,K], Y [M,N]: P=K, Q=N, R=M (both operands
  // output-contiguous), as gemm_tn_pair.
  Gemm ga = make(X, Y1, C1, ldx, ldy1, N1, 0, 0, 0, K, N1, M, acc1);
  Gemm gb = make(X, Y2, C2, ldx, ldy2, N2, 0, 0, 0, K, N2, M, acc2);
  ColSum cs{X, db, M, K, ldx, acc_db, nullptr};
  // db from row partials: the compensated sum over db_rows rows of db_part
  // [db_rows, K] in row order, as one more set of the split reduce
  const bool by_part = db != nullptr && db_part != nullptr && db_rows >= 1 && db_rows <= (1 << 20);
  SplitSet part{db_part, db, nullptr, K, K, (int)K, (int)db_rows, acc_db, 1.0f, 0, nullptr,
                nullptr, 0, 1};
  const SplitSet *extra = by_part ? &part : nullptr;
  const bool cs_ok = db != nullptr && !by_part && colsum_fits(X, M, K, ldx);
  StreamPlan pl;
  if (plan_streamed(ctx, ga, false, false, &gb, &pl)) {
    if (int rc = stream_prepare(ctx, pl, ga, &gb)) return rc;
    if (int rc = launch_stream_pair(ctx, kPairTN, pl.small, ga, gb, cs_ok ? &cs : nullptr, extra,
                                    who))
      return rc;
  } else {
    if (int rc = gemm_dispatch(ctx, ga, 1, false, false)) return rc;
    if (int rc = gemm_dispatch(ctx, gb, 1, false, false)) return rc;
    if (cs_ok || by_part)
      if (int rc = reduce_splits(ctx, nullptr, nullptr, cs_ok ? &cs : nullptr, extra)) return rc;
  }
  if (db == nullptr || cs_ok || by_part) return NUMRS_HIP_OK;
  const int64_t gs[2] = {M, K};
  return numrs_hip_sum_to_shape(ctx, X, gs, 2, db, &K, 1, NUMRS_HIP_UNBROADCAST_CORRECT, acc_db);
}

extern "C" {

int numrs_hip_set_split_reduction(numrs_hip_ctx *ctx, int mode) {
  NRS_CHECK_CTX(ctx);
  if (mode != NUMRS_HIP_SPLIT_REDUCE_FUSED && mode != NUMRS_HIP_SPLIT_REDUCE_SEPARATE)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "split reduction mode %d", mode);
  ctx->split_reduce_mode = mode;
  return NUMRS_HIP_OK;
}

int numrs_hip_linear_forward(numrs_hip_ctx *ctx, const float *x, const float *W, const float *b,
                             float *y, int64_t T, int64_t in, int64_t out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_forward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0) return NUMRS_HIP_OK;
  if (y == nullptr || (in > 0 && (x == nullptr || W == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (in == 0) {  // empty product: y = b broadcast over rows (or 0)
    if (int rc = numrs_hip_fill(ctx, y, T * out, 0.0f)) return rc;
    if (b == nullptr) return NUMRS_HIP_OK;
    const int64_t bs = out;
    const int64_t ys[2] = {T, out};
    return numrs_hip_binary_forward(ctx, NUMRS_HIP_ADD, y, ys, 2, b, &bs, 1, y);
  }
  // y[T,out] = x[T,in] @ W[out,in]^T + b : X = x (R-contig), Y = W^T (R-contig)
  Gemm g = make(x, W, y, in, in, out, 0, 0, 0, T, out, in, 0);
  g.bias = b;
  return gemm_dispatch(ctx, g, 1, true, true);
}

int numrs_hip_linear_backward(numrs_hip_ctx *ctx, const float *g, const float *x, const float *W,
                              float *dx, float *dW, float *db, int64_t T, int64_t in, int64_t out,
                              int acc_dx, int acc_dw, int acc_db, int mode) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_backward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (g == nullptr || (dx && W == nullptr) || (dW && x == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  if (T == 0 || out == 0) {  // empty reductions: zero gradients
    if (dx && !acc_dx && T * in > 0)
      if (int rc = numrs_hip_fill(ctx, dx, T * in, 0.0f)) return rc;
    if (dW && !acc_dw && out * in > 0)
      if (int rc = numrs_hip_fill(ctx, dW, out * in, 0.0f)) return rc;
  } else {
    // db = column sums of g (CORRECT mode), formed by the pair's own launch
    // (tiny products) or by the launch that reduces its splits, rather than
    // by two launches of their own
    ColSum cs{g, db, T, out, out, acc_db};
    const bool want_db = db != nullptr && mode == NUMRS_HIP_UNBROADCAST_CORRECT;
    bool db_done = false;
    if (in > 0) {
      // dx[T,in] = g[T,out] @ W[out,in] : X = g (R-contig), Y = W (Q-contig)  [NN]
      Gemm gx = make(g, W, dx, out, in, in, 0, 0, 0, T, in, out, acc_dx);
      // dW[out,in] = g^T @ x : X = g^T (P-contig), Y = x (Q-contig)          [TN]
      Gemm gw = make(g, x, dW, out, in, in, 0, 0, 0, out, in, T, acc_dw);
      if (int rc = launch_pair(ctx, gx, gw, false, who, want_db ? &cs : nullptr, &db_done))
        return rc;
    } else if (want_db && colsum_fits(g, T, out, out)) {
      if (int rc = reduce_splits(ctx, nullptr, nullptr, &cs)) return rc;
      db_done = true;
    }
    if (db_done) return NUMRS_HIP_OK;
  }
  if (db == nullptr || out == 0) return NUMRS_HIP_OK;
  const int64_t gs[2] = {T, out};
  const int64_t bs = out;
  return numrs_hip_sum_to_shape(ctx, g, gs, 2, db, &bs, 1, mode, acc_db);
}

int numrs_hip_linear_relu_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                  const float *b, float *y, int64_t T, int64_t in, int64_t out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_relu_forward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0) return NUMRS_HIP_OK;
  if (y == nullptr || (in > 0 && (x == nullptr || W == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (in == 0) {  // empty product: ReLU of the broadcast bias
    if (int rc = numrs_hip_linear_forward(ctx, x, W, b, y, T, in, out)) return rc;
    return numrs_hip_unary_forward(ctx, NUMRS_HIP_RELU, y, y, T * out, 0.0f);
  }
  Gemm g = make(x, W, y, in, in, out, 0, 0, 0, T, out, in, 0);
  g.bias = b;
  g.act = kActRelu;
  return gemm_dispatch(ctx, g, 1, true, true);
}

int numrs_hip_linear_gelu_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                  const float *b, float *y, float *pre, int64_t T, int64_t in,
                                  int64_t out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_gelu_forward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0) return NUMRS_HIP_OK;
  if (y == nullptr || pre == nullptr || pre == y || (in > 0 && (x == nullptr || W == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null or aliased pointer", who);
  if (in == 0) {  // empty product: GELU of the broadcast bias
    if (int rc = numrs_hip_linear_forward(ctx, x, W, b, pre, T, in, out)) return rc;
    return numrs_hip_unary_forward(ctx, NUMRS_HIP_GELU, pre, y, T * out, 0.0f);
  }
  Gemm g = make(x, W, y, in, in, out, 0, 0, 0, T, out, in, 0);
  g.bias = b;
  g.act = kActGelu;
  g.pre = pre;
  return gemm_dispatch(ctx, g, 1, true, true);
}

int numrs_hip_linear_gelu_backward(numrs_hip_ctx *ctx, const float *g, const float *pre,
                                   const float *x, const float *W, float *dx, float *dW,
                                   float *db, int64_t T, int64_t in, int64_t out, int acc_dx,
                                   int acc_dw, int acc_db, int mode) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_gelu_backward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0)
    return numrs_hip_linear_backward(ctx, g, x, W, dx, dW, db, T, in, out, acc_dx, acc_dw, acc_db,
                                     mode);
  if (g == nullptr || pre == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  // The pre-activation gradient g * GELU'(pre), then the Linear backward.
  numrs_hip::TempBlock gp(ctx);
  if (int rc = gp.alloc((size_t)T * out * sizeof(float))) return rc;
  if (int rc = numrs_hip_unary_backward(ctx, NUMRS_HIP_GELU, g, pre, gp.f(), T * out, 0.0f, 0))
    return rc;
  return numrs_hip_linear_backward(ctx, gp.f(), x, W, dx, dW, db, T, in, out, acc_dx, acc_dw,
                                   acc_db, mode);
}

int numrs_hip_linear_relu_backward(numrs_hip_ctx *ctx, const float *g, const float *y,
                                   const float *x, const float *W, float *dx, float *dW,
                                   float *db, int64_t T, int64_t in, int64_t out, int acc_dx,
                                   int acc_dw, int acc_db, int mode) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_relu_backward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0)  // empty reductions: the Linear backward's zero gradients
    return numrs_hip_linear_backward(ctx, g, x, W, dx, dW, db, T, in, out, acc_dx, acc_dw, acc_db,
                                     mode);
  if (g == nullptr || y == nullptr || (dx && W == nullptr) || (dW && x == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  if ((dx != nullptr || dW != nullptr) && in > 0 &&
      (db == nullptr || (mode == NUMRS_HIP_UNBROADCAST_CORRECT && T <= kTinyColsumRows))) {
    // The pre-activation gradient (y > 0 ? g : 0) applied as the tiny
    // kernel loads g: one launch for dx, dW and db.
    Gemm gx = make(g, W, dx, out, in, in, 0, 0, 0, T, in, out, acc_dx);
    Gemm gw = make(g, x, dW, out, in, in, 0, 0, 0, out, in, T, acc_dw);
    gx.xmask = gw.xmask = y;
    if ((dx == nullptr || tiny_fits(gx, 1)) && (dW == nullptr || tiny_fits(gw, 1))) {
      const ColSum cs{g, db, T, out, out, acc_db, y};
      const ColSum *csp = db != nullptr ? &cs : nullptr;
      if (dx != nullptr) return launch_tiny(ctx, gx, true, false, dW ? &gw : nullptr, 1, csp);
      return launch_tiny(ctx, gw, false, false, nullptr, 1, csp);
    }
  }
  // Otherwise the masked gradient first, then the Linear backward on it.
  if ((dx == nullptr && dW == nullptr) || in == 0) {
    if (int rc = numrs_hip_linear_backward(ctx, g, x, W, dx, dW, nullptr, T, in, out, acc_dx,
                                           acc_dw, 0, mode))
      return rc;
    return db ? numrs_hip_relu_bias_backward(ctx, g, y, nullptr, db, T, out, mode, acc_db)
              : NUMRS_HIP_OK;
  }
  numrs_hip::TempBlock gm(ctx);
  if (int rc = gm.alloc((size_t)T * out * sizeof(float))) return rc;
  if (int rc = numrs_hip_relu_bias_backward(ctx, g, y, gm.f(), nullptr, T, out, mode, 0))
    return rc;
  return numrs_hip_linear_backward(ctx, gm.f(), x, W, dx, dW, db, T, in, out, acc_dx, acc_dw,
                                   acc_db, mode);
}

int numrs_hip_linear_residual_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                      const float *b, const float *res, float *y, int64_t T,
                                      int64_t in, int64_t out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_linear_residual_forward";
  if (int rc = check_dims(ctx, who, 1, T, in, out)) return rc;
  if (T == 0 || out == 0) return NUMRS_HIP_OK;
  if (y == nullptr || res == nullptr || (in > 0 && (x == nullptr || W == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (in == 0) {  // empty product: y = b broadcast over rows (or 0), then + res
    if (int rc = numrs_hip_linear_forward(ctx, x, W, b, y, T, in, out)) return rc;
    const int64_t ys[2] = {T, out};
    return numrs_hip_binary_forward(ctx, NUMRS_HIP_ADD, res, ys, 2, y, ys, 2, y);
  }
  Gemm g = make(x, W, y, in, in, out, 0, 0, 0, T, out, in, 0);
  g.bias = b;
  g.res = res;
  g.ldr = out;
  return gemm_dispatch(ctx, g, 1, true, true);
}

int numrs_hip_gemm(numrs_hip_ctx *ctx, const float *A, int64_t lda, const float *B, int64_t ldb,
                   float *C, int64_t ldc, int64_t M, int64_t K, int64_t N, int trans_a,
                   int trans_b, float alpha, int accumulate, int64_t batch, int64_t batch_inner,
                   int64_t sa_outer, int64_t sa_inner, int64_t sb_outer, int64_t sb_inner,
                   int64_t sc_outer, int64_t sc_inner) {
  NRS_CHECK_CTX(ctx);
  return gemm_general(ctx, A, lda, B, ldb, C, ldc, M, K, N, trans_a, trans_b, alpha, accumulate,
                      batch, batch_inner, sa_outer, sa_inner, sb_outer, sb_inner, sc_outer,
                      sc_inner);
}

int numrs_hip_matmul_backward(numrs_hip_ctx *ctx, const float *dC, const float *A,
                              const float *B, float *dA, float *dB, int64_t M, int64_t K,
                              int64_t N, int accumulate) {
  NRS_CHECK_CTX(ctx);
  return matmul_backward_impl(ctx, dC, A, B, dA, dB, 1, M, K, N, 0, 0, 0, accumulate);
}

int numrs_hip_matmul_backward_batched(numrs_hip_ctx *ctx, const float *dC, const float *A,
                                      const float *B, float *dA, float *dB, int64_t batch,
                                      int64_t M, int64_t K, int64_t N, int64_t stride_a,
                                      int64_t stride_b, int64_t stride_c, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (stride_a < 0 || stride_b < 0 || stride_c < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "negative batch stride");
  return matmul_backward_impl(ctx, dC, A, B, dA, dB, batch, M, K, N, stride_a, stride_b,
                              stride_c, accumulate);
}

int numrs_hip_matmul(numrs_hip_ctx *ctx, const float *A, const float *B, float *C, int64_t M,
                     int64_t K, int64_t N, int trans_a, int trans_b, int accumulate) {
  NRS_CHECK_CTX(ctx);
  return matmul_impl(ctx, A, B, C, 1, M, K, N, 0, 0, 0, trans_a, trans_b, accumulate);
}

int numrs_hip_matmul_batched(numrs_hip_ctx *ctx, const float *A, const float *B, float *C,
                             int64_t batch, int64_t M, int64_t K, int64_t N, int64_t stride_a,
                             int64_t stride_b, int64_t stride_c, int trans_a, int trans_b,
                             int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (stride_a < 0 || stride_b < 0 || stride_c < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "negative batch stride");
  return matmul_impl(ctx, A, B, C, batch, M, K, N, stride_a, stride_b, stride_c, trans_a,
                     trans_b, accumulate);
}

}  // extern "C"
