// Row-wise kernels: softmax + cross-entropy backward, softmax backward, row
// argmax.  One wave64 owns one row; a 256-thread block holds four rows.  Row
// statistics (max, exp-sum, dot) are wave shuffles, so no LDS or barriers.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kRowsPerBlock = kBlock / 64;

typedef float f4 __attribute__((ext_vector_type(4)));

// Register-resident variants (rows of at most 256*NV columns, cols % 4 == 0,
// 16-byte aligned operands): lane l holds the float4 column groups l,
// l + 64, ... (NV of them), so a row is read from memory once, with float4
// loads, and every row statistic is computed from registers.  Longer or
// unaligned rows use the looped kernels.
template <int NV>
__device__ __forceinline__ int64_t vcol(int lane, int i) {
  return 4 * (int64_t)(lane + 64 * i);
}

// The float4 at column c of row r, for every lane: a column past the row end
// reloads the row's last float4 instead (cols % 4 == 0 and cols >= 4 on the
// register-resident path), so the load needs no branch.  Callers ignore the
// values of such columns.  A load under `if (c < cols)` would make each
// column group its own memory round trip.
template <int VM = 1>
__device__ __forceinline__ f4 load_cols(const float *r, int64_t c, int64_t cols) {
  return numrs_hip::ldv<VM>(r + (c < cols ? c : cols - 4));
}

// cross_entropy_backward, backward.rs:265-301:
//   m = max_j x_j (f32::max fold, NaN ignored)      backward.rs:285
//   s = sum_j exp(x_j - m)                           backward.rs:286
//   dx_j = (exp(x_j - m) / s - t_j) * (g / B)        backward.rs:273,289-291
template <bool LABELS>
__global__ void __launch_bounds__(kBlock)
    softmax_ce_bwd_kernel(const float *__restrict__ g0, const float *__restrict__ x,
                          const float *__restrict__ onehot, const int32_t *__restrict__ labels,
                          float *__restrict__ dx, int64_t B, int64_t C, int acc,
                          float *__restrict__ seed) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const float *xr = x + row * C;
  float m = -INFINITY;
  for (int64_t j = lane; j < C; j += 64) m = fmaxf(m, xr[j]);
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t j = lane; j < C; j += 64) s += expf(xr[j] - m);
  s = wave_sum(s);
  // seed: the loss is the sweep's root; g is its seed 1, written to seed[0]
  if (seed != nullptr && blockIdx.x == 0 && threadIdx.x == 0) seed[0] = 1.0f;
  const float scale = (seed != nullptr ? 1.0f : g0[0]) / (float)B;
  const int32_t label = LABELS ? labels[row] : -1;
  float *out = dx + row * C;
  for (int64_t j = lane; j < C; j += 64) {
    const float t = LABELS ? (j == (int64_t)label ? 1.0f : 0.0f) : onehot[row * C + j];
    const float sm = expf(xr[j] - m) / s;
    const float v = (sm - t) * scale;
    out[j] = acc ? out[j] + v : v;
  }
}

template <bool LABELS, int NV, int VM>
__global__ void __launch_bounds__(kBlock)
    softmax_ce_bwd_vec(const float *__restrict__ g0, const float *__restrict__ x,
                       const float *__restrict__ onehot, const int32_t *__restrict__ labels,
                       float *__restrict__ dx, int64_t B, int64_t C, int acc,
                          float *__restrict__ seed) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const float *xr = x + row * C;
  f4 xv[NV], tv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = vcol<NV>(lane, i);
    xv[i] = load_cols<VM>(xr, c, C);
    if (!LABELS) tv[i] = load_cols<VM>(onehot + row * C, c, C);
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (vcol<NV>(lane, i) < C) {
#pragma unroll
      for (int e = 0; e < 4; ++e) m = fmaxf(m, xv[i][e]);  // backward.rs:285
    }
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (vcol<NV>(lane, i) < C) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[i][e] = expf(xv[i][e] - m);  // backward.rs:286
        s += xv[i][e];
      }
    }
  }
  s = wave_sum(s);
  // seed: the loss is the sweep's root; g is its seed 1, written to seed[0]
  if (seed != nullptr && blockIdx.x == 0 && threadIdx.x == 0) seed[0] = 1.0f;
  const float scale = (seed != nullptr ? 1.0f : g0[0]) / (float)B;
  const int32_t label = LABELS ? labels[row] : -1;
  float *out = dx + row * C;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = vcol<NV>(lane, i);
    if (c < C) {
      f4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = LABELS ? (c + e == (int64_t)label ? 1.0f : 0.0f) : tv[i][e];
        v[e] = (xv[i][e] / s - t) * scale;  // backward.rs:289-291
      }
      if (acc) v += numrs_hip::ldv<VM>(out + c);
      numrs_hip::stv<VM>(out + c, v);
    }
  }
}

// softmax_backward, backward.rs:521-541: dx = y * (g - sum_row(g * y)).
// g and dx may alias (in-place use by attention): each lane reads g[j] before
// it writes dx[j], and the row dot product is complete before any write.
__global__ void __launch_bounds__(kBlock)
    softmax_bwd_kernel(const float *__restrict__ y, const float *g, float *dx, int64_t rows,
                       int64_t cols, int acc) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *yr = y + row * cols, *gr = g + row * cols;
  float d = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) d += gr[j] * yr[j];
  d = wave_sum(d);
  float *out = dx + row * cols;
  for (int64_t j = lane; j < cols; j += 64) {
    const float v = yr[j] * (gr[j] - d);
    out[j] = acc ? out[j] + v : v;
  }
}

template <int NV, int VM>
__global__ void __launch_bounds__(kBlock)
    softmax_bwd_vec(const float *__restrict__ y, const float *g, float *dx, int64_t rows,
                    int64_t cols, int acc) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *yr = y + row * cols, *gr = g + row * cols;
  f4 yv[NV], gv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = vcol<NV>(lane, i);
    yv[i] = load_cols<VM>(yr, c, cols);
    gv[i] = load_cols<VM>(gr, c, cols);
  }
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (vcol<NV>(lane, i) < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) d += gv[i][e] * yv[i][e];
    }
  }
  d = wave_sum(d);  // every lane's reads of g are done before any write below
  float *out = dx + row * cols;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = vcol<NV>(lane, i);
    if (c < cols) {
      f4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = yv[i][e] * (gv[i][e] - d);
      if (acc) v += numrs_hip::ldv<VM>(out + c);
      numrs_hip::stv<VM>(out + c, v);
    }
  }
}

// Row argmax with an explicit tie rule.
//   tie_last = 0 (ops::argmax, backend/cpu/scalar.rs:517-528): a sequential
//     scan that replaces only on strict '>'.  NaN never replaces; a NaN in
//     column 0 is never replaced, so the answer is 0.  Otherwise the answer
//     is the first index holding the maximum of the non-NaN values.
//   tie_last = 1 (Iterator::max_by with partial_cmp, NaN = Equal,
//     autograd/train.rs:213-228): the scan replaces unless current > new, so
//     a NaN (and everything compared with it) replaces; the answer is the last
//     index holding the maximum of the values after the last NaN, or the last
//     NaN's index when it is the final element.
// Both are evaluated as a lane-parallel scan over contiguous segments and a
// wave combine that applies the same rule to (value, index) pairs.
template <typename I>
__device__ __forceinline__ bool better_first(float v, I i, float bv, I bi) {
  // Candidate (v, i) beats (bv, bi) under "first strict maximum".
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

template <typename I>
__device__ __forceinline__ bool better_last(float v, I i, float bv, I bi) {
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i > bi);
}

__global__ void __launch_bounds__(kBlock)
    argmax_kernel(const float *__restrict__ x, int32_t *__restrict__ idx, int64_t rows,
                  int64_t cols, int tie_last) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + row * cols;
  int64_t start = 0;
  if (tie_last) {
    // Last NaN position: the scan restarts after it.
    int64_t last_nan = -1;
    for (int64_t j = lane; j < cols; j += 64)
      if (xr[j] != xr[j]) last_nan = j;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const int64_t o = __shfl_xor(last_nan, off, 64);
      last_nan = o > last_nan ? o : last_nan;
    }
    if (last_nan == cols - 1) {
      if (lane == 0) idx[row] = (int32_t)last_nan;
      return;
    }
    start = last_nan + 1;
  } else if (xr[0] != xr[0]) {
    if (lane == 0) idx[row] = 0;
    return;
  }
  float bv = NAN;
  int64_t bi = -1;
  for (int64_t j = start + lane; j < cols; j += 64) {
    const float v = xr[j];
    const bool take = tie_last ? better_last(v, j, bv, bi) : better_first(v, j, bv, bi);
    if (take) {
      bv = v;
      bi = j;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int64_t oi = __shfl_xor(bi, off, 64);
    const bool take = (oi >= 0) && (bi < 0 || (tie_last ? better_last(ov, oi, bv, bi)
                                                        : better_first(ov, oi, bv, bi)));
    if (take) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) idx[row] = (int32_t)(bi < 0 ? start : bi);
}

// (bv, bi) <- the better of (bv, bi) and (ov, oi); bi < 0 is an empty slot.
template <bool TIE_LAST>
__device__ __forceinline__ void pick_pair(float &bv, int &bi, float ov, int oi) {
  const bool take = (oi >= 0) && (bi < 0 || (TIE_LAST ? better_last(ov, oi, bv, bi)
                                                      : better_first(ov, oi, bv, bi)));
  if (take) {
    bv = ov;
    bi = oi;
  }
}

template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// Every lane ends with the wave's best (value, index) pair: the exchange
// pattern of wave_butterfly (permlane32/16 swaps, then DPP row
// and quad moves), applied to both halves of the pair.
template <bool TIE_LAST>
__device__ __forceinline__ void pair_butterfly(float &bv, int &bi) {
  {
    const unsigned uv = __builtin_bit_cast(unsigned, bv), ui = (unsigned)bi;
    const auto rv = __builtin_amdgcn_permlane32_swap(uv, uv, false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(ui, ui, false, false);
    bv = __builtin_bit_cast(float, (unsigned)rv[0]);
    bi = (int)(unsigned)ri[0];
    pick_pair<TIE_LAST>(bv, bi, __builtin_bit_cast(float, (unsigned)rv[1]), (int)(unsigned)ri[1]);
  }
  {
    const unsigned uv = __builtin_bit_cast(unsigned, bv), ui = (unsigned)bi;
    const auto rv = __builtin_amdgcn_permlane16_swap(uv, uv, false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(ui, ui, false, false);
    bv = __builtin_bit_cast(float, (unsigned)rv[0]);
    bi = (int)(unsigned)ri[0];
    pick_pair<TIE_LAST>(bv, bi, __builtin_bit_cast(float, (unsigned)rv[1]), (int)(unsigned)ri[1]);
  }
  pick_pair<TIE_LAST>(bv, bi, dpp_mov<0x128>(bv), dpp_mov_i<0x128>(bi));  // row_ror:8
  pick_pair<TIE_LAST>(bv, bi, dpp_mov<0x1B>(dpp_mov<0x141>(bv)),
                      dpp_mov_i<0x1B>(dpp_mov_i<0x141>(bi)));  // row_half_mirror, quad [3,2,1,0]
  pick_pair<TIE_LAST>(bv, bi, dpp_mov<0x4E>(bv), dpp_mov_i<0x4E>(bi));  // quad [2,3,0,1]
  pick_pair<TIE_LAST>(bv, bi, dpp_mov<0xB1>(bv), dpp_mov_i<0xB1>(bi));  // quad [1,0,3,2]
}

// Argmax of a register-resident row (lane l holds the float4 groups
// vcol<NV>(l, i)).  A lane visits its elements in increasing column order,
// so within a lane the tie rule reduces to one comparison: first max keeps
// the earlier element (replace on strict '>'), last max takes the later one
// ('>=').  Columns fit in int32 (the host checks), so indices are 32-bit.
template <int NV, bool TIE_LAST>
__device__ __forceinline__ int argmax_regs(const f4 (&xv)[NV], int ncols, int lane) {
  int start = 0;
  if (TIE_LAST) {
    // Last NaN position: the scan restarts after it.
    int last_nan = -1;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (int)vcol<NV>(lane, i);
      if (c < ncols) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (xv[i][e] != xv[i][e]) last_nan = c + e;
      }
    }
    last_nan = __builtin_bit_cast(int, wave_butterfly(
                   __builtin_bit_cast(float, last_nan),
                   [](float a, float b) {
                     return __builtin_bit_cast(float, max(__builtin_bit_cast(int, a),
                                                          __builtin_bit_cast(int, b)));
                   }));
    if (last_nan == ncols - 1) return last_nan;
    start = last_nan + 1;
  } else {
    // x[0] is lane 0's first element; a NaN there stays the maximum.
    const float x0 = __builtin_bit_cast(
        float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, xv[0][0])));
    if (x0 != x0) return 0;
  }
  // Lane scan.  No NaN lies at or after `start` with TIE_LAST; without it a
  // NaN never replaces.
  float bv = 0.0f;
  int bi = -1;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (int)vcol<NV>(lane, i);
    if (c < ncols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = xv[i][e];
        const int j = c + e;
        const bool take = TIE_LAST ? (j >= start && (bi < 0 || v >= bv))
                                   : (v == v && (bi < 0 || v > bv));
        if (take) {
          bv = v;
          bi = j;
        }
      }
    }
  }
  // Wave combine of (value, index) pairs with the full rule, over the lane
  // pairs of an xor butterfly (distances 32, 16, ..., 1), exchanged in
  // registers.  Indices are distinct and the rule is a strict order, so the
  // pair's winner does not depend on which lane holds which operand.
  pair_butterfly<TIE_LAST>(bv, bi);
  return bi < 0 ? start : bi;
}

template <int NV, int VM>
__device__ __forceinline__ void load_row_regs(f4 (&xv)[NV], const float *xr, int ncols, int lane) {
#pragma unroll
  for (int i = 0; i < NV; ++i) xv[i] = load_cols<VM>(xr, vcol<NV>(lane, i), ncols);
}

// One wave per row.  (Measured on MI355X at [16384, 1024]: persistent
// waves that load the next row before reducing the current one ran 10-20%
// slower than this one-shot form, and waves of two rows with all eight
// loads issued first 3% slower.)
template <int NV, bool TIE_LAST, int VM>
__global__ void __launch_bounds__(kBlock)
    argmax_vec(const float *__restrict__ x, int32_t *__restrict__ idx, int64_t rows,
               int64_t cols) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // row is uniform over the wave
  const int ncols = (int)cols;
  f4 xv[NV];
  load_row_regs<NV, VM>(xv, x + row * cols, ncols, lane);
  const int r = argmax_regs<NV, TIE_LAST>(xv, ncols, lane);
  if (lane == 0) idx[row] = r;
}

// Softmax along an inner axis of x[outer, n, inner] (no reference kernel:
// ops/stats/softmax.rs:13-16 rejects an axis).  One thread per (o, i)
// walks the axis with stride `inner`; a wave's threads hold consecutive
// inner indices, so the loads are coalesced.  y = exp(x - max) / sum.
__global__ void __launch_bounds__(kBlock)
    softmax_axis_fwd_kernel(const float *x, float *y, int64_t outer, int64_t n, int64_t inner) {
  const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (o >= outer * inner) return;
  const int64_t b = o / inner, i = o - b * inner;
  const float *src = x + b * n * inner + i;
  float *dst = y + b * n * inner + i;
  float m = -INFINITY;
  for (int64_t k = 0; k < n; ++k) m = fmaxf(m, src[k * inner]);
  float s = 0.0f;
  for (int64_t k = 0; k < n; ++k) s += expf(src[k * inner] - m);
  for (int64_t k = 0; k < n; ++k) dst[k * inner] = expf(src[k * inner] - m) / s;
}

// softmax_backward (backward.rs:521-541) along an inner axis:
// dx = y * (g - sum_axis(g * y)).
__global__ void __launch_bounds__(kBlock)
    softmax_axis_bwd_kernel(const float *__restrict__ y, const float *g, float *dx, int64_t outer,
                            int64_t n, int64_t inner, int acc) {
  const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (o >= outer * inner) return;
  const int64_t b = o / inner, i = o - b * inner;
  const int64_t base = b * n * inner + i;
  float d = 0.0f;
  for (int64_t k = 0; k < n; ++k) d += g[base + k * inner] * y[base + k * inner];
  for (int64_t k = 0; k < n; ++k) {
    const int64_t j = base + k * inner;
    const float v = y[j] * (g[j] - d);
    dx[j] = acc ? dx[j] + v : v;
  }
}

// Number of float4 groups per lane for a register-resident row, or 0 when the
// looped kernel must be used.
inline int row_nv(int64_t cols, bool aligned) {
  if (!aligned || (cols & 3) != 0) return 0;
  if (cols <= 256) return 1;
  if (cols <= 512) return 2;
  if (cols <= 1024) return 4;
  if (cols <= 2048) return 8;
  return 0;
}

}  // namespace

namespace numrs_hip {

// softmax_ce_backward; with `seed` (the loss is the sweep's root) g is its
// seed 1, which the kernel also writes to seed[0].
int softmax_ce_backward_impl(numrs_hip_ctx *ctx, const float *g_scalar, float *seed,
                             const float *logits, const float *onehot, const int32_t *labels,
                             float *dlogits, int64_t B, int64_t C, int accumulate) {
  const char *who = "numrs_hip_softmax_ce_backward";
  if (B < 0 || C < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (B == 0 || C == 0) return seed != nullptr ? numrs_hip_fill(ctx, seed, 1, 1.0f) : NUMRS_HIP_OK;
  if ((g_scalar == nullptr && seed == nullptr) || logits == nullptr || dlogits == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if ((onehot == nullptr) == (labels == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: pass exactly one of onehot/labels", who);
  const unsigned grid = grid_for(B, kRowsPerBlock);
  const int nv = row_nv(C, numrs_hip::aligned16(logits) && numrs_hip::aligned16(dlogits) &&
                               (onehot == nullptr || numrs_hip::aligned16(onehot)));
#define NRS_CE_VEC(NV)                                                                        \
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, B * C), [&](auto V) {                     \
    if (labels != nullptr)                                                                    \
      softmax_ce_bwd_vec<true, NV, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(      \
          g_scalar, logits, onehot, labels, dlogits, B, C, accumulate, seed);                       \
    else                                                                                      \
      softmax_ce_bwd_vec<false, NV, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(     \
          g_scalar, logits, onehot, labels, dlogits, B, C, accumulate, seed);                       \
  });                                                                                         \
  return numrs_hip::check_launch(ctx, "softmax_ce_bwd_vec");
  switch (nv) {
    case 1: { NRS_CE_VEC(1) }
    case 2: { NRS_CE_VEC(2) }
    case 4: { NRS_CE_VEC(4) }
    case 8: { NRS_CE_VEC(8) }
    default: break;
  }
#undef NRS_CE_VEC
  if (labels != nullptr)
    softmax_ce_bwd_kernel<true><<<grid, kBlock, 0, ctx->stream>>>(g_scalar, logits, onehot, labels,
                                                                  dlogits, B, C, accumulate, seed);
  else
    softmax_ce_bwd_kernel<false><<<grid, kBlock, 0, ctx->stream>>>(g_scalar, logits, onehot,
                                                                   labels, dlogits, B, C,
                                                                   accumulate, seed);
  return numrs_hip::check_launch(ctx, "softmax_ce_bwd_kernel");
}

}  // namespace numrs_hip

extern "C" {

int numrs_hip_softmax_ce_backward(numrs_hip_ctx *ctx, const float *g_scalar, const float *logits,
                                  const float *onehot, const int32_t *labels, float *dlogits,
                                  int64_t B, int64_t C, int accumulate) {
  NRS_CHECK_CTX(ctx);
  return numrs_hip::softmax_ce_backward_impl(ctx, g_scalar, nullptr, logits, onehot, labels,
                                             dlogits, B, C, accumulate);
}

int numrs_hip_softmax_backward(numrs_hip_ctx *ctx, const float *y, const float *g, float *dx,
                               int64_t rows, int64_t cols, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_softmax_backward";
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (rows == 0 || cols == 0) return NUMRS_HIP_OK;
  if (y == nullptr || g == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  const unsigned grid = grid_for(rows, kRowsPerBlock);
  const int nv = row_nv(cols, numrs_hip::aligned16(y) && numrs_hip::aligned16(g) &&
                                  numrs_hip::aligned16(dx));
  if (nv == 0) {
    softmax_bwd_kernel<<<grid, kBlock, 0, ctx->stream>>>(y, g, dx, rows, cols, accumulate);
    return numrs_hip::check_launch(ctx, "softmax_bwd_kernel");
  }
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, rows * cols), [&](auto V) {
    constexpr int VM = decltype(V)::value;
    switch (nv) {
      case 1: softmax_bwd_vec<1, VM><<<grid, kBlock, 0, ctx->stream>>>(y, g, dx, rows, cols, accumulate); break;
      case 2: softmax_bwd_vec<2, VM><<<grid, kBlock, 0, ctx->stream>>>(y, g, dx, rows, cols, accumulate); break;
      case 4: softmax_bwd_vec<4, VM><<<grid, kBlock, 0, ctx->stream>>>(y, g, dx, rows, cols, accumulate); break;
      default: softmax_bwd_vec<8, VM><<<grid, kBlock, 0, ctx->stream>>>(y, g, dx, rows, cols, accumulate); break;
    }
  });
  return numrs_hip::check_launch(ctx, "softmax_bwd_kernel");
}

int numrs_hip_argmax_rows(numrs_hip_ctx *ctx, const float *x, int32_t *idx, int64_t rows,
                          int64_t cols, int tie_last) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_argmax_rows";
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (rows == 0) return NUMRS_HIP_OK;
  if (cols == 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "%s: argmax of an empty row", who);
  if (cols > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: row too long", who);
  if (x == nullptr || idx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  const unsigned grid = grid_for(rows, kRowsPerBlock);
  const int tl = tie_last ? 1 : 0;
#define NRS_ARGMAX_VEC(NV)                                                                \
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, rows * cols), [&](auto V) {           \
    if (tl)                                                                               \
      argmax_vec<NV, true, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(x, idx, rows, \
                                                                                  cols);     \
    else                                                                                  \
      argmax_vec<NV, false, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(x, idx,   \
                                                                                   rows, cols); \
  });                                                                                     \
  break;
  switch (row_nv(cols, numrs_hip::aligned16(x))) {
    case 1: NRS_ARGMAX_VEC(1)
    case 2: NRS_ARGMAX_VEC(2)
    case 4: NRS_ARGMAX_VEC(4)
    case 8: NRS_ARGMAX_VEC(8)
    default: argmax_kernel<<<grid, kBlock, 0, ctx->stream>>>(x, idx, rows, cols, tl);
  }
#undef NRS_ARGMAX_VEC
  return numrs_hip::check_launch(ctx, "argmax_kernel");
}

int numrs_hip_softmax_axis_forward(numrs_hip_ctx *ctx, const float *x, float *y, int64_t outer,
                                   int64_t n, int64_t inner) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_softmax_axis_forward";
  if (outer < 0 || n < 0 || inner < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (outer * n * inner == 0) return NUMRS_HIP_OK;
  if (x == nullptr || y == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (inner == 1) return numrs_hip_softmax_forward(ctx, x, y, outer, n, 1.0f);
  softmax_axis_fwd_kernel<<<grid_for(outer * inner, kBlock), kBlock, 0, ctx->stream>>>(
      x, y, outer, n, inner);
  return numrs_hip::check_launch(ctx, "softmax_axis_fwd_kernel");
}

int numrs_hip_softmax_axis_backward(numrs_hip_ctx *ctx, const float *y, const float *g, float *dx,
                                    int64_t outer, int64_t n, int64_t inner, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_softmax_axis_backward";
  if (outer < 0 || n < 0 || inner < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (outer * n * inner == 0) return NUMRS_HIP_OK;
  if (y == nullptr || g == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (inner == 1) return numrs_hip_softmax_backward(ctx, y, g, dx, outer, n, accumulate);
  softmax_axis_bwd_kernel<<<grid_for(outer * inner, kBlock), kBlock, 0, ctx->stream>>>(
      y, g, dx, outer, n, inner, accumulate);
  return numrs_hip::check_launch(ctx, "softmax_axis_bwd_kernel");
}

}  // extern "C"
