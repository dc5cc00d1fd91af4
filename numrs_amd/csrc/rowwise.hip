// Row-wise kernels: softmax + cross-entropy backward, softmax backward, row
// argmax.  One wave64 owns one row; a 256-thread block holds four rows.  Row
// statistics (max, exp-sum, dot) are wave shuffles, so no LDS or barriers.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kRowsPerBlock = kBlock / 64;

// cross_entropy_backward, backward.rs:265-301:
//   m = max_j x_j (f32::max fold, NaN ignored)      backward.rs:285
//   s = sum_j exp(x_j - m)                           backward.rs:286
//   dx_j = (exp(x_j - m) / s - t_j) * (g / B)        backward.rs:273,289-291
template <bool LABELS>
__global__ void __launch_bounds__(kBlock)
    softmax_ce_bwd_kernel(const float *__restrict__ g0, const float *__restrict__ x,
                          const float *__restrict__ onehot, const int32_t *__restrict__ labels,
                          float *__restrict__ dx, int64_t B, int64_t C, int acc) {
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
  const float scale = g0[0] / (float)B;
  const int32_t label = LABELS ? labels[row] : -1;
  float *out = dx + row * C;
  for (int64_t j = lane; j < C; j += 64) {
    const float t = LABELS ? (j == (int64_t)label ? 1.0f : 0.0f) : onehot[row * C + j];
    const float sm = expf(xr[j] - m) / s;
    const float v = (sm - t) * scale;
    out[j] = acc ? out[j] + v : v;
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
__device__ __forceinline__ bool better_first(float v, int64_t i, float bv, int64_t bi) {
  // Candidate (v, i) beats (bv, bi) under "first strict maximum".
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ bool better_last(float v, int64_t i, float bv, int64_t bi) {
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

}  // namespace

extern "C" {

int numrs_hip_softmax_ce_backward(numrs_hip_ctx *ctx, const float *g_scalar, const float *logits,
                                  const float *onehot, const int32_t *labels, float *dlogits,
                                  int64_t B, int64_t C, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_softmax_ce_backward";
  if (B < 0 || C < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (B == 0 || C == 0) return NUMRS_HIP_OK;
  if (g_scalar == nullptr || logits == nullptr || dlogits == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if ((onehot == nullptr) == (labels == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: pass exactly one of onehot/labels", who);
  const unsigned grid = grid_for(B, kRowsPerBlock);
  if (labels != nullptr)
    softmax_ce_bwd_kernel<true><<<grid, kBlock, 0, ctx->stream>>>(g_scalar, logits, onehot, labels,
                                                                  dlogits, B, C, accumulate);
  else
    softmax_ce_bwd_kernel<false><<<grid, kBlock, 0, ctx->stream>>>(g_scalar, logits, onehot,
                                                                   labels, dlogits, B, C,
                                                                   accumulate);
  return numrs_hip::check_launch(ctx, "softmax_ce_bwd_kernel");
}

int numrs_hip_softmax_backward(numrs_hip_ctx *ctx, const float *y, const float *g, float *dx,
                               int64_t rows, int64_t cols, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_softmax_backward";
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (rows == 0 || cols == 0) return NUMRS_HIP_OK;
  if (y == nullptr || g == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  softmax_bwd_kernel<<<grid_for(rows, kRowsPerBlock), kBlock, 0, ctx->stream>>>(y, g, dx, rows,
                                                                                cols, accumulate);
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
  argmax_kernel<<<grid_for(rows, kRowsPerBlock), kBlock, 0, ctx->stream>>>(x, idx, rows, cols,
                                                                           tie_last ? 1 : 0);
  return numrs_hip::check_launch(ctx, "argmax_kernel");
}

}  // extern "C"
