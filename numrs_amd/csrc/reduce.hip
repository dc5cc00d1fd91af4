// Broadcast-reduce gradients: unbroadcast / sum-to-shape (backward.rs:12-39)
// and the fused ReLU + bias backward of y = ReLU(x + b).
//
// Column reductions (the bias case, [rows, cols] -> [cols]) run in two
// deterministic passes:
//   pass 1: a 256-thread block owns 256 columns x kRowsPerBlock rows.  Each
//           wave walks every 4th row of the chunk, so a wave's load is 1 KiB
//           of one row; per-thread float4 column partials are combined across
//           the 4 waves through LDS and written to a [chunks, cols] workspace.
//   pass 2: a block of 64 columns; wave w adds chunks w, w+4, ... and the four
//           wave sums are combined in a fixed order.
// The fused ReLU kernel writes dx in pass 1 while it accumulates, so g and z
// are read exactly once (12 B/element).  No atomics: results do not depend
// on scheduling.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kColsPerBlock = 256;
constexpr int kRowsPerBlock = 64;

typedef float f4 __attribute__((ext_vector_type(4)));

// Column index of element e (0..3) of thread lane `l` in a 256-column strip.
template <bool VEC>
__device__ __forceinline__ int strip_col(int l, int e) {
  return VEC ? 4 * l + e : l + 64 * e;
}

// Pass 1.  RELU: dx = z > 0 ? g : 0 (also written out when dx != nullptr);
// otherwise the reduced value is g itself.
template <bool RELU, bool VEC>
__global__ void __launch_bounds__(kBlock)
    colreduce_pass1(const float *__restrict__ g, const float *__restrict__ z,
                    float *__restrict__ dx, float *__restrict__ partial, int64_t rows,
                    int64_t cols, int acc_dx) {
  __shared__ f4 red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * kColsPerBlock;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsPerBlock;
  const int64_t r1 = min(r0 + (int64_t)kRowsPerBlock, rows);
  f4 sum = {0.f, 0.f, 0.f, 0.f};
  const bool full = VEC && c0 + strip_col<VEC>(lane, 3) < cols;
  for (int64_t r = r0 + wave; r < r1; r += 4) {
    const int64_t off = r * cols + c0;
    if (full) {
      const int64_t i = off + 4 * lane;
      f4 gv = *reinterpret_cast<const f4 *>(g + i);
      if (RELU) {
        const f4 zv = *reinterpret_cast<const f4 *>(z + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = zv[e] > 0.0f ? gv[e] : 0.0f;  // backward.rs:158
        if (dx != nullptr) {
          f4 out = gv;
          if (acc_dx) out += *reinterpret_cast<const f4 *>(dx + i);
          *reinterpret_cast<f4 *>(dx + i) = out;
        }
      }
      sum += gv;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t c = c0 + strip_col<VEC>(lane, e);
        if (c < cols) {
          const int64_t i = r * cols + c;
          float gv = g[i];
          if (RELU) {
            gv = z[i] > 0.0f ? gv : 0.0f;
            if (dx != nullptr) dx[i] = acc_dx ? dx[i] + gv : gv;
          }
          sum[e] += gv;
        }
      }
    }
  }
  red[wave][lane] = sum;
  __syncthreads();
  if (wave == 0) {
    const f4 s = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    float *dst = partial + (int64_t)blockIdx.y * cols + c0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t c = strip_col<VEC>(lane, e);
      if (c0 + c < cols) dst[c] = s[e];
    }
  }
}

// ReLU mask only (no bias gradient requested).
template <bool VEC>
__global__ void __launch_bounds__(kBlock)
    relu_mask_kernel(const float *__restrict__ g, const float *__restrict__ z,
                     float *__restrict__ dx, int64_t n, int acc) {
  const int64_t base = (int64_t)blockIdx.x * (kBlock * 8) + threadIdx.x * 4;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
    if (VEC && i + 3 < n) {
      f4 gv = *reinterpret_cast<const f4 *>(g + i);
      const f4 zv = *reinterpret_cast<const f4 *>(z + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) gv[e] = zv[e] > 0.0f ? gv[e] : 0.0f;
      if (acc) gv += *reinterpret_cast<const f4 *>(dx + i);
      *reinterpret_cast<f4 *>(dx + i) = gv;
    } else {
      for (int e = 0; e < 4; ++e)
        if (i + e < n) {
          const float v = z[i + e] > 0.0f ? g[i + e] : 0.0f;
          dx[i + e] = acc ? dx[i + e] + v : v;
        }
    }
  }
}

// Pass 2 (CORRECT): out[c] (+)= sum over chunks of partial[k][c].  A block
// covers 64 columns; wave w adds chunks w, w+4, ..., and the four wave sums
// are combined in wave order.
__global__ void __launch_bounds__(kBlock)
    colreduce_finalize(const float *__restrict__ partial, float *__restrict__ out, int64_t chunks,
                       int64_t cols, int acc) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  // Loads are issued in batches of 16 before they are added, so a wave waits
  // for one memory round trip per batch instead of one per chunk.
  constexpr int kBatch = 16;
  float s = 0.0f;
  if (c < cols) {
    for (int64_t k0 = wave; k0 < chunks; k0 += 4 * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t k = k0 + 4 * u;
        v[u] = k < chunks ? partial[k * cols + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) s += v[u];
    }
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    const float t = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    out[c] = acc ? out[c] + t : t;
  }
}

// Pass 2 (REFERENCE): the full sum lands in out[0]; with acc = 0 the rest
// of out is zeroed (a fresh zero grad plus the zip-truncated add).
__global__ void __launch_bounds__(kBlock)
    full_reduce_finalize(const float *__restrict__ partial, int64_t count, float *__restrict__ out,
                         int64_t out_n, int acc, int zero_rest) {
  __shared__ float red[kBlock / 64];
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < count; i += kBlock) s += partial[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = ((red[0] + red[1]) + red[2]) + red[3];
    out[0] = acc ? out[0] + t : t;
  }
  if (zero_rest)
    for (int64_t i = 1 + threadIdx.x; i < out_n; i += kBlock) out[i] = 0.0f;
}

// Full sum pass 1: grid-stride partial per block.
__global__ void __launch_bounds__(kBlock)
    full_reduce_pass1(const float *__restrict__ g, int64_t n, float *__restrict__ partial) {
  __shared__ float red[kBlock / 64];
  float s = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    s += g[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

// Row reduction [rows, cols] -> [rows]: one wave per row.
__global__ void __launch_bounds__(kBlock)
    rowreduce_kernel(const float *__restrict__ g, float *__restrict__ out, int64_t rows,
                     int64_t cols, int acc) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float s = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) s += g[r * cols + j];
  s = wave_sum(s);
  if (lane == 0) out[r] = acc ? out[r] + s : s;
}

// General fallback: output element per thread; up to 8 merged axes.
struct AxisPlan {
  int n;                 // merged axes
  int64_t size[8];       // extent of each merged axis in g
  int64_t gstride[8];    // stride in g
  int reduced[8];
};

__global__ void __launch_bounds__(kBlock)
    generic_reduce_kernel(const float *__restrict__ g, float *__restrict__ out, int64_t out_n,
                          AxisPlan plan, int64_t red_n, int acc) {
  const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (o >= out_n) return;
  // Offset of output element o in g, over the kept axes.
  int64_t gbase = 0, rem = o;
  for (int d = plan.n - 1; d >= 0; --d) {
    if (plan.reduced[d]) continue;
    const int64_t c = rem % plan.size[d];
    rem /= plan.size[d];
    gbase += c * plan.gstride[d];
  }
  float s = 0.0f;
  for (int64_t k = 0; k < red_n; ++k) {
    int64_t off = gbase, rk = k;
    for (int d = plan.n - 1; d >= 0; --d) {
      if (!plan.reduced[d]) continue;
      const int64_t c = rk % plan.size[d];
      rk /= plan.size[d];
      off += c * plan.gstride[d];
    }
    s += g[off];
  }
  out[o] = acc ? out[o] + s : s;
}

// LayerNorm backward (new op; closed form, fp32):
//   xh = (x - mean) * rstd,  gg = g * gamma
//   dx = rstd * (gg - mean_row(gg) - xh * mean_row(gg * xh))
//   dgamma = sum_rows g * xh,  dbeta = sum_rows g
// Pass 1: a block owns kLnRows rows; each wave takes every 4th row and
// keeps per-column partials of g*xh and g in its own LDS rows (lane j owns
// columns j, j+64, ...: no sharing, no atomics).  The four wave partials are
// added in wave order into the [chunk, cols] workspace; the dgamma/dbeta
// finalize is colreduce_finalize.
constexpr int kLnMaxCols = 2048;
constexpr int kLnRows = 16;  // rows per block: [4096, 512] gives 256 blocks

__global__ void __launch_bounds__(kBlock)
    layernorm_bwd_pass1(const float *__restrict__ g, const float *__restrict__ x,
                        const float *__restrict__ gamma, const float *__restrict__ mean,
                        const float *__restrict__ rstd, float *__restrict__ dx,
                        float *__restrict__ part_g, float *__restrict__ part_b, int64_t rows,
                        int64_t cols, int acc_dx, int want_params) {
  extern __shared__ float lds[];  // [2][4][cols]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float *pg = lds + wave * cols;
  float *pb = lds + (4 + wave) * cols;
  for (int64_t j = lane; j < cols; j += 64) {
    pg[j] = 0.0f;
    pb[j] = 0.0f;
  }
  const int64_t r0 = (int64_t)blockIdx.x * kLnRows;
  const int64_t r1 = min(r0 + (int64_t)kLnRows, rows);
  const float inv_n = 1.0f / (float)cols;
  for (int64_t r = r0 + wave; r < r1; r += 4) {
    const float *xr = x + r * cols, *gr = g + r * cols;
    const float mu = mean[r], rs = rstd[r];
    float m1 = 0.0f, m2 = 0.0f;
    for (int64_t j = lane; j < cols; j += 64) {
      const float xh = (xr[j] - mu) * rs;
      const float gg = gr[j] * gamma[j];
      m1 += gg;
      m2 += gg * xh;
      pg[j] += gr[j] * xh;
      pb[j] += gr[j];
    }
    m1 = wave_sum(m1) * inv_n;
    m2 = wave_sum(m2) * inv_n;
    if (dx != nullptr) {
      float *dr = dx + r * cols;
      for (int64_t j = lane; j < cols; j += 64) {
        const float xh = (xr[j] - mu) * rs;
        const float gg = gr[j] * gamma[j];
        const float v = rs * ((gg - m1) - xh * m2);
        dr[j] = acc_dx ? dr[j] + v : v;
      }
    }
  }
  if (!want_params) return;
  __syncthreads();
  for (int64_t j = threadIdx.x; j < cols; j += kBlock) {
    const float sg = ((lds[j] + lds[cols + j]) + lds[2 * cols + j]) + lds[3 * cols + j];
    const float sb = ((lds[4 * cols + j] + lds[5 * cols + j]) + lds[6 * cols + j]) +
                     lds[7 * cols + j];
    part_g[(int64_t)blockIdx.x * cols + j] = sg;
    part_b[(int64_t)blockIdx.x * cols + j] = sb;
  }
}

int colreduce(numrs_hip_ctx *ctx, const float *g, const float *z, float *dx, float *out,
              int64_t rows, int64_t cols, int mode, int acc_dx, int acc_out, int64_t out_n) {
  const int64_t strips = (cols + kColsPerBlock - 1) / kColsPerBlock;
  const int64_t chunks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (strips > 0x7fffffff || chunks > 65535)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "column reduction too large");
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)(chunks * cols) * sizeof(float), &ws)) return rc;
  float *partial = static_cast<float *>(ws);
  const bool vec = numrs_hip::aligned16(g) && (z == nullptr || numrs_hip::aligned16(z)) &&
                   (dx == nullptr || numrs_hip::aligned16(dx)) && (cols & 3) == 0;
  dim3 grid((unsigned)strips, (unsigned)chunks);
  if (z != nullptr) {
    if (vec)
      colreduce_pass1<true, true><<<grid, kBlock, 0, ctx->stream>>>(g, z, dx, partial, rows, cols,
                                                                    acc_dx);
    else
      colreduce_pass1<true, false><<<grid, kBlock, 0, ctx->stream>>>(g, z, dx, partial, rows,
                                                                     cols, acc_dx);
  } else {
    if (vec)
      colreduce_pass1<false, true><<<grid, kBlock, 0, ctx->stream>>>(g, z, dx, partial, rows,
                                                                     cols, 0);
    else
      colreduce_pass1<false, false><<<grid, kBlock, 0, ctx->stream>>>(g, z, dx, partial, rows,
                                                                      cols, 0);
  }
  if (int rc = numrs_hip::check_launch(ctx, "colreduce_pass1")) return rc;
  if (mode == NUMRS_HIP_UNBROADCAST_CORRECT) {
    colreduce_finalize<<<grid_for(cols, 64), kBlock, 0, ctx->stream>>>(partial, out, chunks,
                                                                            cols, acc_out);
  } else {
    full_reduce_finalize<<<1, kBlock, 0, ctx->stream>>>(partial, chunks * cols, out, out_n,
                                                        acc_out, !acc_out);
  }
  return numrs_hip::check_launch(ctx, "colreduce_finalize");
}

int full_sum(numrs_hip_ctx *ctx, const float *g, int64_t n, float *out, int64_t out_n, int acc,
             int zero_rest) {
  int64_t blocks = (n + kBlock * 16 - 1) / (kBlock * 16);
  if (blocks < 1) blocks = 1;
  if (blocks > 2048) blocks = 2048;
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)blocks * sizeof(float), &ws)) return rc;
  float *partial = static_cast<float *>(ws);
  full_reduce_pass1<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(g, n, partial);
  if (int rc = numrs_hip::check_launch(ctx, "full_reduce_pass1")) return rc;
  full_reduce_finalize<<<1, kBlock, 0, ctx->stream>>>(partial, blocks, out, out_n, acc, zero_rest);
  return numrs_hip::check_launch(ctx, "full_reduce_finalize");
}

}  // namespace

extern "C" {

int numrs_hip_relu_bias_backward(numrs_hip_ctx *ctx, const float *g, const float *z, float *dx,
                                 float *db, int64_t rows, int64_t cols, int mode,
                                 int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_relu_bias_backward";
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (mode != NUMRS_HIP_UNBROADCAST_CORRECT && mode != NUMRS_HIP_UNBROADCAST_REFERENCE)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: mode %d", who, mode);
  if (g == nullptr || z == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  if (db != nullptr && cols > 0 && rows == 0) {
    // Sum over zero rows.
    if (accumulate) return NUMRS_HIP_OK;
    return numrs_hip_fill(ctx, db, cols, 0.0f);
  }
  if (rows == 0 || cols == 0) return NUMRS_HIP_OK;
  if (db == nullptr) {
    if (dx == nullptr) return NUMRS_HIP_OK;
    const int64_t n = rows * cols;
    const bool vec = numrs_hip::aligned16(g) && numrs_hip::aligned16(z) && numrs_hip::aligned16(dx);
    if (vec)
      relu_mask_kernel<true><<<grid_for(n, kBlock * 8), kBlock, 0, ctx->stream>>>(g, z, dx, n,
                                                                                  accumulate);
    else
      relu_mask_kernel<false><<<grid_for(n, kBlock * 8), kBlock, 0, ctx->stream>>>(g, z, dx, n,
                                                                                   accumulate);
    return numrs_hip::check_launch(ctx, "relu_mask_kernel");
  }
  return colreduce(ctx, g, z, dx, db, rows, cols, mode, accumulate, accumulate, cols);
}

int numrs_hip_layernorm_backward(numrs_hip_ctx *ctx, const float *g, const float *x,
                                 const float *gamma, const float *mean, const float *rstd,
                                 float *dx, float *dgamma, float *dbeta, int64_t rows,
                                 int64_t cols, int acc_dx, int acc_dgamma, int acc_dbeta) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_layernorm_backward";
  if (rows < 0 || cols <= 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: bad size", who);
  if (cols > kLnMaxCols)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: rows longer than %d", who, kLnMaxCols);
  if (rows == 0) {
    int rc = (dgamma && !acc_dgamma) ? numrs_hip_fill(ctx, dgamma, cols, 0.0f) : NUMRS_HIP_OK;
    if (!rc && dbeta && !acc_dbeta) rc = numrs_hip_fill(ctx, dbeta, cols, 0.0f);
    return rc;
  }
  if (g == nullptr || x == nullptr || gamma == nullptr || mean == nullptr || rstd == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  const int want = dgamma != nullptr || dbeta != nullptr;
  if (dx == nullptr && !want) return NUMRS_HIP_OK;
  const int64_t chunks = (rows + kLnRows - 1) / kLnRows;
  if (chunks > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: too many rows", who);
  float *part = nullptr;
  if (want) {
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (size_t)(2 * chunks * cols) * sizeof(float), &ws))
      return rc;
    part = static_cast<float *>(ws);
  }
  const size_t lds = (size_t)8 * cols * sizeof(float);
  layernorm_bwd_pass1<<<(unsigned)chunks, kBlock, lds, ctx->stream>>>(
      g, x, gamma, mean, rstd, dx, part, part ? part + chunks * cols : nullptr, rows, cols,
      acc_dx, want);
  if (int rc = numrs_hip::check_launch(ctx, "layernorm_bwd_pass1")) return rc;
  if (dgamma) {
    colreduce_finalize<<<grid_for(cols, 64), kBlock, 0, ctx->stream>>>(part, dgamma, chunks, cols,
                                                                       acc_dgamma);
    if (int rc = numrs_hip::check_launch(ctx, "colreduce_finalize")) return rc;
  }
  if (dbeta) {
    colreduce_finalize<<<grid_for(cols, 64), kBlock, 0, ctx->stream>>>(part + chunks * cols, dbeta,
                                                                       chunks, cols, acc_dbeta);
    if (int rc = numrs_hip::check_launch(ctx, "colreduce_finalize")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_sum_to_shape(numrs_hip_ctx *ctx, const float *g, const int64_t *gshape, int gnd,
                           float *out, const int64_t *oshape, int ond, int mode, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_sum_to_shape";
  if ((gnd > 0 && gshape == nullptr) || (ond > 0 && oshape == nullptr) || gnd < 0 || ond < 0 ||
      gnd > 8 || ond > 8)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: bad shape arguments", who);
  if (mode != NUMRS_HIP_UNBROADCAST_CORRECT && mode != NUMRS_HIP_UNBROADCAST_REFERENCE)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: mode %d", who, mode);
  int64_t gn = 1, on = 1;
  for (int d = 0; d < gnd; ++d) {
    if (gshape[d] < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative dim", who);
    gn *= gshape[d];
  }
  for (int d = 0; d < ond; ++d) {
    if (oshape[d] < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative dim", who);
    on *= oshape[d];
  }
  if (on == 0) return NUMRS_HIP_OK;
  if (g == nullptr || out == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);

  bool same = gnd == ond;
  for (int d = 0; same && d < gnd; ++d) same = gshape[d] == oshape[d];
  if (same) {  // unbroadcast identity (backward.rs:13-15): plain (accumulating) copy
    if (accumulate) {
      return numrs_hip_binary_backward(ctx, NUMRS_HIP_ADD, g, nullptr, nullptr, out, nullptr, gn,
                                       1);
    }
    return numrs_hip_copy(ctx, out, g, (size_t)gn * sizeof(float));
  }
  if (mode == NUMRS_HIP_UNBROADCAST_REFERENCE) {
    // backward.rs:18-19,38: ops::sum(grad, None); tensor.rs:125-127 adds it at index 0.
    if (gn == 0) return accumulate ? NUMRS_HIP_OK : numrs_hip_fill(ctx, out, on, 0.0f);
    return full_sum(ctx, g, gn, out, on, accumulate, !accumulate);
  }

  // CORRECT: right-aligned broadcast check, then merge adjacent axes of the
  // same kind (kept / reduced).
  if (ond > gnd) return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "%s: target has more axes", who);
  int64_t os[8];
  for (int d = 0; d < gnd; ++d) {
    const int od = d - (gnd - ond);
    os[d] = od >= 0 ? oshape[od] : 1;
    if (os[d] != 1 && os[d] != gshape[d])
      return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "%s: axis %d: %lld does not reduce to %lld",
                             who, d, (long long)gshape[d], (long long)os[d]);
  }
  if (gn == 0) return accumulate ? NUMRS_HIP_OK : numrs_hip_fill(ctx, out, on, 0.0f);
  AxisPlan plan;
  plan.n = 0;
  for (int d = 0; d < gnd; ++d) {
    if (gshape[d] == 1) continue;  // size-1 axes move nothing
    const int red = os[d] == 1;
    if (plan.n > 0 && plan.reduced[plan.n - 1] == red) {
      plan.size[plan.n - 1] *= gshape[d];
    } else {
      plan.size[plan.n] = gshape[d];
      plan.reduced[plan.n] = red;
      ++plan.n;
    }
  }
  if (plan.n == 0)  // every axis has size 1: copy
    return accumulate ? numrs_hip_binary_backward(ctx, NUMRS_HIP_ADD, g, nullptr, nullptr, out,
                                                  nullptr, gn, 1)
                      : numrs_hip_copy(ctx, out, g, sizeof(float));
  if (plan.n == 1 && plan.reduced[0]) return full_sum(ctx, g, gn, out, on, accumulate, 0);
  if (plan.n == 1)
    return accumulate ? numrs_hip_binary_backward(ctx, NUMRS_HIP_ADD, g, nullptr, nullptr, out,
                                                  nullptr, gn, 1)
                      : numrs_hip_copy(ctx, out, g, (size_t)gn * sizeof(float));
  if (plan.n == 2 && plan.reduced[0])  // [R, C] -> [C]: bias / column reduction
    return colreduce(ctx, g, nullptr, nullptr, out, plan.size[0], plan.size[1],
                     NUMRS_HIP_UNBROADCAST_CORRECT, 0, accumulate, on);
  if (plan.n == 2) {  // [R, C] -> [R]
    rowreduce_kernel<<<grid_for(plan.size[0], 4), kBlock, 0, ctx->stream>>>(
        g, out, plan.size[0], plan.size[1], accumulate);
    return numrs_hip::check_launch(ctx, "rowreduce_kernel");
  }
  int64_t stride = 1, red_n = 1;
  for (int d = plan.n - 1; d >= 0; --d) {
    plan.gstride[d] = stride;
    stride *= plan.size[d];
    if (plan.reduced[d]) red_n *= plan.size[d];
  }
  generic_reduce_kernel<<<grid_for(on, kBlock), kBlock, 0, ctx->stream>>>(g, out, on, plan, red_n,
                                                                          accumulate);
  return numrs_hip::check_launch(ctx, "generic_reduce_kernel");
}

}  // extern "C"
