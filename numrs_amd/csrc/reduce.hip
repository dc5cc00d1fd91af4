// Broadcast-reduce gradients: unbroadcast / sum-to-shape (backward.rs:12-39)
// and the fused ReLU + bias backward of y = ReLU(x + b).
//
// Column reductions (the bias case, [rows, cols] -> [cols]) run in two
// deterministic passes:
//   pass 1: the grid is strips x classes.  A 256-thread block owns a strip of
//           512 columns (each lane two float4 column groups, 256 columns
//           apart) and walks the row bands y, y + Q, y + 2Q, ... of its class
//           y (a band is 4 rows, one per wave; Q = gridDim.y).  At any moment
//           the whole grid therefore reads one contiguous stretch of rows,
//           which keeps HBM pages open; on MI355X this sweep order runs the
//           fused ReLU backward at 4096^2 about 10% faster than blocks that
//           each own a private run of rows.  Per-lane column partials are
//           combined across the 4 waves through LDS and written to a
//           [Q, cols] workspace.
//   pass 2: a block of 64 columns; wave w adds classes w, w+4, ... and the
//           four wave sums are combined in a fixed order.
// The fused ReLU kernel writes dx in pass 1 while it accumulates, so g and z
// are read exactly once (12 B/element).  No atomics: results do not depend
// on scheduling.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kColsPerBlock = 512;
constexpr int kBandRows = 4;

typedef float f4 __attribute__((ext_vector_type(4)));
using numrs_hip::ldv;
using numrs_hip::stv;

// Column of element e (0..7) of lane l in a 512-column strip.  VEC: two float4
// groups, 4l..4l+3 and 256+4l..256+4l+3; otherwise l + 64e (coalesced scalars).
template <bool VEC>
__device__ __forceinline__ int strip_col(int l, int e) {
  return VEC ? (e >> 2) * 256 + 4 * l + (e & 3) : l + 64 * e;
}

// Pass 1.  RELU: dx = z > 0 ? g : 0 (also written out when dx != nullptr);
// otherwise the reduced value is g itself.
template <bool RELU, int VEC>
__global__ void __launch_bounds__(kBlock)
    colreduce_pass1(const float *__restrict__ g, const float *__restrict__ z,
                    float *__restrict__ dx, float *__restrict__ partial, int64_t rows,
                    int64_t cols, int acc_dx) {
  __shared__ f4 red[4][2][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * kColsPerBlock;
  const int64_t classes = gridDim.y;
  f4 sum[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // With VEC, cols % 4 == 0, so a float4 group is either wholly inside or
  // wholly outside the matrix.
  const bool full0 = VEC && c0 + strip_col<(VEC != 0)>(lane, 3) < cols;
  const bool full1 = VEC && c0 + strip_col<(VEC != 0)>(lane, 7) < cols;
  // Strips wholly inside the matrix (all but a ragged last one) issue both
  // float4 loads of g and of z before any use, so each wave keeps four loads
  // in flight; a per-lane guard would split them into separate waits.
  const bool whole = VEC && c0 + kColsPerBlock <= cols;
  if (whole) {
    // Whole strip: the next band's loads are issued before the current band
    // is processed (register double buffering), so each wave keeps two
    // bands' loads in flight; bands are still summed in walk order.
    int64_t r = (int64_t)blockIdx.y * kBandRows + wave;
    if (r < rows) {
      const int64_t step = classes * kBandRows;
      f4 ga[2], za[2], gb[2], zb[2];
      auto load = [&](int64_t row, f4 *gv, f4 *zv) {
        const int64_t i0 = row * cols + c0 + 4 * lane;
        gv[0] = ldv<VEC>(g + i0);
        gv[1] = ldv<VEC>(g + i0 + 256);
        if (RELU) {
          zv[0] = ldv<VEC>(z + i0);
          zv[1] = ldv<VEC>(z + i0 + 256);
        }
      };
      auto band = [&](int64_t row, const f4 *gv, const f4 *zv) {
        const int64_t i0 = row * cols + c0 + 4 * lane, i1 = i0 + 256;
        f4 g0 = gv[0], g1 = gv[1];
        if (RELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            g0[e] = zv[0][e] > 0.0f ? g0[e] : 0.0f;  // backward.rs:158
            g1[e] = zv[1][e] > 0.0f ? g1[e] : 0.0f;
          }
          if (dx != nullptr) {
            f4 o0 = g0, o1 = g1;
            if (acc_dx) {
              o0 += ldv<VEC>(dx + i0);
              o1 += ldv<VEC>(dx + i1);
            }
            stv<VEC>(dx + i0, o0);
            stv<VEC>(dx + i1, o1);
          }
        }
        sum[0] += g0;
        sum[1] += g1;
      };
      // Two register sets alternate (a copy out of a set with loads in
      // flight would wait for them).  The prefetch is unconditional -- past
      // the end it re-reads the current row -- so the wait before a band
      // only covers that band's own loads.
      load(r, ga, za);
      while (true) {
        const int64_t r1 = r + step;
        load(r1 < rows ? r1 : r, gb, zb);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the band's work
        band(r, ga, za);
        if (r1 >= rows) break;
        const int64_t r2 = r1 + step;
        load(r2 < rows ? r2 : r1, ga, za);
        __builtin_amdgcn_sched_barrier(0);
        band(r1, gb, zb);
        if (r2 >= rows) break;
        r = r2;
      }
    }
  } else {
    for (int64_t band = blockIdx.y; band * kBandRows < rows; band += classes) {
      const int64_t r = band * kBandRows + wave;
      if (r >= rows) break;  // wave-uniform; later bands of this class are further down
      const int64_t off = r * cols + c0;
      if (VEC) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (!(h == 0 ? full0 : full1)) continue;
          const int64_t i = off + 256 * h + 4 * lane;
          f4 gv = ldv<VEC>(g + i);
          if (RELU) {
            const f4 zv = ldv<VEC>(z + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[e] = zv[e] > 0.0f ? gv[e] : 0.0f;  // backward.rs:158
            if (dx != nullptr) {
              f4 out = gv;
              if (acc_dx) out += ldv<VEC>(dx + i);
              stv<VEC>(dx + i, out);
            }
          }
          sum[h] += gv;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t c = c0 + strip_col<(VEC != 0)>(lane, e);
          if (c < cols) {
            const int64_t i = r * cols + c;
            float gv = g[i];
            if (RELU) {
              gv = z[i] > 0.0f ? gv : 0.0f;
              if (dx != nullptr) dx[i] = acc_dx ? dx[i] + gv : gv;
            }
            sum[e >> 2][e & 3] += gv;
          }
        }
      }
  }
  }
  red[wave][0][lane] = sum[0];
  red[wave][1][lane] = sum[1];
  __syncthreads();
  if (wave < 2) {
    const int h = wave;
    const f4 s = ((red[0][h][lane] + red[1][h][lane]) + red[2][h][lane]) + red[3][h][lane];
    float *dst = partial + (int64_t)blockIdx.y * cols + c0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t c = strip_col<(VEC != 0)>(lane, 4 * h + e);
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
// of kFinWaves waves covers 64 columns; wave w adds chunks w, w + kFinWaves,
// ... (loads issued in batches, so a wave waits for one memory round trip per
// batch), and wave 0 adds the wave sums in wave order.  blockIdx.y selects
// one of two independent (partial, out, acc) sets, so LayerNorm's dgamma and
// dbeta finish in one launch.
constexpr int kFinWaves = 16;

struct FinalizeSet {
  const float *partial[2];
  float *out[2];
  int acc[2];
};

__global__ void __launch_bounds__(64 * kFinWaves)
    colreduce_finalize(FinalizeSet set, int64_t chunks, int64_t cols) {
  __shared__ float red[kFinWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *__restrict__ partial = set.partial[blockIdx.y];
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  constexpr int kBatch = 8;
  float s = 0.0f;
  if (c < cols) {
    for (int64_t k0 = wave; k0 < chunks; k0 += kFinWaves * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t k = k0 + kFinWaves * u;
        v[u] = k < chunks ? partial[k * cols + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) s += v[u];
    }
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    float t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kFinWaves; ++w) t += red[w][lane];
    float *out = set.out[blockIdx.y];
    out[c] = set.acc[blockIdx.y] ? out[c] + t : t;
  }
}

// Launches the finalize for one or two (partial, out) sets (out1 may be null).
int launch_finalize(numrs_hip_ctx *ctx, const float *part0, float *out0, int acc0,
                    const float *part1, float *out1, int acc1, int64_t chunks, int64_t cols) {
  FinalizeSet set{{part0, part1}, {out0, out1}, {acc0, acc1}};
  if (out0 == nullptr) {
    set.partial[0] = part1;
    set.out[0] = out1;
    set.acc[0] = acc1;
    out1 = nullptr;
  }
  if (set.out[0] == nullptr) return NUMRS_HIP_OK;
  dim3 grid(grid_for(cols, 64), out1 != nullptr ? 2 : 1);
  colreduce_finalize<<<grid, 64 * kFinWaves, 0, ctx->stream>>>(set, chunks, cols);
  return numrs_hip::check_launch(ctx, "colreduce_finalize");
}

// Pass 2 (REFERENCE): the full sum lands in out[0]; with acc = 0 the rest
// of out is zeroed (a fresh zero grad plus the zip-truncated add).
__global__ void __launch_bounds__(kBlock)
    full_reduce_finalize(const float *__restrict__ partial, int64_t count, float *__restrict__ out,
                         int64_t out_n, int acc, int zero_rest) {
  __shared__ float red[kBlock / 64];
  // Loads go out in batches of 8 before they are added (in index order).
  float s = 0.0f;
  for (int64_t i0 = threadIdx.x; i0 < count; i0 += 8 * kBlock) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t k = i0 + (int64_t)u * kBlock;
      v[u] = k < count ? partial[k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + (int64_t)u * kBlock < count) s += v[u];
  }
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

// Full sum pass 1: grid-stride partial per block.  With 16-byte aligned g
// (VEC), a thread walks float4 groups, eight loads in flight, into four
// partial sums added in a fixed order.
template <bool VEC>
__global__ void __launch_bounds__(kBlock)
    full_reduce_pass1(const float *__restrict__ g, int64_t n, float *__restrict__ partial) {
  __shared__ float red[kBlock / 64];
  float s = 0.0f;
  if (VEC) {
    const int64_t n4 = n / 4, stride = (int64_t)gridDim.x * kBlock;
    int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (; i + 7 * stride < n4; i += 8 * stride) {
      f4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = reinterpret_cast<const f4 *>(g)[i + u * stride];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[u & 3] += v[u][e];
    }
    for (; i < n4; i += stride) {
      const f4 v = reinterpret_cast<const f4 *>(g)[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[0] += v[e];
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) acc[0] += g[n4 * 4 + threadIdx.x];
    s = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock)
      s += g[i];
  }
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

// Axis reduction x[outer, n, inner] -> out[outer, inner] (ops::sum / ops::mean
// with Some(axis), backend/cpu/scalar.rs:584-700): one thread per output,
// summing its n values in axis order (the reference's order for an inner
// axis); threads of a wave hold consecutive inner indices, so every load
// of the walk is coalesced.  MEAN divides the sum by n afterwards, as the
// reference does (`*x /= axis_size as f32`, scalar.rs:314-316).
__global__ void __launch_bounds__(kBlock)
    axis_reduce_kernel(const float *__restrict__ x, float *__restrict__ out, int64_t outer,
                       int64_t n, int64_t inner, int mean) {
  const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (o >= outer * inner) return;
  const int64_t b = o / inner, i = o - b * inner;
  const float *src = x + b * n * inner + i;
  float s = 0.0f;
  for (int64_t k = 0; k < n; ++k) s += src[k * inner];
  out[o] = mean ? s / (float)n : s;
}

// out[i] = out[i] / d (the mean's division after a column reduction).
__global__ void __launch_bounds__(kBlock)
    div_scalar_kernel(float *__restrict__ out, int64_t count, float d) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < count) out[i] = out[i] / d;
}

// Backward of the axis reduction: dx[o, k, i] (+)= g[o, i] (or g[o, i] / n
// for the mean, the division of mean_backward, backward.rs:224-236).
__global__ void __launch_bounds__(kBlock)
    broadcast_axis_kernel(const float *__restrict__ g, float *__restrict__ dx, int64_t outer,
                          int64_t n, int64_t inner, int mean, int acc) {
  const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (idx >= outer * n * inner) return;
  const int64_t b = idx / (n * inner), i = idx % inner;
  const float gv = g[b * inner + i];
  const float v = mean ? gv / (float)n : gv;
  dx[idx] = acc ? dx[idx] + v : v;
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

// Vectorised pass 1 for rows of at most kLnMaxCols columns with cols % 4 == 0
// and 16-byte aligned operands.  Lane l owns the float4 column groups
// l, l + 64, ... (NV of them), so its partials of g*xh and g stay in
// registers across all rows it visits, and each row is read once with float4
// loads.  The grid sweeps rows in interleaved bands of 4 (one row per wave):
// block b takes bands b, b + gridDim.x, ...  Wave partials are combined in
// wave order through LDS and written to the [gridDim.x, cols] workspaces.
template <int NV, int VM>
__global__ void __launch_bounds__(kBlock)
    layernorm_bwd_vec(const float *__restrict__ g, const float *__restrict__ x,
                      const float *__restrict__ gamma, const float *__restrict__ mean,
                      const float *__restrict__ rstd, float *__restrict__ dx,
                      float *__restrict__ part_g, float *__restrict__ part_b, int64_t rows,
                      int64_t cols, int acc_dx, int want_params) {
  __shared__ f4 red[4][64 * NV];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  bool in[NV];
  f4 gm[NV], pg[NV], pb[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = 4 * (int64_t)(lane + 64 * i);
    in[i] = c < cols;
    gm[i] = in[i] ? *reinterpret_cast<const f4 *>(gamma + c) : f4{0.f, 0.f, 0.f, 0.f};
    pg[i] = f4{0.f, 0.f, 0.f, 0.f};
    pb[i] = f4{0.f, 0.f, 0.f, 0.f};
  }
  const float inv_n = 1.0f / (float)cols;
  // One row of the wave's walk: statistics, dx, and the column partials.
  auto row = [&](int64_t r, const f4 *xv, const f4 *gv, float mu, float rs) {
    float m1 = 0.0f, m2 = 0.0f;
    f4 xh[NV], gg[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[i][e] = (xv[i][e] - mu) * rs;
        gg[i][e] = gv[i][e] * gm[i][e];
        m1 += gg[i][e];
        m2 += gg[i][e] * xh[i][e];
        pg[i][e] += gv[i][e] * xh[i][e];
        pb[i][e] += gv[i][e];
      }
    }
    m1 = wave_sum(m1) * inv_n;
    m2 = wave_sum(m2) * inv_n;
    if (dx != nullptr) {
      float *dr = dx + r * cols;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (!in[i]) continue;
        const int64_t c = 4 * (int64_t)(lane + 64 * i);
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = rs * ((gg[i][e] - m1) - xh[i][e] * m2);
        if (acc_dx) v += ldv<VM>(dr + c);
        stv<VM>(dr + c, v);
      }
    }
  };
  // The wave walks rows band*4 + wave for bands b, b + Q, b + 2Q, ...
  // (Q = gridDim.x).  The next rows' loads, their statistics included, are
  // issued before the current row is processed (a ring of register sets):
  // the memory counter retires loads in issue order, so a statistic loaded
  // after the prefetch would make the wave wait for the prefetch as well.
  const int64_t q = gridDim.x;
  auto load = [&](int64_t r, f4 *xv, f4 *gv, float &mu, float &rs) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      // Lanes past the row end load column 0 and discard it: an
      // unconditional load keeps the wait counts exact.
      const int64_t c = in[i] ? 4 * (int64_t)(lane + 64 * i) : 0;
      const f4 z = {0.f, 0.f, 0.f, 0.f};
      const f4 xl = ldv<VM>(x + r * cols + c);
      const f4 gl = ldv<VM>(g + r * cols + c);
      xv[i] = in[i] ? xl : z;
      gv[i] = in[i] ? gl : z;
    }
    mu = mean[r];
    rs = rstd[r];
  };
  // kDepth register sets form a ring (no copies: a copy out of a set with
  // loads in flight would wait for them): while a row is processed, the
  // next kDepth - 1 rows' loads are in flight.  A prefetch past the end
  // re-reads the row being processed, so the wait before a row only covers
  // that row's own loads.
  constexpr int kDepth = 3;
  int64_t r = (int64_t)blockIdx.x * 4 + wave;
  const int64_t step = 4 * q;
  if (r < rows) {
    f4 xs[kDepth][NV], gs[kDepth][NV];
    float mus[kDepth], rss[kDepth];
#pragma unroll
    for (int k = 0; k + 1 < kDepth; ++k) {
      const int64_t rk = r + k * step;
      load(rk < rows ? rk : r, xs[k], gs[k], mus[k], rss[k]);
    }
    while (true) {
      bool done = false;
#pragma unroll
      for (int k = 0; k < kDepth; ++k) {
        const int64_t rk = r + k * step;           // processed now, from set k
        const int64_t rl = rk + (kDepth - 1) * step;  // loaded now into set k - 1
        const int kl = (k + kDepth - 1) % kDepth;
        load(rl < rows ? rl : rk, xs[kl], gs[kl], mus[kl], rss[kl]);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the row's work
        row(rk, xs[k], gs[k], mus[k], rss[k]);
        if (rk + step >= rows) {
          done = true;
          break;
        }
      }
      if (done) break;
      r += kDepth * step;
    }
  }
  if (!want_params) return;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass) __syncthreads();  // the previous pass's reads are done
#pragma unroll
    for (int i = 0; i < NV; ++i) red[wave][64 * i + lane] = pass ? pb[i] : pg[i];
    __syncthreads();
    float *dst = (pass ? part_b : part_g) + (int64_t)blockIdx.x * cols;
    for (int q = threadIdx.x; q < 64 * NV; q += kBlock) {
      const int64_t c = 4 * (int64_t)q;
      if (c >= cols) continue;
      const f4 t = ((red[0][q] + red[1][q]) + red[2][q]) + red[3][q];
      *reinterpret_cast<f4 *>(dst + c) = t;
    }
  }
}

// Row classes (pass-1 blocks per strip) of a column reduction; its partials
// take chunks * cols floats.
int64_t colreduce_chunks(const numrs_hip_ctx *ctx, int64_t rows, int64_t cols, bool relu) {
  const int64_t strips = (cols + kColsPerBlock - 1) / kColsPerBlock;
  const int64_t bands = (rows + kBandRows - 1) / kBandRows;
  // About one block per CU in all for the fused ReLU kernel (three streams):
  // more blocks in flight scatter the reads over more HBM pages and measured
  // slower.  A plain column sum reads one stream and needs two blocks per CU
  // to keep enough loads in flight.
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const int64_t per_cu = relu ? 1 : 2;
  const int64_t chunks = (per_cu * cus + strips - 1) / strips;
  return std::max<int64_t>(1, std::min<int64_t>({chunks, bands, 65535}));
}

// `partials`: a buffer of at least colreduce_chunks(...) * cols floats, or
// nullptr for the context's workspace.
int colreduce(numrs_hip_ctx *ctx, const float *g, const float *z, float *dx, float *out,
              int64_t rows, int64_t cols, int mode, int acc_dx, int acc_out, int64_t out_n,
              float *partials = nullptr) {
  const int64_t strips = (cols + kColsPerBlock - 1) / kColsPerBlock;
  if (strips > 0x7fffffff)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "column reduction too large");
  const int64_t chunks = colreduce_chunks(ctx, rows, cols, z != nullptr);
  float *partial = partials;
  if (partial == nullptr) {
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (size_t)(chunks * cols) * sizeof(float), &ws))
      return rc;
    partial = static_cast<float *>(ws);
  }
  const bool vec = numrs_hip::aligned16(g) && (z == nullptr || numrs_hip::aligned16(z)) &&
                   (dx == nullptr || numrs_hip::aligned16(dx)) && (cols & 3) == 0;
  dim3 grid((unsigned)strips, (unsigned)chunks);
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, rows * cols), [&](auto V) {
    if (z != nullptr)
      colreduce_pass1<true, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(
          g, z, dx, partial, rows, cols, acc_dx);
    else
      colreduce_pass1<false, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(
          g, z, dx, partial, rows, cols, 0);
  });
  if (int rc = numrs_hip::check_launch(ctx, "colreduce_pass1")) return rc;
  if (mode == NUMRS_HIP_UNBROADCAST_CORRECT)
    return launch_finalize(ctx, partial, out, acc_out, nullptr, nullptr, 0, chunks, cols);
  full_reduce_finalize<<<1, kBlock, 0, ctx->stream>>>(partial, chunks * cols, out, out_n,
                                                      acc_out, !acc_out);
  return numrs_hip::check_launch(ctx, "full_reduce_finalize");
}

int full_sum(numrs_hip_ctx *ctx, const float *g, int64_t n, float *out, int64_t out_n, int acc,
             int zero_rest) {
  // At most one block per CU (more blocks measured slower for a read-only sweep).
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  int64_t blocks = (n + kBlock * 16 - 1) / (kBlock * 16);
  if (blocks < 1) blocks = 1;
  if (blocks > cus) blocks = cus;
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)blocks * sizeof(float), &ws)) return rc;
  float *partial = static_cast<float *>(ws);
  if (numrs_hip::aligned16(g))
    full_reduce_pass1<true><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(g, n, partial);
  else
    full_reduce_pass1<false><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(g, n, partial);
  if (int rc = numrs_hip::check_launch(ctx, "full_reduce_pass1")) return rc;
  full_reduce_finalize<<<1, kBlock, 0, ctx->stream>>>(partial, blocks, out, out_n, acc, zero_rest);
  return numrs_hip::check_launch(ctx, "full_reduce_finalize");
}

// Shared body of numrs_hip_relu_bias_backward (partials == nullptr: the
// context's workspace) and of its allocation-free variant.
int relu_bias_backward(numrs_hip_ctx *ctx, const char *who, const float *g, const float *z,
                       float *dx, float *db, int64_t rows, int64_t cols, int mode, int accumulate,
                       float *partials);

}  // namespace

// Pass-1 partials of the allocation-free fused ReLU + bias backward: a
// file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host the name is
// a stand-in, not a device address); it uses the address that noalloc_init
// resolved for the context's device.
constexpr int64_t kNoAllocPartials = int64_t(1) << 20;  // floats: 4 MiB per GPU
static __device__ __align__(256) float scratch[kNoAllocPartials];

namespace numrs_hip {

int noalloc_init(numrs_hip_ctx *ctx) {
  static std::mutex mu;
  static std::unordered_map<int, float *> by_device;
  std::lock_guard<std::mutex> lock(mu);
  auto it = by_device.find(ctx->device);
  if (it == by_device.end()) {
    // numrs_hip_create has made ctx->device current.  `::scratch` is the
    // array; inside this namespace a bare `scratch` is the workspace function.
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return fail(ctx, NUMRS_HIP_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s",
                  ctx->device, hipGetErrorString(e));
    }
    it = by_device.emplace(ctx->device, static_cast<float *>(p)).first;
  }
  ctx->noalloc_partials = it->second;
  return NUMRS_HIP_OK;
}

}  // namespace numrs_hip

namespace {

int relu_bias_backward(numrs_hip_ctx *ctx, const char *who, const float *g, const float *z,
                       float *dx, float *db, int64_t rows, int64_t cols, int mode, int accumulate,
                       float *partials) {
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
  return colreduce(ctx, g, z, dx, db, rows, cols, mode, accumulate, accumulate, cols, partials);
}

}  // namespace

extern "C" {

int numrs_hip_relu_bias_backward(numrs_hip_ctx *ctx, const float *g, const float *z, float *dx,
                                 float *db, int64_t rows, int64_t cols, int mode,
                                 int accumulate) {
  NRS_CHECK_CTX(ctx);
  return relu_bias_backward(ctx, "numrs_hip_relu_bias_backward", g, z, dx, db, rows, cols, mode,
                            accumulate, nullptr);
}

// The same computation with the pass-1 partials in the static `scratch`
// array: no hipMalloc, hipFree or other allocating call.  Calls that overlap
// on one GPU (two contexts' streams) race on the array; every call writes
// all the partials it reads, so nothing needs clearing between calls.
int numrs_hip_relu_bias_backward_noalloc(numrs_hip_ctx *ctx, const float *g, const float *z,
                                         float *dx, float *db, int64_t rows, int64_t cols,
                                         int mode, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_relu_bias_backward_noalloc";
  if (ctx->noalloc_partials == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_HIP,
                           "%s: the partials array has no device address (status %d at create)",
                           who, ctx->noalloc_status);
  if (db != nullptr && rows > 0 && cols > 0) {
    const int64_t need = colreduce_chunks(ctx, rows, cols, true) * cols;
    if (need > kNoAllocPartials)
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID,
                             "%s: %lld x %lld needs %lld partial floats, above the %lld of the "
                             "allocation-free path",
                             who, (long long)rows, (long long)cols, (long long)need,
                             (long long)kNoAllocPartials);
  }
  return relu_bias_backward(ctx, who, g, z, dx, db, rows, cols, mode, accumulate,
                            ctx->noalloc_partials);
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
  const bool vec = (cols & 3) == 0 && numrs_hip::aligned16(g) && numrs_hip::aligned16(x) &&
                   numrs_hip::aligned16(gamma) && (dx == nullptr || numrs_hip::aligned16(dx));
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const int64_t chunks = vec ? std::min<int64_t>(cus, (rows + 3) / 4)
                             : (rows + kLnRows - 1) / kLnRows;
  if (chunks > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: too many rows", who);
  float *part = nullptr;
  if (want) {
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (size_t)(2 * chunks * cols) * sizeof(float), &ws))
      return rc;
    part = static_cast<float *>(ws);
  }
  float *part_b = part ? part + chunks * cols : nullptr;
  if (vec) {
    const unsigned grid = (unsigned)chunks;
    numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, rows * cols), [&](auto V) {
      constexpr int VM = decltype(V)::value;
      if (cols <= 256)
        layernorm_bwd_vec<1, VM><<<grid, kBlock, 0, ctx->stream>>>(g, x, gamma, mean, rstd, dx,
                                                                   part, part_b, rows, cols,
                                                                   acc_dx, want);
      else if (cols <= 512)
        layernorm_bwd_vec<2, VM><<<grid, kBlock, 0, ctx->stream>>>(g, x, gamma, mean, rstd, dx,
                                                                   part, part_b, rows, cols,
                                                                   acc_dx, want);
      else if (cols <= 1024)
        layernorm_bwd_vec<4, VM><<<grid, kBlock, 0, ctx->stream>>>(g, x, gamma, mean, rstd, dx,
                                                                   part, part_b, rows, cols,
                                                                   acc_dx, want);
      else
        layernorm_bwd_vec<8, VM><<<grid, kBlock, 0, ctx->stream>>>(g, x, gamma, mean, rstd, dx,
                                                                   part, part_b, rows, cols,
                                                                   acc_dx, want);
    });
    if (int rc = numrs_hip::check_launch(ctx, "layernorm_bwd_vec")) return rc;
  } else {
    const size_t lds = (size_t)8 * cols * sizeof(float);
    layernorm_bwd_pass1<<<(unsigned)chunks, kBlock, lds, ctx->stream>>>(
        g, x, gamma, mean, rstd, dx, part, part_b, rows, cols, acc_dx, want);
    if (int rc = numrs_hip::check_launch(ctx, "layernorm_bwd_pass1")) return rc;
  }
  if (!want) return NUMRS_HIP_OK;
  return launch_finalize(ctx, part, dgamma, acc_dgamma, part_b, dbeta, acc_dbeta, chunks, cols);
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

int numrs_hip_reduce_axis(numrs_hip_ctx *ctx, const float *x, int64_t outer, int64_t n,
                          int64_t inner, int mean, float *out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_reduce_axis";
  if (outer < 0 || n < 0 || inner < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  const int64_t on = outer * inner;
  if (on == 0) return NUMRS_HIP_OK;
  if (out == nullptr || (n > 0 && x == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  if (n == 0) return numrs_hip_fill(ctx, out, on, mean ? NAN : 0.0f);
  if (inner == 1) {  // last axis: one wave per row
    rowreduce_kernel<<<grid_for(outer, 4), kBlock, 0, ctx->stream>>>(x, out, outer, n, 0);
    if (int rc = numrs_hip::check_launch(ctx, "rowreduce_kernel")) return rc;
  } else if (outer == 1) {  // leading axis: the column reduction
    if (int rc = colreduce(ctx, x, nullptr, nullptr, out, n, inner, NUMRS_HIP_UNBROADCAST_CORRECT,
                           0, 0, inner))
      return rc;
  } else {
    axis_reduce_kernel<<<grid_for(on, kBlock), kBlock, 0, ctx->stream>>>(x, out, outer, n, inner,
                                                                         mean);
    return numrs_hip::check_launch(ctx, "axis_reduce_kernel");
  }
  if (!mean) return NUMRS_HIP_OK;
  div_scalar_kernel<<<grid_for(on, kBlock), kBlock, 0, ctx->stream>>>(out, on, (float)n);
  return numrs_hip::check_launch(ctx, "div_scalar_kernel");
}

int numrs_hip_broadcast_axis(numrs_hip_ctx *ctx, const float *g, int64_t outer, int64_t n,
                             int64_t inner, int mean, float *dx, int accumulate) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_broadcast_axis";
  if (outer < 0 || n < 0 || inner < 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  const int64_t total = outer * n * inner;
  if (total == 0) return NUMRS_HIP_OK;
  if (g == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  broadcast_axis_kernel<<<grid_for(total, kBlock), kBlock, 0, ctx->stream>>>(g, dx, outer, n,
                                                                             inner, mean,
                                                                             accumulate);
  return numrs_hip::check_launch(ctx, "broadcast_axis_kernel");
}

}  // extern "C"
