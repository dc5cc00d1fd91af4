// Element-streaming kernels: unary/binary backward, sum/mean fill, MSE
// backward, SGD and Adam steps.
//
// All are HBM-bound.  Each thread moves two float4 per operand, placed
// blockDim*4 floats apart so every wave load is a contiguous 1 KiB; scalar
// tails and misaligned operands take the per-element path.  This translation
// unit is built with -ffp-contract=off: the reference (Rust) never fuses
// a*b+c, and the operation order below is the reference's, so results for
// the select/multiply/divide/sqrt kernels are bit-identical to it.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kVecPerThread = 2;
constexpr int kElemsPerBlock = kBlock * 4 * kVecPerThread;

typedef float f4 __attribute__((ext_vector_type(4)));
using numrs_hip::ldv;
using numrs_hip::stv;

// ---------------------------------------------------------------------------
// Unary backward: dx = g * f'(v)
// ---------------------------------------------------------------------------

// powf(v, -0.5) as 1/sqrt(v): both operations are correctly rounded, so the
// result is within an ulp of powf's, at a fraction of the cost of the general
// powf.  powf's special cases are kept: +-0 -> +inf (sqrtf(-0) is -0),
// -inf -> +0 (sqrtf(-inf) is NaN), +inf -> +0, other negatives and NaN -> NaN.
__device__ __forceinline__ float pow_neg_half(float v) {
  if (v == 0.0f) return INFINITY;
  if (v == -INFINITY) return 0.0f;
  return 1.0f / sqrtf(v);
}

// powf(v, e) with the exponents that pow_backward meets most (x^2 and x^3
// layers, reciprocals) evaluated without the general powf.  Each shortcut
// returns exactly what a correctly rounded powf returns, special values
// included: e = 0 -> 1 (also for NaN), e = 1 -> v, e = 2 -> v*v (one rounding
// of the exact square), e = -1 -> 1/v (+-0 -> +-inf), e = -0.5 as above.
// Other exponents use powf.  e is the same for every thread, so the branch is
// uniform.
__device__ __forceinline__ float pow_grad_base(float v, float e) {
  if (e == 2.0f) return v * v;
  if (e == 1.0f) return v;
  if (e == 0.0f) return 1.0f;
  if (e == -1.0f) return 1.0f / v;
  if (e == -0.5f) return pow_neg_half(v);
  return powf(v, e);
}

template <int KIND>
__device__ __forceinline__ float unary_grad(float g, float v, float p) {
  if constexpr (KIND == NUMRS_HIP_RELU) {
    return v > 0.0f ? g : 0.0f;  // backward.rs:158 (strict)
  } else if constexpr (KIND == NUMRS_HIP_SIGMOID) {
    return (g * v) * (1.0f - v);  // backward.rs:172
  } else if constexpr (KIND == NUMRS_HIP_TANH) {
    return g * (1.0f - v * v);  // backward.rs:508-515
  } else if constexpr (KIND == NUMRS_HIP_EXP) {
    return g * v;  // backward.rs:186
  } else if constexpr (KIND == NUMRS_HIP_LOG) {
    return g / v;  // backward.rs:200
  } else if constexpr (KIND == NUMRS_HIP_GELU) {
    const float cdf = 0.5f * (1.0f + erff(v * 0.70710678118654752f));
    const float pdf = 0.39894228040143268f * expf(-0.5f * v * v);
    return g * (cdf + v * pdf);
  } else if constexpr (KIND == NUMRS_HIP_SQRT) {
    return g * (pow_neg_half(v) * 0.5f);  // backward.rs:452-460
  } else if constexpr (KIND == NUMRS_HIP_SIN) {
    return g * cosf(v);  // backward.rs:469-470
  } else if constexpr (KIND == NUMRS_HIP_COS) {
    return g * (sinf(v) * -1.0f);  // backward.rs:478-481
  } else if constexpr (KIND == NUMRS_HIP_TAN) {
    return g * (1.0f + v * v);  // backward.rs:491-498
  } else {  // NUMRS_HIP_POW
    return g * (pow_grad_base(v, p - 1.0f) * p);  // backward.rs:427-435
  }
}

// One thread's 8 elements (two float4 groups kBlock*4 apart); threads whose
// groups both lie inside the array issue every load before any store.
template <int KIND, int VEC, bool ACC>
__device__ __forceinline__ void unary_bwd_body(const float *__restrict__ g,
                                               const float *__restrict__ v,
                                               float *__restrict__ dx, int64_t n, float p) {
  const int64_t base = (int64_t)blockIdx.x * kElemsPerBlock + threadIdx.x * 4;
  const int64_t last = base + (int64_t)(kVecPerThread - 1) * kBlock * 4;
  if (VEC && last + 3 < n) {
    f4 gv[kVecPerThread], vv[kVecPerThread], ov[kVecPerThread];
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      gv[u] = ldv<VEC>(g + i);
      vv[u] = ldv<VEC>(v + i);
      if (ACC) ov[u] = ldv<VEC>(dx + i);
    }
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      f4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = unary_grad<KIND>(gv[u][e], vv[u][e], p);
      stv<VEC>(dx + i, ACC ? ov[u] + r : r);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (i + e < n) {
        const float r = unary_grad<KIND>(g[i + e], v[i + e], p);
        dx[i + e] = ACC ? dx[i + e] + r : r;
      }
    }
  }
}

template <int KIND, int VEC>
__global__ void __launch_bounds__(kBlock)
    unary_bwd_kernel(const float *__restrict__ g, const float *__restrict__ v,
                     float *__restrict__ dx, int64_t n, float p, int acc) {
  if (acc) unary_bwd_body<KIND, VEC, true>(g, v, dx, n, p);
  else unary_bwd_body<KIND, VEC, false>(g, v, dx, n, p);
}

template <int KIND>
int launch_unary(numrs_hip_ctx *ctx, const float *g, const float *v, float *dx, int64_t n,
                 float p, int acc) {
  const unsigned grid = grid_for(n, kElemsPerBlock);
  const bool vec = numrs_hip::aligned16(g) && numrs_hip::aligned16(v) && numrs_hip::aligned16(dx);
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {
    unary_bwd_kernel<KIND, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(g, v, dx, n, p,
                                                                                acc);
  });
  return numrs_hip::check_launch(ctx, "unary_bwd_kernel");
}

// ---------------------------------------------------------------------------
// Binary backward (same shapes)
// ---------------------------------------------------------------------------

template <int KIND>
__device__ __forceinline__ void binary_grad(float g, float x, float y, float &dx, float &dy) {
  if constexpr (KIND == NUMRS_HIP_ADD) {
    dx = g;
    dy = g;
  } else if constexpr (KIND == NUMRS_HIP_SUB) {
    dx = g;
    dy = g * -1.0f;  // backward.rs:65-66
  } else if constexpr (KIND == NUMRS_HIP_MUL) {
    dx = g * y;  // backward.rs:79
    dy = g * x;  // backward.rs:83
  } else {       // DIV, backward.rs:95-104
    dx = g / y;
    const float ysq = y * y;
    const float term = x / ysq;
    dy = (g * term) * -1.0f;
  }
}

// One thread's 8 elements with the outputs present (DX, DY) and the
// accumulate flag (ACC) fixed at compile time: every load is then issued
// before the first store, instead of being sunk into the branches that use it.
// One thread's 8 elements (two float4 groups kBlock*4 apart) with the
// outputs present (DX, DY) and the accumulate flag (ACC) fixed at compile
// time.  Threads whose groups both lie inside the array issue every load
// before any store; the last block's ragged end goes element by element.
template <int KIND, int VEC, bool DX, bool DY, bool ACC>
__device__ __forceinline__ void binary_bwd_body(const float *__restrict__ g,
                                                const float *__restrict__ x,
                                                const float *__restrict__ y,
                                                float *__restrict__ dx, float *__restrict__ dy,
                                                int64_t n) {
  constexpr bool kReadsXY = KIND == NUMRS_HIP_MUL || KIND == NUMRS_HIP_DIV;
  const int64_t base = (int64_t)blockIdx.x * kElemsPerBlock + threadIdx.x * 4;
  const int64_t last = base + (int64_t)(kVecPerThread - 1) * kBlock * 4;
  if (VEC && last + 3 < n) {
    f4 gv[kVecPerThread], xv[kVecPerThread], yv[kVecPerThread], ov[kVecPerThread],
        pv[kVecPerThread];
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      gv[u] = ldv<VEC>(g + i);
      if (kReadsXY) {
        xv[u] = ldv<VEC>(x + i);
        yv[u] = ldv<VEC>(y + i);
      } else {
        xv[u] = yv[u] = f4{0.f, 0.f, 0.f, 0.f};
      }
      if (ACC && DX) ov[u] = ldv<VEC>(dx + i);
      if (ACC && DY) pv[u] = ldv<VEC>(dy + i);
    }
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      f4 a, b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float ae, be;
        binary_grad<KIND>(gv[u][e], xv[u][e], yv[u][e], ae, be);
        a[e] = ae;
        b[e] = be;
      }
      if (DX) stv<VEC>(dx + i, ACC ? ov[u] + a : a);
      if (DY) stv<VEC>(dy + i, ACC ? pv[u] + b : b);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t k = i + e;
      if (k < n) {
        const float xe = kReadsXY ? x[k] : 0.0f;
        const float ye = kReadsXY ? y[k] : 0.0f;
        float a, b;
        binary_grad<KIND>(g[k], xe, ye, a, b);
        if (DX) dx[k] = ACC ? dx[k] + a : a;
        if (DY) dy[k] = ACC ? dy[k] + b : b;
      }
    }
  }
}

template <int KIND, int VEC>
__global__ void __launch_bounds__(kBlock)
    binary_bwd_kernel(const float *__restrict__ g, const float *__restrict__ x,
                      const float *__restrict__ y, float *__restrict__ dx, float *__restrict__ dy,
                      int64_t n, int acc) {
  // The flags are uniform: one branch per thread picks the specialised body.
  if (dx != nullptr && dy != nullptr) {
    if (acc) binary_bwd_body<KIND, VEC, true, true, true>(g, x, y, dx, dy, n);
    else binary_bwd_body<KIND, VEC, true, true, false>(g, x, y, dx, dy, n);
  } else if (dx != nullptr) {
    if (acc) binary_bwd_body<KIND, VEC, true, false, true>(g, x, y, dx, dy, n);
    else binary_bwd_body<KIND, VEC, true, false, false>(g, x, y, dx, dy, n);
  } else if (dy != nullptr) {
    if (acc) binary_bwd_body<KIND, VEC, false, true, true>(g, x, y, dx, dy, n);
    else binary_bwd_body<KIND, VEC, false, true, false>(g, x, y, dx, dy, n);
  }
}

template <int KIND>
int launch_binary(numrs_hip_ctx *ctx, const float *g, const float *x, const float *y, float *dx,
                  float *dy, int64_t n, int acc) {
  const bool reads_xy = KIND == NUMRS_HIP_MUL || KIND == NUMRS_HIP_DIV;
  const bool vec = numrs_hip::aligned16(g) && numrs_hip::aligned16(dx) &&
                   numrs_hip::aligned16(dy) &&
                   (!reads_xy || (numrs_hip::aligned16(x) && numrs_hip::aligned16(y)));
  const unsigned grid = grid_for(n, kElemsPerBlock);
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {
    binary_bwd_kernel<KIND, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(g, x, y, dx, dy,
                                                                                 n, acc);
  });
  return numrs_hip::check_launch(ctx, "binary_bwd_kernel");
}

// ---------------------------------------------------------------------------
// sum/mean backward fill, MSE backward
// ---------------------------------------------------------------------------

template <int VEC>
__global__ void __launch_bounds__(kBlock)
    fill_grad_kernel(const float *__restrict__ g0, float *__restrict__ dx, int64_t n, float nf,
                     int divide, int acc) {
  const float v = divide ? g0[0] / nf : g0[0];  // backward.rs:213 / :228
  const int64_t base = (int64_t)blockIdx.x * kElemsPerBlock + threadIdx.x * 4;
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
    if (VEC && i + 3 < n) {
      f4 r = {v, v, v, v};
      if (acc) r += ldv<VEC>(dx + i);
      stv<VEC>(dx + i, r);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < n) dx[i + e] = acc ? dx[i + e] + v : v;
    }
  }
}

template <int VEC>
__global__ void __launch_bounds__(kBlock)
    mse_bwd_kernel(const float *__restrict__ g0, const float *__restrict__ p,
                   const float *__restrict__ t, float *__restrict__ dp, float *__restrict__ dt,
                   int64_t n, float nf, int acc, float *__restrict__ seed) {
  // seed: the loss is the backward's root -- g is its seed 1 (written here
  // for the root's gradient cell) rather than a value read back from g0.
  if (seed != nullptr && blockIdx.x == 0 && threadIdx.x == 0) seed[0] = 1.0f;
  const float gs = seed != nullptr ? 1.0f : g0[0];
  const int64_t base = (int64_t)blockIdx.x * kElemsPerBlock + threadIdx.x * 4;
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
    if (VEC && i + 3 < n) {
      const f4 pv = ldv<VEC>(p + i);
      const f4 tv = ldv<VEC>(t + i);
      f4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = ((gs * 2.0f) * (pv[e] - tv[e])) / nf;  // backward.rs:250
      if (dp) {
        f4 o = v;
        if (acc) o += ldv<VEC>(dp + i);
        stv<VEC>(dp + i, o);
      }
      if (dt) {
        f4 o = -v;  // backward.rs:257
        if (acc) o = ldv<VEC>(dt + i) + (-v);
        stv<VEC>(dt + i, o);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t k = i + e;
        if (k < n) {
          const float v = ((gs * 2.0f) * (p[k] - t[k])) / nf;  // backward.rs:250
          if (dp) dp[k] = acc ? dp[k] + v : v;
          if (dt) dt[k] = acc ? dt[k] + (-v) : -v;  // backward.rs:257
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Optimizers
// ---------------------------------------------------------------------------

// SGD::step, optim/sgd.rs:87-124 (+ apply_weight_decay, optim/base.rs:26-36).
// One block's kElemsPerBlock elements starting at blk * kElemsPerBlock (shared
// by sgd_kernel and, for 16-byte aligned tensors, sgd_multi_kernel).
template <bool MOMENTUM, bool DECAY, int VEC>
__device__ __forceinline__ void sgd_block(float *__restrict__ p, const float *__restrict__ g,
                                          float *__restrict__ v, int64_t n, float lr, float mu,
                                          float wd, int64_t blk) {
  const int64_t base = blk * kElemsPerBlock + threadIdx.x * 4;
  const int64_t last = base + (int64_t)(kVecPerThread - 1) * kBlock * 4;
  if (VEC && last + 3 < n) {  // both groups' loads before any store (as in adam_kernel)
    f4 pv[kVecPerThread], gv[kVecPerThread], vv[kVecPerThread];
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      pv[u] = ldv<VEC>(p + i);
      gv[u] = ldv<VEC>(g + i);
      if (MOMENTUM) vv[u] = ldv<VEC>(v + i);
    }
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float gg = gv[u][e];
        if (DECAY) gg = gg + wd * pv[u][e];
        if (MOMENTUM) {
          vv[u][e] = mu * vv[u][e] + gg;
          pv[u][e] = pv[u][e] - lr * vv[u][e];
        } else {
          pv[u][e] = pv[u][e] - lr * gg;
        }
      }
      stv<VEC>(p + i, pv[u]);
      if (MOMENTUM) stv<VEC>(v + i, vv[u]);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
    if (VEC && i + 3 < n) {
      f4 pv = ldv<VEC>(p + i);
      f4 gv = ldv<VEC>(g + i);
      f4 vv;
      if (MOMENTUM) vv = ldv<VEC>(v + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float gg = gv[e];
        if (DECAY) gg = gg + wd * pv[e];
        if (MOMENTUM) {
          vv[e] = mu * vv[e] + gg;
          pv[e] = pv[e] - lr * vv[e];
        } else {
          pv[e] = pv[e] - lr * gg;
        }
      }
      stv<VEC>(p + i, pv);
      if (MOMENTUM) stv<VEC>(v + i, vv);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t k = i + e;
        if (k < n) {
          float gg = g[k];
          if (DECAY) gg = gg + wd * p[k];
          if (MOMENTUM) {
            v[k] = mu * v[k] + gg;
            p[k] = p[k] - lr * v[k];
          } else {
            p[k] = p[k] - lr * gg;
          }
        }
      }
    }
  }
}

template <bool MOMENTUM, bool DECAY, int VEC>
__global__ void __launch_bounds__(kBlock)
    sgd_kernel(float *__restrict__ p, const float *__restrict__ g, float *__restrict__ v,
               int64_t n, float lr, float mu, float wd) {
  sgd_block<MOMENTUM, DECAY, VEC>(p, g, v, n, lr, mu, wd, blockIdx.x);
}

// The streaming probe (numrs_hip_stream_probe): y = a + b + c over the first
// `reads` of a, b, c (zeros when reads = 0), stored to y and, when writes =
// 2, to z; with writes = 0 nothing is stored (a block stores its first sum
// into y[blk] only if it equals -1.25, so the loads stay live).  Blocks of
// kElemsPerBlock, every load of a thread before its stores, as the other
// streaming kernels here.
template <int VEC>
__global__ void __launch_bounds__(kBlock)
    stream_probe_kernel(const float *__restrict__ a, const float *__restrict__ b,
                        const float *__restrict__ c, float *__restrict__ y,
                        float *__restrict__ z, int64_t n, int reads, int writes) {
  const int64_t blk = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t wbase = blk * kElemsPerBlock + (int64_t)wave * 256 * kVecPerThread + lane * 4;
  f4 v[kVecPerThread], w[3][kVecPerThread];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const float *src = r == 0 ? a : r == 1 ? b : c;
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = wbase + 256 * u;
      w[r][u] = r < reads && i + 3 < n ? ldv<VEC>(src + i) : f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) v[u] = (w[0][u] + w[1][u]) + w[2][u];
  if (writes == 0) {
    if (v[0][0] == -1.25f) y[blk] = v[0][0];
    return;
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = wbase + 256 * u;
    if (i + 3 < n) {
      stv<VEC>(y + i, v[u]);
      if (writes == 2) stv<VEC>(z + i, v[u]);
    }
  }
}

struct AdamArgs {
  float lr, b1, b2, eps, wd, omb1, omb2, bc1, bc2;
};

__device__ __forceinline__ void adam_elem(float &p, float g, float &m, float &v, const AdamArgs &a,
                                          bool decay) {
  if (decay) g = g + a.wd * p;                   // optim/base.rs:31-33
  m = a.b1 * m + a.omb1 * g;                     // adam.rs:144-146
  v = a.b2 * v + a.omb2 * g * g;                 // adam.rs:149-151
  const float mh = m / a.bc1;                    // adam.rs:160
  const float vh = v / a.bc2;                    // adam.rs:161
  p = p - a.lr * mh / (sqrtf(vh) + a.eps);       // adam.rs:162
}

// Adam::step, optim/adam.rs:124-167, fused into one pass over p, g, m, v.
// One block's kElemsPerBlock elements starting at blk * kElemsPerBlock (shared
// by adam_kernel and, for 16-byte aligned tensors, adam_multi_kernel).
template <bool DECAY, int VEC>
__device__ __forceinline__ void adam_block(float *__restrict__ p, const float *__restrict__ g,
                                           float *__restrict__ m, float *__restrict__ v,
                                           int64_t n, const AdamArgs &a, int64_t blk) {
  const int64_t base = blk * kElemsPerBlock + threadIdx.x * 4;
  if (VEC && (blk + 1) * kElemsPerBlock <= n) {
    // A whole block: wave w owns the kVecPerThread KiB-runs of its 2 KiB
    // stretch of every array, and a lane issues all its loads of one array
    // before the next array's, every load before any store.  On MI355X,
    // measured on this in-place read-4-write-3 stream from HBM: 0.76 of
    // 8 TB/s, against 0.71 with each group's four arrays loaded together and
    // the groups a block apart.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t wbase = blk * kElemsPerBlock + (int64_t)wave * 256 * kVecPerThread + lane * 4;
    f4 pv[kVecPerThread], gv[kVecPerThread], mv[kVecPerThread], vv[kVecPerThread];
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) pv[u] = ldv<VEC>(p + wbase + 256 * u);
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) gv[u] = ldv<VEC>(g + wbase + 256 * u);
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) mv[u] = ldv<VEC>(m + wbase + 256 * u);
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) vv[u] = ldv<VEC>(v + wbase + 256 * u);
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      const int64_t i = wbase + 256 * u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pv[u][e], me = mv[u][e], ve = vv[u][e];
        adam_elem(pe, gv[u][e], me, ve, a, DECAY);
        pv[u][e] = pe;
        mv[u][e] = me;
        vv[u][e] = ve;
      }
      stv<VEC>(p + i, pv[u]);
      stv<VEC>(m + i, mv[u]);
      stv<VEC>(v + i, vv[u]);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kVecPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
    if (VEC && i + 3 < n) {
      f4 pv = ldv<VEC>(p + i);
      const f4 gv = ldv<VEC>(g + i);
      f4 mv = ldv<VEC>(m + i);
      f4 vv = ldv<VEC>(v + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pv[e], me = mv[e], ve = vv[e];
        adam_elem(pe, gv[e], me, ve, a, DECAY);
        pv[e] = pe;
        mv[e] = me;
        vv[e] = ve;
      }
      stv<VEC>(p + i, pv);
      stv<VEC>(m + i, mv);
      stv<VEC>(v + i, vv);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t k = i + e;
        if (k < n) {
          float pe = p[k], me = m[k], ve = v[k];
          adam_elem(pe, g[k], me, ve, a, DECAY);
          p[k] = pe;
          m[k] = me;
          v[k] = ve;
        }
      }
    }
  }
}

template <bool DECAY, int VEC>
__global__ void __launch_bounds__(kBlock)
    adam_kernel(float *__restrict__ p, const float *__restrict__ g, float *__restrict__ m,
                float *__restrict__ v, int64_t n, AdamArgs a) {
  adam_block<DECAY, VEC>(p, g, m, v, n, a, blockIdx.x);
}

// Multi-tensor optimizer launch: up to kMaxMulti parameter tensors share one
// grid; block b belongs to the tensor t with start[t] <= b < start[t+1] and
// covers that tensor's elements from (b - start[t]) * kElemsPerBlock.
constexpr int kMaxMulti = 32;

struct MultiArgs {
  float *p[kMaxMulti];
  const float *g[kMaxMulti];
  float *s1[kMaxMulti];  // SGD velocity / Adam m
  float *s2[kMaxMulti];  // Adam v
  int64_t n[kMaxMulti];
  int64_t start[kMaxMulti + 1];
  int mode[kMaxMulti];  // access mode of each tensor (2: the float4 streaming body)
  int count;
};

__device__ __forceinline__ int multi_find(const MultiArgs &a, int64_t b) {
  int t = 0;
  while (t + 1 < a.count && a.start[t + 1] <= b) ++t;
  return t;
}

template <bool MOMENTUM, bool DECAY>
__global__ void __launch_bounds__(kBlock)
    sgd_multi_kernel(MultiArgs a, float lr, float mu, float wd) {
  const int t = multi_find(a, blockIdx.x);
  float *__restrict__ p = a.p[t];
  const float *__restrict__ g = a.g[t];
  float *__restrict__ v = a.s1[t];
  const int64_t n = a.n[t];
  if (a.mode[t] == 2) {  // a large tensor: the single-tensor kernel's float4 streaming body
    sgd_block<MOMENTUM, DECAY, 2>(p, g, v, n, lr, mu, wd, blockIdx.x - a.start[t]);
    return;
  }
  if (a.mode[t] == 1) {  // aligned: the same body with cached float4 accesses
    sgd_block<MOMENTUM, DECAY, 1>(p, g, v, n, lr, mu, wd, blockIdx.x - a.start[t]);
    return;
  }
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
#pragma unroll
  for (int u = 0; u < 4 * kVecPerThread; ++u) {
    const int64_t k = base + (int64_t)u * kBlock;
    if (k < n) {
      float gg = g[k];
      if (DECAY) gg = gg + wd * p[k];
      if (MOMENTUM) {
        v[k] = mu * v[k] + gg;
        p[k] = p[k] - lr * v[k];
      } else {
        p[k] = p[k] - lr * gg;
      }
    }
  }
}

template <bool DECAY>
__global__ void __launch_bounds__(kBlock) adam_multi_kernel(MultiArgs a, AdamArgs args) {
  const int t = multi_find(a, blockIdx.x);
  const int64_t n = a.n[t];
  if (a.mode[t] == 2) {  // a large tensor: the single-tensor kernel's float4 streaming body
    adam_block<DECAY, 2>(a.p[t], a.g[t], a.s1[t], a.s2[t], n, args, blockIdx.x - a.start[t]);
    return;
  }
  if (a.mode[t] == 1) {  // aligned: the same body with cached float4 accesses
    adam_block<DECAY, 1>(a.p[t], a.g[t], a.s1[t], a.s2[t], n, args, blockIdx.x - a.start[t]);
    return;
  }
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
#pragma unroll
  for (int u = 0; u < 4 * kVecPerThread; ++u) {
    const int64_t k = base + (int64_t)u * kBlock;
    if (k < n) {
      float pe = a.p[t][k], me = a.s1[t][k], ve = a.s2[t][k];
      adam_elem(pe, a.g[t][k], me, ve, args, DECAY);
      a.p[t][k] = pe;
      a.s1[t][k] = me;
      a.s2[t][k] = ve;
    }
  }
}

// Fills `a` for tensors [first, first+cnt); returns the number of blocks.
int64_t multi_pack(MultiArgs &a, float *const *p, const float *const *g, float *const *s1,
                   float *const *s2, const int64_t *n, int first, int cnt) {
  a.count = cnt;
  int64_t blocks = 0;
  for (int i = 0; i < cnt; ++i) {
    a.p[i] = p[first + i];
    a.g[i] = g[first + i];
    a.s1[i] = s1 ? s1[first + i] : nullptr;
    a.s2[i] = s2 ? s2[first + i] : nullptr;
    a.n[i] = n[first + i];
    const bool vec = numrs_hip::aligned16(a.p[i]) && numrs_hip::aligned16(a.g[i]) &&
                     numrs_hip::aligned16(a.s1[i]) && numrs_hip::aligned16(a.s2[i]);
    a.mode[i] = numrs_hip::vec_mode(vec, a.n[i]);
    a.start[i] = blocks;
    blocks += (n[first + i] + kElemsPerBlock - 1) / kElemsPerBlock;
  }
  a.start[cnt] = blocks;
  return blocks;
}

// f32::powi as lowered by Rust/LLVM on x86-64 (compiler-rt __powisf2):
// square-and-multiply over the exponent's bits, low bit first.
float powi_f32(float a, int b) {
  const bool recip = b < 0;
  if (recip) b = -b;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r = r * a;
    b /= 2;
    if (b == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / r : r;
}

int check_n(numrs_hip_ctx *ctx, const char *who, int64_t n) {
  if (n < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative length", who);
  return NUMRS_HIP_OK;
}

}  // namespace

namespace numrs_hip {

// mse_backward; with `seed` (the loss is the sweep's root) g is its seed 1,
// which the kernel also writes to seed[0].
int mse_backward_impl(numrs_hip_ctx *ctx, const float *g_scalar, float *seed, const float *p,
                      const float *t, float *dp, float *dt, int64_t n, int accumulate) {
  if (int rc = check_n(ctx, "numrs_hip_mse_backward", n)) return rc;
  if (n == 0 || (dp == nullptr && dt == nullptr)) {
    return seed != nullptr ? numrs_hip_fill(ctx, seed, 1, 1.0f) : NUMRS_HIP_OK;
  }
  if ((g_scalar == nullptr && seed == nullptr) || p == nullptr || t == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_mse_backward: null pointer");
  const bool vec = numrs_hip::aligned16(p) && numrs_hip::aligned16(t) &&
                   numrs_hip::aligned16(dp) && numrs_hip::aligned16(dt);
  const unsigned grid = grid_for(n, kElemsPerBlock);
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {
    mse_bwd_kernel<decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(
        g_scalar, p, t, dp, dt, n, (float)n, accumulate, seed);
  });
  return numrs_hip::check_launch(ctx, "mse_bwd_kernel");
}

}  // namespace numrs_hip

extern "C" {

int numrs_hip_unary_backward(numrs_hip_ctx *ctx, int kind, const float *g, const float *v,
                             float *dx, int64_t n, float param, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_unary_backward", n)) return rc;
  if (n == 0) return NUMRS_HIP_OK;
  if (g == nullptr || v == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_unary_backward: null pointer");
  switch (kind) {
    case NUMRS_HIP_RELU: return launch_unary<NUMRS_HIP_RELU>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_SIGMOID:
      return launch_unary<NUMRS_HIP_SIGMOID>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_TANH: return launch_unary<NUMRS_HIP_TANH>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_EXP: return launch_unary<NUMRS_HIP_EXP>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_LOG: return launch_unary<NUMRS_HIP_LOG>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_GELU: return launch_unary<NUMRS_HIP_GELU>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_SQRT: return launch_unary<NUMRS_HIP_SQRT>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_SIN: return launch_unary<NUMRS_HIP_SIN>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_COS: return launch_unary<NUMRS_HIP_COS>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_TAN: return launch_unary<NUMRS_HIP_TAN>(ctx, g, v, dx, n, param, accumulate);
    case NUMRS_HIP_POW: return launch_unary<NUMRS_HIP_POW>(ctx, g, v, dx, n, param, accumulate);
    default:
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_unary_backward: kind %d", kind);
  }
}

int numrs_hip_binary_backward(numrs_hip_ctx *ctx, int kind, const float *g, const float *x,
                              const float *y, float *dx, float *dy, int64_t n, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_binary_backward", n)) return rc;
  if (n == 0 || (dx == nullptr && dy == nullptr)) return NUMRS_HIP_OK;
  const bool needs_xy = kind == NUMRS_HIP_MUL || kind == NUMRS_HIP_DIV;
  if (g == nullptr || (needs_xy && (x == nullptr || y == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_binary_backward: null pointer");
  switch (kind) {
    case NUMRS_HIP_ADD: return launch_binary<NUMRS_HIP_ADD>(ctx, g, x, y, dx, dy, n, accumulate);
    case NUMRS_HIP_SUB: return launch_binary<NUMRS_HIP_SUB>(ctx, g, x, y, dx, dy, n, accumulate);
    case NUMRS_HIP_MUL: return launch_binary<NUMRS_HIP_MUL>(ctx, g, x, y, dx, dy, n, accumulate);
    case NUMRS_HIP_DIV: return launch_binary<NUMRS_HIP_DIV>(ctx, g, x, y, dx, dy, n, accumulate);
    default:
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_binary_backward: kind %d",
                             kind);
  }
}

int numrs_hip_fill_grad(numrs_hip_ctx *ctx, const float *g_scalar, float *dx, int64_t n,
                        int divide_by_n, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_fill_grad", n)) return rc;
  if (n == 0) return NUMRS_HIP_OK;
  if (g_scalar == nullptr || dx == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_fill_grad: null pointer");
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(numrs_hip::aligned16(dx), n), [&](auto V) {
    fill_grad_kernel<decltype(V)::value><<<grid_for(n, kElemsPerBlock), kBlock, 0,
                                           ctx->stream>>>(g_scalar, dx, n, (float)n, divide_by_n,
                                                          accumulate);
  });
  return numrs_hip::check_launch(ctx, "fill_grad_kernel");
}

int numrs_hip_mse_backward(numrs_hip_ctx *ctx, const float *g_scalar, const float *p,
                           const float *t, float *dp, float *dt, int64_t n, int accumulate) {
  NRS_CHECK_CTX(ctx);
  return numrs_hip::mse_backward_impl(ctx, g_scalar, nullptr, p, t, dp, dt, n, accumulate);
}

int numrs_hip_stream_probe(numrs_hip_ctx *ctx, const float *a, const float *b, const float *c,
                           float *y, float *z, int64_t n, int reads, int writes) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_stream_probe", n)) return rc;
  if (reads < 0 || reads > 3 || writes < 0 || writes > 2 || n % 4 != 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID,
                           "numrs_hip_stream_probe: reads %d writes %d n %lld", reads, writes,
                           (long long)n);
  if (n == 0) return NUMRS_HIP_OK;
  const float *src[3] = {a, b, c};
  bool ok = y != nullptr && numrs_hip::aligned16(y) && (writes < 2 || numrs_hip::aligned16(z));
  for (int r = 0; r < reads; ++r) ok = ok && numrs_hip::aligned16(src[r]);
  if (!ok)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID,
                           "numrs_hip_stream_probe: null or unaligned operand");
  const unsigned grid = grid_for(n, kElemsPerBlock);
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, n), [&](auto V) {
    stream_probe_kernel<decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(a, b, c, y, z, n,
                                                                              reads, writes);
  });
  return numrs_hip::check_launch(ctx, "stream_probe_kernel");
}

int numrs_hip_sgd_step(numrs_hip_ctx *ctx, float *p, const float *g, float *v, int64_t n,
                       float lr, float mu, float wd) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_sgd_step", n)) return rc;
  if (n == 0) return NUMRS_HIP_OK;
  if (p == nullptr || g == nullptr || (mu != 0.0f && v == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_sgd_step: null pointer");
  const unsigned grid = grid_for(n, kElemsPerBlock);
  const bool vec = numrs_hip::aligned16(p) && numrs_hip::aligned16(g) &&
                   (mu == 0.0f || numrs_hip::aligned16(v));
  const bool mom = mu != 0.0f, dec = wd != 0.0f;
#define NRS_SGD(M, D)                                                                      \
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {                       \
    sgd_kernel<M, D, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(p, g, v, n, lr, mu, \
                                                                          wd);             \
  })
  if (mom && dec) NRS_SGD(true, true);
  else if (mom) NRS_SGD(true, false);
  else if (dec) NRS_SGD(false, true);
  else NRS_SGD(false, false);
#undef NRS_SGD
  return numrs_hip::check_launch(ctx, "sgd_kernel");
}

int numrs_hip_sgd_step_multi(numrs_hip_ctx *ctx, float *const *p, const float *const *g,
                             float *const *v, const int64_t *n, int count, float lr, float mu,
                             float wd) {
  NRS_CHECK_CTX(ctx);
  if (count < 0 || (count > 0 && (p == nullptr || g == nullptr || n == nullptr)) ||
      (mu != 0.0f && count > 0 && v == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_sgd_step_multi: bad arguments");
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (p[i] == nullptr || g[i] == nullptr ||
                                  (mu != 0.0f && v[i] == nullptr))))
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_sgd_step_multi: tensor %d", i);
  for (int first = 0; first < count; first += kMaxMulti) {
    MultiArgs a;
    const int cnt = count - first < kMaxMulti ? count - first : kMaxMulti;
    const int64_t blocks = multi_pack(a, p, g, mu != 0.0f ? v : nullptr, nullptr, n, first, cnt);
    if (blocks == 0) continue;
    if (blocks > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "too many elements");
    const bool mom = mu != 0.0f, dec = wd != 0.0f;
    const unsigned grid = (unsigned)blocks;
    if (mom && dec) sgd_multi_kernel<true, true><<<grid, kBlock, 0, ctx->stream>>>(a, lr, mu, wd);
    else if (mom) sgd_multi_kernel<true, false><<<grid, kBlock, 0, ctx->stream>>>(a, lr, mu, wd);
    else if (dec) sgd_multi_kernel<false, true><<<grid, kBlock, 0, ctx->stream>>>(a, lr, mu, wd);
    else sgd_multi_kernel<false, false><<<grid, kBlock, 0, ctx->stream>>>(a, lr, mu, wd);
    if (int rc = numrs_hip::check_launch(ctx, "sgd_multi_kernel")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_adam_step_multi(numrs_hip_ctx *ctx, float *const *p, const float *const *g,
                              float *const *m, float *const *v, const int64_t *n, int count,
                              float lr, float b1, float b2, float eps, float wd, int t) {
  NRS_CHECK_CTX(ctx);
  if (t < 1) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_adam_step_multi: t < 1");
  if (count < 0 || (count > 0 && (!p || !g || !m || !v || !n)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_adam_step_multi: bad arguments");
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (!p[i] || !g[i] || !m[i] || !v[i])))
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_adam_step_multi: tensor %d", i);
  AdamArgs args;
  args.lr = lr;
  args.b1 = b1;
  args.b2 = b2;
  args.eps = eps;
  args.wd = wd;
  args.omb1 = 1.0f - b1;
  args.omb2 = 1.0f - b2;
  args.bc1 = 1.0f - powi_f32(b1, t);
  args.bc2 = 1.0f - powi_f32(b2, t);
  for (int first = 0; first < count; first += kMaxMulti) {
    MultiArgs a;
    const int cnt = count - first < kMaxMulti ? count - first : kMaxMulti;
    const int64_t blocks = multi_pack(a, p, g, m, v, n, first, cnt);
    if (blocks == 0) continue;
    if (blocks > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "too many elements");
    if (wd != 0.0f) adam_multi_kernel<true><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, args);
    else adam_multi_kernel<false><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, args);
    if (int rc = numrs_hip::check_launch(ctx, "adam_multi_kernel")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_adam_step(numrs_hip_ctx *ctx, float *p, const float *g, float *m, float *v,
                        int64_t n, float lr, float b1, float b2, float eps, float wd, int t) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check_n(ctx, "numrs_hip_adam_step", n)) return rc;
  if (t < 1) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_adam_step: t < 1");
  if (n == 0) return NUMRS_HIP_OK;
  if (p == nullptr || g == nullptr || m == nullptr || v == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_adam_step: null pointer");
  AdamArgs a;
  a.lr = lr;
  a.b1 = b1;
  a.b2 = b2;
  a.eps = eps;
  a.wd = wd;
  a.omb1 = 1.0f - b1;
  a.omb2 = 1.0f - b2;
  a.bc1 = 1.0f - powi_f32(b1, t);  // adam.rs:128
  a.bc2 = 1.0f - powi_f32(b2, t);  // adam.rs:129
  const unsigned grid = grid_for(n, kElemsPerBlock);
  const bool vec = numrs_hip::aligned16(p) && numrs_hip::aligned16(g) &&
                   numrs_hip::aligned16(m) && numrs_hip::aligned16(v);
  const bool dec = wd != 0.0f;
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {
    if (dec)
      adam_kernel<true, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(p, g, m, v, n, a);
    else
      adam_kernel<false, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(p, g, m, v, n, a);
  });
  return numrs_hip::check_launch(ctx, "adam_kernel");
}

}  // extern "C"
