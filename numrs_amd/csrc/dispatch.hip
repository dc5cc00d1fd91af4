// The forward kernels behind numrs's backend DispatchTable
// (backend/dispatch.rs:51-93): `elementwise(a, b, kind)` over the 21
// ElementwiseKinds (llo/elementwise.rs:38-68) and `reduction(a, axis, kind)`
// over the 6 ReductionKinds (llo/reduction.rs:12-19), with the semantics of
// the CPU reference backend (backend/cpu/scalar.rs).
//
// Elementwise: same-shape operands (scalar.rs:13-15 rejects others), one
// thread per two float4 groups with every load issued before the stores; the
// unary kinds read a only.  The exact kinds (+ - * / sqrt abs neg relu
// leaky_relu) give the reference's bits; the others call the device libm.
//
// Reduction: full (axis None) or one axis of x viewed as [outer, n, inner].
//   Sum, Mean            numrs_hip_sum / numrs_hip_reduce_axis
//   Max, Min             fold from -inf / +inf with fmaxf / fminf, which
//                        ignore NaN like f32::max / f32::min
//   ArgMax (full)        first index of the maximum scanning from x[0] with
//                        a strict '>' (scalar.rs:517-528): a NaN never
//                        replaces, and a NaN at x[0] is never replaced
//   ArgMax (axis)        fold from (0, -inf) with a strict '>'
//                        (scalar.rs:345-362, 623-668): NaNs are skipped and
//                        an axis of -inf/NaN gives 0
//   Variance             population variance; full: the mean first, then
//                        the mean of squared deviations (the reference runs
//                        Welford, scalar.rs:529-541); axis: the reference's
//                        two passes (scalar.rs:364-393, 671-717)
// Full reductions are two deterministic passes (block partials, then one
// block); axis reductions take one thread per output walking its axis with
// stride `inner`, so a wave's loads are coalesced over inner indices.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kVec = 2;  // float4 groups per thread
typedef float f4 __attribute__((ext_vector_type(4)));

template <int KIND>
__device__ __forceinline__ float ew(float a, float b) {
  switch (KIND) {
    case NUMRS_HIP_EW_ADD: return a + b;
    case NUMRS_HIP_EW_MUL: return a * b;
    case NUMRS_HIP_EW_SUB: return a - b;
    case NUMRS_HIP_EW_DIV: return a / b;
    case NUMRS_HIP_EW_POW: return powf(a, b);
    case NUMRS_HIP_EW_SQRT: return sqrtf(a);
    case NUMRS_HIP_EW_SIN: return sinf(a);
    case NUMRS_HIP_EW_COS: return cosf(a);
    case NUMRS_HIP_EW_TAN: return tanf(a);
    case NUMRS_HIP_EW_ASIN: return asinf(a);
    case NUMRS_HIP_EW_ACOS: return acosf(a);
    case NUMRS_HIP_EW_ATAN: return atanf(a);
    case NUMRS_HIP_EW_ABS: return fabsf(a);
    case NUMRS_HIP_EW_NEG: return -a;
    case NUMRS_HIP_EW_EXP: return expf(a);
    case NUMRS_HIP_EW_LOG: return logf(a);
    case NUMRS_HIP_EW_RELU: return fmaxf(a, 0.0f);                 // a.max(0.0)
    case NUMRS_HIP_EW_LEAKY_RELU: return a > 0.0f ? a : 0.01f * a;  // scalar.rs:120-125
    case NUMRS_HIP_EW_SIGMOID: return 1.0f / (1.0f + expf(-a));      // scalar.rs:127-131
    case NUMRS_HIP_EW_TANH: return tanhf(a);
    default: return logf(1.0f + expf(a));                            // softplus, scalar.rs:139-143
  }
}

constexpr bool binary_kind(int k) {
  return k == NUMRS_HIP_EW_ADD || k == NUMRS_HIP_EW_MUL || k == NUMRS_HIP_EW_SUB ||
         k == NUMRS_HIP_EW_DIV || k == NUMRS_HIP_EW_POW;
}

template <int KIND, bool VEC>
__global__ void __launch_bounds__(kBlock)
    ew_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ out,
              int64_t n) {
  constexpr bool kB = binary_kind(KIND);
  const int64_t base = (int64_t)blockIdx.x * (kBlock * 4 * kVec) + threadIdx.x * 4;
  const int64_t last = base + (int64_t)(kVec - 1) * kBlock * 4;
  if (VEC && last + 3 < n) {
    f4 av[kVec], bv[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + (int64_t)u * kBlock * 4;
      av[u] = *reinterpret_cast<const f4 *>(a + i);
      bv[u] = kB ? *reinterpret_cast<const f4 *>(b + i) : f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      f4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = ew<KIND>(av[u][e], bv[u][e]);
      *reinterpret_cast<f4 *>(out + base + (int64_t)u * kBlock * 4) = r;
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kVec; ++u) {
    const int64_t i = base + (int64_t)u * kBlock * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i + e < n) out[i + e] = ew<KIND>(a[i + e], kB ? b[i + e] : 0.0f);
  }
}

template <int KIND>
int launch_ew(numrs_hip_ctx *ctx, const float *a, const float *b, float *out, int64_t n) {
  const unsigned grid = grid_for(n, kBlock * 4 * kVec);
  const bool vec = numrs_hip::aligned16(a) && numrs_hip::aligned16(out) &&
                   (!binary_kind(KIND) || numrs_hip::aligned16(b));
  if (vec) ew_kernel<KIND, true><<<grid, kBlock, 0, ctx->stream>>>(a, b, out, n);
  else ew_kernel<KIND, false><<<grid, kBlock, 0, ctx->stream>>>(a, b, out, n);
  return numrs_hip::check_launch(ctx, "ew_kernel");
}

// ---------------------------------------------------------------------------
// Full reductions (two passes).  KIND: 0 max, 1 min, 2 argmax, 3 sum of
// squared deviations from *center.
// ---------------------------------------------------------------------------
struct Pair {
  float v;
  int64_t i;
};

// Candidate (v, i) beats (bv, bi) for "first strict maximum, NaN never wins".
__device__ __forceinline__ bool first_max_beats(float v, int64_t i, float bv, int64_t bi) {
  if (v != v || i < 0) return false;
  if (bi < 0 || bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

template <int KIND>
__global__ void __launch_bounds__(kBlock)
    full_pass1(const float *__restrict__ x, int64_t n, const float *__restrict__ center,
               float *__restrict__ pv, int64_t *__restrict__ pi) {
  __shared__ float sv[kBlock];
  __shared__ int64_t si[kBlock];
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  float acc = KIND == 0 ? -INFINITY : (KIND == 1 ? INFINITY : 0.0f);
  int64_t ai = -1;
  const float c = KIND == 3 ? center[0] : 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    if (KIND == 0) acc = fmaxf(acc, v);
    else if (KIND == 1) acc = fminf(acc, v);
    else if (KIND == 2) {
      if (first_max_beats(v, i, acc, ai)) {
        acc = v;
        ai = i;
      }
    } else {
      const float d = v - c;
      acc += d * d;
    }
  }
  sv[threadIdx.x] = acc;
  si[threadIdx.x] = ai;
  __syncthreads();
  // Fixed-order tree in LDS (deterministic).
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      const float ov = sv[threadIdx.x + s];
      const int64_t oi = si[threadIdx.x + s];
      if (KIND == 0) sv[threadIdx.x] = fmaxf(sv[threadIdx.x], ov);
      else if (KIND == 1) sv[threadIdx.x] = fminf(sv[threadIdx.x], ov);
      else if (KIND == 2) {
        if (first_max_beats(ov, oi, sv[threadIdx.x], si[threadIdx.x])) {
          sv[threadIdx.x] = ov;
          si[threadIdx.x] = oi;
        }
      } else {
        sv[threadIdx.x] += ov;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = sv[0];
    if (KIND == 2) pi[blockIdx.x] = si[0];
  }
}

// Combines the block partials in block order; ARGMAX writes the index as a
// float (the reference's `max_idx as f32`), VARIANCE divides by n.
template <int KIND>
__global__ void __launch_bounds__(64)
    full_final(const float *__restrict__ x, const float *__restrict__ pv,
               const int64_t *__restrict__ pi, int blocks, int64_t n, float *__restrict__ out) {
  if (threadIdx.x != 0) return;
  float acc = KIND == 0 ? -INFINITY : (KIND == 1 ? INFINITY : 0.0f);
  int64_t ai = -1;
  for (int b = 0; b < blocks; ++b) {
    if (KIND == 0) acc = fmaxf(acc, pv[b]);
    else if (KIND == 1) acc = fminf(acc, pv[b]);
    else if (KIND == 2) {
      if (first_max_beats(pv[b], pi[b], acc, ai)) {
        acc = pv[b];
        ai = pi[b];
      }
    } else {
      acc += pv[b];
    }
  }
  if (KIND == 2) {
    // x[0] NaN: nothing ever replaces it (scalar.rs:520-526); all-NaN: 0 too.
    out[0] = (x[0] != x[0] || ai < 0) ? 0.0f : (float)ai;
  } else if (KIND == 3) {
    out[0] = acc / (float)n;
  } else {
    out[0] = acc;
  }
}

// ---------------------------------------------------------------------------
// Axis reductions, one thread per output.  KIND: 0 max, 1 min, 2 argmax,
// 3 variance.
// ---------------------------------------------------------------------------
template <int KIND>
__global__ void __launch_bounds__(kBlock)
    axis_kernel(const float *__restrict__ x, float *__restrict__ out, int64_t outer, int64_t n,
                int64_t inner) {
  const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (o >= outer * inner) return;
  const int64_t b = o / inner, i = o - b * inner;
  const float *src = x + b * n * inner + i;
  if (KIND == 0 || KIND == 1) {
    float acc = KIND == 0 ? -INFINITY : INFINITY;
    for (int64_t k = 0; k < n; ++k) acc = KIND == 0 ? fmaxf(acc, src[k * inner])
                                                    : fminf(acc, src[k * inner]);
    out[o] = acc;
  } else if (KIND == 2) {
    float best = -INFINITY;
    int64_t idx = 0;
    for (int64_t k = 0; k < n; ++k) {
      const float v = src[k * inner];
      if (v > best) {  // scalar.rs:352-358, 663-666
        best = v;
        idx = k;
      }
    }
    out[o] = (float)idx;
  } else {
    float s = 0.0f;
    for (int64_t k = 0; k < n; ++k) s += src[k * inner];
    const float mean = s / (float)n;
    float v = 0.0f;
    for (int64_t k = 0; k < n; ++k) {
      const float d = src[k * inner] - mean;
      v += d * d;
    }
    out[o] = v / (float)n;
  }
}

template <int KIND>
int full_reduction(numrs_hip_ctx *ctx, const float *x, int64_t n, const float *center,
                   float *out) {
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  int64_t blocks = (n + kBlock * 16 - 1) / (kBlock * 16);
  blocks = blocks < 1 ? 1 : (blocks > cus ? cus : blocks);
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)blocks * (sizeof(float) + sizeof(int64_t)), &ws))
    return rc;
  int64_t *pi = static_cast<int64_t *>(ws);
  float *pv = reinterpret_cast<float *>(pi + blocks);
  full_pass1<KIND><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(x, n, center, pv, pi);
  if (int rc = numrs_hip::check_launch(ctx, "full_pass1")) return rc;
  full_final<KIND><<<1, 64, 0, ctx->stream>>>(x, pv, pi, (int)blocks, n, out);
  return numrs_hip::check_launch(ctx, "full_final");
}

template <int KIND>
int axis_reduction(numrs_hip_ctx *ctx, const float *x, int64_t outer, int64_t n, int64_t inner,
                   float *out) {
  axis_kernel<KIND><<<grid_for(outer * inner, kBlock), kBlock, 0, ctx->stream>>>(x, out, outer,
                                                                                 n, inner);
  return numrs_hip::check_launch(ctx, "axis_kernel");
}

}  // namespace

extern "C" {

int numrs_hip_elementwise(numrs_hip_ctx *ctx, int kind, const float *a, const float *b,
                          float *out, int64_t n) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_elementwise";
  if (n < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative size", who);
  if (kind < NUMRS_HIP_EW_ADD || kind > NUMRS_HIP_EW_SOFTPLUS)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: kind %d", who, kind);
  if (n == 0) return NUMRS_HIP_OK;
  const bool needs_b = kind <= NUMRS_HIP_EW_POW;
  if (a == nullptr || out == nullptr || (needs_b && b == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null pointer", who);
  switch (kind) {
#define NRS_EW(K) \
  case K: return launch_ew<K>(ctx, a, b, out, n);
    NRS_EW(NUMRS_HIP_EW_ADD) NRS_EW(NUMRS_HIP_EW_MUL) NRS_EW(NUMRS_HIP_EW_SUB)
    NRS_EW(NUMRS_HIP_EW_DIV) NRS_EW(NUMRS_HIP_EW_POW) NRS_EW(NUMRS_HIP_EW_SQRT)
    NRS_EW(NUMRS_HIP_EW_SIN) NRS_EW(NUMRS_HIP_EW_COS) NRS_EW(NUMRS_HIP_EW_TAN)
    NRS_EW(NUMRS_HIP_EW_ASIN) NRS_EW(NUMRS_HIP_EW_ACOS) NRS_EW(NUMRS_HIP_EW_ATAN)
    NRS_EW(NUMRS_HIP_EW_ABS) NRS_EW(NUMRS_HIP_EW_NEG) NRS_EW(NUMRS_HIP_EW_EXP)
    NRS_EW(NUMRS_HIP_EW_LOG) NRS_EW(NUMRS_HIP_EW_RELU) NRS_EW(NUMRS_HIP_EW_LEAKY_RELU)
    NRS_EW(NUMRS_HIP_EW_SIGMOID) NRS_EW(NUMRS_HIP_EW_TANH) NRS_EW(NUMRS_HIP_EW_SOFTPLUS)
#undef NRS_EW
    default: return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: kind %d", who, kind);
  }
}

int numrs_hip_reduction(numrs_hip_ctx *ctx, int kind, const float *x, const int64_t *shape,
                        int nd, int axis, float *out) {
  NRS_CHECK_CTX(ctx);
  const char *who = "numrs_hip_reduction";
  if (nd < 0 || nd > 8 || (nd > 0 && shape == nullptr) || out == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: bad arguments", who);
  if (kind < NUMRS_HIP_RED_SUM || kind > NUMRS_HIP_RED_VARIANCE)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: kind %d", who, kind);
  int64_t total = 1;
  for (int d = 0; d < nd; ++d) {
    if (shape[d] < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: negative dim", who);
    total *= shape[d];
  }
  if (total > 0 && x == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "%s: null input", who);
  if (axis < 0) {  // axis None: shape [1]
    if (total == 0) {
      // The reference indexes a.data[0] for ArgMax and divides by 0 for
      // Mean / Variance; an empty input is an error here.
      if (kind == NUMRS_HIP_RED_SUM) return numrs_hip_fill(ctx, out, 1, 0.0f);
      if (kind == NUMRS_HIP_RED_MAX) return numrs_hip_fill(ctx, out, 1, -INFINITY);
      if (kind == NUMRS_HIP_RED_MIN) return numrs_hip_fill(ctx, out, 1, INFINITY);
      return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "%s: empty input", who);
    }
    switch (kind) {
      case NUMRS_HIP_RED_SUM: return numrs_hip_sum(ctx, x, total, 0, out);
      case NUMRS_HIP_RED_MEAN: return numrs_hip_sum(ctx, x, total, 1, out);
      case NUMRS_HIP_RED_MAX: return full_reduction<0>(ctx, x, total, nullptr, out);
      case NUMRS_HIP_RED_MIN: return full_reduction<1>(ctx, x, total, nullptr, out);
      case NUMRS_HIP_RED_ARGMAX: return full_reduction<2>(ctx, x, total, nullptr, out);
      default:
        // mean into out[0] first, then the squared deviations from it
        if (int rc = numrs_hip_sum(ctx, x, total, 1, out)) return rc;
        return full_reduction<3>(ctx, x, total, out, out);
    }
  }
  if (axis >= nd) return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "%s: axis %d of %d", who, axis, nd);
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < axis; ++d) outer *= shape[d];
  for (int d = axis + 1; d < nd; ++d) inner *= shape[d];
  const int64_t n = shape[axis];
  if (outer * inner == 0) return NUMRS_HIP_OK;
  if (n == 0) {
    if (kind == NUMRS_HIP_RED_SUM) return numrs_hip_fill(ctx, out, outer * inner, 0.0f);
    if (kind == NUMRS_HIP_RED_MAX) return numrs_hip_fill(ctx, out, outer * inner, -INFINITY);
    if (kind == NUMRS_HIP_RED_MIN) return numrs_hip_fill(ctx, out, outer * inner, INFINITY);
    if (kind == NUMRS_HIP_RED_ARGMAX) return numrs_hip_fill(ctx, out, outer * inner, 0.0f);
    return numrs_hip_fill(ctx, out, outer * inner, NAN);
  }
  switch (kind) {
    case NUMRS_HIP_RED_SUM: return numrs_hip_reduce_axis(ctx, x, outer, n, inner, 0, out);
    case NUMRS_HIP_RED_MEAN: return numrs_hip_reduce_axis(ctx, x, outer, n, inner, 1, out);
    case NUMRS_HIP_RED_MAX: return axis_reduction<0>(ctx, x, outer, n, inner, out);
    case NUMRS_HIP_RED_MIN: return axis_reduction<1>(ctx, x, outer, n, inner, out);
    case NUMRS_HIP_RED_ARGMAX: return axis_reduction<2>(ctx, x, outer, n, inner, out);
    default: return axis_reduction<3>(ctx, x, outer, n, inner, out);
  }
}

}  // extern "C"
