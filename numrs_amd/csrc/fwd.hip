// Forward kernels the autograd engine records nodes for: broadcasting binary
// ops, activations, 2-D transpose, full reductions and losses, row softmax and
// LayerNorm.  They stand where the reference's DispatchTable kernels and the
// inline loops of autograd/ops.rs stand (backend/dispatch.rs:69-93,
// autograd/ops.rs:14-555), so that a whole training step stays on the device.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
typedef float f4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Elementwise binary with numpy broadcasting (promotion_wrappers.rs:25-168)
// ---------------------------------------------------------------------------

template <int OP>
__device__ __forceinline__ float bin(float a, float b) {
  if constexpr (OP == NUMRS_HIP_ADD) return a + b;
  else if constexpr (OP == NUMRS_HIP_SUB) return a - b;
  else if constexpr (OP == NUMRS_HIP_MUL) return a * b;
  else return a / b;
}

struct Bcast {
  int nd;
  int64_t shape[8];
  int64_t sa[8], sb[8];  // element strides of a and b (0 on broadcast axes)
};

template <int OP>
__global__ void __launch_bounds__(kBlock)
    binary_flat_kernel(const float *__restrict__ a, const float *__restrict__ b,
                       float *__restrict__ out, int64_t n, int a_scalar, int b_scalar) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  out[i] = bin<OP>(a[a_scalar ? 0 : i], b[b_scalar ? 0 : i]);
}

// The same for 16-byte aligned operands: two float4 groups per thread, a
// block-width apart, both loaded before either is computed; a scalar operand
// is read once.  Element values equal binary_flat_kernel's (operands may
// alias the output).
template <int OP, int VM>
__global__ void __launch_bounds__(kBlock)
    binary_flat_vec(const float *a, const float *b, float *out, int64_t n, int a_scalar,
                    int b_scalar) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const int64_t i0 = (int64_t)blockIdx.x * kBlock * 8 + 4 * threadIdx.x;
  const int64_t i1 = i0 + 4 * kBlock;
  if (i1 + 3 < n) {
    const float as = a_scalar ? a[0] : 0.0f, bs = b_scalar ? b[0] : 0.0f;
    const f4v sa = {as, as, as, as}, sb = {bs, bs, bs, bs};
    const f4v a0 = a_scalar ? sa : numrs_hip::ldv<VM>(a + i0);
    const f4v a1 = a_scalar ? sa : numrs_hip::ldv<VM>(a + i1);
    const f4v b0 = b_scalar ? sb : numrs_hip::ldv<VM>(b + i0);
    const f4v b1 = b_scalar ? sb : numrs_hip::ldv<VM>(b + i1);
    f4v o0, o1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0[e] = bin<OP>(a0[e], b0[e]);
      o1[e] = bin<OP>(a1[e], b1[e]);
    }
    numrs_hip::stv<VM>(out + i0, o0);
    numrs_hip::stv<VM>(out + i1, o1);
    return;
  }
  for (int e = 0; e < 4; ++e)
    for (int64_t i : {i0 + e, i1 + e})
      if (i < n) out[i] = bin<OP>(a[a_scalar ? 0 : i], b[b_scalar ? 0 : i]);
}

// [rows, cols] op [cols] (the Linear bias add and its relatives).
template <int OP>
__global__ void __launch_bounds__(kBlock)
    binary_rowbcast_kernel(const float *__restrict__ a, const float *__restrict__ b,
                           float *__restrict__ out, int64_t rows, int64_t cols, int b_is_row) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= rows * cols) return;
  const int64_t c = i % cols;
  out[i] = b_is_row ? bin<OP>(a[i], b[c]) : bin<OP>(b[c], a[i]);
}

template <int OP>
__global__ void __launch_bounds__(kBlock)
    binary_bcast_kernel(const float *__restrict__ a, const float *__restrict__ b,
                        float *__restrict__ out, int64_t n, Bcast bc) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  int64_t rem = i, ia = 0, ib = 0;
  for (int d = bc.nd - 1; d >= 0; --d) {
    const int64_t c = rem % bc.shape[d];
    rem /= bc.shape[d];
    ia += c * bc.sa[d];
    ib += c * bc.sb[d];
  }
  out[i] = bin<OP>(a[ia], b[ib]);
}

// ---------------------------------------------------------------------------
// Unary forward (autograd/ops.rs:122-211, 488-554; GELU is new)
// ---------------------------------------------------------------------------

template <int KIND>
__device__ __forceinline__ float un(float x, float p) {
  if constexpr (KIND == NUMRS_HIP_RELU) return fmaxf(x, 0.0f);  // x.max(0.0), NaN -> 0
  else if constexpr (KIND == NUMRS_HIP_SIGMOID) return 1.0f / (1.0f + expf(-x));
  else if constexpr (KIND == NUMRS_HIP_TANH) return tanhf(x);
  else if constexpr (KIND == NUMRS_HIP_EXP) return expf(x);
  else if constexpr (KIND == NUMRS_HIP_LOG) return logf(x);
  else if constexpr (KIND == NUMRS_HIP_GELU) return numrs_hip::gelu_erf(x);
  else if constexpr (KIND == NUMRS_HIP_SQRT) return sqrtf(x);
  else if constexpr (KIND == NUMRS_HIP_SIN) return sinf(x);
  else if constexpr (KIND == NUMRS_HIP_COS) return cosf(x);
  else if constexpr (KIND == NUMRS_HIP_TAN) return tanf(x);
  else return powf(x, p);
}

template <int KIND>
__global__ void __launch_bounds__(kBlock)
    unary_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n, float p) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = un<KIND>(x[i], p);
}

// The same for 16-byte aligned x and y: a thread owns two float4 groups a
// block-width apart and loads both before computing either (kUnaryPerBlock
// elements per block); a group past the end is done element by element.
// Each element's value is the scalar kernel's (x and y may alias).
constexpr int kUnaryPerBlock = kBlock * 8;

template <int KIND, int VM>
__global__ void __launch_bounds__(kBlock)
    unary_fwd_vec(const float *x, float *y, int64_t n, float p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const int64_t i0 = (int64_t)blockIdx.x * kUnaryPerBlock + 4 * threadIdx.x;
  const int64_t i1 = i0 + 4 * kBlock;
  if (i1 + 3 < n) {
    f4v a = numrs_hip::ldv<VM>(x + i0), b = numrs_hip::ldv<VM>(x + i1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = un<KIND>(a[e], p);
      b[e] = un<KIND>(b[e], p);
    }
    numrs_hip::stv<VM>(y + i0, a);
    numrs_hip::stv<VM>(y + i1, b);
    return;
  }
  for (int e = 0; e < 4; ++e) {
    if (i0 + e < n) y[i0 + e] = un<KIND>(x[i0 + e], p);
    if (i1 + e < n) y[i1 + e] = un<KIND>(x[i1 + e], p);
  }
}

// ---------------------------------------------------------------------------
// Transpose (ops/shape/transpose.rs:9-88): 32x32 LDS tiles, padded rows.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(kBlock)
    transpose_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t rows,
                     int64_t cols) {
  __shared__ float tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = x[r * cols + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;  // output row c, column r
    if (c < cols && r < rows) y[c * rows + r] = tile[tx][k];
  }
}

// TS x TS tiles (64 or 128) with float4 global loads and stores, for
// 16-byte aligned matrices whose dimensions are multiples of 4 (each float4
// is then wholly inside or outside the matrix).  With Q = TS/4 float4 groups
// per tile row and K = 256/Q rows per pass, thread t loads rows t/Q + K i,
// columns 4(t%Q)..+3, and stores output row t/Q + K i (a column of x),
// output columns 4(t%Q)..+3, read down the LDS tile.  Row stride TS + 1
// keeps the column reads spread over the banks.
// All loads are issued before the tile is written: a tile row past the
// matrix edge reloads the last row or column group (rows and cols are
// nonzero multiples of 4 here) and is not stored, so no load sits in a branch
// with its use.  VM is the access mode (non-temporal for large matrices).
template <int VM, int TS>
__global__ void __launch_bounds__(kBlock)
    transpose_tile_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t rows,
                          int64_t cols) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  constexpr int kQ = TS / 4;           // float4 groups per tile row
  constexpr int kK = kBlock / kQ;      // tile rows per pass of the block
  constexpr int kPass = TS / kK;
  __shared__ float tile[TS][TS + 1];
  const int64_t r0 = (int64_t)blockIdx.y * TS, c0 = (int64_t)blockIdx.x * TS;
  const int t = threadIdx.x, q = t % kQ, k0 = t / kQ;
  f4v v[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int64_t r = r0 + k0 + kK * i, c = c0 + 4 * q;
    v[i] = numrs_hip::ldv<VM>(x + (r < rows ? r : rows - 1) * cols + (c < cols ? c : cols - 4));
  }
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int k = k0 + kK * i;
    if (r0 + k < rows && c0 + 4 * q < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[k][4 * q + e] = v[i][e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int k = k0 + kK * i;  // output row c0 + k, output columns r0 + 4q..
    const int64_t c = c0 + k, r = r0 + 4 * q;
    if (c < cols && r < rows) {
      f4v o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = tile[4 * q + e][k];
      numrs_hip::stv<VM>(y + c * rows + r, o);
    }
  }
}

// Register transpose for 16-byte aligned matrices of at least 64 x 256 whose
// dimensions are multiples of 4: a workgroup moves a 64 x 256 block of x as
// sixteen 32 x 32 blocks, four per wave, with no LDS and no barrier.  Lane
// (a = lane / 8, q = lane % 8) of a 32 x 32 block loads rows 4a..4a+3 at float4
// column q (eight lanes read one 128-byte run of each row), transposes the
// 4 x 4 in registers and stores output rows 4q..4q+3 at float4 column a (eight
// lanes write 128 contiguous bytes of each).  All sixteen loads of a lane are
// issued before the first store.  A 4 x 4 block past the matrix edge (wholly
// outside, as rows and cols are multiples of 4) reloads the last in-range
// block and is not stored.  At 4096 x 4096 this order measured about 5% faster
// than the LDS tiles on MI355X.
template <int VM>
__global__ void __launch_bounds__(kBlock)
    transpose_reg_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t rows,
                         int64_t cols) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  constexpr int kWR = 2, kWC = 8, kNB = kWR * kWC / 4;  // 32 x 32 blocks: per group, per wave
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, a = l >> 3, q = l & 7;
  const int64_t r0 = (int64_t)blockIdx.y * 32 * kWR, c0 = (int64_t)blockIdx.x * 32 * kWC;
  f4v v[kNB][4];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    const int blk = w + 4 * b;
    const int64_t r = r0 + 32 * (blk / kWC) + 4 * a, c = c0 + 32 * (blk % kWC) + 4 * q;
    const float *src = x + (r < rows ? r : rows - 4) * cols + (c < cols ? c : cols - 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[b][j] = numrs_hip::ldv<VM>(src + j * cols);
  }
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    const int blk = w + 4 * b;
    const int64_t r = r0 + 32 * (blk / kWC) + 4 * a, c = c0 + 32 * (blk % kWC) + 4 * q;
    if (r < rows && c < cols) {
      float *dst = y + c * rows + r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f4v o = {v[b][0][j], v[b][1][j], v[b][2][j], v[b][3][j]};
        numrs_hip::stv<VM>(dst + j * rows, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Full reductions: sum / mean / MSE loss (ops.rs:214-278)
// ---------------------------------------------------------------------------

// kind 0: sum x; 1: sum (x - t)^2.  Each thread walks float4 groups with a
// grid stride (VEC: 16-byte aligned operands), eight loads per operand in
// flight at once, into four independent partial sums that are added in a
// fixed order, then across the wave and the block.
// With dp (KIND 1): dp = ((1 * 2) (x - t)) / n as well, the gradient of the MSE
// loss's backward when the loss is the root (g = 1), with mse_bwd_kernel's
// arithmetic.  seed (may be null) receives 1 from a lone block.
template <int KIND, int VEC>
__global__ void __launch_bounds__(kBlock)
    reduce_pass1(const float *__restrict__ x, const float *__restrict__ t, int64_t n,
                 float *__restrict__ partial, float div, float *__restrict__ dp,
                 float *__restrict__ seed) {
  __shared__ float red[kBlock / 64];
  auto term = [&](float xv, float tv) {
    if (KIND == 0) return xv;
    const float d = xv - tv;
    return d * d;
  };
  float s = 0.0f;
  if (VEC) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const int64_t n4 = n / 4;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const float nf = (float)n;
    auto grad4 = [&](const f4v &xv, const f4v &tv, int64_t j) {
      f4v o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = ((1.0f * 2.0f) * (xv[e] - tv[e])) / nf;
      numrs_hip::stv<VEC>(dp + 4 * j, o);
    };
    for (; i + 7 * stride < n4; i += 8 * stride) {
      f4v xv[8], tv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        xv[u] = numrs_hip::ldv<VEC>(x + 4 * (i + u * stride));
        if (KIND == 1) tv[u] = numrs_hip::ldv<VEC>(t + 4 * (i + u * stride));
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[u & 3] += term(xv[u][e], KIND == 1 ? tv[u][e] : 0.0f);
      if (KIND == 1 && dp != nullptr)
#pragma unroll
        for (int u = 0; u < 8; ++u) grad4(xv[u], tv[u], i + u * stride);
    }
    for (; i < n4; i += stride) {
      const f4v xv = numrs_hip::ldv<VEC>(x + 4 * i);
      f4v tv = {0.f, 0.f, 0.f, 0.f};
      if (KIND == 1) tv = numrs_hip::ldv<VEC>(t + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[0] += term(xv[e], tv[e]);
      if (KIND == 1 && dp != nullptr) grad4(xv, tv, i);
    }
    // The n % 4 tail, taken by the first threads of block 0.
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int64_t k = n4 * 4 + threadIdx.x;
      acc[0] += term(x[k], KIND == 1 ? t[k] : 0.0f);
      if (KIND == 1 && dp != nullptr) dp[k] = ((1.0f * 2.0f) * (x[k] - t[k])) / nf;
    }
    s = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  } else {
    const float nf = (float)n;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock) {
      s += term(x[i], KIND == 1 ? t[i] : 0.0f);
      if (KIND == 1 && dp != nullptr) dp[i] = ((1.0f * 2.0f) * (x[i] - t[i])) / nf;
    }
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    partial[blockIdx.x] = gridDim.x == 1 ? tot / div : tot;  // a lone block writes the result
    if (gridDim.x == 1 && seed != nullptr) seed[0] = 1.0f;
  }
}

// out[0] = (sum of partials) / div   (div = 1 for a plain sum)
__global__ void __launch_bounds__(kBlock)
    reduce_final(const float *__restrict__ partial, int64_t count, float div,
                 float *__restrict__ out, float *__restrict__ seed) {
  __shared__ float red[kBlock / 64];
  // Loads go out in batches of 8 before they are added (in index order), so
  // a thread waits for one memory round trip per batch.
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
    out[0] = (((red[0] + red[1]) + red[2]) + red[3]) / div;
    if (seed != nullptr) seed[0] = 1.0f;
  }
}

// Cross-entropy rows (ops.rs:281-318): per row -sum_j t_j * ((x_j - m) - log(sum e)).
template <bool LABELS>
__global__ void __launch_bounds__(kBlock)
    ce_rows_kernel(const float *__restrict__ x, const float *__restrict__ onehot,
                   const int32_t *__restrict__ labels, float *__restrict__ row_loss, int64_t B,
                   int64_t C) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= B) return;
  const float *xr = x + row * C;
  float m = -INFINITY;
  for (int64_t j = lane; j < C; j += 64) m = fmaxf(m, xr[j]);
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t j = lane; j < C; j += 64) s += expf(xr[j] - m);
  s = wave_sum(s);
  const float ls = logf(s);
  float l = 0.0f;
  for (int64_t j = lane; j < C; j += 64) {
    const float t = LABELS ? (j == (int64_t)labels[row] ? 1.0f : 0.0f) : onehot[row * C + j];
    l += -t * ((xr[j] - m) - ls);
  }
  l = wave_sum(l);
  if (lane == 0) row_loss[row] = l;
}

// The whole cross-entropy loss of a small batch (B <= kCeSmallRows) in one
// workgroup: wave w forms the row losses of rows w, w + 16, ... as
// ce_rows_kernel does and adds them in row order; the 16 wave sums are then
// added in wave order and divided by B.  One launch instead of the row
// kernel and a reduction.
constexpr int kCeSmallWaves = 16;
constexpr int64_t kCeSmallRows = 512;

// RPW > 0 (rows of at most 64 classes, at most RPW rows per wave): every row
// of the wave, with its targets, is loaded into registers before the first is
// reduced (one memory round trip instead of one per row); lane j holds
// column j, and the per-lane values are formed exactly as the loop below
// forms them, so the sums and outputs are the same bits.
template <bool LABELS, int RPW>
__global__ void __launch_bounds__(64 * kCeSmallWaves)
    ce_loss_small_kernel(const float *__restrict__ x, const float *__restrict__ onehot,
                         const int32_t *__restrict__ labels, int64_t B, int64_t C,
                         float *__restrict__ out, float *__restrict__ dx,
                         float *__restrict__ seed) {
  __shared__ float red[kCeSmallWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float acc = 0.0f;
  if constexpr (RPW > 0) {
    const bool in = lane < C;
    const int64_t j = in ? lane : 0;  // lanes past the row read column 0 and discard it
    float xv[RPW], tv[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      int64_t row = wave + (int64_t)k * kCeSmallWaves;
      if (row > B - 1) row = B - 1;  // loaded, not used
      xv[k] = x[row * C + j];
      tv[k] = LABELS ? (j == (int64_t)labels[row] ? 1.0f : 0.0f) : onehot[row * C + j];
    }
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int64_t row = wave + (int64_t)k * kCeSmallWaves;
      if (row >= B) break;
      float m = in ? fmaxf(-INFINITY, xv[k]) : -INFINITY;
      m = wave_max(m);
      float s = in ? 0.0f + expf(xv[k] - m) : 0.0f;
      s = wave_sum(s);
      const float ls = logf(s);
      float l = 0.0f;
      if (in) {
        const float t = tv[k];
        l += -t * ((xv[k] - m) - ls);
        if (dx != nullptr) dx[row * C + j] = (expf(xv[k] - m) / s - t) * (1.0f / (float)B);
      }
      acc += wave_sum(l);
    }
  } else
  for (int64_t row = wave; row < B; row += kCeSmallWaves) {
    const float *xr = x + row * C;
    float m = -INFINITY;
    for (int64_t j = lane; j < C; j += 64) m = fmaxf(m, xr[j]);
    m = wave_max(m);
    float s = 0.0f;
    for (int64_t j = lane; j < C; j += 64) s += expf(xr[j] - m);
    s = wave_sum(s);
    const float ls = logf(s);
    float l = 0.0f;
    for (int64_t j = lane; j < C; j += 64) {
      const float t = LABELS ? (j == (int64_t)labels[row] ? 1.0f : 0.0f) : onehot[row * C + j];
      l += -t * ((xr[j] - m) - ls);
      // With dx: the gradient this loss's backward forms when it is the root
      // (g = 1), with softmax_ce_bwd_kernel's arithmetic on the same m and s.
      if (dx != nullptr) dx[row * C + j] = (expf(xr[j] - m) / s - t) * (1.0f / (float)B);
    }
    acc += wave_sum(l);
  }
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
#pragma unroll
    for (int w = 1; w < kCeSmallWaves; ++w) t += red[w];
    out[0] = t / (float)B;
    if (seed != nullptr) seed[0] = 1.0f;
  }
}

// ---------------------------------------------------------------------------
// Row softmax and LayerNorm forward (new ops for the transformer config)
// ---------------------------------------------------------------------------

// x and y may alias (in-place use by attention): a row is read completely
// (max, sum) before it is written, and each lane reads x[j] before y[j].
__global__ void __launch_bounds__(kBlock)
    softmax_rows_kernel(const float *x, float *y, int64_t rows, int64_t cols, float scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + row * cols;
  float m = -INFINITY;
  for (int64_t j = lane; j < cols; j += 64) m = fmaxf(m, xr[j] * scale);
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) s += expf(xr[j] * scale - m);
  s = wave_sum(s);
  const float inv = 1.0f / s;
  for (int64_t j = lane; j < cols; j += 64) y[row * cols + j] = expf(xr[j] * scale - m) * inv;
}

// y = (x - mean) * rstd * gamma + beta; rstd = 1/sqrt(var + eps), biased var.
__global__ void __launch_bounds__(kBlock)
    layernorm_fwd_kernel(const float *__restrict__ x, const float *__restrict__ gamma,
                         const float *__restrict__ beta, float *__restrict__ y,
                         float *__restrict__ mean, float *__restrict__ rstd, int64_t rows,
                         int64_t cols, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *xr = x + row * cols;
  float s = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) s += xr[j];
  const float mu = wave_sum(s) / (float)cols;
  float v = 0.0f;
  for (int64_t j = lane; j < cols; j += 64) {
    const float d = xr[j] - mu;
    v += d * d;
  }
  const float rs = 1.0f / sqrtf(wave_sum(v) / (float)cols + eps);
  for (int64_t j = lane; j < cols; j += 64)
    y[row * cols + j] = (xr[j] - mu) * rs * gamma[j] + beta[j];
  if (lane == 0) {
    if (mean) mean[row] = mu;
    if (rstd) rstd[row] = rs;
  }
}

// The same for rows of at most 64 * 4 * NV columns (cols % 4 == 0, 16-byte
// aligned operands): a lane holds the float4 column groups lane, lane + 64,
// ... in registers, so the row is read once, both statistics come from
// registers and the output leaves as 16-byte stores.  Each element is
// normalised with the scalar kernel's expression ((x - mu) * rs) * gamma + beta.
template <int NV>
__global__ void __launch_bounds__(kBlock)
    layernorm_fwd_vec(const float *__restrict__ x, const float *__restrict__ gamma,
                      const float *__restrict__ beta, float *__restrict__ y,
                      float *__restrict__ mean, float *__restrict__ rstd, int64_t rows, int cols,
                      float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // uniform over the wave
  const float *xr = x + row * cols;
  f4 xv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = 4 * (lane + 64 * i);
    xv[i] = c < cols ? *reinterpret_cast<const f4 *>(xr + c) : f4{0.f, 0.f, 0.f, 0.f};
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += ((xv[i][0] + xv[i][1]) + xv[i][2]) + xv[i][3];
  const float mu = wave_sum(s) / (float)cols;
  float v = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (4 * (lane + 64 * i) < cols)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = xv[i][e] - mu;
        v += d * d;
      }
  const float rs = 1.0f / sqrtf(wave_sum(v) / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = 4 * (lane + 64 * i);
    if (c < cols) {
      const f4 gv = *reinterpret_cast<const f4 *>(gamma + c);
      const f4 bv = *reinterpret_cast<const f4 *>(beta + c);
      f4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (xv[i][e] - mu) * rs * gv[e] + bv[e];
      *reinterpret_cast<f4 *>(y + row * cols + c) = o;
    }
  }
  if (lane == 0) {
    if (mean) mean[row] = mu;
    if (rstd) rstd[row] = rs;
  }
}

template <int OP>
int launch_binary_fwd(numrs_hip_ctx *ctx, const float *a, const int64_t *as, int and_,
                      const float *b, const int64_t *bs, int bnd, float *out) {
  int64_t an = 1, bn = 1;
  for (int d = 0; d < and_; ++d) an *= as[d];
  for (int d = 0; d < bnd; ++d) bn *= bs[d];
  const int nd = and_ > bnd ? and_ : bnd;
  Bcast bc;
  bc.nd = nd;
  int64_t n = 1;
  for (int d = 0; d < nd; ++d) {
    const int da = d - (nd - and_), db = d - (nd - bnd);
    const int64_t ea = da >= 0 ? as[da] : 1, eb = db >= 0 ? bs[db] : 1;
    if (ea != eb && ea != 1 && eb != 1)
      return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "binary op: shapes do not broadcast");
    bc.shape[d] = ea > eb ? ea : eb;
    n *= bc.shape[d];
  }
  if (n == 0) return NUMRS_HIP_OK;
  const unsigned grid = grid_for(n, kBlock);
  const bool flat = (an == n && bn == n) || (bn == 1 && an == n) || (an == 1 && bn == n);
  if (flat) {
    const int a_scalar = an == 1 && n != 1, b_scalar = bn == 1 && n != 1;
    if (numrs_hip::aligned16(a) && numrs_hip::aligned16(b) && numrs_hip::aligned16(out)) {
      const unsigned vgrid = grid_for(n, kBlock * 8);
      if (numrs_hip::vec_mode(true, n) == 2)
        binary_flat_vec<OP, 2><<<vgrid, kBlock, 0, ctx->stream>>>(a, b, out, n, a_scalar, b_scalar);
      else
        binary_flat_vec<OP, 1><<<vgrid, kBlock, 0, ctx->stream>>>(a, b, out, n, a_scalar, b_scalar);
    } else {
      binary_flat_kernel<OP><<<grid, kBlock, 0, ctx->stream>>>(a, b, out, n, a_scalar, b_scalar);
    }
  } else if (an == n && bnd >= 1 && bn == bs[bnd - 1] && bn == bc.shape[nd - 1]) {
    binary_rowbcast_kernel<OP><<<grid, kBlock, 0, ctx->stream>>>(a, b, out, n / bn, bn, 1);
  } else if (bn == n && and_ >= 1 && an == as[and_ - 1] && an == bc.shape[nd - 1]) {
    binary_rowbcast_kernel<OP><<<grid, kBlock, 0, ctx->stream>>>(b, a, out, n / an, an, 0);
  } else {
    int64_t sa = 1, sb = 1;
    for (int d = nd - 1; d >= 0; --d) {
      const int da = d - (nd - and_), db = d - (nd - bnd);
      const int64_t ea = da >= 0 ? as[da] : 1, eb = db >= 0 ? bs[db] : 1;
      bc.sa[d] = ea == 1 ? 0 : sa;
      bc.sb[d] = eb == 1 ? 0 : sb;
      sa *= ea;
      sb *= eb;
    }
    binary_bcast_kernel<OP><<<grid, kBlock, 0, ctx->stream>>>(a, b, out, n, bc);
  }
  return numrs_hip::check_launch(ctx, "binary forward");
}

int full_reduce(numrs_hip_ctx *ctx, int kind, const float *x, const float *t, int64_t n,
                float div, float *out, float *dp = nullptr, float *seed = nullptr) {
  // One block per CU at most: with more, the partials and the reads spread
  // over more HBM pages (1024 blocks measured 15% slower than 256 at 2^24).
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  int64_t blocks = (n + kBlock * 16 - 1) / (kBlock * 16);
  if (blocks < 1) blocks = 1;
  if (blocks > cus) blocks = cus;
  // A single block (n <= 4096) divides and writes `out` itself.
  float *partial = out;
  if (blocks > 1) {
    void *ws = nullptr;
    if (int rc = numrs_hip::workspace(ctx, (size_t)blocks * sizeof(float), &ws)) return rc;
    partial = static_cast<float *>(ws);
  }
  const bool vec = numrs_hip::aligned16(x) && (kind == 0 || numrs_hip::aligned16(t)) &&
                   (dp == nullptr || numrs_hip::aligned16(dp));
  const unsigned grid = (unsigned)blocks;
  numrs_hip::with_vec_mode(numrs_hip::vec_mode(vec, n), [&](auto V) {
    if (kind == 0)
      reduce_pass1<0, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(x, t, n, partial, div,
                                                                            nullptr, seed);
    else
      reduce_pass1<1, decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(x, t, n, partial, div,
                                                                            dp, seed);
  });
  if (int rc = numrs_hip::check_launch(ctx, "reduce_pass1")) return rc;
  if (blocks == 1) return NUMRS_HIP_OK;
  reduce_final<<<1, kBlock, 0, ctx->stream>>>(partial, blocks, div, out, seed);
  return numrs_hip::check_launch(ctx, "reduce_final");
}

}  // namespace

namespace numrs_hip {

bool cross_entropy_preforms(int64_t B) { return B > 0 && B <= kCeSmallRows; }

int mse_loss_impl(numrs_hip_ctx *ctx, const float *p, const float *t, int64_t n, float *out,
                  float *dp, float *seed) {
  NRS_CHECK_CTX(ctx);
  if (n <= 0 || p == nullptr || t == nullptr || out == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_mse_loss: bad arguments");
  return full_reduce(ctx, 1, p, t, n, (float)n, out, dp, seed);
}

int cross_entropy_loss_impl(numrs_hip_ctx *ctx, const float *logits, const float *onehot,
                            const int32_t *labels, int64_t B, int64_t C, float *out, float *dx,
                            float *seed) {
  NRS_CHECK_CTX(ctx);
  if (B <= 0 || C <= 0 || logits == nullptr || out == nullptr ||
      (onehot == nullptr) == (labels == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_cross_entropy_loss: bad arguments");
  if (B <= kCeSmallRows) {
    // rows per wave for the register path (rows of at most 64 classes)
    const int64_t rpw = (B + kCeSmallWaves - 1) / kCeSmallWaves;
    const int tier = C > 64 ? 0 : rpw <= 4 ? 4 : rpw <= 8 ? 8 : rpw <= 16 ? 16 : 32;
#define NRS_CE(L, R)                                                                \
  ce_loss_small_kernel<L, R><<<1, 64 * kCeSmallWaves, 0, ctx->stream>>>(logits, onehot, \
                                                                        labels, B, C, out, dx, seed)
#define NRS_CE_TIER(L)                  \
  switch (tier) {                       \
    case 4: NRS_CE(L, 4); break;        \
    case 8: NRS_CE(L, 8); break;        \
    case 16: NRS_CE(L, 16); break;      \
    case 32: NRS_CE(L, 32); break;      \
    default: NRS_CE(L, 0); break;       \
  }
    if (labels) {
      NRS_CE_TIER(true)
    } else {
      NRS_CE_TIER(false)
    }
#undef NRS_CE_TIER
#undef NRS_CE
    return numrs_hip::check_launch(ctx, "ce_loss_small_kernel");
  }
  if (dx != nullptr || seed != nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID,
                           "cross-entropy: the gradient is formed with the loss only for "
                           "batches of at most %lld rows", (long long)kCeSmallRows);
  // Row losses live in the scratch region; the reduction below uses the workspace.
  float *rows = nullptr;
  if (int rc = numrs_hip::scratch(ctx, (size_t)B * sizeof(float), &rows)) return rc;
  if (labels)
    ce_rows_kernel<true><<<grid_for(B, 4), kBlock, 0, ctx->stream>>>(logits, onehot, labels, rows, B, C);
  else
    ce_rows_kernel<false><<<grid_for(B, 4), kBlock, 0, ctx->stream>>>(logits, onehot, labels, rows, B, C);
  if (int rc = numrs_hip::check_launch(ctx, "ce_rows_kernel")) return rc;
  return full_reduce(ctx, 0, rows, nullptr, B, (float)B, out);
}

}  // namespace numrs_hip

extern "C" {

int numrs_hip_binary_forward(numrs_hip_ctx *ctx, int kind, const float *a, const int64_t *ashape,
                             int and_, const float *b, const int64_t *bshape, int bnd, float *out) {
  NRS_CHECK_CTX(ctx);
  if (and_ < 0 || bnd < 0 || and_ > 8 || bnd > 8 || (and_ && !ashape) || (bnd && !bshape))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_binary_forward: bad shapes");
  if (a == nullptr || b == nullptr || out == nullptr) {
    int64_t an = 1, bn = 1;
    for (int d = 0; d < and_; ++d) an *= ashape[d];
    for (int d = 0; d < bnd; ++d) bn *= bshape[d];
    if (an != 0 && bn != 0)
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_binary_forward: null pointer");
  }
  switch (kind) {
    case NUMRS_HIP_ADD: return launch_binary_fwd<NUMRS_HIP_ADD>(ctx, a, ashape, and_, b, bshape, bnd, out);
    case NUMRS_HIP_SUB: return launch_binary_fwd<NUMRS_HIP_SUB>(ctx, a, ashape, and_, b, bshape, bnd, out);
    case NUMRS_HIP_MUL: return launch_binary_fwd<NUMRS_HIP_MUL>(ctx, a, ashape, and_, b, bshape, bnd, out);
    case NUMRS_HIP_DIV: return launch_binary_fwd<NUMRS_HIP_DIV>(ctx, a, ashape, and_, b, bshape, bnd, out);
    default: return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_binary_forward: kind %d", kind);
  }
}

int numrs_hip_unary_forward(numrs_hip_ctx *ctx, int kind, const float *x, float *y, int64_t n,
                            float param) {
  NRS_CHECK_CTX(ctx);
  if (n < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_unary_forward: n < 0");
  if (n == 0) return NUMRS_HIP_OK;
  if (x == nullptr || y == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_unary_forward: null pointer");
  const bool vec = numrs_hip::aligned16(x) && numrs_hip::aligned16(y);
  const unsigned grid = grid_for(n, vec ? kUnaryPerBlock : kBlock);
  const int vm = numrs_hip::vec_mode(true, n);
#define NRS_UN(K)                                                                              \
  if (!vec)                                                                                   \
    unary_fwd_kernel<K><<<grid, kBlock, 0, ctx->stream>>>(x, y, n, param);                     \
  else if (vm == 2)                                                                           \
    unary_fwd_vec<K, 2><<<grid, kBlock, 0, ctx->stream>>>(x, y, n, param);                     \
  else                                                                                        \
    unary_fwd_vec<K, 1><<<grid, kBlock, 0, ctx->stream>>>(x, y, n, param);                     \
  break
  switch (kind) {
    case NUMRS_HIP_RELU: NRS_UN(NUMRS_HIP_RELU);
    case NUMRS_HIP_SIGMOID: NRS_UN(NUMRS_HIP_SIGMOID);
    case NUMRS_HIP_TANH: NRS_UN(NUMRS_HIP_TANH);
    case NUMRS_HIP_EXP: NRS_UN(NUMRS_HIP_EXP);
    case NUMRS_HIP_LOG: NRS_UN(NUMRS_HIP_LOG);
    case NUMRS_HIP_GELU: NRS_UN(NUMRS_HIP_GELU);
    case NUMRS_HIP_SQRT: NRS_UN(NUMRS_HIP_SQRT);
    case NUMRS_HIP_SIN: NRS_UN(NUMRS_HIP_SIN);
    case NUMRS_HIP_COS: NRS_UN(NUMRS_HIP_COS);
    case NUMRS_HIP_TAN: NRS_UN(NUMRS_HIP_TAN);
    case NUMRS_HIP_POW: NRS_UN(NUMRS_HIP_POW);
    default: return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_unary_forward: kind %d", kind);
  }
#undef NRS_UN
  return numrs_hip::check_launch(ctx, "unary_fwd_kernel");
}

int numrs_hip_transpose(numrs_hip_ctx *ctx, const float *x, float *y, int64_t rows, int64_t cols) {
  NRS_CHECK_CTX(ctx);
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "transpose: negative size");
  if (rows == 0 || cols == 0) return NUMRS_HIP_OK;
  if (x == nullptr || y == nullptr) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "transpose: null pointer");
  if ((rows + 31) / 32 > 65535) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "transpose: too many rows");
  if ((rows & 3) == 0 && (cols & 3) == 0 && numrs_hip::aligned16(x) && numrs_hip::aligned16(y) &&
      rows >= 64 && cols >= 256) {
    dim3 grid((unsigned)((cols + 255) / 256), (unsigned)((rows + 63) / 64));
    numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, rows * cols), [&](auto V) {
      transpose_reg_kernel<decltype(V)::value><<<grid, kBlock, 0, ctx->stream>>>(x, y, rows, cols);
    });
    return numrs_hip::check_launch(ctx, "transpose_reg_kernel");
  }
  if ((rows & 3) == 0 && (cols & 3) == 0 && numrs_hip::aligned16(x) && numrs_hip::aligned16(y)) {
    // 128 x 128 tiles when both sides hold one: each tile row and column
    // then moves as 512-byte runs, against 256 with 64 x 64 tiles.
    const bool big = rows >= 128 && cols >= 128;
    const int ts = big ? 128 : 64;
    dim3 grid((unsigned)((cols + ts - 1) / ts), (unsigned)((rows + ts - 1) / ts));
    numrs_hip::with_vec_mode(numrs_hip::vec_mode(true, rows * cols), [&](auto V) {
      if (big)
        transpose_tile_kernel<decltype(V)::value, 128><<<grid, kBlock, 0, ctx->stream>>>(x, y,
                                                                                      rows, cols);
      else
        transpose_tile_kernel<decltype(V)::value, 64><<<grid, kBlock, 0, ctx->stream>>>(x, y,
                                                                                     rows, cols);
    });
    return numrs_hip::check_launch(ctx, "transpose_tile_kernel");
  }
  dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
  transpose_kernel<<<grid, kBlock, 0, ctx->stream>>>(x, y, rows, cols);
  return numrs_hip::check_launch(ctx, "transpose_kernel");
}

int numrs_hip_sum(numrs_hip_ctx *ctx, const float *x, int64_t n, int mean, float *out) {
  NRS_CHECK_CTX(ctx);
  if (n < 0 || out == nullptr || (n > 0 && x == nullptr))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_sum: bad arguments");
  if (n == 0) return numrs_hip_fill(ctx, out, 1, mean ? NAN : 0.0f);
  return full_reduce(ctx, 0, x, nullptr, n, mean ? (float)n : 1.0f, out);
}

int numrs_hip_mse_loss(numrs_hip_ctx *ctx, const float *p, const float *t, int64_t n, float *out) {
  return numrs_hip::mse_loss_impl(ctx, p, t, n, out, nullptr, nullptr);
}

int numrs_hip_cross_entropy_loss(numrs_hip_ctx *ctx, const float *logits, const float *onehot,
                                 const int32_t *labels, int64_t B, int64_t C, float *out) {
  return numrs_hip::cross_entropy_loss_impl(ctx, logits, onehot, labels, B, C, out, nullptr,
                                            nullptr);
}

int numrs_hip_softmax_forward(numrs_hip_ctx *ctx, const float *x, float *y, int64_t rows,
                              int64_t cols, float scale) {
  NRS_CHECK_CTX(ctx);
  if (rows < 0 || cols < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "softmax: negative size");
  if (rows == 0 || cols == 0) return NUMRS_HIP_OK;
  if (x == nullptr || y == nullptr) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "softmax: null pointer");
  softmax_rows_kernel<<<grid_for(rows, 4), kBlock, 0, ctx->stream>>>(x, y, rows, cols, scale);
  return numrs_hip::check_launch(ctx, "softmax_rows_kernel");
}

int numrs_hip_layernorm_forward(numrs_hip_ctx *ctx, const float *x, const float *gamma,
                                const float *beta, float *y, float *mean, float *rstd,
                                int64_t rows, int64_t cols, float eps) {
  NRS_CHECK_CTX(ctx);
  if (rows < 0 || cols <= 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "layernorm: bad size");
  if (rows == 0) return NUMRS_HIP_OK;
  if (x == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "layernorm: null pointer");
  const unsigned grid = grid_for(rows, 4);
  const bool vec = cols % 4 == 0 && cols <= 2048 && numrs_hip::aligned16(x) &&
                   numrs_hip::aligned16(gamma) && numrs_hip::aligned16(beta) &&
                   numrs_hip::aligned16(y);
  if (vec) {
    const int c = (int)cols;
    if (cols <= 256)
      layernorm_fwd_vec<1><<<grid, kBlock, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, rows, c, eps);
    else if (cols <= 512)
      layernorm_fwd_vec<2><<<grid, kBlock, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, rows, c, eps);
    else if (cols <= 1024)
      layernorm_fwd_vec<4><<<grid, kBlock, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, rows, c, eps);
    else
      layernorm_fwd_vec<8><<<grid, kBlock, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, rows, c, eps);
    return numrs_hip::check_launch(ctx, "layernorm_fwd_vec");
  }
  layernorm_fwd_kernel<<<grid, kBlock, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, rows, cols,
                                                         eps);
  return numrs_hip::check_launch(ctx, "layernorm_fwd_kernel");
}

}  // extern "C"
