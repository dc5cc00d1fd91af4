// LSTM layer forward and BPTT backward (no reference op: numrs has no
// recurrent layer).  Layouts, all row-major fp32:
//   x      [B, T, I]        input sequence
//   W_ih   [4H, I], W_hh [4H, H], b [4H]   gate order i, f, g, o
//   h_seq, c_seq [B, T, H]  hidden / cell states of every step
//   acts   [B, T, 4H]       gate activations i, f, g, o (after the sigmoid /
//                           tanh), saved by the forward for the backward
//   dG     [B, T, 4H]       gate pre-activation gradients (backward temp)
//
// Forward:  G = x W_ih^T + b for all steps (one MFMA product), then per step
//   t one fused kernel: pre = G_t + h_{t-1} W_hh^T, i,f,o = sigmoid, g = tanh,
//   c_t = f c_{t-1} + i g, h_t = o tanh(c_t).
// Backward: per step t (T-1 .. 0) one fused kernel: dh = dh_out_t +
//   dG_{t+1} W_hh, dc = dh o (1 - tanh^2 c_t) + dc_{t+1} f_{t+1}, and the four
//   gate-gradient formulas into dG_t; then the weight gradients batched over
//   all steps as single products: dW_ih = dG^T x, dW_hh = dG^T H_prev
//   (H_prev = h shifted one step), db = column sum of dG, dx = dG W_ih.
//
// Step kernels: one wave per (64 hidden units, kBatchPerLane batch rows).
// Lane j owns hidden unit j of those rows for every step, so the cell state
// it carries (c, dc) is only ever touched by that lane.  The recurrent
// product reads the weight row segment with coalesced vector loads and the
// h / dG value of the row, identical across the wave, once per k.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBatchPerLane = 2;

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// Forward step t.  whhT is W_hh^T [H, 4H]; G holds x W_ih^T + b on entry and
// the activations on exit (in place: each lane reads its four values first).
__global__ void __launch_bounds__(64)
    lstm_fwd_step(float *G, const float *__restrict__ whhT, const float *__restrict__ h0,
                  const float *__restrict__ c0, float *__restrict__ h_seq,
                  float *__restrict__ c_seq, int B, int T, int H, int t) {
  const int jblocks = (H + 63) / 64;
  const int jb = blockIdx.x % jblocks, bp = blockIdx.x / jblocks;
  const int j = jb * 64 + threadIdx.x;
  const int b0 = bp * kBatchPerLane;
  const int H4 = 4 * H;
  float acc[kBatchPerLane][4];
#pragma unroll
  for (int u = 0; u < kBatchPerLane; ++u)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[u][g] = 0.0f;
  const bool have_prev = t > 0 || h0 != nullptr;
  if (have_prev && j < H) {
    const float *hp[kBatchPerLane];
#pragma unroll
    for (int u = 0; u < kBatchPerLane; ++u) {
      const int b = min(b0 + u, B - 1);
      hp[u] = t > 0 ? h_seq + ((int64_t)b * T + t - 1) * H : h0 + (int64_t)b * H;
    }
    for (int k = 0; k < H; ++k) {
      const float *wrow = whhT + (int64_t)k * H4 + j;
      const float w0 = wrow[0], w1 = wrow[H], w2 = wrow[2 * H], w3 = wrow[3 * H];
#pragma unroll
      for (int u = 0; u < kBatchPerLane; ++u) {
        const float hv = hp[u][k];
        acc[u][0] += hv * w0;
        acc[u][1] += hv * w1;
        acc[u][2] += hv * w2;
        acc[u][3] += hv * w3;
      }
    }
  }
  if (j >= H) return;
#pragma unroll
  for (int u = 0; u < kBatchPerLane; ++u) {
    const int b = b0 + u;
    if (b >= B) break;
    const int64_t gb = ((int64_t)b * T + t) * H4;
    const float i = sigm(G[gb + j] + acc[u][0]);
    const float f = sigm(G[gb + H + j] + acc[u][1]);
    const float g = tanhf(G[gb + 2 * H + j] + acc[u][2]);
    const float o = sigm(G[gb + 3 * H + j] + acc[u][3]);
    const float cp = t > 0 ? c_seq[((int64_t)b * T + t - 1) * H + j]
                           : (c0 != nullptr ? c0[(int64_t)b * H + j] : 0.0f);
    const float c = f * cp + i * g;
    const float h = o * tanhf(c);
    G[gb + j] = i;
    G[gb + H + j] = f;
    G[gb + 2 * H + j] = g;
    G[gb + 3 * H + j] = o;
    c_seq[((int64_t)b * T + t) * H + j] = c;
    h_seq[((int64_t)b * T + t) * H + j] = h;
  }
}

// Backward step t.  whh is W_hh [4H, H]; dG rows t+1 are complete (previous
// launch); dc holds dc_{t+1} * f_{t+1} on entry and dc_t * f_t on exit.
__global__ void __launch_bounds__(64)
    lstm_bwd_step(float *__restrict__ dG, const float *__restrict__ whh,
                  const float *__restrict__ acts, const float *__restrict__ c_seq,
                  const float *__restrict__ c0, const float *__restrict__ dh_out,
                  float *__restrict__ dc, int B, int T, int H, int t) {
  const int jblocks = (H + 63) / 64;
  const int jb = blockIdx.x % jblocks, bp = blockIdx.x / jblocks;
  const int j = jb * 64 + threadIdx.x;
  const int b0 = bp * kBatchPerLane;
  const int H4 = 4 * H;
  float rec[kBatchPerLane];
#pragma unroll
  for (int u = 0; u < kBatchPerLane; ++u) rec[u] = 0.0f;
  if (t + 1 < T && j < H) {
    const float *dn[kBatchPerLane];
#pragma unroll
    for (int u = 0; u < kBatchPerLane; ++u) {
      const int b = min(b0 + u, B - 1);
      dn[u] = dG + ((int64_t)b * T + t + 1) * H4;
    }
    for (int n = 0; n < H4; ++n) {
      const float w = whh[(int64_t)n * H + j];
#pragma unroll
      for (int u = 0; u < kBatchPerLane; ++u) rec[u] += dn[u][n] * w;
    }
  }
  if (j >= H) return;
#pragma unroll
  for (int u = 0; u < kBatchPerLane; ++u) {
    const int b = b0 + u;
    if (b >= B) break;
    const int64_t row = (int64_t)b * T + t;
    const int64_t gb = row * H4;
    const float dh = (dh_out != nullptr ? dh_out[row * H + j] : 0.0f) + rec[u];
    const float i = acts[gb + j], f = acts[gb + H + j], g = acts[gb + 2 * H + j],
                o = acts[gb + 3 * H + j];
    const float c = c_seq[row * H + j];
    const float tc = tanhf(c);
    const float cp = t > 0 ? c_seq[(row - 1) * H + j]
                           : (c0 != nullptr ? c0[(int64_t)b * H + j] : 0.0f);
    const float dcn = t + 1 < T ? dc[(int64_t)b * H + j] : 0.0f;
    const float dct = dh * o * (1.0f - tc * tc) + dcn;
    dG[gb + j] = (dct * g) * i * (1.0f - i);
    dG[gb + H + j] = (dct * cp) * f * (1.0f - f);
    dG[gb + 2 * H + j] = (dct * i) * (1.0f - g * g);
    dG[gb + 3 * H + j] = (dh * tc) * o * (1.0f - o);
    dc[(int64_t)b * H + j] = dct * f;
  }
}

// H_prev[b, t] = h_seq[b, t-1] (t > 0), h0[b] or 0 (t = 0).
__global__ void __launch_bounds__(256)
    shift_hidden(const float *__restrict__ h_seq, const float *__restrict__ h0,
                 float *__restrict__ out, int B, int T, int H) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = (int64_t)B * T * H;
  if (i >= n) return;
  const int64_t j = i % H, row = i / H, t = row % T, b = row / T;
  out[i] = t > 0 ? h_seq[i - H] : (h0 != nullptr ? h0[b * H + j] : 0.0f);
}

unsigned step_grid(int B, int H) {
  return (unsigned)(((H + 63) / 64) * ((B + kBatchPerLane - 1) / kBatchPerLane));
}

int check(numrs_hip_ctx *ctx, int64_t B, int64_t T, int64_t I, int64_t H) {
  if (B <= 0 || T <= 0 || I <= 0 || H <= 0 || B > (1 << 20) || T > (1 << 20) || H > (1 << 16))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "lstm: bad sizes B=%lld T=%lld I=%lld H=%lld",
                           (long long)B, (long long)T, (long long)I, (long long)H);
  return NUMRS_HIP_OK;
}

// Temporary device block from the context's block cache (stream-ordered:
// released blocks are only reused by later work on the same stream).
struct TempBlock {
  numrs_hip_ctx *ctx;
  void *p = nullptr;
  size_t bytes = 0;
  explicit TempBlock(numrs_hip_ctx *c) : ctx(c) {}
  int alloc(size_t b) {
    bytes = b;
    return numrs_hip::block_alloc(ctx, b, &p);
  }
  float *f() const { return static_cast<float *>(p); }
  ~TempBlock() { numrs_hip::block_free(ctx, p, bytes); }
};

// y[b, :] = x[b, t, :] for x [B, T, D] (the last-step head input), and its
// backward dx[b, t, :] (+)= g[b, :] with zeros elsewhere when not accumulating.
__global__ void __launch_bounds__(256)
    time_slice_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t B, int64_t T,
                      int64_t D, int64_t t, int backward, int acc) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (!backward) {
    if (i >= B * D) return;
    const int64_t b = i / D, d = i % D;
    y[i] = x[(b * T + t) * D + d];
  } else {
    // x is g [B, D]; y is dx [B, T, D]
    if (i >= B * T * D) return;
    const int64_t d = i % D, row = i / D, tt = row % T, b = row / T;
    const float v = tt == t ? x[b * D + d] : 0.0f;
    if (acc) {
      if (tt == t) y[i] += v;
    } else {
      y[i] = v;
    }
  }
}

}  // namespace

extern "C" {

int numrs_hip_lstm_forward(numrs_hip_ctx *ctx, const float *x, const float *w_ih,
                           const float *w_hh, const float *b, const float *h0, const float *c0,
                           float *h_seq, float *c_seq, float *acts, int64_t B, int64_t T,
                           int64_t I, int64_t H) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, T, I, H)) return rc;
  if (!x || !w_ih || !w_hh || !h_seq || !c_seq || !acts)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "lstm_forward: null pointer");
  // acts <- x W_ih^T + b for every (b, t) row
  if (int rc = numrs_hip_linear_forward(ctx, x, w_ih, b, acts, B * T, I, 4 * H)) return rc;
  TempBlock whhT(ctx);
  if (int rc = whhT.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
  if (int rc = numrs_hip_transpose(ctx, w_hh, whhT.f(), 4 * H, H)) return rc;
  const unsigned grid = step_grid((int)B, (int)H);
  for (int64_t t = 0; t < T; ++t) {
    lstm_fwd_step<<<grid, 64, 0, ctx->stream>>>(acts, whhT.f(), h0, c0, h_seq, c_seq, (int)B,
                                                (int)T, (int)H, (int)t);
    if (int rc = numrs_hip::check_launch(ctx, "lstm_fwd_step")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_lstm_backward(numrs_hip_ctx *ctx, const float *x, const float *w_ih,
                            const float *w_hh, const float *h0, const float *c0,
                            const float *h_seq, const float *c_seq, const float *acts,
                            const float *dh_seq, float *dx, float *dw_ih, float *dw_hh, float *db,
                            int64_t B, int64_t T, int64_t I, int64_t H, int acc_dx, int acc_dw_ih,
                            int acc_dw_hh, int acc_db) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, T, I, H)) return rc;
  if (!x || !w_ih || !w_hh || !h_seq || !c_seq || !acts)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "lstm_backward: null input");
  const int64_t rows = B * T, H4 = 4 * H;
  TempBlock dG(ctx), dc(ctx);
  if (int rc = dG.alloc((size_t)(rows * H4) * sizeof(float))) return rc;
  if (int rc = dc.alloc((size_t)(B * H) * sizeof(float))) return rc;
  const unsigned grid = step_grid((int)B, (int)H);
  for (int64_t t = T - 1; t >= 0; --t) {
    lstm_bwd_step<<<grid, 64, 0, ctx->stream>>>(dG.f(), w_hh, acts, c_seq, c0, dh_seq, dc.f(),
                                                (int)B, (int)T, (int)H, (int)t);
    if (int rc = numrs_hip::check_launch(ctx, "lstm_bwd_step")) return rc;
  }
  // Weight gradients over all steps at once (batched over time).
  if (dw_ih)  // dW_ih[4H, I] = dG^T x
    if (int rc = numrs_hip_gemm(ctx, dG.f(), H4, x, I, dw_ih, I, H4, rows, I, 1, 0, 1.0f,
                                acc_dw_ih, 1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  if (dw_hh) {  // dW_hh[4H, H] = dG^T H_prev
    TempBlock hp(ctx);
    if (int rc = hp.alloc((size_t)(rows * H) * sizeof(float))) return rc;
    shift_hidden<<<grid_for(rows * H, 256), 256, 0, ctx->stream>>>(h_seq, h0, hp.f(), (int)B,
                                                                   (int)T, (int)H);
    if (int rc = numrs_hip::check_launch(ctx, "shift_hidden")) return rc;
    if (int rc = numrs_hip_gemm(ctx, dG.f(), H4, hp.f(), H, dw_hh, H, H4, rows, H, 1, 0, 1.0f,
                                acc_dw_hh, 1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  }
  if (db) {  // db[4H] = column sum of dG
    const int64_t gs[2] = {rows, H4};
    const int64_t bs = H4;
    if (int rc = numrs_hip_sum_to_shape(ctx, dG.f(), gs, 2, db, &bs, 1,
                                        NUMRS_HIP_UNBROADCAST_CORRECT, acc_db))
      return rc;
  }
  if (dx)  // dx[B*T, I] = dG W_ih
    if (int rc = numrs_hip_gemm(ctx, dG.f(), H4, w_ih, I, dx, I, rows, H4, I, 0, 0, 1.0f, acc_dx,
                                1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  return NUMRS_HIP_OK;
}

int numrs_hip_time_slice(numrs_hip_ctx *ctx, const float *x, float *y, int64_t B, int64_t T,
                         int64_t D, int64_t t, int backward, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (B < 0 || T <= 0 || D < 0 || t < 0 || t >= T || !x || !y)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "time_slice: bad arguments");
  const int64_t n = backward ? B * T * D : B * D;
  if (n == 0) return NUMRS_HIP_OK;
  time_slice_kernel<<<grid_for(n, 256), 256, 0, ctx->stream>>>(x, y, B, T, D, t, backward,
                                                                accumulate);
  return numrs_hip::check_launch(ctx, "time_slice_kernel");
}

}  // extern "C"
