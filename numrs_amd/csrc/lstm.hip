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
// Step kernels: one 1024-thread block per (64 hidden units, kRows batch
// rows).  The step is latency-bound (a few MiB of L2-resident reads), so the
// recurrent reduction is cut into 16 slices, one per wave; the block's h (or
// dG) rows are staged in LDS once, W_hh is packed so a lane's four gate
// weights for one reduction index are one 16-byte load, and each lane issues
// the weight loads of kChunk indices before their FMAs, carrying all kRows
// rows of its hidden unit.  The slices meet in LDS in a fixed order, and wave
// u < kRows finishes row b0 + u, so the cell state of (b, j) (c, dc) is always
// touched by the same thread.
#include <cmath>

#include "common.h"

namespace {

constexpr int kRows = 4;    // batch rows carried by each lane
constexpr int kWaves = 16;  // the recurrent reduction is split across the block's waves
constexpr int kThreads = 64 * kWaves;
// reduction indices whose weight loads are issued together (sized to stay
// within the 128 VGPRs a 1024-thread block allows)
template <bool STAGE, bool FWD>
constexpr int chunk() { return STAGE ? (FWD ? 16 : 12) : (FWD ? 6 : 3); }
constexpr int kFwdStageH = 2048;  // largest H whose h rows the forward stages in LDS
constexpr int kBwdStageH = 1024;  // largest H whose dG rows the backward stages in LDS

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// Packed recurrent weights: P[(k * H + j) * 4 + g] = in[g * sg + k * sk + j],
// so the four gate weights a lane needs for reduction index k are one 16-byte
// load.  Forward: in = W_hh^T [H, 4H] (sg = H, sk = 4H), P[k, j, g] =
// W_hh[gH + j, k].  Backward: in = W_hh [4H, H] (sg = H*H, sk = H), P[k, j, g]
// = W_hh[gH + k, j].
__global__ void __launch_bounds__(256)
    pack_gates(const float *__restrict__ in, float *__restrict__ out, int H, int64_t sg,
               int64_t sk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (g, k, j), j fastest
  const int64_t n = (int64_t)4 * H * H;
  if (i >= n) return;
  const int64_t j = i % H, k = (i / H) % H, g = i / ((int64_t)H * H);
  out[(k * H + j) * 4 + g] = in[g * sg + k * sk + j];
}

// Forward step t.  wp is the forward packing of W_hh; G holds x W_ih^T + b on
// entry and the activations on exit (in place: each thread reads its four
// values first).  Block = 16 waves for 64 hidden units x kRows batch rows:
// wave w forms the partial products over k in its sixteenth of [0, H), LDS
// holds the partials, which are added in wave order, and the first kRows
// waves finish the cells.  The epilogue's inputs, the first weight chunk and
// the staging of the block's h_{t-1} rows in LDS (STAGE) are all issued
// before the first wait, so their memory latencies overlap.
template <bool STAGE>
__global__ void __launch_bounds__(kThreads)
    lstm_fwd_step(float *G, const float4 *__restrict__ wp, const float *__restrict__ h0,
                  const float *__restrict__ c0, float *__restrict__ h_seq,
                  float *__restrict__ c_seq, int B, int T, int H, int t) {
  __shared__ float part[kWaves][kRows * 4][64];
  __shared__ float hs[STAGE ? kRows * kFwdStageH : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int jblocks = (H + 63) / 64;
  const int jb = blockIdx.x % jblocks, bp = blockIdx.x / jblocks;
  const int j = jb * 64 + lane;
  const int b0 = bp * kRows;
  const int H4 = 4 * H;
  const bool has_h = t > 0 || h0 != nullptr;

  // epilogue inputs of cell (b0 + wave, j)
  const int be = b0 + wave;
  const bool epi = wave < kRows && be < B && j < H;
  const int64_t gb = ((int64_t)be * T + t) * H4;
  float gin[4] = {0.0f, 0.0f, 0.0f, 0.0f}, cp = 0.0f;
  if (epi) {
#pragma unroll
    for (int g = 0; g < 4; ++g) gin[g] = G[gb + g * H + j];
    cp = t > 0 ? c_seq[((int64_t)be * T + t - 1) * H + j]
               : (c0 != nullptr ? c0[(int64_t)be * H + j] : 0.0f);
  }

  const float *hp[kRows];
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    const int b = min(b0 + u, B - 1);
    hp[u] = t > 0 ? h_seq + ((int64_t)b * T + t - 1) * H : h0 + (int64_t)b * H;
  }
  const bool work = has_h && j < H;
  const int kc = (H + kWaves - 1) / kWaves;
  const int k0 = wave * kc, k1 = min(H, k0 + kc);
  constexpr int kChunk = chunk<STAGE, true>();
  float4 w[kChunk];
  int k = k0;
  bool full = work && k + kChunk <= k1;
  if (full) {
#pragma unroll
    for (int s = 0; s < kChunk; ++s) w[s] = wp[(int64_t)(k + s) * H + j];
  }
  if (STAGE && has_h) {
    for (int i = threadIdx.x; i < kRows * H; i += kThreads) {
      const int u = i / H;
      hs[i] = hp[u][i - u * H];
    }
    __syncthreads();
  }
  float acc[kRows][4];
#pragma unroll
  for (int u = 0; u < kRows; ++u)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[u][g] = 0.0f;
  if (work) {
    auto step = [&](int kk, const float4 &wv) {
#pragma unroll
      for (int u = 0; u < kRows; ++u) {
        const float hv = STAGE ? hs[u * H + kk] : hp[u][kk];
        acc[u][0] += hv * wv.x;
        acc[u][1] += hv * wv.y;
        acc[u][2] += hv * wv.z;
        acc[u][3] += hv * wv.w;
      }
    };
    if (full) {  // the prefetched chunk
#pragma unroll
      for (int s = 0; s < kChunk; ++s) step(k + s, w[s]);
      k += kChunk;
    }
    for (; k + kChunk <= k1; k += kChunk) {
      float4 wn[kChunk];
#pragma unroll
      for (int s = 0; s < kChunk; ++s) wn[s] = wp[(int64_t)(k + s) * H + j];
#pragma unroll
      for (int s = 0; s < kChunk; ++s) step(k + s, wn[s]);
    }
    for (; k < k1; ++k) step(k, wp[(int64_t)k * H + j]);
  }
#pragma unroll
  for (int u = 0; u < kRows; ++u)
#pragma unroll
    for (int g = 0; g < 4; ++g) part[wave][u * 4 + g][lane] = acc[u][g];
  __syncthreads();
  // thread (wave, lane) adds the kWaves partials of column `wave` (row u =
  // wave / 4, gate wave % 4) in wave order; it alone reads and rewrites it
  {
    float sum = part[0][wave][lane];
#pragma unroll
    for (int v = 1; v < kWaves; ++v) sum += part[v][wave][lane];
    part[0][wave][lane] = sum;
  }
  __syncthreads();
  if (!epi) return;
  const int u = wave;
  const float i = sigm(gin[0] + part[0][u * 4 + 0][lane]);
  const float f = sigm(gin[1] + part[0][u * 4 + 1][lane]);
  const float g = tanhf(gin[2] + part[0][u * 4 + 2][lane]);
  const float o = sigm(gin[3] + part[0][u * 4 + 3][lane]);
  const float c = f * cp + i * g;
  const float h = o * tanhf(c);
  G[gb + j] = i;
  G[gb + H + j] = f;
  G[gb + 2 * H + j] = g;
  G[gb + 3 * H + j] = o;
  c_seq[((int64_t)be * T + t) * H + j] = c;
  h_seq[((int64_t)be * T + t) * H + j] = h;
}

// Backward step t.  wp is the backward packing of W_hh; dG rows t+1 are
// complete (previous launch); dc holds dc_{t+1} * f_{t+1} on entry and
// dc_t * f_t on exit, and each (b, j) is always handled by the same thread.
// The block stages its dG_{t+1} rows in LDS as [u][k][g] (STAGE), and wave w
// reduces over k in its sixteenth of [0, H), all four gates per k:
// dh[b, j] += sum_g dG[b, gH + k] W_hh[gH + k, j].  As in the forward, the
// epilogue's inputs, the first weight chunk and the staging are issued
// before the first wait.
template <bool STAGE>
__global__ void __launch_bounds__(kThreads)
    lstm_bwd_step(float *__restrict__ dG, const float4 *__restrict__ wp,
                  const float *__restrict__ acts, const float *__restrict__ c_seq,
                  const float *__restrict__ c0, const float *__restrict__ dh_out,
                  float *__restrict__ dc, int B, int T, int H, int t) {
  __shared__ float part[kWaves][kRows][64];
  __shared__ float4 ds[STAGE ? kRows * kBwdStageH : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int jblocks = (H + 63) / 64;
  const int jb = blockIdx.x % jblocks, bp = blockIdx.x / jblocks;
  const int j = jb * 64 + lane;
  const int b0 = bp * kRows;
  const int H4 = 4 * H;
  const bool has_next = t + 1 < T;

  // epilogue inputs of cell (b0 + wave, j)
  const int be = b0 + wave;
  const bool epi = wave < kRows && be < B && j < H;
  const int64_t row = (int64_t)be * T + t;
  const int64_t gb = row * H4;
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, c = 0.0f, cp = 0.0f, dho = 0.0f, dcn = 0.0f;
  if (epi) {
#pragma unroll
    for (int g = 0; g < 4; ++g) a[g] = acts[gb + g * H + j];
    c = c_seq[row * H + j];
    cp = t > 0 ? c_seq[(row - 1) * H + j] : (c0 != nullptr ? c0[(int64_t)be * H + j] : 0.0f);
    if (dh_out != nullptr) dho = dh_out[row * H + j];
    if (has_next) dcn = dc[(int64_t)be * H + j];
  }

  const float *dn[kRows];
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    const int b = min(b0 + u, B - 1);
    dn[u] = dG + ((int64_t)b * T + t + 1) * H4;
  }
  const bool work = has_next && j < H;
  const int kc = (H + kWaves - 1) / kWaves;
  const int k0 = wave * kc, k1 = min(H, k0 + kc);
  constexpr int kChunk = chunk<STAGE, false>();
  float4 w[kChunk];
  int k = k0;
  bool full = work && k + kChunk <= k1;
  if (full) {
#pragma unroll
    for (int s = 0; s < kChunk; ++s) w[s] = wp[(int64_t)(k + s) * H + j];
  }
  if (STAGE && has_next) {
    float *dsf = reinterpret_cast<float *>(ds);
    for (int i = threadIdx.x; i < kRows * H4; i += kThreads) {
      const int u = i / H4, n = i - u * H4;
      const int g = n / H, kk = n - g * H;
      dsf[(u * H + kk) * 4 + g] = dn[u][n];
    }
    __syncthreads();
  }
  float rec[kRows];
#pragma unroll
  for (int u = 0; u < kRows; ++u) rec[u] = 0.0f;
  if (work) {
    auto step = [&](int kk, const float4 &wv) {
#pragma unroll
      for (int u = 0; u < kRows; ++u) {
        const float4 d = STAGE ? ds[u * H + kk]
                               : make_float4(dn[u][kk], dn[u][H + kk], dn[u][2 * H + kk],
                                             dn[u][3 * H + kk]);
        rec[u] += d.x * wv.x;
        rec[u] += d.y * wv.y;
        rec[u] += d.z * wv.z;
        rec[u] += d.w * wv.w;
      }
    };
    if (full) {  // the prefetched chunk
#pragma unroll
      for (int s = 0; s < kChunk; ++s) step(k + s, w[s]);
      k += kChunk;
    }
    for (; k + kChunk <= k1; k += kChunk) {
      float4 wn[kChunk];
#pragma unroll
      for (int s = 0; s < kChunk; ++s) wn[s] = wp[(int64_t)(k + s) * H + j];
#pragma unroll
      for (int s = 0; s < kChunk; ++s) step(k + s, wn[s]);
    }
    for (; k < k1; ++k) step(k, wp[(int64_t)k * H + j]);
  }
#pragma unroll
  for (int u = 0; u < kRows; ++u) part[wave][u][lane] = rec[u];
  __syncthreads();
  if (!epi) return;
  const int u = wave;
  float r = part[0][u][lane];
#pragma unroll
  for (int v = 1; v < kWaves; ++v) r += part[v][u][lane];
  const float i = a[0], f = a[1], g = a[2], o = a[3];
  const float dh = dho + r;
  const float tc = tanhf(c);
  const float dct = dh * o * (1.0f - tc * tc) + dcn;
  dG[gb + j] = (dct * g) * i * (1.0f - i);
  dG[gb + H + j] = (dct * cp) * f * (1.0f - f);
  dG[gb + 2 * H + j] = (dct * i) * (1.0f - g * g);
  dG[gb + 3 * H + j] = (dh * tc) * o * (1.0f - o);
  dc[(int64_t)be * H + j] = dct * f;
}

static_assert(kRows * 4 == kWaves, "one LDS column of partials per wave");

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
  return (unsigned)(((H + 63) / 64) * ((B + kRows - 1) / kRows));
}

int check(numrs_hip_ctx *ctx, int64_t B, int64_t T, int64_t I, int64_t H) {
  if (B <= 0 || T <= 0 || I <= 0 || H <= 0 || B > (1 << 20) || T > (1 << 20) || H > (1 << 16))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "lstm: bad sizes B=%lld T=%lld I=%lld H=%lld",
                           (long long)B, (long long)T, (long long)I, (long long)H);
  return NUMRS_HIP_OK;
}

using numrs_hip::TempBlock;

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
  TempBlock whhT(ctx), wp(ctx);
  if (int rc = whhT.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
  if (int rc = wp.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
  if (int rc = numrs_hip_transpose(ctx, w_hh, whhT.f(), 4 * H, H)) return rc;
  pack_gates<<<grid_for(4 * H * H, 256), 256, 0, ctx->stream>>>(whhT.f(), wp.f(), (int)H, H,
                                                                4 * H);
  if (int rc = numrs_hip::check_launch(ctx, "pack_gates")) return rc;
  const unsigned grid = step_grid((int)B, (int)H);
  const float4 *wp4 = reinterpret_cast<const float4 *>(wp.p);
  for (int64_t t = 0; t < T; ++t) {
    if (H <= kFwdStageH)
      lstm_fwd_step<true><<<grid, kThreads, 0, ctx->stream>>>(acts, wp4, h0, c0, h_seq, c_seq,
                                                              (int)B, (int)T, (int)H, (int)t);
    else
      lstm_fwd_step<false><<<grid, kThreads, 0, ctx->stream>>>(acts, wp4, h0, c0, h_seq, c_seq,
                                                               (int)B, (int)T, (int)H, (int)t);
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
  TempBlock wp(ctx);
  if (int rc = wp.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
  pack_gates<<<grid_for(4 * H * H, 256), 256, 0, ctx->stream>>>(w_hh, wp.f(), (int)H, H * H, H);
  if (int rc = numrs_hip::check_launch(ctx, "pack_gates")) return rc;
  const float4 *wp4 = reinterpret_cast<const float4 *>(wp.p);
  const unsigned grid = step_grid((int)B, (int)H);
  for (int64_t t = T - 1; t >= 0; --t) {
    if (H <= kBwdStageH)
      lstm_bwd_step<true><<<grid, kThreads, 0, ctx->stream>>>(
          dG.f(), wp4, acts, c_seq, c0, dh_seq, dc.f(), (int)B, (int)T, (int)H, (int)t);
    else
      lstm_bwd_step<false><<<grid, kThreads, 0, ctx->stream>>>(
          dG.f(), wp4, acts, c_seq, c0, dh_seq, dc.f(), (int)B, (int)T, (int)H, (int)t);
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
