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

// ---------------------------------------------------------------------------
// Tiled step kernels for H % 64 == 0 (the C5 shape): 256-thread workgroups,
// 256 of them at B = 64, H = 256, so one step spans every CU; both read W_hh
// in its stored [4H, H] layout (no repacking launch).
// ---------------------------------------------------------------------------

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kFRows = 16;   // forward: batch rows per workgroup (the MFMA's M)
constexpr int kFUnits = 4;   // forward: hidden units per workgroup (x 4 gates = the MFMA's N)
constexpr int kBRows = 8;    // backward: batch rows per workgroup
constexpr int kBUnits = 8;   // backward: hidden units per workgroup

// Forward step t on fp32 MFMA.  Workgroup (unit group, row group) owns rows
// b0..b0+15 and units j0..j0+3; its 16 gate columns are c = 4g + u, gate g of
// unit j0 + u, i.e. W_hh row n(c) = g*H + j0 + u.  The product
// pre[m][c] = sum_k h_{t-1}[b0+m][k] W_hh[n(c)][k] runs as
// v_mfma_f32_16x16x4f32 with the reduction split over the 4 waves (wave w
// takes k in [w H/4, (w+1) H/4)).  In each 64-long block of a wave's range,
// MFMA s = 4i + e gives lane (r, q) = (l % 16, l / 16) the index
// k = kb + 16i + 4q + e on both operands, so a lane's 16 h values and 16
// weights of the block are four float4 loads each, and the four lanes of a
// row read 64 contiguous bytes per load.  Lane l ends with column l % 16 of rows
// 4(l / 16) .. +3; the four wave partials meet in LDS and are added in wave
// order, and wave 0 finishes the 64 cells (lane = 4m + u).  The epilogue's
// inputs are loaded before the product, so their latencies overlap.
// One layer's forward step for the tiled kernels.  G [B, T, 4H] holds the
// input projection x W_ih^T + b on entry (xin == nullptr) and the
// activations on exit.  With xin (a stacked layer fed by the layer below in
// the same launch), the step reduces its input rows xin[b, t, :] [B, T, I]
// against W_ih [4H, I] as well, and the bias (may be null) stands in for G.
struct FwdStep {
  float *G;
  const float *whh;
  const float *xin, *wih, *bias;
  const float *h0, *c0;
  float *h_seq, *c_seq;
  int H, I, t;
};

__device__ __forceinline__ void fwd_step_tile(const FwdStep &s, int blk, int B, int T) {
  __shared__ float part[4][kFRows][16];
  const int H = s.H, t = s.t;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ugroups = H / kFUnits;
  const int ug = blk % ugroups, rg = blk / ugroups;
  const int j0 = ug * kFUnits, b0 = rg * kFRows;
  const int H4 = 4 * H;

  // epilogue inputs of cell (m, u) = (lane / 4, lane % 4), wave 0
  const int em = lane >> 2, eu = lane & 3;
  const int be = b0 + em, je = j0 + eu;
  const bool epi = wave == 0 && be < B;
  const int64_t gb = ((int64_t)be * T + t) * H4;
  float gin[4] = {0.0f, 0.0f, 0.0f, 0.0f}, cp = 0.0f;
  if (epi) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      gin[g] = s.xin == nullptr ? s.G[gb + g * H + je]
                                : (s.bias != nullptr ? s.bias[g * H + je] : 0.0f);
    cp = t > 0 ? s.c_seq[((int64_t)be * T + t - 1) * H + je]
               : (s.c0 != nullptr ? s.c0[(int64_t)be * H + je] : 0.0f);
  }

  // pre[m][c] = sum_k a[m][k] w[n(c)][k] over one operand pair, the
  // reduction split over the four waves in 64-long blocks.
  const int r = lane & 15, q = lane >> 4;
  const int b = min(b0 + r, B - 1);
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto reduce = [&](const float *arow, const float *wrow, int K) {
    const int kw = K >> 2;
    for (int kb = wave * kw; kb < (wave + 1) * kw; kb += 64) {
      f4 a[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = *reinterpret_cast<const f4 *>(arow + kb + 16 * i + 4 * q);
        w[i] = *reinterpret_cast<const f4 *>(wrow + kb + 16 * i + 4 * q);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e >> 2][e & 3], w[e >> 2][e & 3], acc, 0, 0,
                                                   0);
    }
  };
  const int64_t wr = (int64_t)((r >> 2) * H + j0 + (r & 3));  // W row n(c) of column r
  const bool has_h = t > 0 || s.h0 != nullptr;
  const float *hrow = t > 0 ? s.h_seq + ((int64_t)b * T + t - 1) * H
                            : (s.h0 != nullptr ? s.h0 + (int64_t)b * H : nullptr);
  if (has_h && s.xin != nullptr && H == 256 && s.I == 256) {
    // a stacked layer at H = I = 256 (one 64-long block per wave and operand
    // pair): both pairs' operands are loaded before either's MFMAs, one
    // memory round trip instead of two; the MFMAs run in the order above
    const float *xrow = s.xin + ((int64_t)b * T + t) * s.I;
    const int kb = wave * 64;
    f4 a[2][4], w[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[0][i] = *reinterpret_cast<const f4 *>(hrow + kb + 16 * i + 4 * q);
      w[0][i] = *reinterpret_cast<const f4 *>(s.whh + wr * H + kb + 16 * i + 4 * q);
      a[1][i] = *reinterpret_cast<const f4 *>(xrow + kb + 16 * i + 4 * q);
      w[1][i] = *reinterpret_cast<const f4 *>(s.wih + wr * s.I + kb + 16 * i + 4 * q);
    }
#pragma unroll
    for (int pq = 0; pq < 2; ++pq)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[pq][e >> 2][e & 3], w[pq][e >> 2][e & 3], acc,
                                                   0, 0, 0);
  } else {
    if (has_h) reduce(hrow, s.whh + wr * H, H);
    if (s.xin != nullptr) reduce(s.xin + ((int64_t)b * T + t) * s.I, s.wih + wr * s.I, s.I);
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) part[wave][4 * (lane >> 4) + v][lane & 15] = acc[v];
  __syncthreads();
  if (!epi) return;
  float pre[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int c = 4 * g + eu;
    pre[g] = gin[g] + (((part[0][em][c] + part[1][em][c]) + part[2][em][c]) + part[3][em][c]);
  }
  const float i = sigm(pre[0]);
  const float f = sigm(pre[1]);
  const float g = tanhf(pre[2]);
  const float o = sigm(pre[3]);
  const float c = f * cp + i * g;
  const float h = o * tanhf(c);
  s.G[gb + je] = i;
  s.G[gb + H + je] = f;
  s.G[gb + 2 * H + je] = g;
  s.G[gb + 3 * H + je] = o;
  s.c_seq[((int64_t)be * T + t) * H + je] = c;
  s.h_seq[((int64_t)be * T + t) * H + je] = h;
}

__global__ void __launch_bounds__(256) lstm_fwd_step_tiled(FwdStep s, int B, int T) {
  fwd_step_tile(s, blockIdx.x, B, T);
}

// Two stacked layers in one launch (the diagonal schedule): workgroups
// [0, blocks_a) run step a.t of the lower layer, the rest step b.t of the
// upper one, which reads the lower layer's h at b.t -- finished by the
// previous launch.  (Splitting the upper step's input projection into a job
// of its own, one step ahead, measured slower on MI355X: a launch's time
// follows its workgroup count more than its reduction depth.)
__global__ void __launch_bounds__(256)
    lstm_fwd_diag(FwdStep a, FwdStep b, int blocks_a, int B, int T) {
  if ((int)blockIdx.x < blocks_a)
    fwd_step_tile(a, blockIdx.x, B, T);
  else
    fwd_step_tile(b, blockIdx.x - blocks_a, B, T);
}

// Backward step t on the VALU.  The product dh[b][j] = sum_n dG_{t+1}[b][n]
// W_hh[n][j] has only H output columns over a 4H-long reduction, so it is
// register-blocked rather than MFMA-shaped: workgroup (unit group, row group)
// owns rows b0..b0+7 and units j0..j0+7, wave w the 4 x 4 cell block of rows
// b0 + 4(w / 2) and units j0 + 4(w % 2), and lane l of the wave the
// reduction slice n in [l H/16, (l+1) H/16).  wt is W_hh^T [H, 4H], so a
// lane's slice is contiguous both in the block's four dG rows and in the
// four units' rows of wt: it loads both as float4s (consecutive lanes read
// consecutive slices) and carries the 16 cells.  The 64 lanes' partials are
// then summed through LDS (a chain of cross-lane shuffles measured 3 us
// slower per step), and lane 4c finishes cell c.  dc holds
// dc_{t+1} f_{t+1} on entry and dc_t f_t on exit, each (b, j) touched by one
// lane only.
// One layer's backward step for the tiled kernels.  dG [B, T, 4H] receives
// the step's gate gradients; wt is W_hh^T [H, 4H]; dh_out [B, T, H] (may be
// null) is the gradient arriving at h_t from outside the recurrence.  With
// dG_up (a stacked layer whose output feeds the layer above, run in the same
// launch one step behind), dh also takes dG_up[b, t, :] W_ih_up from the
// upper layer's gate gradients of step t (finished by the previous launch),
// wt_up = W_ih_up^T [H, 4Hu].
struct BwdStep {
  float *dG;
  const float *wt;
  const float *acts, *c_seq, *c0;
  const float *dh_out;
  const float *dG_up, *wt_up;
  float *dc;
  int H, Hu, t;
};

__device__ __forceinline__ void bwd_step_tile(const BwdStep &s, int blk, int B, int T) {
  const int H = s.H, t = s.t;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ugroups = H / kBUnits;
  const int ug = blk % ugroups, rg = blk / ugroups;
  const int rb = rg * kBRows + 4 * (wave >> 1), ub = ug * kBUnits + 4 * (wave & 1);
  const int H4 = 4 * H;
  const bool has_next = t + 1 < T;

  // epilogue inputs of cell ec = lane / 4: row rb + ec / 4, unit ub + ec % 4
  const int ec = lane >> 2;
  const int be = rb + (ec >> 2), je = ub + (ec & 3);
  const bool epi = (lane & 3) == 0 && be < B;
  const int64_t row = (int64_t)be * T + t;
  const int64_t gb = row * H4;
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, c = 0.0f, cp = 0.0f, dho = 0.0f, dcn = 0.0f;
  if (epi) {
#pragma unroll
    for (int g = 0; g < 4; ++g) a[g] = s.acts[gb + g * H + je];
    c = s.c_seq[row * H + je];
    cp = t > 0 ? s.c_seq[(row - 1) * H + je]
               : (s.c0 != nullptr ? s.c0[(int64_t)be * H + je] : 0.0f);
    if (s.dh_out != nullptr) dho = s.dh_out[row * H + je];
    if (has_next) dcn = s.dc[(int64_t)be * H + je];
  }

  float v[16];  // cell (i, u) of the wave's block at 4i + u
#pragma unroll
  for (int k = 0; k < 16; ++k) v[k] = 0.0f;
  // v += sum_n d[row i][n] w[unit u][n] over this lane's slice of a 4Hx-long
  // reduction (d row stride and w row stride 4Hx).
  auto reduce = [&](const float *dbase, int64_t tt, const float *wbase, int Hx) {
    const int Hx4 = 4 * Hx;
    const float *drow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) drow[i] = dbase + ((int64_t)min(rb + i, B - 1) * T + tt) * Hx4;
    const int ns = Hx >> 4;  // slice length, a multiple of 4
    const int n0 = lane * ns;
    const float *wrow[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) wrow[u] = wbase + (int64_t)(ub + u) * Hx4;
    for (int nb = n0; nb < n0 + ns; nb += 16) {
      f4 d[4][4], w[4][4];  // [n group][row], [n group][unit]
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (nb + 4 * e < n0 + ns) {
#pragma unroll
          for (int i = 0; i < 4; ++i) d[e][i] = *reinterpret_cast<const f4 *>(drow[i] + nb + 4 * e);
#pragma unroll
          for (int u = 0; u < 4; ++u) w[e][u] = *reinterpret_cast<const f4 *>(wrow[u] + nb + 4 * e);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (nb + 4 * e < n0 + ns) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
              for (int u = 0; u < 4; ++u) v[4 * i + u] += d[e][i][q] * w[e][u][q];
        }
      }
    }
  };
  if (has_next) reduce(s.dG, t + 1, s.wt, H);
  if (s.dG_up != nullptr) reduce(s.dG_up, t, s.wt_up, s.Hu);
  // The 64 lanes' partials of the wave's 16 cells, summed through LDS: the
  // partials are stored cell-major, lane l reads the 16 partials of cell
  // l / 4 from lanes 16 (l % 4) .. +15 as four float4s and adds them in a
  // fixed pairwise order, and the four quarter sums of a cell (lanes
  // 4c .. 4c+3) are added by two exchanges.
  __shared__ f4 part[4][16][16];  // [wave][cell][lane / 4]: lane l at part[..][l / 4][l % 4]
  float *pw = reinterpret_cast<float *>(&part[wave][0][0]);
#pragma unroll
  for (int k = 0; k < 16; ++k) pw[k * 64 + lane] = v[k];
  __syncthreads();
  float r;
  {
    const f4 *src = &part[wave][ec][4 * (lane & 3)];
    const f4 p0 = src[0], p1 = src[1], p2 = src[2], p3 = src[3];
    r = (((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p1[0] + p1[1]) + (p1[2] + p1[3]))) +
        (((p2[0] + p2[1]) + (p2[2] + p2[3])) + ((p3[0] + p3[1]) + (p3[2] + p3[3])));
  }
  r += __shfl_xor(r, 1, 64);
  r += __shfl_xor(r, 2, 64);
  if (!epi) return;
  const float i = a[0], f = a[1], g = a[2], o = a[3];
  const float dh = dho + r;
  const float tc = tanhf(c);
  const float dct = dh * o * (1.0f - tc * tc) + dcn;
  s.dG[gb + je] = (dct * g) * i * (1.0f - i);
  s.dG[gb + H + je] = (dct * cp) * f * (1.0f - f);
  s.dG[gb + 2 * H + je] = (dct * i) * (1.0f - g * g);
  s.dG[gb + 3 * H + je] = (dh * tc) * o * (1.0f - o);
  s.dc[(int64_t)be * H + je] = dct * f;
}

__global__ void __launch_bounds__(256) lstm_bwd_step_tiled(BwdStep s, int B, int T) {
  bwd_step_tile(s, blockIdx.x, B, T);
}

// Two stacked layers' backward in one launch: workgroups [0, blocks_a) run
// step a.t of the upper layer, the rest step b.t = a.t + 1 of the lower
// layer, whose dh takes the upper layer's dG at b.t from the previous launch.
__global__ void __launch_bounds__(256)
    lstm_bwd_diag(BwdStep a, BwdStep b, int blocks_a, int B, int T) {
  if ((int)blockIdx.x < blocks_a)
    bwd_step_tile(a, blockIdx.x, B, T);
  else
    bwd_step_tile(b, blockIdx.x - blocks_a, B, T);
}

// Backward step on fp32 MFMA (H % 256 == 0; for a stacked lower layer also
// Hu % 256 == 0).  Workgroup (unit group, row group) owns rows b0..b0+15 and
// units j0..j0+15 and computes dh[m][u] = sum_n dG_{t+1}[b0+m][n]
// W_hh[n][j0+u] (+ sum_n dG_up[b0+m][n] W_ih_up[n][j0+u]) as
// v_mfma_f32_16x16x4f32: A = dG row b0 + (l % 16), B = W^T row j0 + (l % 16),
// both at n = nb + 16i + 4(l / 16) + e, so each lane's operands are float4
// loads; the 4H-long reduction is split over 16 waves, 64 per wave, and the
// 16 wave partials meet in LDS and are added in wave order.  Threads 0..255
// then finish one cell each.  A 16 x 16 tile reads each operand row once per
// 16 outputs, a quarter of the VALU step's 4 x 4 blocks.
constexpr int kMRows = 16, kMUnits = 16, kMWaves = 16;

__device__ __forceinline__ void bwd_step_mfma(const BwdStep &s, int blk, int B, int T) {
  __shared__ float part[kMWaves][16][16];
  const int H = s.H, t = s.t;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ugroups = H / kMUnits;
  const int ug = blk % ugroups, rg = blk / ugroups;
  const int j0 = ug * kMUnits, b0 = rg * kMRows;
  const int H4 = 4 * H;
  const bool has_next = t + 1 < T;

  // epilogue inputs of cell (em, eu) = (tid / 16, tid % 16), threads 0..255
  const int tid = threadIdx.x;
  const int em = tid >> 4, eu = tid & 15;
  const int be = b0 + em, je = j0 + eu;
  const bool epi = tid < 256 && be < B;
  const int64_t row = (int64_t)be * T + t;
  const int64_t gb = row * H4;
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, c = 0.0f, cp = 0.0f, dho = 0.0f, dcn = 0.0f;
  if (epi) {
#pragma unroll
    for (int g = 0; g < 4; ++g) a[g] = s.acts[gb + g * H + je];
    c = s.c_seq[row * H + je];
    cp = t > 0 ? s.c_seq[(row - 1) * H + je]
               : (s.c0 != nullptr ? s.c0[(int64_t)be * H + je] : 0.0f);
    if (s.dh_out != nullptr) dho = s.dh_out[row * H + je];
    if (has_next) dcn = s.dc[(int64_t)be * H + je];
  }

  const int r = lane & 15, q = lane >> 4;
  const int b = min(b0 + r, B - 1);
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto reduce = [&](const float *dbase, int64_t tt, const float *wbase, int Hx) {
    const int Hx4 = 4 * Hx;
    const float *drow = dbase + ((int64_t)b * T + tt) * Hx4;
    const float *wrow = wbase + (int64_t)(j0 + r) * Hx4;
    const int kw = Hx4 / kMWaves;  // a multiple of 64
    for (int nb = wave * kw; nb < (wave + 1) * kw; nb += 64) {
      f4 d[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d[i] = *reinterpret_cast<const f4 *>(drow + nb + 16 * i + 4 * q);
        w[i] = *reinterpret_cast<const f4 *>(wrow + nb + 16 * i + 4 * q);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(d[e >> 2][e & 3], w[e >> 2][e & 3], acc, 0, 0,
                                                   0);
    }
  };
  if (has_next) reduce(s.dG, t + 1, s.wt, H);
  if (s.dG_up != nullptr) reduce(s.dG_up, t, s.wt_up, s.Hu);
#pragma unroll
  for (int v = 0; v < 4; ++v) part[wave][4 * q + v][r] = acc[v];
  __syncthreads();
  if (!epi) return;
  float sum = part[0][em][eu];
#pragma unroll
  for (int w = 1; w < kMWaves; ++w) sum += part[w][em][eu];
  const float i = a[0], f = a[1], g = a[2], o = a[3];
  const float dh = dho + sum;
  const float tc = tanhf(c);
  const float dct = dh * o * (1.0f - tc * tc) + dcn;
  s.dG[gb + je] = (dct * g) * i * (1.0f - i);
  s.dG[gb + H + je] = (dct * cp) * f * (1.0f - f);
  s.dG[gb + 2 * H + je] = (dct * i) * (1.0f - g * g);
  s.dG[gb + 3 * H + je] = (dh * tc) * o * (1.0f - o);
  s.dc[(int64_t)be * H + je] = dct * f;
}

__global__ void __launch_bounds__(64 * kMWaves) lstm_bwd_step_mfma(BwdStep s, int B, int T) {
  bwd_step_mfma(s, blockIdx.x, B, T);
}

__global__ void __launch_bounds__(64 * kMWaves)
    lstm_bwd_diag_mfma(BwdStep a, BwdStep b, int blocks_a, int B, int T) {
  if ((int)blockIdx.x < blocks_a)
    bwd_step_mfma(a, blockIdx.x, B, T);
  else
    bwd_step_mfma(b, blockIdx.x - blocks_a, B, T);
}

// Whether the tiled step kernels take this shape.  The forward walks each
// wave's quarter of the reduction in whole 64-long blocks (H % 256 == 0); the
// backward's lane slices are H/16 long in float4 steps (H % 64 == 0).  Both
// read rows of W_hh and of h or dG as float4s.
bool tiled_fwd_fits(int64_t H, const void *whh, const void *h_seq, const void *h0) {
  return H % 256 == 0 && numrs_hip::aligned16(whh) && numrs_hip::aligned16(h_seq) &&
         (h0 == nullptr || numrs_hip::aligned16(h0));
}
bool tiled_bwd_fits(int64_t H, const void *whh, const void *dG) {
  return H % 64 == 0 && numrs_hip::aligned16(whh) && numrs_hip::aligned16(dG);
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

// Row forms of shift_hidden and time_slice_kernel for 16-byte aligned
// arrays whose rows are a whole number of float4s: workgroup r copies row r
// (r = b T + t) with float4 accesses, and the only index arithmetic per
// thread is one 32-bit division (the element kernels above take two or three
// 64-bit divisions per element).
__global__ void __launch_bounds__(64)
    shift_hidden_rows(const float *__restrict__ h_seq, const float *__restrict__ h0,
                      float *__restrict__ out, int T, int H) {
  const int64_t r = blockIdx.x;
  const int b = (int)(r / T), t = (int)(r - (int64_t)b * T);
  const float *src = t > 0 ? h_seq + (r - 1) * H : (h0 != nullptr ? h0 + (int64_t)b * H : nullptr);
  for (int c = 4 * threadIdx.x; c < H; c += 4 * 64) {
    const f4 v = src != nullptr ? *reinterpret_cast<const f4 *>(src + c) : f4{0.0f, 0.0f, 0.0f, 0.0f};
    *reinterpret_cast<f4 *>(out + r * H + c) = v;
  }
}

// forward: y[b, :] = x[b, t, :] (blockIdx.x = b); backward: row r = b T + tt of
// dx [B, T, D] is g[b, :] at tt = t and 0 elsewhere (added to, or only step t
// touched, with acc).
__global__ void __launch_bounds__(64)
    time_slice_rows(const float *__restrict__ x, float *__restrict__ y, int T, int D, int t,
                    int backward, int acc) {
  const int64_t r = blockIdx.x;
  if (!backward) {
    for (int c = 4 * threadIdx.x; c < D; c += 4 * 64)
      *reinterpret_cast<f4 *>(y + r * D + c) =
          *reinterpret_cast<const f4 *>(x + (r * T + t) * D + c);
    return;
  }
  const int b = (int)(r / T), tt = (int)(r - (int64_t)b * T);
  if (acc && tt != t) return;
  for (int c = 4 * threadIdx.x; c < D; c += 4 * 64) {
    const f4 v = tt == t ? *reinterpret_cast<const f4 *>(x + (int64_t)b * D + c)
                         : f4{0.0f, 0.0f, 0.0f, 0.0f};
    f4 *dst = reinterpret_cast<f4 *>(y + r * D + c);
    if (acc) {
      *dst = *dst + v;
    } else {
      *dst = v;
    }
  }
}

// One layer's parameter and input gradients from its gate gradients dG
// [B*T, 4H] of every step, batched over time as single products:
// dW_ih = dG^T x, dW_hh = dG^T H_prev, db = column sum of dG, dx = dG W_ih
// (each output may be null).
int lstm_param_grads(numrs_hip_ctx *ctx, const float *dG, const float *x, const float *w_ih,
                     const float *h_seq, const float *h0, float *dx, float *dw_ih, float *dw_hh,
                     float *db, int64_t B, int64_t T, int64_t I, int64_t H, int acc_dx,
                     int acc_dw_ih, int acc_dw_hh, int acc_db) {
  const int64_t rows = B * T, H4 = 4 * H;
  if (dw_ih)  // dW_ih[4H, I] = dG^T x
    if (int rc = numrs_hip_gemm(ctx, dG, H4, x, I, dw_ih, I, H4, rows, I, 1, 0, 1.0f, acc_dw_ih,
                                1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  if (dw_hh) {  // dW_hh[4H, H] = dG^T H_prev
    TempBlock hp(ctx);
    if (int rc = hp.alloc((size_t)(rows * H) * sizeof(float))) return rc;
    if (H % 4 == 0 && numrs_hip::aligned16(h_seq) && numrs_hip::aligned16(hp.f()) &&
        (h0 == nullptr || numrs_hip::aligned16(h0)) && rows <= 0x7fffffff) {
      shift_hidden_rows<<<(unsigned)rows, 64, 0, ctx->stream>>>(h_seq, h0, hp.f(), (int)T, (int)H);
    } else {
      shift_hidden<<<grid_for(rows * H, 256), 256, 0, ctx->stream>>>(h_seq, h0, hp.f(), (int)B,
                                                                     (int)T, (int)H);
    }
    if (int rc = numrs_hip::check_launch(ctx, "shift_hidden")) return rc;
    if (int rc = numrs_hip_gemm(ctx, dG, H4, hp.f(), H, dw_hh, H, H4, rows, H, 1, 0, 1.0f,
                                acc_dw_hh, 1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  }
  if (db) {  // db[4H] = column sum of dG
    const int64_t gs[2] = {rows, H4};
    const int64_t bs = H4;
    if (int rc = numrs_hip_sum_to_shape(ctx, dG, gs, 2, db, &bs, 1,
                                        NUMRS_HIP_UNBROADCAST_CORRECT, acc_db))
      return rc;
  }
  if (dx)  // dx[B*T, I] = dG W_ih
    if (int rc = numrs_hip_gemm(ctx, dG, H4, w_ih, I, dx, I, rows, H4, I, 0, 0, 1.0f, acc_dx, 1,
                                1, 0, 0, 0, 0, 0, 0))
      return rc;
  return NUMRS_HIP_OK;
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
  if (tiled_fwd_fits(H, w_hh, h_seq, h0)) {
    const unsigned grid = (unsigned)((H / kFUnits) * ((B + kFRows - 1) / kFRows));
    FwdStep st{acts, w_hh, nullptr, nullptr, nullptr, h0, c0, h_seq, c_seq, (int)H, 0, 0};
    for (int64_t t = 0; t < T; ++t) {
      st.t = (int)t;
      lstm_fwd_step_tiled<<<grid, 256, 0, ctx->stream>>>(st, (int)B, (int)T);
      if (int rc = numrs_hip::check_launch(ctx, "lstm_fwd_step_tiled")) return rc;
    }
    return NUMRS_HIP_OK;
  }
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
  if (tiled_bwd_fits(H, w_hh, dG.p)) {
    TempBlock wt(ctx);  // W_hh^T [H, 4H]
    if (int rc = wt.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
    if (int rc = numrs_hip_transpose(ctx, w_hh, wt.f(), 4 * H, H)) return rc;
    BwdStep st{dG.f(), wt.f(), acts, c_seq, c0, dh_seq, nullptr, nullptr, dc.f(), (int)H, 0, 0};
    if (H % 256 == 0) {
      const unsigned grid = (unsigned)((H / kMUnits) * ((B + kMRows - 1) / kMRows));
      for (int64_t t = T - 1; t >= 0; --t) {
        st.t = (int)t;
        lstm_bwd_step_mfma<<<grid, 64 * kMWaves, 0, ctx->stream>>>(st, (int)B, (int)T);
        if (int rc = numrs_hip::check_launch(ctx, "lstm_bwd_step_mfma")) return rc;
      }
    } else {
      const unsigned grid = (unsigned)((H / kBUnits) * ((B + kBRows - 1) / kBRows));
      for (int64_t t = T - 1; t >= 0; --t) {
        st.t = (int)t;
        lstm_bwd_step_tiled<<<grid, 256, 0, ctx->stream>>>(st, (int)B, (int)T);
        if (int rc = numrs_hip::check_launch(ctx, "lstm_bwd_step_tiled")) return rc;
      }
    }
  } else {
    TempBlock wp(ctx);
    if (int rc = wp.alloc((size_t)(4 * H * H) * sizeof(float))) return rc;
    pack_gates<<<grid_for(4 * H * H, 256), 256, 0, ctx->stream>>>(w_hh, wp.f(), (int)H, H * H,
                                                                  H);
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
  }
  return lstm_param_grads(ctx, dG.f(), x, w_ih, h_seq, h0, dx, dw_ih, dw_hh, db, B, T, I, H,
                          acc_dx, acc_dw_ih, acc_dw_hh, acc_db);
}

int numrs_hip_lstm2_forward(numrs_hip_ctx *ctx, const float *x, const float *w_ih1,
                            const float *w_hh1, const float *b1, const float *w_ih2,
                            const float *w_hh2, const float *b2, float *h1_seq, float *c1_seq,
                            float *acts1, float *h2_seq, float *c2_seq, float *acts2, int64_t B,
                            int64_t T, int64_t I, int64_t H1, int64_t H2) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, T, I, H1)) return rc;
  if (int rc = check(ctx, B, T, H1, H2)) return rc;
  if (!x || !w_ih1 || !w_hh1 || !w_ih2 || !w_hh2 || !h1_seq || !c1_seq || !acts1 || !h2_seq ||
      !c2_seq || !acts2)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "lstm2_forward: null pointer");
  const bool diag = tiled_fwd_fits(H1, w_hh1, h1_seq, nullptr) &&
                    tiled_fwd_fits(H2, w_hh2, h2_seq, nullptr) && numrs_hip::aligned16(w_ih2);
  if (!diag) {  // one layer after the other
    if (int rc = numrs_hip_lstm_forward(ctx, x, w_ih1, w_hh1, b1, nullptr, nullptr, h1_seq, c1_seq,
                                        acts1, B, T, I, H1))
      return rc;
    return numrs_hip_lstm_forward(ctx, h1_seq, w_ih2, w_hh2, b2, nullptr, nullptr, h2_seq, c2_seq,
                                  acts2, B, T, H1, H2);
  }
  // acts1 <- x W_ih1^T + b1 for every (b, t) row; the upper layer reduces
  // h1 against W_ih2 inside its steps.
  if (int rc = numrs_hip_linear_forward(ctx, x, w_ih1, b1, acts1, B * T, I, 4 * H1)) return rc;
  FwdStep lo{acts1, w_hh1, nullptr, nullptr, nullptr, nullptr, nullptr, h1_seq, c1_seq,
             (int)H1, 0, 0};
  FwdStep up{acts2, w_hh2, h1_seq, w_ih2, b2, nullptr, nullptr, h2_seq, c2_seq, (int)H2, (int)H1,
             0};
  const int rgroups = (int)((B + kFRows - 1) / kFRows);
  const int g_lo = (int)(H1 / kFUnits) * rgroups, g_up = (int)(H2 / kFUnits) * rgroups;
  // Launch d: lower step d and upper step d - 1.
  for (int64_t d = 0; d <= T; ++d) {
    const int ga = d < T ? g_lo : 0, gb = d >= 1 ? g_up : 0;
    lo.t = (int)d;
    up.t = (int)d - 1;
    lstm_fwd_diag<<<(unsigned)(ga + gb), 256, 0, ctx->stream>>>(lo, up, ga, (int)B, (int)T);
    if (int rc = numrs_hip::check_launch(ctx, "lstm_fwd_diag")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_lstm2_backward(numrs_hip_ctx *ctx, const float *x, const float *w_ih1,
                             const float *w_hh1, const float *w_ih2, const float *w_hh2,
                             const float *h1_seq, const float *c1_seq, const float *acts1,
                             const float *h2_seq, const float *c2_seq, const float *acts2,
                             const float *dh2_seq, float *dx, float *dw_ih1, float *dw_hh1,
                             float *db1, float *dw_ih2, float *dw_hh2, float *db2, int64_t B,
                             int64_t T, int64_t I, int64_t H1, int64_t H2, int acc_dx,
                             int acc_dw_ih1, int acc_dw_hh1, int acc_db1, int acc_dw_ih2,
                             int acc_dw_hh2, int acc_db2) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, T, I, H1)) return rc;
  if (int rc = check(ctx, B, T, H1, H2)) return rc;
  if (!x || !w_ih1 || !w_hh1 || !w_ih2 || !w_hh2 || !h1_seq || !c1_seq || !acts1 || !h2_seq ||
      !c2_seq || !acts2)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "lstm2_backward: null input");
  TempBlock dG1(ctx), dG2(ctx);
  if (int rc = dG1.alloc((size_t)(B * T * 4 * H1) * sizeof(float))) return rc;
  if (int rc = dG2.alloc((size_t)(B * T * 4 * H2) * sizeof(float))) return rc;
  const bool diag = tiled_bwd_fits(H1, w_hh1, dG1.p) && tiled_bwd_fits(H2, w_hh2, dG2.p) &&
                    numrs_hip::aligned16(w_ih2);
  if (!diag) {  // the upper layer's backward, then the lower one's from its dx
    TempBlock dh1(ctx);
    if (int rc = dh1.alloc((size_t)(B * T * H1) * sizeof(float))) return rc;
    if (int rc = numrs_hip_lstm_backward(ctx, h1_seq, w_ih2, w_hh2, nullptr, nullptr, h2_seq,
                                         c2_seq, acts2, dh2_seq, dh1.f(), dw_ih2, dw_hh2, db2, B,
                                         T, H1, H2, 0, acc_dw_ih2, acc_dw_hh2, acc_db2))
      return rc;
    return numrs_hip_lstm_backward(ctx, x, w_ih1, w_hh1, nullptr, nullptr, h1_seq, c1_seq, acts1,
                                   dh1.f(), dx, dw_ih1, dw_hh1, db1, B, T, I, H1, acc_dx,
                                   acc_dw_ih1, acc_dw_hh1, acc_db1);
  }
  TempBlock dc1(ctx), dc2(ctx), wt1(ctx), wt2(ctx), wtu(ctx);
  if (int rc = dc1.alloc((size_t)(B * H1) * sizeof(float))) return rc;
  if (int rc = dc2.alloc((size_t)(B * H2) * sizeof(float))) return rc;
  if (int rc = wt1.alloc((size_t)(4 * H1 * H1) * sizeof(float))) return rc;
  if (int rc = wt2.alloc((size_t)(4 * H2 * H2) * sizeof(float))) return rc;
  if (int rc = wtu.alloc((size_t)(4 * H2 * H1) * sizeof(float))) return rc;
  if (int rc = numrs_hip_transpose(ctx, w_hh1, wt1.f(), 4 * H1, H1)) return rc;  // [H1, 4H1]
  if (int rc = numrs_hip_transpose(ctx, w_hh2, wt2.f(), 4 * H2, H2)) return rc;  // [H2, 4H2]
  if (int rc = numrs_hip_transpose(ctx, w_ih2, wtu.f(), 4 * H2, H1)) return rc;  // [H1, 4H2]
  BwdStep up{dG2.f(), wt2.f(), acts2, c2_seq, nullptr, dh2_seq, nullptr, nullptr, dc2.f(),
             (int)H2, 0, 0};
  BwdStep lo{dG1.f(), wt1.f(), acts1, c1_seq, nullptr, nullptr, dG2.f(), wtu.f(), dc1.f(),
             (int)H1, (int)H2, 0};
  // MFMA steps when both layers' reductions split into 64-long wave blocks.
  const bool mfma = H1 % 256 == 0 && H2 % 256 == 0;
  const int rows_per = mfma ? kMRows : kBRows, units_per = mfma ? kMUnits : kBUnits;
  const int rgroups = (int)((B + rows_per - 1) / rows_per);
  const int g_up = (int)(H2 / units_per) * rgroups, g_lo = (int)(H1 / units_per) * rgroups;
  // Launch d: upper step T-1-d and lower step T-d (the lower layer's dh at
  // step T-d takes the upper layer's dG of that step from launch d-1).
  for (int64_t d = 0; d <= T; ++d) {
    const int ga = d < T ? g_up : 0, gb = d >= 1 ? g_lo : 0;
    up.t = (int)(T - 1 - d);
    lo.t = (int)(T - d);
    if (mfma)
      lstm_bwd_diag_mfma<<<(unsigned)(ga + gb), 64 * kMWaves, 0, ctx->stream>>>(up, lo, ga, (int)B,
                                                                                (int)T);
    else
      lstm_bwd_diag<<<(unsigned)(ga + gb), 256, 0, ctx->stream>>>(up, lo, ga, (int)B, (int)T);
    if (int rc = numrs_hip::check_launch(ctx, "lstm_bwd_diag")) return rc;
  }
  if (int rc = lstm_param_grads(ctx, dG2.f(), h1_seq, w_ih2, h2_seq, nullptr, nullptr, dw_ih2,
                                dw_hh2, db2, B, T, H1, H2, 0, acc_dw_ih2, acc_dw_hh2, acc_db2))
    return rc;
  return lstm_param_grads(ctx, dG1.f(), x, w_ih1, h1_seq, nullptr, dx, dw_ih1, dw_hh1, db1, B, T,
                          I, H1, acc_dx, acc_dw_ih1, acc_dw_hh1, acc_db1);
}

int numrs_hip_time_slice(numrs_hip_ctx *ctx, const float *x, float *y, int64_t B, int64_t T,
                         int64_t D, int64_t t, int backward, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (B < 0 || T <= 0 || D < 0 || t < 0 || t >= T || !x || !y)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "time_slice: bad arguments");
  const int64_t n = backward ? B * T * D : B * D;
  if (n == 0) return NUMRS_HIP_OK;
  const int64_t nrows = backward ? B * T : B;
  if (D % 4 == 0 && numrs_hip::aligned16(x) && numrs_hip::aligned16(y) && nrows <= 0x7fffffff &&
      T <= 0x7fffffff && D <= 0x7fffffff) {
    time_slice_rows<<<(unsigned)nrows, 64, 0, ctx->stream>>>(x, y, (int)T, (int)D, (int)t,
                                                             backward, accumulate);
    return numrs_hip::check_launch(ctx, "time_slice_rows");
  }
  time_slice_kernel<<<grid_for(n, 256), 256, 0, ctx->stream>>>(x, y, B, T, D, t, backward,
                                                                accumulate);
  return numrs_hip::check_launch(ctx, "time_slice_kernel");
}

}  // extern "C"
