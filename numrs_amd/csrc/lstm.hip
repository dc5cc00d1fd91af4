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

// One cell's forward from its gate pre-activations (order i, f, g, o) and
// previous cell state: act = (sigmoid i, sigmoid f, tanh g, sigmoid o),
// c = f c_prev + i g, h = o tanh(c).  Shared by every step kernel, so all
// paths round alike.
__device__ __forceinline__ void cell_forward(const float pre[4], float cp, float act[4], float &c,
                                             float &h) {
  act[0] = sigm(pre[0]);
  act[1] = sigm(pre[1]);
  act[2] = tanhf(pre[2]);
  act[3] = sigm(pre[3]);
  c = act[1] * cp + act[0] * act[2];
  h = act[3] * tanhf(c);
}

// One cell's backward: a = saved activations (i, f, g, o), c / cp = cell
// state at this and the previous step, dh = gradient at h, dcn = dc_{t+1}
// f_{t+1} (0 at the last step).  Gate pre-activation gradients into dg, the
// product dc_t f_t for the step before into dcf.  The gate formulas are the
// reference's sigmoid_backward ((g s)(1 - s), backward.rs:166-177),
// tanh_backward (g (1 - y^2), backward.rs:503-517) and mul_backward
// (backward.rs:74-87) composed through c = f c_prev + i g, h = o tanh(c).
__device__ __forceinline__ void cell_backward(const float a[4], float c, float cp, float dh,
                                              float dcn, float dg[4], float &dcf) {
  const float i = a[0], f = a[1], g = a[2], o = a[3];
  const float tc = tanhf(c);
  const float dct = dh * o * (1.0f - tc * tc) + dcn;
  dg[0] = (dct * g) * i * (1.0f - i);
  dg[1] = (dct * cp) * f * (1.0f - f);
  dg[2] = (dct * i) * (1.0f - g * g);
  dg[3] = (dh * tc) * o * (1.0f - o);
  dcf = dct * f;
}

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
  float pre[4], act[4], c, h;
#pragma unroll
  for (int k = 0; k < 4; ++k) pre[k] = gin[k] + part[0][u * 4 + k][lane];
  cell_forward(pre, cp, act, c, h);
#pragma unroll
  for (int k = 0; k < 4; ++k) G[gb + k * H + j] = act[k];
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
  float dg[4], dcf;
  cell_backward(a, c, cp, dho + r, dcn, dg, dcf);
#pragma unroll
  for (int k = 0; k < 4; ++k) dG[gb + k * H + j] = dg[k];
  dc[(int64_t)be * H + j] = dcf;
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
// activations on exit.  With xin (the first layer's input, I % 64 == 0 and
// I <= 256, or a stacked layer fed by the layer below in the same launch),
// the step reduces its input rows xin[b, t, :] [B, T, I] against
// W_ih [4H, I] as well, before the recurrent rows, and the bias (may be
// null) stands in for G.
struct FwdStep {
  float *G;
  const float *whh;
  const float *xin, *wih, *bias;
  const float *h0, *c0;
  float *h_seq, *c_seq;
  int H, I, t;
  int sep;  // the input reduction in an accumulator of its own, + bias, then + the recurrent one
};

__device__ __forceinline__ void fwd_step_tile(const FwdStep &s, int blk, int B, int T) {
  __shared__ float part[4][kFRows][16], partx[4][kFRows][16];
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
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, accx = {0.0f, 0.0f, 0.0f, 0.0f};
  // K % 64 == 0: a wave's range is K/4 long, walked in groups of up to four
  // 16-long blocks (block i of a group at kb + 16 i), each block four MFMAs
  // -- the same k order for every K.
  auto reduce = [&](f4 &acc, const float *arow, const float *wrow, int K) {
    const int kw = K >> 2, kend = (wave + 1) * kw;
    for (int kb = wave * kw; kb < kend; kb += 64) {
      const int nb = min(4, (kend - kb) >> 4);
      f4 a[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < nb) {
          a[i] = *reinterpret_cast<const f4 *>(arow + kb + 16 * i + 4 * q);
          w[i] = *reinterpret_cast<const f4 *>(wrow + kb + 16 * i + 4 * q);
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if ((e >> 2) < nb)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e >> 2][e & 3], w[e >> 2][e & 3], acc, 0, 0,
                                                     0);
    }
  };
  const int64_t wr = (int64_t)((r >> 2) * H + j0 + (r & 3));  // W row n(c) of column r
  const bool has_h = t > 0 || s.h0 != nullptr;
  const float *hrow = t > 0 ? s.h_seq + ((int64_t)b * T + t - 1) * H
                            : (s.h0 != nullptr ? s.h0 + (int64_t)b * H : nullptr);
  if (has_h && s.xin != nullptr && !s.sep && H == 256 && s.I == 256) {
    // a stacked layer at H = I = 256 (one 64-long block per wave and operand
    // pair): both pairs' operands are loaded before either's MFMAs, one
    // memory round trip instead of two; the MFMAs run in the order below
    const float *xrow = s.xin + ((int64_t)b * T + t) * s.I;
    const int kb = wave * 64;
    f4 a[2][4], w[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[0][i] = *reinterpret_cast<const f4 *>(xrow + kb + 16 * i + 4 * q);
      w[0][i] = *reinterpret_cast<const f4 *>(s.wih + wr * s.I + kb + 16 * i + 4 * q);
      a[1][i] = *reinterpret_cast<const f4 *>(hrow + kb + 16 * i + 4 * q);
      w[1][i] = *reinterpret_cast<const f4 *>(s.whh + wr * H + kb + 16 * i + 4 * q);
    }
#pragma unroll
    for (int pq = 0; pq < 2; ++pq)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[pq][e >> 2][e & 3], w[pq][e >> 2][e & 3], acc,
                                                   0, 0, 0);
  } else {
    // a stacked layer's input reduction first (the persistent kernel forms it
    // while it waits for the recurrent operand), then the recurrent one
    if (s.xin != nullptr)
      reduce(s.sep ? accx : acc, s.xin + ((int64_t)b * T + t) * s.I, s.wih + wr * s.I, s.I);
    if (has_h) reduce(acc, hrow, s.whh + wr * H, H);
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    part[wave][4 * (lane >> 4) + v][lane & 15] = acc[v];
    if (s.sep) partx[wave][4 * (lane >> 4) + v][lane & 15] = accx[v];
  }
  __syncthreads();
  if (!epi) return;
  float pre[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int c = 4 * g + eu;
    if (s.sep)  // x W_ih^T + b, as the product with a bias epilogue
      gin[g] = (((partx[0][em][c] + partx[1][em][c]) + partx[2][em][c]) + partx[3][em][c]) + gin[g];
    pre[g] = gin[g] + (((part[0][em][c] + part[1][em][c]) + part[2][em][c]) + part[3][em][c]);
  }
  float act[4], c, h;
  cell_forward(pre, cp, act, c, h);
#pragma unroll
  for (int k = 0; k < 4; ++k) s.G[gb + k * H + je] = act[k];
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
  // MFMA steps: when set, dbp [2][B, 4H] holds the compensated sums over the
  // steps so far (t descending) of each row's gate gradients, then their
  // compensation terms (kahan_add); the step at t = 0 adds each 16-row
  // group's sums into dbf [row groups, 4H] (tile_bias_partial) -- the bias
  // gradient's partials.
  float *dbp, *dbf;
};

// One step of a compensated (Kahan) sum: sum += v with the rounding error
// carried in comp.  The LSTM bias gradient sums each row's T gate gradients
// this way, as every step kernel forms them, so the per-row partials are
// about as accurate as a pairwise sum.
__device__ __forceinline__ void kahan_add(float &sum, float &comp, float v) {
  const float y = v - comp;
  const float t = sum + y;
  comp = (t - sum) - y;
  sum = t;
}

// The bias partial of one 16-row x 16-unit tile of the MFMA backward steps:
// lds[g][m][u] holds cell (row m, unit u)'s compensated step sum of gate g
// (sum - comp; 0 for rows past B).  Threads 0..63 (gate tid / 16, unit
// tid % 16) add the 16 rows in order as a compensated sum into
// out[g H + j0 + u].  The block meets before and after the LDS is read.
__device__ __forceinline__ void tile_bias_partial(float (*lds)[16][16], float *out, int H,
                                                  int j0) {
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int g = tid >> 4, u = tid & 15;
    float sum = 0.0f, comp = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; ++m) kahan_add(sum, comp, lds[g][m][u]);
    out[g * H + j0 + u] = sum - comp;
  }
}

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
  r = quad_sum(r);
  if (!epi) return;
  float dg[4], dcf;
  cell_backward(a, c, cp, dho + r, dcn, dg, dcf);
#pragma unroll
  for (int k = 0; k < 4; ++k) s.dG[gb + k * H + je] = dg[k];
  s.dc[(int64_t)be * H + je] = dcf;
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
  __shared__ float part[kMWaves][16][16], partu[kMWaves][16][16];
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
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
  auto reduce = [&](f4 &ac, const float *dbase, int64_t tt, const float *wbase, int Hx) {
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
        ac = __builtin_amdgcn_mfma_f32_16x16x4f32(d[e >> 2][e & 3], w[e >> 2][e & 3], ac, 0, 0, 0);
    }
  };
  // The two reductions (own recurrence, upper layer's input gradient) in
  // separate accumulators, each summed over the waves in order, then added:
  // the persistent kernels form the second one in other workgroups.
  if (has_next) reduce(acc, s.dG, t + 1, s.wt, H);
  if (s.dG_up != nullptr) reduce(accu, s.dG_up, t, s.wt_up, s.Hu);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    part[wave][4 * q + v][r] = acc[v];
    partu[wave][4 * q + v][r] = accu[v];
  }
  __syncthreads();
  const bool last = s.dbp != nullptr && t == 0;  // this launch forms the tile's bias partial
  if (!epi && !last) return;
  float dbv[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // the cell's step sums (last step, rows < B)
  if (epi) {
    float sum = part[0][em][eu];
#pragma unroll
    for (int w = 1; w < kMWaves; ++w) sum += part[w][em][eu];
    if (s.dG_up != nullptr) {
      float sumu = partu[0][em][eu];
#pragma unroll
      for (int w = 1; w < kMWaves; ++w) sumu += partu[w][em][eu];
      sum = sum + sumu;
    }
    float dg[4], dcf;
    cell_backward(a, c, cp, dho + sum, dcn, dg, dcf);
#pragma unroll
    for (int k = 0; k < 4; ++k) s.dG[gb + k * H + je] = dg[k];
    s.dc[(int64_t)be * H + je] = dcf;
    if (s.dbp != nullptr) {  // the step at T - 1 starts the sums from zero, as a register would
      float *dp = s.dbp + (int64_t)be * H4 + je, *dq = dp + (int64_t)B * H4;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float bs = has_next ? dp[k * H] : 0.0f, bc = has_next ? dq[k * H] : 0.0f;
        kahan_add(bs, bc, dg[k]);
        dp[k * H] = bs;
        dq[k * H] = bc;
        dbv[k] = bs - bc;
      }
    }
  }
  if (last) {  // every thread is here: part is free once the block has met
    float(*lds)[16][16] = part;
    __syncthreads();
    if (tid < 256) {
#pragma unroll
      for (int k = 0; k < 4; ++k) lds[k][em][eu] = dbv[k];
    }
    tile_bias_partial(lds, s.dbf + (int64_t)(b0 / kMRows) * H4, H, j0);
  }
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

// ---------------------------------------------------------------------------
// Persistent recurrences of two stacked layers (H1 = H2 = 256): one launch
// runs every step of both layers' forward, one every step of their
// backward, instead of T + 1 launches each.
//
// Each layer runs in workgroups of its own, so the two recurrences are two
// chains: the forward's lower chain depends only on itself and the upper one
// on itself and the lower one (which usually runs ahead); the backward's
// upper chain only on itself and the lower one on itself and the upper one.
// A step of row group rg (16 batch rows) reads only the previous step's
// values of the same rows (all units of h, or of dG), so the workgroups of
// a chain and row group meet at per-workgroup step counters instead of a
// grid-wide barrier.  The values that cross workgroups (h, dG) are written
// and read at device scope, one access at a time: stores write through to
// the device's coherence point and loads fetch from it (the sc1 scope bit),
// which the eight XCDs' L2 caches need no write-back or invalidation for (a
// cache-wide write-back and invalidation per step, agent-scope fences,
// measured 3.3x slower than one launch per step).  After a step every lane
// waits for its stores to be acknowledged, the block meets, and one thread
// stores the number of steps the workgroup has finished into its counter
// (device scope).  Before a step one wave reads the counters the step
// depends on at device scope until all have reached it; the block meets
// again and only then loads the step's rows.  (Polling the operands
// themselves, pre-set to a signalling-NaN pattern, flooded the coherence
// point with requests and measured slower; so did both layers in one
// workgroup, whose waits covered twice as many workgroups: a step's wait
// ends when the slowest workgroup it depends on has finished.)
//
// The wait is bounded: after `spin` rounds (kSpinLimit unless the context
// sets another limit), or once another workgroup
// has given up (the abort word after the counters), a workgroup records the
// give-up in the context's status word and returns, so every workgroup
// exits; the host reports it at its next synchronisation.  The host
// launches only a grid that the occupancy query says the device holds at
// once.  The launch is an ordinary one: the stream has drained its earlier
// work when the grid starts, so every workgroup becomes resident once other
// streams' work leaves the CUs, and the bounded wait covers the time until
// then.  (A cooperative launch, whose runtime guarantees co-residency, costs
// about 25 us more per launch on MI355X; COOPERATIVE mode selects it.)
//
// Each wave keeps its slice of the recurrent (and stacked input) weights in
// registers for the whole launch; a step reads only the rows it reduces and
// its cells' saved values, and each lane carries its cell's c (forward) or
// dc f (backward) from step to step in a register.  The per-wave reduction
// slices, the MFMA operand layout and the order in which partials are added
// are those of the per-step kernels (lstm_fwd_diag, lstm_bwd_diag_mfma), so
// both paths give the same bits.
// ---------------------------------------------------------------------------
constexpr int kSpinLimit = 1 << 21;  // wait rounds before giving up (seconds of waiting)
constexpr int kPersistH = 256;       // the hidden size of the persistent kernels
constexpr int kPFUnits = 8;          // forward: hidden units per workgroup (two MFMA tiles)
using numrs_hip::dev_rsrc;
using numrs_hip::ld_dev4;
using numrs_hip::st_dev;

// After a step: every lane's device-scope stores acknowledged, the block
// met, then thread 0 publishes `steps` in the workgroup's counter.
__device__ __forceinline__ void publish_step(unsigned *counter, unsigned steps) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// On the calling wave: waits until the na counters at fa have reached ta
// and the nb counters at fb have reached tb (na, nb <= 64).  Returns false,
// after recording why, when the wait ran out (status 1) or another
// workgroup gave up (the abort word is set).
__device__ bool wait_counters(const unsigned *fa, int na, unsigned ta, const unsigned *fb, int nb,
                              unsigned tb, unsigned *abort_word, int *status, int spin) {
  const int lane = threadIdx.x & 63;
  for (int it = 0;; ++it) {
    bool ok = true;
    if (lane < na)
      ok = __hip_atomic_load(fa + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= ta;
    if (lane < nb)
      ok = ok && __hip_atomic_load(fb + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= tb;
    if (__all(ok)) return true;
    const unsigned ab = __hip_atomic_load(abort_word + (lane & 0), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    if (ab != 0u || it >= spin) {
      if (lane == 0) {
        if (ab == 0u) __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(abort_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Before a step: wave 0 waits (wait_counters); the block meets; false when
// the wait gave up (every thread then returns).
__device__ __forceinline__ bool await_step(const unsigned *fa, int na, unsigned ta,
                                           const unsigned *fb, int nb, unsigned tb,
                                           unsigned *abort_word, int *status, int spin,
                                           int *s_go) {
  if (threadIdx.x < 64) {
    const bool ok = wait_counters(fa, na, ta, fb, nb, tb, abort_word, status, spin);
    if (threadIdx.x == 0) *s_go = ok ? 1 : 0;
  }
  __syncthreads();
  return *s_go != 0;
}

struct Lstm2Fwd {
  float *acts1, *acts2;              // [B, T, 4H]; acts1 holds x W_ih1^T + b1 on entry (NI = 0)
  const float *whh1, *wih2, *whh2;   // [4H, H]
  const float *b2;                   // [4H] or null
  const float *x, *wih1, *b1;        // NI > 0: x [B, T, I], W_ih1 [4H, I], b1 [4H] or null
  float *h1, *c1, *h2, *c2;          // [B, T, H]
  unsigned *count;  // [2][rgroups][H / kPFUnits] steps done (lower, upper), then the abort word
  int *status;
  int B, T;
  int spin;  // wait rounds before giving up
};

// Forward: workgroups [0, n) run the lower layer, [n, 2n) the upper one;
// workgroup (row group rg, unit group ug) owns rows b0..b0+15 and units
// j0..j0+7 of its layer as two kFRows x kFUnits tiles (those of
// lstm_fwd_diag): wave w forms quarter w % 4 of tile w / 4's reduction, and
// waves 0 and 4 finish the tiles' 64 cells each.  Lower step t reads h1 at
// t - 1; upper step t reads h2 at t - 1 and h1 at t.  With NI > 0 (I =
// 64 NI) the lower layer forms x_t W_ih1^T itself, in the per-step kernels'
// order (the input blocks, then the recurrent ones), before it waits for its
// previous step: those MFMAs and their loads overlap the wait.
template <int NI>
__global__ void __launch_bounds__(512) lstm2_fwd_persist(Lstm2Fwd p) {
  constexpr int H = kPersistH, H4 = 4 * H;
  constexpr int ugroups = H / kPFUnits;
  __shared__ float part[8][kFRows][16], partx[NI > 0 ? 8 : 1][kFRows][16];
  __shared__ int s_go;
  const int B = p.B, T = p.T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rgroups = (int)gridDim.x / (2 * ugroups);
  const bool upper = (int)blockIdx.x >= rgroups * ugroups;
  const int blk = upper ? (int)blockIdx.x - rgroups * ugroups : (int)blockIdx.x;
  const int ug = blk % ugroups, rg = blk / ugroups;
  const int tile = wave >> 2;
  const int j0 = ug * kPFUnits + tile * kFUnits, b0 = rg * kFRows;  // the wave's tile
  const int r = lane & 15, q = lane >> 4;
  const int b = min(b0 + r, B - 1);
  const int kb = (wave & 3) * (H / 4) + 4 * q;  // this lane's offset in the wave's 64-long block
  const int64_t wr = (int64_t)((r >> 2) * H + j0 + (r & 3));  // weight row n(c) of column r

  // The wave's weights: lower W_hh1 (wa) and W_ih1 (wi, NI > 0); upper W_hh2
  // (wa) and W_ih2 (wb).
  f4 wa[4], wb[4], wi[NI > 0 ? NI : 1];
  const int kx = (wave & 3) * (16 * NI) + 4 * q;  // this lane's offset in the wave's x range
  {
    const float *srca = (upper ? p.whh2 : p.whh1) + wr * H + kb;
    const float *srcb = p.wih2 + wr * H + kb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wa[i] = *reinterpret_cast<const f4 *>(srca + 16 * i);
      wb[i] = upper ? *reinterpret_cast<const f4 *>(srcb + 16 * i) : f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int i = 0; i < NI; ++i)
      wi[i] = upper ? f4{0.0f, 0.0f, 0.0f, 0.0f}
                    : *reinterpret_cast<const f4 *>(p.wih1 + wr * (16 * NI * 4) + kx + 16 * i);
  }
  const int64_t hbytes = (int64_t)B * T * H * 4;
  const __amdgpu_buffer_rsrc_t rh1 = dev_rsrc(p.h1, hbytes), rh2 = dev_rsrc(p.h2, hbytes);
  // cell (em, eu) = (lane / 4, lane % 4) of the tile of wave 0 or wave 4
  const int em = lane >> 2, eu = lane & 3;
  const int be = b0 + em, je = j0 + eu;
  const bool epi = (wave & 3) == 0 && be < B;
  float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const float *bsrc = upper ? p.b2 : (NI > 0 ? p.b1 : nullptr);
  if (epi && bsrc != nullptr) {
#pragma unroll
    for (int g = 0; g < 4; ++g) bias[g] = bsrc[g * H + je];
  }
  float cst = 0.0f;  // the cell's state at its previous step (zero initial state)
  unsigned *lo_cnt = p.count + rg * ugroups;                       // the row group's lower
  unsigned *up_cnt = p.count + (rgroups + rg) * ugroups;           // and upper counters
  unsigned *mine = (upper ? up_cnt : lo_cnt) + ug;
  unsigned *abort_word = p.count + 2 * rgroups * ugroups;
  float *acts = upper ? p.acts2 : p.acts1;
  float *cs = upper ? p.c2 : p.c1;
  float *hs = upper ? p.h2 : p.h1;

  for (int t = 0; t < T; ++t) {
    float gin[4] = {bias[0], bias[1], bias[2], bias[3]};
    float act[4];
    const int64_t row = (int64_t)be * T + t;
    if (NI == 0 && epi && !upper) {
#pragma unroll
      for (int g = 0; g < 4; ++g) gin[g] = p.acts1[row * H4 + g * H + je];
    }
    // Lower: h1 at t - 1 done, then h1_{t-1} W_hh1^T.  Upper: first h1 at t
    // (the lower chain, which runs ahead) and h1_t W_ih2^T, whose MFMAs then
    // run during the second wait, for h2 at t - 1; then h2_{t-1} W_hh2^T onto
    // the same accumulator (the per-step kernels' order).  Every load is
    // issued before the MFMAs that wait on it (the scheduler would otherwise
    // issue later loads after earlier MFMAs, exposing their latencies one
    // after another).
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, accx = {0.0f, 0.0f, 0.0f, 0.0f};
    if (NI > 0 && !upper) {
      const float *xrow = p.x + ((int64_t)b * T + t) * (16 * NI * 4) + kx;
      f4 xa[NI > 0 ? NI : 1];
#pragma unroll
      for (int i = 0; i < NI; ++i) xa[i] = *reinterpret_cast<const f4 *>(xrow + 16 * i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          accx = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i][e], wi[i][e], accx, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (upper) {
      if (!await_step(lo_cnt, ugroups, (unsigned)(t + 1), lo_cnt, 0, 0u, abort_word, p.status,
                      p.spin, &s_go))
        return;
      const int off = (int)((((int64_t)b * T + t) * H + kb) * 4);
      f4 ai[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ai[i] = ld_dev4(rh1, off + 64 * i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ai[e >> 2][e & 3], wb[e >> 2][e & 3], acc, 0, 0,
                                                   0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (t > 0) {
      if (!await_step(upper ? up_cnt : lo_cnt, ugroups, (unsigned)t, lo_cnt, 0, 0u, abort_word,
                      p.status, p.spin, &s_go))
        return;
      const int off = (int)((((int64_t)b * T + t - 1) * H + kb) * 4);
      f4 ar[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ar[i] = ld_dev4(upper ? rh2 : rh1, off + 64 * i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ar[e >> 2][e & 3], wa[e >> 2][e & 3], acc, 0, 0,
                                                   0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      part[wave][4 * q + v][r] = acc[v];
      if (NI > 0 && !upper) partx[wave][4 * q + v][r] = accx[v];
    }
    __syncthreads();
    if (epi) {
      const int pw = 4 * tile;
      float pre[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = 4 * g + eu;
        if (NI > 0 && !upper)  // x W_ih1^T + b1, as the per-step kernels
          gin[g] = (((partx[pw][em][c] + partx[pw + 1][em][c]) + partx[pw + 2][em][c]) +
                    partx[pw + 3][em][c]) +
                   gin[g];
        pre[g] = gin[g] + (((part[pw][em][c] + part[pw + 1][em][c]) + part[pw + 2][em][c]) +
                           part[pw + 3][em][c]);
      }
      float c, h;
      cell_forward(pre, cst, act, c, h);
      cst = c;
      st_dev(hs + row * H + je, h);
    }
    publish_step(mine, (unsigned)(t + 1));
    // The saved gates and cell state are read only by the backward (a later
    // launch): stored after the step is published, so that its wait covers
    // only h; the next step's publish waits for them.
    if (epi) {
#pragma unroll
      for (int g = 0; g < 4; ++g) acts[row * H4 + g * H + je] = act[g];
      cs[row * H + je] = cst;
    }
  }
}

struct Lstm2Bwd {
  float *dG1, *dG2;                       // [B, T, 4H] gate gradients
  const float *whh1, *wih2, *whh2;        // [4H, H]
  const float *acts1, *c1, *acts2, *c2;   // forward's saved values
  const float *dh2;                       // [B, T, H] gradient at the upper h, or null
  float *up_in;   // [B, T, H] the lower layer's input-gradient term dG2_t W_ih2 per cell
  float *db1f, *db2f;  // [row groups, 4H] bias-gradient partials (tile_bias_partial), or null
  unsigned *count;  // [rgroups][3][H / kMUnits] steps done (upper, lower, helper), then abort
  int *status;
  int B, T;
  int spin;  // wait rounds before giving up
};

// Backward: workgroups [0, n) run the upper layer, [n, 2n) the lower one and
// [2n, 3n) help the lower one; workgroup (row group rg, unit group ug) owns
// rows b0..b0+15 and units j0..j0+15 (kMRows x kMUnits, as
// lstm_bwd_diag_mfma), its 16 waves each a sixteenth of a 4H-long reduction,
// threads 0..255 one cell each.  Step s runs t = T-1-s.  Upper: dh = dh2 +
// dG2_{t+1} W_hh2 (its own previous step).  Helper: dG2_t W_ih2 for its
// tile into up_in, as soon as the upper step s is done (the upper chain runs
// ahead).  Lower: dh = dG1_{t+1} W_hh1 (its own previous step) + up_in
// (the helper's step s), so the lower chain's own step carries one
// reduction, like the upper one.
__global__ void __launch_bounds__(1024) lstm2_bwd_persist(Lstm2Bwd p) {
  constexpr int H = kPersistH, H4 = 4 * H;
  constexpr int ugroups = H / kMUnits;
  __shared__ float part[kMWaves][16][16];
  __shared__ int s_go;
  const int B = p.B, T = p.T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per_layer = (int)gridDim.x / 3;
  const int role = (int)blockIdx.x / per_layer;  // 0 upper, 1 lower, 2 helper
  const int blk = (int)blockIdx.x - role * per_layer;
  const int ug = blk % ugroups, rg = blk / ugroups;
  const int j0 = ug * kMUnits, b0 = rg * kMRows;
  const int r = lane & 15, q = lane >> 4;
  const int b = min(b0 + r, B - 1);
  const int nb = wave * (H4 / kMWaves) + 4 * q;  // this lane's offset in the wave's 64-long block

  // B operands W[n][j0 + r] for n = nb + 16 i + e (strided loads, once):
  // upper W_hh2, lower W_hh1, helper W_ih2.
  f4 w[4];
  {
    const float *src = (role == 0 ? p.whh2 : role == 1 ? p.whh1 : p.wih2) + j0 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) w[i][e] = src[(int64_t)(nb + 16 * i + e) * H];
  }
  const int64_t gbytes = (int64_t)B * T * H4 * 4;
  // the reduction's operand rows: the layer's own dG (step t + 1), or the
  // helper's dG2 (step t)
  const __amdgpu_buffer_rsrc_t rsrc = dev_rsrc(role == 1 ? p.dG1 : p.dG2, gbytes);
  const int tid = threadIdx.x;
  const int em = tid >> 4, eu = tid & 15;
  const int be = b0 + em, je = j0 + eu;
  const bool epi = tid < 256 && be < B;
  float dcf = 0.0f;  // dc_{t+1} f_{t+1} of the cell (0 before its last step)
  // the cell's gate gradients summed over the steps (compensated)
  float dbs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, dbc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float *dbf = role == 0 ? p.db2f : role == 1 ? p.db1f : nullptr;
  const float *acts = role == 1 ? p.acts1 : p.acts2;
  const float *cs = role == 1 ? p.c1 : p.c2;
  float *dGo = role == 1 ? p.dG1 : p.dG2;
  unsigned *up_cnt = p.count + rg * 3 * ugroups;  // the row group's upper, lower, helper counters
  unsigned *lo_cnt = up_cnt + ugroups, *hp_cnt = lo_cnt + ugroups;
  unsigned *mine = up_cnt + role * ugroups + ug;
  unsigned *abort_word = p.count + gridDim.x;

  for (int s = 0; s < T; ++s) {
    const int t = T - 1 - s;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, c = 0.0f, cp = 0.0f, dho = 0.0f;
    const int64_t row = (int64_t)be * T + t;
    if (epi && role != 2) {
#pragma unroll
      for (int g = 0; g < 4; ++g) a[g] = acts[row * H4 + g * H + je];
      c = cs[row * H + je];
      cp = t > 0 ? cs[(row - 1) * H + je] : 0.0f;
      if (role == 0 && p.dh2 != nullptr) dho = p.dh2[row * H + je];
    }
    // upper: its step s - 1; lower: its step s - 1 and the helper's step s;
    // helper: the upper step s
    bool go = true;
    if (role == 0) {
      if (s > 0)
        go = await_step(up_cnt, ugroups, (unsigned)s, up_cnt, 0, 0u, abort_word, p.status,
                        p.spin, &s_go);
    } else if (role == 1) {
      go = await_step(lo_cnt, s > 0 ? ugroups : 0, (unsigned)s, hp_cnt + ug, 1, (unsigned)(s + 1),
                      abort_word, p.status, p.spin, &s_go);
    } else {
      go = await_step(up_cnt, ugroups, (unsigned)(s + 1), up_cnt, 0, 0u, abort_word, p.status,
                      p.spin, &s_go);
    }
    if (!go) return;
    const bool red = role == 2 || s > 0;  // this step has a reduction
    f4 d[4];
    if (red) {
      const int off = (int)((((int64_t)b * T + (role == 2 ? t : t + 1)) * H4 + nb) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) d[i] = ld_dev4(rsrc, off + 64 * i);
    }
    float upin = 0.0f;
    if (epi && role == 1)
      upin = __hip_atomic_load(p.up_in + row * H + je, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first MFMA waits on one
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (red) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(d[e >> 2][e & 3], w[e >> 2][e & 3], acc, 0, 0,
                                                   0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wave][4 * q + v][r] = acc[v];
    __syncthreads();
    if (epi) {
      float sum = part[0][em][eu];
#pragma unroll
      for (int k = 1; k < kMWaves; ++k) sum += part[k][em][eu];
      if (role == 2) {
        st_dev(p.up_in + row * H + je, sum);
      } else {
        if (role == 1) sum = sum + upin;  // (dh2 is null for the lower layer)
        float dg[4];
        cell_backward(a, c, cp, dho + sum, dcf, dg, dcf);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          st_dev(dGo + row * H4 + g * H + je, dg[g]);
          kahan_add(dbs[g], dbc[g], dg[g]);
        }
      }
    }
    publish_step(mine, (unsigned)(s + 1));
  }
  if (dbf != nullptr) {  // every thread of the block is here (part is free after the last publish)
    float(*lds)[16][16] = part;
    if (tid < 256) {
#pragma unroll
      for (int g = 0; g < 4; ++g) lds[g][em][eu] = epi ? dbs[g] - dbc[g] : 0.0f;
    }
    tile_bias_partial(lds, dbf + (int64_t)rg * H4, H, j0);
  }
}

// Sets n 32-bit words at p to `bits` (the persistent kernels' counters).
__global__ void __launch_bounds__(256) fill_bits(unsigned *__restrict__ p, int64_t n, unsigned bits) {
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (; i < n; i += stride) p[i] = bits;
}

int fill_words(numrs_hip_ctx *ctx, void *p, int64_t n, unsigned bits) {
  unsigned grid = grid_for(n, 256);
  if (grid > 8192) grid = 8192;
  fill_bits<<<grid, 256, 0, ctx->stream>>>(static_cast<unsigned *>(p), n, bits);
  return numrs_hip::check_launch(ctx, "fill_bits");
}

// Whether a persistent kernel's grid can run this call: the context allows
// it, no graph is being recorded, the device holds `grid` workgroups of
// `threads` at once (resident workgroups per CU cached in *per_cu), and, in
// COOPERATIVE mode, the device supports cooperative launches.
bool persist_fits(numrs_hip_ctx *ctx, const void *kernel, int threads, unsigned grid,
                  int *per_cu) {
  if (ctx->capturing || ctx->recurrence_mode == NUMRS_HIP_RECURRENCE_PER_STEP) return false;
  if (*per_cu < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    *per_cu = n;
  }
  if (ctx->recurrence_mode == NUMRS_HIP_RECURRENCE_COOPERATIVE) {
    int coop = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, ctx->device) !=
        hipSuccess) {
      (void)hipGetLastError();
      coop = 0;
    }
    if (!coop) return false;
  }
  return (int64_t)*per_cu * ctx->num_cus >= (int64_t)grid;
}

// The persistent forward kernel for NI = I / 64 input blocks per wave (0:
// the input projection is formed before the launch).
const void *persist_fwd_kernel(int ni) {
  switch (ni) {
    case 1: return reinterpret_cast<const void *>(lstm2_fwd_persist<1>);
    case 2: return reinterpret_cast<const void *>(lstm2_fwd_persist<2>);
    case 3: return reinterpret_cast<const void *>(lstm2_fwd_persist<3>);
    case 4: return reinterpret_cast<const void *>(lstm2_fwd_persist<4>);
    default: return reinterpret_cast<const void *>(lstm2_fwd_persist<0>);
  }
}

// Wait rounds before a persistent kernel's wait gives up.
int wait_limit(const numrs_hip_ctx *ctx) {
  return ctx->persist_wait_limit >= 0 ? ctx->persist_wait_limit : kSpinLimit;
}

// Step counters (one per workgroup) and the abort word after them, zeroed,
// from the context's block cache, and the status word of one persistent
// launch.
int persist_words(numrs_hip_ctx *ctx, numrs_hip::TempBlock &cnt, unsigned grid, int **status,
                  bool zero = true) {
  if (int rc = numrs_hip::wait_status_word(ctx, status)) return rc;
  if (int rc = cnt.alloc((size_t)(grid + 1) * sizeof(unsigned))) return rc;
  return zero ? fill_words(ctx, cnt.p, (int64_t)grid + 1, 0u) : NUMRS_HIP_OK;
}

template <typename Args>
int launch_persist(numrs_hip_ctx *ctx, const void *kernel, unsigned grid, int threads, Args a,
                   const char *what) {
  void *args[] = {&a};
  const bool coop = ctx->recurrence_mode == NUMRS_HIP_RECURRENCE_COOPERATIVE;
  const hipError_t e =
      coop ? hipLaunchCooperativeKernel(kernel, dim3(grid), dim3(threads), args, 0, ctx->stream)
           : hipLaunchKernel(kernel, dim3(grid), dim3(threads), args, 0, ctx->stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return numrs_hip::fail(ctx, NUMRS_HIP_E_HIP, "%s launch of %s failed: %s",
                           coop ? "cooperative" : "persistent", what, hipGetErrorString(e));
  }
  ctx->wait_check = true;
  ++ctx->persist_launches;
  return NUMRS_HIP_OK;
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

// Before the persistent backward, in one launch: H_prev of both layers
// (blocks [0, rows) shift h1 into hp1, [rows, 2 rows) h2 into hp2, as
// shift_hidden_rows with zero initial states) and, in the last block, the
// launch's ncnt step counters and abort word zeroed.
__global__ void __launch_bounds__(64)
    lstm2_bwd_prep(const float *__restrict__ h1, float *__restrict__ hp1,
                   const float *__restrict__ h2, float *__restrict__ hp2, int T, int H,
                   int64_t rows, unsigned *__restrict__ cnt, int ncnt) {
  int64_t r = blockIdx.x;
  if (r == 2 * rows) {
    for (int i = threadIdx.x; i < ncnt; i += 64) cnt[i] = 0u;
    return;
  }
  const bool upper = r >= rows;
  if (upper) r -= rows;
  const float *h = upper ? h2 : h1;
  float *out = upper ? hp2 : hp1;
  const int t = (int)(r % T);
  for (int c = 4 * threadIdx.x; c < H; c += 4 * 64) {
    const f4 v = t > 0 ? *reinterpret_cast<const f4 *>(h + (r - 1) * H + c)
                       : f4{0.0f, 0.0f, 0.0f, 0.0f};
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
// H_prev[b, t] = h[b, t - 1] (h0, or zero, at t = 0) into hp [B*T, H].
int shift_rows(numrs_hip_ctx *ctx, const float *h_seq, const float *h0, float *hp, int64_t B,
               int64_t T, int64_t H) {
  const int64_t rows = B * T;
  if (H % 4 == 0 && numrs_hip::aligned16(h_seq) && numrs_hip::aligned16(hp) &&
      (h0 == nullptr || numrs_hip::aligned16(h0)) && rows <= 0x7fffffff) {
    shift_hidden_rows<<<(unsigned)rows, 64, 0, ctx->stream>>>(h_seq, h0, hp, (int)T, (int)H);
  } else {
    shift_hidden<<<grid_for(rows * H, 256), 256, 0, ctx->stream>>>(h_seq, h0, hp, (int)B, (int)T,
                                                                   (int)H);
  }
  return numrs_hip::check_launch(ctx, "shift_hidden");
}

// db_part (may be null): [db_rows, 4H] sums of dG over the steps and the
// rows of each row group (the step kernels' compensated sums), from which db
// is the sum over the groups.  hp_given (may be null): H_prev already formed.
int lstm_param_grads(numrs_hip_ctx *ctx, const float *dG, const float *x, const float *w_ih,
                     const float *h_seq, const float *h0, float *dx, float *dw_ih, float *dw_hh,
                     float *db, int64_t B, int64_t T, int64_t I, int64_t H, int acc_dx,
                     int acc_dw_ih, int acc_dw_hh, int acc_db, const float *db_part = nullptr,
                     int64_t db_rows = 0, const float *hp_given = nullptr) {
  const int64_t rows = B * T, H4 = 4 * H;
  if (dw_ih && dw_hh && rows > 0 && I > 0) {
    // dW_ih[4H, I] = dG^T x and dW_hh[4H, H] = dG^T H_prev in one launch
    // (both read dG), db = column sums of dG in the launch reducing their
    // splits
    TempBlock hp(ctx);
    if (hp_given == nullptr) {
      if (int rc = hp.alloc((size_t)(rows * H) * sizeof(float))) return rc;
      if (int rc = shift_rows(ctx, h_seq, h0, hp.f(), B, T, H)) return rc;
    }
    if (int rc = numrs_hip::gemm_tn2_colsum(ctx, dG, H4, rows, H4, x, I, I, dw_ih, acc_dw_ih,
                                            hp_given ? hp_given : hp.f(), H, H, dw_hh, acc_dw_hh,
                                            db, acc_db, db_part, db_rows))
      return rc;
    dw_ih = dw_hh = db = nullptr;
  }
  if (dw_ih)  // dW_ih[4H, I] = dG^T x
    if (int rc = numrs_hip_gemm(ctx, dG, H4, x, I, dw_ih, I, H4, rows, I, 1, 0, 1.0f, acc_dw_ih,
                                1, 1, 0, 0, 0, 0, 0, 0))
      return rc;
  if (dw_hh) {  // dW_hh[4H, H] = dG^T H_prev
    TempBlock hp(ctx);
    if (int rc = hp.alloc((size_t)(rows * H) * sizeof(float))) return rc;
    if (int rc = shift_rows(ctx, h_seq, h0, hp.f(), B, T, H)) return rc;
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
  // The lower layer reduces x_t against W_ih1 inside its steps where I is a
  // multiple of 64 up to 256; otherwise acts1 <- x W_ih1^T + b1 for every
  // (b, t) row first.  The upper layer reduces h1 against W_ih2 inside its
  // steps.
  const bool in_x = I % 64 == 0 && I <= 256 && numrs_hip::aligned16(x) &&
                    numrs_hip::aligned16(w_ih1);
  if (!in_x)
    if (int rc = numrs_hip_linear_forward(ctx, x, w_ih1, b1, acts1, B * T, I, 4 * H1)) return rc;
  const int rgroups = (int)((B + kFRows - 1) / kFRows);
  if (H1 == kPersistH && H2 == kPersistH && B * T * H1 * 4 < (int64_t{1} << 31)) {
    const unsigned grid = (unsigned)(2 * rgroups * (kPersistH / kPFUnits));
    const void *kern = in_x ? persist_fwd_kernel((int)(I / 64)) : persist_fwd_kernel(0);
    int *per_cu = &ctx->persist_fwd_per_cu[in_x ? I / 64 : 0];
    if (persist_fits(ctx, kern, 512, grid, per_cu)) {
      TempBlock cnt(ctx);
      int *status = nullptr;
      if (int rc = persist_words(ctx, cnt, grid, &status)) return rc;
      Lstm2Fwd a{acts1, acts2, w_hh1, w_ih2, w_hh2, b2, in_x ? x : nullptr, w_ih1, b1,
                 h1_seq, c1_seq, h2_seq, c2_seq, static_cast<unsigned *>(cnt.p), status,
                 (int)B, (int)T, wait_limit(ctx)};
      return launch_persist(ctx, kern, grid, 512, a, "lstm2_fwd_persist");
    }
  }
  FwdStep lo{acts1, w_hh1, in_x ? x : nullptr, in_x ? w_ih1 : nullptr, in_x ? b1 : nullptr,
             nullptr, nullptr, h1_seq, c1_seq, (int)H1, in_x ? (int)I : 0, 0, in_x ? 1 : 0};
  FwdStep up{acts2, w_hh2, h1_seq, w_ih2, b2, nullptr, nullptr, h2_seq, c2_seq, (int)H2, (int)H1,
             0};
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
  // The bias gradients from per-row-group partials [row groups, 4H] that the
  // MFMA step kernels (persistent or per step) form as they go (the per-step
  // launches keep their running sums in [2][B, 4H] first).
  TempBlock db1p(ctx), db2p(ctx), db1f(ctx), db2f(ctx);
  const bool mfma = H1 % 256 == 0 && H2 % 256 == 0;
  const int64_t mgroups = (B + kMRows - 1) / kMRows;
  if (mfma && db1 != nullptr) {
    if (int rc = db1p.alloc((size_t)(2 * B * 4 * H1) * sizeof(float))) return rc;
    if (int rc = db1f.alloc((size_t)(mgroups * 4 * H1) * sizeof(float))) return rc;
  }
  if (mfma && db2 != nullptr) {
    if (int rc = db2p.alloc((size_t)(2 * B * 4 * H2) * sizeof(float))) return rc;
    if (int rc = db2f.alloc((size_t)(mgroups * 4 * H2) * sizeof(float))) return rc;
  }
  if (H1 == kPersistH && H2 == kPersistH && B * T * 4 * H1 * 4 < (int64_t{1} << 31)) {
    const unsigned grid = (unsigned)(3 * ((B + kMRows - 1) / kMRows) * (kPersistH / kMUnits));
    if (persist_fits(ctx, reinterpret_cast<const void *>(lstm2_bwd_persist), 1024, grid,
                     &ctx->persist_bwd_per_cu)) {
      // H_prev of both layers for the weight gradients and the counters'
      // zeroing in one launch ahead of the recurrence
      const int64_t rows = B * T;
      TempBlock hp1(ctx), hp2(ctx);
      const bool prep = numrs_hip::aligned16(h1_seq) && numrs_hip::aligned16(h2_seq) &&
                        2 * rows + 1 <= 0x7fffffff;
      if (prep) {
        if (int rc = hp1.alloc((size_t)(rows * H1) * sizeof(float))) return rc;
        if (int rc = hp2.alloc((size_t)(rows * H2) * sizeof(float))) return rc;
      }
      {
        TempBlock cnt(ctx), up_in(ctx);
        int *status = nullptr;
        if (int rc = persist_words(ctx, cnt, grid, &status, !prep)) return rc;
        if (prep) {
          lstm2_bwd_prep<<<(unsigned)(2 * rows + 1), 64, 0, ctx->stream>>>(
              h1_seq, hp1.f(), h2_seq, hp2.f(), (int)T, (int)H1, rows,
              static_cast<unsigned *>(cnt.p), (int)grid + 1);
          if (int rc = numrs_hip::check_launch(ctx, "lstm2_bwd_prep")) return rc;
        }
        if (int rc = up_in.alloc((size_t)(B * T * H1) * sizeof(float))) return rc;
        Lstm2Bwd a{dG1.f(), dG2.f(), w_hh1, w_ih2, w_hh2, acts1, c1_seq, acts2, c2_seq, dh2_seq,
                   up_in.f(), db1f.f(), db2f.f(), static_cast<unsigned *>(cnt.p), status,
                   (int)B, (int)T, wait_limit(ctx)};
        if (int rc = launch_persist(ctx, reinterpret_cast<const void *>(lstm2_bwd_persist), grid,
                                    1024, a, "lstm2_bwd_persist"))
          return rc;
      }
      if (int rc = lstm_param_grads(ctx, dG2.f(), h1_seq, w_ih2, h2_seq, nullptr, nullptr, dw_ih2,
                                    dw_hh2, db2, B, T, H1, H2, 0, acc_dw_ih2, acc_dw_hh2, acc_db2,
                                    db2f.f(), mgroups, hp2.f()))
        return rc;
      return lstm_param_grads(ctx, dG1.f(), x, w_ih1, h1_seq, nullptr, dx, dw_ih1, dw_hh1, db1, B,
                              T, I, H1, acc_dx, acc_dw_ih1, acc_dw_hh1, acc_db1, db1f.f(),
                              mgroups, hp1.f());
    }
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
  // MFMA steps when both layers' reductions split into 64-long wave blocks.
  BwdStep up{dG2.f(), wt2.f(), acts2, c2_seq, nullptr, dh2_seq, nullptr, nullptr, dc2.f(),
             (int)H2, 0, 0, mfma ? db2p.f() : nullptr, db2f.f()};
  BwdStep lo{dG1.f(), wt1.f(), acts1, c1_seq, nullptr, nullptr, dG2.f(), wtu.f(), dc1.f(),
             (int)H1, (int)H2, 0, mfma ? db1p.f() : nullptr, db1f.f()};
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
                                dw_hh2, db2, B, T, H1, H2, 0, acc_dw_ih2, acc_dw_hh2, acc_db2,
                                db2f.f(), mgroups))
    return rc;
  return lstm_param_grads(ctx, dG1.f(), x, w_ih1, h1_seq, nullptr, dx, dw_ih1, dw_hh1, db1, B, T,
                          I, H1, acc_dx, acc_dw_ih1, acc_dw_hh1, acc_db1, db1f.f(), mgroups);
}

int numrs_hip_set_recurrence_mode(numrs_hip_ctx *ctx, int mode) {
  NRS_CHECK_CTX(ctx);
  if (mode != NUMRS_HIP_RECURRENCE_AUTO && mode != NUMRS_HIP_RECURRENCE_PER_STEP &&
      mode != NUMRS_HIP_RECURRENCE_PLAIN_LAUNCH && mode != NUMRS_HIP_RECURRENCE_COOPERATIVE)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "recurrence mode %d", mode);
  ctx->recurrence_mode = mode;
  return NUMRS_HIP_OK;
}

int numrs_hip_set_persistent_wait_limit(numrs_hip_ctx *ctx, int rounds) {
  NRS_CHECK_CTX(ctx);
  ctx->persist_wait_limit = rounds < 0 ? -1 : rounds;
  return NUMRS_HIP_OK;
}

int64_t numrs_hip_persistent_launches(numrs_hip_ctx *ctx) {
  return ctx == nullptr ? -1 : ctx->persist_launches;
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
