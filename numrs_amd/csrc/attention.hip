// Multi-head attention forward / backward for the transformer configuration
// (no reference op: numrs has no attention and a 2-D-only matmul,
// backward.rs:118-120).  q, k, v, out are [batch*seq, heads*dh] row-major --
// head h of token (b, s) is the dh-slice starting at column h*dh -- so every
// per-(b,h) matrix is addressed in place through the GEMM's two batch levels
// (z = b*heads + h) with leading dimension heads*dh.  P holds the softmax
// probabilities [batch*heads, seq, seq] saved by the forward.
//
//   forward:   S = alpha * Q K^T,  P = softmax_rows(S),  O = P V
//   backward:  dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dP*P)),
//              dQ = alpha * dS K,  dK = alpha * dS^T Q
// with alpha = 1/sqrt(dh), all products fp32 MFMAs.  For dh = 64 and S = 128
// or 256 the forward is one kernel and the backward given the forward's output
// two (waves owning whole query rows, then whole key rows); dh = 64 with S =
// 384 or 512 takes the four-wave row-block kernels; other shapes the batched
// GEMMs and the one-wave-per-row softmax kernels.
#include <cmath>

#include "common.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kRowsPerBlock = 64;  // query rows per workgroup (two 32-row MFMA blocks)
constexpr int kHeadDim = 64;       // dh handled by the fused row-block kernel

// Row-block attention kernel.  One workgroup computes the [64, S] block
// Y = X_z W_z^T of head z (rows row0..row0+63 of X, all S rows of W, reduction
// over dh = 64) with fp32 MFMA, then finishes each row from the registers:
//   MODE 0 (forward):  out = softmax_rows(alpha * Y)            (P)
//   MODE 1 (backward): out = P * (Y - rowsum(Y * P)), Y = dO V^T  (dS)
// so neither S nor dP makes a round trip through HBM.  Wave w owns columns
// [w*S/4, (w+1)*S/4), BJ = S/128 blocks of 32.  Operand fragments are read
// from global memory in the MFMA lane layout: lane (c, h) holds reduction
// indices 8g + 4h + j (j = 0..3) of row c, fed to four 32x32x2 MFMAs.  The
// MFMAs compute Y^T (W as the A operand), so lane (c, h) holds row c of each
// 32-row block at 16 columns: a row's max or sum is a sum over the lane's
// registers, one xor-32 shuffle and the four waves in a fixed order through
// LDS, and its four consecutive columns per register quad leave as one
// 16-byte store.  The softmax is the row kernel's in base 2: s = alpha
// log2(e) y, m = max, e = 2^(s - m) (one v_exp_f32), P = e * (1/sum e).
//
// With EXTRA the kernel also multiplies the finished rows by E_z, the head's
// [S, 64] block of a third matrix, into eo (row stride ldo):
//   MODE 0: eo = P V                       (E = V; the attention output)
//   MODE 1: eo (+)= ealpha * dS K          (E = K; the query gradient)
// The rows already sit in the lane layout of an MFMA operand: register
// 4g + e of block (bi, bj) is element (query 32bi + c, key 32bj + 8g + 4h +
// e), so eo^T = E^T Y^T runs as 32x32x2 MFMAs with that register as B and
// E[key][d] as A, each wave reducing over its own S/4 keys.  A wave stages
// its keys' rows of E in LDS ([key][64], the 16-byte chunks of rows whose
// bit 2 is set XOR-ed by 8 so that the two half-waves' rows fall in
// different banks): the forward for S <= 256 through registers loaded before
// its first MFMAs, otherwise by DMA at the start.  The four wave partials then
// meet in LDS (rows padded to
// 68 floats) and are added in wave order, each thread finishing 16
// consecutive outputs of one row with float4 loads and stores.
constexpr int kPartStride = 68;  // floats per row of a wave's [64, 64] partial in LDS

template <int BJ>
constexpr int extra_lds_floats() {
  return 4 * kRowsPerBlock * kPartStride > 4 * 32 * BJ * kHeadDim ? 4 * kRowsPerBlock * kPartStride
                                                                   : 4 * 32 * BJ * kHeadDim;
}

template <int MODE, int BJ, bool EXTRA>
__global__ void __launch_bounds__(256) attn_rows_kernel(const float *__restrict__ X,
                                                        const float *__restrict__ W,
                                                        const float *__restrict__ P,
                                                        float *__restrict__ out, int S, int H,
                                                        int64_t ldx, int64_t ldw, float alpha,
                                                        const float *__restrict__ E, int64_t lde,
                                                        float *eo, int64_t ldo, float ealpha,
                                                        int eacc) {
  __shared__ float red[4][kRowsPerBlock];
  __shared__ __attribute__((aligned(1024))) float ebuf[EXTRA ? extra_lds_floats<BJ>() : 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hh = lane >> 5;
  // gfx950 dispatches workgroup L (x fastest) to XCD L % 8.  The logical
  // block (row block, head) is permuted so that XCD k owns a contiguous run
  // of heads with all their row blocks: the blocks of a head, which read the
  // same S rows of W and E, then share one XCD's L2.
  int rb = blockIdx.x, z = blockIdx.y;
  {
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      rb = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int row0 = rb * kRowsPerBlock, col0 = wave * 32 * BJ;
  const float *Xz = X + (int64_t)b * S * ldx + (int64_t)head * kHeadDim;
  const float *Wz = W + (int64_t)b * S * ldw + (int64_t)head * kHeadDim;
  const int64_t zoff = (int64_t)z * S * S;
  constexpr int kStage = 8 * BJ;  // DMA instructions per wave (4 rows of E each)
  float *wbuf = ebuf + wave * (32 * BJ * kHeadDim);

  // The wave's S/4 rows of E go to LDS by DMA before anything else (no
  // registers held, complete long before the second product needs them):
  // instruction it writes rows 4 it .. 4 it + 3 of the wave's keys, lane l
  // the 16-byte slot l % 16 of row 4 it + l / 16, which holds chunk
  // (l % 16) ^ 8 of rows whose bit 2 is set.
  // The forward for S <= 256 stages through registers instead: its E loads go
  // out first and are written to LDS after the Q K^T MFMAs (the same layout).
  constexpr bool kRegStage = EXTRA && MODE == 0 && BJ <= 2;
  f4 stage[kRegStage ? kStage : 1];
  if constexpr (kRegStage) {
    const float *Ez = E + (int64_t)b * S * lde + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < kStage; ++it)
      stage[it] = *reinterpret_cast<const f4 *>(
          Ez + (int64_t)(col0 + 4 * it + (lane >> 4)) * lde + 4 * (lane & 15));
  } else if constexpr (EXTRA) {
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const float *Ez = E + ((int64_t)b * S + (int64_t)wave_u * 32 * BJ) * lde +
                      (int64_t)head * kHeadDim;
    const uint32_t lds0 = (uint32_t)(uintptr_t)ebuf + (uint32_t)wave_u * (32 * BJ * kHeadDim * 4);
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int chunk = (lane & 15) ^ (8 * ((kk >> 2) & 1));
      numrs_hip::lds_dma16(Ez, (uint32_t)(4 * ((int64_t)kk * lde + 4 * chunk)), lds0 + 1024u * it);
    }
  }

  // Register i of block (bi, bj) holds row row0 + 32*bi + c and column
  // col0 + 32*bj + 8*(i/4) + 4*hh + (i%4).
  auto col_of = [&](int bj, int i4) { return col0 + 32 * bj + 8 * i4 + 4 * hh; };
  auto row_ptr = [&](float *base, int bi) { return base + zoff + (int64_t)(row0 + 32 * bi + c) * S; };
  // The backward's P block (read from HBM): for S <= 256 its loads go out
  // before the dO V^T MFMAs, which then cover their latency.
  constexpr bool kEarlyP = MODE == 1 && BJ <= 2;
  f4 p[MODE == 1 ? 2 : 1][MODE == 1 ? BJ : 1][4];
  auto load_p = [&]() {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const float *src = row_ptr(const_cast<float *>(P), bi);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          p[bi][bj][i4] = *reinterpret_cast<const f4 *>(src + col_of(bj, i4));
    }
  };
  if constexpr (kEarlyP) {
    load_p();
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
  }

  f16v acc[2][BJ];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = f16v{};
#pragma unroll
  for (int g = 0; g < kHeadDim / 8; ++g) {
    f4 a[2], w[BJ];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
      a[bi] = *reinterpret_cast<const f4 *>(Xz + (int64_t)(row0 + 32 * bi + c) * ldx + 8 * g + 4 * hh);
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
      w[bj] = *reinterpret_cast<const f4 *>(Wz + (int64_t)(col0 + 32 * bj + c) * ldw + 8 * g + 4 * hh);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < BJ; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[bj][j], a[bi][j], acc[bi][bj], 0, 0, 0);
  }

  // Row totals over the wave's columns (in-lane, then the other half-wave),
  // then over the four waves: op 0 = max, 1 = sum.
  auto row_reduce = [&](float (&v)[2], int op) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      v[bi] = op == 0 ? half_pair(v[bi], [](float x, float y) { return fmaxf(x, y); })
                      : half_pair(v[bi], [](float x, float y) { return x + y; });
      if (hh == 0) red[wave][32 * bi + c] = v[bi];
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const int r = 32 * bi + c;
      v[bi] = op == 0 ? fmaxf(fmaxf(red[0][r], red[1][r]), fmaxf(red[2][r], red[3][r]))
                      : ((red[0][r] + red[1][r]) + red[2][r]) + red[3][r];
    }
    __syncthreads();
  };

  if constexpr (kRegStage) {
    // visible to the wave's reads after the row reductions' barriers below
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int slot = (lane & 15) ^ (8 * ((kk >> 2) & 1));
      *reinterpret_cast<f4 *>(wbuf + kk * kHeadDim + 4 * slot) = stage[it];
    }
  }

  float t[2];
  if constexpr (MODE == 0) {
    // Softmax in base 2: the scores scaled by alpha log2(e), then 2^(s - m)
    // is one v_exp_f32 (within a few ulp of expf(alpha (y - max y)), which
    // took a dozen instructions per score and half of this phase).
    const float alpha_l2e = alpha * 1.44269504088896341f;
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float m = -INFINITY;
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          acc[bi][bj][i] = alpha_l2e * acc[bi][bj][i];
          m = fmaxf(m, acc[bi][bj][i]);
        }
      t[bi] = m;
    }
    row_reduce(t, 0);
    float sum[2];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float s = 0.0f;
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = __builtin_amdgcn_exp2f(acc[bi][bj][i] - t[bi]);
          acc[bi][bj][i] = e;
          s += e;
        }
      sum[bi] = s;
    }
    row_reduce(sum, 1);
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const float inv = 1.0f / sum[bi];
      float *dst = row_ptr(out, bi);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          f4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc[bi][bj][4 * i4 + e] * inv;
            acc[bi][bj][4 * i4 + e] = v[e];
          }
          *reinterpret_cast<f4 *>(dst + col_of(bj, i4)) = v;
        }
    }
  } else {
    if constexpr (!kEarlyP) load_p();
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float s = 0.0f;
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[bi][bj][i] * p[bi][bj][i >> 2][i & 3];
      t[bi] = s;
    }
    row_reduce(t, 1);
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float *dst = row_ptr(out, bi);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          f4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = p[bi][bj][i4][e] * (acc[bi][bj][4 * i4 + e] - t[bi]);
            acc[bi][bj][4 * i4 + e] = v[e];
          }
          *reinterpret_cast<f4 *>(dst + col_of(bj, i4)) = v;
        }
    }
  }

  if constexpr (EXTRA) {
    // eo^T partial over the wave's keys: block (bd, bi) holds d rows
    // 32bd + 8(i/4) + 4hh + (i%4) of query 32bi + c.  The staged row of key
    // 32bj + 8g + 4hh + e has its chunks XOR-ed by 8 exactly when hh = 1.
    if constexpr (!kRegStage)
      __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(0));  // the wave's DMA has landed
    f16v o[2][2];
#pragma unroll
    for (int bd = 0; bd < 2; ++bd)
#pragma unroll
      for (int bi = 0; bi < 2; ++bi) o[bd][bi] = f16v{};
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float *er = wbuf + (32 * bj + 8 * g + 4 * hh + e) * kHeadDim + c;
          const float ev[2] = {er[32 * hh], er[32 * (1 - hh)]};
#pragma unroll
          for (int bd = 0; bd < 2; ++bd)
#pragma unroll
            for (int bi = 0; bi < 2; ++bi)
              o[bd][bi] = __builtin_amdgcn_mfma_f32_32x32x2f32(ev[bd], acc[bi][bj][4 * g + e],
                                                               o[bd][bi], 0, 0, 0);
        }
    __syncthreads();  // every wave is done with its staged rows
    float *part = ebuf + wave * (kRowsPerBlock * kPartStride);
#pragma unroll
    for (int bd = 0; bd < 2; ++bd)
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const f4 v = {o[bd][bi][4 * i4], o[bd][bi][4 * i4 + 1], o[bd][bi][4 * i4 + 2],
                        o[bd][bi][4 * i4 + 3]};
          *reinterpret_cast<f4 *>(part + (32 * bi + c) * kPartStride + 32 * bd + 8 * i4 + 4 * hh) = v;
        }
    __syncthreads();
    const int q = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * 16;
    float *dst = eo + (int64_t)(b * S + row0 + q) * ldo + (int64_t)head * kHeadDim + d0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = q * kPartStride + d0 + 4 * j;
      const f4 s0 = *reinterpret_cast<const f4 *>(ebuf + off);
      const f4 s1 = *reinterpret_cast<const f4 *>(ebuf + kRowsPerBlock * kPartStride + off);
      const f4 s2 = *reinterpret_cast<const f4 *>(ebuf + 2 * kRowsPerBlock * kPartStride + off);
      const f4 s3 = *reinterpret_cast<const f4 *>(ebuf + 3 * kRowsPerBlock * kPartStride + off);
      f4 v = ((s0 + s1) + s2) + s3;
      if constexpr (MODE == 1) {
        v = ealpha * v;
        if (eacc) v = *reinterpret_cast<const f4 *>(dst + 4 * j) + v;
      }
      *reinterpret_cast<f4 *>(dst + 4 * j) = v;
    }
  }
}

// Row-block kernel for the backward's dS and dQ at S <= 256 (BJ = S/128 key
// blocks of 32 per wave): the arithmetic of attn_rows_kernel<1, BJ, true> in
// an order that lets the loads overlap the MFMAs (the forward at these
// lengths is attn_fwd_wave_rows_kernel):
//   1. The wave's 16 of the block's 64 rows of X and its S/4 rows of W go to
//      LDS by DMA, then the P block is loaded into registers.  Only
//      the X rows and the first 32 W rows are waited for (vmcnt counts in
//      issue order); the wave's rows of E are loaded into registers after
//      that, so the next W rows, P and E arrive during the product.
//   2. Y = X W^T from LDS: rows at 256 bytes, the 16-byte chunk j of row r
//      stored at slot j ^ (r % 16), so the lanes reading one chunk of 16
//      consecutive rows touch 16 different slots.
//   3. The softmax backward as in attn_rows_kernel, the row totals through
//      `red`, which reuses the X rows' space once every wave is past the
//      product; the dS rows are stored.
//   4. E goes from registers into the wave's own W rows (the layout of
//      attn_rows_kernel's staged E) and eo = E^T-product follows as there,
//      with the wave partials summed in wave order.
// Shared memory: four wave slots of S/4 rows of 64 floats and the 64 X rows:
// 80 KiB at S = 256, two workgroups per CU.
template <int BJ>
constexpr int lds_kernel_floats() {
  return 4 * 32 * BJ * kHeadDim + kRowsPerBlock * kHeadDim > 4 * kRowsPerBlock * kPartStride
             ? 4 * 32 * BJ * kHeadDim + kRowsPerBlock * kHeadDim
             : 4 * kRowsPerBlock * kPartStride;
}

template <int MODE, int BJ>
__global__ void __launch_bounds__(256, 2) attn_rows_lds_kernel(
    const float *__restrict__ X, const float *__restrict__ W, const float *__restrict__ P,
    float *__restrict__ out, int S, int H, int64_t ldx, int64_t ldw, float alpha,
    const float *__restrict__ E, int64_t lde, float *eo, int64_t ldo, float ealpha, int eacc) {
  static_assert(BJ == 1 || BJ == 2, "S <= 256");
  static_assert(MODE == 1, "the softmax backward");
  constexpr int kSlot = 32 * BJ * kHeadDim;  // floats of one wave's key rows
  constexpr int kXRows = 4 * kSlot;          // offset of the X rows
  __shared__ __attribute__((aligned(1024))) float lds[lds_kernel_floats<BJ>()];
  float(*red)[kRowsPerBlock] = reinterpret_cast<float(*)[kRowsPerBlock]>(lds + kXRows);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hh = lane >> 5;
  int rb = blockIdx.x, z = blockIdx.y;
  {
    // XCD k (hardware ids k, k+8, ...) owns a contiguous run of heads
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      rb = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int row0 = rb * kRowsPerBlock, col0 = wave * 32 * BJ;
  const int64_t zoff = (int64_t)z * S * S;
  float *wbuf = lds + wave * kSlot;

  // 1. DMA: instruction it fills rows 4 it .. 4 it + 3 (1 KiB), lane l the
  // 16-byte slot l % 16 of row 4 it + l / 16 with chunk slot ^ (row % 16).
  // The X rows go first, then the wave's W rows in key order: the first 32
  // keys' products start while the next 32 keys' rows are still arriving.
  {
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t base = (uint32_t)(uintptr_t)lds;
    const float *Xw = X + ((int64_t)b * S + row0 + 16 * wave_u) * ldx + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int kk = 4 * it + (lane >> 4);  // row 16 wave + kk of the block; (16 wave + kk) % 16 = kk
      const int chunk = (lane & 15) ^ kk;
      numrs_hip::lds_dma16(Xw, (uint32_t)(4 * ((int64_t)kk * ldx + 4 * chunk)),
                           base + 4u * (uint32_t)(kXRows + wave_u * 16 * kHeadDim) + 1024u * it);
    }
    const float *Ww = W + ((int64_t)b * S + (int64_t)wave_u * 32 * BJ) * ldw + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < 8 * BJ; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int chunk = (lane & 15) ^ (kk & 15);
      numrs_hip::lds_dma16(Ww, (uint32_t)(4 * ((int64_t)kk * ldw + 4 * chunk)),
                           base + 4u * (uint32_t)(wave_u * kSlot) + 1024u * it);
    }
  }

  // (MODE 1) the P block into registers behind the DMA
  auto col_of = [&](int bj, int i4) { return col0 + 32 * bj + 8 * i4 + 4 * hh; };
  auto row_ptr = [&](float *base, int bi) { return base + zoff + (int64_t)(row0 + 32 * bi + c) * S; };
  constexpr int kP = MODE == 1 ? 2 * BJ * 4 : 0;  // register loads of P
  f4 p[2][MODE == 1 ? BJ : 1][4];
  if constexpr (MODE == 1) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const float *src = row_ptr(const_cast<float *>(P), bi);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          p[bi][bj][i4] = *reinterpret_cast<const f4 *>(src + col_of(bj, i4));
    }
  }
  // The kP register loads above are the newest vector-memory operations and
  // the W rows of key block bj > 0 the DMA issued last: at most 8 (BJ - 1) +
  // kP outstanding means the X rows and key block 0 have landed
  // (vector-memory operations complete in issue order).
  __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(8 * (BJ - 1) + kP));
  __syncthreads();  // every wave's X rows are in

  // The wave's E rows into registers, issued only now so that they do not
  // compete with the X and W rows every workgroup waits for; they arrive
  // during the product.
  constexpr int kStage = 8 * BJ;
  f4 stage[kStage];
  {
    const float *Ez = E + (int64_t)b * S * lde + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < kStage; ++it)
      stage[it] = *reinterpret_cast<const f4 *>(Ez + (int64_t)(col0 + 4 * it + (lane >> 4)) * lde +
                                                4 * (lane & 15));
  }

  // 2. Y^T blocks (bi, bj): rows of X as B, the wave's rows of W as A, key
  // block by key block (each accumulator's products in the same order)
  f16v acc[2][BJ];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = f16v{};
  const float *xs = lds + kXRows;
#pragma unroll
  for (int bj = 0; bj < BJ; ++bj) {
    if (bj == 1)  // key block 1's rows (this wave's own DMA; P and E are newer) have landed
      __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(kP + kStage));
#pragma unroll
    for (int g = 0; g < kHeadDim / 8; ++g) {
      const int ch = 2 * g + hh;
      f4 a[2];
#pragma unroll
      for (int bi = 0; bi < 2; ++bi) {
        const int r = 32 * bi + c;
        a[bi] = *reinterpret_cast<const f4 *>(xs + r * kHeadDim + 4 * (ch ^ (r & 15)));
      }
      const int rw = 32 * bj + c;
      const f4 w = *reinterpret_cast<const f4 *>(wbuf + rw * kHeadDim + 4 * (ch ^ (rw & 15)));
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[j], a[bi][j], acc[bi][bj], 0, 0, 0);
    }
  }

  // 3. Row totals over the wave's columns (in-lane, then the other half-wave),
  // then over the four waves: op 0 = max, 1 = sum.
  __syncthreads();  // every wave is done reading the X rows that `red` reuses
  auto row_reduce = [&](float (&v)[2], int op) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      v[bi] = op == 0 ? half_pair(v[bi], [](float x, float y) { return fmaxf(x, y); })
                      : half_pair(v[bi], [](float x, float y) { return x + y; });
      if (hh == 0) red[wave][32 * bi + c] = v[bi];
    }
    __syncthreads();
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const int r = 32 * bi + c;
      v[bi] = op == 0 ? fmaxf(fmaxf(red[0][r], red[1][r]), fmaxf(red[2][r], red[3][r]))
                      : ((red[0][r] + red[1][r]) + red[2][r]) + red[3][r];
    }
    __syncthreads();
  };
  float t[2];
  {
    // dS = P * (Y - rowsum(Y * P))
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float s = 0.0f;
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[bi][bj][i] * p[bi][bj][i >> 2][i & 3];
      t[bi] = s;
    }
    row_reduce(t, 1);
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc[bi][bj][i] = p[bi][bj][i >> 2][i & 3] * (acc[bi][bj][i] - t[bi]);
  }

  // 4. E into the wave's slot (its W rows are consumed), chunks of rows
  // whose bit 2 is set XOR-ed by 8; then the rows leave
#pragma unroll
  for (int it = 0; it < kStage; ++it) {
    const int kk = 4 * it + (lane >> 4);
    const int slot = (lane & 15) ^ (8 * ((kk >> 2) & 1));
    *reinterpret_cast<f4 *>(wbuf + kk * kHeadDim + 4 * slot) = stage[it];
  }
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
    float *dst = row_ptr(out, bi);
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const f4 v = {acc[bi][bj][4 * i4], acc[bi][bj][4 * i4 + 1], acc[bi][bj][4 * i4 + 2],
                      acc[bi][bj][4 * i4 + 3]};
        *reinterpret_cast<f4 *>(dst + col_of(bj, i4)) = v;
      }
  }

  // eo^T partial over the wave's keys, as in attn_rows_kernel
  f16v o[2][2];
#pragma unroll
  for (int bd = 0; bd < 2; ++bd)
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) o[bd][bi] = f16v{};
#pragma unroll
  for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float *er = wbuf + (32 * bj + 8 * g + 4 * hh + e) * kHeadDim + c;
        const float ev[2] = {er[32 * hh], er[32 * (1 - hh)]};
#pragma unroll
        for (int bd = 0; bd < 2; ++bd)
#pragma unroll
          for (int bi = 0; bi < 2; ++bi)
            o[bd][bi] = __builtin_amdgcn_mfma_f32_32x32x2f32(ev[bd], acc[bi][bj][4 * g + e], o[bd][bi],
                                                             0, 0, 0);
      }
  __syncthreads();  // every wave is done with its slot
  float *part = lds + wave * (kRowsPerBlock * kPartStride);
#pragma unroll
  for (int bd = 0; bd < 2; ++bd)
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const f4 v = {o[bd][bi][4 * i4], o[bd][bi][4 * i4 + 1], o[bd][bi][4 * i4 + 2], o[bd][bi][4 * i4 + 3]};
        *reinterpret_cast<f4 *>(part + (32 * bi + c) * kPartStride + 32 * bd + 8 * i4 + 4 * hh) = v;
      }
  __syncthreads();
  const int q = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * 16;
  float *dst = eo + (int64_t)(b * S + row0 + q) * ldo + (int64_t)head * kHeadDim + d0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = q * kPartStride + d0 + 4 * j;
    const f4 s0 = *reinterpret_cast<const f4 *>(lds + off);
    const f4 s1 = *reinterpret_cast<const f4 *>(lds + kRowsPerBlock * kPartStride + off);
    const f4 s2 = *reinterpret_cast<const f4 *>(lds + 2 * kRowsPerBlock * kPartStride + off);
    const f4 s3 = *reinterpret_cast<const f4 *>(lds + 3 * kRowsPerBlock * kPartStride + off);
    f4 v = ((s0 + s1) + s2) + s3;
    if constexpr (MODE == 1) {
      v = ealpha * v;
      if (eacc) v = *reinterpret_cast<const f4 *>(dst + 4 * j) + v;
    }
    *reinterpret_cast<f4 *>(dst + 4 * j) = v;
  }
}

// Forward for dh = 64 and S = 128 or 256 (NKB = S/16 key blocks of 16): a
// workgroup of eight waves owns 128 query rows of one head and wave w the 16
// rows row0 + 16 w .. + 15 against every key, so a row's max and sum stay in
// the wave (no LDS round, no barrier between the product and the softmax) and
// O = P V needs no sum of wave partials.  The products are 16x16x4 fp32 MFMAs
// (lane l = 16 g + j: A row j at reduction slot g, B slot g at column j, D
// column j at rows 4 g + r):
//   S^T block kb = K_kb Q_w^T: for step t = 4 q + e (q, e = 0..3) A holds
//     K[16 kb + j][d] and B Q[16 w + j][d] with d = 16 q + 4 g + e, so step
//     t reduces over dh {16 q + e, 16 q + 4 + e, 16 q + 8 + e, 16 q + 12 + e}
//     and the four lanes of a Q row read 64 contiguous bytes per load; lane
//     (j, g) ends with S[query j][key 16 kb + 4 g + r], r = 0..3.
//   O^T block db = V^T P^T: for each key block kb and r, B is the lane's own
//     register r of block kb (keys 16 kb + 4 g + r over the slots g) and A
//     holds V[16 kb + 4 g + r][4 j + db], so row i of block db is output
//     column 4 i + db and lane (j, g) ends with O[query j][16 g + 4 r + db].
// The lane's Q values load straight into registers; K and V go to LDS by
// DMA, K's 16-byte chunk c of row r at slot c ^ (r % 16) so that the 16
// lanes reading one chunk of 16 rows hit 16 slots (V unpermuted: 16 lanes
// read one row).  Loads, in issue order: Q, the first half of the keys' K
// rows (waited for, with Q), the second half, V.  QK^T over the first half
// of the keys runs while the rest arrives; one barrier in the middle of the
// product makes the second half and V visible, after which the waves run
// apart (a wave's softmax beside the other wave's MFMAs on its SIMD).  The
// softmax is in base 2: m = max y, e = 2^(alpha log2(e) y - alpha log2(e) m)
// (one fma and one v_exp_f32), P = e * (1/sum e).  128 KiB of LDS at S = 256:
// one workgroup per CU, two waves per SIMD.
template <int NKB>
__global__ void __launch_bounds__(512) attn_fwd_wave_rows_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    int64_t ld, float *__restrict__ P, float *__restrict__ O, int64_t ldo, int S, int H,
    float alpha) {
  static_assert(NKB == 8 || NKB == 16, "S = 128 or 256");
  constexpr int kKeys = 16 * NKB;
  constexpr int kHalf = kKeys / 16;  // K rows per wave in each half of the keys
  constexpr int kVPer = kKeys / 32;  // V DMA instructions per wave (4 rows each)
  __shared__ __attribute__((aligned(1024))) float lds[2 * kKeys * kHeadDim];
  const float *ks = lds;
  const float *vs = lds + kKeys * kHeadDim;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  int rb = blockIdx.x, z = blockIdx.y;
  {
    // XCD k (hardware ids k, k+8, ...) owns a contiguous run of heads
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      rb = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int row0 = rb * 128;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  const float *Kh = K + (int64_t)b * S * ld + (int64_t)head * kHeadDim;

  // 1. Loads.  qf[q][e] = Q[16 w + j][16 q + 4 g + e].  DMA instruction it of
  // a run fills 4 rows (1 KiB), lane l the 16-byte slot l % 16 of run row
  // 4 it + l / 16.
  f4 qf[4];
  {
    const float *qr = Q + ((int64_t)b * S + row0 + 16 * wave + j) * ld + (int64_t)head * kHeadDim + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) qf[q] = *reinterpret_cast<const f4 *>(qr + 16 * q);
  }
  auto k_half = [&](int h) {
    const int r0 = h * (kKeys / 2) + kHalf * wave_u;  // the wave's first row of this half
#pragma unroll
    for (int it = 0; it < kHalf / 4; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int chunk = (lane & 15) ^ ((r0 + kk) & 15);
      numrs_hip::lds_dma16(Kh + (int64_t)r0 * ld, (uint32_t)(4 * ((int64_t)kk * ld + 4 * chunk)),
                           base + 4u * (uint32_t)(r0 * kHeadDim) + 1024u * it);
    }
  };
  k_half(0);
  // Q is used here, so the compiler waits for the Q loads -- and with them
  // (vector-memory operations complete in issue order) for the DMA of the
  // first half of K -- before the second half and V are issued.
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]));
  k_half(1);
  {
    const int r0 = kVPer * 4 * wave_u;
    const float *Vw = V + ((int64_t)b * S + r0) * ld + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < kVPer; ++it) {
      const int kk = 4 * it + (lane >> 4);
      numrs_hip::lds_dma16(Vw, (uint32_t)(4 * ((int64_t)kk * ld + 4 * (lane & 15))),
                           base + 4u * (uint32_t)((kKeys + r0) * kHeadDim) + 1024u * it);
    }
  }
  __syncthreads();  // every wave's rows of the first half of K are in

  // 2. S^T = K Q^T, the first half of the key blocks, then (after every
  // wave's second half of K and V have landed) the second; two key blocks at
  // a time (alternating accumulators), each accumulator's steps in t order.
  f4 acc[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) acc[kb] = f4{};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1) {
      __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(0));  // no store has been issued yet
      __syncthreads();
    }
    // step i = (q, key-block pair): the next step's two K reads are issued
    // ahead of this step's eight MFMAs
    constexpr int kPairs = NKB / 4, kSteps = 4 * kPairs;
    auto kread = [&](int i, int d) {
      const int q = i / kPairs, kb = h * NKB / 2 + 2 * (i % kPairs) + d;
      return *reinterpret_cast<const f4 *>(ks + (16 * kb + j) * kHeadDim + 4 * ((4 * q + g) ^ j));
    };
    f4 k0 = kread(0, 0), k1 = kread(0, 1);
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      f4 n0 = k0, n1 = k1;
      if (i + 1 < kSteps) {
        n0 = kread(i + 1, 0);
        n1 = kread(i + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int q = i / kPairs, kb = h * NKB / 2 + 2 * (i % kPairs);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(k0[e], qf[q][e], acc[kb], 0, 0, 0);
        acc[kb + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(k1[e], qf[q][e], acc[kb + 1], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      k0 = n0;
      k1 = n1;
    }
  }

  // 3. Softmax of each query row: the row's 4 NKB values in the lane, then
  // the four lanes j, j + 16, j + 32, j + 48.
  {
    const float a = alpha * 1.44269504088896341f;
    float m = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) m = fmaxf(m, acc[kb][r]);
    m = rows4(m, [](float x, float y) { return fmaxf(x, y); });
    const float am = a * m;  // alpha > 0: the scaled scores' max
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[kb][r], a, -am));
        acc[kb][r] = e;
        sum += e;
      }
    sum = rows4(sum, [](float x, float y) { return x + y; });
    const float inv = 1.0f / sum;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc[kb] = acc[kb] * inv;
  }

  // 4. O = P V, with the P rows leaving (four consecutive keys per lane and
  // block) one store per key block between the MFMA groups (instead of all
  // before them: N3f 28.4 -> 27.7 us at C4)
  float *Pw = P + (int64_t)z * S * S + (int64_t)(row0 + 16 * wave + j) * S + 4 * g;
  f4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f4{};
  // step i = (kb, r): the next step's V read is issued ahead of this step's
  // four MFMAs
  auto vread = [&](int i) {
    return *reinterpret_cast<const f4 *>(vs + (16 * (i >> 2) + 4 * g + (i & 3)) * kHeadDim + 4 * j);
  };
  f4 v = vread(0);
#pragma unroll
  for (int i = 0; i < 4 * NKB; ++i) {
    f4 nv = v;
    if (i + 1 < 4 * NKB) nv = vread(i + 1);
    if ((i & 3) == 0) *reinterpret_cast<f4 *>(Pw + 16 * (i >> 2)) = acc[i >> 2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < 4; ++db)
      o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[db], acc[i >> 2][i & 3], o[db], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    v = nv;
  }
  float *Ow = O + ((int64_t)b * S + row0 + 16 * wave + j) * ldo + (int64_t)head * kHeadDim + 16 * g;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<f4 *>(Ow + 4 * r) = f4{o[0][r], o[1][r], o[2][r], o[3][r]};
}

// Backward for dh = 64 and S = 128 or 256 given the forward's output O (the
// softmax backward's row total rowsum(dP * P) = dO . O), in two launches
// whose waves own whole rows of the products, as the forward's do:
//   attn_bwd_wave_rows_kernel: eight waves of 16 query rows against every
//     key: dP^T = V dO^T (the forward's S^T with V for K and dO for Q), D =
//     dO . O in the wave, dS = P (dP - D) stored to a [B H, S, S] buffer in
//     P's layout, and dQ = alpha dS K (the forward's O = P V with K for V):
//     no sum across waves, no atomics.
//   attn_bwd_wave_keys_kernel: eight waves of 16 keys against every query:
//     dV = P^T dO and dK = alpha dS^T Q.
// Both: one workgroup per CU at S = 256 (128 KiB of LDS), two waves per SIMD.
template <int NKB>
__global__ void __launch_bounds__(512) attn_bwd_wave_rows_kernel(
    const float *__restrict__ K, const float *__restrict__ V, int64_t ld,
    const float *__restrict__ P, const float *__restrict__ dO, const float *__restrict__ O,
    int64_t ldo, float *__restrict__ dS, float *__restrict__ dq, int S, int H, float alpha) {
  static_assert(NKB == 8 || NKB == 16, "S = 128 or 256");
  constexpr int kKeys = 16 * NKB;
  constexpr int kHalf = kKeys / 16;  // V rows per wave in each half of the keys
  constexpr int kKPer = kKeys / 32;  // K DMA instructions per wave (4 rows each)
  __shared__ __attribute__((aligned(1024))) float lds[2 * kKeys * kHeadDim];
  const float *vs = lds;                     // V: chunk c of row r at slot c ^ (r % 16)
  const float *ks = lds + kKeys * kHeadDim;  // K: unpermuted (16 lanes read one row)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  int rb = blockIdx.x, z = blockIdx.y;
  {
    // XCD k (hardware ids k, k+8, ...) owns a contiguous run of heads
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      rb = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int row0 = rb * 128;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  const float *Vh = V + (int64_t)b * S * ld + (int64_t)head * kHeadDim;
  const float *Kh = K + (int64_t)b * S * ld + (int64_t)head * kHeadDim;
  const int64_t prow = (int64_t)z * S * S + (int64_t)(row0 + 16 * wave + j) * S + 4 * g;

  // 1. Loads, in issue order: the lane's dO values ([q][e] = row 16 w + j,
  // column 16 q + 4 g + e), the first half of V (waited for, with them), the
  // second half of V, K, and after the barrier (so that no wave's later loads
  // queue ahead of another wave's first ones) the lane's O values (dO's
  // layout); the lane's P values (pf[kb] = P[query j][16 kb + 4 g ..]) during
  // the second half of dP.
  f4 df[4], of[4];
  const int64_t roff = ((int64_t)b * S + row0 + 16 * wave + j) * ldo + (int64_t)head * kHeadDim + 4 * g;
#pragma unroll
  for (int q = 0; q < 4; ++q) df[q] = *reinterpret_cast<const f4 *>(dO + roff + 16 * q);
  auto v_half = [&](int h) {
    const int r0 = h * (kKeys / 2) + kHalf * wave_u;
#pragma unroll
    for (int it = 0; it < kHalf / 4; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int chunk = (lane & 15) ^ ((r0 + kk) & 15);
      numrs_hip::lds_dma16(Vh + (int64_t)r0 * ld, (uint32_t)(4 * ((int64_t)kk * ld + 4 * chunk)),
                           base + 4u * (uint32_t)(r0 * kHeadDim) + 1024u * it);
    }
  };
  v_half(0);
  // dO is used here, so the compiler waits for it -- and with it
  // (vector-memory operations complete in issue order) for the first half of
  // V -- before the rest is issued.
  asm volatile("" ::"v"(df[0]), "v"(df[1]), "v"(df[2]), "v"(df[3]) : "memory");
  v_half(1);
  {
    const int r0 = 4 * kKPer * wave_u;
#pragma unroll
    for (int it = 0; it < kKPer; ++it) {
      const int kk = 4 * it + (lane >> 4);
      numrs_hip::lds_dma16(Kh + (int64_t)r0 * ld, (uint32_t)(4 * ((int64_t)kk * ld + 4 * (lane & 15))),
                           base + 4u * (uint32_t)((kKeys + r0) * kHeadDim) + 1024u * it);
    }
  }
  __syncthreads();  // every wave's rows of the first half of V are in
#pragma unroll
  for (int q = 0; q < 4; ++q) of[q] = *reinterpret_cast<const f4 *>(O + roff + 16 * q);
  f4 pf[NKB];

  // 2. dP^T = V dO^T, the first half of the key blocks, then (after every
  // wave's second half of V and K have landed) the second; operand reads one
  // step ahead of the MFMAs.
  f4 acc[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) acc[kb] = f4{};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1) {
      __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(0));  // O, the second half of V, K
      __syncthreads();
    }
    constexpr int kPairs = NKB / 4, kSteps = 4 * kPairs;
    auto vread = [&](int i, int d) {
      const int q = i / kPairs, kb = h * NKB / 2 + 2 * (i % kPairs) + d;
      return *reinterpret_cast<const f4 *>(vs + (16 * kb + j) * kHeadDim + 4 * ((4 * q + g) ^ j));
    };
    f4 w0 = vread(0, 0), w1 = vread(0, 1);
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      f4 n0 = w0, n1 = w1;
      if (i + 1 < kSteps) {
        n0 = vread(i + 1, 0);
        n1 = vread(i + 1, 1);
      }
      // the lane's P values, two blocks per step over the first half of the
      // second half's steps (52.6 -> 52.0 us against all sixteen at its start)
      if (h == 1 && 2 * i < NKB) {
        pf[2 * i] = *reinterpret_cast<const f4 *>(P + prow + 16 * (2 * i));
        pf[2 * i + 1] = *reinterpret_cast<const f4 *>(P + prow + 16 * (2 * i + 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      const int q = i / kPairs, kb = h * NKB / 2 + 2 * (i % kPairs);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(w0[e], df[q][e], acc[kb], 0, 0, 0);
        acc[kb + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(w1[e], df[q][e], acc[kb + 1], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      w0 = n0;
      w1 = n1;
    }
  }

  // 3. D = dO . O of query j (the lane's 16 products, then the four lanes of
  // the row), dS = P (dP - D); stored in P's layout during step 4
  float D = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) D += df[q][e] * of[q][e];
  D = rows4(D, [](float x, float y) { return x + y; });
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) acc[kb] = pf[kb] * (acc[kb] - D);

  // 4. dQ = alpha dS K: B is the lane's register r of dS block kb, A holds
  // K[16 kb + 4 g + r][4 j + db]; lane (j, g) ends with dQ[query j][16 g +
  // 4 r + db].  The K read of the next step goes ahead of this step's MFMAs,
  // and dS block kb's store with the first of its four steps (one store
  // between MFMA groups instead of sixteen in a row before them: N3 54.6 ->
  // 52.4 us at C4).
  f4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f4{};
  auto kread = [&](int i) {
    return *reinterpret_cast<const f4 *>(ks + (16 * (i >> 2) + 4 * g + (i & 3)) * kHeadDim + 4 * j);
  };
  f4 kv = kread(0);
#pragma unroll
  for (int i = 0; i < 4 * NKB; ++i) {
    f4 nk = kv;
    if (i + 1 < 4 * NKB) nk = kread(i + 1);
    if ((i & 3) == 0) *reinterpret_cast<f4 *>(dS + prow + 16 * (i >> 2)) = acc[i >> 2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < 4; ++db)
      o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[db], acc[i >> 2][i & 3], o[db], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    kv = nk;
  }
  float *qw = dq + ((int64_t)b * S + row0 + 16 * wave + j) * ld + (int64_t)head * kHeadDim + 16 * g;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<f4 *>(qw + 4 * r) =
        f4{alpha * o[0][r], alpha * o[1][r], alpha * o[2][r], alpha * o[3][r]};
}

// dV = P^T dO and dK = alpha dS^T Q for 128 keys of one head (NQB = S/16):
// wave w owns keys key0 = 128 kg + 16 w .. + 15.  Step t of the S/4 steps
// covers queries 4 t + g at reduction slot g: A holds P (dS) [4 t + g][key0
// + j], loaded from global memory kPD steps ahead into a register ring; B
// holds dO (Q) [4 t + g][4 j + db] from LDS (rows by DMA, unpermuted: 16
// lanes read one row), so block db's column j is output column 4 j + db and
// lane (j, g) ends with dV (dK) [key0 + 4 g + r][4 j + db].
template <int NQB>
__global__ void __launch_bounds__(512) attn_bwd_wave_keys_kernel(
    const float *__restrict__ Q, int64_t ld, const float *__restrict__ P,
    const float *__restrict__ dS, const float *__restrict__ dO, int64_t ldo,
    float *__restrict__ dk, float *__restrict__ dv, int S, int H, float alpha) {
  static_assert(NQB == 8 || NQB == 16, "S = 128 or 256");
  constexpr int kQ = 16 * NQB;     // queries
  constexpr int kSteps = kQ / 4;   // MFMA steps of four queries
  constexpr int kPer = kQ / 32;    // DMA instructions per wave for Q, and for dO
  // Steps of P and dS loaded ahead.  Measured at C4 (N3, from HBM): 4 ahead
  // 54.3 us, 8 54.6, 16 55.6, 32 57.6 -- the loads hit in the caches (dS was
  // just written, P is shared by the head's two key groups), and a longer
  // ring only holds more loads in the memory pipeline.
  constexpr int kPD = 4;
  __shared__ __attribute__((aligned(1024))) float lds[2 * kQ * kHeadDim];
  const float *qs = lds;
  const float *os = lds + kQ * kHeadDim;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  int kg = blockIdx.x, z = blockIdx.y;
  {
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      kg = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int key0 = kg * 128 + 16 * wave;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  {
    const int r0 = 4 * kPer * wave_u;
    const float *qsrc = Q + ((int64_t)b * S + r0) * ld + (int64_t)head * kHeadDim;
    const float *osrc = dO + ((int64_t)b * S + r0) * ldo + (int64_t)head * kHeadDim;
#pragma unroll
    for (int it = 0; it < kPer; ++it) {
      const int kk = 4 * it + (lane >> 4);
      numrs_hip::lds_dma16(qsrc, (uint32_t)(4 * ((int64_t)kk * ld + 4 * (lane & 15))),
                           base + 4u * (uint32_t)(r0 * kHeadDim) + 1024u * it);
      numrs_hip::lds_dma16(osrc, (uint32_t)(4 * ((int64_t)kk * ldo + 4 * (lane & 15))),
                           base + 4u * (uint32_t)((kQ + r0) * kHeadDim) + 1024u * it);
    }
  }
  const int64_t col = (int64_t)z * S * S + (int64_t)g * S + key0 + j;  // query g, key key0 + j
  float pa[kPD], sa[kPD];
#pragma unroll
  for (int t = 0; t < kPD; ++t) {
    pa[t] = P[col + (int64_t)4 * t * S];
    sa[t] = dS[col + (int64_t)4 * t * S];
  }
  // the 2 kPD loads above are the newest vector-memory operations
  __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(2 * kPD));
  __syncthreads();  // every wave's Q and dO rows are in

  f4 vacc[4], kacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    vacc[db] = f4{};
    kacc[db] = f4{};
  }
  auto bread = [&](const float *m, int t) {
    return *reinterpret_cast<const f4 *>(m + (4 * t + g) * kHeadDim + 4 * j);
  };
  f4 bo = bread(os, 0), bq = bread(qs, 0);
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    const float pv = pa[t % kPD], sv = sa[t % kPD];
    if (t + kPD < kSteps) {
      pa[t % kPD] = P[col + (int64_t)4 * (t + kPD) * S];
      sa[t % kPD] = dS[col + (int64_t)4 * (t + kPD) * S];
    }
    f4 no = bo, nq = bq;
    if (t + 1 < kSteps) {
      no = bread(os, t + 1);
      nq = bread(qs, t + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      vacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv, bo[db], vacc[db], 0, 0, 0);
      kacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv, bq[db], kacc[db], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    bo = no;
    bq = nq;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t off = ((int64_t)b * S + key0 + 4 * g + r) * ld + (int64_t)head * kHeadDim + 4 * j;
    *reinterpret_cast<f4 *>(dv + off) = f4{vacc[0][r], vacc[1][r], vacc[2][r], vacc[3][r]};
    *reinterpret_cast<f4 *>(dk + off) =
        f4{alpha * kacc[0][r], alpha * kacc[1][r], alpha * kacc[2][r], alpha * kacc[3][r]};
  }
}

// Whether the fused row-block kernel takes this shape: dh = 64, S a multiple
// of 128 up to 512, rows of both operands at 16-byte strides and 16-byte
// aligned, 16-byte aligned probability matrices.
bool rows_fit(int64_t S, int64_t dh, int64_t ldx, int64_t ldw, const void *x, const void *w,
              const void *p) {
  return dh == kHeadDim && S % 128 == 0 && S <= 512 && ldx % 4 == 0 && ldw % 4 == 0 &&
         numrs_hip::aligned16(x) && numrs_hip::aligned16(w) && numrs_hip::aligned16(p);
}

// The third matrix and its product's output as the fused kernel reads and
// writes them: 16-byte strides and alignment.
bool extra_fit(int64_t lde, int64_t ldo, const void *e, const void *eo) {
  // the DMA's per-lane byte offsets (rows below 128 of a wave's keys) fit 31 bits
  return lde % 4 == 0 && ldo % 4 == 0 && lde < (int64_t{1} << 22) && numrs_hip::aligned16(e) &&
         numrs_hip::aligned16(eo);
}

template <int MODE, bool EXTRA>
int launch_rows(numrs_hip_ctx *ctx, const float *X, int64_t ldx, const float *W, int64_t ldw,
                const float *P, float *out, int64_t B, int64_t S, int64_t H, float alpha,
                const float *E = nullptr, int64_t lde = 0, float *eo = nullptr, int64_t ldo = 0,
                float ealpha = 1.0f, int eacc = 0) {
  const dim3 grid((unsigned)(S / kRowsPerBlock), (unsigned)(B * H));
  const int s = (int)S, h = (int)H;
#define NRS_ROWS(BJ)                                                                            \
  attn_rows_kernel<MODE, BJ, EXTRA><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, s, h, ldx, ldw, \
                                                                    alpha, E, lde, eo, ldo,     \
                                                                    ealpha, eacc)
  switch (S / 128) {
    case 1: NRS_ROWS(1); break;
    case 2: NRS_ROWS(2); break;
    case 3: NRS_ROWS(3); break;
    default: NRS_ROWS(4); break;
  }
#undef NRS_ROWS
  return numrs_hip::check_launch(ctx, "attn_rows_kernel");
}

// attn_rows_lds_kernel takes S <= 256; its DMA's per-lane byte offsets
// (rows below 64 of W, below 16 of X) fit 31 bits.
bool lds_rows_fit(int64_t S, int64_t ldx, int64_t ldw) {
  return S <= 256 && ldx < (int64_t{1} << 22) && ldw < (int64_t{1} << 22);
}

template <int MODE>
int launch_lds_rows(numrs_hip_ctx *ctx, const float *X, int64_t ldx, const float *W, int64_t ldw,
                    const float *P, float *out, int64_t B, int64_t S, int64_t H, float alpha,
                    const float *E, int64_t lde, float *eo, int64_t ldo, float ealpha = 1.0f,
                    int eacc = 0) {
  const dim3 grid((unsigned)(S / kRowsPerBlock), (unsigned)(B * H));
  const int s = (int)S, h = (int)H;
  if (S == 128)
    attn_rows_lds_kernel<MODE, 1><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, s, h, ldx, ldw, alpha,
                                                                 E, lde, eo, ldo, ealpha, eacc);
  else
    attn_rows_lds_kernel<MODE, 2><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, s, h, ldx, ldw, alpha,
                                                                 E, lde, eo, ldo, ealpha, eacc);
  return numrs_hip::check_launch(ctx, "attn_rows_lds_kernel");
}

// attn_fwd_wave_rows_kernel: S = 128 or 256, q, k, v at one row stride.
int launch_wave_rows(numrs_hip_ctx *ctx, const float *q, const float *k, const float *v,
                     int64_t ld, float *P, float *out, int64_t ldo, int64_t B, int64_t S,
                     int64_t H, float alpha) {
  const dim3 grid((unsigned)(S / 128), (unsigned)(B * H));
  const int s = (int)S, h = (int)H;
  if (S == 128)
    attn_fwd_wave_rows_kernel<8><<<grid, 512, 0, ctx->stream>>>(q, k, v, ld, P, out, ldo, s, h, alpha);
  else
    attn_fwd_wave_rows_kernel<16><<<grid, 512, 0, ctx->stream>>>(q, k, v, ld, P, out, ldo, s, h, alpha);
  return numrs_hip::check_launch(ctx, "attn_fwd_wave_rows_kernel");
}

int check(numrs_hip_ctx *ctx, int64_t B, int64_t S, int64_t H, int64_t D, int64_t ld_qkv,
          int64_t ld_out) {
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0 || D % H != 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE,
                           "attention: batch, seq, heads > 0 and dim divisible by heads");
  if (ld_qkv < D || ld_out < D)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE, "attention: row strides below the dim");
  return NUMRS_HIP_OK;
}

}  // namespace

extern "C" {

// q, k, v rows (and dq, dk, dv in the backward) at stride ld_qkv, out / dout
// rows at stride ld_out: q, k, v may be column slices of one packed
// [B*S, 3D] projection (ld_qkv = 3D).
int numrs_hip_attention_forward_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                        const float *v, int64_t ld_qkv, float *P, float *out,
                                        int64_t ld_out, int64_t B, int64_t S, int64_t H,
                                        int64_t D) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, S, H, D, ld_qkv, ld_out)) return rc;
  if (!q || !k || !v || !P || !out)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "attention_forward: null pointer");
  const int64_t dh = D / H, Z = B * H, li = ld_qkv, lo = ld_out;
  const float alpha = 1.0f / sqrtf((float)dh);
  if (rows_fit(S, dh, li, li, q, k, P) && B * H < 65536) {
    // P = softmax_rows(alpha * Q K^T) and O = P V in one kernel
    if (extra_fit(li, lo, v, out) && lds_rows_fit(S, li, li))
      return launch_wave_rows(ctx, q, k, v, li, P, out, lo, B, S, H, alpha);
    if (extra_fit(li, lo, v, out))
      return launch_rows<0, true>(ctx, q, li, k, li, nullptr, P, B, S, H, alpha, v, li, out, lo);
    if (int rc = launch_rows<0, false>(ctx, q, li, k, li, nullptr, P, B, S, H, alpha)) return rc;
    return numrs_hip_gemm(ctx, P, S, v, li, out, lo, S, S, dh, 0, 0, 1.0f, 0, Z, H, H * S * S,
                          S * S, S * li, dh, S * lo, dh);
  }
  // S_z = alpha * Q_z K_z^T  -> P (row-major [S, S] per z)
  if (int rc = numrs_hip_gemm(ctx, q, li, k, li, P, S, S, dh, S, 0, 1, alpha, 0, Z, H, S * li, dh,
                              S * li, dh, H * S * S, S * S))
    return rc;
  // in-place row softmax (each row is read completely before it is written)
  if (int rc = numrs_hip_softmax_forward(ctx, P, P, Z * S, S, 1.0f)) return rc;
  // O_z = P_z V_z
  return numrs_hip_gemm(ctx, P, S, v, li, out, lo, S, S, dh, 0, 0, 1.0f, 0, Z, H, H * S * S,
                        S * S, S * li, dh, S * lo, dh);
}

int numrs_hip_attention_backward_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                         const float *v, int64_t ld_qkv, const float *P,
                                         const float *dout, int64_t ld_out, float *dq, float *dk,
                                         float *dv, int64_t B, int64_t S, int64_t H, int64_t D,
                                         int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, S, H, D, ld_qkv, ld_out)) return rc;
  if (!q || !k || !v || !P || !dout)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "attention_backward: null input");
  const int64_t dh = D / H, Z = B * H, li = ld_qkv, lo = ld_out;
  const float alpha = 1.0f / sqrtf((float)dh);
  // dV_z = P_z^T dO_z
  auto dv_gemm = [&]() {
    return numrs_hip_gemm(ctx, P, S, dout, lo, dv, li, S, S, dh, 1, 0, 1.0f, accumulate, Z, H,
                          H * S * S, S * S, S * lo, dh, S * li, dh);
  };
  if (!dq && !dk) return dv ? dv_gemm() : NUMRS_HIP_OK;
  // dS lives in a block of its own: the products below may split their
  // reduction and write partials to the context workspace while reading dS.
  numrs_hip::TempBlock dSb(ctx);
  if (int rc = dSb.alloc((size_t)(Z * S * S) * sizeof(float))) return rc;
  float *dS = dSb.f();
  const numrs_hip::BatchedMat dSm{dS, S, H * S * S, S * S};
  const numrs_hip::BatchedMat Km{k, li, S * li, dh}, Qm{q, li, S * li, dh};
  const numrs_hip::BatchedOut dQ{dq, li, S * li, dh}, dK{dk, li, S * li, dh};
  if (rows_fit(S, dh, lo, li, dout, v, P) && numrs_hip::aligned16(dS) && B * H < 65536) {
    // dS = P * (dP - rowsum(dP * P)) with dP = dO V^T, and dQ = alpha dS K,
    // in one kernel; then dV and dK = alpha dS^T Q as one pair launch.
    if (dq && extra_fit(li, li, k, dq) && lds_rows_fit(S, lo, li)) {
      if (int rc = launch_lds_rows<1>(ctx, dout, lo, v, li, P, dS, B, S, H, 1.0f, k, li, dq, li,
                                      alpha, accumulate))
        return rc;
    } else if (dq && extra_fit(li, li, k, dq)) {
      if (int rc = launch_rows<1, true>(ctx, dout, lo, v, li, P, dS, B, S, H, 1.0f, k, li, dq, li,
                                        alpha, accumulate))
        return rc;
    } else {
      if (int rc = launch_rows<1, false>(ctx, dout, lo, v, li, P, dS, B, S, H, 1.0f)) return rc;
      if (dq)
        if (int rc = numrs_hip::gemm_nn_tn_pair(ctx, dSm, Km, dQ, Qm, {nullptr, 0, 0, 0}, S, S,
                                                dh, alpha, accumulate, Z, H))
          return rc;
    }
    if (!dk) return dv ? dv_gemm() : NUMRS_HIP_OK;
    const numrs_hip::BatchedMat Pm{P, S, H * S * S, S * S}, dOm{dout, lo, S * lo, dh};
    const numrs_hip::BatchedOut dV{dv, li, S * li, dh};
    return numrs_hip::gemm_tn_pair(ctx, Pm, dOm, dV, 1.0f, dSm, Qm, dK, alpha, S, S, dh,
                                   accumulate, Z, H);
  }
  if (dv)
    if (int rc = dv_gemm()) return rc;
  // dP_z = dO_z V_z^T
  if (int rc = numrs_hip_gemm(ctx, dout, lo, v, li, dS, S, S, dh, S, 0, 1, 1.0f, 0, Z, H, S * lo,
                              dh, S * li, dh, H * S * S, S * S))
    return rc;
  // dS = P * (dP - rowsum(dP * P)), in place over dP
  if (int rc = numrs_hip_softmax_backward(ctx, P, dS, dS, Z * S, S, 0)) return rc;
  // dQ_z = alpha * dS_z K_z ;  dK_z = alpha * dS_z^T Q_z  (one launch for both)
  return numrs_hip::gemm_nn_tn_pair(ctx, dSm, Km, dQ, Qm, dK, S, S, dh, alpha, accumulate, Z, H);
}

// The backward given also the forward's output `out` (rows at ld_out, like
// dout): for dh = 64, S = 128 or 256 and all three grads written (not
// accumulated), the query-row kernel (dS, dQ) then the key-row kernel (dV,
// dK); otherwise the row-block path above.
int numrs_hip_attention_backward_out_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                             const float *v, int64_t ld_qkv, const float *P,
                                             const float *out, const float *dout, int64_t ld_out,
                                             float *dq, float *dk, float *dv, int64_t B, int64_t S,
                                             int64_t H, int64_t D, int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, S, H, D, ld_qkv, ld_out)) return rc;
  if (!q || !k || !v || !P || !dout || !out)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "attention_backward: null input");
  const int64_t dh = D / H, li = ld_qkv, lo = ld_out;
  using numrs_hip::aligned16;
  const bool keys = dq && dk && dv && !accumulate && dh == kHeadDim && (S == 128 || S == 256) &&
                    B * H < 65536 && D <= 4096 && li % 4 == 0 && lo % 4 == 0 && S * li < (int64_t{1} << 29) &&
                    lo < (int64_t{1} << 22) && aligned16(q) && aligned16(k) && aligned16(v) &&
                    aligned16(P) && aligned16(out) && aligned16(dout) && aligned16(dq) &&
                    aligned16(dk) && aligned16(dv);
  if (!keys)
    return numrs_hip_attention_backward_strided(ctx, q, k, v, li, P, dout, lo, dq, dk, dv, B, S, H,
                                                D, accumulate);
  const float alpha = 1.0f / sqrtf((float)dh);
  // dS between the two launches, in P's layout
  numrs_hip::TempBlock dSb(ctx);
  if (int rc = dSb.alloc((size_t)(B * H * S * S) * sizeof(float))) return rc;
  float *dS = dSb.f();
  const dim3 grid((unsigned)(S / 128), (unsigned)(B * H));
  const int s = (int)S, h = (int)H;
  if (S == 128)
    attn_bwd_wave_rows_kernel<8><<<grid, 512, 0, ctx->stream>>>(k, v, li, P, dout, out, lo, dS, dq, s, h,
                                                                alpha);
  else
    attn_bwd_wave_rows_kernel<16><<<grid, 512, 0, ctx->stream>>>(k, v, li, P, dout, out, lo, dS, dq, s, h,
                                                                 alpha);
  if (int rc = numrs_hip::check_launch(ctx, "attn_bwd_wave_rows_kernel")) return rc;
  if (S == 128)
    attn_bwd_wave_keys_kernel<8><<<grid, 512, 0, ctx->stream>>>(q, li, P, dS, dout, lo, dk, dv, s, h, alpha);
  else
    attn_bwd_wave_keys_kernel<16><<<grid, 512, 0, ctx->stream>>>(q, li, P, dS, dout, lo, dk, dv, s, h, alpha);
  return numrs_hip::check_launch(ctx, "attn_bwd_wave_keys_kernel");
}

int numrs_hip_attention_forward(numrs_hip_ctx *ctx, const float *q, const float *k, const float *v,
                                float *P, float *out, int64_t B, int64_t S, int64_t H,
                                int64_t D) {
  return numrs_hip_attention_forward_strided(ctx, q, k, v, D, P, out, D, B, S, H, D);
}

int numrs_hip_attention_backward(numrs_hip_ctx *ctx, const float *q, const float *k,
                                 const float *v, const float *P, const float *dout, float *dq,
                                 float *dk, float *dv, int64_t B, int64_t S, int64_t H, int64_t D,
                                 int accumulate) {
  return numrs_hip_attention_backward_strided(ctx, q, k, v, D, P, dout, D, dq, dk, dv, B, S, H, D,
                                              accumulate);
}

}  // extern "C"
