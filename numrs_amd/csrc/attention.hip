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
// with alpha = 1/sqrt(dh).  All products are fp32 MFMA GEMMs; the row
// softmax and its backward are the one-wave-per-row kernels.
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

  // 4. P rows leave (four consecutive keys per lane and block), then O = P V
  {
    float *Pw = P + (int64_t)z * S * S + (int64_t)(row0 + 16 * wave + j) * S + 4 * g;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) *reinterpret_cast<f4 *>(Pw + 16 * kb) = acc[kb];
  }
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

// ---------------------------------------------------------------------------
// Key-block backward (dh = 64, S = 128 or 256): one workgroup per (head, 128
// keys) forms dV and dK for its keys over all S queries, and its share of dQ,
// without storing dS.  The softmax backward's row total needs every key of a
// row, so it comes from the forward output instead:
//   rowsum(dP * P) = sum_k P[q,k] (dO[q] . V[k]) = dO[q] . O[q]   (O = P V),
// 64 products per query, formed in the kernel from the staged dO rows.
//
// Wave w owns keys 32w..32w+31 of the group and keeps their V fragments in
// registers.  For each block of 64 queries (Q and dO rows staged in LDS by
// DMA, double-buffered; the next block's O rows and P values loaded into
// registers during this block, the P loads spread over the dV, dK products):
//   D = dO . O        per query, into LDS, before the block starts,
//   dP - D            MFMAs from accumulators set to -D, laid out as [query,
//                     key]: lane (c, h) holds key c and queries 8(i/4) + 4h +
//                     (i%4) of each 32-query block,
//   dS = P * (dP - D) in registers,
//   dV += P^T dO, dK += dS^T Q   with those registers as the B operand (the
//                     reduction runs over the queries they hold),
//   dS -> LDS ([query][key], 16-byte chunk j of row q at slot j ^ (q % 32)),
//   dQ[block] = dS K  wave w forms the 32 x 32 block (query half w/2, d half
//                     w%2) over the group's 128 keys, K staged in LDS at the
//                     start ([key][64], chunks of rows with bit 2 set XOR 8).
// The operands of each product's next step are read from LDS before the
// current step's MFMAs.  dQ adds alpha * dS K over the S/128 key groups.  At
// S = 256 the two groups' contributions go to rows zeroed by
// attn_bwd_zero_kernel through hardware float atomics: 0 + a + b is the same
// sum in either order, so the result does not depend on which group lands
// first.  At S = 128 the one group stores.
// Shared memory: K 32 KiB, two Q/dO tile pairs 64 KiB, dS 32 KiB: one
// workgroup per CU, four waves.
constexpr int kKeyGroup = 128;
constexpr int kKsOff = 0;                              // [128][64] K rows
constexpr int kTileOff = kKeyGroup * kHeadDim;         // two buffers of Q [64][64], dO [64][64]
constexpr int kTileFloats = 2 * kRowsPerBlock * kHeadDim;
constexpr int kDsOff = kTileOff + 2 * kTileFloats;     // [64][128] dS
constexpr int kDOff = kDsOff + kRowsPerBlock * kKeyGroup;  // the block's 64 row totals
constexpr int kKeysLds = kDOff + kRowsPerBlock;

// dq's rows set to 0 before two key groups add into them: workgroup w
// clears rows 16 w .. 16 w + 15 (B S is a multiple of 16), a float4 per
// thread and row (blockDim = D / 4).
__global__ void __launch_bounds__(1024) attn_bwd_zero_kernel(float *__restrict__ dq, int64_t ldq) {
  float *row = dq + (int64_t)blockIdx.x * 16 * ldq + 4 * threadIdx.x;
#pragma unroll
  for (int r = 0; r < 16; ++r) *reinterpret_cast<f4 *>(row + r * ldq) = f4{0.0f, 0.0f, 0.0f, 0.0f};
}

template <bool ATOMIC>
__global__ void __launch_bounds__(256, 1) attn_bwd_keys_kernel(
    const float *Q, const float *K, const float *V, int64_t ldq, const float *P, const float *dO,
    int64_t ldo, const float *O, float *dq, float *dk, float *dv, int S, int H, float alpha) {
  // (no __restrict__: the loads must not move across the memory fences below)
  __shared__ __attribute__((aligned(1024))) float lds[kKeysLds];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hh = lane >> 5;
  int kg = blockIdx.x, z = blockIdx.y;
  {
    // XCD k (hardware ids k, k+8, ...) owns a contiguous run of heads
    const int nb = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    if ((nb & 7) == 0) {
      const int logical = (lin & 7) * (nb >> 3) + (lin >> 3);
      kg = logical % gridDim.x;
      z = logical / gridDim.x;
    }
  }
  const int b = z / H, head = z - b * H;
  const int k0 = kg * kKeyGroup, kw = k0 + 32 * wave;  // the group's and the wave's first key
  const int64_t tok0 = (int64_t)b * S;
  const float *Qz = Q + tok0 * ldq + head * kHeadDim;
  const float *Kz = K + tok0 * ldq + head * kHeadDim;
  const float *Vz = V + tok0 * ldq + head * kHeadDim;
  const float *dOz = dO + tok0 * ldo + head * kHeadDim;
  const float *Oz = O + tok0 * ldo + head * kHeadDim;
  // P rows of head z, and dq rows of (b, head): 32-bit byte offsets (the
  // launch keeps S * ldq below 2^29), row part in the scalar offset
  const __amdgpu_buffer_rsrc_t prs = numrs_hip::dev_rsrc(P + (int64_t)z * S * S, (int64_t)S * S * 4);
  const __amdgpu_buffer_rsrc_t qrs = numrs_hip::dev_rsrc(dq + tok0 * ldq + head * kHeadDim, (int64_t)S * ldq * 4);
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // K rows 32 wave .. +31 of the group by DMA: instruction it fills rows
  // 4 it .. 4 it + 3, lane l the 16-byte slot l % 16 of row 4 it + l / 16,
  // holding chunk slot ^ 8 when the row's bit 2 is set.
  {
    const float *src = Kz + (int64_t)(k0 + 32 * wave_u) * ldq;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int kk = 4 * it + (lane >> 4);
      const int chunk = (lane & 15) ^ (8 * ((kk >> 2) & 1));
      numrs_hip::lds_dma16(src, (uint32_t)(4 * ((int64_t)kk * ldq + 4 * chunk)),
                           base + 4u * (uint32_t)(kKsOff + 32 * wave_u * kHeadDim) + 1024u * it);
    }
  }
  // Q and dO rows 16 wave .. +15 of query block qb into tile buffer t, chunk
  // j of tile row r at slot j ^ (r % 16).
  auto stage_tiles = [&](int qb, int t) {
    const int r0 = qb * kRowsPerBlock + 16 * wave_u;
    const float *qs = Qz + (int64_t)r0 * ldq;
    const float *os = dOz + (int64_t)r0 * ldo;
    const uint32_t qd = base + 4u * (uint32_t)(kTileOff + t * kTileFloats + 16 * wave_u * kHeadDim);
    const uint32_t od = qd + 4u * (uint32_t)(kRowsPerBlock * kHeadDim);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int kk = 4 * it + (lane >> 4);  // (16 wave + kk) % 16 = kk
      const int chunk = (lane & 15) ^ kk;
      numrs_hip::lds_dma16(qs, (uint32_t)(4 * ((int64_t)kk * ldq + 4 * chunk)), qd + 1024u * it);
      numrs_hip::lds_dma16(os, (uint32_t)(4 * ((int64_t)kk * ldo + 4 * chunk)), od + 1024u * it);
    }
  };
  // P[q][key kw + c] for the lane's 32 queries of block qb, values
  // 4n .. 4n + 3 of them (n < 8)
  const int p_lane = 4 * (4 * hh * S + kw + c);  // query 4h, key kw + c
  auto load_p_part = [&](int qb, float (&pr)[2][16], int n) {
#pragma unroll
    for (int m = 4 * n; m < 4 * n + 4; ++m) {
      const int bi = m >> 4, i = m & 15;
      const int q = qb * kRowsPerBlock + 32 * bi + 8 * (i >> 2) + (i & 3);  // + 4h in p_lane
      pr[bi][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, p_lane, 4 * q * S, 0));
    }
  };
  // The softmax backward's row totals D = dO . O for the wave's tile rows
  // 16 wave + l / 4 of block qb: lane l multiplies 16 of the 64 products
  // (d = 16 (l % 4) ..), the four lanes of a row add in xor order, and the
  // first writes D to LDS.  The wave's dO rows are the ones it staged.
  auto load_o = [&](int qb, f4 (&of)[4]) {
    const float *src = Oz + (int64_t)(qb * kRowsPerBlock + 16 * wave + (lane >> 2)) * ldo + 16 * (lane & 3);
#pragma unroll
    for (int e = 0; e < 4; ++e) of[e] = *reinterpret_cast<const f4 *>(src + 4 * e);
  };
  auto row_totals = [&](int t, const f4 (&of)[4]) {
    const int r = 16 * wave + (lane >> 2);
    const float *os = lds + kTileOff + t * kTileFloats + kRowsPerBlock * kHeadDim;
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f4 d = *reinterpret_cast<const f4 *>(os + r * kHeadDim + 4 * ((4 * (lane & 3) + e) ^ (r & 15)));
#pragma unroll
      for (int u = 0; u < 4; ++u) sum += d[u] * of[e][u];
    }
    sum = quad_sum(sum);
    if ((lane & 3) == 0) lds[kDOff + r] = sum;
  };

  stage_tiles(0, 0);
  f4 vr[8];  // V[key kw + c][8g + 4h .. +3]
#pragma unroll
  for (int g = 0; g < 8; ++g)
    vr[g] = *reinterpret_cast<const f4 *>(Vz + (int64_t)(kw + c) * ldq + 8 * g + 4 * hh);
  float pr[2][16];
#pragma unroll
  for (int n = 0; n < 8; ++n) load_p_part(0, pr, n);
  f4 of[4];
  load_o(0, of);
  // Loads stay where they are written: no memory access or instruction moves
  // across this point (the explicit waits below count on what precedes them).
  auto pin = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  pin();
  __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(0));
  row_totals(0, of);

  f16v dvacc[2], dkacc[2];
#pragma unroll
  for (int dj = 0; dj < 2; ++dj) {
    dvacc[dj] = f16v{};
    dkacc[dj] = f16v{};
  }
  const int nq = S / kRowsPerBlock;
  for (int qb = 0; qb < nq; ++qb) {
    const int t = qb & 1;
    __syncthreads();  // block qb's tiles (waited for by every wave) are in
    float prn[2][16];
    const bool more = qb + 1 < nq;
    if (more) {
      stage_tiles(qb + 1, t ^ 1);
      load_o(qb + 1, of);
    }
    pin();  // the prefetch goes out before this block's products (P's in the dV, dK loop)
    const float *qs = lds + kTileOff + t * kTileFloats;
    const float *os = qs + kRowsPerBlock * kHeadDim;

    // dP - D = dO V^T - D: the accumulators start at -D of their queries;
    // A = dO rows (query 32 bi + c), B = the wave's V fragments.  Operands
    // of step g + 1 are read before step g's MFMAs.
    f16v acc[2];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f4 d = *reinterpret_cast<const f4 *>(lds + kDOff + 32 * bi + 8 * g + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[bi][4 * g + e] = -d[e];
      }
    auto read_a = [&](int g, f4 (&a)[2]) {
#pragma unroll
      for (int bi = 0; bi < 2; ++bi) {
        const int r = 32 * bi + c;
        a[bi] = *reinterpret_cast<const f4 *>(os + r * kHeadDim + 4 * ((2 * g + hh) ^ (r & 15)));
      }
    };
    f4 a[2][2];
    read_a(0, a[0]);
#pragma unroll
    for (int g = 0; g < kHeadDim / 8; ++g) {
      if (g + 1 < kHeadDim / 8) read_a(g + 1, a[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this step's MFMAs
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int bi = 0; bi < 2; ++bi)
          acc[bi] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[g & 1][bi][j], vr[g][j], acc[bi], 0, 0, 0);
    }
    // dS = P * (dP - D)
    float ds[2][16];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int i = 0; i < 16; ++i) ds[bi][i] = pr[bi][i] * acc[bi][i];
    // dV += P^T dO, dK += dS^T Q: A = dO or Q at [query][32 dj + c], group n
    // = (bi, g) of four queries; group n + 1's operands are read before group
    // n's MFMAs.
    auto read_grp = [&](int n, float (&ao)[4][2], float (&aq)[4][2]) {
      const int bi = n >> 2, g = n & 3;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 32 * bi + 8 * g + 4 * hh + j;
#pragma unroll
        for (int dj = 0; dj < 2; ++dj) {
          const int col = 4 * (((32 * dj + c) >> 2) ^ (r & 15)) + (c & 3);
          ao[j][dj] = os[r * kHeadDim + col];
          aq[j][dj] = qs[r * kHeadDim + col];
        }
      }
    };
    float ao[2][4][2], aq[2][4][2];
    read_grp(0, ao[0], aq[0]);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      if (n + 1 < 8) read_grp(n + 1, ao[(n + 1) & 1], aq[(n + 1) & 1]);
      if (more) load_p_part(qb + 1, prn, n);  // the next block's P, four loads per group
      pin();
      const int bi = n >> 2, g = n & 3;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int dj = 0; dj < 2; ++dj) {
          dvacc[dj] = __builtin_amdgcn_mfma_f32_32x32x2f32(ao[n & 1][j][dj], pr[bi][4 * g + j],
                                                           dvacc[dj], 0, 0, 0);
          dkacc[dj] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[n & 1][j][dj], ds[bi][4 * g + j],
                                                           dkacc[dj], 0, 0, 0);
        }
    }
    // dS -> LDS [query][group key]
    {
      const int kc = 32 * wave + c;
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int q = 32 * bi + 8 * (i >> 2) + 4 * hh + (i & 3);
          lds[kDsOff + q * kKeyGroup + 4 * ((kc >> 2) ^ (q & 31)) + (c & 3)] = ds[bi][i];
        }
    }
    __syncthreads();
    // dQ block (query half qi, d half di) = dS K over the group's keys; step
    // g + 1's operands are read before step g's MFMAs
    const int qi = wave_u >> 1, di = wave_u & 1;  // wave-uniform (scalar offsets below)
    f16v qacc = f16v{};
    {
      const int r = 32 * qi + c;
      auto read_q = [&](int g, f4 &ad, float (&kv)[4]) {
        ad = *reinterpret_cast<const f4 *>(lds + kDsOff + r * kKeyGroup + 4 * ((2 * g + hh) ^ (r & 31)));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kk = 8 * g + 4 * hh + j;  // (kk >> 2) & 1 == hh
          kv[j] = lds[kKsOff + kk * kHeadDim + ((32 * di + c) ^ (32 * hh))];
        }
      };
      f4 ad[2];
      float kv[2][4];
      read_q(0, ad[0], kv[0]);
#pragma unroll
      for (int g = 0; g < kKeyGroup / 8; ++g) {
        if (g + 1 < kKeyGroup / 8) read_q(g + 1, ad[(g + 1) & 1], kv[(g + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          qacc = __builtin_amdgcn_mfma_f32_32x32x2f32(ad[g & 1][j], kv[g & 1][j], qacc, 0, 0, 0);
      }
    }
    // the next block's tiles and P have landed (and the last block's dQ
    // writes are done) before this block's dQ leaves
    pin();
    __builtin_amdgcn_s_waitcnt(numrs_hip::wait_vm(0));
    if (more) {
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int i = 0; i < 16; ++i) pr[bi][i] = prn[bi][i];
      // every wave read this block's D at its start, before the dS barrier
      row_totals(t ^ 1, of);
    }
    {
      const int lane_off = 4 * (int)(4 * hh * ldq + 32 * di + c);  // query + 4h, column 32 di + c
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = qb * kRowsPerBlock + 32 * qi + 8 * (i >> 2) + (i & 3);
        if constexpr (ATOMIC)
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(alpha * qacc[i], qrs, lane_off, 4 * q * (int)ldq, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, alpha * qacc[i]), qrs, lane_off,
                                                4 * q * (int)ldq, 0);
      }
    }
  }
  // dV and dK rows of the wave's keys: lane (c, h) holds key kw + c at d
  // = 32 dj + 8 g + 4 h + (0..3)
#pragma unroll
  for (int dj = 0; dj < 2; ++dj)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t off = (tok0 + kw + c) * ldq + head * kHeadDim + 32 * dj + 8 * g + 4 * hh;
      const f4 v = {dvacc[dj][4 * g], dvacc[dj][4 * g + 1], dvacc[dj][4 * g + 2], dvacc[dj][4 * g + 3]};
      const f4 w = {alpha * dkacc[dj][4 * g], alpha * dkacc[dj][4 * g + 1], alpha * dkacc[dj][4 * g + 2],
                    alpha * dkacc[dj][4 * g + 3]};
      *reinterpret_cast<f4 *>(dv + off) = v;
      *reinterpret_cast<f4 *>(dk + off) = w;
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
// accumulated), the key-block kernel; otherwise the row-block path above.
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
  const bool atomic = S > kKeyGroup;  // two key groups add into dq
  if (atomic) {
    // B S < 2^24 rows (B H < 65536, S <= 256), D / 4 <= 1024 threads
    attn_bwd_zero_kernel<<<(unsigned)(B * S / 16), (unsigned)(D / 4), 0, ctx->stream>>>(dq, li);
    if (int rc = numrs_hip::check_launch(ctx, "attn_bwd_zero_kernel")) return rc;
  }
  const dim3 grid((unsigned)(S / kKeyGroup), (unsigned)(B * H));
  if (atomic)
    attn_bwd_keys_kernel<true><<<grid, 256, 0, ctx->stream>>>(q, k, v, li, P, dout, lo, out, dq, dk,
                                                             dv, (int)S, (int)H, alpha);
  else
    attn_bwd_keys_kernel<false><<<grid, 256, 0, ctx->stream>>>(q, k, v, li, P, dout, lo, out, dq,
                                                              dk, dv, (int)S, (int)H, alpha);
  return numrs_hip::check_launch(ctx, "attn_bwd_keys_kernel");
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
