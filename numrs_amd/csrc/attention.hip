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
// 16-byte store.  The softmax follows the row kernel's arithmetic: m = max,
// e = expf(s - m), P = e * (1/sum e).
template <int MODE, int BJ>
__global__ void __launch_bounds__(256) attn_rows_kernel(const float *__restrict__ X,
                                                        const float *__restrict__ W,
                                                        const float *__restrict__ P,
                                                        float *__restrict__ out, int S, int H,
                                                        int64_t ld, float alpha) {
  __shared__ float red[4][kRowsPerBlock];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int z = blockIdx.y, b = z / H, head = z - b * H;
  const int row0 = blockIdx.x * kRowsPerBlock, col0 = wave * 32 * BJ;
  const float *Xz = X + (int64_t)b * S * ld + (int64_t)head * kHeadDim;
  const float *Wz = W + (int64_t)b * S * ld + (int64_t)head * kHeadDim;
  const int64_t zoff = (int64_t)z * S * S;

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
      a[bi] = *reinterpret_cast<const f4 *>(Xz + (int64_t)(row0 + 32 * bi + c) * ld + 8 * g + 4 * hh);
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
      w[bj] = *reinterpret_cast<const f4 *>(Wz + (int64_t)(col0 + 32 * bj + c) * ld + 8 * g + 4 * hh);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < BJ; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[bj][j], a[bi][j], acc[bi][bj], 0, 0, 0);
  }

  // Register i of block (bi, bj) holds row row0 + 32*bi + c and column
  // col0 + 32*bj + 8*(i/4) + 4*hh + (i%4).
  auto col_of = [&](int bj, int i4) { return col0 + 32 * bj + 8 * i4 + 4 * hh; };
  auto row_ptr = [&](float *base, int bi) { return base + zoff + (int64_t)(row0 + 32 * bi + c) * S; };
  // Row totals over the wave's columns (in-lane, then the other half-wave),
  // then over the four waves: op 0 = max, 1 = sum.
  auto row_reduce = [&](float (&v)[2], int op) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const float o = __shfl_xor(v[bi], 32, 64);
      v[bi] = op == 0 ? fmaxf(v[bi], o) : v[bi] + o;
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
  if (MODE == 0) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      float m = -INFINITY;
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          acc[bi][bj][i] = alpha * acc[bi][bj][i];
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
          const float e = expf(acc[bi][bj][i] - t[bi]);
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
          const f4 v = {acc[bi][bj][4 * i4] * inv, acc[bi][bj][4 * i4 + 1] * inv,
                        acc[bi][bj][4 * i4 + 2] * inv, acc[bi][bj][4 * i4 + 3] * inv};
          *reinterpret_cast<f4 *>(dst + col_of(bj, i4)) = v;
        }
    }
  } else {
    f4 p[2][BJ][4];
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const float *src = row_ptr(const_cast<float *>(P), bi);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) p[bi][bj][i4] = *reinterpret_cast<const f4 *>(src + col_of(bj, i4));
    }
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
          for (int e = 0; e < 4; ++e)
            v[e] = p[bi][bj][i4][e] * (acc[bi][bj][4 * i4 + e] - t[bi]);
          *reinterpret_cast<f4 *>(dst + col_of(bj, i4)) = v;
        }
    }
  }
}

// Whether the fused row-block kernel takes this shape: dh = 64, S a multiple
// of 128 up to 512, 16-byte aligned rows and probability matrices.
bool rows_fit(int64_t S, int64_t dh, int64_t D, const void *x, const void *w, const void *p) {
  return dh == kHeadDim && S % 128 == 0 && S <= 512 && D % 4 == 0 && numrs_hip::aligned16(x) &&
         numrs_hip::aligned16(w) && numrs_hip::aligned16(p);
}

template <int MODE>
int launch_rows(numrs_hip_ctx *ctx, const float *X, const float *W, const float *P, float *out,
                int64_t B, int64_t S, int64_t H, int64_t D, float alpha) {
  const dim3 grid((unsigned)(S / kRowsPerBlock), (unsigned)(B * H));
  switch (S / 128) {
    case 1: attn_rows_kernel<MODE, 1><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, (int)S, (int)H, D, alpha); break;
    case 2: attn_rows_kernel<MODE, 2><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, (int)S, (int)H, D, alpha); break;
    case 3: attn_rows_kernel<MODE, 3><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, (int)S, (int)H, D, alpha); break;
    default: attn_rows_kernel<MODE, 4><<<grid, 256, 0, ctx->stream>>>(X, W, P, out, (int)S, (int)H, D, alpha); break;
  }
  return numrs_hip::check_launch(ctx, "attn_rows_kernel");
}

int check(numrs_hip_ctx *ctx, int64_t B, int64_t S, int64_t H, int64_t D) {
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0 || D % H != 0)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_SHAPE,
                           "attention: batch, seq, heads > 0 and dim divisible by heads");
  return NUMRS_HIP_OK;
}

}  // namespace

extern "C" {

int numrs_hip_attention_forward(numrs_hip_ctx *ctx, const float *q, const float *k, const float *v,
                                float *P, float *out, int64_t B, int64_t S, int64_t H,
                                int64_t D) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, S, H, D)) return rc;
  if (!q || !k || !v || !P || !out)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "attention_forward: null pointer");
  const int64_t dh = D / H, Z = B * H;
  const float alpha = 1.0f / sqrtf((float)dh);
  if (rows_fit(S, dh, D, q, k, P) && B * H < 65536) {
    // P = softmax_rows(alpha * Q K^T) in one kernel
    if (int rc = launch_rows<0>(ctx, q, k, nullptr, P, B, S, H, D, alpha)) return rc;
    return numrs_hip_gemm(ctx, P, S, v, D, out, D, S, S, dh, 0, 0, 1.0f, 0, Z, H, H * S * S,
                          S * S, S * D, dh, S * D, dh);
  }
  // S_z = alpha * Q_z K_z^T  -> P (row-major [S, S] per z)
  if (int rc = numrs_hip_gemm(ctx, q, D, k, D, P, S, S, dh, S, 0, 1, alpha, 0, Z, H, S * D, dh,
                              S * D, dh, H * S * S, S * S))
    return rc;
  // in-place row softmax (each row is read completely before it is written)
  if (int rc = numrs_hip_softmax_forward(ctx, P, P, Z * S, S, 1.0f)) return rc;
  // O_z = P_z V_z
  return numrs_hip_gemm(ctx, P, S, v, D, out, D, S, S, dh, 0, 0, 1.0f, 0, Z, H, H * S * S, S * S,
                        S * D, dh, S * D, dh);
}

int numrs_hip_attention_backward(numrs_hip_ctx *ctx, const float *q, const float *k,
                                 const float *v, const float *P, const float *dout, float *dq,
                                 float *dk, float *dv, int64_t B, int64_t S, int64_t H, int64_t D,
                                 int accumulate) {
  NRS_CHECK_CTX(ctx);
  if (int rc = check(ctx, B, S, H, D)) return rc;
  if (!q || !k || !v || !P || !dout)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "attention_backward: null input");
  const int64_t dh = D / H, Z = B * H;
  const float alpha = 1.0f / sqrtf((float)dh);
  // dV_z = P_z^T dO_z
  if (dv)
    if (int rc = numrs_hip_gemm(ctx, P, S, dout, D, dv, D, S, S, dh, 1, 0, 1.0f, accumulate, Z, H,
                                H * S * S, S * S, S * D, dh, S * D, dh))
      return rc;
  if (!dq && !dk) return NUMRS_HIP_OK;
  // dS lives in a block of its own: the dQ/dK products below may split their
  // reduction and write partials to the context workspace while reading dS.
  numrs_hip::TempBlock dSb(ctx);
  if (int rc = dSb.alloc((size_t)(Z * S * S) * sizeof(float))) return rc;
  float *dP = dSb.f();
  if (rows_fit(S, dh, D, dout, v, P) && rows_fit(S, dh, D, dout, v, dP) && B * H < 65536) {
    // dS = P * (dP - rowsum(dP * P)) with dP = dO V^T, in one kernel
    if (int rc = launch_rows<1>(ctx, dout, v, P, dP, B, S, H, D, 1.0f)) return rc;
  } else {
    // dP_z = dO_z V_z^T
    if (int rc = numrs_hip_gemm(ctx, dout, D, v, D, dP, S, S, dh, S, 0, 1, 1.0f, 0, Z, H, S * D,
                                dh, S * D, dh, H * S * S, S * S))
      return rc;
    // dS = P * (dP - rowsum(dP * P)), in place over dP
    if (int rc = numrs_hip_softmax_backward(ctx, P, dP, dP, Z * S, S, 0)) return rc;
  }
  // dQ_z = alpha * dS_z K_z ;  dK_z = alpha * dS_z^T Q_z  (one launch for both)
  const numrs_hip::BatchedMat dS{dP, S, H * S * S, S * S};
  const numrs_hip::BatchedMat Km{k, D, S * D, dh}, Qm{q, D, S * D, dh};
  const numrs_hip::BatchedOut dQ{dq, D, S * D, dh}, dK{dk, D, S * D, dh};
  return numrs_hip::gemm_nn_tn_pair(ctx, dS, Km, dQ, Qm, dK, S, S, dh, alpha, accumulate, Z, H);
}

}  // extern "C"
