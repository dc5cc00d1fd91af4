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
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)(Z * S * S) * sizeof(float), &ws)) return rc;
  float *dP = static_cast<float *>(ws);
  // dP_z = dO_z V_z^T
  if (int rc = numrs_hip_gemm(ctx, dout, D, v, D, dP, S, S, dh, S, 0, 1, 1.0f, 0, Z, H, S * D, dh,
                              S * D, dh, H * S * S, S * S))
    return rc;
  // dS = P * (dP - rowsum(dP * P)), in place over dP
  if (int rc = numrs_hip_softmax_backward(ctx, P, dP, dP, Z * S, S, 0)) return rc;
  // dQ_z = alpha * dS_z K_z ;  dK_z = alpha * dS_z^T Q_z  (one launch for both)
  const numrs_hip::BatchedMat dS{dP, S, H * S * S, S * S};
  const numrs_hip::BatchedMat Km{k, D, S * D, dh}, Qm{q, D, S * D, dh};
  const numrs_hip::BatchedOut dQ{dq, D, S * D, dh}, dK{dk, D, S * D, dh};
  return numrs_hip::gemm_nn_tn_pair(ctx, dS, Km, dQ, Qm, dK, S, S, dh, alpha, accumulate, Z, H);
}

}  // extern "C"
