/*
 * numrs_hip.h -- C ABI of the MI355X (gfx950) backend for numrs's reverse-mode
 * autograd hot path.
 *
 * The reference (rjaguiluz/numrs, Rust) runs every backward node on the host:
 * each BackwardFn (numrs-core/src/autograd/mod.rs:136) borrows host Arrays and
 * returns freshly allocated ones, and Tensor::backward
 * (autograd/tensor.rs:173-215) adds them into the inputs' grad cells with
 * accumulate_gradient (tensor.rs:120-132).  This library replaces those bodies
 * with HIP kernels on device-resident buffers, so a Rust `hip` backend under
 * numrs-core/src/backend/hip would bind exactly these symbols.
 *
 * Conventions
 *   - Every pointer argument that names tensor data is a DEVICE pointer owned
 *     by the caller (allocate with numrs_hip_malloc or any hipMalloc).  fp32,
 *     row-major, contiguous.
 *   - Every call is asynchronous on the context's stream and returns an int
 *     status: NUMRS_HIP_OK (0) or a negative code; the message is available
 *     from numrs_hip_last_error(ctx).  No call aborts the process.
 *   - `accumulate` = 1 means out += result (the reference's
 *     accumulate_gradient); 0 means out = result.
 *   - Entry points that need scratch memory take it from the context's
 *     workspace, which grows on first use of a larger size (numrs_hip_reserve
 *     pre-sizes it).
 *   - One context per host thread; the reference autograd is single-threaded
 *     (Rc/RefCell, thread-local grad mode: autograd/mod.rs:194-206).
 */
#ifndef NUMRS_HIP_H
#define NUMRS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct numrs_hip_ctx numrs_hip_ctx;

enum {
  NUMRS_HIP_OK = 0,
  NUMRS_HIP_E_INVALID = -1, /* null pointer, negative size, bad enum value   */
  NUMRS_HIP_E_SHAPE = -2,   /* shapes that do not fit together              */
  NUMRS_HIP_E_HIP = -3,     /* a HIP runtime call failed                    */
  NUMRS_HIP_E_NOMEM = -4,   /* device allocation failed                     */
  NUMRS_HIP_E_NODEV = -5    /* no usable gfx950 device                      */
};

/* Unbroadcast modes for bias / broadcast-reduce gradients. */
enum {
  /* Column/axis reduction to the target shape (what the mathematics asks). */
  NUMRS_HIP_UNBROADCAST_CORRECT = 0,
  /* The reference's behaviour: any shape mismatch becomes a full sum
   * (backward.rs:12-39) that accumulate_gradient's zip() adds into element 0
   * only (tensor.rs:120-132). */
  NUMRS_HIP_UNBROADCAST_REFERENCE = 1
};

/* Unary backward kinds: dx = g * f'(.) with the saved forward value `v`. */
enum {
  NUMRS_HIP_RELU = 0,    /* v = x (input):  x > 0 ? g : 0      backward.rs:152-163 */
  NUMRS_HIP_SIGMOID = 1, /* v = s (output): (g*s)*(1-s)         backward.rs:166-177 */
  NUMRS_HIP_TANH = 2,    /* v = y (output): g*(1-y*y)           backward.rs:503-517 */
  NUMRS_HIP_EXP = 3,     /* v = e (output): g*e                 backward.rs:180-191 */
  NUMRS_HIP_LOG = 4,     /* v = x (input):  g/x                 backward.rs:194-205 */
  NUMRS_HIP_GELU = 5,    /* v = x (input):  g*(Phi(x)+x*phi(x)) exact-erf GELU (no reference op) */
  NUMRS_HIP_SQRT = 6,    /* v = x (input):  g*(x^-0.5*0.5)      backward.rs:441-463 */
  NUMRS_HIP_SIN = 7,     /* v = x (input):  g*cos(x)            backward.rs:466-472 */
  NUMRS_HIP_COS = 8,     /* v = x (input):  g*(sin(x)*-1)       backward.rs:475-483 */
  NUMRS_HIP_TAN = 9,     /* v = t (output): g*(1+t*t)           backward.rs:486-500 */
  NUMRS_HIP_POW = 10     /* v = x (input):  g*(x^(p-1)*p)       backward.rs:407-438 */
};

/* Binary backward kinds (same-shape operands; broadcasting is a separate
 * numrs_hip_sum_to_shape on the result). */
enum {
  NUMRS_HIP_ADD = 0, /* dx = g,   dy = g                 backward.rs:43-54   */
  NUMRS_HIP_SUB = 1, /* dx = g,   dy = g*-1              backward.rs:57-70   */
  NUMRS_HIP_MUL = 2, /* dx = g*y, dy = g*x               backward.rs:74-87   */
  NUMRS_HIP_DIV = 3  /* dx = g/y, dy = (g*(x/(y*y)))*-1  backward.rs:90-109  */
};

/* Optimizers beyond SGD and Adam (autograd/optim/mod.rs:1-41).  Their
 * hyperparameters are passed as a float array in the reference constructor's
 * order; the state slots s1/s2 per kind are listed. */
enum {
  NUMRS_HIP_OPT_ADAMW = 0,    /* lr, b1, b2, eps, wd;            s1 m, s2 v      adamw.rs:50-83 */
  NUMRS_HIP_OPT_RMSPROP = 1,  /* lr, alpha, eps, wd, momentum;   s1 v, s2 buf*   rmsprop.rs:47-81 */
  NUMRS_HIP_OPT_ADAGRAD = 2,  /* lr, eps, wd;                    s1 sum g^2      adagrad.rs:43-63 */
  NUMRS_HIP_OPT_NADAM = 3,    /* lr, b1, b2, eps, wd;            s1 m, s2 v      nadam.rs:57-90 */
  NUMRS_HIP_OPT_RADAM = 4,    /* lr, b1, b2, eps, wd;            s1 m, s2 v      radam.rs:53-86 */
  NUMRS_HIP_OPT_ADADELTA = 5, /* rho, eps, wd;                   s1 E[g^2], s2 E[dx^2]  adadelta.rs:53-81 */
  NUMRS_HIP_OPT_ADABOUND = 6, /* lr, final_lr, b1, b2, eps, wd, gamma; s1 m, s2 v  adabound.rs:70-107 */
  NUMRS_HIP_OPT_RPROP = 7,    /* lr_init, eta+, eta-, lr_min, lr_max; s1 step sizes (start
                                 at lr_init), s2 previous gradient (start at 0)  rprop.rs:63-94 */
  NUMRS_HIP_OPT_LAMB = 8      /* lr, b1, b2, eps, wd;            s1 m, s2 v      lamb.rs:63-96 */
};
/* (* RMSprop's s2 is used only when momentum > 0.) */

/* LR schedulers (autograd/optim/schedulers.rs); hyperparameters in the
 * constructor's order, counts passed as floats. */
enum {
  NUMRS_HIP_SCHED_STEP = 0,        /* step_size, gamma          schedulers.rs:20-61 */
  NUMRS_HIP_SCHED_EXPONENTIAL = 1, /* gamma                     schedulers.rs:68-102 */
  NUMRS_HIP_SCHED_COSINE = 2,      /* t_max, eta_min            schedulers.rs:113-153 */
  NUMRS_HIP_SCHED_PLATEAU = 3,     /* factor, patience, min_lr  schedulers.rs:172-238 */
  NUMRS_HIP_SCHED_WARMUP = 4       /* warmup_steps, start_lr    schedulers.rs:249-295 */
};

/* ---------------------------------------------------------------------- */
/* Context, memory, streams, timing                                        */
/* ---------------------------------------------------------------------- */

/* Creates a context on HIP device `device` with its own stream (default
 * priority).  Fails with NUMRS_HIP_E_NODEV when the device is absent or not
 * gfx950.  Replaces nothing in the reference (its ops run on the caller's
 * thread); it is the state a backend/hip module would hold, like
 * DispatchTable's OnceCell (backend/dispatch.rs:713-721). */
int numrs_hip_create(int device, numrs_hip_ctx **out);
int numrs_hip_destroy(numrs_hip_ctx *ctx);
/* Message of the last failed call on this context ("" if none). */
const char *numrs_hip_last_error(numrs_hip_ctx *ctx);
/* Message of the last failed numrs_hip_create on this thread. */
const char *numrs_hip_create_error(void);
/* Number of compute units and the gcn arch name ("gfx950..."). */
int numrs_hip_device_info(numrs_hip_ctx *ctx, int *num_cus, char *arch, size_t arch_len);

/* Device memory.  Replaces the host Vec<f32> behind Array::data
 * (array/array.rs:14-22) and the zero-filled grad cell of Tensor::new
 * (autograd/tensor.rs:41-59). */
int numrs_hip_malloc(numrs_hip_ctx *ctx, size_t bytes, void **dptr);
int numrs_hip_free(numrs_hip_ctx *ctx, void *dptr);
int numrs_hip_upload(numrs_hip_ctx *ctx, void *dst, const void *host_src, size_t bytes);
int numrs_hip_download(numrs_hip_ctx *ctx, void *host_dst, const void *src, size_t bytes);
int numrs_hip_copy(numrs_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
/* No counterpart in the reference: a measurement aid for callers that time
 * the library against the device.  One launch streams n floats (n % 4 == 0,
 * operands 16-byte aligned) in the access pattern of the library's streaming
 * kernels (float4, non-temporal from 2^23 floats on): it reads the first
 * `reads` (0..3) of a, b, c and writes their sum to y and, for writes = 2,
 * to z; writes = 0 stores nothing (y must still hold one float per 2048
 * elements).  Its time is the ceiling a kernel moving the same bytes in the
 * same read/write mix and number of launches can reach. */
int numrs_hip_stream_probe(numrs_hip_ctx *ctx, const float *a, const float *b, const float *c,
                           float *y, float *z, int64_t n, int reads, int writes);
/* Fills `n` floats with `value` by a kernel (safe inside HIP graph capture).
 * value = 0 is Tensor::zero_grad (autograd/tensor.rs:135-142). */
int numrs_hip_fill(numrs_hip_ctx *ctx, float *dst, int64_t n, float value);
/* Waits for all work queued on the context's stream. */
int numrs_hip_sync(numrs_hip_ctx *ctx);
/* Grows the workspace to at least `bytes` (otherwise it grows on demand). */
int numrs_hip_reserve(numrs_hip_ctx *ctx, size_t bytes);
/* The context's hipStream_t, for callers that enqueue their own work. */
void *numrs_hip_stream(numrs_hip_ctx *ctx);

/* HIP events recorded on the context's stream; slot in [0, 256). */
int numrs_hip_timer_record(numrs_hip_ctx *ctx, int slot);
int numrs_hip_timer_elapsed_ms(numrs_hip_ctx *ctx, int slot_start, int slot_end, float *ms);

/* No counterpart in the reference (numrs runs a training step's ops one by
 * one, train.rs:159-183): graph recording and replay, for training loops
 * that repeat one fixed step (same shapes, same buffers; new data copied
 * into the input tensors between replays) and want one launch per step.
 * numrs_hip_graph_begin starts recording the context's stream: the calls
 * that follow queue nothing, they are recorded.  numrs_hip_graph_end turns
 * the recording into a replayable graph; numrs_hip_graph_launch queues one
 * replay on the context's stream, ordered with other work there.
 *   - Run the step once before recording it: a workspace that must grow,
 *     host uploads or downloads and synchronisations fail while recording
 *     (numrs_hip_graph_abort then discards the recording; the recorded calls
 *     never ran, so zero the gradients they would have written).
 *   - Kernel arguments are those of the recording: host-side values that
 *     change per step (a scheduler's learning rate, Adam's step count) are
 *     not updated by replays, and the engine refuses to record optimizers
 *     whose step depends on a host-side step count.
 *   - Tensors created during the recording must stay alive while the graph
 *     is replayed; blocks they release during the recording are held by the
 *     graph until numrs_hip_graph_destroy.
 *   - Eager calls between replays may grow the context's workspace: while
 *     any graph exists the old region is kept (the graph's kernels address
 *     it) and freed when the last graph is destroyed.
 *   - numrs_hip_graph_destroy during another recording returns 0 and
 *     destroys the graph when that recording ends or is aborted. */
typedef struct numrs_hip_graph numrs_hip_graph;
int numrs_hip_graph_begin(numrs_hip_ctx *ctx);
int numrs_hip_graph_end(numrs_hip_ctx *ctx, numrs_hip_graph **out);
int numrs_hip_graph_abort(numrs_hip_ctx *ctx);
int numrs_hip_graph_launch(numrs_hip_graph *g);
int numrs_hip_graph_destroy(numrs_hip_graph *g);

/* ---------------------------------------------------------------------- */
/* Dense contractions (fp32 MFMA)                                          */
/* ---------------------------------------------------------------------- */

/* matmul_backward (autograd/backward.rs:113-149) for C[M,N] = A[M,K] @ B[K,N]:
 *   dA[M,K] = dC @ B^T,  dB[K,N] = A^T @ dC.
 * dA == NULL or dB == NULL skips that gradient (the reference always computes
 * both; skipping is what its caller discards at tensor.rs:205-209).  Both
 * products run in ONE launch of an LDS-tiled v_mfma_f32_32x32x2f32 kernel. */
int numrs_hip_matmul_backward(numrs_hip_ctx *ctx, const float *dC, const float *A,
                              const float *B, float *dA, float *dB, int64_t M, int64_t K,
                              int64_t N, int accumulate);

/* The same for `batch` independent products laid out with element strides
 * stride_a, stride_b, stride_c between consecutive matrices (dA/dB use the
 * A/B strides).  Attention's batched grads use this; the reference has only
 * 2-D matmul (backward.rs:118-120). */
int numrs_hip_matmul_backward_batched(numrs_hip_ctx *ctx, const float *dC, const float *A,
                                      const float *B, float *dA, float *dB, int64_t batch,
                                      int64_t M, int64_t K, int64_t N, int64_t stride_a,
                                      int64_t stride_b, int64_t stride_c, int accumulate);

/* General product C[M,N] (+)= op(A) @ op(B), op = transpose when trans_* = 1
 * (A stored [K,M] / B stored [N,K]).  The forward of Tensor::matmul
 * (autograd/ops.rs:101-119 -> ops::matmul -> DispatchTable.matmul,
 * backend/dispatch.rs:69-93) and the Linear forward x @ W^T
 * (autograd/nn.rs:217-235) without materialising W^T. */
int numrs_hip_matmul(numrs_hip_ctx *ctx, const float *A, const float *B, float *C, int64_t M,
                     int64_t K, int64_t N, int trans_a, int trans_b, int accumulate);

/* No counterpart in the reference: where the products of one call cut their
 * reduction into split-K ranges (weight gradients over many tokens), how the
 * partial products are added.  FUSED (the default): inside the products' own
 * launch -- the grid's last workgroups (or the last split to arrive) add each
 * output block's partials once all of its splits have stored them, with no
 * workgroup waiting for another.  SEPARATE: one more launch after the
 * products.  Both add the splits in the same order with the same
 * arithmetic: the same bits. */
#define NUMRS_HIP_SPLIT_REDUCE_FUSED 0
#define NUMRS_HIP_SPLIT_REDUCE_SEPARATE 1
int numrs_hip_set_split_reduction(numrs_hip_ctx *ctx, int mode);

/* Batched form of numrs_hip_matmul with element strides between matrices. */
int numrs_hip_matmul_batched(numrs_hip_ctx *ctx, const float *A, const float *B, float *C,
                             int64_t batch, int64_t M, int64_t K, int64_t N, int64_t stride_a,
                             int64_t stride_b, int64_t stride_c, int trans_a, int trans_b,
                             int accumulate);

/* Linear layer y[T,out] = x[T,in] @ W[out,in]^T + b (b may be NULL) as one
 * MFMA product with the bias added in its epilogue.  Same values as the
 * reference's Transpose -> MatMul -> Add node sequence (autograd/nn.rs:217-235)
 * without materialising W^T. */
int numrs_hip_linear_forward(numrs_hip_ctx *ctx, const float *x, const float *W, const float *b,
                             float *y, int64_t T, int64_t in, int64_t out);
/* Its backward from g = dL/dy: dx = g @ W and dW = g^T @ x in one launch
 * (what matmul_backward + transpose_backward compute for those nodes,
 * backward.rs:113-149, 305-312), db = unbroadcast(g) in `mode`
 * (backward.rs:43-54).  Any of dx/dW/db may be NULL; one accumulate flag per
 * output. */
int numrs_hip_linear_backward(numrs_hip_ctx *ctx, const float *g, const float *x, const float *W,
                              float *dx, float *dW, float *db, int64_t T, int64_t in, int64_t out,
                              int acc_dx, int acc_dw, int acc_db, int mode);
/* No counterpart in the reference: the Linear layer followed by ReLU
 * (nn.rs:217-235, then ReLU::forward, nn.rs:306-320), y = max(x @ W^T + b, 0)
 * with the ReLU forward kernel's x.max(0), applied in the product's
 * epilogue. */
int numrs_hip_linear_relu_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                  const float *b, float *y, int64_t T, int64_t in, int64_t out);
/* Its backward from g = dL/dy, y the forward's output: the pre-activation
 * gradient (y > 0) ? g : 0 -- relu_backward's strict mask (backward.rs:152-163);
 * y > 0 exactly where the pre-activation is > 0 -- then the Linear backward
 * as numrs_hip_linear_backward.  Small products apply the mask as the GEMM
 * loads g (dx, dW and db in one launch); larger ones form the masked
 * gradient first. */
int numrs_hip_linear_relu_backward(numrs_hip_ctx *ctx, const float *g, const float *y,
                                   const float *x, const float *W, float *dx, float *dW,
                                   float *db, int64_t T, int64_t in, int64_t out, int acc_dx,
                                   int acc_dw, int acc_db, int mode);
/* No counterpart in the reference: the Linear layer followed by GELU (the
 * exact-erf GELU of the unary kernels), y = GELU(x @ W^T + b), with the
 * pre-activation x @ W^T + b also stored in `pre` [T, out] (not aliasing y)
 * by the product's epilogue -- the values of numrs_hip_linear_forward then
 * numrs_hip_unary_forward(GELU), bit for bit. */
int numrs_hip_linear_gelu_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                  const float *b, float *y, float *pre, int64_t T, int64_t in,
                                  int64_t out);
/* Its backward from g = dL/dy: g * GELU'(pre) (numrs_hip_unary_backward),
 * then numrs_hip_linear_backward on it. */
int numrs_hip_linear_gelu_backward(numrs_hip_ctx *ctx, const float *g, const float *pre,
                                   const float *x, const float *W, float *dx, float *dW,
                                   float *db, int64_t T, int64_t in, int64_t out, int acc_dx,
                                   int acc_dw, int acc_db, int mode);
/* No counterpart in the reference: y = res + (x @ W^T + b), res [T, out] (may
 * alias y), the residual added in the product's epilogue after the bias --
 * the values of numrs_hip_linear_forward followed by an elementwise add
 * (Linear::forward, nn.rs:217-235, then ops::add), bit for bit.  Its backward
 * is numrs_hip_linear_backward from g plus dres = g. */
int numrs_hip_linear_residual_forward(numrs_hip_ctx *ctx, const float *x, const float *W,
                                      const float *b, const float *res, float *y, int64_t T,
                                      int64_t in, int64_t out);

/* General strided product, the building block of attention's batched
 * gradients: for z in [0, batch), with zo = z / batch_inner and
 * zi = z % batch_inner, operand A_z starts at A + zo*sa_outer + zi*sa_inner
 * with leading dimension lda (likewise B_z, C_z), and
 *   C_z[M,N] (+)= alpha * op(A_z) @ op(B_z),  op = transpose when trans_* = 1.
 * Two batch levels address head-interleaved layouts ([batch, seq, heads,
 * dim]) in place.  No reference counterpart (its matmul is 2-D only,
 * backward.rs:118-120). */
int numrs_hip_gemm(numrs_hip_ctx *ctx, const float *A, int64_t lda, const float *B, int64_t ldb,
                   float *C, int64_t ldc, int64_t M, int64_t K, int64_t N, int trans_a,
                   int trans_b, float alpha, int accumulate, int64_t batch, int64_t batch_inner,
                   int64_t sa_outer, int64_t sa_inner, int64_t sb_outer, int64_t sb_inner,
                   int64_t sc_outer, int64_t sc_inner);

/* Multi-head attention (no reference op).  q, k, v, out are
 * [B*S, D] row-major with head h of token (b, s) in columns [h*D/H, (h+1)*D/H).
 * Forward: P = softmax(Q K^T / sqrt(D/H)) per (b, h) into P [B*H, S, S],
 * out = P V.  Backward from the saved P: dV = P^T dO, dS = softmax_backward(P,
 * dO V^T), dQ = dS K / sqrt(dh), dK = dS^T Q / sqrt(dh); dq/dk/dv may be NULL;
 * uses B*H*S*S floats of workspace. */
int numrs_hip_attention_forward(numrs_hip_ctx *ctx, const float *q, const float *k, const float *v,
                                float *P, float *out, int64_t B, int64_t S, int64_t H, int64_t D);
int numrs_hip_attention_backward(numrs_hip_ctx *ctx, const float *q, const float *k,
                                 const float *v, const float *P, const float *dout, float *dq,
                                 float *dk, float *dv, int64_t B, int64_t S, int64_t H, int64_t D,
                                 int accumulate);
/* The same with explicit row strides: q, k, v (and dq, dk, dv) rows at
 * ld_qkv, out / dout rows at ld_out, both >= D.  With ld_qkv = 3D, q, k, v
 * can be the three column blocks of one packed [B*S, 3D] projection. */
int numrs_hip_attention_forward_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                        const float *v, int64_t ld_qkv, float *P, float *out,
                                        int64_t ld_out, int64_t B, int64_t S, int64_t H,
                                        int64_t D);
int numrs_hip_attention_backward_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                         const float *v, int64_t ld_qkv, const float *P,
                                         const float *dout, int64_t ld_out, float *dq, float *dk,
                                         float *dv, int64_t B, int64_t S, int64_t H, int64_t D,
                                         int accumulate);
/* The backward given also the forward's output out (rows at ld_out, like
 * dout), from which the softmax backward's row totals come as dO . O.  For
 * D/H = 64, S = 128 or 256, all three grads non-NULL and accumulate = 0 it
 * runs two kernels: one over query rows (dS = P (dP - dO . O) into a
 * B*H*S*S-float block of the context's memory, and dQ), then one over key
 * rows (dV and dK); every output element is written once, with no atomics.
 * Other calls behave as numrs_hip_attention_backward_strided. */
int numrs_hip_attention_backward_out_strided(numrs_hip_ctx *ctx, const float *q, const float *k,
                                             const float *v, int64_t ld_qkv, const float *P,
                                             const float *out, const float *dout, int64_t ld_out,
                                             float *dq, float *dk, float *dv, int64_t B, int64_t S,
                                             int64_t H, int64_t D, int accumulate);

/* How the two-layer LSTM calls run their recurrences (no reference op).
 * AUTO (the default): one persistent launch for all steps of the forward
 * and one for the backward where they apply (H1 = H2 = 256, 16-byte aligned
 * operands, not while recording a graph, and the occupancy query says the
 * device holds the whole grid at once); per-step launches otherwise.  The
 * persistent kernels start with an ordinary launch: the stream has finished
 * its earlier work by then, so the grid becomes resident as soon as work of
 * other streams leaves the CUs, and every wait for another workgroup is
 * bounded.  A persistent launch whose wait runs out returns its error from
 * the next call that synchronises the stream.  PER_STEP: always one launch
 * per diagonal step.  PLAIN_LAUNCH: the persistent kernels, ordinary launch
 * (AUTO's form; kept for scripts that name it).  COOPERATIVE: the persistent
 * kernels through hipLaunchCooperativeKernel, whose runtime guarantees
 * co-residency but adds about 25 us per launch on MI355X (and rocprofv3's
 * teardown faults after such launches).  All modes give the same bits. */
#define NUMRS_HIP_RECURRENCE_AUTO 0
#define NUMRS_HIP_RECURRENCE_PER_STEP 1
#define NUMRS_HIP_RECURRENCE_PLAIN_LAUNCH 2
#define NUMRS_HIP_RECURRENCE_COOPERATIVE 3
int numrs_hip_set_recurrence_mode(numrs_hip_ctx *ctx, int mode);
/* Number of persistent recurrence launches queued on the context so far
 * (-1 for a null context). */
int64_t numrs_hip_persistent_launches(numrs_hip_ctx *ctx);
/* Poll rounds a persistent kernel's wait for another workgroup's step makes
 * before it gives up (rounds < 0: the default, 2^21, seconds of waiting).
 * A tiny limit forces the give-up path from the host, for testing: the
 * kernels still exit, and the next call that synchronises the stream
 * returns the give-up error. */
int numrs_hip_set_persistent_wait_limit(numrs_hip_ctx *ctx, int rounds);

/* LSTM layer (no reference op), gate order i, f, g, o:
 * x [B, T, I], W_ih [4H, I], W_hh [4H, H], b [4H] (NULL = 0), h0/c0 [B, H]
 * (NULL = 0).  Forward writes h_seq, c_seq [B, T, H] and the gate
 * activations acts [B, T, 4H] the backward needs.  Backward (BPTT) from
 * dh_seq [B, T, H] (NULL = 0): dx [B, T, I], dW_ih, dW_hh, db (any may be
 * NULL; one accumulate flag each); the weight gradients are single products
 * over all steps. */
int numrs_hip_lstm_forward(numrs_hip_ctx *ctx, const float *x, const float *w_ih,
                           const float *w_hh, const float *b, const float *h0, const float *c0,
                           float *h_seq, float *c_seq, float *acts, int64_t B, int64_t T,
                           int64_t I, int64_t H);
int numrs_hip_lstm_backward(numrs_hip_ctx *ctx, const float *x, const float *w_ih,
                            const float *w_hh, const float *h0, const float *c0,
                            const float *h_seq, const float *c_seq, const float *acts,
                            const float *dh_seq, float *dx, float *dw_ih, float *dw_hh, float *db,
                            int64_t B, int64_t T, int64_t I, int64_t H, int acc_dx, int acc_dw_ih,
                            int acc_dw_hh, int acc_db);
/* No counterpart in the reference (numrs has no recurrent layer): two
 * stacked LSTM layers, x [B, T, I] -> layer 1 (W_ih1 [4H1, I], W_hh1
 * [4H1, H1], b1) -> h1_seq [B, T, H1] -> layer 2 (W_ih2 [4H2, H1], W_hh2
 * [4H2, H2], b2) -> h2_seq [B, T, H2], zero initial states; the saved
 * c/acts sequences as in numrs_hip_lstm_forward.  Same values as two
 * numrs_hip_lstm_forward calls up to fp32 rounding order.  When both layers
 * take the tiled steps (H1, H2 multiples of 256) the layers interleave: one
 * launch runs layer 1's step t and layer 2's step t - 1, which reduces h1
 * against W_ih2 inside the step (T + 1 dependent launches instead of 2T). */
int numrs_hip_lstm2_forward(numrs_hip_ctx *ctx, const float *x, const float *w_ih1,
                            const float *w_hh1, const float *b1, const float *w_ih2,
                            const float *w_hh2, const float *b2, float *h1_seq, float *c1_seq,
                            float *acts1, float *h2_seq, float *c2_seq, float *acts2, int64_t B,
                            int64_t T, int64_t I, int64_t H1, int64_t H2);
/* Its BPTT from dh2_seq [B, T, H2] (may be NULL): the gradients of x and of
 * both layers' parameters (each may be NULL, one accumulate flag each).
 * With H1, H2 multiples of 64 one launch runs layer 2's step t and layer
 * 1's step t + 1, whose dh takes dG2 W_ih2 of its step directly (T + 1
 * dependent launches instead of 2T). */
int numrs_hip_lstm2_backward(numrs_hip_ctx *ctx, const float *x, const float *w_ih1,
                             const float *w_hh1, const float *w_ih2, const float *w_hh2,
                             const float *h1_seq, const float *c1_seq, const float *acts1,
                             const float *h2_seq, const float *c2_seq, const float *acts2,
                             const float *dh2_seq, float *dx, float *dw_ih1, float *dw_hh1,
                             float *db1, float *dw_ih2, float *dw_hh2, float *db2, int64_t B,
                             int64_t T, int64_t I, int64_t H1, int64_t H2, int acc_dx,
                             int acc_dw_ih1, int acc_dw_hh1, int acc_db1, int acc_dw_ih2,
                             int acc_dw_hh2, int acc_db2);
/* y[b, :] = x[b, t, :] for x [B, T, D] (backward = 0), or its backward
 * y[b, t, :] (+)= x[b, :] over a [B, T, D] gradient, zero elsewhere when not
 * accumulating (backward = 1). */
int numrs_hip_time_slice(numrs_hip_ctx *ctx, const float *x, float *y, int64_t B, int64_t T,
                         int64_t D, int64_t t, int backward, int accumulate);

/* ---------------------------------------------------------------------- */
/* Broadcast-reduce gradients                                              */
/* ---------------------------------------------------------------------- */

/* unbroadcast (backward.rs:12-39) + accumulate_gradient (tensor.rs:120-132):
 * reduces g (shape gshape[0..gnd)) onto out (shape oshape[0..ond)), shapes
 * right-aligned numpy style.  CORRECT sums every axis where out has size 1
 * or is missing; REFERENCE sums everything into out[0] (accumulate = 0 then
 * writes [sum, 0, ..., 0], the reference's fresh zero grad plus the zip). */
int numrs_hip_sum_to_shape(numrs_hip_ctx *ctx, const float *g, const int64_t *gshape, int gnd,
                           float *out, const int64_t *oshape, int ond, int mode, int accumulate);

/* ops::sum / ops::mean over one axis (ops/reduction/sum.rs:7-10 ->
 * backend/cpu/scalar.rs:584-700): x viewed as [outer, n, inner] with the
 * reduced axis in the middle; out[outer, inner] (the axis removed).  The
 * mean divides the sum by n.  Empty axis: 0 (sum) or NaN (mean). */
int numrs_hip_reduce_axis(numrs_hip_ctx *ctx, const float *x, int64_t outer, int64_t n,
                          int64_t inner, int mean, float *out);
/* Backward of the axis reduction: dx[outer, n, inner] (+)= g[outer, inner],
 * divided by n for the mean (sum_backward / mean_backward, backward.rs:208-236,
 * along the axis the forward reduced). */
int numrs_hip_broadcast_axis(numrs_hip_ctx *ctx, const float *g, int64_t outer, int64_t n,
                             int64_t inner, int mean, float *dx, int accumulate);

/* relu_backward (backward.rs:152-163) fused with the bias branch of
 * add_backward (backward.rs:43-54) for y = ReLU(x + b), x[rows,cols],
 * b[cols]:  dx = (z > 0) ? g : 0 with z = x + b the saved pre-activation,
 * db = column sum of dx (mode CORRECT) or its full sum in db[0] (REFERENCE).
 * dx or db may be NULL.  Reads g and z once: 12 B/element. */
int numrs_hip_relu_bias_backward(numrs_hip_ctx *ctx, const float *g, const float *z, float *dx,
                                 float *db, int64_t rows, int64_t cols, int mode, int accumulate);

/* No counterpart in the reference.  numrs_hip_relu_bias_backward for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): same arguments and
 * results, but the column-sum partials live in a static per-GPU array of
 * 2^20 floats (4 MiB) instead of the context workspace, and the call makes no
 * hipMalloc / hipFree or other allocating call.  A shape whose partials
 * exceed the array returns NUMRS_HIP_E_INVALID (on a 256-CU MI355X: more
 * than 2^20 columns with db requested).  Calls that overlap on one GPU (two
 * contexts) race on the array. */
int numrs_hip_relu_bias_backward_noalloc(numrs_hip_ctx *ctx, const float *g, const float *z,
                                         float *dx, float *db, int64_t rows, int64_t cols,
                                         int mode, int accumulate);

/* ---------------------------------------------------------------------- */
/* Elementwise backward                                                    */
/* ---------------------------------------------------------------------- */

/* dx (+)= g * f'(v) for the unary kinds above; `param` is the exponent for
 * NUMRS_HIP_POW and ignored otherwise. */
int numrs_hip_unary_backward(numrs_hip_ctx *ctx, int kind, const float *g, const float *v,
                             float *dx, int64_t n, float param, int accumulate);

/* Binary backward for same-shape operands; dx or dy may be NULL. */
int numrs_hip_binary_backward(numrs_hip_ctx *ctx, int kind, const float *g, const float *x,
                              const float *y, float *dx, float *dy, int64_t n, int accumulate);

/* sum_backward / mean_backward (backward.rs:208-236): dx (+)= g[0] * scale
 * with scale = 1 (sum) or the f32 division g[0]/n performed as in the
 * reference when divide_by_n = 1 (mean). g_scalar is a device pointer. */
int numrs_hip_fill_grad(numrs_hip_ctx *ctx, const float *g_scalar, float *dx, int64_t n,
                        int divide_by_n, int accumulate);

/* mse_backward (backward.rs:239-261): dp = ((g*2)*(p-t))/n, dt = -dp.
 * g_scalar is a device pointer; dp or dt may be NULL. */
int numrs_hip_mse_backward(numrs_hip_ctx *ctx, const float *g_scalar, const float *p,
                           const float *t, float *dp, float *dt, int64_t n, int accumulate);

/* ---------------------------------------------------------------------- */
/* Row-wise kernels                                                        */
/* ---------------------------------------------------------------------- */

/* cross_entropy_backward (backward.rs:265-301): per row softmax of the
 * logits[B,C] minus the target, times g[0]/B.  The target is either a
 * one-hot float matrix (onehot != NULL, as the reference takes it) or int32
 * class labels (labels != NULL; a label outside [0,C) yields an all-zero
 * target row, as a zero one-hot row would). */
int numrs_hip_softmax_ce_backward(numrs_hip_ctx *ctx, const float *g_scalar, const float *logits,
                                  const float *onehot, const int32_t *labels, float *dlogits,
                                  int64_t B, int64_t C, int accumulate);

/* softmax_backward (backward.rs:521-541), rows of length cols:
 * dx (+)= y * (g - sum_row(g*y)). */
int numrs_hip_softmax_backward(numrs_hip_ctx *ctx, const float *y, const float *g, float *dx,
                               int64_t rows, int64_t cols, int accumulate);

/* Row argmax as int32.  tie_last = 0: first maximum (ops::argmax,
 * backend/cpu/scalar.rs:517-528); tie_last = 1: last maximum with NaN
 * compared as Equal (Trainer::evaluate's max_by, autograd/train.rs:213-228). */
int numrs_hip_argmax_rows(numrs_hip_ctx *ctx, const float *x, int32_t *idx, int64_t rows,
                          int64_t cols, int tie_last);

/* ---------------------------------------------------------------------- */
/* Optimizer steps                                                         */
/* ---------------------------------------------------------------------- */

/* SGD::step for one parameter (optim/sgd.rs:87-124, weight decay
 * optim/base.rs:26-36): g' = g + wd*p; mu != 0: v = mu*v + g', p -= lr*v;
 * else p -= lr*g'.  v may be NULL when mu == 0. */
int numrs_hip_sgd_step(numrs_hip_ctx *ctx, float *p, const float *g, float *v, int64_t n,
                       float lr, float mu, float wd);

/* SGD over `count` parameter tensors in one launch (the per-parameter loop
 * of sgd.rs:88-121 fused): p[i], g[i], v[i] (v may be NULL when mu == 0)
 * of n[i] elements each.  The pointer arrays are host arrays. */
int numrs_hip_sgd_step_multi(numrs_hip_ctx *ctx, float *const *p, const float *const *g,
                             float *const *v, const int64_t *n, int count, float lr, float mu,
                             float wd);

/* Adam::step for one parameter (optim/adam.rs:124-167) at step t (the
 * already-incremented counter): bias corrections 1 - b^t are computed on the
 * host with f32::powi's semantics, then one fused pass updates p, m, v
 * (28 B/element). */
int numrs_hip_adam_step(numrs_hip_ctx *ctx, float *p, const float *g, float *m, float *v,
                        int64_t n, float lr, float b1, float b2, float eps, float wd, int t);
/* Adam over `count` parameter tensors in one launch (adam.rs:131-164 fused). */
int numrs_hip_adam_step_multi(numrs_hip_ctx *ctx, float *const *p, const float *const *g,
                              float *const *m, float *const *v, const int64_t *n, int count,
                              float lr, float b1, float b2, float eps, float wd, int t);

/* One step of optimizer `kind` over `count` parameter tensors in one launch
 * (each Optimizer::step loop over params fused): p[i], g[i] and the kind's
 * state slots s1[i]/s2[i] (see the enum) of n[i] elements; `hyper` holds the
 * kind's nhyper hyperparameters; t is the already-incremented step counter
 * for the Adam-family kinds.  Element arithmetic follows each reference
 * step in order (bit-identical for all kinds but LAMB, whose layer norms are
 * blocked sums).  Pointer arrays are host arrays. */
int numrs_hip_optimizer_step(numrs_hip_ctx *ctx, int kind, float *const *p,
                             const float *const *g, float *const *s1, float *const *s2,
                             const int64_t *n, int count, const float *hyper, int nhyper, int t);
/* Lookahead's slow-weight sync (optim/lookahead.rs:88-120):
 * slow = slow + alpha*(fast - slow); fast = slow. */
int numrs_hip_lookahead_update(numrs_hip_ctx *ctx, float *const *fast, float *const *slow,
                               const int64_t *n, int count, float alpha);
/* out[0] = sum_i x[i]*y[i] (device scalar), two deterministic passes: the
 * dot product of L-BFGS's two-loop recursion (optim/lbfgs.rs:109-111). */
int numrs_hip_dot(numrs_hip_ctx *ctx, const float *x, const float *y, int64_t n, float *out);

/* ---------------------------------------------------------------------- */
/* Forward kernels the engine records (DispatchTable / ops.rs analogues)   */
/* ---------------------------------------------------------------------- */

/* out = a (op) b with numpy broadcasting, kind in NUMRS_HIP_ADD..DIV
 * (ops::add/sub/mul/div via promotion_wrappers.rs:25-168). */
int numrs_hip_binary_forward(numrs_hip_ctx *ctx, int kind, const float *a, const int64_t *ashape,
                             int and_, const float *b, const int64_t *bshape, int bnd, float *out);
/* DispatchTable (backend/dispatch.rs:51-93) kinds, in the reference's order:
 * ElementwiseKind (llo/elementwise.rs:38-68) and ReductionKind
 * (llo/reduction.rs:12-19). */
enum {
  NUMRS_HIP_EW_ADD = 0, NUMRS_HIP_EW_MUL, NUMRS_HIP_EW_SUB, NUMRS_HIP_EW_DIV, NUMRS_HIP_EW_POW,
  NUMRS_HIP_EW_SQRT, NUMRS_HIP_EW_SIN, NUMRS_HIP_EW_COS, NUMRS_HIP_EW_TAN, NUMRS_HIP_EW_ASIN,
  NUMRS_HIP_EW_ACOS, NUMRS_HIP_EW_ATAN, NUMRS_HIP_EW_ABS, NUMRS_HIP_EW_NEG, NUMRS_HIP_EW_EXP,
  NUMRS_HIP_EW_LOG, NUMRS_HIP_EW_RELU, NUMRS_HIP_EW_LEAKY_RELU, NUMRS_HIP_EW_SIGMOID,
  NUMRS_HIP_EW_TANH, NUMRS_HIP_EW_SOFTPLUS
};
enum {
  NUMRS_HIP_RED_SUM = 0, NUMRS_HIP_RED_MAX, NUMRS_HIP_RED_MIN, NUMRS_HIP_RED_MEAN,
  NUMRS_HIP_RED_ARGMAX, NUMRS_HIP_RED_VARIANCE
};
/* DispatchTable.elementwise: out[i] = kind(a[i], b[i]) for same-shape
 * operands (backend/cpu/scalar.rs:11-150); the unary kinds (SQRT..SOFTPLUS)
 * read a only and b may be NULL. */
int numrs_hip_elementwise(numrs_hip_ctx *ctx, int kind, const float *a, const float *b,
                          float *out, int64_t n);
/* DispatchTable.reduction: x[shape] reduced over all elements (axis < 0:
 * out has 1 value) or over `axis` (out holds the shape without that axis),
 * kind NUMRS_HIP_RED_* with the reference's semantics
 * (backend/cpu/scalar.rs:495-788): ArgMax returns the index as a float,
 * Variance is the population variance. */
int numrs_hip_reduction(numrs_hip_ctx *ctx, int kind, const float *x, const int64_t *shape,
                        int nd, int axis, float *out);
/* y = f(x) for the unary kinds (ops.rs:122-211, 453-554; GELU exact-erf). */
int numrs_hip_unary_forward(numrs_hip_ctx *ctx, int kind, const float *x, float *y, int64_t n,
                            float param);
/* y[cols,rows] = x[rows,cols]^T (ops/shape/transpose.rs:9-88). */
int numrs_hip_transpose(numrs_hip_ctx *ctx, const float *x, float *y, int64_t rows, int64_t cols);
/* out[0] = sum(x) or mean(x) (ops.rs:214-252). */
int numrs_hip_sum(numrs_hip_ctx *ctx, const float *x, int64_t n, int mean, float *out);
/* out[0] = mean((p-t)^2) (ops.rs:255-278). */
int numrs_hip_mse_loss(numrs_hip_ctx *ctx, const float *p, const float *t, int64_t n, float *out);
/* out[0] = mean over rows of softmax cross-entropy (ops.rs:281-334); one-hot
 * target or int32 labels. */
int numrs_hip_cross_entropy_loss(numrs_hip_ctx *ctx, const float *logits, const float *onehot,
                                 const int32_t *labels, int64_t B, int64_t C, float *out);
/* Row softmax of x*scale over the last axis (the reference's Softmax module
 * cannot run on an axis: ops/stats/softmax.rs:13-16). */
int numrs_hip_softmax_forward(numrs_hip_ctx *ctx, const float *x, float *y, int64_t rows,
                              int64_t cols, float scale);
/* Softmax along one axis of x viewed as [outer, n, inner] (the reference's
 * ops::softmax rejects an axis, ops/stats/softmax.rs:13-16); the last axis
 * (inner = 1) uses the row kernels.  Backward: softmax_backward
 * (backward.rs:521-541) along the same axis, dx (+)= y * (g - sum(g*y)). */
int numrs_hip_softmax_axis_forward(numrs_hip_ctx *ctx, const float *x, float *y, int64_t outer,
                                   int64_t n, int64_t inner);
int numrs_hip_softmax_axis_backward(numrs_hip_ctx *ctx, const float *y, const float *g, float *dx,
                                    int64_t outer, int64_t n, int64_t inner, int accumulate);
/* LayerNorm over the last axis (no reference op): y = (x-mean)*rstd*gamma +
 * beta, rstd = 1/sqrt(biased var + eps); mean/rstd per row (may be NULL). */
int numrs_hip_layernorm_forward(numrs_hip_ctx *ctx, const float *x, const float *gamma,
                                const float *beta, float *y, float *mean, float *rstd,
                                int64_t rows, int64_t cols, float eps);
/* LayerNorm backward from the saved mean/rstd: dx, dgamma = sum_rows g*xhat,
 * dbeta = sum_rows g (any may be NULL; one accumulate flag each); rows of at
 * most 2048.  One pass over g and x plus two column finalizes. */
int numrs_hip_layernorm_backward(numrs_hip_ctx *ctx, const float *g, const float *x,
                                 const float *gamma, const float *mean, const float *rstd,
                                 float *dx, float *dgamma, float *dbeta, int64_t rows,
                                 int64_t cols, int acc_dx, int acc_dgamma, int acc_dbeta);

/* ---------------------------------------------------------------------- */
/* Tensor engine: numrs's Tensor / backward / optimizers, device-resident   */
/* ---------------------------------------------------------------------- */

/* A tensor handle (autograd/tensor.rs:18-33): device data, a grad cell
 * shared by every reference to the tensor, and the node that produced it.
 * Handles must be freed before their context is destroyed.  Errors are
 * reported through numrs_hip_last_error of the tensor's context. */
typedef struct numrs_hip_tensor numrs_hip_tensor;
typedef struct numrs_hip_optim numrs_hip_optim;

/* Grad mode, thread-local (is_grad_enabled / set_grad_enabled, mod.rs:194-206). */
void numrs_hip_set_grad_enabled(int enabled);
int numrs_hip_is_grad_enabled(void);
/* Broadcast-gradient mode of the engine's add/sub/mul/div nodes. */
int numrs_hip_set_unbroadcast_mode(numrs_hip_ctx *ctx, int mode);

/* Tensor::new (tensor.rs:41-59): uploads `host`. */
int numrs_hip_tensor_new(numrs_hip_ctx *ctx, const float *host, const int64_t *shape, int ndim,
                         int requires_grad, numrs_hip_tensor **out);
int numrs_hip_tensor_free(numrs_hip_tensor *t);
/* Writes up to cap dims into shape; returns ndim (Tensor::shape, :86-88). */
int numrs_hip_tensor_shape(const numrs_hip_tensor *t, int64_t *shape, int cap);
int64_t numrs_hip_tensor_numel(const numrs_hip_tensor *t);
int numrs_hip_tensor_requires_grad(const numrs_hip_tensor *t);
int numrs_hip_tensor_is_leaf(const numrs_hip_tensor *t);
/* Tensor::values (:91-93): downloads n = numel floats. */
int numrs_hip_tensor_values(numrs_hip_tensor *t, float *host, int64_t n);
/* Tensor::gradient (:96-98): 1 and the grad copied into host, or 0 when the
 * tensor has no grad (None). */
int numrs_hip_tensor_gradient(numrs_hip_tensor *t, float *host, int64_t n);
/* Tensor::set_gradient (:110-117) and zero_grad (:135-142). */
int numrs_hip_tensor_set_gradient(numrs_hip_tensor *t, const float *host, int64_t n);
int numrs_hip_tensor_zero_grad(numrs_hip_tensor *t);
/* Device pointers of the values and grad (grad NULL when none; materialised). */
int numrs_hip_tensor_device_ptrs(numrs_hip_tensor *t, float **data, float **grad);
/* Tensor::backward (:173-215). */
int numrs_hip_tensor_backward(numrs_hip_tensor *t);
/* Tensor::detach (:146-154). */
int numrs_hip_tensor_detach(numrs_hip_tensor *t, numrs_hip_tensor **out);
/* Tensor::add/sub/mul/div (ops.rs:16-98), kind NUMRS_HIP_ADD..DIV. */
int numrs_hip_tensor_binary(int kind, numrs_hip_tensor *a, numrs_hip_tensor *b,
                            numrs_hip_tensor **out);
/* Tensor::relu/sigmoid/tanh/exp/log/sqrt/sin/cos/tan/pow (ops.rs:121-554)
 * and gelu; param = exponent for NUMRS_HIP_POW. */
int numrs_hip_tensor_unary(int kind, numrs_hip_tensor *a, float param, numrs_hip_tensor **out);
/* Tensor::matmul (ops.rs:101-119), 2-D. */
int numrs_hip_tensor_matmul(numrs_hip_tensor *a, numrs_hip_tensor *b, numrs_hip_tensor **out);
/* Tensor::transpose (tensor.rs:242-259), 2-D. */
int numrs_hip_tensor_transpose(numrs_hip_tensor *a, numrs_hip_tensor **out);
/* Tensor::reshape (ops.rs:353-369). */
int numrs_hip_tensor_reshape(numrs_hip_tensor *a, const int64_t *shape, int ndim,
                             numrs_hip_tensor **out);
/* Tensor::sum / Tensor::mean (ops.rs:214-252) -> [1]. */
int numrs_hip_tensor_sum(numrs_hip_tensor *a, int mean, numrs_hip_tensor **out);
/* Tensor::mse_loss (ops.rs:255-278) -> [1]. */
int numrs_hip_tensor_mse_loss(numrs_hip_tensor *pred, numrs_hip_tensor *target,
                              numrs_hip_tensor **out);
/* Tensor::cross_entropy_loss (ops.rs:281-334), one-hot target -> [1]. */
int numrs_hip_tensor_cross_entropy_loss(numrs_hip_tensor *logits, numrs_hip_tensor *target,
                                        numrs_hip_tensor **out);
/* The same with int32 class labels (host array of logits rows) instead of a
 * one-hot tensor: the reference builds the one-hot on the host first. */
int numrs_hip_tensor_cross_entropy_labels(numrs_hip_tensor *logits, const int32_t *host_labels,
                                          numrs_hip_tensor **out);
/* Row softmax over the last axis (Softmax module, nn.rs:345-375, on an axis). */
int numrs_hip_tensor_softmax(numrs_hip_tensor *a, numrs_hip_tensor **out);
/* Tensor sum / mean over one axis (0 <= axis < ndim): the axis is removed
 * from the shape, a 1-D input gives [1] (ops::sum / ops::mean with
 * Some(axis), backend/cpu/scalar.rs:584-700; the reference's autograd
 * records OpKind::Sum { axis } but only ever reduces fully, ops.rs:214-252,
 * and its sum_backward ignores the axis, backward.rs:208-221). */
int numrs_hip_tensor_sum_axis(numrs_hip_tensor *a, int64_t axis, int mean, numrs_hip_tensor **out);
/* Tensor softmax along one axis (0 <= axis < ndim); the reference rejects an
 * axis (ops/stats/softmax.rs:13-16). */
int numrs_hip_tensor_softmax_axis(numrs_hip_tensor *a, int64_t axis, numrs_hip_tensor **out);
/* LayerNorm over the last axis (no reference op). */
int numrs_hip_tensor_layer_norm(numrs_hip_tensor *x, numrs_hip_tensor *gamma,
                                numrs_hip_tensor *beta, float eps, numrs_hip_tensor **out);

/* Linear node y = x @ W^T + b over x [T, in], W [out, in], b [out] or NULL:
 * one node with Linear::forward's values and gradients (nn.rs:217-235). */
int numrs_hip_tensor_linear(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                            numrs_hip_tensor **out);
/* No counterpart in the reference: a Linear node followed by ReLU
 * (nn.rs:217-235, then ReLU::forward, nn.rs:306-320) as one node, y =
 * max(x @ W^T + b, 0), with numrs_hip_linear_relu_forward/_backward.  Same
 * values and parameter gradients as the two nodes; the pre-activation is not
 * a tensor of its own. */
int numrs_hip_tensor_linear_relu(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                                 numrs_hip_tensor **out);
/* No counterpart in the reference: a Linear node followed by GELU as one
 * node, y = GELU(x @ W^T + b) (numrs_hip_linear_gelu_forward/_backward; the
 * pre-activation is saved inside the node).  Same values and gradients as
 * the two nodes. */
int numrs_hip_tensor_linear_gelu(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                                 numrs_hip_tensor **out);
/* No counterpart in the reference: the residual step y = res + (x @ W^T + b)
 * of a residual block -- Linear::forward (nn.rs:217-235) then the Add node
 * (add_backward, backward.rs:43-54) -- as one node, res [T, out] added in the
 * product's epilogue (numrs_hip_linear_residual_forward).  res's gradient is
 * g; x, W and b get the Linear node's gradients. */
int numrs_hip_tensor_linear_residual(numrs_hip_tensor *x, numrs_hip_tensor *W,
                                     numrs_hip_tensor *b, numrs_hip_tensor *res,
                                     numrs_hip_tensor **out);
/* No counterpart in the reference: two stacked LSTM layers as one node,
 * x [B, T, I] -> h2_seq [B, T, H2] (numrs_hip_lstm2_forward/_backward); b1
 * and b2 may be NULL.  Same values and gradients as two LSTM nodes up to
 * fp32 rounding order. */
int numrs_hip_tensor_lstm2(numrs_hip_tensor *x, numrs_hip_tensor *w_ih1, numrs_hip_tensor *w_hh1,
                           numrs_hip_tensor *b1, numrs_hip_tensor *w_ih2,
                           numrs_hip_tensor *w_hh2, numrs_hip_tensor *b2,
                           numrs_hip_tensor **out);
/* LSTM layer node: x [B, T, I] -> h_seq [B, T, H] (numrs_hip_lstm_forward). */
int numrs_hip_tensor_lstm(numrs_hip_tensor *x, numrs_hip_tensor *w_ih, numrs_hip_tensor *w_hh,
                          numrs_hip_tensor *b, numrs_hip_tensor **out);
/* Time-step slice node: x [B, T, D] -> x[:, t, :] [B, D]. */
int numrs_hip_tensor_time_slice(numrs_hip_tensor *x, int64_t t, numrs_hip_tensor **out);
/* Multi-head attention node over q, k, v [B*S, D] (numrs_hip_attention_forward). */
int numrs_hip_tensor_attention(numrs_hip_tensor *q, numrs_hip_tensor *k, numrs_hip_tensor *v,
                               int64_t batch, int64_t seq, int64_t heads, numrs_hip_tensor **out);
/* The same node over one packed projection qkv [B*S, 3D] (q, k, v its column
 * blocks, as a Linear to 3D features produces them): out [B*S, D]; the
 * backward writes the packed grad [B*S, 3D]. */
int numrs_hip_tensor_attention_qkv(numrs_hip_tensor *qkv, int64_t batch, int64_t seq,
                                   int64_t heads, numrs_hip_tensor **out);

/* SGD::new (optim/sgd.rs:47-69) / Adam::new (optim/adam.rs:64-99) over
 * parameter tensors; step / zero_grad / learning_rate / set_learning_rate
 * are the Optimizer trait (optim/base.rs:8-23). */
int numrs_hip_optim_sgd(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                        float momentum, float wd, numrs_hip_optim **out);
int numrs_hip_optim_adam(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                         float b1, float b2, float eps, float wd, numrs_hip_optim **out);
int numrs_hip_optim_step(numrs_hip_optim *opt);
int numrs_hip_optim_zero_grad(numrs_hip_optim *opt);
int numrs_hip_optim_set_lr(numrs_hip_optim *opt, float lr);
float numrs_hip_optim_lr(const numrs_hip_optim *opt);
int numrs_hip_optim_free(numrs_hip_optim *opt);
/* Optimizer state for checkpoints (TrainingState.optimizer_state of the
 * reference's JSON checkpoint, llo/model.rs:207-220, ops/model.rs:550-588,
 * where the reference leaves it empty).  Up to two state slots per parameter
 * -- SGD: velocity; Adam: m, v; the NUMRS_HIP_OPT_* kinds: their two state
 * arrays -- plus the step counter t.  Lookahead and L-BFGS are not exported.
 * get/set copy one slot of one parameter (n = the parameter's element count)
 * between host memory and the device, synchronously. */
int numrs_hip_optim_state_info(const numrs_hip_optim *o, int *n_params, int *n_slots,
                               int64_t *step);
int numrs_hip_optim_state_get(numrs_hip_optim *o, int param, int slot, float *host, int64_t n);
int numrs_hip_optim_state_set(numrs_hip_optim *o, int param, int slot, const float *host,
                              int64_t n);
int numrs_hip_optim_set_step(numrs_hip_optim *o, int64_t step);

/* AdamW::new, RMSprop::new, AdaGrad::new, NAdam::new, RAdam::new,
 * AdaDelta::new, AdaBound::new, Rprop::new, LAMB::new over parameter tensors
 * (kind and hyperparameters as for numrs_hip_optimizer_step).  AdaDelta's
 * learning rate reads 1 and ignores sets (adadelta.rs:139-146); Rprop's is
 * the mean step size and a set resets every step size (rprop.rs:163-181). */
int numrs_hip_optim_create(numrs_hip_ctx *ctx, int kind, numrs_hip_tensor **params, int n,
                           const float *hyper, int nhyper, numrs_hip_optim **out);
/* Lookahead::new (optim/lookahead.rs:59-84) wrapping `inner`, which it takes
 * over (freeing the Lookahead frees it); slow weights start at the current
 * parameter values.  Its lr is the inner optimizer's. */
int numrs_hip_optim_lookahead(numrs_hip_optim *inner, numrs_hip_tensor **params, int n, int k,
                              float alpha, numrs_hip_optim **out);
/* LBFGS::new (optim/lbfgs.rs:60-76): two-loop recursion over the flattened
 * parameters with `history_size` (s, y) pairs; max_iter is kept but unused,
 * as in the reference. */
int numrs_hip_optim_lbfgs(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                          int history_size, int max_iter, numrs_hip_optim **out);

/* LR schedulers over an engine optimizer (optim/schedulers.rs).  step()
 * follows Scheduler::step; ReduceLROnPlateau takes step_metric() instead
 * (its step() is refused, as the reference panics there). */
typedef struct numrs_hip_scheduler numrs_hip_scheduler;
int numrs_hip_scheduler_create(int kind, const float *hyper, int nhyper,
                               numrs_hip_scheduler **out);
int numrs_hip_scheduler_step(numrs_hip_scheduler *s, numrs_hip_optim *opt);
int numrs_hip_scheduler_step_metric(numrs_hip_scheduler *s, float metric, numrs_hip_optim *opt);
float numrs_hip_scheduler_get_lr(const numrs_hip_scheduler *s);
int numrs_hip_scheduler_free(numrs_hip_scheduler *s);

#ifdef __cplusplus
}
#endif
#endif /* NUMRS_HIP_H */
