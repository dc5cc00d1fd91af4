/*
 * numrs_oracle.c -- CPU restatement of numrs's reverse-mode autograd hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP backend is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it; the product library (numrs_amd/csrc) never links,
 * calls or falls back to it.
 *
 * Reference: rjaguiluz/numrs, crate numrs-core (Rust).  Every function below
 * names the reference file:line it restates.  The reference cannot be built in
 * this image (no cargo/rustc, crates not vendored), so there is no oracle/_ref;
 * the restatement is pinned instead by the reference's own known-answer tests,
 * closed forms, finite differences and fp64 brute force (see tests/).
 *
 * Two arithmetic flavours exist where the reference's order matters:
 *   - "faithful" (fp32, the reference's exact operation order; compiled with
 *     -ffp-contract=off so a*b+c is never fused, as in Rust), and
 *   - "_f64" (same mathematics, float64 accumulation, rounded once to fp32);
 *     long reductions are compared against this one.
 *
 * Pinning status per function (what fixes each one):
 *   orc_matmul_backward(_f64)    KAT tests/autograd_matmul.rs:6-47; fp64 brute force; non-square closed form
 *   orc_relu_backward            KAT tests/autograd_activations.rs:5-24; strict '>' at 0
 *   orc_sigmoid_backward         closed form s(1-s); finite differences
 *   orc_tanh_backward            closed form 1-y^2; finite differences
 *   orc_exp/log_backward         closed forms; finite differences
 *   orc_sum/mean_backward        KAT tests/autograd_reduction.rs:6-40
 *   orc_mse_backward / mse_loss  KAT tests/autograd_loss.rs:5-37
 *   orc_cross_entropy_*          KAT tests/autograd_loss.rs:40-54; finite differences; torch fp64 vectors
 *   orc_softmax_backward         closed form Jacobian (fp64 brute force); finite differences
 *   orc_sub/mul/div_backward     KAT tests/autograd_basic.rs:15-117; finite differences
 *   orc_pow/sqrt/sin/cos/tan_bwd closed forms; finite differences
 *   orc_unbroadcast_reference    code reading of backward.rs:12-39 + tensor.rs:120-132 (bias KAT in tests)
 *   orc_sum_to_shape_f64         numpy sum over broadcast axes
 *   orc_sgd_step                 KATs tests/autograd/optim/sgd.rs:8-80
 *   orc_adam_step, orc_powi      KATs tests/autograd/optim/adam.rs:8-62; compiler-rt __powisf2 semantics
 *   orc_argmax_rows              KATs tests/ops_reduction_complex.rs:27-46, ops/reduction/argmax.rs:49-80
 *   orc_sum_avx2_order           equals sequential/fp64 sum on exactly representable inputs
 *   orc_gelu_backward_f64        NEW op (no reference): finite differences + torch fp64 vectors
 *   orc_layernorm_backward_f64   NEW op (no reference): finite differences + torch fp64 vectors
 *   orc_elementwise              exact kinds bit-exact vs numpy float32 (fmax for relu); the libm kinds
 *                                within 2 ulp of float64 numpy; KATs tests/ops_elementwise.rs,
 *                                ops_math.rs
 *   orc_reduction                numpy nanmax/nanmin/sum/mean/var on finite data; the NaN and tie
 *                                rules of ArgMax spelled out case by case; KATs
 *                                tests/ops_reduction_complex.rs
 *   orc_reduce_axis              exact on integer-valued inputs vs numpy; sum over the axis then the
 *                                rest equals the full sum; axis = last/first/middle agree with
 *                                transposed row sums
 *   orc_broadcast_axis           finite differences of sum/mean(x, axis) . g
 *   orc_softmax_axis_f64         NEW (no reference axis softmax): equals orc_softmax_rows_f64 of the
 *                                axis moved last; sums to 1 along the axis
 *   orc_softmax_axis_backward_f64  finite differences of sum(g * softmax(x, axis)); equals
 *                                orc_softmax_backward_f64 of the axis moved last
 *   orc_adamw/rmsprop/adagrad/nadam/radam/adadelta/adabound/rprop/lamb_step
 *                                KATs tests/autograd/optim/standard_opts.rs, advanced_opts.rs;
 *                                float64 closed forms of each update rule over several steps;
 *                                special cases (AdamW wd=0 vs Adam, RAdam's SGD branch, Rprop
 *                                sign flips and signum(+-0))
 *   orc_lookahead_sync           closed form slow + a(fast - slow)
 *   orc_dot_seq                  exact on integer-valued inputs; float64 dot
 *   orc_sched_*                  closed forms (gamma^k, cosine, linear ramp) and plateau traces
 *   orc_sum_avx2_order_mt        exact on integer-valued inputs for every thread count; equals
 *                                orc_sum_avx2_order with one thread
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* Reductions in the reference's own order                                    */
/* ------------------------------------------------------------------------- */

/* ops::sum(a, None) on an AVX2 host: backend/cpu/simd.rs:247-283.
 * Eight lane accumulators fed in chunks of 8, then the 8 lanes summed in lane
 * order (s.iter().sum()), then the scalar tail added in index order. */
EXPORT float orc_sum_avx2_order(const float *x, int64_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + x[i + l];
  float s = 0.0f;
  for (int l = 0; l < 8; ++l) s = s + acc[l];
  for (; i < n; ++i) s = s + x[i];
  return s;
}

/* Iterator::sum over f32 (sequential, left to right): autograd/ops.rs:235
 * (Tensor::mean) and ops.rs:257-260 (mse_loss). */
EXPORT float orc_sum_seq(const float *x, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s = s + x[i];
  return s;
}

/* ops::sum(a, Some(last_axis)) on AVX2: backend/cpu/simd.rs:431-467 -- every
 * row reduced with the same 8-lane order as the full sum. */
EXPORT void orc_sum_rows_avx2_order(const float *x, int64_t rows, int64_t cols, float *out) {
  for (int64_t r = 0; r < rows; ++r) out[r] = orc_sum_avx2_order(x + r * cols, cols);
}

/* The 8-lane sum compiled for AVX2 (the instructions simd.rs:247-283 uses),
 * vectorised at O3: the same additions in the same order, so the same bits. */
__attribute__((target("avx2"), optimize("O3"))) static float sum8_avx2(const float *x,
                                                                        int64_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + x[i + l];
  float s = 0.0f;
  for (int l = 0; l < 8; ++l) s = s + acc[l];
  for (; i < n; ++i) s = s + x[i];
  return s;
}

struct sum_job {
  const float *x;
  int64_t n;
  int avx2;
  float out;
};

static void *sum_worker(void *arg) {
  struct sum_job *j = (struct sum_job *)arg;
  j->out = j->avx2 ? sum8_avx2(j->x, j->n) : orc_sum_avx2_order(j->x, j->n);
  return NULL;
}

/* A full sum on `threads` host threads, the shape of Rayon's par_iter().sum()
 * (backend/cpu/scalar.rs:500) with each thread's contiguous chunk reduced in
 * the 8-lane order of simd.rs:247-283: chunks of a multiple of 8 elements,
 * partial sums added in chunk order.  Used as the all-cores CPU baseline of
 * the reduction rows; its bits depend on the thread count (as Rayon's do). */
EXPORT float orc_sum_avx2_order_mt(const float *x, int64_t n, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  const int avx2 = __builtin_cpu_supports("avx2");
  int64_t chunk = (n + threads - 1) / threads;
  chunk = (chunk + 7) / 8 * 8;
  struct sum_job jobs[256];
  pthread_t tid[256];
  int created[256];
  for (int t = 0; t < threads; ++t) {
    const int64_t lo = (int64_t)t * chunk;
    const int64_t hi = lo + chunk < n ? lo + chunk : n;
    jobs[t].x = x + (lo < n ? lo : n);
    jobs[t].n = hi > lo ? hi - lo : 0;
    jobs[t].avx2 = avx2;
    jobs[t].out = 0.0f;
    created[t] = t > 0 && jobs[t].n > 0 && pthread_create(&tid[t], NULL, sum_worker, &jobs[t]) == 0;
    if (t > 0 && !created[t]) sum_worker(&jobs[t]);  /* no thread: sum it here */
  }
  sum_worker(&jobs[0]);
  float s = jobs[0].out;
  for (int t = 1; t < threads; ++t) {
    if (created[t]) pthread_join(tid[t], NULL);
    s = s + jobs[t].out;
  }
  return s;
}

/* 2-D transpose, ops/shape/transpose.rs:9-33 (blocking does not change values). */
EXPORT void orc_transpose(const float *x, int64_t rows, int64_t cols, float *y) {
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < cols; ++j) y[j * rows + i] = x[i * cols + j];
}

/* ------------------------------------------------------------------------- */
/* Gradient accumulation: autograd/tensor.rs:120-132                          */
/* ------------------------------------------------------------------------- */

/* grad += incoming via zip(): only min(n_dst, n_src) leading elements change. */
EXPORT void orc_accumulate(float *dst, int64_t n_dst, const float *src, int64_t n_src) {
  int64_t n = n_dst < n_src ? n_dst : n_src;
  for (int64_t i = 0; i < n; ++i) dst[i] = dst[i] + src[i];
}

/* ------------------------------------------------------------------------- */
/* matmul_backward: autograd/backward.rs:113-149                              */
/* ------------------------------------------------------------------------- */

/* dA[i,j] = sum_l dC[i,l]*B[j,l]   (backward.rs:123-132)
 * dB[i,j] = sum_l A[l,i]*dC[l,j]   (backward.rs:136-145)
 * fp32 accumulator, l ascending, exactly as the reference loops.
 * Row ranges let bench.py time a bounded sample: rows [a0,a1) of dA and
 * rows [b0,b1) of dB are computed. */
EXPORT void orc_matmul_backward_rows(const float *dC, const float *A, const float *B, float *dA,
                                     float *dB, int64_t M, int64_t K, int64_t N, int64_t a0,
                                     int64_t a1, int64_t b0, int64_t b1) {
  if (dA)
    for (int64_t i = a0; i < a1; ++i)
      for (int64_t j = 0; j < K; ++j) {
        float sum = 0.0f;
        for (int64_t l = 0; l < N; ++l) sum = sum + dC[i * N + l] * B[j * N + l];
        dA[i * K + j] = sum;
      }
  if (dB)
    for (int64_t i = b0; i < b1; ++i)
      for (int64_t j = 0; j < N; ++j) {
        float sum = 0.0f;
        for (int64_t l = 0; l < M; ++l) sum = sum + A[l * K + i] * dC[l * N + j];
        dB[i * N + j] = sum;
      }
}

EXPORT void orc_matmul_backward(const float *dC, const float *A, const float *B, float *dA,
                                float *dB, int64_t M, int64_t K, int64_t N) {
  orc_matmul_backward_rows(dC, A, B, dA, dB, M, K, N, 0, M, 0, K);
}

/* Same contraction with float64 accumulation, rounded once, over rows
 * [a0,a1) of dA and [b0,b1) of dB.  Loop order is cache-friendly (i-l-j);
 * fp64 sums of these lengths are insensitive to order at fp32 output scale. */
EXPORT void orc_matmul_backward_f64_rows(const float *dC, const float *A, const float *B,
                                         float *dA, float *dB, int64_t M, int64_t K, int64_t N,
                                         int64_t a0, int64_t a1, int64_t b0, int64_t b1,
                                         double *work) {
  /* work must hold max(K, N) doubles */
  if (dA)
    for (int64_t i = a0; i < a1; ++i) {
      for (int64_t j = 0; j < K; ++j) {
        double s = 0.0;
        const float *c = dC + i * N, *b = B + j * N;
        for (int64_t l = 0; l < N; ++l) s += (double)c[l] * (double)b[l];
        work[j] = s;
      }
      for (int64_t j = 0; j < K; ++j) dA[i * K + j] = (float)work[j];
    }
  if (dB)
    for (int64_t i = b0; i < b1; ++i) {
      for (int64_t j = 0; j < N; ++j) work[j] = 0.0;
      for (int64_t l = 0; l < M; ++l) {
        double a = (double)A[l * K + i];
        const float *c = dC + l * N;
        for (int64_t j = 0; j < N; ++j) work[j] += a * (double)c[j];
      }
      for (int64_t j = 0; j < N; ++j) dB[i * N + j] = (float)work[j];
    }
}

EXPORT void orc_matmul_backward_f64(const float *dC, const float *A, const float *B, float *dA,
                                    float *dB, int64_t M, int64_t K, int64_t N, double *work) {
  orc_matmul_backward_f64_rows(dC, A, B, dA, dB, M, K, N, 0, M, 0, K, work);
}

/* Forward C[M,N] = A[M,K] @ B[K,N] with float64 accumulation.  The reference
 * forward goes through cblas_sgemm (backend/blas/mod.rs:216-361, MKL, not
 * vendored): its large-shape bits are not reproducible here, so this is the
 * mathematical product, rounded once. */
EXPORT void orc_matmul_f64(const float *A, const float *B, float *C, int64_t M, int64_t K,
                           int64_t N, double *work) {
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t j = 0; j < N; ++j) work[j] = 0.0;
    for (int64_t l = 0; l < K; ++l) {
      double a = (double)A[i * K + l];
      const float *b = B + l * N;
      for (int64_t j = 0; j < N; ++j) work[j] += a * (double)b[j];
    }
    for (int64_t j = 0; j < N; ++j) C[i * N + j] = (float)work[j];
  }
}

/* ------------------------------------------------------------------------- */
/* Elementwise backward functions (fp32, reference operation order)           */
/* ------------------------------------------------------------------------- */

/* backward.rs:152-163: x > 0 ? g : 0 (strict; grad at 0 is 0). */
EXPORT void orc_relu_backward(const float *g, const float *x, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = (x[i] > 0.0f) ? g[i] : 0.0f;
}

/* backward.rs:166-177: (go * s) * (1 - s), s = forward output. */
EXPORT void orc_sigmoid_backward(const float *g, const float *s, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = (g[i] * s[i]) * (1.0f - s[i]);
}

/* backward.rs:180-191: go * exp_out. */
EXPORT void orc_exp_backward(const float *g, const float *e, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = g[i] * e[i];
}

/* backward.rs:194-205: go / x. */
EXPORT void orc_log_backward(const float *g, const float *x, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = g[i] / x[i];
}

/* backward.rs:503-517: y^2 via ops::pow (powf), 1 - y^2 via ops::sub, then
 * go * (1 - y^2) via ops::mul. */
EXPORT void orc_tanh_backward(const float *g, const float *y, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float ysq = powf(y[i], 2.0f);
    float om = 1.0f - ysq;
    dx[i] = g[i] * om;
  }
}

/* backward.rs:486-500: go * (1 + tan^2), tan^2 via powf. */
EXPORT void orc_tan_backward(const float *g, const float *t, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float sq = powf(t[i], 2.0f);
    dx[i] = g[i] * (1.0f + sq);
  }
}

/* backward.rs:407-438: go * (x^(n-1) * n) (powf, then two muls). */
EXPORT void orc_pow_backward(const float *g, const float *x, float expo, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float t1 = powf(x[i], expo - 1.0f);
    float t2 = t1 * expo;
    dx[i] = g[i] * t2;
  }
}

/* backward.rs:441-463: go * (x^(-0.5) * 0.5). */
EXPORT void orc_sqrt_backward(const float *g, const float *x, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float t1 = powf(x[i], -0.5f);
    float t2 = t1 * 0.5f;
    dx[i] = g[i] * t2;
  }
}

/* backward.rs:466-472: go * cos(x). */
EXPORT void orc_sin_backward(const float *g, const float *x, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = g[i] * cosf(x[i]);
}

/* backward.rs:475-483: go * (sin(x) * -1). */
EXPORT void orc_cos_backward(const float *g, const float *x, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = g[i] * (sinf(x[i]) * -1.0f);
}

/* backward.rs:57-70 (same shapes): dx = g, dy = g * -1. */
EXPORT void orc_sub_backward(const float *g, float *dx, float *dy, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (dx) dx[i] = g[i];
    if (dy) dy[i] = g[i] * -1.0f;
  }
}

/* backward.rs:74-87 (same shapes): dx = g * y, dy = g * x. */
EXPORT void orc_mul_backward(const float *g, const float *x, const float *y, float *dx, float *dy,
                             int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (dx) dx[i] = g[i] * y[i];
    if (dy) dy[i] = g[i] * x[i];
  }
}

/* backward.rs:90-109 (same shapes): dx = g / y; dy = (g * (x / (y*y))) * -1. */
EXPORT void orc_div_backward(const float *g, const float *x, const float *y, float *dx, float *dy,
                             int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (dx) dx[i] = g[i] / y[i];
    if (dy) {
      float ysq = y[i] * y[i];
      float term = x[i] / ysq;
      float gt = g[i] * term;
      dy[i] = gt * -1.0f;
    }
  }
}

/* backward.rs:208-221: every element gets g[0]. */
EXPORT void orc_sum_backward(float g0, float *dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = g0;
}

/* backward.rs:224-236: every element gets g[0] / (n as f32). */
EXPORT void orc_mean_backward(float g0, float *dx, int64_t n) {
  float v = g0 / (float)n;
  for (int64_t i = 0; i < n; ++i) dx[i] = v;
}

/* backward.rs:239-261: dp = ((g*2)*(p-t))/n; dt = -dp. */
EXPORT void orc_mse_backward(float g0, const float *p, const float *t, float *dp, float *dt,
                             int64_t n) {
  float nf = (float)n;
  for (int64_t i = 0; i < n; ++i) {
    float v = ((g0 * 2.0f) * (p[i] - t[i])) / nf;
    if (dp) dp[i] = v;
    if (dt) dt[i] = -v;
  }
}

/* Forward mse_loss, ops.rs:255-262: sequential f32 sum of (p-t)^2 (powi(2) is
 * an exact single multiply), then / n. */
EXPORT float orc_mse_loss(const float *p, const float *t, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float d = p[i] - t[i];
    s = s + d * d;
  }
  return s / (float)n;
}

/* Forward Tensor::mean, ops.rs:234-237. */
EXPORT float orc_mean_fwd(const float *x, int64_t n) { return orc_sum_seq(x, n) / (float)n; }

/* Rust f32::max: NaN-ignoring maximum (used by the fold at backward.rs:285). */
static float rust_fmax(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : b;
}

/* backward.rs:265-301: per row, max (fold from -inf), sequential exp sum,
 * softmax = exp(x-max)/sum, dx = (softmax - target) * (g/B). */
EXPORT void orc_cross_entropy_backward(float g0, const float *logits, const float *onehot,
                                       float *dx, int64_t B, int64_t C) {
  float scale = g0 / (float)B;
  for (int64_t i = 0; i < B; ++i) {
    const float *x = logits + i * C;
    const float *t = onehot + i * C;
    float mx = -INFINITY;
    for (int64_t j = 0; j < C; ++j) mx = rust_fmax(mx, x[j]);
    float es = 0.0f;
    for (int64_t j = 0; j < C; ++j) es = es + expf(x[j] - mx);
    for (int64_t j = 0; j < C; ++j) {
      float sm = expf(x[j] - mx) / es;
      dx[i * C + j] = (sm - t[j]) * scale;
    }
  }
}

/* Forward cross_entropy_loss, ops.rs:281-318. */
EXPORT float orc_cross_entropy_loss(const float *logits, const float *onehot, int64_t B,
                                    int64_t C) {
  float total = 0.0f;
  for (int64_t i = 0; i < B; ++i) {
    const float *x = logits + i * C;
    const float *t = onehot + i * C;
    float mx = -INFINITY;
    for (int64_t j = 0; j < C; ++j) mx = rust_fmax(mx, x[j]);
    float es = 0.0f;
    for (int64_t j = 0; j < C; ++j) es = es + expf(x[j] - mx);
    float sl = 0.0f;
    for (int64_t j = 0; j < C; ++j) {
      float ls = (x[j] - mx) - logf(es);
      sl = sl + (-t[j] * ls);
    }
    total = total + sl;
  }
  return total / (float)B;
}

/* backward.rs:521-541 (2-D, axis 1): t1 = g*S; r = row-sum(t1) (AVX2 order,
 * simd.rs:431-467); dx = S * (g - r). */
EXPORT void orc_softmax_backward(const float *y, const float *g, float *dx, int64_t rows,
                                 int64_t cols, float *work) {
  /* work holds cols floats */
  for (int64_t r = 0; r < rows; ++r) {
    const float *s = y + r * cols, *go = g + r * cols;
    for (int64_t j = 0; j < cols; ++j) work[j] = go[j] * s[j];
    float rs = orc_sum_avx2_order(work, cols);
    for (int64_t j = 0; j < cols; ++j) dx[r * cols + j] = s[j] * (go[j] - rs);
  }
}

/* ------------------------------------------------------------------------- */
/* Unbroadcast: backward.rs:12-39 followed by accumulate (tensor.rs:120-132)  */
/* ------------------------------------------------------------------------- */

/* REFERENCE mode: a gradient whose shape differs from the target is summed to
 * one scalar (ops::sum(grad, None) -> AVX2 order), and accumulate_gradient's
 * zip() then adds it into element 0 of the target grad only. */
EXPORT void orc_unbroadcast_reference_accumulate(const float *g, int64_t n, float *out_grad) {
  out_grad[0] = out_grad[0] + orc_sum_avx2_order(g, n);
}

/* CORRECT mode: sum over the broadcast axes (numpy semantics, shapes right
 * aligned; an output axis of size 1 or a missing leading axis is summed),
 * float64 accumulation.  out is overwritten. */
EXPORT int orc_sum_to_shape_f64(const float *g, const int64_t *gshape, int gnd, float *out,
                                const int64_t *oshape, int ond, double *work) {
  if (ond > gnd || gnd > 8) return -1;
  int64_t os[8], gstr[8];
  for (int d = 0; d < gnd; ++d) {
    int od = d - (gnd - ond);
    os[d] = od >= 0 ? oshape[od] : 1;
    if (os[d] != 1 && os[d] != gshape[d]) return -2;
  }
  int64_t on = 1, gn = 1;
  for (int d = 0; d < gnd; ++d) { on *= os[d]; gn *= gshape[d]; }
  int64_t s = 1;
  for (int d = gnd - 1; d >= 0; --d) { gstr[d] = s; s *= os[d]; }
  for (int64_t i = 0; i < on; ++i) work[i] = 0.0;
  for (int64_t i = 0; i < gn; ++i) {
    int64_t rem = i, oi = 0;
    for (int d = gnd - 1; d >= 0; --d) {
      int64_t c = rem % gshape[d];
      rem /= gshape[d];
      if (os[d] != 1) oi += c * gstr[d];
    }
    work[oi] += (double)g[i];
  }
  for (int64_t i = 0; i < on; ++i) out[i] = (float)work[i];
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Optimizers                                                                  */
/* ------------------------------------------------------------------------- */

/* f32::powi(t as i32): Rust lowers it to llvm.powi.f32, which on x86-64 is the
 * compiler-rt routine __powisf2 -- binary exponentiation by squaring, result
 * multiplied in for each set bit of the exponent, low bit first. */
EXPORT float orc_powi(float a, int b) {
  int recip = b < 0;
  float r = 1.0f;
  if (recip) b = -b;
  for (;;) {
    if (b & 1) r = r * a;
    b /= 2;
    if (b == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / r : r;
}

/* SGD::step for one parameter, optim/sgd.rs:87-124 with
 * apply_weight_decay (optim/base.rs:26-36):
 *   g' = g + wd*p  (only when wd != 0)
 *   mu != 0: v = mu*v + g'; p -= lr*v      else p -= lr*g'            */
EXPORT void orc_sgd_step(float *p, const float *g, float *v, int64_t n, float lr, float mu,
                         float wd) {
  for (int64_t i = 0; i < n; ++i) {
    float gg = g[i];
    if (wd != 0.0f) gg = gg + wd * p[i];
    if (mu != 0.0f) {
      v[i] = mu * v[i] + gg;
      p[i] = p[i] - lr * v[i];
    } else {
      p[i] = p[i] - lr * gg;
    }
  }
}

/* Adam::step for one parameter at step t (already incremented),
 * optim/adam.rs:124-167:
 *   bc1 = 1 - b1^t, bc2 = 1 - b2^t (powi);  g' = g + wd*p (wd != 0)
 *   m = b1*m + (1-b1)*g';  v = b2*v + ((1-b2)*g')*g'
 *   p -= (lr * (m/bc1)) / (sqrt(v/bc2) + eps)                          */
EXPORT void orc_adam_step(float *p, const float *g, float *m, float *v, int64_t n, float lr,
                          float b1, float b2, float eps, float wd, int t) {
  float bc1 = 1.0f - orc_powi(b1, t);
  float bc2 = 1.0f - orc_powi(b2, t);
  float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
  for (int64_t i = 0; i < n; ++i) {
    float gg = g[i];
    if (wd != 0.0f) gg = gg + wd * p[i];
    m[i] = b1 * m[i] + omb1 * gg;
    v[i] = b2 * v[i] + omb2 * gg * gg;
    float mh = m[i] / bc1;
    float vh = v[i] / bc2;
    p[i] = p[i] - lr * mh / (sqrtf(vh) + eps);
  }
}

/* ------------------------------------------------------------------------- */
/* Integer paths                                                               */
/* ------------------------------------------------------------------------- */

/* Row argmax.  tie_last = 0: ops::argmax, first maximum wins via strict '>'
 * (backend/cpu/scalar.rs:517-528, axis form :625-672).  tie_last = 1:
 * Trainer::evaluate's Iterator::max_by with partial_cmp (autograd/train.rs:
 * 213-228) -- the last of equal maxima wins, and an incomparable pair (NaN)
 * counts as Equal, so the later element replaces the running maximum. */
EXPORT void orc_argmax_rows(const float *x, int64_t rows, int64_t cols, int32_t *idx,
                            int tie_last) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *v = x + r * cols;
    int64_t best = 0;
    float bv = v[0];
    for (int64_t j = 1; j < cols; ++j) {
      if (!tie_last) {
        if (v[j] > bv) { bv = v[j]; best = j; }
      } else {
        /* max_by keeps the later element unless cmp(cur, new) == Greater */
        int greater = (bv > v[j]);
        if (!greater) { bv = v[j]; best = j; }
      }
    }
    idx[r] = (int32_t)best;
  }
}

/* ------------------------------------------------------------------------- */
/* Forward activations (autograd/ops.rs)                                       */
/* ------------------------------------------------------------------------- */

/* ops.rs:124-127: x.max(0.0) (Rust f32::max, NaN-ignoring). */
EXPORT void orc_relu(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = rust_fmax(x[i], 0.0f);
}

/* ops.rs:147-152: 1 / (1 + exp(-x)). */
EXPORT void orc_sigmoid(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------------------------- */
/* NEW ops the BASELINE configs need (absent from the reference): fp64 math   */
/* ------------------------------------------------------------------------- */

/* GELU (exact erf form) backward: d/dx [x * Phi(x)] = Phi(x) + x * phi(x). */
EXPORT void orc_gelu_backward_f64(const float *g, const float *x, float *dx, int64_t n) {
  const double inv_sqrt2 = 0.70710678118654752440, inv_sqrt2pi = 0.39894228040143267794;
  for (int64_t i = 0; i < n; ++i) {
    double xv = x[i];
    double cdf = 0.5 * (1.0 + erf(xv * inv_sqrt2));
    double pdf = inv_sqrt2pi * exp(-0.5 * xv * xv);
    dx[i] = (float)((double)g[i] * (cdf + xv * pdf));
  }
}

EXPORT void orc_gelu_f64(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    double xv = x[i];
    y[i] = (float)(xv * 0.5 * (1.0 + erf(xv * 0.70710678118654752440)));
  }
}

/* LayerNorm over the last axis: y = (x - mu) * rstd * gamma + beta, with
 * rstd = 1/sqrt(var + eps), var the biased variance.  Backward (fp64):
 *   xh = (x-mu)*rstd;  gg = g*gamma
 *   dx = rstd * (gg - mean(gg) - xh * mean(gg*xh))
 *   dgamma = sum_rows g*xh;  dbeta = sum_rows g
 * mean/rstd outputs (if non-NULL) receive the per-row statistics. */
EXPORT void orc_layernorm_fwd_f64(const float *x, const float *gamma, const float *beta, float *y,
                                  float *mean, float *rstd, int64_t rows, int64_t cols,
                                  float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * cols;
    double mu = 0.0, var = 0.0;
    for (int64_t j = 0; j < cols; ++j) mu += xr[j];
    mu /= (double)cols;
    for (int64_t j = 0; j < cols; ++j) var += (xr[j] - mu) * (xr[j] - mu);
    var /= (double)cols;
    double rs = 1.0 / sqrt(var + (double)eps);
    for (int64_t j = 0; j < cols; ++j)
      y[r * cols + j] = (float)((xr[j] - mu) * rs * gamma[j] + beta[j]);
    if (mean) mean[r] = (float)mu;
    if (rstd) rstd[r] = (float)rs;
  }
}

EXPORT void orc_layernorm_backward_f64(const float *g, const float *x, const float *gamma,
                                       float *dx, float *dgamma, float *dbeta, int64_t rows,
                                       int64_t cols, float eps, double *work) {
  /* work holds 2*cols doubles */
  double *dg = work, *db = work + cols;
  for (int64_t j = 0; j < cols; ++j) dg[j] = db[j] = 0.0;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * cols, *gr = g + r * cols;
    double mu = 0.0, var = 0.0;
    for (int64_t j = 0; j < cols; ++j) mu += xr[j];
    mu /= (double)cols;
    for (int64_t j = 0; j < cols; ++j) var += (xr[j] - mu) * (xr[j] - mu);
    var /= (double)cols;
    double rs = 1.0 / sqrt(var + (double)eps);
    double m1 = 0.0, m2 = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      double xh = (xr[j] - mu) * rs;
      double gg = (double)gr[j] * gamma[j];
      m1 += gg;
      m2 += gg * xh;
      dg[j] += (double)gr[j] * xh;
      db[j] += (double)gr[j];
    }
    m1 /= (double)cols;
    m2 /= (double)cols;
    if (dx)
      for (int64_t j = 0; j < cols; ++j) {
        double xh = (xr[j] - mu) * rs;
        double gg = (double)gr[j] * gamma[j];
        dx[r * cols + j] = (float)(rs * (gg - m1 - xh * m2));
      }
  }
  for (int64_t j = 0; j < cols; ++j) {
    if (dgamma) dgamma[j] = (float)dg[j];
    if (dbeta) dbeta[j] = (float)db[j];
  }
}

/* Row softmax forward (fp64), used to build attention inputs for tests. */
EXPORT void orc_softmax_rows_f64(const float *x, float *y, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * cols;
    double mx = -INFINITY, s = 0.0;
    for (int64_t j = 0; j < cols; ++j) mx = xr[j] > mx ? xr[j] : mx;
    for (int64_t j = 0; j < cols; ++j) s += exp((double)xr[j] - mx);
    for (int64_t j = 0; j < cols; ++j) y[r * cols + j] = (float)(exp((double)xr[j] - mx) / s);
  }
}

/* Softmax backward with float64 row sums (tight reference for long rows). */
EXPORT void orc_softmax_backward_f64(const float *y, const float *g, float *dx, int64_t rows,
                                     int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *s = y + r * cols, *go = g + r * cols;
    double rs = 0.0;
    for (int64_t j = 0; j < cols; ++j) rs += (double)go[j] * (double)s[j];
    for (int64_t j = 0; j < cols; ++j) dx[r * cols + j] = (float)((double)s[j] * ((double)go[j] - rs));
  }
}

/* ------------------------------------------------------------------------- */
/* Axis reductions and axis softmax                                          */
/* ------------------------------------------------------------------------- */
/* x viewed as [outer, n, inner] with the reduced axis in the middle. */

/* ops::sum / ops::mean with Some(axis): every output starts at 0.0 and adds
 * its n values in axis order (backend/cpu/scalar.rs:722-770, the generic
 * axis loop visits elements in linear order; :305-312 for the last axis),
 * then the mean divides by n (:314-316, :785-788). */
EXPORT void orc_reduce_axis(const float *x, int64_t outer, int64_t n, int64_t inner, int mean,
                            float *out) {
  for (int64_t b = 0; b < outer; ++b)
    for (int64_t i = 0; i < inner; ++i) {
      float s = 0.0f;
      for (int64_t k = 0; k < n; ++k) s += x[(b * n + k) * inner + i];
      out[b * inner + i] = mean ? s / (float)n : s;
    }
}

/* Backward of the axis reduction: sum_backward / mean_backward
 * (backward.rs:208-236) applied per reduced slice, dx = g (or g / n). */
EXPORT void orc_broadcast_axis(const float *g, int64_t outer, int64_t n, int64_t inner, int mean,
                               float *dx) {
  for (int64_t b = 0; b < outer; ++b)
    for (int64_t k = 0; k < n; ++k)
      for (int64_t i = 0; i < inner; ++i) {
        const float gv = g[b * inner + i];
        dx[(b * n + k) * inner + i] = mean ? gv / (float)n : gv;
      }
}

/* Softmax along an axis (NEW: the reference rejects an axis,
 * ops/stats/softmax.rs:13-16), float64 throughout. */
EXPORT void orc_softmax_axis_f64(const float *x, int64_t outer, int64_t n, int64_t inner,
                                 float *y) {
  for (int64_t b = 0; b < outer; ++b)
    for (int64_t i = 0; i < inner; ++i) {
      const float *xs = x + b * n * inner + i;
      double mx = -INFINITY, s = 0.0;
      for (int64_t k = 0; k < n; ++k) mx = xs[k * inner] > mx ? xs[k * inner] : mx;
      for (int64_t k = 0; k < n; ++k) s += exp((double)xs[k * inner] - mx);
      for (int64_t k = 0; k < n; ++k)
        y[b * n * inner + i + k * inner] = (float)(exp((double)xs[k * inner] - mx) / s);
    }
}

/* softmax_backward (backward.rs:521-541) along an axis, float64 sums:
 * dx = y * (g - sum_axis(g * y)). */
EXPORT void orc_softmax_axis_backward_f64(const float *y, const float *g, int64_t outer, int64_t n,
                                          int64_t inner, float *dx) {
  for (int64_t b = 0; b < outer; ++b)
    for (int64_t i = 0; i < inner; ++i) {
      const int64_t base = b * n * inner + i;
      double d = 0.0;
      for (int64_t k = 0; k < n; ++k) d += (double)g[base + k * inner] * (double)y[base + k * inner];
      for (int64_t k = 0; k < n; ++k) {
        const int64_t j = base + k * inner;
        dx[j] = (float)((double)y[j] * ((double)g[j] - d));
      }
    }
}

/* ------------------------------------------------------------------------- */
/* DispatchTable forward kernels (backend/cpu/scalar.rs)                     */
/* ------------------------------------------------------------------------- */

/* elementwise_scalar (scalar.rs:11-150): kinds in ElementwiseKind order
 * (llo/elementwise.rs:38-68).  Rust's f32 methods call the C library. */
EXPORT void orc_elementwise(int kind, const float *a, const float *b, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = a[i], y = b ? b[i] : 0.0f;
    float r;
    switch (kind) {
      case 0: r = x + y; break;
      case 1: r = x * y; break;
      case 2: r = x - y; break;
      case 3: r = x / y; break;
      case 4: r = powf(x, y); break;
      case 5: r = sqrtf(x); break;
      case 6: r = sinf(x); break;
      case 7: r = cosf(x); break;
      case 8: r = tanf(x); break;
      case 9: r = asinf(x); break;
      case 10: r = acosf(x); break;
      case 11: r = atanf(x); break;
      case 12: r = fabsf(x); break;
      case 13: r = -x; break;
      case 14: r = expf(x); break;
      case 15: r = logf(x); break;
      case 16: r = fmaxf(x, 0.0f); break;                     /* x.max(0.0) */
      case 17: r = x > 0.0f ? x : 0.01f * x; break;          /* :120-125 */
      case 18: r = 1.0f / (1.0f + expf(-x)); break;          /* :127-131 */
      case 19: r = tanhf(x); break;
      default: r = logf(1.0f + expf(x)); break;              /* softplus, :139-143 */
    }
    out[i] = r;
  }
}

/* reduce_scalar (scalar.rs:495-788), ReductionKind order Sum, Max, Min, Mean,
 * ArgMax, Variance (llo/reduction.rs:12-19).  axis < 0: all elements (the
 * Rayon sum of :500 is restated as a sequential sum; its split order is not
 * fixed).  axis >= 0: x viewed as [outer, n, inner]. */
EXPORT int orc_reduction(int kind, const float *x, const int64_t *shape, int nd, int axis,
                         float *out) {
  int64_t total = 1;
  for (int d = 0; d < nd; ++d) total *= shape[d];
  if (axis < 0) {
    if (total == 0) return -1;
    float r = 0.0f;
    switch (kind) {
      case 0: for (int64_t i = 0; i < total; ++i) r += x[i]; break;
      case 1: r = -INFINITY; for (int64_t i = 0; i < total; ++i) r = fmaxf(r, x[i]); break;
      case 2: r = INFINITY; for (int64_t i = 0; i < total; ++i) r = fminf(r, x[i]); break;
      case 3: for (int64_t i = 0; i < total; ++i) r += x[i]; r = r / (float)total; break;
      case 4: { /* :517-528 */
        int64_t mi = 0;
        float mv = x[0];
        for (int64_t i = 1; i < total; ++i)
          if (x[i] > mv) { mv = x[i]; mi = i; }
        r = (float)mi;
        break;
      }
      default: { /* Welford, :529-541 */
        const float nn = (float)total;
        float mean = 0.0f, m2 = 0.0f;
        for (int64_t i = 0; i < total; ++i) {
          const float delta = x[i] - mean;
          mean += delta / (float)(i + 1);
          const float delta2 = x[i] - mean;
          m2 += delta * delta2;
        }
        r = m2 / nn;
      }
    }
    out[0] = r;
    return 0;
  }
  if (axis >= nd) return -1;
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < axis; ++d) outer *= shape[d];
  for (int d = axis + 1; d < nd; ++d) inner *= shape[d];
  const int64_t n = shape[axis];
  for (int64_t b = 0; b < outer; ++b)
    for (int64_t i = 0; i < inner; ++i) {
      const float *s = x + b * n * inner + i;
      float r = 0.0f;
      switch (kind) {
        case 0: for (int64_t k = 0; k < n; ++k) r += s[k * inner]; break;
        case 1: r = -INFINITY; for (int64_t k = 0; k < n; ++k) r = fmaxf(r, s[k * inner]); break;
        case 2: r = INFINITY; for (int64_t k = 0; k < n; ++k) r = fminf(r, s[k * inner]); break;
        case 3: for (int64_t k = 0; k < n; ++k) r += s[k * inner]; r = r / (float)n; break;
        case 4: { /* :345-362, 623-668: fold from (0, -inf), strict '>' */
          float mv = -INFINITY;
          int64_t mi = 0;
          for (int64_t k = 0; k < n; ++k)
            if (s[k * inner] > mv) { mv = s[k * inner]; mi = k; }
          r = (float)mi;
          break;
        }
        default: { /* :364-393, 671-717: mean, then mean of squared deviations */
          float sum = 0.0f;
          for (int64_t k = 0; k < n; ++k) sum += s[k * inner];
          const float mean = sum / (float)n;
          float v = 0.0f;
          for (int64_t k = 0; k < n; ++k) {
            const float d = s[k * inner] - mean;
            v += d * d;
          }
          r = v / (float)n;
        }
      }
      out[b * inner + i] = r;
    }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* The other optimizers (autograd/optim/) and the LR schedulers              */
/* ------------------------------------------------------------------------- */
/* Each step is one parameter tensor, in the reference's operation order
 * (Rust evaluates a*b*c as (a*b)*c and never contracts).  Scalars the
 * reference derives once per step are derived here the same way: powi is
 * orc_powi, powf/cosf/sqrtf are the C library's, as Rust's f32 methods call
 * them on Linux. */

/* f32::signum: 1.0 for +0.0 and positives, -1.0 for -0.0 and negatives. */
static float orc_signum(float x) { return isnan(x) ? x : copysignf(1.0f, x); }

/* AdamW::step, optim/adamw.rs:92-129 (decay applied to the parameter). */
EXPORT void orc_adamw_step(float *p, const float *g, float *m, float *v, int64_t n, float lr,
                           float b1, float b2, float eps, float wd, int t) {
  const float bc1 = 1.0f - orc_powi(b1, t), bc2 = 1.0f - orc_powi(b2, t);
  for (int64_t i = 0; i < n; ++i) m[i] = b1 * m[i] + (1.0f - b1) * g[i];
  for (int64_t i = 0; i < n; ++i) v[i] = b2 * v[i] + (1.0f - b2) * g[i] * g[i];
  for (int64_t i = 0; i < n; ++i) {
    const float mh = m[i] / bc1, vh = v[i] / bc2;
    p[i] = p[i] - lr * (mh / (sqrtf(vh) + eps) + wd * p[i]);
  }
}

/* RMSprop::step, optim/rmsprop.rs:90-135 (apply_weight_decay first). */
EXPORT void orc_rmsprop_step(float *p, const float *g0, float *v, float *buf, int64_t n,
                             float lr, float alpha, float eps, float wd, float mom) {
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd != 0.0f) g = g + wd * p[i];
    v[i] = alpha * v[i] + (1.0f - alpha) * g * g;
    if (mom > 0.0f) {
      buf[i] = mom * buf[i] + g / (sqrtf(v[i]) + eps);
      p[i] = p[i] - lr * buf[i];
    } else {
      p[i] = p[i] - lr * g / (sqrtf(v[i]) + eps);
    }
  }
}

/* AdaGrad::step, optim/adagrad.rs:72-99. */
EXPORT void orc_adagrad_step(float *p, const float *g0, float *acc, int64_t n, float lr,
                             float eps, float wd) {
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd != 0.0f) g = g + wd * p[i];
    acc[i] = acc[i] + g * g;
    p[i] = p[i] - lr * g / (sqrtf(acc[i]) + eps);
  }
}

/* NAdam::step, optim/nadam.rs:99-145 (bias corrections with powf). */
EXPORT void orc_nadam_step(float *p, const float *g0, float *m, float *v, int64_t n, float lr,
                           float b1, float b2, float eps, float wd, int t) {
  const float tf = (float)t;
  const float bc1 = 1.0f - powf(b1, tf), bc2 = 1.0f - powf(b2, tf);
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd != 0.0f) g = g + wd * p[i];
    m[i] = b1 * m[i] + (1.0f - b1) * g;
    v[i] = b2 * v[i] + (1.0f - b2) * g * g;
    const float mh = m[i] / bc1, vh = v[i] / bc2;
    const float mbar = b1 * mh + (1.0f - b1) * g / bc1;
    p[i] = p[i] - lr * mbar / (sqrtf(vh) + eps);
  }
}

/* RAdam::step, optim/radam.rs:95-161: the rectification term is derived once
 * per step; returns 1 when the adaptive (rectified) update was used. */
EXPORT int orc_radam_step(float *p, const float *g0, float *m, float *v, int64_t n, float lr,
                          float b1, float b2, float eps, float wd, int t) {
  const float tf = (float)t;
  const float bc1 = 1.0f - powf(b1, tf), bc2 = 1.0f - powf(b2, tf);
  const float rho_inf = 2.0f / (1.0f - b2) - 1.0f;
  const float rho_t = rho_inf - 2.0f * tf * powf(b2, tf) / bc2;
  const int adaptive = rho_t > 5.0f;
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd != 0.0f) g = g + wd * p[i];
    m[i] = b1 * m[i] + (1.0f - b1) * g;
    v[i] = b2 * v[i] + (1.0f - b2) * g * g;
  }
  if (adaptive) {
    const float r = sqrtf((rho_t - 4.0f) * (rho_t - 2.0f) * rho_inf /
                          ((rho_inf - 4.0f) * (rho_inf - 2.0f) * rho_t));
    for (int64_t i = 0; i < n; ++i) {
      const float mh = m[i] / bc1, vh = v[i] / bc2;
      p[i] = p[i] - lr * r * mh / (sqrtf(vh) + eps);
    }
  } else {
    for (int64_t i = 0; i < n; ++i) p[i] = p[i] - lr * (m[i] / bc1);
  }
  return adaptive;
}

/* AdaDelta::step, optim/adadelta.rs:90-131 (deltas use the old E[dx^2]). */
EXPORT void orc_adadelta_step(float *p, const float *g0, float *eg, float *ed, int64_t n,
                              float rho, float eps, float wd) {
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd != 0.0f) g = g + wd * p[i];
    eg[i] = rho * eg[i] + (1.0f - rho) * g * g;
    const float delta = (sqrtf(ed[i] + eps) / sqrtf(eg[i] + eps)) * g;
    ed[i] = rho * ed[i] + (1.0f - rho) * delta * delta;
    p[i] = p[i] - delta;
  }
}

/* AdaBound::step, optim/adabound.rs:116-179 (decay only when wd > 0). */
EXPORT void orc_adabound_step(float *p, const float *g0, float *m, float *v, int64_t n, float lr,
                              float final_lr, float b1, float b2, float eps, float wd, float gamma,
                              int t) {
  const float gamma_t = gamma * (float)t;
  const float lower = final_lr * (1.0f - 1.0f / (gamma_t + 1.0f));
  const float upper = final_lr * (1.0f + 1.0f / fmaxf(gamma_t, 1e-8f));
  const float bc1 = 1.0f - orc_powi(b1, t), bc2 = 1.0f - orc_powi(b2, t);
  const float step_size = lr * (sqrtf(bc2) / bc1);
  for (int64_t i = 0; i < n; ++i) {
    float g = g0[i];
    if (wd > 0.0f) g = g + wd * p[i];
    m[i] = b1 * m[i] + (1.0f - b1) * g;
    v[i] = b2 * v[i] + (1.0f - b2) * g * g;
  }
  for (int64_t i = 0; i < n; ++i) {
    const float mh = m[i] / bc1, vh = v[i] / bc2;
    const float denom = sqrtf(vh) + eps;
    const float lr_t = step_size / denom;
    const float lr_c = fminf(fmaxf(lr_t, lower), upper);
    p[i] = p[i] - lr_c * mh;
  }
}

/* Rprop::step, optim/rprop.rs:103-155 (init :63-93) (step sizes start at lr_init). */
EXPORT void orc_rprop_step(float *p, const float *g, float *step, float *prev, int64_t n,
                           float eta_plus, float eta_minus, float lr_min, float lr_max) {
  for (int64_t i = 0; i < n; ++i) {
    const float sp = g[i] * prev[i];
    if (sp > 0.0f) {
      step[i] = fminf(step[i] * eta_plus, lr_max);
      p[i] = p[i] - step[i] * orc_signum(g[i]);
      prev[i] = g[i];
    } else if (sp < 0.0f) {
      step[i] = fmaxf(step[i] * eta_minus, lr_min);
      prev[i] = 0.0f;
    } else {
      p[i] = p[i] - step[i] * orc_signum(g[i]);
      prev[i] = g[i];
    }
  }
}

/* LAMB::step, optim/lamb.rs:105-176: Adam direction (+ wd*p when wd > 0),
 * layer norms as sequential f32 sums of squares, trust ratio ||w||/||r||
 * (1 when either is 0).  `u` is scratch of n floats.  Returns the ratio. */
EXPORT float orc_lamb_step(float *p, const float *g, float *m, float *v, float *u, int64_t n,
                           float lr, float b1, float b2, float eps, float wd, int t) {
  for (int64_t i = 0; i < n; ++i) {
    m[i] = b1 * m[i] + (1.0f - b1) * g[i];
    v[i] = b2 * v[i] + (1.0f - b2) * g[i] * g[i];
  }
  const float bc1 = 1.0f - orc_powi(b1, t), bc2 = 1.0f - orc_powi(b2, t);
  for (int64_t i = 0; i < n; ++i) {
    const float mh = m[i] / bc1, vh = v[i] / bc2;
    u[i] = mh / (sqrtf(vh) + eps);
  }
  if (wd > 0.0f)
    for (int64_t i = 0; i < n; ++i) u[i] = u[i] + wd * p[i];
  float w2 = 0.0f, u2 = 0.0f;
  for (int64_t i = 0; i < n; ++i) w2 = w2 + p[i] * p[i];
  for (int64_t i = 0; i < n; ++i) u2 = u2 + u[i] * u[i];
  const float wn = sqrtf(w2), un = sqrtf(u2);
  const float trust = (wn > 0.0f && un > 0.0f) ? wn / un : 1.0f;
  for (int64_t i = 0; i < n; ++i) p[i] = p[i] - lr * trust * u[i];
  return trust;
}

/* Lookahead slow-weight update, optim/lookahead.rs:88-120:
 * slow = slow + alpha*(fast - slow); fast = slow. */
EXPORT void orc_lookahead_sync(float *fast, float *slow, int64_t n, float alpha) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = slow[i] + alpha * (fast[i] - slow[i]);
    slow[i] = s;
    fast[i] = s;
  }
}

/* L-BFGS dot product, optim/lbfgs.rs:109-111: sequential f32 sum of products. */
EXPORT float orc_dot_seq(const float *a, const float *b, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s = s + a[i] * b[i];
  return s;
}

/* LR schedulers, optim/schedulers.rs.  State is a float[6] owned by the
 * caller: [0] kind-specific counter, [1] initial/target lr, [2] best metric,
 * [3] epochs since improvement.  Each call returns the learning rate the
 * optimizer holds afterwards (given its current `lr`). */
EXPORT float orc_sched_step_lr(float *st, float lr, int step_size, float gamma) {  /* schedulers.rs:43-61 */
  if (st[0] == 0.0f) st[1] = lr;
  st[0] = st[0] + 1.0f;
  if (((int64_t)st[0]) % step_size == 0) lr = lr * gamma;
  return lr;
}
EXPORT float orc_sched_exponential(float *st, float lr, float gamma) {  /* schedulers.rs:88-102 */
  if (st[0] == 0.0f) st[1] = lr;
  st[0] = st[0] + 1.0f;
  return lr * gamma;
}
EXPORT float orc_sched_cosine(float *st, float lr, int t_max, float eta_min) {  /* schedulers.rs:136-153 */
  if (st[0] == 0.0f) st[1] = lr;
  st[0] = st[0] + 1.0f;
  const float pi = 3.14159265358979323846f;
  const float t = (float)(int64_t)st[0], tm = (float)t_max;
  return eta_min + (st[1] - eta_min) * (1.0f + cosf(pi * t / tm)) / 2.0f;
}
EXPORT float orc_sched_plateau(float *st, float lr, float metric, float factor, int patience,
                               float min_lr) {  /* schedulers.rs:205-227 */
  if (st[1] == 0.0f) st[1] = lr;
  if (st[0] == 0.0f) { st[0] = 1.0f; st[2] = INFINITY; st[3] = 0.0f; }
  if (metric < st[2]) {
    st[2] = metric;
    st[3] = 0.0f;
  } else {
    st[3] = st[3] + 1.0f;
    if ((int)st[3] >= patience) {
      const float nl = fmaxf(lr * factor, min_lr);
      if (nl < lr) {
        lr = nl;
        st[3] = 0.0f;
      }
    }
  }
  return lr;
}
EXPORT float orc_sched_warmup(float *st, float lr, int warmup, float start_lr) {  /* schedulers.rs:272-295 */
  if (st[0] == 0.0f) {
    st[1] = lr;
    lr = start_lr;
  }
  st[0] = st[0] + 1.0f;
  const int cur = (int)st[0];
  if (cur <= warmup) lr = start_lr + (st[1] - start_lr) * ((float)cur / (float)warmup);
  return lr;
}
