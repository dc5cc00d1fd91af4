// The optimizers beyond SGD and Adam (autograd/optim/*), the Lookahead
// slow-weight update, the dot product L-BFGS needs, and the LR schedulers.
//
// Every elementwise update is one multi-tensor launch (all of an optimizer's
// parameters in one grid: block b belongs to tensor t when
// start[t] <= b < start[t+1]) reading p, g and up to two state buffers once
// and writing p and the state once.  Per-step scalars (bias corrections,
// RAdam's rectification, AdaBound's bounds) are derived on the host exactly
// as the reference derives them (powi by square-and-multiply, powf / sqrtf /
// cosf from the C library), so the per-element arithmetic below -- in the
// reference's operation order, built with -ffp-contract=off -- gives the
// reference's bits.  LAMB's layer norms are sums over a whole tensor: they
// are formed from per-block partials in block order (deterministic, but not
// the reference's sequential order), then the trust ratio is applied in a
// second launch.
#include <cmath>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kPerThread = 8;
constexpr int kElemsPerBlock = kBlock * kPerThread;
constexpr int kMaxTensors = 32;

struct OptTensors {
  float *p[kMaxTensors];
  const float *g[kMaxTensors];
  float *s1[kMaxTensors];
  float *s2[kMaxTensors];
  float *aux[kMaxTensors];  // LAMB: the direction u of each tensor
  int64_t n[kMaxTensors];
  int64_t start[kMaxTensors + 1];
  int count;
};

// Per-step scalars; which fields a kind uses is set by derive() below.
struct OptScalars {
  float lr, b1, b2, eps, wd;
  float omb1, omb2;  // 1 - b1, 1 - b2 (the reference's (1.0 - beta) per element)
  float bc1, bc2;    // bias corrections
  float x0, x1, x2;  // kind-specific (RAdam r; AdaBound bounds/step; Rprop limits)
  int flag;          // RMSprop momentum on; RAdam adaptive; decay on
};

__device__ __forceinline__ int tensor_of(const OptTensors &a, int64_t b) {
  int t = 0;
  while (t + 1 < a.count && a.start[t + 1] <= b) ++t;
  return t;
}

__device__ __forceinline__ float signum(float x) {  // f32::signum
  return isnan(x) ? x : copysignf(1.0f, x);
}

// One element of one optimizer step; s1/s2 are the state slots.
template <int KIND>
__device__ __forceinline__ void opt_elem(float &p, float g, float &s1, float &s2,
                                         const OptScalars &a) {
  if constexpr (KIND == NUMRS_HIP_OPT_ADAMW) {  // adamw.rs:92-129
    s1 = a.b1 * s1 + a.omb1 * g;
    s2 = a.b2 * s2 + a.omb2 * g * g;
    const float mh = s1 / a.bc1, vh = s2 / a.bc2;
    p = p - a.lr * (mh / (sqrtf(vh) + a.eps) + a.wd * p);
  } else if constexpr (KIND == NUMRS_HIP_OPT_RMSPROP) {  // rmsprop.rs:90-135
    if (a.wd != 0.0f) g = g + a.wd * p;
    s1 = a.b1 * s1 + a.omb1 * g * g;  // b1 = alpha
    if (a.flag) {                      // momentum > 0 (b2 = momentum)
      s2 = a.b2 * s2 + g / (sqrtf(s1) + a.eps);
      p = p - a.lr * s2;
    } else {
      p = p - a.lr * g / (sqrtf(s1) + a.eps);
    }
  } else if constexpr (KIND == NUMRS_HIP_OPT_ADAGRAD) {  // adagrad.rs:72-99
    if (a.wd != 0.0f) g = g + a.wd * p;
    s1 = s1 + g * g;
    p = p - a.lr * g / (sqrtf(s1) + a.eps);
  } else if constexpr (KIND == NUMRS_HIP_OPT_NADAM) {  // nadam.rs:99-145
    if (a.wd != 0.0f) g = g + a.wd * p;
    s1 = a.b1 * s1 + a.omb1 * g;
    s2 = a.b2 * s2 + a.omb2 * g * g;
    const float mh = s1 / a.bc1, vh = s2 / a.bc2;
    const float mbar = a.b1 * mh + a.omb1 * g / a.bc1;
    p = p - a.lr * mbar / (sqrtf(vh) + a.eps);
  } else if constexpr (KIND == NUMRS_HIP_OPT_RADAM) {  // radam.rs:95-161
    if (a.wd != 0.0f) g = g + a.wd * p;
    s1 = a.b1 * s1 + a.omb1 * g;
    s2 = a.b2 * s2 + a.omb2 * g * g;
    if (a.flag) {
      const float mh = s1 / a.bc1, vh = s2 / a.bc2;
      p = p - a.lr * a.x0 * mh / (sqrtf(vh) + a.eps);  // x0 = r
    } else {
      p = p - a.lr * (s1 / a.bc1);
    }
  } else if constexpr (KIND == NUMRS_HIP_OPT_ADADELTA) {  // adadelta.rs:90-131
    if (a.wd != 0.0f) g = g + a.wd * p;
    s1 = a.b1 * s1 + a.omb1 * g * g;  // b1 = rho
    const float delta = (sqrtf(s2 + a.eps) / sqrtf(s1 + a.eps)) * g;
    s2 = a.b1 * s2 + a.omb1 * delta * delta;
    p = p - delta;
  } else if constexpr (KIND == NUMRS_HIP_OPT_ADABOUND) {  // adabound.rs:116-179
    if (a.wd > 0.0f) g = g + a.wd * p;
    s1 = a.b1 * s1 + a.omb1 * g;
    s2 = a.b2 * s2 + a.omb2 * g * g;
    const float mh = s1 / a.bc1, vh = s2 / a.bc2;
    const float lr_t = a.x2 / (sqrtf(vh) + a.eps);  // x2 = step size
    const float lr_c = fminf(fmaxf(lr_t, a.x0), a.x1);  // x0 lower, x1 upper
    p = p - lr_c * mh;
  } else if constexpr (KIND == NUMRS_HIP_OPT_RPROP) {  // rprop.rs:103-155
    // s1 = step size, s2 = previous gradient; b1 = eta+, b2 = eta-,
    // x0 = lr_min, x1 = lr_max
    const float sp = g * s2;
    if (sp > 0.0f) {
      s1 = fminf(s1 * a.b1, a.x1);
      p = p - s1 * signum(g);
      s2 = g;
    } else if (sp < 0.0f) {
      s1 = fmaxf(s1 * a.b2, a.x0);
      s2 = 0.0f;
    } else {
      p = p - s1 * signum(g);
      s2 = g;
    }
  }
}

template <int KIND>
__global__ void __launch_bounds__(kBlock) opt_multi_kernel(OptTensors a, OptScalars s) {
  const int t = tensor_of(a, blockIdx.x);
  const int64_t n = a.n[t];
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
  float *__restrict__ p = a.p[t];
  const float *__restrict__ g = a.g[t];
  float *__restrict__ s1 = a.s1[t];
  float *__restrict__ s2 = a.s2[t];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t k = base + (int64_t)u * kBlock;
    if (k < n) {
      float pe = p[k];
      float e1 = s1 != nullptr ? s1[k] : 0.0f;
      float e2 = s2 != nullptr ? s2[k] : 0.0f;
      opt_elem<KIND>(pe, g[k], e1, e2, s);
      p[k] = pe;
      if (s1 != nullptr) s1[k] = e1;
      if (s2 != nullptr) s2[k] = e2;
    }
  }
}

// LAMB pass 1 (lamb.rs:118-150): moments in place, the direction
// u = m_hat/(sqrt(v_hat)+eps) (+ wd*p when wd > 0) into aux, and this
// block's partial sums of p^2 and u^2 into part[2*b], part[2*b+1].
__global__ void __launch_bounds__(kBlock)
    lamb_pass1(OptTensors a, OptScalars s, float *__restrict__ part) {
  __shared__ float red[2][kBlock / 64];
  const int t = tensor_of(a, blockIdx.x);
  const int64_t n = a.n[t];
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
  float *__restrict__ p = a.p[t];
  const float *__restrict__ g = a.g[t];
  float *__restrict__ m = a.s1[t];
  float *__restrict__ v = a.s2[t];
  float *__restrict__ u = a.aux[t];
  float w2 = 0.0f, u2 = 0.0f;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int64_t k = base + (int64_t)i * kBlock;
    if (k < n) {
      const float gk = g[k];
      const float mk = s.b1 * m[k] + s.omb1 * gk;
      const float vk = s.b2 * v[k] + s.omb2 * gk * gk;
      m[k] = mk;
      v[k] = vk;
      const float mh = mk / s.bc1, vh = vk / s.bc2;
      float uk = mh / (sqrtf(vh) + s.eps);
      const float pk = p[k];
      if (s.wd > 0.0f) uk = uk + s.wd * pk;
      u[k] = uk;
      w2 += pk * pk;
      u2 += uk * uk;
    }
  }
  w2 = wave_sum(w2);
  u2 = wave_sum(u2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[0][wave] = w2;
    red[1][wave] = u2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a0 = red[0][0], a1 = red[1][0];
    for (int w = 1; w < kBlock / 64; ++w) {
      a0 += red[0][w];
      a1 += red[1][w];
    }
    part[2 * blockIdx.x] = a0;
    part[2 * blockIdx.x + 1] = a1;
  }
}

// LAMB pass 2 (lamb.rs:152-167): block t adds tensor t's block partials
// (thread-strided, then wave and LDS order: deterministic) and forms the
// trust ratio ||w||/||u||, or 1 when either norm is 0.
__global__ void __launch_bounds__(kBlock)
    lamb_ratio(OptTensors a, const float *__restrict__ part, float *__restrict__ ratio) {
  __shared__ float red[2][kBlock / 64];
  const int t = blockIdx.x;
  float w2 = 0.0f, u2 = 0.0f;
  for (int64_t b = a.start[t] + threadIdx.x; b < a.start[t + 1]; b += kBlock) {
    w2 += part[2 * b];
    u2 += part[2 * b + 1];
  }
  w2 = wave_sum(w2);
  u2 = wave_sum(u2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[0][wave] = w2;
    red[1][wave] = u2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a0 = red[0][0], a1 = red[1][0];
    for (int w = 1; w < kBlock / 64; ++w) {
      a0 += red[0][w];
      a1 += red[1][w];
    }
    const float wn = sqrtf(a0), un = sqrtf(a1);
    ratio[t] = (wn > 0.0f && un > 0.0f) ? wn / un : 1.0f;
  }
}

// LAMB pass 3 (lamb.rs:169-172): p -= (lr * ratio) * u.
__global__ void __launch_bounds__(kBlock)
    lamb_apply(OptTensors a, float lr, const float *__restrict__ ratio) {
  const int t = tensor_of(a, blockIdx.x);
  const int64_t n = a.n[t];
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
  float *__restrict__ p = a.p[t];
  const float *__restrict__ u = a.aux[t];
  const float step = lr * ratio[t];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int64_t k = base + (int64_t)i * kBlock;
    if (k < n) p[k] = p[k] - step * u[k];
  }
}

// Lookahead (lookahead.rs:88-120): slow = slow + alpha*(fast - slow); fast = slow.
__global__ void __launch_bounds__(kBlock) lookahead_kernel(OptTensors a, float alpha) {
  const int t = tensor_of(a, blockIdx.x);
  const int64_t n = a.n[t];
  const int64_t base = (int64_t)(blockIdx.x - a.start[t]) * kElemsPerBlock + threadIdx.x;
  float *__restrict__ fast = a.p[t];
  float *__restrict__ slow = a.s1[t];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int64_t k = base + (int64_t)i * kBlock;
    if (k < n) {
      const float sv = slow[k] + alpha * (fast[k] - slow[k]);
      slow[k] = sv;
      fast[k] = sv;
    }
  }
}

// Dot product in two deterministic passes: per-block partials, then one block
// adds them in order.
constexpr int kDotBlocks = 1024;

__global__ void __launch_bounds__(kBlock)
    dot_pass1(const float *__restrict__ x, const float *__restrict__ y, int64_t n,
              float *__restrict__ part) {
  __shared__ float red[kBlock / 64];
  float s = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock)
    s += x[i] * y[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
    for (int w = 1; w < kBlock / 64; ++w) t += red[w];
    part[blockIdx.x] = t;
  }
}

__global__ void __launch_bounds__(kBlock)
    dot_pass2(const float *__restrict__ part, int blocks, float *__restrict__ out) {
  __shared__ float red[kBlock / 64];
  float s = 0.0f;
  for (int i = threadIdx.x; i < blocks; i += kBlock) s += part[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
    for (int w = 1; w < kBlock / 64; ++w) t += red[w];
    *out = t;
  }
}

__global__ void __launch_bounds__(kBlock)
    vec_kernel(float *__restrict__ out, const float *__restrict__ a, const float *__restrict__ b,
               float s, int64_t n, int op) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  float r;
  switch (op) {
    case numrs_hip::kVecSub: r = a[i] - b[i]; break;
    case numrs_hip::kVecAxmy: r = a[i] - s * b[i]; break;
    case numrs_hip::kVecScale: r = s * a[i]; break;
    case numrs_hip::kVecAypx: r = a[i] + b[i] * s; break;
    case numrs_hip::kVecNeg: r = -a[i]; break;
    default: r = a[i] + s * b[i]; break;
  }
  out[i] = r;
}

// f32::powi as compiled for x86-64 (compiler-rt __powisf2).
float powi_host(float a, int b) {
  const bool recip = b < 0;
  if (recip) b = -b;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r = r * a;
    b /= 2;
    if (b == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / r : r;
}

int hyper_count(int kind) {
  switch (kind) {
    case NUMRS_HIP_OPT_ADAMW:
    case NUMRS_HIP_OPT_RMSPROP:
    case NUMRS_HIP_OPT_NADAM:
    case NUMRS_HIP_OPT_RADAM:
    case NUMRS_HIP_OPT_RPROP:
    case NUMRS_HIP_OPT_LAMB:
      return 5;
    case NUMRS_HIP_OPT_ADAGRAD:
    case NUMRS_HIP_OPT_ADADELTA:
      return 3;
    case NUMRS_HIP_OPT_ADABOUND:
      return 7;
    default:
      return -1;
  }
}

bool uses_t(int kind) {
  return kind == NUMRS_HIP_OPT_ADAMW || kind == NUMRS_HIP_OPT_NADAM ||
         kind == NUMRS_HIP_OPT_RADAM || kind == NUMRS_HIP_OPT_ADABOUND ||
         kind == NUMRS_HIP_OPT_LAMB;
}

// Which state slots a kind reads and writes: every kind keeps a first slot;
// AdaGrad and momentum-free RMSprop have no second one.
void state_slots(int kind, const float *h, bool *s1, bool *s2) {
  *s1 = true;
  *s2 = !(kind == NUMRS_HIP_OPT_ADAGRAD ||
          (kind == NUMRS_HIP_OPT_RMSPROP && !(h[4] > 0.0f)));
}

// Derives the per-step scalars of `kind` from its hyperparameters (in the
// reference constructor's order) and the step counter t.
OptScalars derive(int kind, const float *h, int t) {
  OptScalars s{};
  switch (kind) {
    case NUMRS_HIP_OPT_ADAMW:
    case NUMRS_HIP_OPT_LAMB:  // lr, beta1, beta2, eps, weight_decay
      s.lr = h[0], s.b1 = h[1], s.b2 = h[2], s.eps = h[3], s.wd = h[4];
      s.omb1 = 1.0f - s.b1, s.omb2 = 1.0f - s.b2;
      s.bc1 = 1.0f - powi_host(s.b1, t), s.bc2 = 1.0f - powi_host(s.b2, t);
      break;
    case NUMRS_HIP_OPT_RMSPROP:  // lr, alpha, eps, weight_decay, momentum
      s.lr = h[0], s.b1 = h[1], s.eps = h[2], s.wd = h[3], s.b2 = h[4];
      s.omb1 = 1.0f - s.b1;
      s.flag = h[4] > 0.0f;
      break;
    case NUMRS_HIP_OPT_ADAGRAD:  // lr, eps, weight_decay
      s.lr = h[0], s.eps = h[1], s.wd = h[2];
      break;
    case NUMRS_HIP_OPT_NADAM:
    case NUMRS_HIP_OPT_RADAM: {  // lr, beta1, beta2, eps, weight_decay (powf corrections)
      s.lr = h[0], s.b1 = h[1], s.b2 = h[2], s.eps = h[3], s.wd = h[4];
      s.omb1 = 1.0f - s.b1, s.omb2 = 1.0f - s.b2;
      const float tf = (float)t;
      s.bc1 = 1.0f - powf(s.b1, tf), s.bc2 = 1.0f - powf(s.b2, tf);
      if (kind == NUMRS_HIP_OPT_RADAM) {  // radam.rs:100-113, 136-138
        const float rho_inf = 2.0f / (1.0f - s.b2) - 1.0f;
        const float rho_t = rho_inf - 2.0f * tf * powf(s.b2, tf) / s.bc2;
        s.flag = rho_t > 5.0f;
        if (s.flag)
          s.x0 = sqrtf((rho_t - 4.0f) * (rho_t - 2.0f) * rho_inf /
                       ((rho_inf - 4.0f) * (rho_inf - 2.0f) * rho_t));
      }
      break;
    }
    case NUMRS_HIP_OPT_ADADELTA:  // rho, eps, weight_decay
      s.b1 = h[0], s.eps = h[1], s.wd = h[2];
      s.omb1 = 1.0f - s.b1;
      break;
    case NUMRS_HIP_OPT_ADABOUND: {  // lr, final_lr, beta1, beta2, eps, weight_decay, gamma
      s.lr = h[0];
      const float final_lr = h[1];
      s.b1 = h[2], s.b2 = h[3], s.eps = h[4], s.wd = h[5];
      const float gamma = h[6];
      s.omb1 = 1.0f - s.b1, s.omb2 = 1.0f - s.b2;
      const float gamma_t = gamma * (float)t;  // adabound.rs:121-123
      s.x0 = final_lr * (1.0f - 1.0f / (gamma_t + 1.0f));
      s.x1 = final_lr * (1.0f + 1.0f / fmaxf(gamma_t, 1e-8f));
      s.bc1 = 1.0f - powi_host(s.b1, t), s.bc2 = 1.0f - powi_host(s.b2, t);
      s.x2 = s.lr * (sqrtf(s.bc2) / s.bc1);
      break;
    }
    case NUMRS_HIP_OPT_RPROP:  // lr_init, eta_plus, eta_minus, lr_min, lr_max
      s.lr = h[0], s.b1 = h[1], s.b2 = h[2], s.x0 = h[3], s.x1 = h[4];
      break;
  }
  return s;
}

int64_t pack(OptTensors &a, float *const *p, const float *const *g, float *const *s1,
             float *const *s2, const int64_t *n, int first, int cnt) {
  a.count = cnt;
  int64_t blocks = 0;
  for (int i = 0; i < cnt; ++i) {
    a.p[i] = p[first + i];
    a.g[i] = g != nullptr ? g[first + i] : nullptr;
    a.s1[i] = s1 != nullptr ? s1[first + i] : nullptr;
    a.s2[i] = s2 != nullptr ? s2[first + i] : nullptr;
    a.aux[i] = nullptr;
    a.n[i] = n[first + i];
    a.start[i] = blocks;
    blocks += (n[first + i] + kElemsPerBlock - 1) / kElemsPerBlock;
  }
  a.start[cnt] = blocks;
  return blocks;
}

template <int KIND>
int launch_kind(numrs_hip_ctx *ctx, const OptTensors &a, const OptScalars &s, int64_t blocks) {
  opt_multi_kernel<KIND><<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, s);
  return numrs_hip::check_launch(ctx, "opt_multi_kernel");
}

int launch_elementwise(numrs_hip_ctx *ctx, int kind, const OptTensors &a, const OptScalars &s,
                       int64_t blocks) {
  switch (kind) {
    case NUMRS_HIP_OPT_ADAMW: return launch_kind<NUMRS_HIP_OPT_ADAMW>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_RMSPROP: return launch_kind<NUMRS_HIP_OPT_RMSPROP>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_ADAGRAD: return launch_kind<NUMRS_HIP_OPT_ADAGRAD>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_NADAM: return launch_kind<NUMRS_HIP_OPT_NADAM>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_RADAM: return launch_kind<NUMRS_HIP_OPT_RADAM>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_ADADELTA: return launch_kind<NUMRS_HIP_OPT_ADADELTA>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_ADABOUND: return launch_kind<NUMRS_HIP_OPT_ADABOUND>(ctx, a, s, blocks);
    case NUMRS_HIP_OPT_RPROP: return launch_kind<NUMRS_HIP_OPT_RPROP>(ctx, a, s, blocks);
    default: return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "optimizer kind %d", kind);
  }
}

}  // namespace

namespace numrs_hip {

int vec_op(numrs_hip_ctx *ctx, float *out, const float *a, const float *b, float s, int64_t n,
           int op) {
  if (n <= 0) return NUMRS_HIP_OK;
  vec_kernel<<<grid_for(n, kBlock), kBlock, 0, ctx->stream>>>(out, a, b, s, n, op);
  return check_launch(ctx, "vec_kernel");
}

}  // namespace numrs_hip

// ---------------------------------------------------------------------------
// LR schedulers (optim/schedulers.rs), host-side state machines driving an
// engine optimizer's learning rate through numrs_hip_optim_lr/_set_lr.
// ---------------------------------------------------------------------------
struct numrs_hip_scheduler {
  int kind;
  float h[3];
  int64_t epoch = 0;  // current_epoch / current_step
  float initial_lr = 0.0f;  // initial_lr / target_lr
  float best = INFINITY;
  int64_t since = 0;
};

extern "C" {

int numrs_hip_optimizer_step(numrs_hip_ctx *ctx, int kind, float *const *p,
                             const float *const *g, float *const *s1, float *const *s2,
                             const int64_t *n, int count, const float *hyper, int nhyper, int t) {
  NRS_CHECK_CTX(ctx);
  const int want = hyper_count(kind);
  if (want < 0) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "optimizer kind %d", kind);
  if (hyper == nullptr || nhyper != want)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID,
                           "optimizer kind %d takes %d hyperparameters, got %d", kind, want,
                           nhyper);
  if (uses_t(kind) && t < 1)
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "optimizer step counter t < 1");
  bool need1, need2;
  state_slots(kind, hyper, &need1, &need2);
  if (count < 0 || (count > 0 && (p == nullptr || g == nullptr || n == nullptr ||
                                  (need1 && s1 == nullptr) || (need2 && s2 == nullptr))))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_optimizer_step: bad arguments");
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (p[i] == nullptr || g[i] == nullptr ||
                                  (need1 && s1[i] == nullptr) || (need2 && s2[i] == nullptr))))
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_optimizer_step: tensor %d", i);
  const OptScalars s = derive(kind, hyper, t);
  for (int first = 0; first < count; first += kMaxTensors) {
    const int cnt = count - first < kMaxTensors ? count - first : kMaxTensors;
    OptTensors a;
    const int64_t blocks = pack(a, p, g, need1 ? s1 : nullptr, need2 ? s2 : nullptr, n, first, cnt);
    if (blocks == 0) continue;
    if (blocks > 0x7fffffff) return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "too many elements");
    if (kind != NUMRS_HIP_OPT_LAMB) {
      if (int rc = launch_elementwise(ctx, kind, a, s, blocks)) return rc;
      continue;
    }
    // LAMB: direction into a temporary per tensor, partial norms, ratios,
    // then the update.  Scratch layout: [ratios | partials | directions].
    int64_t total = 0;
    for (int i = 0; i < cnt; ++i) total += a.n[i];
    float *buf = nullptr;
    const int64_t head = kMaxTensors + 2 * blocks;
    if (int rc = numrs_hip::scratch(ctx, (size_t)(head + total) * sizeof(float), &buf)) return rc;
    float *ratio = buf, *part = buf + kMaxTensors;
    int64_t off = head;
    for (int i = 0; i < cnt; ++i) {
      a.aux[i] = buf + off;
      off += a.n[i];
    }
    lamb_pass1<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, s, part);
    if (int rc = numrs_hip::check_launch(ctx, "lamb_pass1")) return rc;
    lamb_ratio<<<(unsigned)cnt, kBlock, 0, ctx->stream>>>(a, part, ratio);
    if (int rc = numrs_hip::check_launch(ctx, "lamb_ratio")) return rc;
    lamb_apply<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, s.lr, ratio);
    if (int rc = numrs_hip::check_launch(ctx, "lamb_apply")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_lookahead_update(numrs_hip_ctx *ctx, float *const *fast, float *const *slow,
                               const int64_t *n, int count, float alpha) {
  NRS_CHECK_CTX(ctx);
  if (count < 0 || (count > 0 && (fast == nullptr || slow == nullptr || n == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_lookahead_update: bad arguments");
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (fast[i] == nullptr || slow[i] == nullptr)))
      return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_lookahead_update: tensor %d",
                             i);
  for (int first = 0; first < count; first += kMaxTensors) {
    const int cnt = count - first < kMaxTensors ? count - first : kMaxTensors;
    OptTensors a;
    const int64_t blocks = pack(a, fast, nullptr, slow, nullptr, n, first, cnt);
    if (blocks == 0) continue;
    lookahead_kernel<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, alpha);
    if (int rc = numrs_hip::check_launch(ctx, "lookahead_kernel")) return rc;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_dot(numrs_hip_ctx *ctx, const float *x, const float *y, int64_t n, float *out) {
  NRS_CHECK_CTX(ctx);
  if (n < 0 || out == nullptr || (n > 0 && (x == nullptr || y == nullptr)))
    return numrs_hip::fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_dot: bad arguments");
  int blocks = (int)((n + kBlock * 8 - 1) / (kBlock * 8));
  if (blocks < 1) blocks = 1;
  if (blocks > kDotBlocks) blocks = kDotBlocks;
  void *ws = nullptr;
  if (int rc = numrs_hip::workspace(ctx, (size_t)blocks * sizeof(float), &ws)) return rc;
  float *part = static_cast<float *>(ws);
  dot_pass1<<<blocks, kBlock, 0, ctx->stream>>>(x, y, n, part);
  if (int rc = numrs_hip::check_launch(ctx, "dot_pass1")) return rc;
  dot_pass2<<<1, kBlock, 0, ctx->stream>>>(part, blocks, out);
  return numrs_hip::check_launch(ctx, "dot_pass2");
}

int numrs_hip_scheduler_create(int kind, const float *hyper, int nhyper,
                               numrs_hip_scheduler **out) {
  if (out == nullptr) return NUMRS_HIP_E_INVALID;
  *out = nullptr;
  static const int want[] = {2, 1, 2, 3, 2};
  if (kind < 0 || kind > NUMRS_HIP_SCHED_WARMUP || hyper == nullptr || nhyper != want[kind])
    return NUMRS_HIP_E_INVALID;
  if ((kind == NUMRS_HIP_SCHED_STEP || kind == NUMRS_HIP_SCHED_COSINE ||
       kind == NUMRS_HIP_SCHED_WARMUP) && !(hyper[0] >= 1.0f))
    return NUMRS_HIP_E_INVALID;  // step_size / t_max / warmup_steps are counts >= 1
  auto *s = new numrs_hip_scheduler();
  s->kind = kind;
  for (int i = 0; i < nhyper; ++i) s->h[i] = hyper[i];
  *out = s;
  return NUMRS_HIP_OK;
}

int numrs_hip_scheduler_step(numrs_hip_scheduler *s, numrs_hip_optim *opt) {
  if (s == nullptr || opt == nullptr) return NUMRS_HIP_E_INVALID;
  const float lr = numrs_hip_optim_lr(opt);
  switch (s->kind) {
    case NUMRS_HIP_SCHED_STEP: {  // schedulers.rs:43-61
      if (s->epoch == 0) s->initial_lr = lr;
      s->epoch += 1;
      if (s->epoch % (int64_t)s->h[0] == 0) return numrs_hip_optim_set_lr(opt, lr * s->h[1]);
      return NUMRS_HIP_OK;
    }
    case NUMRS_HIP_SCHED_EXPONENTIAL:  // schedulers.rs:88-102
      if (s->epoch == 0) s->initial_lr = lr;
      s->epoch += 1;
      return numrs_hip_optim_set_lr(opt, lr * s->h[0]);
    case NUMRS_HIP_SCHED_COSINE:  // schedulers.rs:136-153
      if (s->epoch == 0) s->initial_lr = lr;
      s->epoch += 1;
      return numrs_hip_optim_set_lr(opt, numrs_hip_scheduler_get_lr(s));
    case NUMRS_HIP_SCHED_WARMUP: {  // schedulers.rs:272-295
      if (s->epoch == 0) {
        s->initial_lr = lr;  // target_lr
        if (int rc = numrs_hip_optim_set_lr(opt, s->h[1])) return rc;
      }
      s->epoch += 1;
      const int64_t w = (int64_t)s->h[0];
      if (s->epoch <= w)
        return numrs_hip_optim_set_lr(
            opt, s->h[1] + (s->initial_lr - s->h[1]) * ((float)s->epoch / (float)w));
      return NUMRS_HIP_OK;
    }
    default:  // ReduceLROnPlateau takes a metric (schedulers.rs:229-233)
      return NUMRS_HIP_E_INVALID;
  }
}

int numrs_hip_scheduler_step_metric(numrs_hip_scheduler *s, float metric, numrs_hip_optim *opt) {
  if (s == nullptr || opt == nullptr || s->kind != NUMRS_HIP_SCHED_PLATEAU)
    return NUMRS_HIP_E_INVALID;
  // schedulers.rs:205-227
  if (s->initial_lr == 0.0f) s->initial_lr = numrs_hip_optim_lr(opt);
  if (metric < s->best) {
    s->best = metric;
    s->since = 0;
  } else {
    s->since += 1;
    if (s->since >= (int64_t)s->h[1]) {
      const float cur = numrs_hip_optim_lr(opt);
      const float nl = fmaxf(cur * s->h[0], s->h[2]);
      if (nl < cur) {
        if (int rc = numrs_hip_optim_set_lr(opt, nl)) return rc;
        s->since = 0;
      }
    }
  }
  return NUMRS_HIP_OK;
}

float numrs_hip_scheduler_get_lr(const numrs_hip_scheduler *s) {
  if (s == nullptr) return NAN;
  switch (s->kind) {
    case NUMRS_HIP_SCHED_STEP:  // schedulers.rs:57-60
      return s->initial_lr * powf(s->h[1], (float)(s->epoch / (int64_t)s->h[0]));
    case NUMRS_HIP_SCHED_EXPONENTIAL:  // :99-101
      return s->initial_lr * powf(s->h[0], (float)s->epoch);
    case NUMRS_HIP_SCHED_COSINE: {  // :147-152
      const float pi = 3.14159265358979323846f;
      const float t = (float)s->epoch, tm = (float)(int64_t)s->h[0];
      return s->h[1] + (s->initial_lr - s->h[1]) * (1.0f + cosf(pi * t / tm)) / 2.0f;
    }
    case NUMRS_HIP_SCHED_PLATEAU:  // :235-237
      return s->initial_lr;
    case NUMRS_HIP_SCHED_WARMUP: {  // :288-294
      const int64_t w = (int64_t)s->h[0];
      if (s->epoch >= w) return s->initial_lr;
      return s->h[1] + (s->initial_lr - s->h[1]) * ((float)s->epoch / (float)w);
    }
    default:
      return NAN;
  }
}

int numrs_hip_scheduler_free(numrs_hip_scheduler *s) {
  delete s;
  return NUMRS_HIP_OK;
}

}  // extern "C"
