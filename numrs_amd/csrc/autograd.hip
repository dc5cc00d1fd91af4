// Device-resident autograd engine: numrs's Tensor / ComputeNode / backward
// (autograd/tensor.rs, autograd/mod.rs, autograd/ops.rs) with every buffer on
// the GPU and every BackwardFn body a kernel of this library.
//
// Semantics kept from the reference:
//   * A tensor that requires grad owns a grad cell shared by all handles and
//     graph references to it (Rc<RefCell<Array>>, tensor.rs:18-33).  The cell
//     is logically zero at creation (tensor.rs:41-83); it is materialised
//     lazily: the first backward producer writes it (accumulate = 0), later
//     producers add (accumulate = 1) -- accumulate_gradient, tensor.rs:120-132.
//   * backward() seeds ones of the output's shape (set_gradient, :178-183),
//     builds the DFS post-order of build_topo (:218-239; non-leaf nodes are
//     visited once, inputs in order), and walks it in reverse (:191-212),
//     handing each node's grad to its backward body, which writes directly
//     into the grads of the inputs that require grad (:205-209).
//   * A node is recorded only when grad mode is on and an input requires
//     grad (ops.rs:21 and every op); grad mode is thread-local (mod.rs:194-206).
//   * Broadcast gradients go through unbroadcast (backward.rs:12-39) in the
//     context's mode: CORRECT (axis sums) or REFERENCE (the reference's
//     full sum into element 0).
// Every BackwardFn is linear in its incoming grad, so a node whose grad was
// never written (still logically zero) contributes nothing and is skipped.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <unordered_set>
#include <utility>
#include <vector>

#include "common.h"

namespace {

using numrs_hip::fail;

thread_local bool g_grad_enabled = true;  // mod.rs:194-206

enum class Op {
  Leaf, Add, Sub, Mul, Div, MatMul, Transpose, Unary, Sum, Mean, MSE, CrossEntropy,
  CrossEntropyLabels, Reshape, Softmax, LayerNorm, Attention, Linear, LSTM, TimeSlice, SumAxis,
  SoftmaxAxis, LSTM2
};

struct Storage {
  numrs_hip_ctx *ctx = nullptr;
  float *ptr = nullptr;
  size_t bytes = 0;
  ~Storage() { numrs_hip::block_free(ctx, ptr, bytes); }
};
using Buf = std::shared_ptr<Storage>;

struct GradCell {
  Buf buf;
  bool valid = false;  // false: logically zero
  // A scalar loss's cell whose buffer holds the backward seed 1, written by the
  // loss's forward kernel together with the root gradient it pre-formed;
  // cleared by every other write to the cell.
  bool seed_preset = false;
};

struct Node;
struct Impl {
  numrs_hip_ctx *ctx = nullptr;
  std::vector<int64_t> shape;
  Buf data;
  std::shared_ptr<GradCell> grad;  // null when the tensor does not require grad
  bool requires_grad = false;
  bool is_leaf = true;
  std::shared_ptr<Node> node;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};
using T = std::shared_ptr<Impl>;

struct Node {
  uint64_t id;
  Op op;
  int kind = 0;       // unary kind / mean flag
  float param = 0.f;  // pow exponent, LayerNorm eps
  int64_t dims[3] = {0, 0, 0};  // attention batch, seq, heads; axis ops' [outer, n, inner]
  std::vector<T> inputs;
  std::vector<Buf> saved;  // LayerNorm mean/rstd, int32 labels
};

uint64_t next_node_id() {  // NodeId::new, mod.rs:46-51
  static uint64_t counter = 0;
  return counter++;
}

int alloc_buf(numrs_hip_ctx *ctx, int64_t count, size_t elem, Buf *out) {
  auto s = std::make_shared<Storage>();
  s->ctx = ctx;
  s->bytes = (size_t)count * elem;
  void *p = nullptr;
  if (int rc = numrs_hip::block_alloc(ctx, s->bytes, &p)) return rc;
  s->ptr = static_cast<float *>(p);
  *out = std::move(s);
  return NUMRS_HIP_OK;
}

int make_tensor(numrs_hip_ctx *ctx, std::vector<int64_t> shape, bool requires_grad, T *out) {
  auto t = std::make_shared<Impl>();
  t->ctx = ctx;
  t->shape = std::move(shape);
  if (int rc = alloc_buf(ctx, t->numel(), sizeof(float), &t->data)) return rc;
  t->requires_grad = requires_grad;
  if (requires_grad) t->grad = std::make_shared<GradCell>();
  *out = std::move(t);
  return NUMRS_HIP_OK;
}

// Tensor::from_operation (tensor.rs:62-83): attaches the node when recording.
void attach(T &out, Op op, std::vector<T> inputs, int kind = 0, float param = 0.f,
            std::vector<Buf> saved = {}) {
  auto n = std::make_shared<Node>();
  n->id = next_node_id();
  n->op = op;
  n->kind = kind;
  n->param = param;
  n->inputs = std::move(inputs);
  n->saved = std::move(saved);
  out->node = std::move(n);
  out->is_leaf = false;
}

bool recording(std::initializer_list<const T *> ins) {
  if (!g_grad_enabled) return false;
  for (const T *t : ins)
    if ((*t)->requires_grad) return true;
  return false;
}

// Grad buffer of `t` for a producer; *acc tells whether to add (1) or write (0).
int grad_target(const T &t, float **ptr, int *acc) {
  GradCell &c = *t->grad;
  c.seed_preset = false;
  if (!c.buf)
    if (int rc = alloc_buf(t->ctx, t->numel(), sizeof(float), &c.buf)) return rc;
  *acc = c.valid ? 1 : 0;
  c.valid = true;
  *ptr = c.buf->ptr;
  return NUMRS_HIP_OK;
}

// Grad of `t` as a materialised buffer (zero-filled if never written).
int grad_materialise(const T &t) {
  GradCell &c = *t->grad;
  c.seed_preset = false;
  if (!c.buf)
    if (int rc = alloc_buf(t->ctx, t->numel(), sizeof(float), &c.buf)) return rc;
  if (!c.valid) {
    if (int rc = numrs_hip_fill(t->ctx, c.buf->ptr, t->numel(), 0.0f)) return rc;
    c.valid = true;
  }
  return NUMRS_HIP_OK;
}

bool same_shape(const std::vector<int64_t> &a, const std::vector<int64_t> &b) { return a == b; }

// ---------------------------------------------------------------------------
// Backward bodies (backward.rs), writing into input grads
// ---------------------------------------------------------------------------

// dst_grad(in) (+)= unbroadcast(src) where src has shape `gshape`.
int add_into(const T &in, const float *src, const std::vector<int64_t> &gshape) {
  numrs_hip_ctx *ctx = in->ctx;
  float *dst;
  int acc;
  if (int rc = grad_target(in, &dst, &acc)) return rc;
  return numrs_hip_sum_to_shape(ctx, src, gshape.data(), (int)gshape.size(), dst,
                                in->shape.data(), (int)in->shape.size(), ctx->unbroadcast_mode,
                                acc);
}

int temp(numrs_hip_ctx *ctx, int64_t n, Buf *out) { return alloc_buf(ctx, n, sizeof(float), out); }

int bw_add_sub(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0], &y = n.inputs[1];
  numrs_hip_ctx *ctx = out->ctx;
  const int64_t N = out->numel();
  if (x->requires_grad)
    if (int rc = add_into(x, g, out->shape)) return rc;  // backward.rs:50 / :62
  if (!y->requires_grad) return NUMRS_HIP_OK;
  if (n.op == Op::Add) return add_into(y, g, out->shape);  // backward.rs:51
  // sub: dy = unbroadcast(g * -1), backward.rs:65-67
  if (same_shape(y->shape, out->shape)) {
    float *dst;
    int acc;
    if (int rc = grad_target(y, &dst, &acc)) return rc;
    return numrs_hip_binary_backward(ctx, NUMRS_HIP_SUB, g, nullptr, nullptr, nullptr, dst, N, acc);
  }
  Buf t;
  if (int rc = temp(ctx, N, &t)) return rc;
  if (int rc = numrs_hip_binary_backward(ctx, NUMRS_HIP_SUB, g, nullptr, nullptr, nullptr, t->ptr,
                                         N, 0))
    return rc;
  return add_into(y, t->ptr, out->shape);
}

int bw_mul_div(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0], &y = n.inputs[1];
  numrs_hip_ctx *ctx = out->ctx;
  const int64_t N = out->numel();
  const int kind = n.op == Op::Mul ? NUMRS_HIP_MUL : NUMRS_HIP_DIV;
  const bool flat = same_shape(x->shape, out->shape) && same_shape(y->shape, out->shape);
  if (flat) {
    // backward.rs:74-109 on equal shapes: one fused pass per grad (separate
    // calls when both inputs share one grad cell, e.g. x * x).
    float *dx = nullptr, *dy = nullptr;
    int ax = 0, ay = 0;
    if (x->requires_grad && y->requires_grad && x->grad == y->grad) {
      if (int rc = grad_target(x, &dx, &ax)) return rc;
      if (int rc = numrs_hip_binary_backward(ctx, kind, g, x->data->ptr, y->data->ptr, dx, nullptr,
                                             N, ax))
        return rc;
      return numrs_hip_binary_backward(ctx, kind, g, x->data->ptr, y->data->ptr, nullptr, dx, N, 1);
    }
    if (x->requires_grad)
      if (int rc = grad_target(x, &dx, &ax)) return rc;
    if (y->requires_grad)
      if (int rc = grad_target(y, &dy, &ay)) return rc;
    if (dx && dy && ax != ay) {
      if (int rc = numrs_hip_binary_backward(ctx, kind, g, x->data->ptr, y->data->ptr, dx, nullptr,
                                             N, ax))
        return rc;
      return numrs_hip_binary_backward(ctx, kind, g, x->data->ptr, y->data->ptr, nullptr, dy, N, ay);
    }
    return numrs_hip_binary_backward(ctx, kind, g, x->data->ptr, y->data->ptr, dx, dy, N,
                                     dx ? ax : ay);
  }
  // Broadcasting operands: form the full-shape products with the forward
  // kernels, then unbroadcast (backward.rs:79-84, 95-106).
  const auto &os = out->shape;
  Buf t;
  if (int rc = temp(ctx, N, &t)) return rc;
  if (x->requires_grad) {
    // mul: g * y   div: g / y
    if (int rc = numrs_hip_binary_forward(ctx, kind, g, os.data(), (int)os.size(), y->data->ptr,
                                          y->shape.data(), (int)y->shape.size(), t->ptr))
      return rc;
    if (int rc = add_into(x, t->ptr, os)) return rc;
  }
  if (!y->requires_grad) return NUMRS_HIP_OK;
  if (kind == NUMRS_HIP_MUL) {  // g * x
    if (int rc = numrs_hip_binary_forward(ctx, NUMRS_HIP_MUL, g, os.data(), (int)os.size(),
                                          x->data->ptr, x->shape.data(), (int)x->shape.size(),
                                          t->ptr))
      return rc;
    return add_into(y, t->ptr, os);
  }
  // div: ((g * (x / (y*y))) * -1), backward.rs:99-104
  Buf ysq, term;
  const int64_t ny = y->numel();
  if (int rc = temp(ctx, ny, &ysq)) return rc;
  if (int rc = numrs_hip_binary_forward(ctx, NUMRS_HIP_MUL, y->data->ptr, y->shape.data(),
                                        (int)y->shape.size(), y->data->ptr, y->shape.data(),
                                        (int)y->shape.size(), ysq->ptr))
    return rc;
  if (int rc = temp(ctx, N, &term)) return rc;
  if (int rc = numrs_hip_binary_forward(ctx, NUMRS_HIP_DIV, x->data->ptr, x->shape.data(),
                                        (int)x->shape.size(), ysq->ptr, y->shape.data(),
                                        (int)y->shape.size(), term->ptr))
    return rc;
  if (int rc = numrs_hip_binary_forward(ctx, NUMRS_HIP_MUL, g, os.data(), (int)os.size(),
                                        term->ptr, os.data(), (int)os.size(), t->ptr))
    return rc;
  const int64_t one = 1;
  const float neg = -1.0f;
  Buf negb;
  if (int rc = temp(ctx, 1, &negb)) return rc;
  if (int rc = numrs_hip_fill(ctx, negb->ptr, 1, neg)) return rc;
  if (int rc = numrs_hip_binary_forward(ctx, NUMRS_HIP_MUL, t->ptr, os.data(), (int)os.size(),
                                        negb->ptr, &one, 1, term->ptr))
    return rc;
  return add_into(y, term->ptr, os);
}

int bw_matmul(const T &out, const float *g, Node &n) {
  const T &a = n.inputs[0], &b = n.inputs[1];
  numrs_hip_ctx *ctx = out->ctx;
  const int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
  float *da = nullptr, *db = nullptr;
  int aa = 0, ab = 0;
  if (a->requires_grad && b->requires_grad && a->grad == b->grad) {  // x @ x
    if (int rc = grad_target(a, &da, &aa)) return rc;
    if (int rc = numrs_hip_matmul_backward(ctx, g, a->data->ptr, b->data->ptr, da, nullptr, M, K,
                                           N, aa))
      return rc;
    return numrs_hip_matmul_backward(ctx, g, a->data->ptr, b->data->ptr, nullptr, da, M, K, N, 1);
  }
  // dA only when A requires grad (the reference computes and drops it, tensor.rs:206).
  if (a->requires_grad)
    if (int rc = grad_target(a, &da, &aa)) return rc;
  if (b->requires_grad)
    if (int rc = grad_target(b, &db, &ab)) return rc;
  if (da && db && aa != ab) {
    if (int rc = numrs_hip_matmul_backward(ctx, g, a->data->ptr, b->data->ptr, da, nullptr, M, K,
                                           N, aa))
      return rc;
    return numrs_hip_matmul_backward(ctx, g, a->data->ptr, b->data->ptr, nullptr, db, M, K, N, ab);
  }
  return numrs_hip_matmul_backward(ctx, g, a->data->ptr, b->data->ptr, da, db, M, K, N,
                                   da ? aa : ab);
}

int bw_transpose(const T &out, const float *g, Node &n) {  // backward.rs:305-312
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  numrs_hip_ctx *ctx = out->ctx;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  // out is [c, r]; its transpose is x's [r, c]
  const int64_t r = out->shape[0], c = out->shape[1];
  if (!acc) return numrs_hip_transpose(ctx, g, dst, r, c);
  Buf t;
  if (int rc = temp(ctx, x->numel(), &t)) return rc;
  if (int rc = numrs_hip_transpose(ctx, g, t->ptr, r, c)) return rc;
  return numrs_hip_binary_backward(ctx, NUMRS_HIP_ADD, t->ptr, nullptr, nullptr, dst, nullptr,
                                   x->numel(), 1);
}

int bw_unary(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  // sigmoid/tanh/exp/tan read the forward output (backward.rs:166-191,
  // 486-517); the others read the input.
  const bool uses_output = n.kind == NUMRS_HIP_SIGMOID || n.kind == NUMRS_HIP_TANH ||
                           n.kind == NUMRS_HIP_EXP || n.kind == NUMRS_HIP_TAN;
  const float *v = uses_output ? out->data->ptr : x->data->ptr;
  return numrs_hip_unary_backward(out->ctx, n.kind, g, v, dst, x->numel(), n.param, acc);
}

int bw_sum(const T &out, const float *g, Node &n) {  // backward.rs:208-236
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  return numrs_hip_fill_grad(out->ctx, g, dst, x->numel(), n.op == Op::Mean, acc);
}

// The sweep's root, when it is a scalar loss whose backward kernel writes
// the seed itself (see backward()); taken by that node's backward.
thread_local const Impl *g_seed_root = nullptr;

// The root's gradient cell when `out` is the root whose seed is still to be
// written (then the loss kernel writes it), else null.
float *take_seed(const T &out) {
  if (g_seed_root == nullptr || out.get() != g_seed_root) return nullptr;
  g_seed_root = nullptr;
  return out->grad->buf->ptr;
}

// A loss whose forward kernel pre-formed its root gradient (saved[slot]) and
// wrote the seed 1 into its own cell: when the loss is this sweep's root and
// the input's cell has never held a buffer, the cell takes the pre-formed
// buffer and no backward kernel runs.  Returns true when it did.
bool adopt_preformed(const T &out, Node &n, size_t slot, const T &x) {
  if (slot >= n.saved.size() || !n.saved[slot]) return false;
  if (g_seed_root != out.get() || !out->grad->seed_preset || x->grad->valid || x->grad->buf) {
    // Not adoptable now, and never later (the first sweep through the loss
    // makes the input's cell valid or leaves the loss a non-root): release
    // the buffer.  Stream order keeps it intact for work already queued.
    n.saved[slot].reset();
    return false;
  }
  g_seed_root = nullptr;  // the seed is already in the root's cell
  x->grad->buf = std::move(n.saved[slot]);
  x->grad->valid = true;
  return true;
}

int bw_mse(const T &out, const float *g, Node &n) {  // backward.rs:239-261
  const T &p = n.inputs[0], &t = n.inputs[1];
  if (p->requires_grad && !t->requires_grad && adopt_preformed(out, n, 0, p)) return NUMRS_HIP_OK;
  float *dp = nullptr, *dt = nullptr;
  int ap = 0, at = 0;
  if (p->requires_grad)
    if (int rc = grad_target(p, &dp, &ap)) return rc;
  if (t->requires_grad && !(p->requires_grad && p->grad == t->grad))
    if (int rc = grad_target(t, &dt, &at)) return rc;
  numrs_hip_ctx *ctx = out->ctx;
  float *seed = (dp || dt) ? take_seed(out) : nullptr;
  if (dp && dt && ap != at) {
    if (int rc = numrs_hip::mse_backward_impl(ctx, g, seed, p->data->ptr, t->data->ptr, dp,
                                              nullptr, p->numel(), ap))
      return rc;
    return numrs_hip_mse_backward(ctx, g, p->data->ptr, t->data->ptr, nullptr, dt, p->numel(),
                                  at);
  }
  return numrs_hip::mse_backward_impl(ctx, g, seed, p->data->ptr, t->data->ptr, dp, dt,
                                      p->numel(), dp ? ap : at);
}

int bw_ce(const T &out, const float *g, Node &n) {  // backward.rs:265-301
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;  // the target's grad is [0]: nothing to add
  if (adopt_preformed(out, n, n.op == Op::CrossEntropyLabels ? 1 : 0, x)) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  const int64_t B = x->shape[0], C = x->shape[1];
  float *seed = take_seed(out);
  if (n.op == Op::CrossEntropyLabels)
    return numrs_hip::softmax_ce_backward_impl(
        out->ctx, g, seed, x->data->ptr, nullptr,
        reinterpret_cast<const int32_t *>(n.saved[0]->ptr), dst, B, C, acc);
  return numrs_hip::softmax_ce_backward_impl(out->ctx, g, seed, x->data->ptr,
                                             n.inputs[1]->data->ptr, nullptr, dst, B, C, acc);
}

int bw_reshape(const T &out, const float *g, Node &n) {  // backward.rs:315-330
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  if (!acc) return numrs_hip_copy(out->ctx, dst, g, (size_t)x->numel() * sizeof(float));
  return numrs_hip_binary_backward(out->ctx, NUMRS_HIP_ADD, g, nullptr, nullptr, dst, nullptr,
                                   x->numel(), 1);
}

int bw_softmax(const T &out, const float *g, Node &n) {  // backward.rs:521-541
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  const int64_t cols = out->shape.back();
  return numrs_hip_softmax_backward(out->ctx, out->data->ptr, g, dst, out->numel() / cols, cols,
                                    acc);
}

// sum/mean over one axis: the incoming grad [outer, inner] broadcast back
// along the reduced axis (divided by n for the mean), backward.rs:208-236
// applied per reduced slice.
int bw_sum_axis(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  return numrs_hip_broadcast_axis(out->ctx, g, n.dims[0], n.dims[1], n.dims[2], n.kind, dst, acc);
}

int bw_softmax_axis(const T &out, const float *g, Node &n) {  // backward.rs:521-541
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  return numrs_hip_softmax_axis_backward(out->ctx, out->data->ptr, g, dst, n.dims[0], n.dims[1],
                                         n.dims[2], acc);
}

int bw_layernorm(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0], &gm = n.inputs[1], &bt = n.inputs[2];
  const int64_t cols = x->shape.back(), rows = x->numel() / cols;
  float *dx = nullptr, *dg = nullptr, *db = nullptr;
  int ax = 0, ag = 0, ab = 0;
  // One tensor as both gamma and beta: its two gradients add, in a second call.
  const bool shared_gb = gm->requires_grad && bt->requires_grad && gm->grad == bt->grad;
  if (x->requires_grad)
    if (int rc = grad_target(x, &dx, &ax)) return rc;
  if (gm->requires_grad)
    if (int rc = grad_target(gm, &dg, &ag)) return rc;
  if (bt->requires_grad && !shared_gb)
    if (int rc = grad_target(bt, &db, &ab)) return rc;
  if (int rc = numrs_hip_layernorm_backward(out->ctx, g, x->data->ptr, gm->data->ptr,
                                            n.saved[0]->ptr, n.saved[1]->ptr, dx, dg, db, rows,
                                            cols, ax, ag, ab))
    return rc;
  if (!shared_gb) return NUMRS_HIP_OK;
  if (int rc = grad_target(bt, &db, &ab)) return rc;
  return numrs_hip_layernorm_backward(out->ctx, g, x->data->ptr, gm->data->ptr, n.saved[0]->ptr,
                                      n.saved[1]->ptr, nullptr, nullptr, db, rows, cols, 0, 0, 1);
}

// Attention over one packed projection qkv [B*S, 3D]: its grad is written (or
// added) as the packed [B*S, 3D] block dq | dk | dv.
int bw_attention_packed(const T &out, const float *g, Node &n) {
  const T &qkv = n.inputs[0];
  if (!qkv->requires_grad) return NUMRS_HIP_OK;
  const int64_t D = out->shape[1];
  const float *p = qkv->data->ptr;
  float *d;
  int acc;
  if (int rc = grad_target(qkv, &d, &acc)) return rc;
  return numrs_hip_attention_backward_out_strided(out->ctx, p, p + D, p + 2 * D, 3 * D,
                                                  n.saved[0]->ptr, out->data->ptr, g, D, d, d + D,
                                                  d + 2 * D, n.dims[0], n.dims[1], n.dims[2], D,
                                                  acc);
}

int bw_attention(const T &out, const float *g, Node &n) {
  if (n.inputs.size() == 1) return bw_attention_packed(out, g, n);
  const T &q = n.inputs[0], &k = n.inputs[1], &v = n.inputs[2];
  float *dq = nullptr, *dk = nullptr, *dv = nullptr;
  int aq = 1, ak = 1, av = 1;
  if (q->requires_grad)
    if (int rc = grad_target(q, &dq, &aq)) return rc;
  if (k->requires_grad && k->grad != q->grad)
    if (int rc = grad_target(k, &dk, &ak)) return rc;
  if (v->requires_grad && v->grad != q->grad && v->grad != k->grad)
    if (int rc = grad_target(v, &dv, &av)) return rc;
  // One accumulate flag for the three grads: zero-fill any first-written one.
  const int acc = (dq && aq) || (dk && ak) || (dv && av);
  numrs_hip_ctx *ctx = out->ctx;
  if (acc) {
    if (dq && !aq) if (int rc = numrs_hip_fill(ctx, dq, q->numel(), 0.0f)) return rc;
    if (dk && !ak) if (int rc = numrs_hip_fill(ctx, dk, k->numel(), 0.0f)) return rc;
    if (dv && !av) if (int rc = numrs_hip_fill(ctx, dv, v->numel(), 0.0f)) return rc;
  }
  const int64_t D = q->shape[1];
  if (int rc = numrs_hip_attention_backward_out_strided(
          ctx, q->data->ptr, k->data->ptr, v->data->ptr, D, n.saved[0]->ptr, out->data->ptr, g, D,
          dq, dk, dv, n.dims[0], n.dims[1], n.dims[2], D, acc))
    return rc;
  // Shared grad cells (self-attention on one tensor): the remaining grads add.
  if (k->requires_grad && !dk) {
    float *t;
    int a;
    if (int rc = grad_target(k, &t, &a)) return rc;
    if (int rc = numrs_hip_attention_backward(ctx, q->data->ptr, k->data->ptr, v->data->ptr,
                                              n.saved[0]->ptr, g, nullptr, t, nullptr, n.dims[0],
                                              n.dims[1], n.dims[2], D, 1))
      return rc;
  }
  if (v->requires_grad && !dv) {
    float *t;
    int a;
    if (int rc = grad_target(v, &t, &a)) return rc;
    return numrs_hip_attention_backward(ctx, q->data->ptr, k->data->ptr, v->data->ptr,
                                        n.saved[0]->ptr, g, nullptr, nullptr, t, n.dims[0],
                                        n.dims[1], n.dims[2], D, 1);
  }
  return NUMRS_HIP_OK;
}

int bw_linear(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0], &W = n.inputs[1];
  const bool relu = (n.kind & 1) != 0, has_res = (n.kind & 2) != 0, gelu = (n.kind & 4) != 0;
  const size_t nb = n.inputs.size() - (has_res ? 1 : 0);
  const T *b = nb > 2 ? &n.inputs[2] : nullptr;
  // the residual's gradient is g (add_backward, backward.rs:43-54)
  if (has_res && n.inputs.back()->requires_grad)
    if (int rc = add_into(n.inputs.back(), g, out->shape)) return rc;
  const int64_t Tn = x->shape[0], in = x->shape[1], outf = W->shape[0];
  numrs_hip_ctx *ctx = out->ctx;
  float *dx = nullptr, *dW = nullptr, *db = nullptr;
  int ax = 0, aw = 0, ab = 0;
  const bool shared = x->requires_grad && W->requires_grad && x->grad == W->grad;
  if (x->requires_grad)
    if (int rc = grad_target(x, &dx, &ax)) return rc;
  if (W->requires_grad && !shared)
    if (int rc = grad_target(W, &dW, &aw)) return rc;
  if (b && (*b)->requires_grad)
    if (int rc = grad_target(*b, &db, &ab)) return rc;
  // The output went through ReLU: its saved value masks g.
  const float *y = out->data->ptr;
  auto run = [&](float *dx_, float *dW_, float *db_, int ax_, int aw_, int ab_) {
    if (gelu)
      return numrs_hip_linear_gelu_backward(ctx, g, n.saved[0]->ptr, x->data->ptr, W->data->ptr,
                                            dx_, dW_, db_, Tn, in, outf, ax_, aw_, ab_,
                                            ctx->unbroadcast_mode);
    if (relu)
      return numrs_hip_linear_relu_backward(ctx, g, y, x->data->ptr, W->data->ptr, dx_, dW_, db_,
                                            Tn, in, outf, ax_, aw_, ab_, ctx->unbroadcast_mode);
    return numrs_hip_linear_backward(ctx, g, x->data->ptr, W->data->ptr, dx_, dW_, db_, Tn, in,
                                     outf, ax_, aw_, ab_, ctx->unbroadcast_mode);
  };
  if (int rc = run(dx, dW, db, ax, aw, ab)) return rc;
  if (shared) {  // x is W: its second gradient adds
    float *t;
    int a;
    if (int rc = grad_target(W, &t, &a)) return rc;
    return run(nullptr, t, nullptr, 0, 1, 0);
  }
  return NUMRS_HIP_OK;
}

int bw_lstm(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0], &wih = n.inputs[1], &whh = n.inputs[2];
  const T *b = n.inputs.size() > 3 ? &n.inputs[3] : nullptr;
  const int64_t B = x->shape[0], Tn = x->shape[1], I = x->shape[2], H = whh->shape[1];
  float *dx = nullptr, *dwi = nullptr, *dwh = nullptr, *db = nullptr;
  int ax = 0, awi = 0, awh = 0, ab = 0;
  if (x->requires_grad)
    if (int rc = grad_target(x, &dx, &ax)) return rc;
  // One tensor as both W_ih and W_hh (I == H): its second gradient adds, in a
  // second call.
  const bool shared_w = wih->requires_grad && whh->requires_grad && whh->grad == wih->grad;
  if (wih->requires_grad)
    if (int rc = grad_target(wih, &dwi, &awi)) return rc;
  if (whh->requires_grad && !shared_w)
    if (int rc = grad_target(whh, &dwh, &awh)) return rc;
  if (b && (*b)->requires_grad)
    if (int rc = grad_target(*b, &db, &ab)) return rc;
  if (int rc = numrs_hip_lstm_backward(out->ctx, x->data->ptr, wih->data->ptr, whh->data->ptr,
                                       nullptr, nullptr, out->data->ptr, n.saved[1]->ptr,
                                       n.saved[0]->ptr, g, dx, dwi, dwh, db, B, Tn, I, H, ax, awi,
                                       awh, ab))
    return rc;
  if (!shared_w) return NUMRS_HIP_OK;
  if (int rc = grad_target(whh, &dwh, &awh)) return rc;
  return numrs_hip_lstm_backward(out->ctx, x->data->ptr, wih->data->ptr, whh->data->ptr, nullptr,
                                 nullptr, out->data->ptr, n.saved[1]->ptr, n.saved[0]->ptr, g,
                                 nullptr, nullptr, dwh, nullptr, B, Tn, I, H, 0, 0, 1, 0);
}

// Two stacked LSTM layers (inputs x, W_ih1, W_hh1, [b1], W_ih2, W_hh2, [b2];
// kind bit 0 / 1: b1 / b2 present; saved acts1, c1, h1, acts2, c2).  A
// parameter whose grad cell is shared with another input (one tensor used
// twice) gets its gradient in a temporary first, added in afterwards.
int bw_lstm2(const T &out, const float *g, Node &n) {
  const bool hb1 = (n.kind & 1) != 0, hb2 = (n.kind & 2) != 0;
  size_t k = 0;
  const T &x = n.inputs[k++];
  const T *ps[6] = {};  // W_ih1, W_hh1, b1, W_ih2, W_hh2, b2
  ps[0] = &n.inputs[k++];
  ps[1] = &n.inputs[k++];
  if (hb1) ps[2] = &n.inputs[k++];
  ps[3] = &n.inputs[k++];
  ps[4] = &n.inputs[k++];
  if (hb2) ps[5] = &n.inputs[k++];
  numrs_hip_ctx *ctx = out->ctx;
  const int64_t B = x->shape[0], Tn = x->shape[1], I = x->shape[2];
  const int64_t H1 = (*ps[1])->shape[1], H2 = (*ps[4])->shape[1];
  const T *all[7] = {&x, ps[0], ps[1], ps[2], ps[3], ps[4], ps[5]};
  float *dst[7] = {};
  int acc[7] = {};
  Buf tmp[7];
  for (int i = 0; i < 7; ++i) {
    if (all[i] == nullptr || !(*all[i])->requires_grad) continue;
    bool shared = false;
    for (int j = 0; j < 7; ++j)
      if (j != i && all[j] != nullptr && (*all[j])->requires_grad &&
          (*all[j])->grad == (*all[i])->grad)
        shared = true;
    if (shared) {
      if (int rc = temp(ctx, (*all[i])->numel(), &tmp[i])) return rc;
      dst[i] = tmp[i]->ptr;
    } else if (int rc = grad_target(*all[i], &dst[i], &acc[i])) {
      return rc;
    }
  }
  if (int rc = numrs_hip_lstm2_backward(
          ctx, x->data->ptr, (*ps[0])->data->ptr, (*ps[1])->data->ptr, (*ps[3])->data->ptr,
          (*ps[4])->data->ptr, n.saved[2]->ptr, n.saved[1]->ptr, n.saved[0]->ptr, out->data->ptr,
          n.saved[4]->ptr, n.saved[3]->ptr, g, dst[0], dst[1], dst[2], dst[3], dst[4], dst[5],
          dst[6], B, Tn, I, H1, H2, acc[0], acc[1], acc[2], acc[3], acc[4], acc[5], acc[6]))
    return rc;
  for (int i = 0; i < 7; ++i)
    if (tmp[i])
      if (int rc = add_into(*all[i], tmp[i]->ptr, (*all[i])->shape)) return rc;
  return NUMRS_HIP_OK;
}

int bw_time_slice(const T &out, const float *g, Node &n) {
  const T &x = n.inputs[0];
  if (!x->requires_grad) return NUMRS_HIP_OK;
  float *dst;
  int acc;
  if (int rc = grad_target(x, &dst, &acc)) return rc;
  return numrs_hip_time_slice(out->ctx, g, dst, x->shape[0], x->shape[1], x->shape[2], n.dims[0],
                              1, acc);
}

int run_backward_fn(const T &out) {
  Node &n = *out->node;
  const float *g = out->grad->buf->ptr;
  switch (n.op) {
    case Op::Add:
    case Op::Sub: return bw_add_sub(out, g, n);
    case Op::Mul:
    case Op::Div: return bw_mul_div(out, g, n);
    case Op::MatMul: return bw_matmul(out, g, n);
    case Op::Transpose: return bw_transpose(out, g, n);
    case Op::Unary: return bw_unary(out, g, n);
    case Op::Sum:
    case Op::Mean: return bw_sum(out, g, n);
    case Op::MSE: return bw_mse(out, g, n);
    case Op::CrossEntropy:
    case Op::CrossEntropyLabels: return bw_ce(out, g, n);
    case Op::Reshape: return bw_reshape(out, g, n);
    case Op::Softmax: return bw_softmax(out, g, n);
    case Op::LayerNorm: return bw_layernorm(out, g, n);
    case Op::Attention: return bw_attention(out, g, n);
    case Op::Linear: return bw_linear(out, g, n);
    case Op::LSTM: return bw_lstm(out, g, n);
    case Op::LSTM2: return bw_lstm2(out, g, n);
    case Op::TimeSlice: return bw_time_slice(out, g, n);
    case Op::SumAxis: return bw_sum_axis(out, g, n);
    case Op::SoftmaxAxis: return bw_softmax_axis(out, g, n);
    case Op::Leaf: return NUMRS_HIP_OK;
  }
  return NUMRS_HIP_OK;
}

// build_topo (tensor.rs:218-239) without recursion: post-order DFS over
// inputs in order, each non-leaf node visited once.  Leaves carry no
// backward body, so they are not listed.
std::vector<Impl *> build_topo(const T &root) {
  std::vector<Impl *> order;
  std::unordered_set<uint64_t> visited;
  std::vector<std::pair<Impl *, size_t>> stack;
  if (!root->node) return order;
  visited.insert(root->node->id);
  stack.emplace_back(root.get(), 0);
  while (!stack.empty()) {
    auto &[t, i] = stack.back();
    if (i < t->node->inputs.size()) {
      Impl *in = t->node->inputs[i].get();
      ++i;
      if (in->node && visited.insert(in->node->id).second) stack.emplace_back(in, 0);
      continue;
    }
    order.push_back(t);
    stack.pop_back();
  }
  return order;
}

int backward(const T &root) {  // tensor.rs:173-215
  numrs_hip_ctx *ctx = root->ctx;
  if (!root->requires_grad) return fail(ctx, NUMRS_HIP_E_INVALID, "Tensor does not require gradients");
  GradCell &rg = *root->grad;
  if (!rg.buf)
    if (int rc = alloc_buf(ctx, root->numel(), sizeof(float), &rg.buf)) return rc;
  // Seed ones (:178-183).  A scalar MSE or cross-entropy root has its seed
  // written by its own backward kernel, which takes g = 1 directly: one
  // launch fewer per step.  If that kernel does not run, the fill follows.
  const Op rop = root->node ? root->node->op : Op::Leaf;
  const bool seed_in_kernel = root->numel() == 1 && (rop == Op::MSE || rop == Op::CrossEntropy ||
                                                     rop == Op::CrossEntropyLabels);
  if (seed_in_kernel)
    g_seed_root = root.get();
  else if (int rc = numrs_hip_fill(ctx, rg.buf->ptr, root->numel(), 1.0f))
    return rc;
  rg.valid = true;
  std::vector<Impl *> topo = build_topo(root);
  int rc = NUMRS_HIP_OK;
  for (auto it = topo.rbegin(); it != topo.rend() && rc == NUMRS_HIP_OK; ++it) {
    Impl *t = *it;
    if (!t->grad || !t->grad->valid) continue;  // grad still zero: contributes nothing
    // Non-owning handle: the root keeps the whole graph alive during the sweep.
    T self(std::shared_ptr<Impl>{}, t);
    rc = run_backward_fn(self);
  }
  if (g_seed_root != nullptr) {  // the root's kernel did not take the seed
    g_seed_root = nullptr;
    if (rc == NUMRS_HIP_OK) rc = numrs_hip_fill(ctx, rg.buf->ptr, root->numel(), 1.0f);
  }
  return rc;
}

// ---------------------------------------------------------------------------
// Forward ops (autograd/ops.rs)
// ---------------------------------------------------------------------------

int op_binary(int kind, const T &a, const T &b, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  const size_t nd = std::max(a->shape.size(), b->shape.size());
  std::vector<int64_t> os(nd);
  for (size_t d = 0; d < nd; ++d) {
    const int da = (int)d - (int)(nd - a->shape.size()), db = (int)d - (int)(nd - b->shape.size());
    const int64_t ea = da >= 0 ? a->shape[da] : 1, eb = db >= 0 ? b->shape[db] : 1;
    if (ea != eb && ea != 1 && eb != 1)
      return fail(ctx, NUMRS_HIP_E_SHAPE, "shapes do not broadcast");
    os[d] = std::max(ea, eb);
  }
  const bool rec = recording({&a, &b});
  T r;
  if (int rc = make_tensor(ctx, os, rec, &r)) return rc;
  if (int rc = numrs_hip_binary_forward(ctx, kind, a->data->ptr, a->shape.data(),
                                        (int)a->shape.size(), b->data->ptr, b->shape.data(),
                                        (int)b->shape.size(), r->data->ptr))
    return rc;
  if (rec) {
    static const Op ops[4] = {Op::Add, Op::Sub, Op::Mul, Op::Div};
    attach(r, ops[kind], {a, b});
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_matmul(const T &a, const T &b, T *out) {  // ops.rs:101-119
  numrs_hip_ctx *ctx = a->ctx;
  if (a->shape.size() != 2 || b->shape.size() != 2 || a->shape[1] != b->shape[0])
    return fail(ctx, NUMRS_HIP_E_SHAPE, "matmul expects [M,K] @ [K,N]");
  const int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
  const bool rec = recording({&a, &b});
  T r;
  if (int rc = make_tensor(ctx, {M, N}, rec, &r)) return rc;
  if (int rc = numrs_hip_matmul(ctx, a->data->ptr, b->data->ptr, r->data->ptr, M, K, N, 0, 0, 0))
    return rc;
  if (rec) attach(r, Op::MatMul, {a, b});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_transpose(const T &a, T *out) {  // tensor.rs:242-259
  numrs_hip_ctx *ctx = a->ctx;
  if (a->shape.size() != 2) return fail(ctx, NUMRS_HIP_E_SHAPE, "transpose expects 2-D");
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, {a->shape[1], a->shape[0]}, rec, &r)) return rc;
  if (int rc = numrs_hip_transpose(ctx, a->data->ptr, r->data->ptr, a->shape[0], a->shape[1]))
    return rc;
  if (rec) attach(r, Op::Transpose, {a});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_unary(int kind, const T &a, float param, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, a->shape, rec, &r)) return rc;
  if (int rc = numrs_hip_unary_forward(ctx, kind, a->data->ptr, r->data->ptr, a->numel(), param))
    return rc;
  if (rec) attach(r, Op::Unary, {a}, kind, param);
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_sum(const T &a, bool mean, T *out) {  // ops.rs:214-252
  numrs_hip_ctx *ctx = a->ctx;
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, {1}, rec, &r)) return rc;
  if (int rc = numrs_hip_sum(ctx, a->data->ptr, a->numel(), mean ? 1 : 0, r->data->ptr)) return rc;
  if (rec) attach(r, mean ? Op::Mean : Op::Sum, {a});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// Largest loss input whose root gradient the forward kernel pre-forms.  The
// buffer is held by the loss node from the forward until a backward sweep
// adopts or drops it (or the loss dies), so a loss computed with grad
// recording but never differentiated (a validation loss) costs at most this
// much extra memory; above it the saved launch is worth little anyway.
constexpr int64_t kPreformMaxElems = int64_t(1) << 22;

// Buffers for a loss's pre-formed root gradient (n floats) and for its own
// gradient cell (the seed), when `want`; *pre stays null otherwise.
int preform_buffers(const T &r, bool want, int64_t n, Buf *pre) {
  if (!want || n > kPreformMaxElems) return NUMRS_HIP_OK;
  if (int rc = alloc_buf(r->ctx, n, sizeof(float), pre)) return rc;
  return alloc_buf(r->ctx, 1, sizeof(float), &r->grad->buf);
}

int op_mse(const T &p, const T &t, T *out) {  // ops.rs:255-278
  numrs_hip_ctx *ctx = p->ctx;
  if (p->numel() != t->numel()) return fail(ctx, NUMRS_HIP_E_SHAPE, "mse_loss: size mismatch");
  const bool rec = recording({&p, &t});
  T r;
  if (int rc = make_tensor(ctx, {1}, rec, &r)) return rc;
  // A loss that may be the backward's root forms that gradient (dp) and the
  // seed with its own kernel; bw_mse adopts them when it is the root.
  Buf pre;
  if (int rc = preform_buffers(r, rec && p->requires_grad && !t->requires_grad, p->numel(), &pre))
    return rc;
  if (int rc = numrs_hip::mse_loss_impl(ctx, p->data->ptr, t->data->ptr, p->numel(),
                                        r->data->ptr, pre ? pre->ptr : nullptr,
                                        pre ? r->grad->buf->ptr : nullptr))
    return rc;
  if (pre) r->grad->seed_preset = true;
  if (rec) attach(r, Op::MSE, {p, t}, 0, 0.f, {pre});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_ce(const T &x, const T &t, T *out) {  // ops.rs:281-334
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 2 || t->shape.size() != 2)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "CrossEntropy expect 2D tensors [batch, classes]");
  if (x->shape != t->shape) return fail(ctx, NUMRS_HIP_E_SHAPE, "CrossEntropy: shape mismatch");
  const bool rec = recording({&x, &t});
  T r;
  if (int rc = make_tensor(ctx, {1}, rec, &r)) return rc;
  Buf pre;
  if (int rc = preform_buffers(r, rec && x->requires_grad &&
                                      numrs_hip::cross_entropy_preforms(x->shape[0]),
                               x->numel(), &pre))
    return rc;
  if (int rc = numrs_hip::cross_entropy_loss_impl(
          ctx, x->data->ptr, t->data->ptr, nullptr, x->shape[0], x->shape[1], r->data->ptr,
          pre ? pre->ptr : nullptr, pre ? r->grad->buf->ptr : nullptr))
    return rc;
  if (pre) r->grad->seed_preset = true;
  if (rec) attach(r, Op::CrossEntropy, {x, t}, 0, 0.f, {pre});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_ce_labels(const T &x, const int32_t *host_labels, T *out) {
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 2) return fail(ctx, NUMRS_HIP_E_SHAPE, "CrossEntropy expects [batch, classes]");
  const int64_t B = x->shape[0], C = x->shape[1];
  for (int64_t i = 0; i < B; ++i)
    if (host_labels[i] < 0 || host_labels[i] >= C)
      return fail(ctx, NUMRS_HIP_E_INVALID, "label %d of row %lld outside [0,%lld)",
                  host_labels[i], (long long)i, (long long)C);
  Buf lab;
  if (int rc = alloc_buf(ctx, B, sizeof(int32_t), &lab)) return rc;
  if (int rc = numrs_hip_upload(ctx, lab->ptr, host_labels, (size_t)B * sizeof(int32_t))) return rc;
  const bool rec = recording({&x});
  T r;
  if (int rc = make_tensor(ctx, {1}, rec, &r)) return rc;
  Buf pre;
  if (int rc = preform_buffers(r, rec && x->requires_grad && numrs_hip::cross_entropy_preforms(B),
                               x->numel(), &pre))
    return rc;
  if (int rc = numrs_hip::cross_entropy_loss_impl(
          ctx, x->data->ptr, nullptr, reinterpret_cast<const int32_t *>(lab->ptr), B, C,
          r->data->ptr, pre ? pre->ptr : nullptr, pre ? r->grad->buf->ptr : nullptr))
    return rc;
  if (pre) r->grad->seed_preset = true;
  if (rec) attach(r, Op::CrossEntropyLabels, {x}, 0, 0.f, {lab, pre});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// Tensor::reshape (ops.rs:353-369) over ops::reshape's shape rules
// (ops/shape/reshape.rs:43-100): at most one -1, inferred from the element
// count; any other negative size, or a count that does not match, is an error.
int op_reshape(const T &a, std::vector<int64_t> shape, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  const int64_t total = a->numel();
  int64_t known = 1;
  int infer = -1;
  for (size_t i = 0; i < shape.size(); ++i) {
    const int64_t d = shape[i];
    if (d == -1) {
      if (infer >= 0)
        return fail(ctx, NUMRS_HIP_E_SHAPE, "Can only specify one unknown dimension with -1");
      infer = (int)i;
    } else if (d < 0) {
      return fail(ctx, NUMRS_HIP_E_SHAPE, "Invalid dimension size: %lld", (long long)d);
    } else {
      known *= d;
    }
  }
  if (infer >= 0) {
    if (known == 0)
      return fail(ctx, NUMRS_HIP_E_SHAPE, "Cannot infer dimension when other dimensions are zero");
    if (total % known != 0)
      return fail(ctx, NUMRS_HIP_E_SHAPE, "Cannot reshape array of size %lld", (long long)total);
    shape[infer] = total / known;
  } else if (known != total) {
    return fail(ctx, NUMRS_HIP_E_SHAPE, "Cannot reshape array of size %lld", (long long)total);
  }
  const int64_t n = total;
  const bool rec = recording({&a});
  // ops::reshape returns a new Array (ops.rs:356): the result owns a copy, so
  // an in-place optimizer update of the source leaves it unchanged.
  T r;
  if (int rc = make_tensor(ctx, std::move(shape), rec, &r)) return rc;
  if (int rc = numrs_hip_copy(ctx, r->data->ptr, a->data->ptr, (size_t)n * sizeof(float)))
    return rc;
  if (rec) attach(r, Op::Reshape, {a});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_softmax(const T &a, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  if (a->shape.empty()) return fail(ctx, NUMRS_HIP_E_SHAPE, "softmax of a scalar");
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, a->shape, rec, &r)) return rc;
  const int64_t cols = a->shape.back();
  if (int rc = numrs_hip_softmax_forward(ctx, a->data->ptr, r->data->ptr, a->numel() / cols, cols,
                                         1.0f))
    return rc;
  if (rec) attach(r, Op::Softmax, {a});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// x viewed as [outer, n, inner] around `axis`.
int axis_view(const T &a, int64_t axis, int64_t v[3]) {
  const int64_t nd = (int64_t)a->shape.size();
  if (axis < 0 || axis >= nd)
    return fail(a->ctx, NUMRS_HIP_E_SHAPE, "axis %lld out of range for %lld dimensions",
                (long long)axis, (long long)nd);
  v[0] = v[2] = 1;
  for (int64_t d = 0; d < axis; ++d) v[0] *= a->shape[d];
  v[1] = a->shape[axis];
  for (int64_t d = axis + 1; d < nd; ++d) v[2] *= a->shape[d];
  return NUMRS_HIP_OK;
}

// ops::sum / ops::mean with Some(axis): the axis is removed from the shape,
// a 1-D input gives shape [1] (backend/cpu/scalar.rs:584-597).
int op_sum_axis(const T &a, int64_t axis, bool mean, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  int64_t v[3];
  if (int rc = axis_view(a, axis, v)) return rc;
  std::vector<int64_t> shape;
  for (size_t d = 0; d < a->shape.size(); ++d)
    if ((int64_t)d != axis) shape.push_back(a->shape[d]);
  if (shape.empty()) shape.push_back(1);
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, shape, rec, &r)) return rc;
  if (int rc = numrs_hip_reduce_axis(ctx, a->data->ptr, v[0], v[1], v[2], mean ? 1 : 0,
                                     r->data->ptr))
    return rc;
  if (rec) {
    attach(r, Op::SumAxis, {a}, mean ? 1 : 0);
    std::copy(v, v + 3, r->node->dims);
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_softmax_axis(const T &a, int64_t axis, T *out) {
  numrs_hip_ctx *ctx = a->ctx;
  int64_t v[3];
  if (int rc = axis_view(a, axis, v)) return rc;
  const bool rec = recording({&a});
  T r;
  if (int rc = make_tensor(ctx, a->shape, rec, &r)) return rc;
  if (int rc = numrs_hip_softmax_axis_forward(ctx, a->data->ptr, r->data->ptr, v[0], v[1], v[2]))
    return rc;
  if (rec) {
    attach(r, Op::SoftmaxAxis, {a});
    std::copy(v, v + 3, r->node->dims);
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_layernorm(const T &x, const T &gamma, const T &beta, float eps, T *out) {
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.empty()) return fail(ctx, NUMRS_HIP_E_SHAPE, "layer_norm of a scalar");
  const int64_t cols = x->shape.back(), rows = x->numel() / cols;
  if (gamma->numel() != cols || beta->numel() != cols)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "layer_norm: gamma/beta must have the last-axis length");
  const bool rec = recording({&x, &gamma, &beta});
  T r;
  if (int rc = make_tensor(ctx, x->shape, rec, &r)) return rc;
  Buf mean, rstd;
  if (int rc = alloc_buf(ctx, rows, sizeof(float), &mean)) return rc;
  if (int rc = alloc_buf(ctx, rows, sizeof(float), &rstd)) return rc;
  if (int rc = numrs_hip_layernorm_forward(ctx, x->data->ptr, gamma->data->ptr, beta->data->ptr,
                                           r->data->ptr, mean->ptr, rstd->ptr, rows, cols, eps))
    return rc;
  if (rec) attach(r, Op::LayerNorm, {x, gamma, beta}, 0, eps, {mean, rstd});
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// act 1: y = ReLU(x W^T + b) as one node (the Linear -> ReLU pair of a
// Sequential), whose backward masks g by y > 0 before the Linear backward.
// act 2: y = GELU(x W^T + b) as one node, the pre-activation saved by the
// product's epilogue for GELU's backward.
// res: y = res + (x W^T + b) as one node (a residual block's "x + Linear(a)"),
// the residual added in the product's epilogue; its gradient is g itself.
// Node kind: bit 0 ReLU, bit 1 residual (the last input), bit 2 GELU.
int op_linear(const T &x, const T &W, const T *b, T *out, int act = 0, const T *res = nullptr) {
  const int relu = act == 1;
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 2 || W->shape.size() != 2 || x->shape[1] != W->shape[1])
    return fail(ctx, NUMRS_HIP_E_SHAPE, "linear expects x [T,in], W [out,in]");
  if (b && ((*b)->numel() != W->shape[0]))
    return fail(ctx, NUMRS_HIP_E_SHAPE, "linear: bias must have out elements");
  if (res && ((*res)->shape != std::vector<int64_t>{x->shape[0], W->shape[0]} || act))
    return fail(ctx, NUMRS_HIP_E_SHAPE, "linear: residual must be [T, out] (and no activation)");
  std::vector<const T *> all{&x, &W};
  if (b) all.push_back(b);
  if (res) all.push_back(res);
  bool rec = false;
  for (const T *t : all) rec = rec || ((*t)->requires_grad && g_grad_enabled);
  T r;
  if (int rc = make_tensor(ctx, {x->shape[0], W->shape[0]}, rec, &r)) return rc;
  const float *bp = b ? (*b)->data->ptr : nullptr;
  int rc = 0;
  Buf pre;
  if (act == 2) {
    if ((rc = alloc_buf(ctx, x->shape[0] * W->shape[0], sizeof(float), &pre))) return rc;
    rc = numrs_hip_linear_gelu_forward(ctx, x->data->ptr, W->data->ptr, bp, r->data->ptr,
                                       pre->ptr, x->shape[0], x->shape[1], W->shape[0]);
  } else if (res)
    rc = numrs_hip_linear_residual_forward(ctx, x->data->ptr, W->data->ptr, bp, (*res)->data->ptr,
                                           r->data->ptr, x->shape[0], x->shape[1], W->shape[0]);
  else
    rc = (relu ? numrs_hip_linear_relu_forward : numrs_hip_linear_forward)(
        ctx, x->data->ptr, W->data->ptr, bp, r->data->ptr, x->shape[0], x->shape[1], W->shape[0]);
  if (rc) return rc;
  if (rec) {
    std::vector<T> ins{x, W};
    if (b) ins.push_back(*b);
    if (res) ins.push_back(*res);
    if (act == 2)
      attach(r, Op::Linear, std::move(ins), 4, 0.f, {pre});
    else
      attach(r, Op::Linear, std::move(ins), (relu ? 1 : 0) | (res ? 2 : 0));
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_lstm(const T &x, const T &wih, const T &whh, const T *b, T *out) {
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 3 || wih->shape.size() != 2 || whh->shape.size() != 2)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "lstm expects x [B,T,I], W_ih [4H,I], W_hh [4H,H]");
  const int64_t B = x->shape[0], Tn = x->shape[1], I = x->shape[2], H = whh->shape[1];
  if (wih->shape[0] != 4 * H || wih->shape[1] != I || whh->shape[0] != 4 * H ||
      (b && (*b)->numel() != 4 * H))
    return fail(ctx, NUMRS_HIP_E_SHAPE, "lstm: weight shapes do not match H = %lld", (long long)H);
  const bool rec = b ? recording({&x, &wih, &whh, b}) : recording({&x, &wih, &whh});
  T r;
  if (int rc = make_tensor(ctx, {B, Tn, H}, rec, &r)) return rc;
  Buf acts, cseq;
  if (int rc = alloc_buf(ctx, B * Tn * 4 * H, sizeof(float), &acts)) return rc;
  if (int rc = alloc_buf(ctx, B * Tn * H, sizeof(float), &cseq)) return rc;
  if (int rc = numrs_hip_lstm_forward(ctx, x->data->ptr, wih->data->ptr, whh->data->ptr,
                                      b ? (*b)->data->ptr : nullptr, nullptr, nullptr,
                                      r->data->ptr, cseq->ptr, acts->ptr, B, Tn, I, H))
    return rc;
  if (rec) {
    std::vector<T> ins{x, wih, whh};
    if (b) ins.push_back(*b);
    attach(r, Op::LSTM, std::move(ins), 0, 0.f, {acts, cseq});
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_lstm2(const T &x, const T &wih1, const T &whh1, const T *b1, const T &wih2,
             const T &whh2, const T *b2, T *out) {
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 3 || wih1->shape.size() != 2 || whh1->shape.size() != 2 ||
      wih2->shape.size() != 2 || whh2->shape.size() != 2)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "lstm2 expects x [B,T,I] and 2-D weights");
  const int64_t B = x->shape[0], Tn = x->shape[1], I = x->shape[2];
  const int64_t H1 = whh1->shape[1], H2 = whh2->shape[1];
  if (wih1->shape != std::vector<int64_t>{4 * H1, I} ||
      whh1->shape != std::vector<int64_t>{4 * H1, H1} ||
      wih2->shape != std::vector<int64_t>{4 * H2, H1} ||
      whh2->shape != std::vector<int64_t>{4 * H2, H2} || (b1 && (*b1)->numel() != 4 * H1) ||
      (b2 && (*b2)->numel() != 4 * H2))
    return fail(ctx, NUMRS_HIP_E_SHAPE, "lstm2: weight shapes do not match H1 = %lld, H2 = %lld",
                (long long)H1, (long long)H2);
  const T *all[7] = {&x, &wih1, &whh1, b1, &wih2, &whh2, b2};
  bool rec = false;
  for (const T *t : all) rec = rec || (t != nullptr && (*t)->requires_grad && g_grad_enabled);
  T r;
  if (int rc = make_tensor(ctx, {B, Tn, H2}, rec, &r)) return rc;
  Buf acts1, c1, h1, acts2, c2;
  if (int rc = alloc_buf(ctx, B * Tn * 4 * H1, sizeof(float), &acts1)) return rc;
  if (int rc = alloc_buf(ctx, B * Tn * H1, sizeof(float), &c1)) return rc;
  if (int rc = alloc_buf(ctx, B * Tn * H1, sizeof(float), &h1)) return rc;
  if (int rc = alloc_buf(ctx, B * Tn * 4 * H2, sizeof(float), &acts2)) return rc;
  if (int rc = alloc_buf(ctx, B * Tn * H2, sizeof(float), &c2)) return rc;
  if (int rc = numrs_hip_lstm2_forward(
          ctx, x->data->ptr, wih1->data->ptr, whh1->data->ptr, b1 ? (*b1)->data->ptr : nullptr,
          wih2->data->ptr, whh2->data->ptr, b2 ? (*b2)->data->ptr : nullptr, h1->ptr, c1->ptr,
          acts1->ptr, r->data->ptr, c2->ptr, acts2->ptr, B, Tn, I, H1, H2))
    return rc;
  if (rec) {
    std::vector<T> ins{x, wih1, whh1};
    if (b1) ins.push_back(*b1);
    ins.push_back(wih2);
    ins.push_back(whh2);
    if (b2) ins.push_back(*b2);
    attach(r, Op::LSTM2, std::move(ins), (b1 ? 1 : 0) | (b2 ? 2 : 0), 0.f,
           {acts1, c1, h1, acts2, c2});
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_time_slice(const T &x, int64_t t, T *out) {
  numrs_hip_ctx *ctx = x->ctx;
  if (x->shape.size() != 3 || t < 0 || t >= x->shape[1])
    return fail(ctx, NUMRS_HIP_E_SHAPE, "time_slice expects [B,T,D] and 0 <= t < T");
  const bool rec = recording({&x});
  T r;
  if (int rc = make_tensor(ctx, {x->shape[0], x->shape[2]}, rec, &r)) return rc;
  if (int rc = numrs_hip_time_slice(ctx, x->data->ptr, r->data->ptr, x->shape[0], x->shape[1],
                                    x->shape[2], t, 0, 0))
    return rc;
  if (rec) {
    attach(r, Op::TimeSlice, {x});
    r->node->dims[0] = t;
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

int op_attention(const T &q, const T &k, const T &v, int64_t B, int64_t S, int64_t H, T *out) {
  numrs_hip_ctx *ctx = q->ctx;
  if (q->shape.size() != 2 || q->shape != k->shape || q->shape != v->shape)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "attention: q, k, v must be equal [batch*seq, dim]");
  if (B <= 0 || S <= 0 || H <= 0 || q->shape[0] != B * S || q->shape[1] % H != 0)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "attention: rows != batch*seq or dim %% heads != 0");
  const bool rec = recording({&q, &k, &v});
  T r;
  if (int rc = make_tensor(ctx, q->shape, rec, &r)) return rc;
  Buf P;
  if (int rc = alloc_buf(ctx, B * H * S * S, sizeof(float), &P)) return rc;
  if (int rc = numrs_hip_attention_forward(ctx, q->data->ptr, k->data->ptr, v->data->ptr, P->ptr,
                                           r->data->ptr, B, S, H, q->shape[1]))
    return rc;
  if (rec) {
    attach(r, Op::Attention, {q, k, v}, 0, 0.f, {P});
    r->node->dims[0] = B;
    r->node->dims[1] = S;
    r->node->dims[2] = H;
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// Attention over a packed projection qkv [B*S, 3D]: q, k, v are its column
// blocks (row stride 3D), the output is [B*S, D].
int op_attention_qkv(const T &qkv, int64_t B, int64_t S, int64_t H, T *out) {
  numrs_hip_ctx *ctx = qkv->ctx;
  if (qkv->shape.size() != 2 || qkv->shape[1] % 3 != 0)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "attention_qkv: qkv must be [batch*seq, 3*dim]");
  const int64_t D = qkv->shape[1] / 3;
  if (B <= 0 || S <= 0 || H <= 0 || qkv->shape[0] != B * S || D % H != 0)
    return fail(ctx, NUMRS_HIP_E_SHAPE, "attention_qkv: rows != batch*seq or dim %% heads != 0");
  const bool rec = recording({&qkv});
  T r;
  if (int rc = make_tensor(ctx, {B * S, D}, rec, &r)) return rc;
  Buf P;
  if (int rc = alloc_buf(ctx, B * H * S * S, sizeof(float), &P)) return rc;
  const float *p = qkv->data->ptr;
  if (int rc = numrs_hip_attention_forward_strided(ctx, p, p + D, p + 2 * D, 3 * D, P->ptr,
                                                   r->data->ptr, D, B, S, H, D))
    return rc;
  if (rec) {
    attach(r, Op::Attention, {qkv}, 0, 0.f, {P});
    r->node->dims[0] = B;
    r->node->dims[1] = S;
    r->node->dims[2] = H;
  }
  *out = std::move(r);
  return NUMRS_HIP_OK;
}

// ---------------------------------------------------------------------------
// Optimizers (optim/base.rs, sgd.rs, adam.rs)
// ---------------------------------------------------------------------------

// An engine optimizer: SGD / Adam (their own kernels), one of the
// NUMRS_HIP_OPT_* kinds (numrs_hip_optimizer_step), a Lookahead around an
// inner optimizer, or L-BFGS over the flattened parameters.
enum class Family { SGD, Adam, Kind, Lookahead, LBFGS };

struct Optim {
  numrs_hip_ctx *ctx = nullptr;
  Family fam = Family::SGD;
  bool adam = false;
  std::vector<T> params;
  std::vector<Buf> s1, s2;  // SGD velocity | Adam m, v | the kind's state slots
  float lr = 0.f, mu = 0.f, wd = 0.f, b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  int t = 0;
  // NUMRS_HIP_OPT_* kinds
  int kind = -1;
  float hyper[8] = {};
  int nhyper = 0;
  // Lookahead (lookahead.rs:28-47)
  numrs_hip_optim *inner = nullptr;
  std::vector<Buf> slow;
  int la_k = 0, la_counter = 0;
  float la_alpha = 0.f;
  // L-BFGS (lbfgs.rs:20-36): history of (s, y) over the flattened parameters
  int history = 0, max_iter = 0;
  int64_t total = 0;
  std::vector<Buf> s_hist, y_hist;
  Buf cur_p, cur_g, prev_p, prev_g, work_q, work_r, scalar;
  bool has_prev = false;
  ~Optim();
};

}  // namespace

struct numrs_hip_tensor {
  T t;
};
struct numrs_hip_optim {
  Optim o;
};

namespace {
Optim::~Optim() {
  if (inner != nullptr) delete inner;
}
}  // namespace

namespace {

int wrap(T t, numrs_hip_tensor **out) {
  *out = new numrs_hip_tensor{std::move(t)};
  return NUMRS_HIP_OK;
}

int check2(const numrs_hip_tensor *a, const numrs_hip_tensor *b, numrs_hip_tensor **out) {
  if (a == nullptr || b == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  if (a->t->ctx != b->t->ctx)
    return fail(a->t->ctx, NUMRS_HIP_E_INVALID, "tensors belong to different contexts");
  *out = nullptr;
  return NUMRS_HIP_OK;
}

int new_optim(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, bool adam, Optim *o) {
  o->ctx = ctx;
  o->adam = adam;
  for (int i = 0; i < n; ++i) {
    if (params[i] == nullptr) return fail(ctx, NUMRS_HIP_E_INVALID, "null parameter %d", i);
    const T &p = params[i]->t;
    o->params.push_back(p);
    Buf a, b;
    // Velocities / moments start at zero (sgd.rs:53-60, adam.rs:72-86).
    if (int rc = alloc_buf(ctx, p->numel(), sizeof(float), &a)) return rc;
    if (int rc = numrs_hip_fill(ctx, a->ptr, p->numel(), 0.0f)) return rc;
    if (adam) {
      if (int rc = alloc_buf(ctx, p->numel(), sizeof(float), &b)) return rc;
      if (int rc = numrs_hip_fill(ctx, b->ptr, p->numel(), 0.0f)) return rc;
    }
    o->s1.push_back(a);
    o->s2.push_back(b);
  }
  return NUMRS_HIP_OK;
}

}  // namespace

namespace {

int kind_hyper_count(int kind) {
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

// The Adam-family kinds advance a step counter at the top of step().
bool kind_uses_t(int kind) {
  return kind == NUMRS_HIP_OPT_ADAMW || kind == NUMRS_HIP_OPT_NADAM ||
         kind == NUMRS_HIP_OPT_RADAM || kind == NUMRS_HIP_OPT_ADABOUND ||
         kind == NUMRS_HIP_OPT_LAMB;
}

// Downloads a device scalar (synchronises the stream).
int read_scalar(numrs_hip_ctx *ctx, const float *dev, float *host) {
  return numrs_hip_download(ctx, host, dev, sizeof(float));
}

// Rprop::learning_rate: the mean step size over every parameter.
float rprop_mean_step(const Optim &o) {
  float total = 0.0f;
  int64_t count = 0;
  for (size_t i = 0; i < o.s1.size(); ++i) {
    if (!o.s1[i]) continue;
    const int64_t n = o.params[i]->numel();
    if (n == 0) continue;
    float *dev = nullptr;
    if (numrs_hip::scratch(o.ctx, sizeof(float), &dev)) return NAN;
    if (numrs_hip_sum(o.ctx, o.s1[i]->ptr, n, 0, dev)) return NAN;
    float part = 0.0f;
    if (read_scalar(o.ctx, dev, &part)) return NAN;
    total = total + part;
    count += n;
  }
  return total / (float)count;
}

// Lookahead::step, lookahead.rs:88-120.
int lookahead_step(Optim &o) {
  if (int rc = numrs_hip_optim_step(o.inner)) return rc;
  o.la_counter += 1;
  if (o.la_counter < o.la_k) return NUMRS_HIP_OK;
  o.la_counter = 0;
  std::vector<float *> fast, slow;
  std::vector<int64_t> ns;
  for (size_t i = 0; i < o.params.size(); ++i) {
    fast.push_back(o.params[i]->data->ptr);
    slow.push_back(o.slow[i]->ptr);
    ns.push_back(o.params[i]->numel());
  }
  return numrs_hip_lookahead_update(o.ctx, fast.data(), slow.data(), ns.data(), (int)ns.size(),
                                    o.la_alpha);
}

// Flattens the parameters (and their gradients, zeros when absent) into
// dst, lbfgs.rs:80-106.
int flatten(Optim &o, float *dst, bool grads) {
  int64_t off = 0;
  for (const T &p : o.params) {
    const int64_t n = p->numel();
    if (n > 0) {
      if (!grads) {
        if (int rc = numrs_hip_copy(o.ctx, dst + off, p->data->ptr, (size_t)n * sizeof(float)))
          return rc;
      } else if (p->grad && p->grad->valid) {
        if (int rc = numrs_hip_copy(o.ctx, dst + off, p->grad->buf->ptr, (size_t)n * sizeof(float)))
          return rc;
      } else {
        if (int rc = numrs_hip_fill(o.ctx, dst + off, n, 0.0f)) return rc;
      }
    }
    off += n;
  }
  return NUMRS_HIP_OK;
}

int dot_host(Optim &o, const float *x, const float *y, float *out) {
  if (int rc = numrs_hip_dot(o.ctx, x, y, o.total, o.scalar->ptr)) return rc;
  return read_scalar(o.ctx, o.scalar->ptr, out);
}

// LBFGS::step, lbfgs.rs:157-212, with the two-loop recursion of :114-154;
// vectors stay on the device, the recursion's scalars are f32 host values.
int lbfgs_step(Optim &o) {
  using namespace numrs_hip;
  const int64_t n = o.total;
  if (int rc = flatten(o, o.cur_p->ptr, false)) return rc;
  if (int rc = flatten(o, o.cur_g->ptr, true)) return rc;
  if (o.has_prev) {
    Buf sb, yb;
    if (int rc = alloc_buf(o.ctx, n, sizeof(float), &sb)) return rc;
    if (int rc = alloc_buf(o.ctx, n, sizeof(float), &yb)) return rc;
    if (int rc = vec_op(o.ctx, sb->ptr, o.cur_p->ptr, o.prev_p->ptr, 0.f, n, kVecSub)) return rc;
    if (int rc = vec_op(o.ctx, yb->ptr, o.cur_g->ptr, o.prev_g->ptr, 0.f, n, kVecSub)) return rc;
    float sy = 0.f;
    if (int rc = dot_host(o, sb->ptr, yb->ptr, &sy)) return rc;
    if (sy > 1e-10f) {
      o.s_hist.push_back(sb);
      o.y_hist.push_back(yb);
      if ((int)o.s_hist.size() > o.history) {
        o.s_hist.erase(o.s_hist.begin());
        o.y_hist.erase(o.y_hist.begin());
      }
    }
  }
  // direction d = -H g, written into work_r
  float *q = o.work_q->ptr, *r = o.work_r->ptr;
  const int m = (int)o.s_hist.size();
  if (m == 0) {
    if (int rc = vec_op(o.ctx, r, o.cur_g->ptr, nullptr, 0.f, n, kVecNeg)) return rc;
  } else {
    if (int rc = numrs_hip_copy(o.ctx, q, o.cur_g->ptr, (size_t)n * sizeof(float))) return rc;
    std::vector<float> alpha(m), rho(m);
    for (int i = m - 1; i >= 0; --i) {
      float ys = 0.f, sq = 0.f;
      if (int rc = dot_host(o, o.y_hist[i]->ptr, o.s_hist[i]->ptr, &ys)) return rc;
      rho[i] = 1.0f / fmaxf(ys, 1e-10f);
      if (int rc = dot_host(o, o.s_hist[i]->ptr, q, &sq)) return rc;
      alpha[i] = rho[i] * sq;
      if (int rc = vec_op(o.ctx, q, q, o.y_hist[i]->ptr, alpha[i], n, kVecAxmy)) return rc;
    }
    float sy = 0.f, yy = 0.f;
    if (int rc = dot_host(o, o.s_hist[m - 1]->ptr, o.y_hist[m - 1]->ptr, &sy)) return rc;
    if (int rc = dot_host(o, o.y_hist[m - 1]->ptr, o.y_hist[m - 1]->ptr, &yy)) return rc;
    const float gamma = sy / fmaxf(yy, 1e-10f);
    if (int rc = vec_op(o.ctx, r, q, nullptr, gamma, n, kVecScale)) return rc;
    for (int i = 0; i < m; ++i) {
      float yr = 0.f;
      if (int rc = dot_host(o, o.y_hist[i]->ptr, r, &yr)) return rc;
      const float beta = rho[i] * yr;
      if (int rc = vec_op(o.ctx, r, r, o.s_hist[i]->ptr, alpha[i] - beta, n, kVecAypx))
        return rc;
    }
    if (int rc = vec_op(o.ctx, r, r, nullptr, 0.f, n, kVecNeg)) return rc;
  }
  // p += lr * d, per parameter (lbfgs.rs:187-197)
  int64_t off = 0;
  for (const T &p : o.params) {
    const int64_t k = p->numel();
    if (int rc = vec_op(o.ctx, p->data->ptr, p->data->ptr, r + off, o.lr, k, kVecAxpy)) return rc;
    off += k;
  }
  // keep this step's flattened state (lbfgs.rs:199-201)
  if (!o.has_prev) {
    if (int rc = alloc_buf(o.ctx, n > 0 ? n : 1, sizeof(float), &o.prev_p)) return rc;
    if (int rc = alloc_buf(o.ctx, n > 0 ? n : 1, sizeof(float), &o.prev_g)) return rc;
  }
  std::swap(o.prev_p, o.cur_p);
  std::swap(o.prev_g, o.cur_g);
  if (!o.cur_p) {
    if (int rc = alloc_buf(o.ctx, n > 0 ? n : 1, sizeof(float), &o.cur_p)) return rc;
    if (int rc = alloc_buf(o.ctx, n > 0 ? n : 1, sizeof(float), &o.cur_g)) return rc;
  }
  o.has_prev = true;
  return NUMRS_HIP_OK;
}

}  // namespace

extern "C" {

void numrs_hip_set_grad_enabled(int enabled) { g_grad_enabled = enabled != 0; }
int numrs_hip_is_grad_enabled(void) { return g_grad_enabled ? 1 : 0; }

int numrs_hip_set_unbroadcast_mode(numrs_hip_ctx *ctx, int mode) {
  NRS_CHECK_CTX(ctx);
  if (mode != NUMRS_HIP_UNBROADCAST_CORRECT && mode != NUMRS_HIP_UNBROADCAST_REFERENCE)
    return fail(ctx, NUMRS_HIP_E_INVALID, "unbroadcast mode %d", mode);
  ctx->unbroadcast_mode = mode;
  return NUMRS_HIP_OK;
}

int numrs_hip_tensor_new(numrs_hip_ctx *ctx, const float *host, const int64_t *shape, int ndim,
                         int requires_grad, numrs_hip_tensor **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr || ndim < 0 || ndim > 8 || (ndim > 0 && shape == nullptr))
    return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_tensor_new: bad arguments");
  std::vector<int64_t> s(shape, shape + ndim);
  for (int64_t d : s)
    if (d < 0) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_tensor_new: negative dimension");
  T t;
  if (int rc = make_tensor(ctx, s, requires_grad != 0, &t)) return rc;
  if (t->numel() > 0) {
    if (host == nullptr) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_tensor_new: null data");
    if (int rc = numrs_hip_upload(ctx, t->data->ptr, host, (size_t)t->numel() * sizeof(float)))
      return rc;
  }
  return wrap(std::move(t), out);
}

int numrs_hip_tensor_free(numrs_hip_tensor *t) {
  delete t;
  return NUMRS_HIP_OK;
}

int numrs_hip_tensor_shape(const numrs_hip_tensor *t, int64_t *shape, int cap) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  const int nd = (int)t->t->shape.size();
  for (int i = 0; i < nd && i < cap && shape; ++i) shape[i] = t->t->shape[i];
  return nd;
}

int64_t numrs_hip_tensor_numel(const numrs_hip_tensor *t) {
  return t == nullptr ? NUMRS_HIP_E_INVALID : t->t->numel();
}

int numrs_hip_tensor_requires_grad(const numrs_hip_tensor *t) {
  return t == nullptr ? NUMRS_HIP_E_INVALID : (t->t->requires_grad ? 1 : 0);
}

int numrs_hip_tensor_is_leaf(const numrs_hip_tensor *t) {
  return t == nullptr ? NUMRS_HIP_E_INVALID : (t->t->is_leaf ? 1 : 0);
}

int numrs_hip_tensor_values(numrs_hip_tensor *t, float *host, int64_t n) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  if (n != t->t->numel()) return fail(t->t->ctx, NUMRS_HIP_E_SHAPE, "values: buffer of %lld for %lld elements", (long long)n, (long long)t->t->numel());
  return numrs_hip_download(t->t->ctx, host, t->t->data->ptr, (size_t)n * sizeof(float));
}

int numrs_hip_tensor_gradient(numrs_hip_tensor *t, float *host, int64_t n) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  const T &x = t->t;
  if (!x->grad) return 0;  // Option::None (tensor.rs:96-98)
  if (n != x->numel()) return fail(x->ctx, NUMRS_HIP_E_SHAPE, "gradient: buffer size mismatch");
  if (int rc = grad_materialise(x)) return rc;
  if (int rc = numrs_hip_download(x->ctx, host, x->grad->buf->ptr, (size_t)n * sizeof(float)))
    return rc;
  return 1;
}

int numrs_hip_tensor_set_gradient(numrs_hip_tensor *t, const float *host, int64_t n) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  const T &x = t->t;
  if (!x->grad) return fail(x->ctx, NUMRS_HIP_E_INVALID, "Tensor does not require gradients");
  if (n != x->numel()) return fail(x->ctx, NUMRS_HIP_E_SHAPE, "set_gradient: size mismatch");
  if (!x->grad->buf)
    if (int rc = alloc_buf(x->ctx, n, sizeof(float), &x->grad->buf)) return rc;
  x->grad->seed_preset = false;
  if (int rc = numrs_hip_upload(x->ctx, x->grad->buf->ptr, host, (size_t)n * sizeof(float))) return rc;
  x->grad->valid = true;
  return NUMRS_HIP_OK;
}

int numrs_hip_tensor_zero_grad(numrs_hip_tensor *t) {  // tensor.rs:135-142
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  if (t->t->grad) {
    t->t->grad->valid = false;
    t->t->grad->seed_preset = false;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_tensor_device_ptrs(numrs_hip_tensor *t, float **data, float **grad) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  if (data) *data = t->t->data->ptr;
  if (grad) {
    *grad = nullptr;
    if (t->t->grad) {
      if (int rc = grad_materialise(t->t)) return rc;
      *grad = t->t->grad->buf->ptr;
    }
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_tensor_backward(numrs_hip_tensor *t) {
  if (t == nullptr) return NUMRS_HIP_E_INVALID;
  return backward(t->t);
}

// detach clones the values (tensor.rs:146-154, data.clone()): an optimizer
// step on the source later does not change the detached tensor.
int numrs_hip_tensor_detach(numrs_hip_tensor *t, numrs_hip_tensor **out) {
  if (t == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  const T &src = t->t;
  T r;
  if (int rc = make_tensor(src->ctx, src->shape, false, &r)) return rc;
  if (int rc = numrs_hip_copy(src->ctx, r->data->ptr, src->data->ptr,
                              (size_t)src->numel() * sizeof(float)))
    return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_binary(int kind, numrs_hip_tensor *a, numrs_hip_tensor *b,
                            numrs_hip_tensor **out) {
  if (int rc = check2(a, b, out)) return rc;
  if (kind < NUMRS_HIP_ADD || kind > NUMRS_HIP_DIV)
    return fail(a->t->ctx, NUMRS_HIP_E_INVALID, "binary kind %d", kind);
  T r;
  if (int rc = op_binary(kind, a->t, b->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_unary(int kind, numrs_hip_tensor *a, float param, numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  if (kind < NUMRS_HIP_RELU || kind > NUMRS_HIP_POW)
    return fail(a->t->ctx, NUMRS_HIP_E_INVALID, "unary kind %d", kind);
  T r;
  if (int rc = op_unary(kind, a->t, param, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_matmul(numrs_hip_tensor *a, numrs_hip_tensor *b, numrs_hip_tensor **out) {
  if (int rc = check2(a, b, out)) return rc;
  T r;
  if (int rc = op_matmul(a->t, b->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_transpose(numrs_hip_tensor *a, numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_transpose(a->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_reshape(numrs_hip_tensor *a, const int64_t *shape, int ndim,
                             numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr || ndim < 0 || ndim > 8 || (ndim && !shape))
    return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_reshape(a->t, std::vector<int64_t>(shape, shape + ndim), &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_sum(numrs_hip_tensor *a, int mean, numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_sum(a->t, mean != 0, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_mse_loss(numrs_hip_tensor *pred, numrs_hip_tensor *target,
                              numrs_hip_tensor **out) {
  if (int rc = check2(pred, target, out)) return rc;
  T r;
  if (int rc = op_mse(pred->t, target->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_cross_entropy_loss(numrs_hip_tensor *logits, numrs_hip_tensor *target,
                                        numrs_hip_tensor **out) {
  if (int rc = check2(logits, target, out)) return rc;
  T r;
  if (int rc = op_ce(logits->t, target->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_cross_entropy_labels(numrs_hip_tensor *logits, const int32_t *host_labels,
                                          numrs_hip_tensor **out) {
  if (logits == nullptr || host_labels == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_ce_labels(logits->t, host_labels, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_softmax(numrs_hip_tensor *a, numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_softmax(a->t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_sum_axis(numrs_hip_tensor *a, int64_t axis, int mean,
                              numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_sum_axis(a->t, axis, mean != 0, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_softmax_axis(numrs_hip_tensor *a, int64_t axis, numrs_hip_tensor **out) {
  if (a == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_softmax_axis(a->t, axis, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_layer_norm(numrs_hip_tensor *x, numrs_hip_tensor *gamma,
                                numrs_hip_tensor *beta, float eps, numrs_hip_tensor **out) {
  if (x == nullptr || gamma == nullptr || beta == nullptr || out == nullptr)
    return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_layernorm(x->t, gamma->t, beta->t, eps, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_linear(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                            numrs_hip_tensor **out) {
  if (x == nullptr || W == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_linear(x->t, W->t, b ? &b->t : nullptr, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_linear_relu(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                                 numrs_hip_tensor **out) {
  if (x == nullptr || W == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_linear(x->t, W->t, b ? &b->t : nullptr, &r, 1)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_linear_gelu(numrs_hip_tensor *x, numrs_hip_tensor *W, numrs_hip_tensor *b,
                                 numrs_hip_tensor **out) {
  if (x == nullptr || W == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_linear(x->t, W->t, b ? &b->t : nullptr, &r, 2)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_linear_residual(numrs_hip_tensor *x, numrs_hip_tensor *W,
                                     numrs_hip_tensor *b, numrs_hip_tensor *res,
                                     numrs_hip_tensor **out) {
  if (x == nullptr || W == nullptr || res == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_linear(x->t, W->t, b ? &b->t : nullptr, &r, 0, &res->t)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_lstm(numrs_hip_tensor *x, numrs_hip_tensor *w_ih, numrs_hip_tensor *w_hh,
                          numrs_hip_tensor *b, numrs_hip_tensor **out) {
  if (x == nullptr || w_ih == nullptr || w_hh == nullptr || out == nullptr)
    return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_lstm(x->t, w_ih->t, w_hh->t, b ? &b->t : nullptr, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_lstm2(numrs_hip_tensor *x, numrs_hip_tensor *w_ih1, numrs_hip_tensor *w_hh1,
                           numrs_hip_tensor *b1, numrs_hip_tensor *w_ih2,
                           numrs_hip_tensor *w_hh2, numrs_hip_tensor *b2,
                           numrs_hip_tensor **out) {
  if (x == nullptr || w_ih1 == nullptr || w_hh1 == nullptr || w_ih2 == nullptr ||
      w_hh2 == nullptr || out == nullptr)
    return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_lstm2(x->t, w_ih1->t, w_hh1->t, b1 ? &b1->t : nullptr, w_ih2->t, w_hh2->t,
                        b2 ? &b2->t : nullptr, &r))
    return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_time_slice(numrs_hip_tensor *x, int64_t t, numrs_hip_tensor **out) {
  if (x == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_time_slice(x->t, t, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_attention(numrs_hip_tensor *q, numrs_hip_tensor *k, numrs_hip_tensor *v,
                               int64_t batch, int64_t seq, int64_t heads, numrs_hip_tensor **out) {
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_attention(q->t, k->t, v->t, batch, seq, heads, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_tensor_attention_qkv(numrs_hip_tensor *qkv, int64_t batch, int64_t seq,
                                   int64_t heads, numrs_hip_tensor **out) {
  if (qkv == nullptr || out == nullptr) return NUMRS_HIP_E_INVALID;
  T r;
  if (int rc = op_attention_qkv(qkv->t, batch, seq, heads, &r)) return rc;
  return wrap(std::move(r), out);
}

int numrs_hip_optim_sgd(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                        float momentum, float wd, numrs_hip_optim **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr || n < 0 || (n > 0 && params == nullptr)) return NUMRS_HIP_E_INVALID;
  auto *o = new numrs_hip_optim();
  o->o.lr = lr;
  o->o.mu = momentum;
  o->o.wd = wd;
  if (int rc = new_optim(ctx, params, n, false, &o->o)) {
    delete o;
    return rc;
  }
  *out = o;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_adam(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                         float b1, float b2, float eps, float wd, numrs_hip_optim **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr || n < 0 || (n > 0 && params == nullptr)) return NUMRS_HIP_E_INVALID;
  auto *o = new numrs_hip_optim();
  o->o.lr = lr;
  o->o.b1 = b1;
  o->o.b2 = b2;
  o->o.eps = eps;
  o->o.wd = wd;
  if (int rc = new_optim(ctx, params, n, true, &o->o)) {
    delete o;
    return rc;
  }
  *out = o;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_step(numrs_hip_optim *opt) {
  if (opt == nullptr) return NUMRS_HIP_E_INVALID;
  Optim &o = opt->o;
  // A recorded graph replays its kernels with the arguments of the recording:
  // optimizers whose step passes a host-side step count (bias corrections,
  // Lookahead's k, L-BFGS's host-side line state) would repeat one step's
  // values on every replay.
  if (o.ctx != nullptr && o.ctx->capturing &&
      (o.adam || o.fam == Family::Lookahead || o.fam == Family::LBFGS ||
       (o.fam == Family::Kind && kind_uses_t(o.kind))))
    return fail(o.ctx, NUMRS_HIP_E_INVALID,
                "this optimizer's step depends on a host-side step count and cannot be recorded "
                "into a graph; record SGD steps, or run this optimizer eagerly");
  switch (o.fam) {
    case Family::Lookahead: return lookahead_step(o);
    case Family::LBFGS: return lbfgs_step(o);
    default: break;
  }
  if (o.adam) ++o.t;  // adam.rs:125
  if (o.fam == Family::Kind && kind_uses_t(o.kind)) ++o.t;  // e.g. adamw.rs:93
  std::vector<float *> ps, ms, vs;
  std::vector<const float *> gs;
  std::vector<int64_t> ns;
  for (size_t i = 0; i < o.params.size(); ++i) {
    const T &p = o.params[i];
    if (!p->requires_grad) continue;  // sgd.rs:91-93, adam.rs:134-136
    if (int rc = grad_materialise(p)) return rc;
    ps.push_back(p->data->ptr);
    gs.push_back(p->grad->buf->ptr);
    ms.push_back(o.s1[i] ? o.s1[i]->ptr : nullptr);
    vs.push_back(o.s2[i] ? o.s2[i]->ptr : nullptr);
    ns.push_back(p->numel());
  }
  if (ps.empty()) return NUMRS_HIP_OK;
  const int count = (int)ps.size();
  if (o.fam == Family::Kind)
    return numrs_hip_optimizer_step(o.ctx, o.kind, ps.data(), gs.data(), ms.data(), vs.data(),
                                    ns.data(), count, o.hyper, o.nhyper, o.t);
  if (o.adam)
    return numrs_hip_adam_step_multi(o.ctx, ps.data(), gs.data(), ms.data(), vs.data(), ns.data(),
                                     count, o.lr, o.b1, o.b2, o.eps, o.wd, o.t);
  return numrs_hip_sgd_step_multi(o.ctx, ps.data(), gs.data(), o.mu != 0.0f ? ms.data() : nullptr,
                                  ns.data(), count, o.lr, o.mu, o.wd);
}

int numrs_hip_optim_zero_grad(numrs_hip_optim *opt) {  // sgd.rs:126-130
  if (opt == nullptr) return NUMRS_HIP_E_INVALID;
  if (opt->o.fam == Family::Lookahead) return numrs_hip_optim_zero_grad(opt->o.inner);
  for (const T &p : opt->o.params)
    if (p->grad) p->grad->valid = false;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_set_lr(numrs_hip_optim *opt, float lr) {
  if (opt == nullptr) return NUMRS_HIP_E_INVALID;
  Optim &o = opt->o;
  if (o.fam == Family::Lookahead) return numrs_hip_optim_set_lr(o.inner, lr);  // lookahead.rs:130
  if (o.fam == Family::Kind) {
    if (o.kind == NUMRS_HIP_OPT_ADADELTA) return NUMRS_HIP_OK;  // adadelta.rs:144-146
    if (o.kind == NUMRS_HIP_OPT_RPROP) {  // rprop.rs:174-181: every step size = lr
      for (size_t i = 0; i < o.s1.size(); ++i)
        if (o.s1[i])
          if (int rc = numrs_hip_fill(o.ctx, o.s1[i]->ptr, o.params[i]->numel(), lr)) return rc;
      o.hyper[0] = lr;
      return NUMRS_HIP_OK;
    }
    o.hyper[0] = lr;
  }
  o.lr = lr;
  return NUMRS_HIP_OK;
}

float numrs_hip_optim_lr(const numrs_hip_optim *opt) {
  if (opt == nullptr) return NAN;
  const Optim &o = opt->o;
  if (o.fam == Family::Lookahead) return numrs_hip_optim_lr(o.inner);  // lookahead.rs:126
  if (o.fam == Family::Kind) {
    if (o.kind == NUMRS_HIP_OPT_ADADELTA) return 1.0f;  // adadelta.rs:139-142
    if (o.kind == NUMRS_HIP_OPT_RPROP) return rprop_mean_step(o);  // rprop.rs:163-172
    return o.hyper[0];
  }
  return o.lr;
}

int numrs_hip_optim_free(numrs_hip_optim *opt) {
  delete opt;
  return NUMRS_HIP_OK;
}

// Optimizer state for checkpoints: the per-parameter state slots (SGD
// velocity; Adam m, v; the other kinds' s1/s2) and the step counter.
// Lookahead and L-BFGS keep state of another shape and are not exported.
int numrs_hip_optim_state_info(const numrs_hip_optim *opt, int *n_params, int *n_slots,
                               int64_t *step) {
  if (opt == nullptr) return NUMRS_HIP_E_INVALID;
  const Optim &o = opt->o;
  if (o.fam == Family::Lookahead || o.fam == Family::LBFGS)
    return fail(o.ctx, NUMRS_HIP_E_INVALID, "optimizer state export covers SGD, Adam and the "
                "element-wise kinds, not Lookahead or L-BFGS");
  int slots = 0;
  for (size_t i = 0; i < o.params.size(); ++i) {
    if (o.s1[i]) slots = std::max(slots, 1);
    if (o.s2[i]) slots = 2;
  }
  if (n_params != nullptr) *n_params = (int)o.params.size();
  if (n_slots != nullptr) *n_slots = slots;
  if (step != nullptr) *step = o.t;
  return NUMRS_HIP_OK;
}

namespace {
int state_buf(const Optim &o, int param, int slot, int64_t n, float **ptr) {
  if (o.fam == Family::Lookahead || o.fam == Family::LBFGS)
    return fail(o.ctx, NUMRS_HIP_E_INVALID, "no exportable state for Lookahead or L-BFGS");
  if (param < 0 || param >= (int)o.params.size() || slot < 0 || slot > 1)
    return fail(o.ctx, NUMRS_HIP_E_INVALID, "state slot %d of parameter %d does not exist", slot,
                param);
  const Buf &b = slot == 0 ? o.s1[param] : o.s2[param];
  if (!b) return fail(o.ctx, NUMRS_HIP_E_INVALID, "parameter %d has no state slot %d", param, slot);
  if (n != o.params[param]->numel())
    return fail(o.ctx, NUMRS_HIP_E_SHAPE, "state of parameter %d holds %lld values, not %lld",
                param, (long long)o.params[param]->numel(), (long long)n);
  *ptr = b->ptr;
  return NUMRS_HIP_OK;
}
}  // namespace

int numrs_hip_optim_state_get(numrs_hip_optim *opt, int param, int slot, float *host, int64_t n) {
  if (opt == nullptr || (host == nullptr && n > 0)) return NUMRS_HIP_E_INVALID;
  float *p = nullptr;
  if (int rc = state_buf(opt->o, param, slot, n, &p)) return rc;
  return numrs_hip_download(opt->o.ctx, host, p, (size_t)n * sizeof(float));
}

int numrs_hip_optim_state_set(numrs_hip_optim *opt, int param, int slot, const float *host,
                              int64_t n) {
  if (opt == nullptr || (host == nullptr && n > 0)) return NUMRS_HIP_E_INVALID;
  float *p = nullptr;
  if (int rc = state_buf(opt->o, param, slot, n, &p)) return rc;
  return numrs_hip_upload(opt->o.ctx, p, host, (size_t)n * sizeof(float));
}

int numrs_hip_optim_set_step(numrs_hip_optim *opt, int64_t step) {
  if (opt == nullptr || step < 0 || step > 0x7fffffff) return NUMRS_HIP_E_INVALID;
  opt->o.t = (int)step;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_create(numrs_hip_ctx *ctx, int kind, numrs_hip_tensor **params, int n,
                           const float *hyper, int nhyper, numrs_hip_optim **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr || n < 0 || (n > 0 && params == nullptr) || hyper == nullptr ||
      nhyper < 1 || nhyper > 8)
    return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_optim_create: bad arguments");
  *out = nullptr;
  if (kind_hyper_count(kind) != nhyper)
    return fail(ctx, NUMRS_HIP_E_INVALID, "optimizer kind %d takes %d hyperparameters, got %d",
                kind, kind_hyper_count(kind), nhyper);
  auto *o = new numrs_hip_optim();
  Optim &op = o->o;
  op.ctx = ctx;
  op.fam = Family::Kind;
  op.kind = kind;
  op.nhyper = nhyper;
  for (int i = 0; i < nhyper; ++i) op.hyper[i] = hyper[i];
  op.lr = hyper[0];
  // State slots start at zero, Rprop's step sizes at lr_init (rprop.rs:71-76).
  const bool two = !(kind == NUMRS_HIP_OPT_ADAGRAD ||
                     (kind == NUMRS_HIP_OPT_RMSPROP && !(hyper[4] > 0.0f)));
  for (int i = 0; i < n; ++i) {
    if (params[i] == nullptr) {
      delete o;
      return fail(ctx, NUMRS_HIP_E_INVALID, "null parameter %d", i);
    }
    const T &p = params[i]->t;
    op.params.push_back(p);
    Buf a, b;
    const float first = kind == NUMRS_HIP_OPT_RPROP ? hyper[0] : 0.0f;
    int rc = alloc_buf(ctx, p->numel(), sizeof(float), &a);
    if (!rc) rc = numrs_hip_fill(ctx, a->ptr, p->numel(), first);
    if (!rc && two) rc = alloc_buf(ctx, p->numel(), sizeof(float), &b);
    if (!rc && two) rc = numrs_hip_fill(ctx, b->ptr, p->numel(), 0.0f);
    if (rc) {
      delete o;
      return rc;
    }
    op.s1.push_back(a);
    op.s2.push_back(b);
  }
  *out = o;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_lookahead(numrs_hip_optim *inner, numrs_hip_tensor **params, int n, int k,
                              float alpha, numrs_hip_optim **out) {
  if (inner == nullptr || out == nullptr || n < 0 || (n > 0 && params == nullptr) || k < 1)
    return NUMRS_HIP_E_INVALID;
  numrs_hip_ctx *ctx = inner->o.ctx;
  *out = nullptr;
  auto *o = new numrs_hip_optim();
  Optim &op = o->o;
  op.ctx = ctx;
  op.fam = Family::Lookahead;
  op.la_k = k;
  op.la_alpha = alpha;
  for (int i = 0; i < n; ++i) {
    if (params[i] == nullptr) {
      delete o;
      return fail(ctx, NUMRS_HIP_E_INVALID, "null parameter %d", i);
    }
    const T &p = params[i]->t;
    op.params.push_back(p);
    Buf b;  // slow weights start as the current values (lookahead.rs:66-75)
    int rc = alloc_buf(ctx, p->numel(), sizeof(float), &b);
    if (!rc) rc = numrs_hip_copy(ctx, b->ptr, p->data->ptr, (size_t)p->numel() * sizeof(float));
    if (rc) {
      delete o;
      return rc;
    }
    op.slow.push_back(b);
  }
  op.inner = inner;  // taken over only on success
  *out = o;
  return NUMRS_HIP_OK;
}

int numrs_hip_optim_lbfgs(numrs_hip_ctx *ctx, numrs_hip_tensor **params, int n, float lr,
                          int history_size, int max_iter, numrs_hip_optim **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr || n < 0 || (n > 0 && params == nullptr) || history_size < 0)
    return NUMRS_HIP_E_INVALID;
  *out = nullptr;
  auto *o = new numrs_hip_optim();
  Optim &op = o->o;
  op.ctx = ctx;
  op.fam = Family::LBFGS;
  op.lr = lr;
  op.history = history_size;
  op.max_iter = max_iter;
  for (int i = 0; i < n; ++i) {
    if (params[i] == nullptr) {
      delete o;
      return fail(ctx, NUMRS_HIP_E_INVALID, "null parameter %d", i);
    }
    op.params.push_back(params[i]->t);
    op.total += params[i]->t->numel();
  }
  const int64_t m = op.total > 0 ? op.total : 1;
  int rc = alloc_buf(ctx, m, sizeof(float), &op.cur_p);
  if (!rc) rc = alloc_buf(ctx, m, sizeof(float), &op.cur_g);
  if (!rc) rc = alloc_buf(ctx, m, sizeof(float), &op.work_q);
  if (!rc) rc = alloc_buf(ctx, m, sizeof(float), &op.work_r);
  if (!rc) rc = alloc_buf(ctx, 1, sizeof(float), &op.scalar);
  if (rc) {
    delete o;
    return rc;
  }
  *out = o;
  return NUMRS_HIP_OK;
}

}  // extern "C"
