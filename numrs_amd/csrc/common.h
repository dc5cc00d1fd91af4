// Internal declarations shared by the HIP translation units of libnumrs_hip.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <unordered_map>
#include <vector>

#include "numrs_hip.h"

constexpr int kMaxTimers = 256;

struct numrs_hip_ctx {
  int device = 0;
  int num_cus = 0;
  char arch[64] = {0};
  hipStream_t stream = nullptr;
  hipEvent_t events[kMaxTimers] = {};
  void *workspace = nullptr;  // reduction partials (reused by every call)
  size_t workspace_bytes = 0;
  void *scratch = nullptr;    // a second region for values that must outlive a
  size_t scratch_bytes = 0;   // workspace user inside the same call
  // Stream-ordered block cache of the tensor engine: every kernel runs on
  // `stream`, so a block released by one tensor can be handed to the next
  // allocation without a device synchronisation.
  std::unordered_map<size_t, std::vector<void *>> free_blocks;
  size_t cached_bytes = 0;
  // Engine blocks still owned by tensors.  numrs_hip_destroy with live blocks
  // only marks the context destroyed; the last block_free then deletes it, so
  // tensors may safely outlive their context's destroy call.
  int64_t live_blocks = 0;
  bool destroyed = false;
  int unbroadcast_mode = NUMRS_HIP_UNBROADCAST_CORRECT;
  // Graph recording (numrs_hip_graph_begin .. _end): while `capturing`,
  // blocks released by tensors are held in `capture_held` instead of going
  // back to the cache -- the recorded kernels may use them on every replay
  // -- and the graph takes them over when the recording ends.
  bool capturing = false;
  std::vector<std::pair<void *, size_t>> capture_held;
  // Instantiated graphs not yet destroyed.  Their kernels address the
  // workspace and scratch regions as they were when recorded, so while any
  // exist a region that grows keeps its old buffer in `retired`; the last
  // graph_destroy (or the context's destroy) frees them.
  int64_t live_graphs = 0;
  std::vector<void *> retired;
  // graph_destroy calls made while a recording is open; run when it ends.
  std::vector<struct numrs_hip_graph *> pending_destroy;
  // Give-up word of the persistent recurrence kernels (lstm.hip): a device
  // int, allocated on first use, that a kernel sets when a bounded wait for
  // another workgroup's step ran out.  wait_check marks that such a kernel
  // was queued since the word was last read; the next call that synchronises
  // the stream reads it and reports a give-up as an error.
  int *wait_status = nullptr;
  bool wait_check = false;
  // A NUMRS_HIP_RECURRENCE_* mode (numrs_hip_set_recurrence_mode), and the
  // persistent kernels' resident workgroups per CU (-1: not queried; the
  // forward per input-block count 0..4).
  int recurrence_mode = 0;
  int persist_fwd_per_cu[5] = {-1, -1, -1, -1, -1};
  int persist_bwd_per_cu = -1;
  int64_t persist_launches = 0;  // persistent launches queued on this context
  int persist_wait_limit = -1;   // wait rounds before a give-up (-1: the kernels' default)
  // Arrival counters of the products that reduce their split-K partials
  // inside their own launch (gemm.hip): zero between launches -- each
  // launch's last arrival at a counter sets it back -- so they are cleared
  // only when the region is allocated.
  unsigned *arrivals = nullptr;
  size_t arrival_words = 0;
  int split_reduce_mode = NUMRS_HIP_SPLIT_REDUCE_FUSED;  // numrs_hip_set_split_reduction
  // Device address of reduce.hip's static partials array on this context's
  // device, resolved at creation (the allocation-free entry point uses it).
  float *noalloc_partials = nullptr;
  int noalloc_status = 0;
  char last_error[512] = {0};
};

namespace numrs_hip {

// Records a formatted message on the context and returns `code`.
int fail(numrs_hip_ctx *ctx, int code, const char *fmt, ...);

// Returns the context's workspace with at least `bytes` bytes (grows it).
int workspace(numrs_hip_ctx *ctx, size_t bytes, void **out);

// Second scratch region (see numrs_hip_ctx::scratch).
int scratch(numrs_hip_ctx *ctx, size_t bytes, float **out);

// The context's arrival counters, at least `words` of them, all zero when
// the stream reaches the next launch (grows and clears the region).
int arrival_counters(numrs_hip_ctx *ctx, size_t words, unsigned **out);

// Cached device allocation for engine tensors; sizes are rounded up so that
// released blocks are reusable.  block_free returns the block to the cache
// (or, while a graph is being recorded, to the recording's held set).
int block_alloc(numrs_hip_ctx *ctx, size_t bytes, void **out);
void block_free(numrs_hip_ctx *ctx, void *p, size_t bytes);
size_t block_round(size_t bytes);
void cache_release(numrs_hip_ctx *ctx);

// Temporary device block from the context's block cache, released at scope
// exit (stream-ordered: a released block is only reused by later work on the
// same stream).  Unlike the workspace, a block stays valid while the calls
// made inside its scope use the workspace themselves.
struct TempBlock {
  numrs_hip_ctx *ctx;
  void *p = nullptr;
  size_t bytes = 0;
  explicit TempBlock(numrs_hip_ctx *c) : ctx(c) {}
  TempBlock(const TempBlock &) = delete;
  TempBlock &operator=(const TempBlock &) = delete;
  int alloc(size_t b) {
    bytes = b;
    return block_alloc(ctx, b, &p);
  }
  float *f() const { return static_cast<float *>(p); }
  ~TempBlock() { block_free(ctx, p, bytes); }
};

// Checks the launch that was just enqueued.
int check_launch(numrs_hip_ctx *ctx, const char *what);

// The context's give-up word for persistent kernels (zeroed on allocation),
// and the check of it after a stream synchronisation (no-op unless such a
// kernel ran since the last check).
int wait_status_word(numrs_hip_ctx *ctx, int **out);

int check_wait_status(numrs_hip_ctx *ctx);

// Loss backward kernels for the engine's root node: with `seed` non-null the
// incoming gradient is the sweep's seed 1 (not read from g_scalar) and the
// kernel writes that 1 into seed[0], the root's gradient cell, so the seed
// needs no launch of its own.  seed == nullptr is numrs_hip_mse_backward /
// numrs_hip_softmax_ce_backward.
int mse_backward_impl(numrs_hip_ctx *ctx, const float *g_scalar, float *seed, const float *p,
                      const float *t, float *dp, float *dt, int64_t n, int accumulate);
int softmax_ce_backward_impl(numrs_hip_ctx *ctx, const float *g_scalar, float *seed,
                             const float *logits, const float *onehot, const int32_t *labels,
                             float *dlogits, int64_t B, int64_t C, int accumulate);

// Resolves, with the context's device current, the device address of the
// static partials array of the allocation-free column reduction (reduce.hip)
// into ctx->noalloc_partials; once per device, later contexts reuse it.
int noalloc_init(numrs_hip_ctx *ctx);

// Vector operations of the L-BFGS two-loop recursion (optim/lbfgs.rs),
// out[i] = f(a[i], b[i], s) in the reference's operation order.
enum VecOp {
  kVecSub = 0,    // a - b
  kVecAxmy = 1,   // a - s*b
  kVecScale = 2,  // s*a
  kVecAypx = 3,   // a + b*s
  kVecNeg = 4,    // -a
  kVecAxpy = 5    // a + s*b
};
int vec_op(numrs_hip_ctx *ctx, float *out, const float *a, const float *b, float s, int64_t n,
           int op);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Access modes of the streaming kernels: 0 per element, 1 float4, 2 float4
// with the non-temporal hint.  Arrays of at least kStreamElems floats (32 MB)
// are unlikely to stay in the 256 MB Infinity Cache from one kernel of a
// training step to the next, and streaming them past the caches measured
// 13-14% faster on MI355X from HBM (read-2-write-1: 0.70 -> 0.80 of 8 TB/s;
// read-3-write-2: 0.70 -> 0.79).  Smaller arrays keep cached accesses, so a
// consumer kernel can find them in the cache.  (2^23 rather than 2^24: the
// C4 attention softmax backward at 2^23 elements went 0.64 -> 0.71 of HBM,
// and the C4 step time did not change.)
constexpr int64_t kStreamElems = int64_t(1) << 23;
inline int vec_mode(bool vec, int64_t n) { return !vec ? 0 : (n >= kStreamElems ? 2 : 1); }

// Calls f(std::integral_constant<int, mode>{}) for a runtime access mode,
// so that a launch site can pass the mode as a template argument.
template <typename F>
void with_vec_mode(int mode, F &&f) {
  if (mode == 2)
    f(std::integral_constant<int, 2>{});
  else if (mode == 1)
    f(std::integral_constant<int, 1>{});
  else
    f(std::integral_constant<int, 0>{});
}

typedef float nrs_f4 __attribute__((ext_vector_type(4)));

// Device-scope accesses for values that one workgroup hands to another,
// possibly on another XCD, inside one launch: stores write through to the
// device's coherence point and loads fetch from it (the sc1 scope bit), so
// the XCDs' L2 caches need no cache-wide write-back or invalidation.  A
// writer waits for its stores to be acknowledged (s_waitcnt) before it
// publishes them with a device-scope atomic; a reader loads them only after
// it has seen that atomic.
constexpr int kScDevice = 16;          // buffer access cache-policy bits: sc1
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3: 32-bit data format
// Buffer resource over `bytes` bytes at p (bytes < 2^31); loads past the end
// return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const float *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                           kBufWord3);
}
// (The buffer-load builtin returns raw 32-bit words; the loaded bits are
// reinterpreted as floats, never converted.)
__device__ __forceinline__ nrs_f4 ld_dev4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(nrs_f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kScDevice));
}
__device__ __forceinline__ float ld_dev1(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kScDevice));
}
__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int V>
__device__ __forceinline__ nrs_f4 ldv(const float *p) {
  if constexpr (V == 2)
    return __builtin_nontemporal_load(reinterpret_cast<const nrs_f4 *>(p));
  else
    return *reinterpret_cast<const nrs_f4 *>(p);
}

template <int V>
__device__ __forceinline__ void stv(float *p, nrs_f4 v) {
  if constexpr (V == 2)
    __builtin_nontemporal_store(v, reinterpret_cast<nrs_f4 *>(p));
  else
    *reinterpret_cast<nrs_f4 *>(p) = v;
}

// GELU, exact-erf form: x * 0.5 * (1 + erf(x / sqrt 2)); shared by the unary
// forward kernel and the GEMM epilogue, so both round alike.
__device__ __forceinline__ float gelu_erf(float x) {
  return x * 0.5f * (1.0f + erff(x * 0.70710678118654752f));
}

// A batched row-major fp32 matrix: element (i, j) of batch z = zo*inner + zi
// sits at p + zo*so + zi*si + i*ld + j.
struct BatchedMat {
  const float *p;
  int64_t ld, so, si;
};
struct BatchedOut {
  float *p;
  int64_t ld, so, si;
};

// C1_z = alpha X_z Y1_z ([M,K] x [K,N]) and C2_z = alpha X_z^T Y2_z
// ([K,M] x [M,N]) for z < batch, in one launch where the streamed path fits
// (the shape of the Linear backward and of attention's dQ/dK).  Either
// output may be null; accumulate adds into the outputs.
int gemm_nn_tn_pair(numrs_hip_ctx *ctx, BatchedMat X, BatchedMat Y1, BatchedOut C1, BatchedMat Y2,
                    BatchedOut C2, int64_t M, int64_t K, int64_t N, float alpha, int accumulate,
                    int64_t batch, int64_t binner);
// The MSE loss (numrs_hip_mse_loss) that, with dp, also writes the gradient
// its backward forms as the sweep's root (g = 1: dp = (2 (p - t)) / n, the
// backward kernel's arithmetic) and, with seed, writes 1 there.
int mse_loss_impl(numrs_hip_ctx *ctx, const float *p, const float *t, int64_t n, float *out,
                  float *dp, float *seed);
// The same for the cross-entropy loss (numrs_hip_cross_entropy_loss): dx =
// (softmax - target) / B, for batches where cross_entropy_preforms(B).
int cross_entropy_loss_impl(numrs_hip_ctx *ctx, const float *logits, const float *onehot,
                            const int32_t *labels, int64_t B, int64_t C, float *out, float *dx,
                            float *seed);
bool cross_entropy_preforms(int64_t B);

// C1_z = alpha1 X1_z^T Y1_z and C2_z = alpha2 X2_z^T Y2_z (X [M,K], Y [M,N],
// C [K,N]) for z < batch, in one launch where the streamed path fits
// (attention's dV = P^T dO with dK = alpha dS^T Q).  Either output may be
// null; accumulate adds into the outputs.
int gemm_tn_pair(numrs_hip_ctx *ctx, BatchedMat X1, BatchedMat Y1, BatchedOut C1, float alpha1,
                 BatchedMat X2, BatchedMat Y2, BatchedOut C2, float alpha2, int64_t M, int64_t K,
                 int64_t N, int accumulate, int64_t batch, int64_t binner);
// Two weight gradients of one left operand, C1[K,N1] = X^T Y1 and
// C2[K,N2] = X^T Y2 (X [M,K] at row stride ldx, Y1 [M,N1], Y2 [M,N2]), in
// one launch with a joint split plan where the streamed path fits, and the
// column sums db[K] of X (null for none) formed by the launch that reduces
// the splits (the LSTM's dW_ih, dW_hh and db): from db_part [db_rows, K],
// partial sums of X over row groups added in row order as a compensated sum,
// when given, else as the CORRECT-mode unbroadcast of X.  acc* add into the
// outputs.
int gemm_tn2_colsum(numrs_hip_ctx *ctx, const float *X, int64_t ldx, int64_t M, int64_t K,
                    const float *Y1, int64_t ldy1, int64_t N1, float *C1, int acc1,
                    const float *Y2, int64_t ldy2, int64_t N2, float *C2, int acc2, float *db,
                    int acc_db, const float *db_part, int64_t db_rows);


// One LDS DMA instruction: each lane copies 16 bytes from base + off (off in
// bytes, per lane; base uniform) into LDS at lds + 16 * lane.  Written as
// inline asm so that the compiler neither sinks the issue towards the next
// barrier nor adds its own vmcnt waits for it (it cannot tell which LDS stage
// an LDS DMA writes, so it would wait for every outstanding one before any
// fragment read).  The caller places the vmcnt waits: vector-memory
// operations complete in issue order.  The s_nop covers the M0 write -> LDS
// DMA hazard.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop


// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (expcnt and lgkmcnt left at their no-wait maxima).  The
// 6-bit vmcnt is split: bits 3:0 of the immediate hold vmcnt[3:0] and bits
// 15:14 hold vmcnt[5:4].
constexpr int wait_vm(int n) { return 0x3f70 | (n & 15) | ((n >> 4) << 14); }

}  // namespace numrs_hip

#define NRS_CHECK_CTX(ctx)                       \
  do {                                           \
    if ((ctx) == nullptr) return NUMRS_HIP_E_INVALID; \
  } while (0)

#define NRS_HIP(ctx, call)                                                              \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess)                                                               \
      return numrs_hip::fail((ctx), NUMRS_HIP_E_HIP, "%s failed: %s", #call,            \
                             hipGetErrorString(e_));                                    \
  } while (0)

// Grid sizing for element-streaming kernels.
inline unsigned grid_for(int64_t work_items, int per_block) {
  int64_t g = (work_items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 0x7fffffff) g = 0x7fffffff;
  return static_cast<unsigned>(g);
}

// Wavefront (64 lanes) reductions: a butterfly over lane distances 32, 16,
// 8, 4, 2, 1, after which every lane holds the same value, formed from the
// same pairs in the same order as an xor-shuffle butterfly.  The exchanges
// stay in registers (one VALU operation each, against an LDS-crossbar round
// trip per ds_bpermute step of __shfl_xor):
//   distance 32: v_permlane32_swap of v with itself returns (low halves,
//                high halves) in every lane;
//   distance 16: v_permlane16_swap likewise returns (even rows, odd rows) of
//                each 32-lane half;
//   distance 8:  DPP row_ror:8 within each 16-lane row;
//   distance 4:  DPP row_half_mirror (lane i of 8 reads 7 - i = i ^ 7), then
//                a reversed quad (i ^ 3);
//   distance 2, 1: DPP quad permutations [2,3,0,1] and [1,0,3,2].
// x + y and fmaxf(x, y) give the same bits as y + x and fmaxf(y, x) on gfx950
// (signed zeros and NaN payloads included), so which operand of a pair a
// lane holds does not change the result.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}

template <class Op>
__device__ __forceinline__ float wave_butterfly(float v, Op op) {
  const unsigned u32 = __builtin_bit_cast(unsigned, v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u32, u32, false, false);
  v = op(__builtin_bit_cast(float, (unsigned)r32[0]), __builtin_bit_cast(float, (unsigned)r32[1]));
  const unsigned u16 = __builtin_bit_cast(unsigned, v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u16, u16, false, false);
  v = op(__builtin_bit_cast(float, (unsigned)r16[0]), __builtin_bit_cast(float, (unsigned)r16[1]));
  v = op(v, dpp_mov<0x128>(v));                    // row_ror:8
  v = op(v, dpp_mov<0x1B>(dpp_mov<0x141>(v)));     // row_half_mirror, quad [3,2,1,0]
  v = op(v, dpp_mov<0x4E>(v));                     // quad [2,3,0,1]
  v = op(v, dpp_mov<0xB1>(v));                     // quad [1,0,3,2]
  return v;
}

// v op (v of the lane 32 away), in every lane: the first butterfly level.
template <class Op>
__device__ __forceinline__ float half_pair(float v, Op op) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return op(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

// op over the lane's column of the wave's four 16-lane rows (lanes l,
// l ^ 16, l ^ 32, l ^ 48): distance 32, then distance 16, as wave_butterfly
// begins.
template <class Op>
__device__ __forceinline__ float rows4(float v, Op op) {
  v = half_pair(v, op);
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return op(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

// Sum over each quad of lanes: distance 1, then distance 2.
__device__ __forceinline__ float quad_sum(float v) {
  v = v + dpp_mov<0xB1>(v);
  return v + dpp_mov<0x4E>(v);
}

__device__ inline float wave_sum(float v) {
  return wave_butterfly(v, [](float a, float b) { return a + b; });
}

__device__ inline float wave_max(float v) {
  return wave_butterfly(v, [](float a, float b) { return fmaxf(a, b); });
}
