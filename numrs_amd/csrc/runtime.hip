// Context, device memory, workspace, timing and error reporting.
#include <cstring>
#include <string>

#include "common.h"

namespace numrs_hip {

int fail(numrs_hip_ctx *ctx, int code, const char *fmt, ...) {
  if (ctx != nullptr) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(ctx->last_error, sizeof(ctx->last_error), fmt, ap);
    va_end(ap);
  }
  return code;
}

// A buffer the recorded kernels address cannot move, and growing one needs a
// device synchronisation, which a recording stream does not allow.
static int refuse_growth(numrs_hip_ctx *ctx, const char *what, size_t bytes) {
  return fail(ctx, NUMRS_HIP_E_INVALID,
              "%s must grow to %zu bytes while a graph is being recorded: run the step once "
              "before recording it",
              what, bytes);
}

// Releases the old buffer of a region that grows.  An instantiated graph's
// kernels keep the address they were recorded with, so while a graph lives
// the buffer is retired instead and freed when the last graph is destroyed.
static hipError_t release_region(numrs_hip_ctx *ctx, void *p) {
  if (p == nullptr) return hipSuccess;
  if (ctx->live_graphs > 0) {
    ctx->retired.push_back(p);
    return hipSuccess;
  }
  return hipFree(p);
}

static void free_retired(numrs_hip_ctx *ctx) {
  for (void *p : ctx->retired) (void)hipFree(p);
  ctx->retired.clear();
}

int workspace(numrs_hip_ctx *ctx, size_t bytes, void **out) {
  if (bytes <= ctx->workspace_bytes && ctx->workspace != nullptr) {
    *out = ctx->workspace;
    return NUMRS_HIP_OK;
  }
  if (ctx->capturing) return refuse_growth(ctx, "the workspace", bytes);
  // Growing: earlier kernels may still read the old buffer, so drain first.
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  NRS_HIP(ctx, release_region(ctx, ctx->workspace));
  ctx->workspace = nullptr;
  ctx->workspace_bytes = 0;
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  if (hipMalloc(&ctx->workspace, want) != hipSuccess) {
    ctx->workspace = nullptr;
    return fail(ctx, NUMRS_HIP_E_NOMEM, "workspace allocation of %zu bytes failed", want);
  }
  ctx->workspace_bytes = want;
  *out = ctx->workspace;
  return NUMRS_HIP_OK;
}

int scratch(numrs_hip_ctx *ctx, size_t bytes, float **out) {
  if (bytes <= ctx->scratch_bytes && ctx->scratch != nullptr) {
    *out = static_cast<float *>(ctx->scratch);
    return NUMRS_HIP_OK;
  }
  if (ctx->capturing) return refuse_growth(ctx, "the scratch region", bytes);
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  NRS_HIP(ctx, release_region(ctx, ctx->scratch));
  ctx->scratch = nullptr;
  ctx->scratch_bytes = 0;
  size_t want = bytes < (1u << 16) ? (1u << 16) : bytes;
  if (hipMalloc(&ctx->scratch, want) != hipSuccess) {
    ctx->scratch = nullptr;
    (void)hipGetLastError();
    return fail(ctx, NUMRS_HIP_E_NOMEM, "scratch allocation of %zu bytes failed", want);
  }
  ctx->scratch_bytes = want;
  *out = static_cast<float *>(ctx->scratch);
  return NUMRS_HIP_OK;
}

int arrival_counters(numrs_hip_ctx *ctx, size_t words, unsigned **out) {
  if (words <= ctx->arrival_words && ctx->arrivals != nullptr) {
    *out = ctx->arrivals;
    return NUMRS_HIP_OK;
  }
  if (ctx->capturing) return refuse_growth(ctx, "the arrival counters", words * sizeof(unsigned));
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  NRS_HIP(ctx, release_region(ctx, ctx->arrivals));
  ctx->arrivals = nullptr;
  ctx->arrival_words = 0;
  const size_t want = words < 4096 ? 4096 : words;
  if (hipMalloc(&ctx->arrivals, want * sizeof(unsigned)) != hipSuccess) {
    ctx->arrivals = nullptr;
    (void)hipGetLastError();
    return fail(ctx, NUMRS_HIP_E_NOMEM, "arrival counter allocation of %zu words failed", want);
  }
  NRS_HIP(ctx, hipMemsetAsync(ctx->arrivals, 0, want * sizeof(unsigned), ctx->stream));
  ctx->arrival_words = want;
  *out = ctx->arrivals;
  return NUMRS_HIP_OK;
}

size_t block_round(size_t bytes) {
  if (bytes <= 4096) return (bytes + 255) & ~size_t(255);
  // Round up to 1/8 steps of the enclosing power of two.
  size_t p = 1;
  while (p < bytes) p <<= 1;
  const size_t step = p / 8;
  return (bytes + step - 1) / step * step;
}

int block_alloc(numrs_hip_ctx *ctx, size_t bytes, void **out) {
  *out = nullptr;
  if (bytes == 0) return NUMRS_HIP_OK;
  if (ctx->destroyed) return fail(ctx, NUMRS_HIP_E_INVALID, "context already destroyed");
  const size_t size = block_round(bytes);
  auto it = ctx->free_blocks.find(size);
  if (it != ctx->free_blocks.end() && !it->second.empty()) {
    *out = it->second.back();
    it->second.pop_back();
    ctx->cached_bytes -= size;
    ++ctx->live_blocks;
    return NUMRS_HIP_OK;
  }
  if (hipMalloc(out, size) != hipSuccess) {
    (void)hipGetLastError();
    if (!ctx->capturing) cache_release(ctx);  // releasing synchronises the stream
    if (ctx->capturing || hipMalloc(out, size) != hipSuccess) {
      *out = nullptr;
      (void)hipGetLastError();
      return fail(ctx, NUMRS_HIP_E_NOMEM, "device allocation of %zu bytes failed", size);
    }
  }
  ++ctx->live_blocks;
  return NUMRS_HIP_OK;
}

void block_free(numrs_hip_ctx *ctx, void *p, size_t bytes) {
  if (p == nullptr) return;
  if (ctx->capturing) {  // still live: the recording owns it now
    ctx->capture_held.emplace_back(p, bytes);
    return;
  }
  --ctx->live_blocks;
  if (ctx->destroyed) {
    (void)hipFree(p);
    if (ctx->live_blocks == 0) delete ctx;
    return;
  }
  const size_t size = block_round(bytes);
  ctx->free_blocks[size].push_back(p);
  ctx->cached_bytes += size;
}

void cache_release(numrs_hip_ctx *ctx) {
  (void)hipStreamSynchronize(ctx->stream);
  for (auto &kv : ctx->free_blocks)
    for (void *p : kv.second) (void)hipFree(p);
  ctx->free_blocks.clear();
  ctx->cached_bytes = 0;
}

int wait_status_word(numrs_hip_ctx *ctx, int **out) {
  if (ctx->wait_status == nullptr) {
    if (ctx->capturing) return refuse_growth(ctx, "the wait status word", sizeof(int));
    if (hipMalloc(&ctx->wait_status, 256) != hipSuccess) {
      ctx->wait_status = nullptr;
      (void)hipGetLastError();
      return fail(ctx, NUMRS_HIP_E_NOMEM, "wait status allocation failed");
    }
    NRS_HIP(ctx, hipMemsetAsync(ctx->wait_status, 0, 256, ctx->stream));
  }
  *out = ctx->wait_status;
  return NUMRS_HIP_OK;
}

int check_wait_status(numrs_hip_ctx *ctx) {
  if (!ctx->wait_check || ctx->wait_status == nullptr) return NUMRS_HIP_OK;
  ctx->wait_check = false;
  int v = 0;
  NRS_HIP(ctx, hipMemcpyAsync(&v, ctx->wait_status, sizeof(int), hipMemcpyDeviceToHost,
                              ctx->stream));
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (v == 0) return NUMRS_HIP_OK;
  NRS_HIP(ctx, hipMemsetAsync(ctx->wait_status, 0, sizeof(int), ctx->stream));
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return fail(ctx, NUMRS_HIP_E_HIP,
              "a persistent LSTM recurrence kernel gave up waiting for another workgroup's "
              "step (code %d): its outputs are invalid",
              v);
}

int check_launch(numrs_hip_ctx *ctx, const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(ctx, NUMRS_HIP_E_HIP, "launch of %s failed: %s", what, hipGetErrorString(e));
  return NUMRS_HIP_OK;
}

}  // namespace numrs_hip

using numrs_hip::fail;

static thread_local char g_create_error[512] = {0};

// Calls that wait for the stream or move host memory are refused before they
// reach HIP while a graph is being recorded: HIP would otherwise invalidate
// the whole recording.
#define NRS_NOT_RECORDING(ctx, what)                                                         \
  do {                                                                                    \
    if ((ctx)->capturing)                                                                 \
      return fail((ctx), NUMRS_HIP_E_INVALID, "%s is not allowed while a graph is being "  \
                  "recorded", (what));                                                    \
  } while (0)

namespace {

__global__ void fill_kernel(float *__restrict__ dst, int64_t n, float value) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = value;
}

// Device-to-device copy of n16 16-byte words (grid-stride).
__global__ void __launch_bounds__(256)
    copy_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, int64_t n16) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace

extern "C" {

int numrs_hip_create(int device, numrs_hip_ctx **out) {
  g_create_error[0] = 0;
  if (out == nullptr) return NUMRS_HIP_E_INVALID;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= device || device < 0) {
    snprintf(g_create_error, sizeof(g_create_error), "no HIP device %d (count %d)", device, count);
    return NUMRS_HIP_E_NODEV;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    snprintf(g_create_error, sizeof(g_create_error), "hipGetDeviceProperties(%d) failed", device);
    return NUMRS_HIP_E_NODEV;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    snprintf(g_create_error, sizeof(g_create_error),
             "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    return NUMRS_HIP_E_NODEV;
  }
  auto *ctx = new numrs_hip_ctx();
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  std::strncpy(ctx->arch, prop.gcnArchName, sizeof(ctx->arch) - 1);
  if (hipSetDevice(device) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    snprintf(g_create_error, sizeof(g_create_error), "stream creation on device %d failed",
             device);
    delete ctx;
    return NUMRS_HIP_E_HIP;
  }
  for (int i = 0; i < kMaxTimers; ++i) {
    if (hipEventCreate(&ctx->events[i]) != hipSuccess) {
      snprintf(g_create_error, sizeof(g_create_error), "hipEventCreate failed");
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ctx->events[j]);
      (void)hipStreamDestroy(ctx->stream);
      delete ctx;
      return NUMRS_HIP_E_HIP;
    }
  }
  // A failure here only disables the allocation-free entry point, which then
  // reports it; every other entry point works without the array.
  ctx->noalloc_status = numrs_hip::noalloc_init(ctx);
  *out = ctx;
  return NUMRS_HIP_OK;
}

const char *numrs_hip_create_error(void) { return g_create_error; }

int numrs_hip_destroy(numrs_hip_ctx *ctx) {
  NRS_CHECK_CTX(ctx);
  (void)hipSetDevice(ctx->device);
  if (ctx->capturing) (void)numrs_hip_graph_abort(ctx);
  (void)hipStreamSynchronize(ctx->stream);
  for (int i = 0; i < kMaxTimers; ++i) (void)hipEventDestroy(ctx->events[i]);
  numrs_hip::cache_release(ctx);
  if (ctx->workspace != nullptr) (void)hipFree(ctx->workspace);
  if (ctx->scratch != nullptr) (void)hipFree(ctx->scratch);
  ctx->workspace = ctx->scratch = nullptr;
  if (ctx->arrivals != nullptr) (void)hipFree(ctx->arrivals);
  ctx->arrivals = nullptr;
  numrs_hip::free_retired(ctx);
  if (ctx->wait_status != nullptr) (void)hipFree(ctx->wait_status);
  ctx->wait_status = nullptr;
  (void)hipStreamDestroy(ctx->stream);
  ctx->stream = nullptr;
  ctx->destroyed = true;
  if (ctx->live_blocks == 0) delete ctx;  // else the last engine block frees it
  return NUMRS_HIP_OK;
}

// ---------------------------------------------------------------------------
// Graph recording and replay of a fixed sequence of work on the context's
// stream (a training step with fixed shapes and buffers).
// ---------------------------------------------------------------------------

struct numrs_hip_graph {
  numrs_hip_ctx *ctx;
  hipGraph_t graph;
  hipGraphExec_t exec;
  // blocks tensors released during the recording: the recorded kernels may
  // use them on every replay, so they return to the cache only on destroy
  std::vector<std::pair<void *, size_t>> held;
};

static void return_held(numrs_hip_ctx *ctx, std::vector<std::pair<void *, size_t>> &held) {
  for (auto &b : held) numrs_hip::block_free(ctx, b.first, b.second);
  held.clear();
}

// Destroys an instantiated graph; the context is not recording.  Returns
// whether the graph's reference was the context's last (the caller then
// deletes the destroyed context).
static bool destroy_graph(numrs_hip_graph *g) {
  numrs_hip_ctx *ctx = g->ctx;
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  return_held(ctx, g->held);
  delete g;
  if (--ctx->live_graphs == 0) numrs_hip::free_retired(ctx);
  return --ctx->live_blocks == 0 && ctx->destroyed;
}

// Runs the graph_destroy calls made while the recording that just ended was
// open.  The stream holds no replay of them: launches are refused while
// recording, and the recording's own work was never queued.
static bool run_pending_destroys(numrs_hip_ctx *ctx) {
  std::vector<numrs_hip_graph *> pending;
  pending.swap(ctx->pending_destroy);
  if (!pending.empty() && !ctx->destroyed) (void)hipStreamSynchronize(ctx->stream);
  bool last = false;
  for (numrs_hip_graph *g : pending) last = destroy_graph(g);
  return last;
}

int numrs_hip_graph_begin(numrs_hip_ctx *ctx) {
  NRS_CHECK_CTX(ctx);
  if (ctx->destroyed) return fail(ctx, NUMRS_HIP_E_INVALID, "context already destroyed");
  if (ctx->capturing)
    return fail(ctx, NUMRS_HIP_E_INVALID, "a graph is already being recorded on this context");
  NRS_HIP(ctx, hipSetDevice(ctx->device));
  NRS_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
  ctx->capturing = true;
  ctx->capture_held.clear();
  return NUMRS_HIP_OK;
}

int numrs_hip_graph_abort(numrs_hip_ctx *ctx) {
  NRS_CHECK_CTX(ctx);
  if (!ctx->capturing) return NUMRS_HIP_OK;
  ctx->capturing = false;
  hipGraph_t graph = nullptr;
  (void)hipStreamEndCapture(ctx->stream, &graph);
  (void)hipGetLastError();
  if (graph != nullptr) (void)hipGraphDestroy(graph);
  // Nothing recorded ever ran, so the held blocks are free again.
  std::vector<std::pair<void *, size_t>> held;
  held.swap(ctx->capture_held);
  return_held(ctx, held);
  if (run_pending_destroys(ctx)) delete ctx;
  return NUMRS_HIP_OK;
}

int numrs_hip_graph_end(numrs_hip_ctx *ctx, numrs_hip_graph **out) {
  NRS_CHECK_CTX(ctx);
  if (out == nullptr) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_graph_end: null out pointer");
  *out = nullptr;
  if (!ctx->capturing) return fail(ctx, NUMRS_HIP_E_INVALID, "no graph is being recorded");
  ctx->capturing = false;
  std::vector<std::pair<void *, size_t>> held;
  held.swap(ctx->capture_held);
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  if (e != hipSuccess || graph == nullptr) {
    (void)hipGetLastError();
    if (graph != nullptr) (void)hipGraphDestroy(graph);
    return_held(ctx, held);
    (void)run_pending_destroys(ctx);  // the context is not destroyed while recording
    return fail(ctx, NUMRS_HIP_E_HIP, "graph recording failed: %s", hipGetErrorString(e));
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipGraphDestroy(graph);
    return_held(ctx, held);
    (void)run_pending_destroys(ctx);
    return fail(ctx, NUMRS_HIP_E_HIP, "graph instantiation failed: %s", hipGetErrorString(e));
  }
  *out = new numrs_hip_graph{ctx, graph, exec, std::move(held)};
  ++ctx->live_blocks;  // the graph keeps the context alive, like a tensor's block
  ++ctx->live_graphs;
  (void)run_pending_destroys(ctx);  // the new graph keeps the context alive
  return NUMRS_HIP_OK;
}

int numrs_hip_graph_launch(numrs_hip_graph *g) {
  if (g == nullptr) return NUMRS_HIP_E_INVALID;
  numrs_hip_ctx *ctx = g->ctx;
  if (ctx->destroyed) return fail(ctx, NUMRS_HIP_E_INVALID, "context already destroyed");
  if (ctx->capturing)
    return fail(ctx, NUMRS_HIP_E_INVALID, "cannot replay a graph into a recording");
  NRS_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
  return NUMRS_HIP_OK;
}

int numrs_hip_graph_destroy(numrs_hip_graph *g) {
  if (g == nullptr) return NUMRS_HIP_OK;
  numrs_hip_ctx *ctx = g->ctx;
  if (ctx->capturing) {
    // A stream synchronisation would invalidate the open recording: the
    // graph is destroyed when the recording ends (or is aborted).
    ctx->pending_destroy.push_back(g);
    return NUMRS_HIP_OK;
  }
  // Queued replays finish first (a destroyed context's stream was drained).
  if (!ctx->destroyed) NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (destroy_graph(g)) delete ctx;
  return NUMRS_HIP_OK;
}

const char *numrs_hip_last_error(numrs_hip_ctx *ctx) {
  return ctx == nullptr ? "null context" : ctx->last_error;
}

int numrs_hip_device_info(numrs_hip_ctx *ctx, int *num_cus, char *arch, size_t arch_len) {
  NRS_CHECK_CTX(ctx);
  if (num_cus != nullptr) *num_cus = ctx->num_cus;
  if (arch != nullptr && arch_len > 0) {
    std::strncpy(arch, ctx->arch, arch_len - 1);
    arch[arch_len - 1] = 0;
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_malloc(numrs_hip_ctx *ctx, size_t bytes, void **dptr) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "numrs_hip_malloc");
  if (dptr == nullptr) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_malloc: null out pointer");
  *dptr = nullptr;
  NRS_HIP(ctx, hipSetDevice(ctx->device));
  if (bytes == 0) return NUMRS_HIP_OK;
  if (hipMalloc(dptr, bytes) != hipSuccess) {
    *dptr = nullptr;
    (void)hipGetLastError();
    return fail(ctx, NUMRS_HIP_E_NOMEM, "hipMalloc of %zu bytes failed", bytes);
  }
  return NUMRS_HIP_OK;
}

int numrs_hip_free(numrs_hip_ctx *ctx, void *dptr) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "numrs_hip_free");
  if (dptr == nullptr) return NUMRS_HIP_OK;
  NRS_HIP(ctx, hipFree(dptr));
  return NUMRS_HIP_OK;
}

int numrs_hip_upload(numrs_hip_ctx *ctx, void *dst, const void *host_src, size_t bytes) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "a host-to-device upload");
  if (bytes == 0) return NUMRS_HIP_OK;
  if (dst == nullptr || host_src == nullptr)
    return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_upload: null pointer");
  NRS_HIP(ctx, hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream));
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return NUMRS_HIP_OK;
}

int numrs_hip_download(numrs_hip_ctx *ctx, void *host_dst, const void *src, size_t bytes) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "a device-to-host download");
  if (bytes == 0) return NUMRS_HIP_OK;
  if (host_dst == nullptr || src == nullptr)
    return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_download: null pointer");
  NRS_HIP(ctx, hipMemcpyAsync(host_dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return numrs_hip::check_wait_status(ctx);
}

int numrs_hip_copy(numrs_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
  NRS_CHECK_CTX(ctx);
  if (bytes == 0) return NUMRS_HIP_OK;
  if (dst == nullptr || src == nullptr)
    return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_copy: null pointer");
  if (bytes % 16 == 0 && numrs_hip::aligned16(dst) && numrs_hip::aligned16(src)) {
    // a kernel of our own: safe under graph capture and visible to counters
    const int64_t n16 = (int64_t)(bytes / 16);
    unsigned grid = grid_for(n16, 256);
    if (grid > 8192) grid = 8192;
    copy_kernel<<<grid, 256, 0, ctx->stream>>>(static_cast<const float4 *>(src),
                                                static_cast<float4 *>(dst), n16);
    return numrs_hip::check_launch(ctx, "copy_kernel");
  }
  NRS_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return NUMRS_HIP_OK;
}

int numrs_hip_fill(numrs_hip_ctx *ctx, float *dst, int64_t n, float value) {
  NRS_CHECK_CTX(ctx);
  if (n < 0) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_fill: negative size");
  if (n == 0) return NUMRS_HIP_OK;
  if (dst == nullptr) return fail(ctx, NUMRS_HIP_E_INVALID, "numrs_hip_fill: null pointer");
  unsigned grid = grid_for(n, 256);
  if (grid > 65536) grid = 65536;
  fill_kernel<<<grid, 256, 0, ctx->stream>>>(dst, n, value);
  return numrs_hip::check_launch(ctx, "fill_kernel");
}

int numrs_hip_sync(numrs_hip_ctx *ctx) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "numrs_hip_sync");
  NRS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return numrs_hip::check_wait_status(ctx);
}

int numrs_hip_reserve(numrs_hip_ctx *ctx, size_t bytes) {
  NRS_CHECK_CTX(ctx);
  void *p = nullptr;
  return numrs_hip::workspace(ctx, bytes, &p);
}

void *numrs_hip_stream(numrs_hip_ctx *ctx) {
  return ctx == nullptr ? nullptr : static_cast<void *>(ctx->stream);
}

int numrs_hip_timer_record(numrs_hip_ctx *ctx, int slot) {
  NRS_CHECK_CTX(ctx);
  if (slot < 0 || slot >= kMaxTimers)
    return fail(ctx, NUMRS_HIP_E_INVALID, "timer slot %d outside [0,%d)", slot, kMaxTimers);
  NRS_HIP(ctx, hipEventRecord(ctx->events[slot], ctx->stream));
  return NUMRS_HIP_OK;
}

int numrs_hip_timer_elapsed_ms(numrs_hip_ctx *ctx, int slot_start, int slot_end, float *ms) {
  NRS_CHECK_CTX(ctx);
  NRS_NOT_RECORDING(ctx, "numrs_hip_timer_elapsed_ms");
  if (ms == nullptr || slot_start < 0 || slot_start >= kMaxTimers || slot_end < 0 ||
      slot_end >= kMaxTimers)
    return fail(ctx, NUMRS_HIP_E_INVALID, "bad timer slots %d,%d", slot_start, slot_end);
  NRS_HIP(ctx, hipEventSynchronize(ctx->events[slot_end]));
  NRS_HIP(ctx, hipEventElapsedTime(ms, ctx->events[slot_start], ctx->events[slot_end]));
  return numrs_hip::check_wait_status(ctx);
}

}  // extern "C"
