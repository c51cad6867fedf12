// p0k_runtime.cpp — the C ABI (include/p0k.h): context, buffer pool, copies, events, and the gemm / rowstats entry
// points. It stands where the reference's WebGPU runtime stands (src/core/gpu.js): one HIP device and one stream per
// context instead of a GPUDevice and its queue, hipMalloc'd buffers in a size-keyed pool instead of GPUBuffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/p0k.h"
#include "p0k_device.h"
#include "p0k_internal.h"
#include "p0k_launch.h"

namespace {

thread_local std::string g_err;

int set_err(int code, const std::string &msg) {
  g_err = msg;
  return code;
}
int hip_err(hipError_t e, const char *what) {
  return set_err(P0K_E_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}
#define HIPCHK(call, what)                   \
  do {                                       \
    hipError_t e_ = (call);                  \
    if (e_ != hipSuccess) return hip_err(e_, what); \
  } while (0)

struct PooledBuf { void *ptr; uint64_t seq; };

int scratch_setup(int device, hipStream_t s);   // the allocation-free gemm's per-device array (below)
void scratch_release(int device, const void *owner);

}  // namespace

struct p0k_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  // pool accounting, as src/core/gpu.js:33-34, 87-138: every live byte is counted; a freed buffer is kept for the next
  // request of exactly the same (16-byte rounded) size while pooled + live stays within the high-water mark + the
  // largest buffer; reused buffers are cleared before they are handed out again.
  std::unordered_map<void *, uint64_t> live;
  std::map<uint64_t, std::vector<PooledBuf>> pool;
  uint64_t alive = 0, peak = 0, pooled = 0, hw = 0, max_buf = 0, seq = 0;
  uint64_t creates = 0, reuses = 0, evictions = 0, pooled_n = 0;
  uint64_t cap() const { return hw + max_buf; }
  // workspace of the split-K decode GEMV: fp32 partial tiles (grown on demand) and one arrival counter per 128-column
  // tile (zeroed once here; every call leaves them at zero again)
  float *ws_part = nullptr;
  uint64_t ws_part_bytes = 0;
  uint32_t *ws_cnt = nullptr;
  static constexpr uint32_t WS_COUNTERS = 1u << 16;
  // X' of the rms / lnmod prologues for the load-to-LDS GEMM (M x K fp16, grown on demand)
  void *ws_x = nullptr;
  uint64_t ws_x_bytes = 0;
  // 256 zero bytes: the padding taps of the load-to-LDS conv3 gather read them
  void *ws_zero = nullptr;
  // workspaces replaced by larger ones while a graph captured after their allocation may still address them: freed
  // only with the context. graph_epoch counts the graphs captured on the stream; a workspace allocated in the current
  // epoch is in no graph and is freed as soon as it is replaced. Workspaces grow to powers of two, so the retired
  // ones add up to less than the live one.
  std::vector<void *> ws_retired;
  uint64_t graph_epoch = 0, ws_part_epoch = 0, ws_x_epoch = 0;
  // this context called p0k_gemm_noalloc and holds its device's scratch array until it is destroyed
  bool owns_scratch = false;
  // CU count of the device and the P0K_* tuning switches, read at creation and by p0k_ctx_reload_env
  p0k::Tuning tune;
};

struct p0k_event { hipEvent_t ev; int device; };

extern "C" {

int p0k_abi_version(void) { return P0K_ABI_VERSION; }
const char *p0k_last_error(void) { return g_err.c_str(); }

int p0k_ctx_create(int device, p0k_ctx **out) {
  if (!out) return set_err(P0K_E_ARG, "ctx_create: out is NULL");
  *out = nullptr;
  int n = 0;
  HIPCHK(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (device < 0 || device >= n) return set_err(P0K_E_ARG, "ctx_create: no HIP device " + std::to_string(device));
  HIPCHK(hipSetDevice(device), "hipSetDevice");
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_err(P0K_E_UNSUPPORTED, std::string("ctx_create: this library is built for gfx950, the device is ") + prop.gcnArchName);
  p0k_ctx *c = new p0k_ctx();
  c->device = device;
  c->tune = p0k::tuning_from_env((unsigned)prop.multiProcessorCount);
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) { delete c; return hip_err(e, "hipStreamCreate"); }
  e = hipMalloc((void **)&c->ws_cnt, sizeof(uint32_t) * p0k_ctx::WS_COUNTERS);
  if (e == hipSuccess) e = hipMemset(c->ws_cnt, 0, sizeof(uint32_t) * p0k_ctx::WS_COUNTERS);
  if (e == hipSuccess) e = hipMalloc(&c->ws_zero, 256);
  if (e == hipSuccess) e = hipMemset(c->ws_zero, 0, 256);
  if (e != hipSuccess) {
    if (c->ws_cnt) (void)hipFree(c->ws_cnt);
    if (c->ws_zero) (void)hipFree(c->ws_zero);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return hip_err(e, "workspace counters");
  }
  if (int rs = scratch_setup(device, c->stream)) {
    p0k_ctx_destroy(c);
    return rs;
  }
  *out = c;
  return P0K_OK;
}

void p0k_ctx_destroy(p0k_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->owns_scratch) scratch_release(c->device, c);
  for (auto &kv : c->live) (void)hipFree(kv.first);
  for (auto &kv : c->pool)
    for (auto &b : kv.second) (void)hipFree(b.ptr);
  if (c->ws_part) (void)hipFree(c->ws_part);
  if (c->ws_x) (void)hipFree(c->ws_x);
  if (c->ws_zero) (void)hipFree(c->ws_zero);
  if (c->ws_cnt) (void)hipFree(c->ws_cnt);
  for (void *p : c->ws_retired) (void)hipFree(p);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

int p0k_ctx_reload_env(p0k_ctx *c) {
  if (!c) return set_err(P0K_E_ARG, "ctx_reload_env: NULL context");
  std::lock_guard<std::mutex> lk(c->mu);
  c->tune = p0k::tuning_from_env(c->tune.cus);
  return P0K_OK;
}

int p0k_ctx_cus(p0k_ctx *c) { return c ? (int)c->tune.cus : 0; }

void *p0k_ctx_stream(p0k_ctx *c) { return c ? (void *)c->stream : nullptr; }

int p0k_device_info_get(p0k_ctx *c, p0k_device_info *out) {
  if (!c || !out) return set_err(P0K_E_ARG, "device_info: NULL argument");
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties");
  memset(out, 0, sizeof *out);
  snprintf(out->name, sizeof out->name, "%s", prop.name);
  if (!out->name[0])   // some drivers report no marketing name: name the device by its ISA and size instead
    snprintf(out->name, sizeof out->name, "AMD %.16s, %d CUs, %zu GiB", prop.gcnArchName, prop.multiProcessorCount,
             (size_t)(prop.totalGlobalMem >> 30));
  snprintf(out->arch, sizeof out->arch, "%s", prop.gcnArchName);
  out->cus = prop.multiProcessorCount;
  out->xcds_hint = 8;
  out->hbm_bytes = prop.totalGlobalMem;
  out->clock_khz = prop.clockRate;
  out->mem_clock_khz = prop.memoryClockRate;
  out->mem_bus_width = prop.memoryBusWidth;
  return P0K_OK;
}

// ------------------------------------------------------------------------------------------------ buffers
static void evict(p0k_ctx *c, uint64_t room) {     // release pooled buffers, oldest first, until at most `room` pooled
  while (c->pooled > room) {
    uint64_t best_size = 0; size_t best_i = 0; uint64_t best_seq = UINT64_MAX;
    for (auto &kv : c->pool)
      for (size_t i = 0; i < kv.second.size(); i++)
        if (kv.second[i].seq < best_seq) { best_seq = kv.second[i].seq; best_size = kv.first; best_i = i; }
    if (best_seq == UINT64_MAX) break;
    auto &v = c->pool[best_size];
    (void)hipFree(v[best_i].ptr);
    v.erase(v.begin() + best_i);
    if (v.empty()) c->pool.erase(best_size);
    c->pooled -= best_size; c->pooled_n--; c->evictions++;
  }
}

// alloc / free queue a clear or call hipFree: neither belongs in a graph being captured on the context's stream
static int refuse_capture(p0k_ctx *c, const char *what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIPCHK(hipStreamIsCapturing(c->stream, &cs), "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return set_err(P0K_E_ARG, std::string(what) + ": not allowed while the context's stream is captured into a graph "
                                                  "(allocate and free buffers before p0k_graph_begin or after p0k_graph_end)");
  return P0K_OK;
}

int p0k_alloc(p0k_ctx *c, uint64_t bytes, void **out) {
  if (!c || !out) return set_err(P0K_E_ARG, "alloc: NULL argument");
  *out = nullptr;
  std::lock_guard<std::mutex> lk(c->mu);
  if (int r = refuse_capture(c, "alloc")) return r;
  uint64_t size = std::max<uint64_t>(16, (bytes + 15) / 16 * 16);
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  auto it = c->pool.find(size);
  if (it != c->pool.end() && !it->second.empty()) {
    void *p = it->second.back().ptr;
    it->second.pop_back();
    if (it->second.empty()) c->pool.erase(it);
    c->pooled -= size; c->pooled_n--; c->reuses++;
    HIPCHK(hipMemsetAsync(p, 0, size, c->stream), "hipMemsetAsync");   // cleared like a new buffer (gpu.js:96-97)
    c->live[p] = size; c->alive += size;
    c->peak = std::max(c->peak, c->alive); c->hw = std::max(c->hw, c->alive);
    *out = p;
    return P0K_OK;
  }
  uint64_t cap = std::max(c->cap(), c->alive + size);
  evict(c, cap - c->alive - size);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) {
    evict(c, 0);                                   // retry once with the pool drained
    e = hipMalloc(&p, size);
    if (e != hipSuccess) return set_err(P0K_E_NOMEM, "alloc: hipMalloc(" + std::to_string(size) + ") failed: " + hipGetErrorString(e));
  }
  HIPCHK(hipMemsetAsync(p, 0, size, c->stream), "hipMemsetAsync");
  c->live[p] = size; c->alive += size; c->creates++;
  c->max_buf = std::max(c->max_buf, size);
  c->peak = std::max(c->peak, c->alive); c->hw = std::max(c->hw, c->alive);
  *out = p;
  return P0K_OK;
}

int p0k_free(p0k_ctx *c, void *p) {
  if (!c) return set_err(P0K_E_ARG, "free: NULL context");
  if (!p) return P0K_OK;
  std::lock_guard<std::mutex> lk(c->mu);
  if (int r = refuse_capture(c, "free")) return r;
  auto it = c->live.find(p);
  if (it == c->live.end()) return set_err(P0K_E_ARG, "free: not a live buffer of this context");
  uint64_t size = it->second;
  c->live.erase(it);
  c->alive -= size;
  // a pooled buffer is only handed out again through p0k_alloc, whose clear is queued on the same stream after any
  // work still reading it, so no wait is needed here
  if (c->alive + c->pooled + size <= c->cap()) {
    c->pool[size].push_back({p, ++c->seq});
    c->pooled += size; c->pooled_n++;
    return P0K_OK;
  }
  HIPCHK(hipFree(p), "hipFree");
  return P0K_OK;
}

int p0k_drain_pool(p0k_ctx *c) {
  if (!c) return set_err(P0K_E_ARG, "drain_pool: NULL context");
  std::lock_guard<std::mutex> lk(c->mu);
  HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  evict(c, 0);
  return P0K_OK;
}

int p0k_pool_stats_get(p0k_ctx *c, p0k_pool_stats *s) {
  if (!c || !s) return set_err(P0K_E_ARG, "pool_stats: NULL argument");
  std::lock_guard<std::mutex> lk(c->mu);
  s->alive = c->alive; s->peak = c->peak; s->pooled = c->pooled; s->high_water = c->hw; s->max_buf = c->max_buf;
  s->creates = c->creates; s->reuses = c->reuses; s->evictions = c->evictions;
  s->live_buffers = c->live.size(); s->pooled_buffers = c->pooled_n;
  return P0K_OK;
}

static int check_range(p0k_ctx *c, const void *buf, uint64_t off, uint64_t n, const char *what) {
  auto it = c->live.find(const_cast<void *>(buf));
  if (it == c->live.end()) return set_err(P0K_E_ARG, std::string(what) + ": not a live buffer of this context");
  if (off > it->second || n > it->second - off)
    return set_err(P0K_E_ARG, std::string(what) + ": range [" + std::to_string(off) + ", +" + std::to_string(n) +
                                  ") outside the buffer of " + std::to_string(it->second) + " bytes");
  return P0K_OK;
}

int p0k_upload(p0k_ctx *c, void *dst, uint64_t off, const void *src, uint64_t n) {
  if (!c || !dst || (!src && n)) return set_err(P0K_E_ARG, "upload: NULL argument");
  {
    std::lock_guard<std::mutex> lk(c->mu);
    if (int r = check_range(c, dst, off, n, "upload")) return r;
  }
  if (!n) return P0K_OK;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  HIPCHK(hipMemcpyAsync((uint8_t *)dst + off, src, n, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync H2D");
  HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");   // the host memory may be reused on return
  return P0K_OK;
}

int p0k_download(p0k_ctx *c, const void *src, uint64_t off, void *dst, uint64_t n) {
  if (!c || !src || (!dst && n)) return set_err(P0K_E_ARG, "download: NULL argument");
  {
    std::lock_guard<std::mutex> lk(c->mu);
    if (int r = check_range(c, src, off, n, "download")) return r;
  }
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  if (n) HIPCHK(hipMemcpyAsync(dst, (const uint8_t *)src + off, n, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync D2H");
  HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return P0K_OK;
}

int p0k_copy(p0k_ctx *c, void *dst, uint64_t doff, const void *src, uint64_t soff, uint64_t n) {
  if (!c || !dst || !src) return set_err(P0K_E_ARG, "copy: NULL argument");
  {
    std::lock_guard<std::mutex> lk(c->mu);
    if (int r = check_range(c, dst, doff, n, "copy dst")) return r;
    if (int r = check_range(c, src, soff, n, "copy src")) return r;
  }
  if (!n) return P0K_OK;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  HIPCHK(hipMemcpyAsync((uint8_t *)dst + doff, (const uint8_t *)src + soff, n, hipMemcpyDeviceToDevice, c->stream),
         "hipMemcpyAsync D2D");
  return P0K_OK;
}

int p0k_sync(p0k_ctx *c) {
  if (!c) return set_err(P0K_E_ARG, "sync: NULL context");
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return P0K_OK;
}

// ------------------------------------------------------------------------------------------------ the op
int p0k_gemm_check(const p0k_gemm_args *a) {
  std::string err;
  int r = p0k::prepare_gemm(a, nullptr, nullptr, &err, p0k::tuning_from_env(256));
  if (r) return set_err(r, err);
  return P0K_OK;
}

double p0k_gemm_flops(const p0k_gemm_args *a) { return a ? 2.0 * a->M * a->N * a->K : 0.0; }

int p0k_gemm_plan(p0k_ctx *c, const p0k_gemm_args *a, p0k_tile *out) {
  if (!c) return set_err(P0K_E_ARG, "gemm_plan: NULL context");
  p0k::Tuning tune;
  {
    std::lock_guard<std::mutex> lk(c->mu);
    tune = c->tune;
  }
  std::string err;
  p0k::Plan plan;
  int r = p0k::prepare_gemm(a, nullptr, &plan, &err, tune);
  if (r) return set_err(r, err);
  if (out) { out->bm = plan.bm; out->bn = plan.bn; out->kernel = plan.kernel; }
  return P0K_OK;
}

int p0k_select_tile(const p0k_gemm_args *a, p0k_tile *out) {
  std::string err;
  p0k::Plan plan;
  int r = p0k::prepare_gemm(a, nullptr, &plan, &err, p0k::tuning_from_env(256));
  if (r) return set_err(r, err);
  if (out) { out->bm = plan.bm; out->bn = plan.bn; out->kernel = plan.kernel; }
  return P0K_OK;
}

// every operand must be a live buffer of this context, and its stated size must lie inside the allocation
static int check_operand(p0k_ctx *c, const void *buf, uint64_t size, const char *what) {
  if (!buf) return P0K_OK;
  auto it = c->live.find(const_cast<void *>(buf));
  if (it == c->live.end()) return set_err(P0K_E_ARG, std::string("gemm: ") + what + " is not a live buffer of this context");
  if (size > it->second)
    return set_err(P0K_E_ARG, std::string("gemm: ") + what + " size " + std::to_string(size) + " exceeds its allocation of " +
                                  std::to_string(it->second) + " bytes");
  return P0K_OK;
}

// grow a workspace of the context to at least `need` bytes, rounded up to a power of two (not while the stream is
// being captured into a graph). The buffer it replaces is freed after the stream has drained when no graph was
// captured since it was allocated; otherwise it is kept until the context goes, since replaying such a graph still
// addresses it.
static int grow_ws(p0k_ctx *c, void **buf, uint64_t *bytes, uint64_t *epoch, uint64_t need, const char *what) {
  std::lock_guard<std::mutex> lk(c->mu);
  if (need <= *bytes) return P0K_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIPCHK(hipStreamIsCapturing(c->stream, &cs), "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return set_err(P0K_E_ARG, std::string("gemm: the ") + what + " workspace must grow (" + std::to_string(need) +
                                  " bytes): make one call of this shape before capturing a graph");
  uint64_t size = 256;
  while (size < need) size <<= 1;
  void *old = *buf;
  if (old && *epoch == c->graph_epoch) {        // in no graph: free it first, so its memory can serve the new one
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    HIPCHK(hipFree(old), "hipFree");
    old = nullptr;
    *buf = nullptr;
    *bytes = 0;
  }
  void *nb = nullptr;
  hipError_t me = hipMalloc(&nb, size);
  if (me != hipSuccess) return set_err(P0K_E_NOMEM, std::string("gemm: ") + what + " workspace of " + std::to_string(size) + " bytes");
  if (old) c->ws_retired.push_back(old);
  *buf = nb;
  *bytes = size;
  *epoch = c->graph_epoch;
  return P0K_OK;
}

int p0k_ctx_workspace_stats(p0k_ctx *c, uint64_t *live_bytes, uint64_t *retired_buffers) {
  if (!c) return set_err(P0K_E_ARG, "workspace_stats: NULL context");
  std::lock_guard<std::mutex> lk(c->mu);
  if (live_bytes) *live_bytes = c->ws_part_bytes + c->ws_x_bytes;
  if (retired_buffers) *retired_buffers = c->ws_retired.size();
  return P0K_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------ scratch
// The allocation-free gemm (p0k_gemm_noalloc) takes every workspace from this array instead of the context's grown
// buffers. Layout: [0, 256 KiB) one arrival counter per 128-column tile of the split decode (zero between calls:
// the last item of a tile resets its counter), [256 KiB, +256) the zero block the conv3 gather's padding taps read,
// [512 KiB, 32 MiB) either the split decode's fp32 partials or the rms / lnmod / PixelNorm X' of one call. Each
// device holds its own copy; host code reaches it only through the address hipGetSymbolAddress returns for that
// device (the array's name on the host is a stand-in, not a device address).
static constexpr uint64_t SCRATCH_BYTES = 32ull << 20, SCRATCH_CNT = 0, SCRATCH_ZERO = 256ull << 10,
                          SCRATCH_WS = 512ull << 10;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[MAX_DEVICES];
const void *g_scratch_owner[MAX_DEVICES];   // the context whose p0k_gemm_noalloc calls use the array (one at a time)

__global__ void k_zero_words(uint32_t *p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// once per device, with that device current and from a context's set-up (not under graph capture): resolve the
// device address of `scratch` and clear its counters and zero block with a fill kernel
int scratch_setup(int device, hipStream_t s) {
  if (device < 0 || device >= MAX_DEVICES) return set_err(P0K_E_UNSUPPORTED, "scratch: device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device]) return P0K_OK;
  void *ptr = nullptr;
  HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  const uint32_t words = (uint32_t)((SCRATCH_ZERO + 256) / 4);
  hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, s, (uint32_t *)ptr, words);
  HIPCHK(hipGetLastError(), "scratch clear launch");
  HIPCHK(hipStreamSynchronize(s), "hipStreamSynchronize");
  g_scratch_ptr[device] = (uint8_t *)ptr;
  return P0K_OK;
}
void scratch_release(int device, const void *owner) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (device >= 0 && device < MAX_DEVICES && g_scratch_owner[device] == owner) g_scratch_owner[device] = nullptr;
}
}  // namespace

// Where one call's workspaces come from: the context's buffers, grown on demand (p0k_gemm), or the device's scratch
// array, refused when too small (p0k_gemm_noalloc).
struct WsSource {
  p0k_ctx *c;
  uint8_t *scratch;   // non-null: the allocation-free path
  int part(uint64_t need, float **out) {
    if (scratch) {
      if (need > SCRATCH_BYTES - SCRATCH_WS)
        return set_err(P0K_E_ARG, "gemm_noalloc: the split decode needs " + std::to_string(need) +
                                      " bytes of partials, the scratch array holds " +
                                      std::to_string(SCRATCH_BYTES - SCRATCH_WS));
      *out = (float *)(scratch + SCRATCH_WS);
      return P0K_OK;
    }
    if (int r = grow_ws(c, (void **)&c->ws_part, &c->ws_part_bytes, &c->ws_part_epoch, need, "decode")) return r;
    *out = c->ws_part;
    return P0K_OK;
  }
  int xws(uint64_t need, void **out) {
    if (scratch) {
      if (need > SCRATCH_BYTES - SCRATCH_WS)
        return set_err(P0K_E_ARG, "gemm_noalloc: the prologue needs " + std::to_string(need) +
                                      " bytes of X', the scratch array holds " + std::to_string(SCRATCH_BYTES - SCRATCH_WS));
      *out = scratch + SCRATCH_WS;
      return P0K_OK;
    }
    if (int r = grow_ws(c, &c->ws_x, &c->ws_x_bytes, &c->ws_x_epoch, need, "prologue")) return r;
    *out = c->ws_x;
    return P0K_OK;
  }
  uint32_t *counters() { return scratch ? (uint32_t *)(scratch + SCRATCH_CNT) : c->ws_cnt; }
  const void *zero() { return scratch ? (const void *)(scratch + SCRATCH_ZERO) : c->ws_zero; }
};

static int gemm_run(p0k_ctx *c, const p0k_gemm_args *a, WsSource ws) {
  if (!c) return set_err(P0K_E_ARG, "gemm: NULL context");
  std::string err;
  p0k::Params p;
  p0k::Plan plan;
  p0k::Tuning tune;
  {
    std::lock_guard<std::mutex> lk(c->mu);
    tune = c->tune;
  }
  int r = p0k::prepare_gemm(a, &p, &plan, &err, tune);
  if (r) return set_err(r, err);
  {
    std::lock_guard<std::mutex> lk(c->mu);
    const struct { const void *b; uint64_t s; const char *n; } ops[] = {
        {a->w_buf, a->w_off + a->w_bytes, "w"}, {a->x_buf, a->x_size, "x"}, {a->y_buf, a->y_size, "y"},
        {a->ev_buf, a->ev_size, "ev"}, {a->st_buf, a->st_size, "stats"}, {a->pv_buf, a->pv_size, "pv"},
        {a->bv_buf, a->bv_size, "bv"}, {a->gt_buf, a->gt_size, "gt"}, {a->rope_buf, a->rope_size, "rope"}};
    for (auto &o : ops)
      if (int rr = check_operand(c, o.b, o.s, o.n)) return rr;
  }
  if (a->M == 0 || a->N == 0) return P0K_OK;
  {
    // a call enqueued while the stream is being captured (p0k_graph_begin, or a caller's own capture of
    // p0k_ctx_stream) may put the current workspaces into a graph: from here on they are kept when replaced
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIPCHK(hipStreamIsCapturing(c->stream, &cs), "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone) {
      std::lock_guard<std::mutex> lk(c->mu);
      c->graph_epoch++;
    }
  }
  p.W = (const uint8_t *)a->w_buf + a->w_off;
  p.X = (const uint8_t *)a->x_buf + a->x_off;
  p.Y = (uint8_t *)a->y_buf + a->y_off;
  p.ST = a->st_buf; p.PV = a->pv_buf; p.EV = a->ev_buf; p.BV = a->bv_buf; p.RP = a->rope_buf;
  p.GT = (const uint16_t *)a->gt_buf;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  hipError_t e;
  if (plan.kernel == p0k::K_GEMV_SN) {
    e = p0k::launch_gemv_sn(p, plan.we, plan.xm, c->stream);
  } else if (plan.kernel == p0k::K_GEMV || plan.kernel == p0k::K_GEMV_MF) {
    const uint32_t tiles = (a->N + 127) / 128;
    float *part = nullptr;
    if (plan.S > 1) {
      if (tiles > p0k_ctx::WS_COUNTERS) return set_err(P0K_E_UNSUPPORTED, "gemm: N too large for the decode workspace");
      const uint64_t need = (uint64_t)plan.S * a->M * tiles * 128u * sizeof(float);
      if (need >= (1ull << 32)) return set_err(P0K_E_UNSUPPORTED, "gemm: decode split workspace of 4 GiB or more");
      if (int rr = ws.part(need, &part)) return rr;
    }
    e = p0k::launch_gemv(p, plan.we, plan.xm, part, ws.counters(), plan.S, plan.KS, c->stream, plan.kernel == p0k::K_GEMV_MF,
                          tune.gemv_mq4, plan.mx, plan.narrow);
  } else if (plan.kernel == p0k::K_MFMA_DMA && plan.xm == P0K_X_CONV3) {
    p.Z = (const uint8_t *)ws.zero();
    if (p.flags & p0k::F_PN) {
      // PixelNorm + SiLU once per input element into the X' workspace; the gather then reads plain fp16 voxels
      const uint64_t need = (uint64_t)p.nvox * p.Ci * 2u;
      void *xw = nullptr;
      if (int rr = ws.xws(need, &xw)) return rr;
      e = p0k::launch_xprep(p, plan.xm, (uint16_t *)xw, c->stream);
      if (e != hipSuccess) return hip_err(e, "gemm prologue launch");
      p.X = (const uint8_t *)xw;
    }
    e = p0k::launch_gemm_dma(p, plan.we, P0K_X_CONV3, plan.bm, plan.bn, tune.cus, false, c->stream);
  } else if (plan.kernel == p0k::K_MFMA_DMA) {
    if (plan.xm != P0K_X_F16) {
      // the prologue once per element into the X' workspace; the GEMM then reads fp16 rows
      const uint64_t need = (uint64_t)a->M * a->K * 2u;
      void *xw = nullptr;
      if (int rr = ws.xws(need, &xw)) return rr;
      e = p0k::launch_xprep(p, plan.xm, (uint16_t *)xw, c->stream);
      if (e != hipSuccess) return hip_err(e, "gemm prologue launch");
      p.X = (const uint8_t *)xw;
      p.ldx = a->K;
      p.kx0 = 0;
    }
    e = p0k::launch_gemm_dma(p, plan.we, P0K_X_F16, plan.bm, plan.bn, tune.cus, tune.dma_tail, c->stream);
  } else {
    e = p0k::launch_gemm_mfma(p, plan.we, plan.xm, plan.bm, plan.bn, c->stream);
  }
  if (e != hipSuccess) return hip_err(e, "gemm launch");
  return P0K_OK;
}

extern "C" {

int p0k_gemm(p0k_ctx *c, const p0k_gemm_args *a) { return gemm_run(c, a, WsSource{c, nullptr}); }

int p0k_gemm_noalloc(p0k_ctx *c, const p0k_gemm_args *a) {
  if (!c) return set_err(P0K_E_ARG, "gemm_noalloc: NULL context");
  uint8_t *sp;
  {
    // the first context to call takes the device's array and keeps it until it is destroyed: calls of another
    // context (another stream) could overlap with its calls on the GPU and corrupt each other's partials and
    // counters, so they are refused
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    sp = (c->device >= 0 && c->device < MAX_DEVICES) ? g_scratch_ptr[c->device] : nullptr;
    if (sp) {
      if (g_scratch_owner[c->device] && g_scratch_owner[c->device] != c)
        return set_err(P0K_E_ARG, "gemm_noalloc: the scratch array of device " + std::to_string(c->device) +
                                      " is held by another live context (one context per device may use it)");
      g_scratch_owner[c->device] = c;
      c->owns_scratch = true;
    }
  }
  if (!sp) return set_err(P0K_E_UNSUPPORTED, "gemm_noalloc: the scratch array of this device is not set up");
  return gemm_run(c, a, WsSource{c, sp});
}

uint64_t p0k_gemm_noalloc_scratch_bytes(void) { return SCRATCH_BYTES - SCRATCH_WS; }

int p0k_rowstats_check(const p0k_rowstats_args *a) {
  std::string err;
  int r = p0k::prepare_rowstats(a, &err);
  if (r) return set_err(r, err);
  return P0K_OK;
}

int p0k_rowstats(p0k_ctx *c, const p0k_rowstats_args *a) {
  if (!c) return set_err(P0K_E_ARG, "rowstats: NULL context");
  std::string err;
  int r = p0k::prepare_rowstats(a, &err);
  if (r) return set_err(r, err);
  {
    std::lock_guard<std::mutex> lk(c->mu);
    auto x = c->live.find(const_cast<void *>(a->x_buf)), s = c->live.find(a->st_buf);
    if (x == c->live.end() || s == c->live.end()) return set_err(P0K_E_ARG, "rowstats: x / st are not live buffers of this context");
    if (a->x_size > x->second || a->st_size > s->second) return set_err(P0K_E_ARG, "rowstats: a size exceeds its allocation");
  }
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  hipError_t e = p0k::launch_rowstats((const uint8_t *)a->x_buf + a->x_off, a->ld ? a->ld : a->cols, a->c0, a->rows,
                                      a->cols, a->mode, a->eps, a->st_buf, a->st_off, c->stream);
  if (e != hipSuccess) return hip_err(e, "rowstats launch");
  return P0K_OK;
}

// ------------------------------------------------------------------------------------------------ pixstats / GroupNorm
static int check_live(p0k_ctx *c, const void *buf, uint64_t size, const char *op, const char *what) {
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->live.find(const_cast<void *>(buf));
  if (it == c->live.end()) return set_err(P0K_E_ARG, std::string(op) + ": " + what + " is not a live buffer of this context");
  if (size > it->second) return set_err(P0K_E_ARG, std::string(op) + ": " + what + " size exceeds its allocation");
  return P0K_OK;
}

int p0k_pixstats(p0k_ctx *c, const p0k_pixstats_args *a) {
  if (!c) return set_err(P0K_E_ARG, "pixstats: NULL context");
  std::string err;
  int r = p0k::prepare_pixstats(a, &err);
  if (r) return set_err(r, err);
  if ((r = check_live(c, a->x_buf, a->x_size, "pixstats", "x")) || (r = check_live(c, a->r_buf, a->r_size, "pixstats", "r")))
    return r;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  hipError_t e = p0k::launch_pixstats((const uint8_t *)a->x_buf + a->x_off, a->V, a->C, a->eps != 0.0f ? a->eps : 1e-8f,
                                      a->r_buf + a->ro, c->stream);
  if (e != hipSuccess) return hip_err(e, "pixstats launch");
  return P0K_OK;
}

int p0k_attention_check(const p0k_attn_args *a) {
  std::string err;
  int r = p0k::prepare_attention(a, nullptr, &err);
  if (r) return set_err(r, err);
  return P0K_OK;
}

double p0k_attention_flops(const p0k_attn_args *a) {
  if (!a) return 0.0;
  const double Lk = a->Lk ? a->Lk : a->Lq;
  return 4.0 * a->Lq * Lk * 128.0 * a->Hq;
}

int p0k_attention(p0k_ctx *c, const p0k_attn_args *a) {
  if (!c) return set_err(P0K_E_ARG, "attention: NULL context");
  std::string err;
  p0k::AttnParams p;
  int r = p0k::prepare_attention(a, &p, &err);
  if (r) return set_err(r, err);
  if ((r = check_live(c, a->q_buf, a->q_size, "attention", "q")) || (r = check_live(c, a->k_buf, a->k_size, "attention", "k")) ||
      (r = check_live(c, a->v_buf, a->v_size, "attention", "v")) || (r = check_live(c, a->o_buf, a->o_size, "attention", "o")))
    return r;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  hipError_t e = p0k::launch_attention(p, (int)c->tune.cus, c->tune.attn_bq, c->stream);
  if (e != hipSuccess) return hip_err(e, "attention launch");
  return P0K_OK;
}

uint64_t p0k_gn_part_bytes(uint32_t pix) { return (uint64_t)((pix + 63) / 64) * 512; }

static int gn_run(p0k_ctx *c, const p0k_gn_args *a, int what, uint32_t *nwg_out) {
  if (!c) return set_err(P0K_E_ARG, "groupnorm: NULL context");
  std::string err;
  int r = p0k::prepare_gn(a, what, &err);
  if (r) return set_err(r, err);
  if ((r = check_live(c, a->part_buf, a->part_size, "groupnorm", "part"))) return r;
  if ((what & 1) && (r = check_live(c, a->x_buf, a->x_size, "groupnorm", "x"))) return r;
  if ((what & 2) && ((r = check_live(c, a->gb_buf, a->gb_size, "groupnorm", "gb")) ||
                     (r = check_live(c, a->ab_buf, a->ab_size, "groupnorm", "ab"))))
    return r;
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  const uint32_t nwg = (a->pix + 63) / 64;
  if (what & 1) {
    hipError_t e = p0k::launch_gn_partial((const uint8_t *)a->x_buf + a->x_off, a->pix, a->C, a->part_buf, a->wg_off, c->stream);
    if (e != hipSuccess) return hip_err(e, "groupnorm partial launch");
  }
  if (what & 2) {
    const uint32_t n = (what & 1) ? a->wg_off + nwg : (a->nwg ? a->nwg : nwg);
    const float *gb = a->gb_buf;
    hipError_t e = p0k::launch_gn_finalize(a->part_buf, n, a->C, a->eps != 0.0f ? a->eps : 1e-6f,
                                           (const float *)((const uint8_t *)gb + a->g_off),
                                           (const float *)((const uint8_t *)gb + a->b_off), a->ab_buf + a->ab_off, c->stream);
    if (e != hipSuccess) return hip_err(e, "groupnorm finalize launch");
  }
  if (nwg_out) *nwg_out = nwg;
  return P0K_OK;
}

int p0k_gn_partial(p0k_ctx *c, const p0k_gn_args *a, uint32_t *nwg_out) { return gn_run(c, a, 1, nwg_out); }
int p0k_gn_finalize(p0k_ctx *c, const p0k_gn_args *a) { return gn_run(c, a, 2, nullptr); }
int p0k_groupnorm_stats(p0k_ctx *c, const p0k_gn_args *a) { return gn_run(c, a, 3, nullptr); }

// ------------------------------------------------------------------------------------------------ graphs
struct p0k_graph { hipGraph_t graph; hipGraphExec_t exec; };

int p0k_graph_begin(p0k_ctx *c) {
  if (!c) return set_err(P0K_E_ARG, "graph_begin: NULL context");
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  return P0K_OK;
}
int p0k_graph_end(p0k_ctx *c, p0k_graph **out) {
  if (!c || !out) return set_err(P0K_E_ARG, "graph_end: NULL argument");
  *out = nullptr;
  hipGraph_t g = nullptr;
  HIPCHK(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture");
  {
    std::lock_guard<std::mutex> lk(c->mu);
    c->graph_epoch++;                  // the workspaces now in use may be addressed by this graph
  }
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) { (void)hipGraphDestroy(g); return hip_err(e, "hipGraphInstantiate"); }
  *out = new p0k_graph{g, ex};
  return P0K_OK;
}
int p0k_graph_launch(p0k_ctx *c, p0k_graph *g) {
  if (!c || !g) return set_err(P0K_E_ARG, "graph_launch: NULL argument");
  HIPCHK(hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
  return P0K_OK;
}
void p0k_graph_destroy(p0k_graph *g) {
  if (!g) return;
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  delete g;
}

// ------------------------------------------------------------------------------------------------ events
int p0k_event_create(p0k_ctx *c, p0k_event **out) {
  if (!c || !out) return set_err(P0K_E_ARG, "event_create: NULL argument");
  HIPCHK(hipSetDevice(c->device), "hipSetDevice");
  p0k_event *ev = new p0k_event();
  ev->device = c->device;
  hipError_t e = hipEventCreate(&ev->ev);
  if (e != hipSuccess) { delete ev; return hip_err(e, "hipEventCreate"); }
  *out = ev;
  return P0K_OK;
}
int p0k_event_record(p0k_ctx *c, p0k_event *ev) {
  if (!c || !ev) return set_err(P0K_E_ARG, "event_record: NULL argument");
  HIPCHK(hipEventRecord(ev->ev, c->stream), "hipEventRecord");
  return P0K_OK;
}
int p0k_event_elapsed_ms(p0k_event *a, p0k_event *b, float *ms) {
  if (!a || !b || !ms) return set_err(P0K_E_ARG, "event_elapsed: NULL argument");
  HIPCHK(hipEventSynchronize(b->ev), "hipEventSynchronize");
  HIPCHK(hipEventElapsedTime(ms, a->ev, b->ev), "hipEventElapsedTime");
  return P0K_OK;
}
void p0k_event_destroy(p0k_event *ev) {
  if (!ev) return;
  (void)hipEventDestroy(ev->ev);
  delete ev;
}

}  // extern "C"
