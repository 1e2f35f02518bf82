// Context, stream-ordered memory pool, transfers, events and errors.
//
// One context = one device + one HIP stream (default priority).  Device
// memory comes from a size-class pool: freed blocks go back to a free list
// and are handed out again to later work on the same stream, which is safe
// because the stream executes in order.  This replaces the reference
// WebGPU runtime's buffer pool (backend-webgpu/src/runtime.ts:51-57,167-201)
// without its write-hazard flushes: a single in-order stream has none.
#include <math.h>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <stdexcept>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace hb {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": launch failed: " + hipGetErrorString(e));
}

struct Staging {
  void* host = nullptr;  // pinned
  size_t cap = 0;
  hipEvent_t done = nullptr;  // recorded after the copy that last read it
  bool pending = false;
};

struct Context {
  int device = 0;
  int cus = 0;  // compute units of the device
  hipStream_t stream = nullptr;
  std::map<size_t, std::vector<void*>> free_list;  // size class -> blocks
  std::unordered_map<void*, size_t> live;            // block -> size class
  uint64_t live_bytes = 0, cached_bytes = 0;
  Staging staging[2];
  int next_staging = 0;
  // RoPE cos/sin tables [L][D/2] (float2), keyed by (L, D, base)
  std::map<std::tuple<int64_t, int64_t, double>, void*> rope_tables;
  // stream capture: blocks freed while capturing stay out of the free list
  // (a replay still writes them) until their graph is destroyed
  bool capturing = false;
  std::vector<void*> held;
  std::map<void*, std::vector<void*>> graph_held;  // hipGraphExec_t -> held blocks
};

static size_t size_class(size_t bytes) {
  // 256-byte granularity up to 64 KiB, then steps of 1/16 of the next power of two
  if (bytes == 0) bytes = 1;
  if (bytes <= 65536) return (bytes + 255) & ~(size_t)255;
  size_t p = 1;
  while (p < bytes) p <<= 1;
  size_t step = p / 16;
  return (bytes + step - 1) / step * step;
}

static Context* C(uintptr_t ctx) {
  if (!ctx) throw std::runtime_error("null context");
  return reinterpret_cast<Context*>(ctx);
}

hipStream_t stream_of(uintptr_t ctx) { return C(ctx)->stream; }
int device_of(uintptr_t ctx) { return C(ctx)->device; }
int cu_count(uintptr_t ctx) { return C(ctx)->cus; }

// Device memory and events belong to the current device, so a context
// creates them only while its own device is current (hb_init makes it
// current on the calling thread); otherwise the call fails instead of
// placing them on another device.
static void require_current(const Context* c) {
  int dev = -1;
  HB_CHECK_HIP(hipGetDevice(&dev));
  if (dev != c->device)
    throw std::runtime_error("context of device " + std::to_string(c->device) + " used while device " +
                             std::to_string(dev) + " is current (call hipSetDevice(" + std::to_string(c->device) +
                             ") on this thread first)");
}

void* pool_alloc(uintptr_t ctx, size_t bytes) {
  Context* c = C(ctx);
  size_t sc = size_class(bytes);
  auto it = c->free_list.find(sc);
  void* p = nullptr;
  if (it != c->free_list.end() && !it->second.empty()) {
    p = it->second.back();
    it->second.pop_back();
    c->cached_bytes -= sc;
  } else {
    require_current(c);
    hipError_t e = hipMalloc(&p, sc);
    if (e != hipSuccess && c->capturing)  // the retry below would synchronize the recording stream
      throw std::runtime_error("hb_alloc: out of device memory for " + std::to_string(bytes) +
                               " bytes while recording a graph");
    if (e != hipSuccess) {
      // release the cache once and retry before failing
      HB_CHECK_HIP(hipStreamSynchronize(c->stream));
      for (auto& kv : c->free_list)
        for (void* q : kv.second) (void)hipFree(q);
      c->free_list.clear();
      c->cached_bytes = 0;
      (void)hipGetLastError();
      e = hipMalloc(&p, sc);
      if (e != hipSuccess)
        throw std::runtime_error("hb_alloc: out of device memory for " + std::to_string(bytes) + " bytes: " +
                                 hipGetErrorString(e));
    }
  }
  c->live[p] = sc;
  c->live_bytes += sc;
  return p;
}

void pool_free(uintptr_t ctx, void* p) {
  if (!p) return;
  Context* c = C(ctx);
  auto it = c->live.find(p);
  if (it == c->live.end()) throw std::runtime_error("hb_free: pointer is not a live block of this context");
  if (c->capturing) {  // still live for the graph being recorded
    c->held.push_back(p);
    return;
  }
  size_t sc = it->second;
  c->live.erase(it);
  c->live_bytes -= sc;
  c->free_list[sc].push_back(p);
  c->cached_bytes += sc;
}

static Staging& staging_for(Context* c, size_t bytes) {
  Staging& s = c->staging[c->next_staging];
  c->next_staging ^= 1;
  if (s.pending) {
    HB_CHECK_HIP(hipEventSynchronize(s.done));
    s.pending = false;
  }
  if (s.cap < bytes) {
    if (s.host) HB_CHECK_HIP(hipHostFree(s.host));
    s.host = nullptr;
    size_t cap = 1 << 20;
    while (cap < bytes) cap <<= 1;
    HB_CHECK_HIP(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
    s.cap = cap;
  }
  if (!s.done) {
    require_current(c);
    HB_CHECK_HIP(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
  }
  return s;
}

// Largest single staging chunk; bigger uploads are split.
static constexpr size_t kStageChunk = 64u << 20;

static void upload_raw(Context* c, void* dst, const void* src, size_t bytes) {
  if (c->capturing)  // a recorded copy would re-read the staging buffer at every replay
    throw std::runtime_error("upload while recording a graph (run the sequence once before recording it)");
  size_t done = 0;
  while (done < bytes) {
    size_t n = bytes - done < kStageChunk ? bytes - done : kStageChunk;
    Staging& s = staging_for(c, n);
    std::memcpy(s.host, (const char*)src + done, n);
    HB_CHECK_HIP(hipMemcpyAsync((char*)dst + done, s.host, n, hipMemcpyHostToDevice, c->stream));
    HB_CHECK_HIP(hipEventRecord(s.done, c->stream));
    s.pending = true;
    done += n;
  }
}

// cos/sin of the RoPE angles under the CPU backend's f32 angle rule
// (restated in backend-webgpu/src/backend.ts:1185-1195): inv_i =
// f32(2^f32(-f32(i/half) * f32(log2 base))), theta = f32(l * inv_i), cos and
// sin evaluated in f64 and stored as f32.  Built on the host once per
// (L, D, base) and kept on the device for the context's lifetime.
const float* rope_table(uintptr_t ctx, int64_t L, int64_t D, double base) {
  Context* c = C(ctx);
  auto key = std::make_tuple(L, D, base);
  auto it = c->rope_tables.find(key);
  if (it != c->rope_tables.end()) return (const float*)it->second;
  int64_t half = D / 2;
  std::vector<float> tab((size_t)(2 * L * half));
  float lb = (float)log2(base);
  for (int64_t i = 0; i < half; i++) {
    float frac = (float)((double)i / (double)half);
    float ex = (float)(-(double)frac * (double)lb);
    float inv = (float)exp2((double)ex);
    for (int64_t l = 0; l < L; l++) {
      float th = (float)((double)l * (double)inv);
      tab[(size_t)(2 * (l * half + i))] = (float)cos((double)th);
      tab[(size_t)(2 * (l * half + i) + 1)] = (float)sin((double)th);
    }
  }
  void* d = nullptr;
  require_current(c);
  HB_CHECK_HIP(hipMalloc(&d, tab.size() * sizeof(float) + 16));
  upload_raw(c, d, tab.data(), tab.size() * sizeof(float));
  c->rope_tables[key] = d;
  return (const float*)d;
}

}  // namespace hb

using namespace hb;

extern "C" {

const char* hb_last_error(void) { return g_last_error.c_str(); }
int hb_abi_version(void) { return HB_ABI_VERSION; }

int hb_init(int device, uintptr_t* ctx) {
  HB_API_BEGIN
  HB_REQUIRE(ctx, "hb_init: null output");
  int n = 0;
  HB_CHECK_HIP(hipGetDeviceCount(&n));
  HB_REQUIRE(device >= 0 && device < n, "hb_init: device " + std::to_string(device) + " out of range (" +
                                            std::to_string(n) + " devices)");
  HB_CHECK_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  HB_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  HB_REQUIRE(arch.rfind("gfx950", 0) == 0, "hb_init: libhipbackend is built for gfx950 (MI355X); device is " + arch);
  sdpa_scratch_init(device);
  Context* c = new Context();
  c->device = device;
  c->cus = prop.multiProcessorCount;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    throw std::runtime_error(std::string("hb_init: stream: ") + hipGetErrorString(e));
  }
  *ctx = reinterpret_cast<uintptr_t>(c);
  HB_API_END
}

int hb_destroy(uintptr_t ctx) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_CHECK_HIP(hipSetDevice(c->device));
  HB_CHECK_HIP(hipStreamSynchronize(c->stream));
  for (auto& kv : c->graph_held) (void)hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(kv.first));
  for (auto& kv : c->free_list)
    for (void* p : kv.second) (void)hipFree(p);
  for (auto& kv : c->live) (void)hipFree(kv.first);
  for (auto& kv : c->rope_tables) (void)hipFree(kv.second);
  for (auto& s : c->staging) {
    if (s.host) (void)hipHostFree(s.host);
    if (s.done) (void)hipEventDestroy(s.done);
  }
  (void)hipStreamDestroy(c->stream);
  delete c;
  HB_API_END
}

int hb_device_info(uintptr_t ctx, char* buf, size_t cap) {
  HB_API_BEGIN
  Context* c = C(ctx);
  hipDeviceProp_t p;
  HB_CHECK_HIP(hipGetDeviceProperties(&p, c->device));
  std::string s = std::string("{\"name\":\"") + p.name + "\",\"arch\":\"" + p.gcnArchName +
                  "\",\"cus\":" + std::to_string(p.multiProcessorCount) +
                  ",\"hbm_bytes\":" + std::to_string((unsigned long long)p.totalGlobalMem) +
                  ",\"lds_per_block\":" + std::to_string((unsigned long long)p.sharedMemPerBlock) +
                  ",\"clock_khz\":" + std::to_string(p.clockRate) +
                  ",\"mem_clock_khz\":" + std::to_string(p.memoryClockRate) +
                  ",\"mem_bus_bits\":" + std::to_string(p.memoryBusWidth) +
                  ",\"l2_bytes\":" + std::to_string(p.l2CacheSize) +
                  ",\"warp_size\":" + std::to_string(p.warpSize) + "}";
  HB_REQUIRE(buf && cap > s.size(), "hb_device_info: buffer too small");
  std::memcpy(buf, s.c_str(), s.size() + 1);
  HB_API_END
}

int hb_alloc(uintptr_t ctx, size_t bytes, uintptr_t* ptr) {
  HB_API_BEGIN
  HB_REQUIRE(ptr, "hb_alloc: null output");
  *ptr = reinterpret_cast<uintptr_t>(pool_alloc(ctx, bytes));
  HB_API_END
}

int hb_free(uintptr_t ctx, uintptr_t ptr) {
  HB_API_BEGIN
  pool_free(ctx, reinterpret_cast<void*>(ptr));
  HB_API_END
}

int hb_pool_stats(uintptr_t ctx, uint64_t* live_bytes, uint64_t* cached_bytes, uint64_t* live_blocks) {
  HB_API_BEGIN
  Context* c = C(ctx);
  if (live_bytes) *live_bytes = c->live_bytes;
  if (cached_bytes) *cached_bytes = c->cached_bytes;
  if (live_blocks) *live_blocks = c->live.size();
  HB_API_END
}

int hb_pool_trim(uintptr_t ctx) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_CHECK_HIP(hipStreamSynchronize(c->stream));
  for (auto& kv : c->free_list)
    for (void* p : kv.second) HB_CHECK_HIP(hipFree(p));
  c->free_list.clear();
  c->cached_bytes = 0;
  HB_API_END
}

int hb_upload(uintptr_t ctx, uintptr_t dst, const void* src, size_t bytes) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_REQUIRE(bytes == 0 || (dst && src), "hb_upload: null pointer");
  upload_raw(c, (void*)dst, src, bytes);
  HB_API_END
}

int hb_download(uintptr_t ctx, void* dst, uintptr_t src, size_t bytes) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_REQUIRE(!c->capturing, "hb_download: the stream is recording a graph");
  HB_REQUIRE(bytes == 0 || (dst && src), "hb_download: null pointer");
  size_t done = 0;
  while (done < bytes) {
    size_t n = bytes - done < kStageChunk ? bytes - done : kStageChunk;
    Staging& s = staging_for(c, n);
    HB_CHECK_HIP(hipMemcpyAsync(s.host, (const char*)src + done, n, hipMemcpyDeviceToHost, c->stream));
    HB_CHECK_HIP(hipStreamSynchronize(c->stream));
    std::memcpy((char*)dst + done, s.host, n);
    done += n;
  }
  if (bytes == 0) HB_CHECK_HIP(hipStreamSynchronize(c->stream));
  HB_API_END
}

int hb_copy(uintptr_t ctx, uintptr_t dst, uintptr_t src, size_t bytes) {
  HB_API_BEGIN
  Context* c = C(ctx);
  if (bytes) HB_CHECK_HIP(hipMemcpyAsync((void*)dst, (const void*)src, bytes, hipMemcpyDeviceToDevice, c->stream));
  HB_API_END
}

int hb_sync(uintptr_t ctx) {
  HB_API_BEGIN
  HB_REQUIRE(!C(ctx)->capturing, "hb_sync: the stream is recording a graph");
  HB_CHECK_HIP(hipStreamSynchronize(C(ctx)->stream));
  HB_API_END
}

int hb_event_create(uintptr_t ctx, uintptr_t* ev) {
  HB_API_BEGIN
  HB_REQUIRE(ev, "hb_event_create: null output");
  require_current(C(ctx));
  hipEvent_t e;
  HB_CHECK_HIP(hipEventCreate(&e));
  *ev = reinterpret_cast<uintptr_t>(e);
  HB_API_END
}

int hb_event_record(uintptr_t ctx, uintptr_t ev) {
  HB_API_BEGIN
  HB_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), C(ctx)->stream));
  HB_API_END
}

int hb_event_elapsed(uintptr_t start, uintptr_t end, float* ms) {
  HB_API_BEGIN
  HB_REQUIRE(ms, "hb_event_elapsed: null output");
  HB_CHECK_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(end)));
  HB_CHECK_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(end)));
  HB_API_END
}

int hb_event_destroy(uintptr_t ev) {
  HB_API_BEGIN
  HB_CHECK_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  HB_API_END
}

// ---- stream capture (no counterpart in the reference: a recorded forward
// replayed without per-op host work, for small batches that the host's
// launches bound)

int hb_capture_begin(uintptr_t ctx) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_REQUIRE(!c->capturing, "hb_capture_begin: already capturing");
  HB_CHECK_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed));
  c->capturing = true;
  c->held.clear();
  HB_API_END
}

int hb_capture_end(uintptr_t ctx, uintptr_t* exec) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_REQUIRE(c->capturing, "hb_capture_end: not capturing");
  HB_REQUIRE(exec, "hb_capture_end: null output");
  *exec = 0;
  c->capturing = false;
  std::vector<void*> held;
  held.swap(c->held);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  hipGraphExec_t x = nullptr;
  if (e == hipSuccess) e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    for (void* p : held) pool_free(ctx, p);  // nothing will replay them
    throw std::runtime_error(std::string("hb_capture_end: ") + hipGetErrorString(e));
  }
  c->graph_held[(void*)x] = std::move(held);
  *exec = reinterpret_cast<uintptr_t>(x);
  HB_API_END
}

int hb_graph_launch(uintptr_t ctx, uintptr_t exec) {
  HB_API_BEGIN
  Context* c = C(ctx);
  HB_REQUIRE(c->graph_held.count((void*)exec), "hb_graph_launch: not a graph of this context");
  HB_CHECK_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), c->stream));
  HB_API_END
}

int hb_graph_destroy(uintptr_t ctx, uintptr_t exec) {
  HB_API_BEGIN
  Context* c = C(ctx);
  auto it = c->graph_held.find((void*)exec);
  HB_REQUIRE(it != c->graph_held.end(), "hb_graph_destroy: not a graph of this context");
  HB_CHECK_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)));
  std::vector<void*> held;
  held.swap(it->second);
  c->graph_held.erase(it);
  for (void* p : held) pool_free(ctx, p);  // reused only by work enqueued after the last replay
  HB_API_END
}

}  // extern "C"
