// Runtime of libforge_hip.so: device selection, the library stream, a caching
// device allocator, copies, small asynchronous read-backs, events and the
// per-entry-point profiler.
#include "common.h"

#include <mutex>
#include <unordered_map>
#include <vector>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace fg {

static thread_local char g_err[1024] = "";
static bool g_init = false;
static int g_device = -1;
static int g_cus = 0;
static hipStream_t g_stream = nullptr;

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
hipStream_t stream() { return g_stream; }
bool initialized() { return g_init; }
int device_cu_count() { return g_cus; }

// ── caching allocator ──────────────────────────────────────────────────────
// Sizes are rounded up to one of four steps per power of two (waste <= 25%),
// and freed blocks are kept in exact-size free lists.  Training steps repeat
// the same shapes, so after the first step no hipMalloc/hipFree happens.
//
// Graph pools: while a graph is being captured, blocks handed out belong to
// that graph's pool.  A block of a live graph that is freed goes back to the
// graph's own free lists, never to the shared ones, so no work outside the
// graph can be given memory that a replay of the graph writes.  Destroying
// the graph moves its free blocks to the shared lists; its blocks that are
// still held return there when they are freed.  Calls that overlap a capture
// from other threads are not supported (the library has one stream).
typedef std::unordered_map<size_t, std::vector<void*>> FreeLists;
struct Block {
  size_t rs;
  int pool;  // 0: shared; > 0: graph pool id
};
static std::mutex g_mu;
static std::unordered_map<void*, Block> g_live;
static FreeLists g_pool;
static std::unordered_map<int, FreeLists> g_gpools;  // live graph pools
static int g_cap_pool = 0;                          // pool of the capture in progress
static int g_next_pool = 1;
static size_t g_in_use = 0, g_cached = 0;

static size_t round_size(size_t b) {
  if (b <= 512) return 512;
  size_t p = 1;
  while (p <= b / 2) p <<= 1;  // p = largest power of two <= b
  size_t step = p / 4 < 512 ? 512 : p / 4;
  return (b + step - 1) / step * step;
}

static void release_cached_locked() {
  for (auto& kv : g_pool)
    for (void* p : kv.second) (void)hipFree(p);
  g_pool.clear();
  size_t held = 0;
  for (auto& gp : g_gpools)
    for (auto& kv : gp.second) held += kv.first * kv.second.size();
  g_cached = held;
}

static bool take_locked(FreeLists& fl, size_t rs, void** out) {
  auto it = fl.find(rs);
  if (it == fl.end() || it->second.empty()) return false;
  *out = it->second.back();
  it->second.pop_back();
  return true;
}

int alloc(void** out, size_t bytes) {
  *out = nullptr;
  size_t rs = round_size(bytes ? bytes : 1);
  std::lock_guard<std::mutex> lk(g_mu);
  // During a capture the graph's own free blocks come first, then shared
  // ones: a shared free block was last used by work queued before the
  // capture began, which precedes every launch of the graph on the stream.
  bool got = (g_cap_pool && take_locked(g_gpools[g_cap_pool], rs, out)) || take_locked(g_pool, rs, out);
  if (got) {
    g_cached -= rs;
  } else {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, rs);
    if (e != hipSuccess && !g_cap_pool) {
      (void)hipGetLastError();
      (void)hipStreamSynchronize(g_stream);
      release_cached_locked();
      e = hipMalloc(&p, rs);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(FG_ERR_OOM, "device allocation of %zu bytes failed (%zu in use)", rs, g_in_use);
    }
    *out = p;
  }
  g_live[*out] = Block{rs, g_cap_pool};
  g_in_use += rs;
  return FG_OK;
}

int release(void* p) {
  if (!p) return FG_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_live.find(p);
  if (it == g_live.end()) return set_error(FG_ERR_ARG, "fg_free: %p was not allocated by fg_malloc", p);
  const Block b = it->second;
  g_live.erase(it);
  g_in_use -= b.rs;
  // A block freed during a capture may be used by the captured work whatever
  // its origin, so it joins the capture's pool.
  const int pool = g_cap_pool ? g_cap_pool : b.pool;
  auto gp = pool ? g_gpools.find(pool) : g_gpools.end();
  if (gp != g_gpools.end()) gp->second[b.rs].push_back(p);
  else g_pool[b.rs].push_back(p);
  g_cached += b.rs;
  return FG_OK;
}

bool capturing() { return g_cap_pool != 0; }

// Moves a graph pool's free blocks to the shared lists and forgets the pool.
static void drop_pool(int pool) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_gpools.find(pool);
  if (it == g_gpools.end()) return;
  for (auto& kv : it->second)
    for (void* p : kv.second) g_pool[kv.first].push_back(p);
  g_gpools.erase(it);
}

Workspace::~Workspace() {
  if (ptr) release(ptr);
}
int Workspace::get(size_t bytes) { return alloc(&ptr, bytes); }

// ── zero fill kernel (graph-safe replacement for hipMemsetAsync) ───────────
__global__ void zero_words_kernel(uint32_t* __restrict__ p, int64_t nwords) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint4 z = make_uint4(0, 0, 0, 0);
  int64_t n4 = nwords / 4;
  uint4* p4 = reinterpret_cast<uint4*>(p);
  for (int64_t k = i; k < n4; k += stride) p4[k] = z;
  for (int64_t k = n4 * 4 + i; k < nwords; k += stride) p[k] = 0u;
}
__global__ void zero_bytes_kernel(uint8_t* __restrict__ p, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = i; k < n; k += stride) p[k] = 0;
}

__global__ void fill_f32_kernel(float* __restrict__ p, float v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t k = i; k < n; k += stride) p[k] = v;
}

static unsigned grid_for(int64_t work, int block) {
  int64_t g = (work + block - 1) / block;
  int64_t cap = (int64_t)(g_cus > 0 ? g_cus : 256) * 16;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (unsigned)g;
}

// ── small asynchronous read-backs ──────────────────────────────────────────
static const int kSlots = 256;
static const size_t kSlotBytes = 4096;
static uint8_t* g_pinned = nullptr;
static hipEvent_t g_slot_ev[kSlots];
static int g_slot_gen[kSlots];
static int g_next_slot = 0;

// ── small host-to-device uploads through pinned staging ────────────────────
// Copies of <= kStageBytes are memcpy'd into a pinned slot and queued without
// draining the stream (token ids, targets, embedding plans each step); a slot
// is reused only once its previous copy has completed.
static const int kStageSlots = 16;
static const size_t kStageBytes = 1 << 20;
static uint8_t* g_stage = nullptr;
static hipEvent_t g_stage_ev[kStageSlots];
static int g_stage_next = 0;

// ── profiler ───────────────────────────────────────────────────────────────
struct KRecord {
  std::string name;
  long calls = 0, launches = 0;
  double ms = 0, kms = 0, flop = 0, bytes = 0;  // ms: scope brackets; kms: the kernels alone
};
struct KPending {
  int slot;
  hipEvent_t a, b;
  bool kernel;  // a launch's own events (kms) rather than a scope's (ms)
};
static bool g_kprof = false;
static std::vector<KRecord> g_krec;
static std::vector<KPending> g_kpend;
static std::vector<hipEvent_t> g_evpool;
static std::vector<int> g_kopen;  // slots of the open scopes, innermost last

static hipEvent_t take_event() {
  if (!g_evpool.empty()) {
    hipEvent_t e = g_evpool.back();
    g_evpool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

KProfScope::KProfScope(const char* name, double flop, double bytes) {
  if (!g_kprof || !name) return;
  int s = -1;
  for (size_t i = 0; i < g_krec.size(); ++i)
    if (g_krec[i].name == name) { s = (int)i; break; }
  if (s < 0) {
    g_krec.push_back(KRecord());
    g_krec.back().name = name;
    s = (int)g_krec.size() - 1;
  }
  slot = s;
  g_krec[s].calls += 1;
  g_krec[s].flop += flop;
  g_krec[s].bytes += bytes;
  KPending p;
  p.slot = s;
  p.a = take_event();
  p.b = nullptr;
  p.kernel = false;
  (void)hipEventRecord(p.a, g_stream);
  pend = (int)g_kpend.size();
  g_kpend.push_back(p);
  g_kopen.push_back(s);
}
void KProfScope::end() {
  if (slot < 0) return;
  hipEvent_t b = take_event();
  (void)hipEventRecord(b, g_stream);
  g_kpend[pend].b = b;
  if (!g_kopen.empty()) g_kopen.pop_back();
  slot = -1;
}

bool kprof_launch_events(hipEvent_t* start, hipEvent_t* stop) {
  if (!g_kprof || g_kopen.empty()) return false;
  KPending p;
  p.slot = g_kopen.back();
  p.a = take_event();
  p.b = take_event();
  p.kernel = true;
  g_krec[p.slot].launches += 1;
  g_kpend.push_back(p);
  *start = p.a;
  *stop = p.b;
  return true;
}

static void kprof_drain() {
  (void)hipStreamSynchronize(g_stream);
  for (auto& p : g_kpend) {
    float ms = 0;
    if (p.b && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) (p.kernel ? g_krec[p.slot].kms : g_krec[p.slot].ms) += ms;
    g_evpool.push_back(p.a);
    if (p.b) g_evpool.push_back(p.b);
  }
  g_kpend.clear();
}

}  // namespace fg

using namespace fg;

extern "C" {

int fg_device_count(int* count) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  if (count) *count = n;
  return FG_OK;
}

int fg_init(int device) {
  if (g_init) {
    if (device != g_device) return set_error(FG_ERR_ARG, "fg_init: already initialised on device %d", g_device);
    return FG_OK;
  }
  int n = 0;
  fg_device_count(&n);
  if (n <= 0) return set_error(FG_ERR_INIT, "no HIP device visible");
  if (device < 0 || device >= n) return set_error(FG_ERR_ARG, "device %d out of range (have %d)", device, n);
  FG_HIP_CHECK(hipSetDevice(device));
  FG_HIP_CHECK(hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, device));
  FG_HIP_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  FG_HIP_CHECK(hipHostMalloc((void**)&g_pinned, kSlots * kSlotBytes, hipHostMallocDefault));
  for (int i = 0; i < kSlots; ++i) {
    FG_HIP_CHECK(hipEventCreateWithFlags(&g_slot_ev[i], hipEventDisableTiming));
    g_slot_gen[i] = 0;
  }
  FG_HIP_CHECK(hipHostMalloc((void**)&g_stage, kStageSlots * kStageBytes, hipHostMallocDefault));
  for (int i = 0; i < kStageSlots; ++i) FG_HIP_CHECK(hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming));
  g_device = device;
  g_init = true;
  return FG_OK;
}

const char* fg_last_error(void) { return g_err; }

int fg_malloc(void** ptr, size_t bytes) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(ptr != nullptr, "fg_malloc: null out pointer");
  return alloc(ptr, bytes);
}

int fg_free(void* ptr) {
  FG_REQUIRE_INIT();
  return release(ptr);
}

int fg_empty_cache(void) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_empty_cache");
  FG_HIP_CHECK(hipStreamSynchronize(g_stream));
  std::lock_guard<std::mutex> lk(g_mu);
  release_cached_locked();
  return FG_OK;
}

int fg_mem_stats(size_t* in_use, size_t* cached) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (in_use) *in_use = g_in_use;
  if (cached) *cached = g_cached;
  return FG_OK;
}

int fg_h2d(void* dst, const void* src, size_t bytes) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_h2d");
  if (!bytes) return FG_OK;
  FG_ARG_CHECK(dst && src, "fg_h2d: null pointer");
  if (bytes <= kStageBytes) {
    const int s = g_stage_next;
    g_stage_next = (g_stage_next + 1) % kStageSlots;
    FG_HIP_CHECK(hipEventSynchronize(g_stage_ev[s]));
    uint8_t* slot = g_stage + (size_t)s * kStageBytes;
    memcpy(slot, src, bytes);
    FG_HIP_CHECK(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, g_stream));
    FG_HIP_CHECK(hipEventRecord(g_stage_ev[s], g_stream));
    return FG_OK;
  }
  FG_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  FG_HIP_CHECK(hipStreamSynchronize(g_stream));
  return FG_OK;
}

int fg_d2h(void* dst, const void* src, size_t bytes) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_d2h");
  if (!bytes) return FG_OK;
  FG_ARG_CHECK(dst && src, "fg_d2h: null pointer");
  FG_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  FG_HIP_CHECK(hipStreamSynchronize(g_stream));
  return FG_OK;
}

int fg_d2d(void* dst, const void* src, size_t bytes) {
  FG_REQUIRE_INIT();
  if (!bytes) return FG_OK;
  FG_ARG_CHECK(dst && src, "fg_d2d: null pointer");
  FG_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return FG_OK;
}

int fg_zero(void* ptr, size_t bytes) {
  FG_REQUIRE_INIT();
  if (!bytes) return FG_OK;
  FG_ARG_CHECK(ptr, "fg_zero: null pointer");
  if (((uintptr_t)ptr % 16) == 0 && bytes % 4 == 0) {
    int64_t nw = (int64_t)(bytes / 4);
    FG_LAUNCH(zero_words_kernel, dim3(grid_for(nw / 4 + 1, 256)), dim3(256), 0, (uint32_t*)ptr, nw);
  } else {
    FG_LAUNCH(zero_bytes_kernel, dim3(grid_for((int64_t)bytes, 256)), dim3(256), 0, (uint8_t*)ptr,
              (int64_t)bytes);
  }
  return FG_OK;
}

int fg_sync(void) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_sync");
  FG_HIP_CHECK(hipStreamSynchronize(g_stream));
  return FG_OK;
}

int fg_read_async(const void* src, size_t bytes, int* ticket) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_read_async");
  FG_ARG_CHECK(src && ticket, "fg_read_async: null pointer");
  FG_ARG_CHECK(bytes <= kSlotBytes, "fg_read_async: %zu bytes exceeds the %zu-byte slot", bytes, kSlotBytes);
  int s = g_next_slot;
  g_next_slot = (g_next_slot + 1) % kSlots;
  // The slot's previous copy must have landed before it is overwritten.
  FG_HIP_CHECK(hipEventSynchronize(g_slot_ev[s]));
  g_slot_gen[s] += 1;
  FG_HIP_CHECK(hipMemcpyAsync(g_pinned + (size_t)s * kSlotBytes, src, bytes, hipMemcpyDeviceToHost, g_stream));
  FG_HIP_CHECK(hipEventRecord(g_slot_ev[s], g_stream));
  *ticket = (g_slot_gen[s] & 0x7fffff) * kSlots + s;
  return FG_OK;
}

int fg_read_wait(int ticket, void* dst, size_t bytes) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_read_wait");
  FG_ARG_CHECK(ticket >= 0 && dst, "fg_read_wait: bad ticket or null pointer");
  FG_ARG_CHECK(bytes <= kSlotBytes, "fg_read_wait: %zu bytes exceeds the slot", bytes);
  int s = ticket % kSlots, gen = ticket / kSlots;
  if ((g_slot_gen[s] & 0x7fffff) != gen) return set_error(FG_ERR_ARG, "fg_read_wait: ticket %d is stale", ticket);
  FG_HIP_CHECK(hipEventSynchronize(g_slot_ev[s]));
  memcpy(dst, g_pinned + (size_t)s * kSlotBytes, bytes);
  return FG_OK;
}

int fg_event_create(void** ev) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(ev, "fg_event_create: null pointer");
  hipEvent_t e = nullptr;
  FG_HIP_CHECK(hipEventCreate(&e));
  *ev = (void*)e;
  return FG_OK;
}
int fg_event_record(void* ev) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_event_record");
  FG_HIP_CHECK(hipEventRecord((hipEvent_t)ev, g_stream));
  return FG_OK;
}
int fg_event_elapsed_ms(void* a, void* b, float* ms) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_event_elapsed_ms");
  FG_HIP_CHECK(hipEventSynchronize((hipEvent_t)b));
  FG_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
  return FG_OK;
}
int fg_event_destroy(void* ev) {
  FG_REQUIRE_INIT();
  FG_HIP_CHECK(hipEventDestroy((hipEvent_t)ev));
  return FG_OK;
}

int fg_kprof_enable(int on) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_kprof_enable");
  if (!on && g_kprof) kprof_drain();
  g_kprof = on != 0;
  return FG_OK;
}
int fg_kprof_reset(void) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_kprof_reset");
  kprof_drain();
  g_krec.clear();
  return FG_OK;
}
int fg_kprof_report(char* buf, size_t len) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_kprof_report");
  FG_ARG_CHECK(buf && len > 2, "fg_kprof_report: buffer too small");
  kprof_drain();
  std::string s = "[";
  char line[512];
  for (size_t i = 0; i < g_krec.size(); ++i) {
    const KRecord& r = g_krec[i];
    snprintf(line, sizeof(line),
             "%s{\"name\":\"%s\",\"calls\":%ld,\"launches\":%ld,\"ms\":%.6f,\"kernel_ms\":%.6f,\"flop\":%.6e,"
             "\"bytes\":%.6e}",
             i ? "," : "", r.name.c_str(), r.calls, r.launches, r.ms, r.kms, r.flop, r.bytes);
    s += line;
  }
  s += "]";
  if (s.size() + 1 > len) return set_error(FG_ERR_ARG, "fg_kprof_report: need %zu bytes", s.size() + 1);
  memcpy(buf, s.c_str(), s.size() + 1);
  return FG_OK;
}

int fg_fill_f32(float* ptr, float value, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && (n == 0 || ptr), "fg_fill_f32: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(fill_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, ptr, value, n);
  return FG_OK;
}

// ── graphs ─────────────────────────────────────────────────────────────────
// The library's work on its stream between fg_graph_begin and fg_graph_end is
// recorded (not run) into a HIP graph; fg_graph_launch replays it on the
// stream.  Memory that the recorded work allocates belongs to the graph's
// pool (see the allocator) until fg_graph_destroy.
namespace {
struct GraphRec {
  hipGraph_t graph;
  hipGraphExec_t exec;
  int pool;
};
bool g_kprof_saved = false;

void end_capture_state(int pool) {
  drop_pool(pool);
  g_kprof = g_kprof_saved;
}
}  // namespace

int fg_graph_begin(void) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(!g_cap_pool, "fg_graph_begin: a capture is already in progress");
  if (g_kprof) kprof_drain();
  g_kprof_saved = g_kprof;
  g_kprof = false;
  int pool;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    pool = g_next_pool++;
    g_gpools[pool];
  }
  hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    end_capture_state(pool);
    return set_error(FG_ERR_HIP, "hipStreamBeginCapture failed: %s", hipGetErrorString(e));
  }
  g_cap_pool = pool;
  return FG_OK;
}

int fg_graph_end(void** graph) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(g_cap_pool, "fg_graph_end: no capture in progress");
  FG_ARG_CHECK(graph, "fg_graph_end: null out pointer");
  *graph = nullptr;
  const int pool = g_cap_pool;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  g_cap_pool = 0;
  if (e != hipSuccess || !g) {
    (void)hipGetLastError();
    if (g) (void)hipGraphDestroy(g);
    end_capture_state(pool);
    return set_error(FG_ERR_HIP, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
  }
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiateWithFlags(&x, g, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipGraphDestroy(g);
    end_capture_state(pool);
    return set_error(FG_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
  }
  g_kprof = g_kprof_saved;
  *graph = new GraphRec{g, x, pool};
  return FG_OK;
}

int fg_graph_abort(void) {
  FG_REQUIRE_INIT();
  if (!g_cap_pool) return FG_OK;
  const int pool = g_cap_pool;
  hipGraph_t g = nullptr;
  (void)hipStreamEndCapture(g_stream, &g);
  (void)hipGetLastError();
  g_cap_pool = 0;
  if (g) (void)hipGraphDestroy(g);
  end_capture_state(pool);
  return FG_OK;
}

int fg_graph_launch(void* graph) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_graph_launch");
  FG_ARG_CHECK(graph, "fg_graph_launch: null graph");
  FG_HIP_CHECK(hipGraphLaunch(static_cast<GraphRec*>(graph)->exec, g_stream));
  return FG_OK;
}

int fg_graph_destroy(void* graph) {
  FG_REQUIRE_INIT();
  FG_NO_CAPTURE("fg_graph_destroy");
  if (!graph) return FG_OK;
  GraphRec* r = static_cast<GraphRec*>(graph);
  FG_HIP_CHECK(hipStreamSynchronize(g_stream));  // replays in flight finish first
  (void)hipGraphExecDestroy(r->exec);
  (void)hipGraphDestroy(r->graph);
  drop_pool(r->pool);
  delete r;
  return FG_OK;
}

}  // extern "C"
