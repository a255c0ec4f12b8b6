// lm_common.hip -- ABI version, error reporting, workspace sizing, factor prep.
#include "lm_impl.h"

static thread_local std::string g_err;

int lm_fail_v(int code, const char* fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  g_err = buf;
  return code;
}

extern "C" int lm_version(void) { return LM_ABI_VERSION; }
extern "C" const char* lm_last_error(void) { return g_err.c_str(); }
extern "C" size_t lm_workspace_size(int64_t M, int64_t N, int32_t rank) { return ws_layout(M, N, rank).total; }

// ---- kernel timer -----------------------------------------------------------
#include <atomic>
#include <map>
#include <mutex>
#include <vector>

namespace {
struct TimerRec {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pairs;
  hipEvent_t open = nullptr;
};
std::atomic<bool> g_timer_on{false};
std::mutex g_timer_mu;
std::map<std::string, TimerRec> g_timer;

void timer_clear_locked() {
  for (auto& kv : g_timer) {
    for (auto& p : kv.second.pairs) {
      (void)hipEventDestroy(p.first);
      (void)hipEventDestroy(p.second);
    }
    if (kv.second.open) (void)hipEventDestroy(kv.second.open);
  }
  g_timer.clear();
}
}  // namespace

bool lm_timer_on() { return g_timer_on.load(std::memory_order_relaxed); }

void lm_timer_mark(const char* family, hipStream_t st, bool begin) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  TimerRec& r = g_timer[family];
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return;
  (void)hipEventRecord(e, st);
  if (begin) {
    if (r.open) (void)hipEventDestroy(r.open);
    r.open = e;
  } else if (r.open) {
    r.pairs.emplace_back(r.open, e);
    r.open = nullptr;
  } else {
    (void)hipEventDestroy(e);
  }
}

extern "C" int lm_timer_enable(int32_t enable) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  timer_clear_locked();
  g_timer_on.store(enable != 0);
  return LM_OK;
}

extern "C" int lm_timer_read(const char* family, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  double ms = 0.0;
  int64_t n = 0;
  auto it = g_timer.find(family ? family : "");
  if (it != g_timer.end()) {
    for (auto& p : it->second.pairs) {
      HIP_TRY(hipEventSynchronize(p.second));
      float t = 0.0f;
      HIP_TRY(hipEventElapsedTime(&t, p.first, p.second));
      ms += t;
      ++n;
    }
  }
  if (total_ms) *total_ms = ms;
  if (launches) *launches = n;
  return LM_OK;
}

int launch_prep(const PrepItem& it, hipStream_t st) {
  TimedLaunch timed("prep", st);
  int64_t total = prep_units(it);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_prep1, dim3((unsigned)blocks), dim3(256), 0, st, it, total);
  LAUNCH_CHECK();
  return LM_OK;
}


// ---- host -> device staging of descriptor tables ---------------------------
// The stack entries upload per-call descriptor tables.  They go through a
// small pool of pinned host buffers, each guarded by an event recorded after
// its copy, so the entry points return without synchronizing the stream: a
// buffer is reused once its previous copy has completed (waiting on the
// oldest one when all are in flight).
namespace {
struct StageSlot {
  void* host = nullptr;
  size_t cap = 0;
  hipEvent_t ev = nullptr;
  int device = -1;
  uint64_t stamp = 0;
};
std::mutex g_stage_mu;
std::vector<StageSlot> g_stage;
uint64_t g_stage_clock = 0;
constexpr size_t kStageSlots = 8;
}  // namespace

int lm_stage_h2d(void* dst, const void* src, size_t bytes, hipStream_t st) {
  if (bytes == 0) return LM_OK;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_stage_mu);
  StageSlot* pick = nullptr;
  for (auto& s : g_stage)  // a free slot of this device that is large enough
    if (s.device == dev && s.cap >= bytes && hipEventQuery(s.ev) == hipSuccess) { pick = &s; break; }
  if (!pick && g_stage.size() < kStageSlots) {
    g_stage.emplace_back();
    pick = &g_stage.back();
    pick->device = dev;
    HIP_TRY(hipEventCreateWithFlags(&pick->ev, hipEventDisableTiming));
  }
  if (!pick) {  // every slot busy or too small: wait for the oldest of this device
    for (auto& s : g_stage)
      if (s.device == dev && (!pick || s.stamp < pick->stamp)) pick = &s;
    if (!pick) return fail(LM_EHIP, "no staging slot for device %d", dev);
    HIP_TRY(hipEventSynchronize(pick->ev));
  }
  if (pick->cap < bytes) {
    if (pick->host) HIP_TRY(hipHostFree(pick->host));
    pick->host = nullptr;
    pick->cap = 0;
    const size_t cap = bytes < 65536 ? 65536 : bytes * 2;
    HIP_TRY(hipHostMalloc(&pick->host, cap, hipHostMallocDefault));
    pick->cap = cap;
  }
  memcpy(pick->host, src, bytes);
  HIP_TRY(hipMemcpyAsync(dst, pick->host, bytes, hipMemcpyHostToDevice, st));
  HIP_TRY(hipEventRecord(pick->ev, st));
  pick->stamp = ++g_stage_clock;
  return LM_OK;
}
