// Error state and library metadata of the C ABI.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace fsc {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(err));
    return 1;
  }
  return 0;
}

// ---------------------------------------------------------------- persistent launches
namespace {
struct GridKey {
  const void* kernel;
  size_t lds;
  int dev;
  int max_per_cu;
  int64_t cap;
};
std::mutex g_grid_mu;
std::vector<GridKey> g_grid_cache;
}  // namespace

unsigned persist_grid(int64_t n, const void* kernel, size_t lds, int max_per_cu) {
  const unsigned full = xcd_grid(n);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return full;                      // the one-block-per-node grid is always correct
  }
  std::lock_guard<std::mutex> lk(g_grid_mu);
  for (const GridKey& k : g_grid_cache)
    if (k.kernel == kernel && k.lds == lds && k.dev == dev && k.max_per_cu == max_per_cu)
      return (unsigned)std::min<int64_t>(full, k.cap);
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, lds) != hipSuccess || cus <= 0 ||
      per_cu <= 0) {
    (void)hipGetLastError();
    return full;
  }
  per_cu = std::min(per_cu, max_per_cu);
  const int64_t cap = std::max<int64_t>(8, (int64_t)cus * per_cu / 8 * 8);
  g_grid_cache.push_back(GridKey{kernel, lds, dev, max_per_cu, cap});
  return (unsigned)std::min<int64_t>(full, cap);
}

// ---------------------------------------------------------------- launch timing
// Opt-in measurement of one kernel's launches with HIP events recorded on the launch
// stream (fsc_timing_begin / fsc_timing_end).  Off by default; costs nothing when off.
namespace {
struct Timing {
  std::mutex mu;
  bool on = false;
  std::string kernel;
  std::vector<hipEvent_t> events;   // start/stop pairs
};
Timing g_timing;
}  // namespace

int timing_mark_begin(const char* kernel, hipStream_t st) {
  if (!g_timing.on) return -1;
  std::lock_guard<std::mutex> lk(g_timing.mu);
  if (!g_timing.on || g_timing.kernel != kernel) return -1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return -1;
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return -1;
  }
  g_timing.events.push_back(a);
  g_timing.events.push_back(b);
  (void)hipEventRecord(a, st);
  return (int)g_timing.events.size() - 1;
}

void timing_mark_end(int slot, hipStream_t st) {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lk(g_timing.mu);
  (void)hipEventRecord(g_timing.events[slot], st);
}

}  // namespace fsc

extern "C" {

int fsc_timing_begin(const char* kernel_name) {
  FSC_CHECK_ARG(kernel_name != nullptr, "fsc_timing_begin: null kernel name");
  std::lock_guard<std::mutex> lk(fsc::g_timing.mu);
  FSC_CHECK_ARG(!fsc::g_timing.on, "fsc_timing_begin: timing already active");
  fsc::g_timing.on = true;
  fsc::g_timing.kernel = kernel_name;
  fsc::g_timing.events.clear();
  return 0;
}

int fsc_timing_end(double* total_ms, int64_t* launches) {
  FSC_CHECK_ARG(total_ms && launches, "fsc_timing_end: null output");
  std::lock_guard<std::mutex> lk(fsc::g_timing.mu);
  FSC_CHECK_ARG(fsc::g_timing.on, "fsc_timing_end: timing not active");
  double tot = 0.0;
  int err = 0;
  auto& ev = fsc::g_timing.events;
  for (size_t i = 0; i + 1 < ev.size(); i += 2) {
    float ms = 0.f;
    if (hipEventSynchronize(ev[i + 1]) != hipSuccess || hipEventElapsedTime(&ms, ev[i], ev[i + 1]) != hipSuccess)
      err = 1;
    tot += ms;
  }
  *total_ms = tot;
  *launches = (int64_t)(ev.size() / 2);
  for (auto e : ev) (void)hipEventDestroy(e);
  ev.clear();
  fsc::g_timing.on = false;
  if (err) {
    fsc::set_error("fsc_timing_end: event query failed");
    return 2;
  }
  return 0;
}

const char* fsc_last_error(void) { return fsc::g_last_error.c_str(); }

int fsc_abi_version(void) { return 2; }

}  // extern "C"
