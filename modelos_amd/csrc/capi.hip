// Library-wide C ABI pieces: version, per-thread error message, launch check,
// process-wide kernel timing.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "pkm_common.h"

namespace {
thread_local char g_last_error[1024] = "";

// Kernel timing records, process-wide (backward passes launch from the
// autograd engine's device thread): (kernel name, start, stop).
struct TimingRecord {
  const char* name;
  hipEvent_t start, stop;
};
constexpr size_t kMaxTimingRecords = 4096;
std::mutex g_timing_mu;
std::atomic<bool> g_timing_on{false};
std::vector<TimingRecord> g_timing;  // guarded by g_timing_mu
uint64_t g_timing_generation = 0;    // guarded by g_timing_mu; bumped when the records are released

void release_timing_locked() {
  for (TimingRecord& r : g_timing) {
    if (r.start) (void)hipEventDestroy(r.start);
    if (r.stop) (void)hipEventDestroy(r.stop);
  }
  g_timing.clear();
  ++g_timing_generation;
}
}  // namespace

KernelSpan::KernelSpan(const char* name, hipStream_t st) : slot(-1), generation(0), stream(st) {
  if (!g_timing_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (!g_timing_on.load(std::memory_order_relaxed) || g_timing.size() >= kMaxTimingRecords) return;
  TimingRecord r{name, nullptr, nullptr};
  if (hipEventCreate(&r.start) != hipSuccess) return;
  if (hipEventCreate(&r.stop) != hipSuccess || hipEventRecord(r.start, st) != hipSuccess) {
    (void)hipEventDestroy(r.start);
    if (r.stop) (void)hipEventDestroy(r.stop);
    return;
  }
  g_timing.push_back(r);
  slot = (long)g_timing.size() - 1;
  generation = g_timing_generation;
}

KernelSpan::~KernelSpan() {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  // the records may have been released (timing ended) since the constructor
  if (generation != g_timing_generation || g_timing[slot].stop == nullptr) return;
  if (hipEventRecord(g_timing[slot].stop, stream) != hipSuccess) {
    (void)hipEventDestroy(g_timing[slot].stop);
    g_timing[slot].stop = nullptr;
  }
}

int pkm_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Reports a failed kernel launch (bad configuration, missing code object for
// the device) without synchronising: hipGetLastError only reads launch status.
int pkm_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return PKM_OK;
}

extern "C" int pkm_version(void) { return (0 << 16) | 1; }

extern "C" const char* pkm_last_error_string(void) { return g_last_error; }

extern "C" int pkm_kernel_timing_begin(void) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  release_timing_locked();
  g_timing_on.store(true);
  return PKM_OK;
}

extern "C" int pkm_kernel_timing_read(const char* kernel, float* ms_out, int64_t cap, int64_t* count_out) {
  PKM_REQUIRE(kernel != nullptr && count_out != nullptr && cap >= 0 && (cap == 0 || ms_out != nullptr),
              PKM_ERR_INVALID_ARGUMENT, "pkm_kernel_timing_read: bad arguments");
  std::lock_guard<std::mutex> lock(g_timing_mu);
  int64_t n = 0;
  for (const TimingRecord& r : g_timing) {
    if (r.stop == nullptr || strcmp(r.name, kernel) != 0) continue;
    if (n < cap) {
      hipError_t e = hipEventSynchronize(r.stop);
      float ms = 0.f;
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
      if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "pkm_kernel_timing_read: %s", hipGetErrorString(e));
      ms_out[n] = ms;
    }
    ++n;
  }
  *count_out = n;
  return PKM_OK;
}

extern "C" int pkm_kernel_timing_end(void) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  g_timing_on.store(false);
  release_timing_locked();
  return PKM_OK;
}
