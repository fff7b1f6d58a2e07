// C-ABI housekeeping: the thread-local error string, the launch counter and small
// utility kernels shared by the entry points in route.hip, dispatch.hip and experts.hip.
#include <string.h>

#include <mutex>
#include <vector>

#include "nsmoe_capi_internal.h"

namespace nsmoe {

static thread_local char g_last_error[512] = "";
static std::atomic<uint64_t> g_launches{0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void note_launch() { g_launches.fetch_add(1, std::memory_order_relaxed); }

__global__ void fill_i32_kernel(int32_t* __restrict__ dst, int64_t n, int32_t value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}

int fill_i32(int32_t* dst, int64_t n, int32_t value, hipStream_t stream) {
  if (n <= 0) return NSMOE_OK;
  int64_t blocks = cdiv(n, 256);
  if (blocks > 1024) blocks = 1024;
  fill_i32_kernel<<<(unsigned)blocks, 256, 0, stream>>>(dst, n, value);
  return check_launch("fill_i32_kernel");
}

// ---- kernel timing ----------------------------------------------------------------------
struct TimingState {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> start, stop;
  std::vector<const char*> names;
  size_t used = 0;
};
static TimingState g_timing;

KernelTimer::KernelTimer(const char* name, hipStream_t stream) : slot_(-1), stream_(stream) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  if (!g_timing.enabled || g_timing.used >= g_timing.start.size()) return;
  slot_ = (int)g_timing.used++;
  g_timing.names[slot_] = name;
  hipEventRecord(g_timing.start[slot_], stream_);
}

void KernelTimer::stop() {
  if (slot_ < 0) return;
  std::lock_guard<std::mutex> lock(g_timing.mu);
  hipEventRecord(g_timing.stop[slot_], stream_);
}

}  // namespace nsmoe

using nsmoe::g_timing;

// Enables (capacity > 0 event pairs) or disables timing; clears all records.
extern "C" int nsmoe_timing_enable(int32_t capacity) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  for (auto e : g_timing.start) hipEventDestroy(e);
  for (auto e : g_timing.stop) hipEventDestroy(e);
  g_timing.start.clear();
  g_timing.stop.clear();
  g_timing.names.clear();
  g_timing.used = 0;
  g_timing.enabled = capacity > 0;
  for (int i = 0; i < capacity; ++i) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
      nsmoe::set_error("timing: hipEventCreate failed");
      g_timing.enabled = false;
      return nsmoe::NSMOE_EHIP;
    }
    g_timing.start.push_back(a);
    g_timing.stop.push_back(b);
    g_timing.names.push_back(nullptr);
  }
  return nsmoe::NSMOE_OK;
}

// Total milliseconds and launch count recorded for kernel `name` (waits for the events).
extern "C" int nsmoe_timing_read(const char* name, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  double t = 0.0;
  int64_t n = 0;
  for (size_t i = 0; i < g_timing.used; ++i) {
    if (!g_timing.names[i] || strcmp(g_timing.names[i], name) != 0) continue;
    if (hipEventSynchronize(g_timing.stop[i]) != hipSuccess) {
      nsmoe::set_error("timing: hipEventSynchronize failed");
      return nsmoe::NSMOE_EHIP;
    }
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, g_timing.start[i], g_timing.stop[i]) != hipSuccess) {
      nsmoe::set_error("timing: hipEventElapsedTime failed");
      return nsmoe::NSMOE_EHIP;
    }
    t += ms;
    ++n;
  }
  *total_ms = t;
  *launches = n;
  return nsmoe::NSMOE_OK;
}

extern "C" const char* nsmoe_last_error(void) { return nsmoe::g_last_error; }

extern "C" uint64_t nsmoe_launch_count(void) {
  return nsmoe::g_launches.load(std::memory_order_relaxed);
}

extern "C" int32_t nsmoe_abi_version(void) { return 3; }
