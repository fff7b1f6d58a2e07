// C-ABI housekeeping: the thread-local error string, the launch counter and small
// utility kernels shared by the entry points in route.hip, dispatch.hip and experts.hip.
#include <stdlib.h>
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

// ---- tuning options ------------------------------------------------------------------
struct OptionSpec {
  const char* name;
  int64_t lo, hi;           // accepted range besides 0
  const int64_t* allowed;   // or an explicit list (terminated by 0), when non-NULL
};
static const int64_t kFwdRows[] = {32, 64, 96, 0};
static const int64_t kBwdRows[] = {48, 64, 80, 96, 0};
static const int64_t kDxRows[] = {64, 96, 0};
static const int64_t kRouterWaves[] = {8, 16, 0};
static const OptionSpec kOptions[OPT_COUNT] = {
    {"side_stream", 1, 1, nullptr},   {"fwd_rows", 0, 0, kFwdRows},
    {"fwd_dist", 2, 6, nullptr},      {"bwd_rows", 0, 0, kBwdRows},
    {"bwd_dist", 2, 4, nullptr},      {"dx_rows", 0, 0, kDxRows},
    {"dx_dist", 2, 4, nullptr},       {"xcd_run", 1, 1024, nullptr},
    {"dw_stages", 2, 4, nullptr},     {"router_waves", 0, 0, kRouterWaves},
    {"pack_in_place", 1, 1, nullptr},
};
static std::atomic<int64_t> g_options[OPT_COUNT];

int64_t option(OptionId id) { return g_options[id].load(std::memory_order_relaxed); }

static int option_index(const char* name) {
  if (!name) return -1;
  for (int i = 0; i < OPT_COUNT; ++i)
    if (strcmp(kOptions[i].name, name) == 0) return i;
  return -1;
}

// ---- side stream -------------------------------------------------------------------------
//
// Per host thread and device: one extra stream (default priority, non-blocking) and a
// fork and a join event per slot, all created on first use.  side_fork makes the side
// stream wait for the work already enqueued on `s` and returns it; side_join makes `s`
// wait for everything enqueued on the side stream since.  Both are event-ordered, so the
// pattern is also what a HIP graph capture of `s` records (the side stream joins the
// capture at the fork and leaves it at the join).  Measured on MI355X under ROCm 7, a
// replayed graph gains nothing from the fork (its branches are not overlapped) and pays
// for the extra nodes, so work enqueued while `s` is being captured stays on `s`.  Eager
// calls fork only with the "side_stream" option set: measured at T = 8192, the fork and
// join calls cost more host time per step (0.44 against 0.30 ms of enqueue for a 0.31 ms
// GPU step) than the overlap saves, which leaves an eager step host-bound.
constexpr int kSideSlots = 4;
constexpr int kMaxDevices = 64;

struct SideState {
  hipStream_t stream = nullptr;
  hipEvent_t fork[kSideSlots] = {};
  hipEvent_t join[kSideSlots] = {};
  bool failed = false;
};

static thread_local SideState g_side[kMaxDevices];

static bool side_init(SideState& st, hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
    return false;  // captured work stays on s
  if (st.stream) return true;
  if (st.failed) return false;
  bool ok = hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking) == hipSuccess;
  for (int i = 0; ok && i < kSideSlots; ++i)
    ok = hipEventCreateWithFlags(&st.fork[i], hipEventDisableTiming) == hipSuccess &&
         hipEventCreateWithFlags(&st.join[i], hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    for (int i = 0; i < kSideSlots; ++i) {
      if (st.fork[i]) hipEventDestroy(st.fork[i]);
      if (st.join[i]) hipEventDestroy(st.join[i]);
      st.fork[i] = st.join[i] = nullptr;
    }
    if (st.stream) hipStreamDestroy(st.stream);
    st.stream = nullptr;
    st.failed = true;
    (void)hipGetLastError();
  }
  return ok;
}

hipStream_t side_fork(hipStream_t s, int slot) {
  if (!option(OPT_SIDE_STREAM) || slot < 0 || slot >= kSideSlots) return s;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return s;
  SideState& st = g_side[dev];
  if (!side_init(st, s)) return s;
  if (hipEventRecord(st.fork[slot], s) != hipSuccess ||
      hipStreamWaitEvent(st.stream, st.fork[slot], 0) != hipSuccess) {
    (void)hipGetLastError();
    return s;
  }
  return st.stream;
}

int side_join(hipStream_t s, hipStream_t side, int slot) {
  if (side == s) return NSMOE_OK;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("side_join: no current device");
    return NSMOE_EHIP;
  }
  SideState& st = g_side[dev];
  hipError_t e = hipEventRecord(st.join[slot], side);
  if (e == hipSuccess) e = hipStreamWaitEvent(s, st.join[slot], 0);
  if (e != hipSuccess) {
    set_error("side_join: %s", hipGetErrorString(e));
    return NSMOE_EHIP;
  }
  return NSMOE_OK;
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

extern "C" int32_t nsmoe_abi_version(void) { return 8; }

extern "C" int nsmoe_set_option(const char* name, int64_t value) {
  const int i = nsmoe::option_index(name);
  if (i < 0) {
    nsmoe::set_error("set_option: unknown option '%s'", name ? name : "(null)");
    return nsmoe::NSMOE_EINVAL;
  }
  const nsmoe::OptionSpec& o = nsmoe::kOptions[i];
  bool ok = value == 0;
  if (!ok && o.allowed) {
    for (const int64_t* v = o.allowed; *v; ++v) ok = ok || *v == value;
  } else if (!ok) {
    ok = value >= o.lo && value <= o.hi;
  }
  if (!ok) {
    nsmoe::set_error("set_option: %lld is not a value of '%s'", (long long)value, name);
    return nsmoe::NSMOE_EINVAL;
  }
  nsmoe::g_options[i].store(value, std::memory_order_relaxed);
  return nsmoe::NSMOE_OK;
}

extern "C" int64_t nsmoe_get_option(const char* name) {
  const int i = nsmoe::option_index(name);
  return i < 0 ? -1 : nsmoe::option((nsmoe::OptionId)i);
}
