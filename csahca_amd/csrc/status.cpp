// status.cpp -- error state of the C ABI (thread-local last-error message), the
// launch profiler (per-dispatch device durations from hipExtLaunchKernel events)
// and the device clock stamp (timing inside a captured graph).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace csahca {
namespace {
thread_local std::string g_last_error;

struct ProfRecord {
  const char* name;
  hipEvent_t start;
  hipEvent_t stop;
};
struct ProfResult {
  const char* name;
  int64_t launches;
  double total_ms;
  double min_ms;
  double max_ms;
};
thread_local bool g_prof_on = false;
thread_local std::vector<hipEvent_t> g_pool;
thread_local size_t g_pool_used = 0;
thread_local std::vector<ProfRecord> g_records;
thread_local std::vector<ProfResult> g_results;
}  // namespace

int fail(int code, const char* msg) {
  g_last_error = msg ? msg : "";
  return code;
}

int fail_hip(hipError_t err, const char* where) {
  char buf[512];
  std::snprintf(buf, sizeof(buf), "%s: HIP error %d (%s)", where, static_cast<int>(err),
                hipGetErrorString(err));
  g_last_error = buf;
  return CSAHCA_ERR_HIP;
}

void clear_error() { g_last_error.clear(); }

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

bool profiling_active() { return g_prof_on; }

bool profile_take_events(hipEvent_t* start, hipEvent_t* stop) {
  while (g_pool.size() < g_pool_used + 2) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return false;
    g_pool.push_back(e);
  }
  *start = g_pool[g_pool_used++];
  *stop = g_pool[g_pool_used++];
  return true;
}

void profile_record(const char* name, hipEvent_t start, hipEvent_t stop) {
  g_records.push_back(ProfRecord{name, start, stop});
}

}  // namespace csahca

using namespace csahca;

extern "C" const char* csahca_last_error(void) { return g_last_error.c_str(); }

extern "C" int csahca_abi_version(void) { return 1; }

extern "C" int csahca_profile_begin(void) {
  g_records.clear();
  g_results.clear();
  g_pool_used = 0;
  g_prof_on = true;
  return CSAHCA_OK;
}

extern "C" int csahca_profile_end(void) {
  g_prof_on = false;
  g_results.clear();
  for (const ProfRecord& r : g_records) {
    const hipError_t e = hipEventSynchronize(r.stop);
    if (e != hipSuccess) return -fail_hip(e, "csahca_profile_end");
    float ms = 0.f;
    const hipError_t e2 = hipEventElapsedTime(&ms, r.start, r.stop);
    if (e2 != hipSuccess) return -fail_hip(e2, "csahca_profile_end");
    ProfResult* slot = nullptr;
    for (ProfResult& p : g_results)
      if (std::strcmp(p.name, r.name) == 0) slot = &p;
    if (slot == nullptr) {
      g_results.push_back(ProfResult{r.name, 0, 0.0, 1e30, 0.0});
      slot = &g_results.back();
    }
    slot->launches += 1;
    slot->total_ms += ms;
    if (ms < slot->min_ms) slot->min_ms = ms;
    if (ms > slot->max_ms) slot->max_ms = ms;
  }
  g_records.clear();
  g_pool_used = 0;
  return static_cast<int>(g_results.size());
}

extern "C" int csahca_profile_result(int i, const char** name, int64_t* launches, double* total_ms,
                                     double* min_ms, double* max_ms) {
  if (i < 0 || static_cast<size_t>(i) >= g_results.size())
    return fail(CSAHCA_ERR_ARGUMENT, "profile result index out of range");
  const ProfResult& p = g_results[static_cast<size_t>(i)];
  if (name) *name = p.name;
  if (launches) *launches = p.launches;
  if (total_ms) *total_ms = p.total_ms;
  if (min_ms) *min_ms = p.min_ms;
  if (max_ms) *max_ms = p.max_ms;
  return CSAHCA_OK;
}

// Device clock stamp: one wavefront stores the device wall clock (a constant
// rate counter, csahca_device_clock_khz) at dst when the stream reaches it.
// Two stamps captured into one HIP graph around a run of kernels time that
// run on the device, without the graph's own launch and without event
// nodes in the graph.
namespace csahca {
namespace {
__global__ __launch_bounds__(64) void clock_stamp_kernel(uint64_t* dst) {
  if (threadIdx.x == 0) *dst = wall_clock64();
}
}  // namespace
}  // namespace csahca

extern "C" int csahca_device_clock_stamp(uint64_t* dst, void* stream) {
  clear_error();
  CSAHCA_REQUIRE(dst != nullptr, "null clock stamp pointer");
  return launch("clock_stamp_kernel", clock_stamp_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), dst);
}

extern "C" int64_t csahca_device_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return khz;
}
