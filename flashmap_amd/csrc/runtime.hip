// Library runtime: errors, device properties, profiling events.
#include <mutex>
#include <string>
#include <vector>

#include "fm_host.h"

namespace fm {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int device_info(DeviceInfo *info) {
  static std::mutex mu;
  static std::vector<DeviceInfo> cache;
  int dev = 0;
  FM_CHECK_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1);
  if (cache[dev].cus == 0) {
    int cus = 0;
    FM_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    cache[dev].cus = cus;
  }
  *info = cache[dev];
  return FM_OK;
}

// Profiling: event pairs recorded around the main attention kernel.
struct ProfileState {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> pool;  // created lazily, reused
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  size_t next = 0;
};
static ProfileState g_prof;

static hipEvent_t take_event() {
  if (g_prof.next < g_prof.pool.size()) return g_prof.pool[g_prof.next++];
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  g_prof.pool.push_back(e);
  g_prof.next = g_prof.pool.size();
  return e;
}

void profile_before(hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  if (!g_prof.enabled) return;
  hipEvent_t a = take_event();
  if (a == nullptr) return;
  hipEventRecord(a, stream);
  g_prof.pending.push_back({a, nullptr});
}

void profile_after(hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  if (!g_prof.enabled || g_prof.pending.empty() || g_prof.pending.back().second != nullptr) return;
  hipEvent_t b = take_event();
  if (b == nullptr) {
    g_prof.pending.pop_back();
    return;
  }
  hipEventRecord(b, stream);
  g_prof.pending.back().second = b;
}

// Measurement hook: one wavefront reads the shader-clock counter (s_memtime) and the
// 100 MHz real-time counter (s_memrealtime), spins until `spin` shader-clock ticks have
// passed (a bounded loop: the counter only grows) and stores both elapsed counts with a
// vector store, so (ticks / (real ticks / 100 MHz)) is the shader clock of that moment.
__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t *out, uint64_t spin) {
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  uint64_t t = t0;
  while (t - t0 < spin) t = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[0] = t - t0;
    out[1] = r1 - r0;
  }
}

}  // namespace fm

extern "C" {

const char *fm_last_error(void) { return fm::g_last_error.c_str(); }

int fm_abi_version(void) { return FM_ABI_VERSION; }

int fm_device_cus(int device, int *num_cus) {
  FM_REQUIRE(num_cus != nullptr, "num_cus is NULL");
  FM_CHECK_HIP(hipDeviceGetAttribute(num_cus, hipDeviceAttributeMultiprocessorCount, device));
  return FM_OK;
}

int fm_profile_enable(int enable) {
  std::lock_guard<std::mutex> lock(fm::g_prof.mu);
  fm::g_prof.enabled = enable != 0;
  return FM_OK;
}

int fm_clock_probe(uint64_t *out, uint64_t spin_ticks, void *stream) {
  FM_REQUIRE(out != nullptr && ((uintptr_t)out & 15) == 0, "out must be a 16-byte aligned device pointer");
  FM_REQUIRE(spin_ticks > 0 && spin_ticks <= (1ull << 24), "spin_ticks must lie in (0, 2^24]");
  fm::clock_probe_kernel<<<1, 64, 0, (hipStream_t)stream>>>(out, spin_ticks);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

int fm_profile_read(double *total_ms, int64_t *launches) {
  FM_REQUIRE(total_ms != nullptr && launches != nullptr, "NULL output pointer");
  std::lock_guard<std::mutex> lock(fm::g_prof.mu);
  double sum = 0.0;
  int64_t count = 0;
  for (auto &pr : fm::g_prof.pending) {
    if (pr.second == nullptr) continue;
    FM_CHECK_HIP(hipEventSynchronize(pr.second));
    float ms = 0.f;
    FM_CHECK_HIP(hipEventElapsedTime(&ms, pr.first, pr.second));
    sum += ms;
    ++count;
  }
  fm::g_prof.pending.clear();
  fm::g_prof.next = 0;
  *total_ms = sum;
  *launches = count;
  return FM_OK;
}

}  // extern "C"
