// The C ABI's shared pieces: the per-thread last-error string, the version query, the library's
// set-up (vsp_init) and the fault record of the bounded waits.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "common.h"
#include "vesper_kernels.h"

namespace {
thread_local char g_last_error[512] = "";
std::mutex g_init_mutex;
bool g_initialised = false;
unsigned* g_fault_host = nullptr;    // the fault record: kFaultWords words of pinned host memory
unsigned* g_fault_device = nullptr;  // its address for kernels
std::atomic<int> g_wait_limit{1 << 19};
std::atomic<int> g_scan_segments{2};
}  // namespace

namespace vsp {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  g_last_error[0] = '\0';
  return OK;
}

unsigned* fault_record() { return g_fault_device; }
int wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }
int scan_segments() { return g_scan_segments.load(std::memory_order_relaxed); }

}  // namespace vsp

extern "C" const char* vsp_last_error(void) { return g_last_error; }

extern "C" int vsp_init(void) {
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_initialised) return vsp::OK;
  if (g_fault_host == nullptr) {
    void* host = nullptr;
    hipError_t err = hipHostMalloc(&host, vsp::kFaultWords * sizeof(unsigned), hipHostMallocMapped);
    if (err != hipSuccess) return vsp::fail(vsp::ERR_LAUNCH, "vsp_init: pinned fault record: %s", hipGetErrorString(err));
    std::memset(host, 0, vsp::kFaultWords * sizeof(unsigned));
    void* dev = nullptr;
    err = hipHostGetDevicePointer(&dev, host, 0);
    if (err != hipSuccess) {
      (void)hipHostFree(host);
      return vsp::fail(vsp::ERR_LAUNCH, "vsp_init: fault record address: %s", hipGetErrorString(err));
    }
    g_fault_host = static_cast<unsigned*>(host);
    g_fault_device = static_cast<unsigned*>(dev);
  }
  const int st = vsp::ring_scratch_init();
  if (st != vsp::OK) return st;
  g_initialised = true;
  g_last_error[0] = '\0';
  return vsp::OK;
}

extern "C" unsigned vsp_fault_bits(void) {
  if (g_fault_host == nullptr) return 0;
  unsigned bits = 0;
  for (int i = 0; i < vsp::kFaultWords; ++i)
    if (__atomic_load_n(&g_fault_host[i], __ATOMIC_RELAXED) != 0) bits |= 1u << i;
  return bits;
}

extern "C" void vsp_clear_faults(void) {
  if (g_fault_host == nullptr) return;
  for (int i = 0; i < vsp::kFaultWords; ++i) __atomic_store_n(&g_fault_host[i], 0u, __ATOMIC_RELAXED);
}

extern "C" int vsp_set_wait_limit(int polls) {
  return g_wait_limit.exchange(polls < 0 ? (1 << 19) : polls, std::memory_order_relaxed);
}

extern "C" int vsp_set_scan_segments(int form) {
  return g_scan_segments.exchange(form == 0 || form == 1 ? form : 2, std::memory_order_relaxed);
}

extern "C" int vsp_abi_version(void) { return VSP_ABI_VERSION; }
