// Status reporting for the C ABI (host code only).
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "common.h"
#include "tsfast_hip.h"

namespace {
thread_local char g_msg[256];
}

namespace {
// Bitwise-reproducible look-back scans by default (tsfast_hip_set_deterministic)
std::atomic<int> g_deterministic{1};
// Polls without progress before a look-back gives up (lookback.h kSpinMax).
std::atomic<uint32_t> g_spin_limit{1u << 20};
// The alarm word: 4 bytes of mapped, coherent host memory (visible to every device), allocated
// on first use; a look-back that gives up stores 1 there with a system-scope store.
std::once_flag g_alarm_once;
unsigned* g_alarm_host = nullptr;
unsigned* g_alarm_dev = nullptr;
// Look-back scans are numbered from 1 as they are enqueued; a give-up writes its scan's number
// into the alarm word, and the host remembers the last number it reported.
std::atomic<uint32_t> g_epoch{0};
std::atomic<uint32_t> g_reported{0};
}  // namespace

uint32_t tsf_next_epoch() {
  uint32_t e = g_epoch.fetch_add(1, std::memory_order_relaxed) + 1;
  if (e == 0) e = g_epoch.fetch_add(1, std::memory_order_relaxed) + 1;  // skip 0 on wrap-around
  return e;
}

int tsf_deterministic() { return g_deterministic.load(std::memory_order_relaxed); }

uint32_t tsf_lookback_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

unsigned* tsf_lookback_alarm() {
  std::call_once(g_alarm_once, [] {
    void* p = nullptr;
    if (hipHostMalloc(&p, 64, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess) {
      (void)hipGetLastError();  // no alarm word; leave no error behind for the next launch check
      return;
    }
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipHostFree(p);
      return;
    }
    g_alarm_host = static_cast<unsigned*>(p);
    __atomic_store_n(g_alarm_host, 0u, __ATOMIC_RELAXED);
    g_alarm_dev = static_cast<unsigned*>(d);
  });
  return g_alarm_dev;
}

int tsf_record_hip_error(hipError_t e) {
  if (e == hipSuccess) return TSF_OK;
  snprintf(g_msg, sizeof(g_msg), "HIP error %d: %s", (int)e, hipGetErrorString(e));
  return TSF_ERR_HIP;
}

extern "C" {

int tsfast_hip_version(void) { return 1; }

void tsfast_hip_set_deterministic(int on) { g_deterministic.store(on ? 1 : 0, std::memory_order_relaxed); }
int tsfast_hip_get_deterministic(void) { return tsf_deterministic(); }

int tsfast_hip_lookback_gave_up(int clear) {
  if (!tsf_lookback_alarm()) return -1;
  const uint32_t a = __atomic_load_n(g_alarm_host, __ATOMIC_ACQUIRE);
  if (a == 0 || a == g_reported.load(std::memory_order_relaxed)) return 0;
  if (clear) g_reported.store(a, std::memory_order_relaxed);
  return 1;
}

int64_t tsfast_hip_set_lookback_spin_limit(int64_t polls) {
  if (polls < 0) polls = 0;
  if (polls > (int64_t)UINT32_MAX) polls = UINT32_MAX;
  return (int64_t)g_spin_limit.exchange((uint32_t)polls, std::memory_order_relaxed);
}

const char* tsfast_hip_status_string(int status) {
  switch (status) {
    case TSF_OK:
      return "ok";
    case TSF_ERR_ARG:
      return "invalid size or pointer argument";
    case TSF_ERR_WORKSPACE:
      return "workspace missing or too small";
    case TSF_ERR_UNSUPPORTED:
      return "shape not supported by the kernels";
    case TSF_ERR_SCRATCH:
      return "shape needs more scratch than the no-allocation entry point's fixed device array holds";
    case TSF_ERR_HIP:
      return g_msg[0] ? g_msg : "HIP error";
    default:
      return "unknown status";
  }
}

}  // extern "C"
