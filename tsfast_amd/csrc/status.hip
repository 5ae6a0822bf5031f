// Status reporting for the C ABI (host code only).
#include <stdio.h>

#include <atomic>

#include "common.h"
#include "tsfast_hip.h"

namespace {
thread_local char g_msg[256];
}

namespace {
std::atomic<int> g_deterministic{0};
}

int tsf_deterministic() { return g_deterministic.load(std::memory_order_relaxed); }

int tsf_record_hip_error(hipError_t e) {
  if (e == hipSuccess) return TSF_OK;
  snprintf(g_msg, sizeof(g_msg), "HIP error %d: %s", (int)e, hipGetErrorString(e));
  return TSF_ERR_HIP;
}

extern "C" {

int tsfast_hip_version(void) { return 1; }

void tsfast_hip_set_deterministic(int on) { g_deterministic.store(on ? 1 : 0, std::memory_order_relaxed); }
int tsfast_hip_get_deterministic(void) { return tsf_deterministic(); }

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
