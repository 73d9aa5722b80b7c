// Status reporting shared by every entry point of the C ABI.

#include <string.h>

#include "tq_internal.h"

namespace {
thread_local char g_last_hip_error[256] = "";
thread_local hipEvent_t g_timing_start = nullptr;
thread_local hipEvent_t g_timing_stop = nullptr;
}

namespace tq {
tq_status record_hip_error(hipError_t err) {
  const char* msg = hipGetErrorString(err);
  strncpy(g_last_hip_error, msg != nullptr ? msg : "unknown HIP error", sizeof(g_last_hip_error) - 1);
  g_last_hip_error[sizeof(g_last_hip_error) - 1] = '\0';
  return TQ_ERR_HIP;
}

TimingEvents take_timing_events() {
  TimingEvents t{g_timing_start, g_timing_stop};
  g_timing_start = g_timing_stop = nullptr;
  return t;
}
}  // namespace tq

extern "C" tq_status tq_set_timing_events(void* start_event, void* stop_event) {
  g_timing_start = static_cast<hipEvent_t>(start_event);
  g_timing_stop = static_cast<hipEvent_t>(stop_event);
  return TQ_OK;
}

extern "C" const char* tq_status_string(tq_status status) {
  switch (status) {
    case TQ_OK: return "ok";
    case TQ_ERR_INVALID_ARGUMENT: return "invalid argument";
    case TQ_ERR_UNSUPPORTED: return "unsupported shape";
    case TQ_ERR_WORKSPACE: return "workspace missing or too small";
    case TQ_ERR_HIP: return "HIP runtime error";
  }
  return "unknown status";
}

extern "C" int32_t tq_abi_version(void) { return 3; }

extern "C" const char* tq_last_hip_error(void) { return g_last_hip_error; }
