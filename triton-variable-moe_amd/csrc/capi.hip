// Status strings and version of the C ABI (include/vmoe.h).

#include "vmoe_common.h"

extern "C" const char* vmoe_status_string(int status) {
  switch (status) {
    case VMOE_OK: return "ok";
    case VMOE_ERR_INVALID_ARG: return "invalid argument";
    case VMOE_ERR_UNSUPPORTED:
      return "unsupported shape or alignment (dimensions and leading dimensions must be "
             "multiples of 8 elements, buffers 16-byte aligned)";
    case VMOE_ERR_LAUNCH: return "kernel launch failed";
    case VMOE_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

extern "C" int vmoe_version(void) { return 1; }

namespace vmoe {
thread_local LaunchTiming g_launch_timing = {nullptr, nullptr};
}

extern "C" int vmoe_set_launch_timing(void* start_event, void* stop_event) {
  if (start_event && !stop_event) return VMOE_ERR_INVALID_ARG;
  vmoe::g_launch_timing.start = reinterpret_cast<hipEvent_t>(start_event);
  vmoe::g_launch_timing.stop = reinterpret_cast<hipEvent_t>(stop_event);
  return VMOE_OK;
}
