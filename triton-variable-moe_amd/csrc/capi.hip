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
