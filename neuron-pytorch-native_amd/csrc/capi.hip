// Library-level C ABI entry points (status text, ABI version).
#include "npn_common.h"

extern "C" const char* npn_status_string(int status) {
  switch (status) {
    case NPN_OK: return "ok";
    case NPN_ERR_NULL: return "a required pointer is NULL";
    case NPN_ERR_SHAPE: return "a size is out of the supported range or inconsistent";
    case NPN_ERR_ALIGN: return "a pointer is not aligned as required";
    case NPN_ERR_WORKSPACE: return "workspace missing or too small";
    case NPN_ERR_LAUNCH: return "the HIP runtime rejected a kernel launch";
    case NPN_ERR_VALUE: return "an argument value is out of range";
    case NPN_ERR_SCRATCH:
      return "the problem needs more than the no-allocation entry point's fixed scratch";
    default: return "unknown status";
  }
}

extern "C" int npn_abi_version(void) { return 102; }
