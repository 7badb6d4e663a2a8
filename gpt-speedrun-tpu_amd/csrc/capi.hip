// Library identity and status strings of the gptrig C ABI.
#include "common.h"

extern "C" {

const char* gptrig_version(void) { return "gptrig 0.1.0 (gfx950)"; }

const char* gptrig_status_string(int status) {
  switch (status) {
    case GPTRIG_OK:
      return "ok";
    case GPTRIG_E_NULL:
      return "a required pointer is NULL";
    case GPTRIG_E_SHAPE:
      return "sizes, strides or alignment violate the contract";
    case GPTRIG_E_DTYPE:
      return "unsupported element type";
    case GPTRIG_E_UNSUPPORTED:
      return "configuration not implemented";
    case GPTRIG_E_LAUNCH:
      return "HIP kernel launch failed";
    case GPTRIG_E_WORKSPACE:
      return "workspace too small";
    default:
      return "unknown status";
  }
}

}  // extern "C"
