// Return-code text of the C ABI.
#include "dk_common.h"

extern "C" const char* dk_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case DK_ERR_INVALID: return "invalid argument (size, rank or null pointer)";
    case DK_ERR_ALIGN: return "misaligned pointer, stride or offset";
    case DK_ERR_WORKSPACE: return "workspace missing or too small";
    case DK_ERR_CAPTURE: return "one-time set-up due under stream capture: call once outside capture first";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
