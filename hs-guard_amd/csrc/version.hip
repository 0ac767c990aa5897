// Library version and error text of libhsg.so.
#include "hsg_common.h"

extern "C" int hsg_version(void) { return 100; }

extern "C" const char* hsg_error_string(int code) {
  switch (code) {
    case HSG_OK: return "ok";
    case HSG_ERR_ARG: return "invalid argument (null pointer or inconsistent size)";
    case HSG_ERR_ALIGN: return "pointer or stride breaks the kernel's vector-load alignment";
    case HSG_ERR_SHAPE: return "head size, window or tick length outside what the kernels support";
    case HSG_ERR_BLAS: return "hipBLASLt call failed";
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown hsg error";
  }
}
