// ABI helpers: error strings and version.
#include <hip/hip_runtime.h>
#include "xv_kernels.h"

extern "C" const char* xv_error_string(int code) { return hipGetErrorString((hipError_t)code); }
extern "C" int xv_abi_version(void) { return 1; }
