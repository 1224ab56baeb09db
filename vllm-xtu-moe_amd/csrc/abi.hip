// Library-level entry points: version and error strings.
#include <hip/hip_runtime.h>

extern "C" {

const char* xtu_version(void) { return "xtu-moe-amd 0.2 gfx950"; }

const char* xtu_error_string(int err) { return hipGetErrorString((hipError_t)err); }

}  // extern "C"
