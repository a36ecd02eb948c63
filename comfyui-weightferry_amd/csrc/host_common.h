// Host-only helpers of the library's file and thread code (the GGUF reader, the SSD tier's ring): the HIP runtime
// API and the thread-local error message of the C ABI. No device code, so these sources also build with a plain
// host compiler.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "../../include/weightferry.h"

namespace wf {

void set_error(const char* fmt, ...);

}  // namespace wf
