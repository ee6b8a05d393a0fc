// Host-side helpers shared by the translation units of libweightstream_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/ws_hip.h"
#include "ws_device.hpp"

namespace ws {

// Status of the launch just issued: a configuration error is reported at
// launch, anything asynchronous surfaces on the caller's next sync.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? WS_OK : (int)e;
}

// Math mode of this library build (math_mode.hip: WS_MATH_EXACT in
// libweightstream_hip.so, WS_MATH_NATIVE in libweightstream_hip_native.so).
int math_mode();

// Compute units of the current device (queried once per device).
int cu_count();

}  // namespace ws
