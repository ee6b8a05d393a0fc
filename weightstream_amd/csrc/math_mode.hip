// The math mode is fixed when the library is built, not set at run time, so
// no call can change the numerics of another: this file is compiled once per
// library, with WS_NATIVE_MATH defined for libweightstream_hip_native.so.
#include "ws_internal.hpp"

namespace ws {

#ifdef WS_NATIVE_MATH
int math_mode() { return WS_MATH_NATIVE; }
#else
int math_mode() { return WS_MATH_EXACT; }
#endif

}  // namespace ws
