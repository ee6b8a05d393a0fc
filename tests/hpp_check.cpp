// Compiled and run by tests/test_abi.py on the CPU: include/ws_hip.hpp
// compiles against include/ws_hip.h, links against the library, and its
// launch mirrors throw weightstream_hip::Error with the library's code for
// arguments the library rejects before touching a device.
#include <cstdio>

#include "ws_hip.hpp"

namespace wl = weightstream_hip::launch;

template <class F>
static int expect_code(const char *what, int want, F f) {
    try {
        f();
    } catch (const weightstream_hip::Error &e) {
        if (e.code == want) return 0;
        std::printf("%s: code %d, want %d (%s)\n", what, e.code, want, e.what());
        return 1;
    }
    std::printf("%s: no exception\n", what);
    return 1;
}

int main() {
    const auto fake = (const uint8_t *)(uintptr_t)4096;  // never dereferenced
    float *out = (float *)(uintptr_t)8192;
    int bad = 0;
    bad += expect_code("fp8_gemm k=100", WS_ERR_SHAPE,
                       [&] { wl::fp8_gemm(fake, fake, fake, fake, out, 1, 16, 100); });
    bad += expect_code("fp8_gemm null a", WS_ERR_INVALID_ARG,
                       [&] { wl::fp8_gemm(nullptr, fake, fake, fake, out, 1, 16, 128); });
    bad += expect_code("fp8_gemm_tl kind 10", WS_ERR_INVALID_ARG, [&] {
        wl::fp8_gemm_tl_on((wl::TlGemm)10, fake, (const uint32_t *)fake, fake,
                           (const uint32_t *)fake, out, 1, nullptr);
    });
    bad += expect_code("moe_local_slots top_k 17", WS_ERR_SHAPE, [&] {
        wl::moe_local_slots((const int32_t *)fake, (int32_t *)out, (int32_t *)out,
                            (int32_t *)out, 17, 0, 8);
    });
    bad += expect_code("moe_grouped_tl kind 5", WS_ERR_INVALID_ARG, [&] {
        wl::moe_grouped_tl_cached_on((wl::TlMoe)5, fake, fake, fake, fake, (const int32_t *)fake,
                                     (const int32_t *)fake, out, 4, 4, 2, nullptr, 128, 128, 4);
    });
    if (!weightstream_hip::built_with_hip()) bad++;
    std::printf(bad ? "FAIL\n" : "ok\n");
    return bad;
}
