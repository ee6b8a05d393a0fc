"""ws_expf and ws_logf (weightstream_amd/csrc/ws_expf.h) equals the host glibc expf on
every one of the 2^32 float inputs. The reference's sigmoid/silu/softmax
(weightstream-ref/src/num.rs:47-88) call Rust's f32::exp, which is the
platform libm expf; the GPU routing kernels evaluate ws_expf so the scores,
and therefore the selected experts and weights, are bit-identical. Likewise ws_logf (weightstream_amd/csrc/ws_logf.h) equals
glibc logf, Rust's f32::ln, on every input, and so the sqrtsoftplus score
sqrt(ln(1 + exp(x))) of num.rs:82-88 / moe.rs:38-42 equals the host
library's composition on every input."""
import oracle_lib as O


def test_ws_expf_equals_glibc_exhaustive():
    assert O.expfcheck().ws_expf_mismatches(0, 1 << 32) == 0


def test_ws_logf_equals_glibc_exhaustive():
    assert O.expfcheck().ws_math_mismatches(0, 0, 1 << 32) == 0


def test_sqrtsoftplus_score_equals_glibc_exhaustive():
    assert O.expfcheck().ws_math_mismatches(1, 0, 1 << 32) == 0


def test_ws_logf_special_values_and_closed_forms():
    """Special cases glibc's logf defines and a wrong branch would break
    (log(1) = +0, log(+-0) = -inf, log(inf) = inf, NaN for negative and NaN
    inputs, subnormals), and closed forms: log(2^j) = float(j ln 2)."""
    import math
    import struct

    import numpy as np
    lib = O.expfcheck()
    bits = lambda x: struct.unpack("<I", struct.pack("<f", x))[0]
    got = np.empty(1, np.uint32)
    want = {1.0: 0x00000000, 0.0: 0xFF800000, -0.0: 0xFF800000, float("inf"): 0x7F800000,
            -1.0: 0x7FC00000, float("nan"): 0x7FC00000}
    for x, w in want.items():
        assert lib.ws_math_mismatches(0, bits(x), bits(x) + 1) == 0, x
        lib.glibc_math_bits(0, bits(x), 1, got.ctypes.data)
        assert got[0] == w, x
    for j in [-149, -130, -126, -1, 1, 2, 10, 127]:
        x = float(np.float32(2.0 ** j))
        assert lib.ws_math_mismatches(0, bits(x), bits(x) + 1) == 0, j
        lib.glibc_math_bits(0, bits(x), 1, got.ctypes.data)
        assert got[0] == bits(float(np.float32(j * math.log(2.0)))), j
