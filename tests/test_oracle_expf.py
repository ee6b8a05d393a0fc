"""ws_expf (weightstream_amd/csrc/ws_expf.h) equals the host glibc expf on
every one of the 2^32 float inputs. The reference's sigmoid/silu/softmax
(weightstream-ref/src/num.rs:47-88) call Rust's f32::exp, which is the
platform libm expf; the GPU routing kernels evaluate ws_expf so the scores,
and therefore the selected experts and weights, are bit-identical."""
import oracle_lib as O


def test_ws_expf_equals_glibc_exhaustive():
    assert O.expfcheck().ws_expf_mismatches(0, 1 << 32) == 0
