"""Loader of the in-tree HIP libraries.

libweightstream_hip.so (EXACT math) is the product;
libweightstream_hip_native.so is the same ABI built with the CDNA4 scaled
MFMAs (NATIVE math). There is no CPU or PyTorch fallback: if a library is
missing, loading it raises.
"""
import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libweightstream_hip.so")
LIB_NATIVE_PATH = os.path.join(PKG, "libweightstream_hip_native.so")
HEADER = os.path.join(ROOT, "include", "ws_hip.h")

_libs = {}


def header_symbols():
    """Every function the C header declares (ws_*)."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ws_[a-z0-9_]+)\s*\(", txt)))


def load(native=False):
    """The EXACT library, or with native=True the NATIVE-math build."""
    lib = _libs.get(native)
    if lib is None:
        path = LIB_NATIVE_PATH if native else LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(
                "%s is not built (python -m weightstream_amd.build); "
                "weightstream_amd has no fallback path" % os.path.basename(path))
        lib = C.CDLL(path)
        _declare(lib)
        _libs[native] = lib
    return lib


_p = C.c_void_p
_i64 = C.c_int64
_i = C.c_int
_f = C.c_float
_u32 = C.c_uint32

SIGNATURES = {
    "ws_init": (_i, []),
    "ws_built_with_hip": (_i, []),
    "ws_error_string": (C.c_char_p, [_i]),
    "ws_expf_probe": (_i, [_u32, _u32, _p, _p]),
    "ws_math_probe": (_i, [_i, _u32, _u32, _p, _p]),
    "ws_get_math_mode": (_i, []),
    "ws_snap8": (_i, [_p, _i64, _p]),
    "ws_emit8": (_i, [_p, _p, _p, _i64, _p]),
    "ws_emit8_packed": (_i, [_p, _p, _p, _i64, _p]),
    "ws_pack_scales": (_i, [_p, _p, _i64, _p]),
    "ws_weight_quant_fp4": (_i, [_p, _p, _p, _i64, _i64, _p]),
    "ws_weight_quant_fp8": (_i, [_p, _p, _p, _i64, _i64, _p]),
    "ws_packed_fp4_scale_bytes": (C.c_size_t, [_i64, _i64]),
    "ws_prepack_fp4": (_i, [_p, _p, _i64, _i64, _p, _p, _p]),
    "ws_gemm_workspace_size": (C.c_size_t, [_i64, _i64, _i64]),
    "ws_set_gemm_workspace": (_i, [_p, C.c_size_t, _p]),
    "ws_fp8_gemm": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_fp8_gemm_acc": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_fp8_gemm_tile": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_fp8_gemm_bf16": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_fp8_gemm_f32s": (_i, [_p, _p, _p, _p, _p, _i, _i64, _i64, _i64, _p]),
    "ws_tl_gemm_shape": (_i, [_i, _p, _p]),
    "ws_fp8_gemm_tl": (_i, [_i, _p, _p, _p, _p, _p, _i64, _p]),
    "ws_act_quant_f32s": (_i, [_p, _p, _p, _i64, _i64, _p]),
    "ws_fp4_gemm": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_fp4_gemm_tile": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_moe_gate_logits": (_i, [_p, _p, _i, _p, _i64, _i64, _i64, _p]),
    "ws_moe_topk": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _f, _i, _f, _p]),
    "ws_moe_gate": (_i, [_p, _p, _p, _p, _i64, _i64, _p]),
    "ws_moe_gate_m": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_moe_select": (_i, [_p, _p, _p, _p, _i64, _i64, _f, _p]),
    "ws_moe_route": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p]),
    "ws_swiglu": (_i, [_p, _p, _p, _i64, _f, _p]),
    "ws_acc_f32": (_i, [_p, _p, _i64, _p]),
    "ws_shared_expert_workspace_size": (C.c_size_t, [_i64, _i64, _i64]),
    "ws_shared_expert_fp8": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p,
                                  C.c_size_t, _p]),
    "ws_shared_expert_fp8_w13": (_i, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p,
                                      C.c_size_t, _p]),
    "ws_fp8_gemv_acc": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_moe_gate_shared_w13": (_i, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f, _p]),
    "ws_shared_expert_down_acc": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "ws_moe_decode_route_shared": (_i, [_p, _p, _i, _f, _i, _f, _p, _p, _p, _p, _p, _p, _p, _p,
                                        _p, _p, _i64, _i64, _i64, _i64, _f, _p, _p, _p, _i64,
                                        _p, _p, _p, C.c_size_t, _p]),
    "ws_shared_expert_fp8_w13_acc": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _p,
                                          C.c_size_t, _p]),
    "ws_expert_glu_quant": (_i, [_p] * 10 + [_i64, _i64, _i64, _i64, _f, _p]),
    "ws_expert_glu_quant_x": (_i, [_p] * 9 + [_i64, _i64, _i64, _i64, _f, _p]),
    "ws_expert_glu_quant_route": (_i, [_p, _p, _i, _f, _i, _f] + [_p] * 9 + [_i64, _i64, _i64, _i64, _f, _p]),
    "ws_moe_local_slots": (_i, [_p] * 4 + [_i64, _i64, _i64, _p]),
    "ws_moe_dispatch_ids": (_i, [_p, _p, _i64, _i64, _i64, _p]),
    "ws_expert_glu": (_i, [_p] * 11 + [_i64, _i64, _i64, _i64, _p]),
    "ws_expert_quant": (_i, [_p] * 5 + [_i64, _i64, _p]),
    "ws_expert_reduce": (_i, [_p] * 8 + [_i64, _i64, _i64, _i64, _i64, _p]),
    "ws_moe_decode_workspace_size": (C.c_size_t, [_i64, _i64, _i64]),
    "ws_moe_decode": (_i, [_p] * 10 + [_i64, _i64, _i64, _i64, _f, _p, C.c_size_t, _p]),
    "ws_moe_decode_route": (_i, [_p, _p, _i, _f, _i, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                 _i64, _i64, _i64, _i64, _f, _p, C.c_size_t, _p]),
    "ws_moe_decode_route_noalloc": (_i, [_p, _p, _i, _f, _i, _f] + [_p] * 10 +
                                    [_i64, _i64, _i64, _i64, _f, _p]),
    "ws_moe_dispatch": (_i, [_p] * 10 + [_i64, _i64, _i64, _i64, _p]),
    "ws_moe_dispatch_tl": (_i, [_p] * 10 + [_i64, _i64, _i64, _i64, _p]),
    "ws_moe_grouped_tl": (_i, [_i] + [_p] * 7 + [_i64] * 6 + [_p]),
    "ws_moe_swiglu_route": (_i, [_p] * 4 + [_i64, _i64, _p]),
    "ws_moe_grouped_glu_quant": (_i, [_p] * 12 + [_i64, _i64, _i64, _i64, _i64, _f, _p]),
    "ws_moe_grouped_down": (_i, [_p] * 7 + [_i64, _i64, _i64, _i64, _p]),
    "ws_moe_combine_f32": (_i, [_p] * 3 + [_i64, _i64, _i64, _i64, _p]),
    "ws_moe_prefill_workspace_size": (C.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "ws_moe_prefill": (_i, [_p] * 10 + [_i64] * 5 + [_f, _p, C.c_size_t, _p]),
}


def _declare(lib):
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args


class WsError(RuntimeError):
    def __init__(self, fn, code):
        msg = load().ws_error_string(code).decode()  # same strings in both builds
        super().__init__("%s failed: %s (code %d)" % (fn, msg, code))
        self.code = code


def check(fn, code):
    """Raise on a nonzero status, as launch.rs `.unwrap()`s every launch."""
    if code != 0:
        raise WsError(fn, code)
