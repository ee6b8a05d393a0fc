"""ctypes binding of the C oracle (oracle/liboracle.so).

Test infrastructure: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg only. It is the checker, never the product.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")

_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_sz = C.c_size_t

SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSOFTPLUS = 0, 1, 2


def _load(name):
    path = os.path.join(ORACLE_DIR, name)
    if not os.path.exists(path):
        subprocess.check_call(["make", "-s", "-C", ORACLE_DIR])
    return C.CDLL(path)


lib = _load("liboracle.so")

_sigs = {
    "or_e4m3_to_f32": (C.c_float, [C.c_uint8]),
    "or_f32_to_e4m3": (C.c_uint8, [C.c_float]),
    "or_f32_to_e2m1": (C.c_uint8, [C.c_float]),
    "or_e8m0_to_f32": (C.c_float, [C.c_uint8]),
    "or_log2_ceil": (C.c_int32, [C.c_float]),
    "or_pow2i": (C.c_float, [C.c_int32]),
    "or_ue8m0_round_scale": (C.c_float, [C.c_float, C.c_float]),
    "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
    "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "or_fp4_value": (C.c_float, [C.c_uint8]),
    "or_pack_fp4": (C.c_uint8, [C.c_uint8, C.c_uint8]),
    "or_dequant_fp8_blockwise": (None, [_u8p, _u8p, _sz, _sz, _f32p]),
    "or_dequant_fp4_packed": (None, [_u8p, _u8p, _sz, _sz, _f32p]),
    "or_fp8_snap": (None, [_f32p, _sz, _sz]),
    "or_fp4_snap_e8m0": (None, [_f32p, _sz, _sz]),
    "or_fp4_snap_e4m3": (None, [_f32p, _sz, _sz]),
    "or_fp8_act_emit": (None, [_f32p, _sz, _u8p, _u8p]),
    "or_fp8_gemv": (None, [_u8p, _u8p, _sz, _sz, _f32p, _f32p]),
    "or_fp4_gemv": (None, [_u8p, _u8p, _sz, _sz, _f32p, _f32p]),
    "or_gemm_q": (None, [_u8p, _u8p, _sz, _u8p, _u8p, _sz, _sz, C.c_int, _f32p]),
    "or_act_quant_f32s": (None, [_f32p, _sz, _sz, _sz, _u8p, _f32p]),
    "or_weight_quant_fp8_f32s": (None, [_f32p, _sz, _sz, _sz, _u8p, _f32p]),
    "or_gemm_f32s": (None, [_u8p, _f32p, _sz, _u8p, _f32p, _sz, _sz, _sz, _f32p]),
    "or_weight_quant_fp8": (None, [_f32p, _sz, _sz, _u8p, _u8p]),
    "or_weight_quant_fp4": (None, [_f32p, _sz, _sz, _u8p, _u8p]),
    "or_dot": (C.c_float, [_f32p, _f32p, _sz]),
    "or_gemv_f32": (None, [_f32p, _sz, _sz, _f32p, _f32p]),
    "or_sigmoid": (C.c_float, [C.c_float]),
    "or_silu": (C.c_float, [C.c_float]),
    "or_softplus": (C.c_float, [C.c_float]),
    "or_softmax": (None, [_f32p, _sz]),
    "or_expf": (C.c_float, [C.c_float]),
    "or_score": (None, [_f32p, _sz, C.c_int, C.c_float]),
    "or_route": (None, [_f32p, _f32p, _sz, _sz, C.c_int, C.c_float, _i32p, _f32p]),
    "or_expert_fp4": (None, [_u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _f32p,
                             C.c_float, C.c_float, _f32p]),
    "or_expert_hidden_fp4": (None, [_u8p, _u8p, _u8p, _u8p, _sz, _sz, _f32p, C.c_float,
                                     C.c_float, _f32p]),
    "or_shared_fp8": (None, [_u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _f32p,
                             C.c_float, _f32p]),
    "or_moe_routed": (None, [_u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _f32p, _i32p,
                             _f32p, _sz, C.c_float, _f32p]),
    "or_dispatch": (None, [_i32p, _f32p, _sz, _sz, _sz, _i32p, _f32p, _i32p, _i32p, _i32p,
                           _i32p, _i32p, _i32p]),
    "or_set_threads": (None, [C.c_int]),
    "or_probe_digest": (C.c_uint64, [C.c_int, C.c_uint64, C.c_uint64]),
    "or_probe_bytes": (None, [C.c_int, C.c_uint32, C.c_uint32, C.c_void_p]),
}
for _n, (_r, _a) in _sigs.items():
    _f = getattr(lib, _n)
    _f.restype = _r
    _f.argtypes = _a

# scalar primitives re-exported under their reference names
e4m3_to_f32 = lib.or_e4m3_to_f32
f32_to_e4m3 = lib.or_f32_to_e4m3
f32_to_e2m1 = lib.or_f32_to_e2m1
e8m0_to_f32 = lib.or_e8m0_to_f32
log2_ceil = lib.or_log2_ceil
pow2i = lib.or_pow2i
ue8m0_round_scale = lib.or_ue8m0_round_scale
f32_to_bf16 = lib.or_f32_to_bf16
bf16_to_f32 = lib.or_bf16_to_f32
pack_fp4 = lib.or_pack_fp4
sigmoid = lib.or_sigmoid
silu = lib.or_silu
softplus = lib.or_softplus
expf = lib.or_expf


def set_threads(n):
    """Threads for the oracle's GEMV row loops (1 = the reference's scalar loop)."""
    lib.or_set_threads(int(n))


def fp4_value(nib):
    return lib.or_fp4_value(nib)


def _p(a, t):
    return a.ctypes.data_as(t)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def e4m3_decode_table():
    return np.array([e4m3_to_f32(b) for b in range(256)], dtype=np.float32)


def dequant_fp8_blockwise(w, s, rows, cols):
    w, s = _c(w, np.uint8), _c(s, np.uint8)
    out = np.empty(rows * cols, np.float32)
    lib.or_dequant_fp8_blockwise(_p(w, _u8p), _p(s, _u8p), rows, cols, _p(out, _f32p))
    return out.reshape(rows, cols)


def dequant_fp4_packed(w, s, rows, cols):
    w, s = _c(w, np.uint8), _c(s, np.uint8)
    out = np.empty(rows * cols, np.float32)
    lib.or_dequant_fp4_packed(_p(w, _u8p), _p(s, _u8p), rows, cols, _p(out, _f32p))
    return out.reshape(rows, cols)


def fp8_snap(x, block=32):
    x = _c(x, np.float32).copy()
    lib.or_fp8_snap(_p(x, _f32p), x.size, block)
    return x


def fp4_snap_e8m0(x, block=32):
    x = _c(x, np.float32).copy()
    lib.or_fp4_snap_e8m0(_p(x, _f32p), x.size, block)
    return x


def fp4_snap_e4m3(x, block=16):
    x = _c(x, np.float32).copy()
    lib.or_fp4_snap_e4m3(_p(x, _f32p), x.size, block)
    return x


def fp8_act_emit(x):
    """f32 [.., K] -> (e4m3 bytes [.., K], UE8M0 bytes [.., K/32])."""
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.uint8)
    s = np.empty(x.shape[:-1] + (x.shape[-1] // 32,), np.uint8)
    lib.or_fp8_act_emit(_p(x, _f32p), x.size, _p(q, _u8p), _p(s, _u8p))
    return q, s


def fp8_gemv(w, s, rows, cols, x):
    w, s, x = _c(w, np.uint8), _c(s, np.uint8), _c(x, np.float32)
    y = np.empty(rows, np.float32)
    lib.or_fp8_gemv(_p(w, _u8p), _p(s, _u8p), rows, cols, _p(x, _f32p), _p(y, _f32p))
    return y


def fp4_gemv(w, s, rows, cols, x):
    w, s, x = _c(w, np.uint8), _c(s, np.uint8), _c(x, np.float32)
    y = np.empty(rows, np.float32)
    lib.or_fp4_gemv(_p(w, _u8p), _p(s, _u8p), rows, cols, _p(x, _f32p), _p(y, _f32p))
    return y


def gemm_q(aq, as_, M, w, ws, N, K, w_fp4):
    aq, as_, w, ws = (_c(a, np.uint8) for a in (aq, as_, w, ws))
    y = np.empty(M * N, np.float32)
    lib.or_gemm_q(_p(aq, _u8p), _p(as_, _u8p), M, _p(w, _u8p), _p(ws, _u8p), N, K,
                  int(bool(w_fp4)), _p(y, _f32p))
    return y.reshape(M, N)


def act_quant_f32s(x, block=128):
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty((M, K // block), np.float32)
    lib.or_act_quant_f32s(_p(x, _f32p), M, K, block, _p(q, _u8p), _p(s, _f32p))
    return q, s


def weight_quant_fp8_f32s(w, block=128):
    w = _c(w, np.float32)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(((N + block - 1) // block, K // block), np.float32)
    lib.or_weight_quant_fp8_f32s(_p(w, _f32p), N, K, block, _p(q, _u8p), _p(s, _f32p))
    return q, s


def gemm_f32s(aq, as_, w, ws, block=128):
    aq, w = _c(aq, np.uint8), _c(w, np.uint8)
    as_, ws = _c(as_, np.float32), _c(ws, np.float32)
    M, K = aq.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib.or_gemm_f32s(_p(aq, _u8p), _p(as_, _f32p), M, _p(w, _u8p), _p(ws, _f32p), N, K,
                     block, _p(y, _f32p))
    return y


def weight_quant_fp8(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty(((rows + 31) // 32, (cols + 31) // 32), np.uint8)
    lib.or_weight_quant_fp8(_p(w, _f32p), rows, cols, _p(q, _u8p), _p(s, _u8p))
    return q, s


def weight_quant_fp4(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols // 2), np.uint8)
    s = np.empty((rows, (cols + 31) // 32), np.uint8)
    lib.or_weight_quant_fp4(_p(w, _f32p), rows, cols, _p(q, _u8p), _p(s, _u8p))
    return q, s


def dot(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    return lib.or_dot(_p(a, _f32p), _p(b, _f32p), a.size)


def gemv_f32(w, x):
    w, x = _c(w, np.float32), _c(x, np.float32)
    n, k = w.shape
    y = np.empty(n, np.float32)
    lib.or_gemv_f32(_p(w, _f32p), n, k, _p(x, _f32p), _p(y, _f32p))
    return y


def softmax(x):
    x = _c(x, np.float32).copy()
    lib.or_softmax(_p(x, _f32p), x.size)
    return x


def score(logits, score_func=SCORE_SIGMOID, gate_temp=1.0):
    s = _c(logits, np.float32).copy()
    lib.or_score(_p(s, _f32p), s.size, score_func, gate_temp)
    return s


def route(scores, bias, top_k, norm_topk_prob=True, route_scale=1.0):
    scores, bias = _c(scores, np.float32), _c(bias, np.float32)
    idx = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    lib.or_route(_p(scores, _f32p), _p(bias, _f32p), scores.size, top_k,
                 int(bool(norm_topk_prob)), route_scale, _p(idx, _i32p), _p(w, _f32p))
    return idx, w


def expert_fp4(w1, s1, w3, s3, w2, s2, dim, inter, x, rw, limit=10.0):
    a = [_c(v, np.uint8) for v in (w1, s1, w3, s3, w2, s2)]
    x = _c(x, np.float32)
    y = np.empty(dim, np.float32)
    lib.or_expert_fp4(*[_p(v, _u8p) for v in a], dim, inter, _p(x, _f32p), rw, limit,
                      _p(y, _f32p))
    return y


def expert_hidden_fp4(w1, s1, w3, s3, dim, inter, x, rw, limit=10.0):
    """The expert's SwiGLU hidden state (times rw) before its FP8 snap."""
    a = [_c(v, np.uint8) for v in (w1, s1, w3, s3)]
    x = _c(x, np.float32)
    h = np.empty(inter, np.float32)
    lib.or_expert_hidden_fp4(*[_p(v, _u8p) for v in a], dim, inter, _p(x, _f32p), rw, limit,
                             _p(h, _f32p))
    return h


def shared_fp8(w1, s1, w3, s3, w2, s2, dim, inter, x, limit=10.0):
    a = [_c(v, np.uint8) for v in (w1, s1, w3, s3, w2, s2)]
    x = _c(x, np.float32)
    y = np.empty(dim, np.float32)
    lib.or_shared_fp8(*[_p(v, _u8p) for v in a], dim, inter, _p(x, _f32p), limit,
                      _p(y, _f32p))
    return y


def moe_routed(w1, s1, w3, s3, w2, s2, dim, inter, x, idx, w, limit=10.0):
    a = [_c(v, np.uint8) for v in (w1, s1, w3, s3, w2, s2)]
    x = _c(x, np.float32)
    idx, w = _c(idx, np.int32), _c(w, np.float32)
    y = np.empty(dim, np.float32)
    lib.or_moe_routed(*[_p(v, _u8p) for v in a], dim, inter, _p(x, _f32p), _p(idx, _i32p),
                      _p(w, _f32p), idx.size, limit, _p(y, _f32p))
    return y


def dispatch(topk_idx, topk_w, n_experts, tiles):
    ti, tw = _c(topk_idx, np.int32).ravel(), _c(topk_w, np.float32).ravel()
    routes = ti.size
    order = np.full(tiles * 32, -7, np.int32)
    lw = np.full(tiles * 32, -7.0, np.float32)
    rp = np.empty(routes, np.int32)
    te = np.empty(tiles, np.int32)
    cnt = np.empty(n_experts, np.int32)
    off = np.empty(n_experts, np.int32)
    ps = np.empty(n_experts, np.int32)
    nt = np.empty(1, np.int32)
    lib.or_dispatch(_p(ti, _i32p), _p(tw, _f32p), routes, n_experts, tiles, _p(order, _i32p),
                    _p(lw, _f32p), _p(rp, _i32p), _p(te, _i32p), _p(cnt, _i32p),
                    _p(off, _i32p), _p(ps, _i32p), _p(nt, _i32p))
    return dict(order=order, layout_w=lw, route_pos=rp, tile_expert=te, count=cnt,
                offset=off, psum=ps, num_tiles=int(nt[0]))


_expf_lib = None


def expfcheck():
    global _expf_lib
    if _expf_lib is None:
        _expf_lib = _load("libexpfcheck.so")
        _expf_lib.ws_expf_mismatches.restype = C.c_uint64
        _expf_lib.ws_expf_mismatches.argtypes = [C.c_uint64, C.c_uint64]
        _expf_lib.glibc_expf_digest.restype = C.c_uint64
        _expf_lib.glibc_expf_digest.argtypes = [C.c_uint64, C.c_uint64]
        _expf_lib.glibc_expf_bits.restype = None
        _expf_lib.glibc_expf_bits.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p]
        _expf_lib.ws_math_mismatches.restype = C.c_uint64
        _expf_lib.ws_math_mismatches.argtypes = [C.c_int, C.c_uint64, C.c_uint64]
        _expf_lib.glibc_math_digest.restype = C.c_uint64
        _expf_lib.glibc_math_digest.argtypes = [C.c_int, C.c_uint64, C.c_uint64]
        _expf_lib.glibc_math_bits.restype = None
        _expf_lib.glibc_math_bits.argtypes = [C.c_int, C.c_uint32, C.c_uint32, C.c_void_p]
    return _expf_lib
