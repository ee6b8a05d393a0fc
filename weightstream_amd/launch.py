"""Host mirror of weightstream-gpu's launch.rs over the HIP C ABI.

One function per reference wrapper, same names and argument order as
weightstream-gpu/src/launch.rs, minus the `&Cuda` handle, which is replaced
by an optional `stream=` keyword (the `*_on` variants). Arguments are torch
device tensors (their data pointers are passed) or plain ints/floats. Every
call enqueues on the stream and returns immediately; a rejected argument or a
failed launch raises WsError, where launch.rs panics.

`Hip.global()` mirrors weightstream_cuda::gpu::Cuda::global() (gpu.rs:93):
one process-wide handle holding `stream` and `aux_stream`.
"""
import threading

import torch

from . import _lib

_lock = threading.Lock()


class Hip:
    """Process-wide runtime handle (gpu.rs:42-81): a main and an aux stream."""
    _inst = None

    def __init__(self):
        lib = _lib.load()
        _lib.check("ws_init", lib.ws_init())
        self.stream = torch.cuda.current_stream()
        self.aux_stream = torch.cuda.Stream()

    @classmethod
    def global_(cls):
        with _lock:
            if cls._inst is None:
                cls._inst = Hip()
            return cls._inst


def built_with_hip():
    """weightstream-cuda lib.rs:11-13 built_with_cuda()."""
    return bool(_lib.load().ws_built_with_hip())


MATH_EXACT, MATH_NATIVE = 0, 1

# Which library build the calls below go to. The math mode is fixed inside
# each library (no C-side state); this host-side choice only picks the build.
_mode = threading.local()


def _native():
    return getattr(_mode, "native", False)


def set_math_mode(mode):
    """Route this thread's later calls to the EXACT library
    (libweightstream_hip.so, bf16 MFMA on exactly dequantised operands) or to
    the NATIVE build (FP8/MXFP4 scaled MFMA). Returns the previous mode."""
    if mode not in (MATH_EXACT, MATH_NATIVE):
        raise ValueError("unknown math mode %r" % (mode,))
    prev = MATH_NATIVE if _native() else MATH_EXACT
    _mode.native = mode == MATH_NATIVE
    _lib.load(native=_mode.native)
    return prev


def get_math_mode():
    """The math mode of the library the calls go to (asked of the library)."""
    return _lib.load(native=_native()).ws_get_math_mode()


class math_mode:
    """Context manager: `with math_mode(MATH_NATIVE): ...`."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        self.prev = set_math_mode(self.mode)

    def __exit__(self, *exc):
        set_math_mode(self.prev)


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise ValueError("weightstream_amd expects device tensors")
    return t.data_ptr()


def _s(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _call(name, *args):
    fn = getattr(_lib.load(native=_native()), name)
    _lib.check(name, fn(*args))


# ---- actquant.cu (launch.rs:296-326) -------------------------------------
def snap8(x, n, stream=None):
    _call("ws_snap8", _ptr(x), n, _s(stream))


def emit8(x, q, s, n, stream=None):
    _call("ws_emit8", _ptr(x), _ptr(q), _ptr(s), n, _s(stream))


def emit8_packed(x, q, s, n, stream=None):
    _call("ws_emit8_packed", _ptr(x), _ptr(q), _ptr(s), n, _s(stream))


def pack_scales(src, dst, n, stream=None):
    _call("ws_pack_scales", _ptr(src), _ptr(dst), n, _s(stream))


def act_quant_f32s(x, q, s, m, k, stream=None):
    _call("ws_act_quant_f32s", _ptr(x), _ptr(q), _ptr(s), m, k, _s(stream))


def weight_quant_fp4(w, q, s, rows, cols, stream=None):
    _call("ws_weight_quant_fp4", _ptr(w), _ptr(q), _ptr(s), rows, cols, _s(stream))


def weight_quant_fp8(w, q, s, rows, cols, stream=None):
    _call("ws_weight_quant_fp8", _ptr(w), _ptr(q), _ptr(s), rows, cols, _s(stream))


def packed_fp4_scale_bytes(rows, cols):
    return int(_lib.load().ws_packed_fp4_scale_bytes(rows, cols))


def prepack_fp4(w, s, rows, cols, pw, ps, stream=None):
    """On-disk FP4 layout -> the fragment-major layout the expert kernels read."""
    _call("ws_prepack_fp4", _ptr(w), _ptr(s), rows, cols, _ptr(pw), _ptr(ps), _s(stream))


def prepack_fp4_new(w, s, rows, cols, stream=None):
    """Allocate and fill the packed copy of (w, s); returns (pw, ps)."""
    pw = torch.empty(rows * cols // 2, dtype=torch.uint8, device=w.device)
    ps = torch.empty(packed_fp4_scale_bytes(rows, cols), dtype=torch.uint8, device=w.device)
    prepack_fp4(w, s, rows, cols, pw, ps, stream=stream)
    return pw, ps


# ---- GEMMs (launch.rs:344-377, 717-804) -------------------------------------
def gemm_workspace_size(m, n, k):
    """Bytes of split-K workspace the GEMMs need for (m, n, k)."""
    return int(_lib.load().ws_gemm_workspace_size(m, n, k))


def set_gemm_workspace(ws, stream=None):
    """Register (a uint8 device tensor) or clear (None) the split-K workspace
    of `stream` (default: the current stream) on the current device; GEMMs
    issued on that stream use it. The caller keeps `ws` alive while it is
    set. The registration goes to every library build (EXACT and NATIVE), so a
    GEMM on `stream` takes the split-K path whichever math mode it runs in."""
    ptr, size = (None, 0) if ws is None else (_ptr(ws), ws.numel() * ws.element_size())
    for native in (False, True):
        try:
            lib = _lib.load(native=native)
        except RuntimeError:
            if native != _native():
                continue        # that build is absent; only the active one must exist
            raise
        _lib.check("ws_set_gemm_workspace", lib.ws_set_gemm_workspace(ptr, size, _s(stream)))



def fp8_gemm(a, sa, b, sb, out, m, n, k, stream=None):
    _call("ws_fp8_gemm", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m, n, k, _s(stream))


def fp8_gemm_acc(a, sa, b, sb, c, m, n, k, stream=None):
    """c += a . b^T (fp8_gemm then acc_f32, launch.rs:717-742 and :1175-1179,
    the add in the GEMM's epilogue: the same bits)."""
    _call("ws_fp8_gemm_acc", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(c), m, n, k, _s(stream))


def fp8_gemm_on(a, sa, b, sb, out, m, n, k, stream):
    fp8_gemm(a, sa, b, sb, out, m, n, k, stream=stream)


def fp8_gemm_tile(a, sa, b, sb, out, m, n, k, stream=None):
    _call("ws_fp8_gemm_tile", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m, n, k,
          _s(stream))


# launch.rs:325-339 TlGemm kinds: (N, K) hard-coded per TileLang kernel
TL_QA, TL_QB, TL_WKV, TL_WO_A, TL_WO_B, TL_SHARED_W13, TL_SHARED_W13_FUSED, TL_SHARED_W2, \
    TL_ENGRAM_WKV, TL_DRAFTER_MAIN_PROJ = range(10)


def tl_gemm_shape(kind):
    """(N, K) of a TlGemm kind."""
    import ctypes
    n, k = ctypes.c_int64(), ctypes.c_int64()
    _lib.check("ws_tl_gemm_shape", _lib.load().ws_tl_gemm_shape(kind, ctypes.byref(n),
                                                                 ctypes.byref(k)))
    return n.value, k.value


def fp8_gemm_tl(kind, a, sa, b, sb, out, m, stream=None):
    """launch.rs:341 fp8_gemm_tl: sa = the activation's packed scale words,
    sb = the weight's packed per-row scale table (pack_weight_scales)."""
    _call("ws_fp8_gemm_tl", int(kind), _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m,
          _s(stream))


def fp8_gemm_tl_on(kind, a, sa, b, sb, out, m, stream):
    fp8_gemm_tl(kind, a, sa, b, sb, out, m, stream=stream)


def fp8_gemm_bf16(a, sa, b, sb, out, m, n, k, stream=None):
    _call("ws_fp8_gemm_bf16", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m, n, k,
          _s(stream))


def fp8_gemm_f32s(a, sa, b, sb, out, m, n, k, out_bf16=False, stream=None):
    _call("ws_fp8_gemm_f32s", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), int(out_bf16),
          m, n, k, _s(stream))


def fp4_gemm(a, sa, b, sb, out, m, n, k, stream=None):
    _call("ws_fp4_gemm", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m, n, k, _s(stream))


def fp4_gemm_tile(a, sa, b, sb, out, m, n, k, stream=None):
    _call("ws_fp4_gemm_tile", _ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(out), m, n, k,
          _s(stream))


# ---- routing (launch.rs:998-1100) ---------------------------------------------
SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSOFTPLUS = 0, 1, 2


def moe_gate_logits(x, gate_w, logits, m, dim, n_experts, stream=None):
    bf16 = gate_w.dtype in (torch.bfloat16, torch.int16, torch.uint16)
    _call("ws_moe_gate_logits", _ptr(x), _ptr(gate_w), int(bf16), _ptr(logits), m, dim,
          n_experts, _s(stream))


def moe_topk(logits, bias, scores_out, out_idx, out_w, m, n_experts, top_k,
             score_func=SCORE_SIGMOID, gate_temp=1.0, norm_topk_prob=True, route_scale=1.0,
             stream=None):
    _call("ws_moe_topk", _ptr(logits), _ptr(bias), _ptr(scores_out), _ptr(out_idx),
          _ptr(out_w), m, n_experts, top_k, score_func, gate_temp, int(norm_topk_prob),
          route_scale, _s(stream))


def moe_gate(x, gate_w, bias, scores, dim, n_experts, stream=None):
    _call("ws_moe_gate", _ptr(x), _ptr(gate_w), _ptr(bias), _ptr(scores), dim, n_experts,
          _s(stream))


def moe_gate_m(x, gate_w, bias, scores, m, dim, n_experts, stream=None):
    _call("ws_moe_gate_m", _ptr(x), _ptr(gate_w), _ptr(bias), _ptr(scores), m, dim, n_experts,
          _s(stream))


def moe_select(scores, bias, out_w, out_i, n_experts, top_k, route_scale, stream=None):
    _call("ws_moe_select", _ptr(scores), _ptr(bias), _ptr(out_w), _ptr(out_i), n_experts, top_k,
          route_scale, _s(stream))


def moe_route(x, gate_w, bias, out_w, out_i, dim, n_experts, top_k, route_scale, stream=None):
    _call("ws_moe_route", _ptr(x), _ptr(gate_w), _ptr(bias), _ptr(out_w), _ptr(out_i), dim,
          n_experts, top_k, route_scale, _s(stream))


def swiglu(gate, up, out, n, rw, stream=None):
    _call("ws_swiglu", _ptr(gate), _ptr(up), _ptr(out), n, rw, _s(stream))


def acc_f32(x, y, n, stream=None):
    """launch.rs:1175 acc_f32: y += x."""
    _call("ws_acc_f32", _ptr(x), _ptr(y), n, _s(stream))


def shared_expert_workspace_size(m, dim, inter):
    return int(_lib.load().ws_shared_expert_workspace_size(m, dim, inter))


def shared_expert_fp8_w13(x, w13, s13, w2, s2, y, m, dim, inter, workspace, swiglu_limit=10.0,
                          stream=None):
    """The shared expert with w1 / w3 fused row-wise into w13 [2 * inter, dim]
    (engine.rs:1520 load_q8_combined_rows, :4067 one GEMM for gate and up)."""
    _call("ws_shared_expert_fp8_w13", _ptr(x), _ptr(w13), _ptr(s13), _ptr(w2), _ptr(s2), _ptr(y),
          m, dim, inter, swiglu_limit, _ptr(workspace),
          workspace.numel() * workspace.element_size(), _s(stream))


def fp8_gemv_acc(x, w, sw, h, m, n, k, stream=None):
    """h[m, n] += emit8(x) . w^T in one launch (emit8 + fp8_gemm + acc_f32,
    launch.rs:1175; m <= 16)."""
    _call("ws_fp8_gemv_acc", _ptr(x), _ptr(w), _ptr(sw), _ptr(h), m, n, k, _s(stream))


def shared_expert_fp8_w13_acc(x, w13, s13, w2, s2, yr, h, m, dim, inter, workspace,
                              swiglu_limit=10.0, stream=None):
    """h = h + (yr + shared(x)): the shared expert, engine.rs:4532's
    y_moe += expert_y and the residual add, fused (two launches for m <= 16)."""
    _call("ws_shared_expert_fp8_w13_acc", _ptr(x), _ptr(w13), _ptr(s13), _ptr(w2), _ptr(s2),
          _ptr(yr), _ptr(h), m, dim, inter, swiglu_limit, _ptr(workspace),
          workspace.numel() * workspace.element_size(), _s(stream))


def moe_gate_shared_w13(h, gate_w, logits, w13, s13, hs, m, dim, n_experts, inter,
                        swiglu_limit=10.0, stream=None):
    """Gate logits (f32 gate) and the shared expert's SwiGLU hidden state hs
    (f32) in one launch (m <= 8)."""
    _call("ws_moe_gate_shared_w13", _ptr(h), _ptr(gate_w), _ptr(logits), _ptr(w13), _ptr(s13),
          _ptr(hs), m, dim, n_experts, inter, swiglu_limit, _s(stream))


def shared_expert_down_acc(hs, w2, s2, yr, h, m, dim, inter, stream=None):
    """h = h + (yr + emit8(hs) . w2^T) in one launch (m <= 16)."""
    _call("ws_shared_expert_down_acc", _ptr(hs), _ptr(w2), _ptr(s2), _ptr(yr), _ptr(h), m, dim,
          inter, _s(stream))


def shared_expert_fp8(x, w1, s1, w3, s3, w2, s2, y, m, dim, inter, workspace,
                      swiglu_limit=10.0, stream=None):
    """moe.rs:210-250 shared_expert_hidden for m tokens (engine.rs:4063
    moe_shared_step): FP8 gate/up, SwiGLU, FP8 down; y written."""
    _call("ws_shared_expert_fp8", _ptr(x), _ptr(w1), _ptr(s1), _ptr(w3), _ptr(s3), _ptr(w2),
          _ptr(s2), _ptr(y), m, dim, inter, swiglu_limit, _ptr(workspace),
          workspace.numel() * workspace.element_size(), _s(stream))


# ---- routed experts, decode (launch.rs:89-206) ---------------------------------
def moe_local_slots(gate_idx, local_slots, local_experts, local_count, top_k, e_start, e_len,
                    stream=None):
    """launch.rs:89: the gate's picks in [e_start, e_start + e_len), ascending
    expert id, as slot indices and local expert rows."""
    _call("ws_moe_local_slots", _ptr(gate_idx), _ptr(local_slots), _ptr(local_experts),
          _ptr(local_count), top_k, e_start, e_len, _s(stream))


def moe_dispatch_ids(gate_idx, dispatch_idx, top_k, e_start, e_len, stream=None):
    """launch.rs:658: int64 local expert rows (-1: another rank's)."""
    _call("ws_moe_dispatch_ids", _ptr(gate_idx), _ptr(dispatch_idx), top_k, e_start, e_len,
          _s(stream))


def expert_glu(act_x, act_x_s, w1, w1_s, w3, w3_s, route_w, local_slots, local_experts,
               local_count, h_slots, n, k, top_k, e_len, stream=None):
    """launch.rs:116: f32 h of each local slot (packed w1 / w3 slabs of e_len
    experts)."""
    _call("ws_expert_glu", _ptr(act_x), _ptr(act_x_s), _ptr(w1), _ptr(w1_s), _ptr(w3),
          _ptr(w3_s), _ptr(route_w), _ptr(local_slots), _ptr(local_experts), _ptr(local_count),
          _ptr(h_slots), n, k, top_k, e_len, _s(stream))


def expert_quant(h_slots, local_slots, local_count, q_slots, s_slots, n, top_k, stream=None):
    """launch.rs:148: FP8 1x32 emit of each local slot's h row."""
    _call("ws_expert_quant", _ptr(h_slots), _ptr(local_slots), _ptr(local_count), _ptr(q_slots),
          _ptr(s_slots), n, top_k, _s(stream))


def expert_reduce(act_slots, act_s_slots, w2, w2_s, gate_idx, local_slots, local_count, y, dim,
                  inter, top_k, e_start, e_len, stream=None):
    """launch.rs:178: y = sum over local_slots (ascending expert id) of
    w2_e . h_slot."""
    _call("ws_expert_reduce", _ptr(act_slots), _ptr(act_s_slots), _ptr(w2), _ptr(w2_s),
          _ptr(gate_idx), _ptr(local_slots), _ptr(local_count), _ptr(y), dim, inter, top_k,
          e_start, e_len, _s(stream))


def expert_glu_quant(act_x, act_x_s, topk_idx, topk_w, w1, w1_s, w3, w3_s, q_slots, s_slots,
                     n, k, n_experts, top_k, swiglu_limit=10.0, stream=None):
    """expert_glu + expert_quant fused for the picks of the top-k output: row p
    of q_slots / s_slots is pick p."""
    _call("ws_expert_glu_quant", _ptr(act_x), _ptr(act_x_s), _ptr(topk_idx), _ptr(topk_w),
          _ptr(w1), _ptr(w1_s), _ptr(w3), _ptr(w3_s), _ptr(q_slots), _ptr(s_slots), k, n,
          n_experts, top_k, swiglu_limit, _s(stream))


def expert_glu_quant_x(x, topk_idx, topk_w, w1, w1_s, w3, w3_s, q_slots, s_slots, n, k,
                       n_experts, top_k, swiglu_limit=10.0, stream=None):
    """expert_glu_quant with the FP8 activation quantisation of f32 x fused in."""
    _call("ws_expert_glu_quant_x", _ptr(x), _ptr(topk_idx), _ptr(topk_w), _ptr(w1), _ptr(w1_s),
          _ptr(w3), _ptr(w3_s), _ptr(q_slots), _ptr(s_slots), k, n, n_experts, top_k,
          swiglu_limit, _s(stream))


def expert_glu_quant_route(logits, bias, score_func, gate_temp, norm_topk_prob, route_scale, x,
                           w1, s1, w3, s3, hq, hs, topk_idx, topk_w, dim, inter, n_experts, top_k,
                           swiglu_limit=10.0, stream=None):
    """The gate/up kernel of moe_decode_route on its own: routing from the
    logits fused in; picks to topk_idx / topk_w, hidden states to hq / hs."""
    _call("ws_expert_glu_quant_route", _ptr(logits), _ptr(bias), int(score_func), float(gate_temp),
          int(norm_topk_prob), float(route_scale), _ptr(x), _ptr(w1), _ptr(s1), _ptr(w3),
          _ptr(s3), _ptr(hq), _ptr(hs), _ptr(topk_idx), _ptr(topk_w), dim, inter, n_experts,
          top_k, swiglu_limit, _s(stream))


def moe_decode_workspace_size(dim, inter, top_k):
    return int(_lib.load().ws_moe_decode_workspace_size(dim, inter, top_k))


def moe_decode(x, topk_idx, topk_w, w1, s1, w3, s3, w2, s2, y, dim, inter, n_experts, top_k,
               workspace, swiglu_limit=10.0, stream=None):
    _call("ws_moe_decode", _ptr(x), _ptr(topk_idx), _ptr(topk_w), _ptr(w1), _ptr(s1), _ptr(w3),
          _ptr(s3), _ptr(w2), _ptr(s2), _ptr(y), dim, inter, n_experts, top_k, swiglu_limit,
          _ptr(workspace), workspace.numel() * workspace.element_size(), _s(stream))


def moe_decode_route(logits, bias, score_func, gate_temp, norm_topk_prob, route_scale, x, w1, s1,
                     w3, s3, w2, s2, y, topk_idx, topk_w, dim, inter, n_experts, top_k,
                     workspace, swiglu_limit=10.0, stream=None):
    """moe_select fused with the routed MoE for one token (two kernels): the
    picks land in topk_idx / topk_w, the output in y."""
    _call("ws_moe_decode_route", _ptr(logits), _ptr(bias), int(score_func), float(gate_temp),
          int(norm_topk_prob), float(route_scale), _ptr(x), _ptr(w1), _ptr(s1), _ptr(w3),
          _ptr(s3), _ptr(w2), _ptr(s2), _ptr(y), _ptr(topk_idx), _ptr(topk_w), dim, inter,
          n_experts, top_k, swiglu_limit, _ptr(workspace),
          workspace.numel() * workspace.element_size(), _s(stream))


def moe_decode_route_shared(logits, bias, score_func, gate_temp, norm_topk_prob, route_scale, x,
                            w1, s1, w3, s3, w2, s2, y, topk_idx, topk_w, dim, inter, n_experts,
                            top_k, hs_shared, w2_shared, s2_shared, shared_inter, ys, h,
                            workspace, swiglu_limit=10.0, stream=None):
    """moe_decode_route with the shared down GEMV on extra workgroups of the
    gate/up launch and h = h + (y + ys) at the end of the down kernel."""
    _call("ws_moe_decode_route_shared", _ptr(logits), _ptr(bias), int(score_func),
          float(gate_temp), int(norm_topk_prob), float(route_scale), _ptr(x), _ptr(w1), _ptr(s1),
          _ptr(w3), _ptr(s3), _ptr(w2), _ptr(s2), _ptr(y), _ptr(topk_idx), _ptr(topk_w), dim,
          inter, n_experts, top_k, swiglu_limit, _ptr(hs_shared), _ptr(w2_shared),
          _ptr(s2_shared), shared_inter, _ptr(ys), _ptr(h), _ptr(workspace),
          workspace.numel() * workspace.element_size(), _s(stream))


def moe_decode_route_noalloc(logits, bias, score_func, gate_temp, norm_topk_prob, route_scale, x,
                             w1, s1, w3, s3, w2, s2, y, topk_idx, topk_w, dim, inter, n_experts,
                             top_k, swiglu_limit=10.0, stream=None):
    """moe_decode_route on the library's fixed device scratch (no workspace,
    no allocation; calls that overlap on one GPU race)."""
    _call("ws_moe_decode_route_noalloc", _ptr(logits), _ptr(bias), int(score_func),
          float(gate_temp), int(norm_topk_prob), float(route_scale), _ptr(x), _ptr(w1), _ptr(s1),
          _ptr(w3), _ptr(s3), _ptr(w2), _ptr(s2), _ptr(y), _ptr(topk_idx), _ptr(topk_w), dim,
          inter, n_experts, top_k, swiglu_limit, _s(stream))


# ---- routed experts, M tokens (launch.rs:430-689) -------------------------------
def moe_tiles(routes, n_experts):
    """Upper bound on 32-slot tiles (engine.rs:4131, 6232-6233)."""
    return (routes + 31) // 32 + min(routes, n_experts)


def moe_dispatch_tl(topk_idx, topk_weights, order, layout_weights, route_pos, tile_expert,
                    expert_count, expert_offset, expert_psum, num_tiles, rows, top_k, tiles,
                    n_experts, stream=None):
    """launch.rs:430: int64 ids (moe_dispatch_ids) go to ws_moe_dispatch_tl,
    int32 ids (moe_topk) to ws_moe_dispatch; same outputs."""
    name = "ws_moe_dispatch_tl" if topk_idx.dtype == torch.int64 else "ws_moe_dispatch"
    _call(name, _ptr(topk_idx), _ptr(topk_weights), _ptr(order), _ptr(layout_weights),
          _ptr(route_pos), _ptr(tile_expert), _ptr(expert_count), _ptr(expert_offset),
          _ptr(expert_psum), _ptr(num_tiles), rows, top_k, tiles, n_experts, _s(stream))


TL_MOE_GATE_UP, TL_MOE_DOWN = 0, 1


def moe_grouped_tl(kind, a, sfa, weights, sfb, order, tile_expert, out, tiles, tokens, top_k,
                   n, k, n_experts, stream=None):
    """launch.rs:478-580 moe_grouped_tl(_cached)(_on): out[slot] = A row .
    w_e^T for the used tiles; GATE_UP gathers the routes' token rows, DOWN
    reads the slot rows. weights / sfb: a packed slab (prepack_fp4)."""
    _call("ws_moe_grouped_tl", int(kind), _ptr(a), _ptr(sfa), _ptr(weights), _ptr(sfb),
          _ptr(order), _ptr(tile_expert), _ptr(out), tiles, tokens, top_k, n, k, n_experts,
          _s(stream))


moe_grouped_tl_cached = moe_grouped_tl


def moe_grouped_tl_cached_on(kind, a, sfa, weights, sfb, order, tile_expert, out, tiles, tokens,
                             top_k, stream, *, n, k, n_experts):
    """launch.rs:542 argument order: the stream right after top_k; the slab's
    shape (n, k, n_experts), which the reference reads from its tensor map,
    as keywords."""
    moe_grouped_tl(kind, a, sfa, weights, sfb, order, tile_expert, out, tiles, tokens, top_k, n,
                   k, n_experts, stream=stream)


def moe_swiglu_route(gate, up, weights, out, inter, rows, stream=None):
    """launch.rs:673: route-weighted SwiGLU over the grouped layout."""
    _call("ws_moe_swiglu_route", _ptr(gate), _ptr(up), _ptr(weights), _ptr(out), inter, rows,
          _s(stream))


def moe_grouped_glu_quant(xq, xs, order, layout_w, tile_expert, num_tiles, w1, s1, w3, s3, hq,
                          hs, dim, inter, n_experts, top_k, tiles, swiglu_limit=10.0,
                          stream=None):
    _call("ws_moe_grouped_glu_quant", _ptr(xq), _ptr(xs), _ptr(order), _ptr(layout_w),
          _ptr(tile_expert), _ptr(num_tiles), _ptr(w1), _ptr(s1), _ptr(w3), _ptr(s3), _ptr(hq),
          _ptr(hs), dim, inter, n_experts, top_k, tiles, swiglu_limit, _s(stream))


def moe_grouped_down(hq, hs, tile_expert, num_tiles, w2, s2, out, dim, inter, n_experts, tiles,
                     stream=None):
    _call("ws_moe_grouped_down", _ptr(hq), _ptr(hs), _ptr(tile_expert), _ptr(num_tiles),
          _ptr(w2), _ptr(s2), _ptr(out), dim, inter, n_experts, tiles, _s(stream))


def moe_combine_f32(y, route_pos, out, dim, top_k, rows, tiles, stream=None):
    """launch.rs:689 (y = grouped down output, out = result; trailing tiles
    bounds the slots)."""
    _call("ws_moe_combine_f32", _ptr(y), _ptr(route_pos), _ptr(out), dim, top_k, rows, tiles,
          _s(stream))


def moe_prefill_workspace_size(rows, dim, inter, top_k, n_experts):
    return int(_lib.load().ws_moe_prefill_workspace_size(rows, dim, inter, top_k, n_experts))


def moe_prefill(x, topk_idx, topk_w, w1, s1, w3, s3, w2, s2, y, rows, dim, inter, n_experts,
                top_k, workspace, swiglu_limit=10.0, stream=None):
    _call("ws_moe_prefill", _ptr(x), _ptr(topk_idx), _ptr(topk_w), _ptr(w1), _ptr(s1), _ptr(w3),
          _ptr(s3), _ptr(w2), _ptr(s2), _ptr(y), rows, dim, inter, n_experts, top_k, swiglu_limit,
          _ptr(workspace), workspace.numel() * workspace.element_size(), _s(stream))
