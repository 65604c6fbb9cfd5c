"""MI355X (gfx950) pointer-table quantized MoE expert GEMV -- Python host mirror.

Thin ctypes bindings over the C ABI in include/ggml_hip_moe_cache.h (the
library built by build.py), mirroring the reference's operator interface
(kernels/moe-cache.cuh:15-40): enabled / wants / mul_mat_vec_q / step /
active / pin_host, plus the activation quantizers and introspection.

The HIP library is the only compute path.  Loading fails loudly when it has
not been built, and the GEMV/quantizer wrappers refuse non-GPU tensors.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libggml_hip_moe_cache.so"

# ggml_type numbering (ggml.h)
F32, Q4_0, Q5_0, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 0, 2, 6, 8, 9, 10, 11, 12, 13, 14, 15
WEIGHT_TYPES = (Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
KQUANTS = (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292)}
TYPE_NAMES = {Q4_0: "q4_0", Q5_0: "q5_0", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K",
              Q5_K: "q5_K", Q6_K: "q6_K", Q8_1: "q8_1", Q8_K: "q8_K"}

# GLU ops
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_GEGLU_ERF, GLU_GEGLU_QUICK, GLU_SWIGLU_CLAMP = range(7)
# activation formats
ACT_Q8_1, ACT_Q8_K, ACT_F32 = 0, 1, 2
ACT_SHARED_F32 = 0x100       # ffn_down_combine flag: the shared expert's rows are fp32
ACT_DOT_Q8_K = 0x200         # ffn_down_combine flag (fp32 rows): the dots run on q8_K of the rows
# graph node ops for fusion detection
OP_MUL_MAT, OP_MUL_MAT_ID, OP_ADD_ID, OP_MUL, OP_ADD, OP_GLU, OP_OTHER = range(1, 8)

MISS_CAP = 8190
STATS_WORDS = 2 + MISS_CAP


def row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    assert k % be == 0, (t, k)
    return k // be * bb


class Tensor(C.Structure):
    """ggml_hip_moe_tensor: POD mirror of the ggml_tensor fields the path reads."""
    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4), ("data", C.c_void_p),
                ("name", C.c_char_p), ("has_buffer", C.c_int32), ("is_view", C.c_int32)]


class Fusion(C.Structure):
    """ggml_hip_moe_fusion: mirror of ggml_cuda_mm_fusion_args_device (+ explicit extensions)."""
    _fields_ = [("gate", C.c_void_p), ("x_bias", C.c_void_p), ("gate_bias", C.c_void_p),
                ("x_scale", C.c_void_p), ("gate_scale", C.c_void_p), ("glu_op", C.c_int32),
                ("glu_limit", C.c_float), ("shared_up", C.c_void_p), ("shared_gate", C.c_void_p),
                ("shared_dst", C.c_void_p), ("shared_stride_col_dst", C.c_int64), ("shared_type", C.c_int32),
                ("shared_src1", C.c_void_p), ("shared_stride_col_y", C.c_int64), ("bias_stride", C.c_int64)]


class Node(C.Structure):
    """ggml_hip_moe_node: one graph node (op, result tensor, node-index or leaf sources)."""
    _fields_ = [("op", C.c_int32), ("t", Tensor), ("src", C.c_int32 * 3), ("leaf", Tensor * 3),
                ("glu_op", C.c_int32), ("glu_limit", C.c_float), ("glu_swapped", C.c_int32)]


class Config(C.Structure):
    _fields_ = [("enabled", C.c_int32), ("slots", C.c_int32), ("budget_gb", C.c_double), ("margin_gb", C.c_double),
                ("seed_path", C.c_char_p), ("max_promotions", C.c_int32), ("verbose", C.c_int32),
                ("async_promotions", C.c_int32)]


class EntryInfo(C.Structure):
    _fields_ = [("id", C.c_int32), ("type", C.c_int32), ("n_experts", C.c_int32), ("n_slots", C.c_int32),
                ("expert_bytes", C.c_uint64), ("n_resident", C.c_int32), ("stamps_clock", C.c_uint32)]


class Totals(C.Structure):
    _fields_ = [("steps", C.c_uint64), ("hits", C.c_uint64), ("misses", C.c_uint64), ("promotions", C.c_uint64),
                ("evictions", C.c_uint64), ("clock", C.c_uint32), ("last_step_misses", C.c_uint32),
                ("last_step_hits", C.c_uint32), ("admission_size", C.c_uint32)]


# (name, restype, argtypes) of every function in include/ggml_hip_moe_cache.h
_I64, _VP, _I32 = C.c_int64, C.c_void_p, C.c_int32
_GEMV_TAIL = [_I64] * 4 + [_I64] * 4 + [_I64] * 2 + [_I64] * 4 + [_I64, _VP]
SIGNATURES = [
    ("ggml_hip_moe_cache_enabled", C.c_int, []),
    ("ggml_hip_moe_cache_wants", C.c_int, [C.POINTER(Tensor)]),
    ("ggml_hip_moe_cache_mul_mat_vec_q", C.c_int,
     [C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, _VP] + _GEMV_TAIL),
    ("ggml_hip_moe_cache_step", C.c_int, [_VP]),
    ("ggml_hip_moe_cache_active", C.c_int, []),
    ("ggml_hip_moe_cache_pin_host", C.c_int, [C.POINTER(Tensor)]),
    ("ggml_hip_mul_mat_vec_q_moe", C.c_int, [C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, _VP] + _GEMV_TAIL),
    ("ggml_hip_moe_mul_mat_vec_ex", C.c_int,
     [C.c_int, C.c_int, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, _VP]
     + [_I64] * 3 + [_I64] * 3 + [_I64] * 4 + [_I64, _VP]),
    ("ggml_hip_quantize_q8_1", C.c_int, [_VP, _VP, _I64, _I64, _I64, _I64, _VP]),
    ("ggml_hip_quantize_q8_K", C.c_int, [_VP, _VP, _I64, _I64, _I64, _I64, _VP]),
    ("ggml_hip_quantize_q8_0_as_q8_1", C.c_int, [_VP, _VP, _I64, _I64, _I64, _I64, _VP]),
    ("ggml_hip_moe_combine_q8_1", C.c_int,
     [_VP, _I64, _VP, _I32, _VP, _I64, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP, C.c_float, _VP]),
    ("ggml_hip_moe_ffn_gate_up_norm", C.c_int,
     [C.c_int, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, C.c_float, _VP, _VP]
     + [_I64] * 3 + [_I64] * 2 + [_I64] * 4 + [_VP, _I64, _VP, _I64, _I64, _VP, _I64, _VP]),
    ("ggml_hip_moe_ffn_gate_up_norm_ex", C.c_int,
     [C.c_int, C.c_int, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, C.c_float, _VP, _VP]
     + [_I64] * 3 + [_I64] * 2 + [_I64] * 4 + [_VP, _I64, _VP, _I64, _I64, _VP, _I64, _VP]),
    ("ggml_hip_moe_ffn_down_combine", C.c_int,
     [C.c_int, C.c_int, C.POINTER(Tensor), C.POINTER(Fusion), _VP, _VP, _VP, _VP, _VP]
     + [_I64] * 3 + [_I64] * 2 + [_I64] * 4 + [_VP]),
    ("ggml_hip_moe_mul_mat_q_workspace_bytes", C.c_int64, [_I64, _I64, _I64]),
    ("ggml_hip_moe_mul_mat_q", C.c_int,
     [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _I64, _VP]),
    ("ggml_hip_moe_cache_configure", C.c_int, [C.POINTER(Config)]),
    ("ggml_hip_moe_cache_get_config", C.c_int, [C.POINTER(Config)]),
    ("ggml_hip_moe_cache_num_entries", C.c_int, []),
    ("ggml_hip_moe_cache_entry_info", C.c_int, [_I32, C.POINTER(EntryInfo)]),
    ("ggml_hip_moe_cache_entry_slots", C.c_int, [_I32, _VP, _I32, _VP, _I32]),
    ("ggml_hip_moe_cache_entry_table", C.c_int, [_I32, _VP, _I32]),
    ("ggml_hip_moe_cache_entry_device", C.c_int, [_I32, C.POINTER(_VP), C.POINTER(_VP), C.POINTER(_VP)]),
    ("ggml_hip_moe_cache_device_globals", C.c_int, [C.POINTER(_VP), C.POINTER(_VP)]),
    ("ggml_hip_moe_cache_stats_snapshot", C.c_int, [_VP, _I32, _VP]),
    ("ggml_hip_moe_cache_stamps_snapshot", C.c_int, [_I32, _VP, _I32, _VP]),
    ("ggml_hip_moe_cache_totals", C.c_int, [C.POINTER(Totals)]),
    ("ggml_hip_moe_cache_reset", C.c_int, []),
    ("ggml_hip_moe_mul_mat_id_workspace_bytes", C.c_int64,
     [C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion)]),
    ("ggml_hip_moe_mul_mat_id", C.c_int,
     [C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor),
      C.POINTER(Fusion), _VP, _I64, _VP]),
    ("ggml_hip_moe_mul_mat_id_noalloc", C.c_int,
     [C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Fusion), _VP]),
    ("ggml_hip_moe_fusion_detect", C.c_int,
     [C.POINTER(Node), _I32, _I32, C.POINTER(Fusion), C.POINTER(Tensor), C.POINTER(_I32), C.POINTER(_I32),
      C.POINTER(_I32)]),
    ("ggml_hip_ssm_conv_f32", C.c_int,
     [_VP, _I64, _I64, _I64, _VP, C.c_int32, _I64, _VP, C.c_int32, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
      _VP]),
    ("ggml_hip_moe_trace_append", C.c_int, [C.c_char_p, C.c_char_p, C.c_void_p, _I64, _I64, _I64]),
    ("ggml_hip_moe_trace_close", C.c_int, []),
    ("ggml_hip_moe_check_status", C.c_int, [_VP]),
    ("ggml_hip_moe_debug_set_spin_limit", C.c_int, [_I64]),
    ("ggml_hip_moe_last_error", C.c_char_p, []),
    ("ggml_hip_moe_version", C.c_char_p, []),
]


class MoeError(RuntimeError):
    pass


def bind(path) -> C.CDLL:
    lib = C.CDLL(str(path))
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


_lib = None


def lib() -> C.CDLL:
    """The gfx950 library; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise MoeError(f"{LIB_PATH} is missing: build it with `python a6000-custom-kernels_amd/build.py` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
        _lib = bind(LIB_PATH)
    return _lib


E_INVALID, E_UNSUPPORTED, E_DEVICE, E_DISABLED, E_STATE, E_TIMEOUT = -1, -2, -3, -4, -5, -6


def check(rc: int, what: str = "") -> int:
    if rc < 0:
        msg = lib().ggml_hip_moe_last_error().decode(errors="replace")
        raise MoeError(f"{what}: {msg} (rc={rc})")
    return rc


def make_tensor(wtype: int, ne00: int, ne01: int, ne02: int, data_ptr: int, name: str = "",
                has_buffer: bool = True, is_view: bool = False, keep: list | None = None) -> Tensor:
    t = Tensor()
    rb = row_bytes(wtype, ne00)
    t.type = wtype
    t.ne[:] = [ne00, ne01, ne02, 1]
    t.nb[:] = [BLOCK[wtype][1], rb, rb * ne01, rb * ne01 * ne02]
    t.data = data_ptr
    nm = name.encode()
    t.name = nm
    if keep is not None:
        keep.append(nm)
    t.has_buffer = 1 if has_buffer else 0
    t.is_view = 1 if is_view else 0
    return t


# ---------------------------------------------------------------------------
# torch-facing helpers (device memory + streams are torch's)
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise MoeError("HIP path requires device tensors (no CPU fallback)")


def quantize_q8_1(x, out=None, stream=None, kind: str = "q8_1"):
    """x: float32 [rows, k] on the GPU -> uint8 [rows, k/32*36] (q8_1 layout)."""
    torch = _torch()
    _require_gpu(x)
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, k // 32 * 36), dtype=torch.uint8, device=x.device)
    fn = lib().ggml_hip_quantize_q8_1 if kind == "q8_1" else lib().ggml_hip_quantize_q8_0_as_q8_1
    check(fn(x.data_ptr(), out.data_ptr(), k, rows, x.stride(0), out.stride(0) // 36, _stream(stream)), "quantize_q8_1")
    return out


def quantize_q8_K(x, out=None, stream=None):
    torch = _torch()
    _require_gpu(x)
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, k // 256 * 292), dtype=torch.uint8, device=x.device)
    check(lib().ggml_hip_quantize_q8_K(x.data_ptr(), out.data_ptr(), k, rows, x.stride(0), out.stride(0) // 292,
                                       _stream(stream)), "quantize_q8_K")
    return out


def make_fusion(*, gate=None, x_bias=None, gate_bias=None, x_scale=None, gate_scale=None, glu_op=GLU_SWIGLU,
                glu_limit=0.0, shared_up=None, shared_gate=None, shared_dst=None, shared_type=-1,
                shared_src1=None, shared_stride_col_y=0, bias_stride=0) -> Fusion:
    f = Fusion()
    f.gate = _ptr(gate)
    f.x_bias, f.gate_bias = _ptr(x_bias), _ptr(gate_bias)
    f.x_scale, f.gate_scale = _ptr(x_scale), _ptr(gate_scale)
    f.glu_op, f.glu_limit = glu_op, glu_limit
    f.shared_up, f.shared_gate, f.shared_dst = _ptr(shared_up), _ptr(shared_gate), _ptr(shared_dst)
    f.shared_stride_col_dst = shared_dst.shape[-1] if shared_dst is not None else 0
    f.shared_type = shared_type
    f.shared_src1 = _ptr(shared_src1)
    f.shared_stride_col_y = shared_stride_col_y
    f.bias_stride = bias_stride
    return f


def mul_mat_vec(*, wtype, weights, ids, y, dst, K, R, n_experts, use_cache=False, act=ACT_Q8_1, gate_host=None,
                fusion: Fusion | None = None, nchannels_y=1, name="", stream=None, weights_ptr=None, gate_ptr=None):
    """Run the GEMV through ggml_hip_moe_mul_mat_vec_ex.

    weights: device uint8 tensor [n_experts, R, row_bytes] (use_cache=False) or a pinned host pointer
    (weights_ptr, use_cache=True); ids: int32 [n_tok, n_used] (device); y: activation blocks,
    [n_tok, nchannels_y, act_row_bytes] (device), or fp32 rows [n_tok, nchannels_y, K] with act=ACT_F32;
    dst: float32 [n_tok, n_used, R] (device).
    """
    n_tok, n_used = ids.shape
    _require_gpu(ids, y, dst)
    keep = []
    ptr = weights_ptr if weights_ptr is not None else weights.data_ptr()
    src0 = make_tensor(wtype, K, R, n_experts, ptr, name=name, keep=keep)
    g = None
    if gate_ptr is not None:
        g = make_tensor(wtype, K, R, n_experts, gate_ptr, name=name.replace("up", "gate"), keep=keep)
    ablk = {ACT_Q8_1: (32, 36), ACT_Q8_K: (256, 292), ACT_F32: (1, 4)}[act]
    act_row = K // ablk[0]
    rc = lib().ggml_hip_moe_mul_mat_vec_ex(
        1 if use_cache else 0, act, C.byref(src0), C.byref(g) if g is not None else None,
        C.byref(fusion) if fusion is not None else None, y.data_ptr(), ids.data_ptr(), dst.data_ptr(),
        K, R, n_experts, n_tok, nchannels_y, n_used,
        nchannels_y * act_row, n_used * R, act_row, R, ids.stride(0), _stream(stream))
    check(rc, "mul_mat_vec")
    return dst


def ffn_gate_up_norm(*, wtype, weights, ids, x, dst, K, R, n_experts, norm_weight=None, eps=1e-6,
                     fusion: Fusion | None = None, y_out=None, dst_q8_1=None, shared_dst_q8_1=None, use_cache=False,
                     gate_host=None, name="", stream=None, weights_ptr=None, gate_ptr=None, act=ACT_Q8_1):
    """Gate/up GEMV whose activation is RMSNorm(x) * norm_weight, quantized to q8_1 (act=ACT_Q8_1) or
    q8_K (act=ACT_Q8_K) in the same launch (ggml_hip_moe_ffn_gate_up_norm_ex).  x: fp32 [n_tok, K]
    (device, 16-byte aligned rows); ids: int32 [n_tok, n_used]; dst: float32 [n_tok, n_used, R];
    y_out: optional uint8 [n_tok, K/32*36] (q8_1) or [n_tok, K/256*292] (q8_K);
    dst_q8_1 / shared_dst_q8_1: optional uint8 [n_tok, n_used, R/32*36] / [n_tok, R/32*36] q8_1 copies."""
    n_tok, n_used = ids.shape
    _require_gpu(ids, x, dst, norm_weight, y_out)
    keep = []
    ptr = weights_ptr if weights_ptr is not None else weights.data_ptr()
    src0 = make_tensor(wtype, K, R, n_experts, ptr, name=name, keep=keep)
    g = make_tensor(wtype, K, R, n_experts, gate_ptr, name=name.replace("up", "gate"), keep=keep) if gate_ptr else None
    yblk = 292 if act == ACT_Q8_K else 36
    rc = lib().ggml_hip_moe_ffn_gate_up_norm_ex(
        1 if use_cache else 0, act, C.byref(src0), C.byref(g) if g is not None else None,
        C.byref(fusion) if fusion is not None else None, x.data_ptr(), _ptr(norm_weight), eps, ids.data_ptr(),
        dst.data_ptr(), K, R, n_experts, n_tok, n_used, x.stride(0), n_used * R, R, ids.stride(0),
        _ptr(y_out), y_out.stride(0) // yblk if y_out is not None else 0,
        _ptr(dst_q8_1), dst_q8_1.stride(0) // 36 if dst_q8_1 is not None else 0,
        dst_q8_1.stride(1) // 36 if dst_q8_1 is not None else 0,
        _ptr(shared_dst_q8_1), shared_dst_q8_1.stride(0) // 36 if shared_dst_q8_1 is not None else 0, _stream(stream))
    check(rc, "ffn_gate_up_norm")
    return dst


def ffn_down_combine(*, wtype, weights, ids, h, router_w, x_out, K, R, n_experts, residual=None, act=ACT_F32,
                     fusion: Fusion | None = None, use_cache=False, name="", stream=None, weights_ptr=None):
    """Down GEMV over every pick plus the shared expert, combined into x_out = residual + shared +
    sum_c router_w[c] * o_c in the same launch (ggml_hip_moe_ffn_down_combine).
    h: pick rows [n_tok, n_used, K] fp32 (act=ACT_F32) or q8_1 blocks [n_tok, n_used, K/32*36];
    router_w: fp32 [n_tok, n_used]; x_out / residual: fp32 [n_tok, R]."""
    n_tok, n_used = ids.shape
    _require_gpu(ids, h, router_w, x_out, residual)
    keep = []
    ptr = weights_ptr if weights_ptr is not None else weights.data_ptr()
    src0 = make_tensor(wtype, K, R, n_experts, ptr, name=name, keep=keep)
    unit = 1 if (act & 0xFF) == ACT_F32 else 36   # h strides in floats or in q8_1 blocks
    rc = lib().ggml_hip_moe_ffn_down_combine(
        1 if use_cache else 0, act, C.byref(src0), C.byref(fusion) if fusion is not None else None, h.data_ptr(),
        ids.data_ptr(), router_w.data_ptr(), _ptr(residual), x_out.data_ptr(), K, R, n_experts, n_tok, n_used,
        h.stride(0) // unit, h.stride(1) // unit, x_out.stride(0), ids.stride(0), _stream(stream))
    check(rc, "ffn_down_combine")
    return x_out


def mul_mat_q(*, wtype, weights, ids, y, dst, K, R, n_experts, gate=None, glu_op=GLU_SWIGLU, glu_limit=0.0,
              nchannels_y=1, workspace=None, stream=None):
    """Prefill-shaped MUL_MAT_ID through ggml_hip_moe_mul_mat_q (expert-grouped int8 MFMA).

    weights/gate: device uint8 [n_experts, R, row_bytes] (Q4_K or Q5_K); ids: int32 [n_tok, n_used];
    y: q8_K rows [n_tok, nchannels_y, K/256*292] (device, 256-byte aligned); dst: float32 [n_tok, n_used, R].
    Returns dst.
    """
    torch = _torch()
    n_tok, n_used = ids.shape
    _require_gpu(weights, ids, y, dst, gate)
    keep = []
    src0 = make_tensor(wtype, K, R, n_experts, weights.data_ptr(), keep=keep)
    f = make_fusion(gate=gate, glu_op=glu_op, glu_limit=glu_limit) if gate is not None else None
    nbytes = int(lib().ggml_hip_moe_mul_mat_q_workspace_bytes(K, n_experts, n_tok * n_used))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dst.device)
    nb = K // 256
    rc = lib().ggml_hip_moe_mul_mat_q(C.byref(src0), C.byref(f) if f is not None else None, y.data_ptr(),
                                      ids.data_ptr(), dst.data_ptr(), K, R, n_experts, n_tok, nchannels_y, n_used,
                                      nchannels_y * nb, n_used * R, nb, R, ids.stride(0), workspace.data_ptr(),
                                      workspace.numel(), _stream(stream))
    check(rc, "mul_mat_q")
    return dst


def torch_tensor_desc(t, ggml_type: int, name: str = "", keep: list | None = None) -> Tensor:
    """ggml view of a torch tensor: ne / nb are the reversed shape / byte strides."""
    d = Tensor()
    es = t.element_size()
    ne = list(t.shape)[::-1]
    nb = [st * es for st in list(t.stride())[::-1]]
    while len(ne) < 4:                       # trailing dimensions of extent 1, contiguous
        nb.append(nb[-1] * ne[-1] if nb else es)
        ne.append(1)
    d.type = ggml_type
    d.ne[:] = ne
    d.nb[:] = nb
    d.data = t.data_ptr()
    nm = name.encode()
    d.name = nm
    if keep is not None:
        keep.append(nm)
    d.has_buffer = 1
    d.is_view = 0
    return d


GGML_F32, GGML_I32 = 0, 26


def mul_mat_id(*, wtype, weights, x, ids, dst, K, R, n_experts, fusion=None, workspace=None, stream=None):
    """MUL_MAT_ID at the op level through ggml_hip_moe_mul_mat_id.

    weights: device uint8 [n_experts, R, row_bytes]; x: float32 [tokens, channels, K] (rows contiguous);
    ids: int32 [tokens, >= n_used] (a column slice is a top-k view); dst: float32 [tokens, n_used, R]
    (any row strides).  Returns dst.
    """
    torch = _torch()
    _require_gpu(weights, x, ids, dst)
    keep = []
    src0 = make_tensor(wtype, K, R, n_experts, weights.data_ptr(), keep=keep)
    s1 = torch_tensor_desc(x, GGML_F32)
    it = torch_tensor_desc(ids, GGML_I32)
    dt = torch_tensor_desc(dst, GGML_F32)
    fp = C.byref(fusion) if fusion is not None else None
    nbytes = int(lib().ggml_hip_moe_mul_mat_id_workspace_bytes(C.byref(src0), C.byref(s1), C.byref(it), fp))
    if nbytes < 0:
        raise MoeError("mul_mat_id: " + lib().ggml_hip_moe_last_error().decode(errors="replace"))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dst.device)
    rc = lib().ggml_hip_moe_mul_mat_id(C.byref(src0), C.byref(s1), C.byref(it), C.byref(dt), None, fp,
                                       workspace.data_ptr(), workspace.numel(), _stream(stream))
    check(rc, "mul_mat_id")
    return dst


def fusion_detect(nodes, i_up, library=None):
    """Graph-level fusion detection through ggml_hip_moe_fusion_detect.

    nodes: a sequence of Node.  Returns (n_covered, fusion, gate_host or None, covered flags, out_node).
    """
    L = library if library is not None else lib()
    n = len(nodes)
    arr = (Node * n)(*nodes)
    f = Fusion()
    gh = Tensor()
    has_gh = C.c_int32(0)
    covered = (C.c_int32 * n)()
    out_node = C.c_int32(-1)
    rc = L.ggml_hip_moe_fusion_detect(arr, n, i_up, C.byref(f), C.byref(gh), C.byref(has_gh), covered,
                                      C.byref(out_node))
    if rc < 0:
        raise MoeError("fusion_detect: " + L.ggml_hip_moe_last_error().decode(errors="replace"))
    return rc, f, (gh if has_gh.value else None), [bool(c) for c in covered], out_node.value


def ssm_conv(x, w, *, bias=None, silu=False, out=None, n_t=None, stream=None):
    """SSM_CONV through ggml_hip_ssm_conv_f32.

    x: float32 [n_s, nr, nc - 1 + n_t] (conv_x, rows contiguous); w: float32 or float16 [nr, nc];
    bias: float32 [nr] (with silu only); out: float32 [n_s, n_t, nr] (allocated when None).
    """
    torch = _torch()
    n_s, nr, cols = x.shape
    nc = w.shape[1]
    n_t = cols - nc + 1 if n_t is None else n_t
    if out is None:
        out = torch.empty((n_s, n_t, nr), dtype=torch.float32, device=x.device)
    _require_gpu(x, w, bias, out)
    if w.dtype == torch.float16:
        wt = 1
    elif w.dtype == torch.float32:
        wt = 0
    else:
        raise TypeError("ssm_conv: weights must be float32 or float16")
    es = w.element_size()
    rc = lib().ggml_hip_ssm_conv_f32(x.data_ptr(), x.stride(2) * 4, x.stride(1) * 4, x.stride(0) * 4, w.data_ptr(), wt,
                                     w.stride(0) * es, _ptr(bias), 1 if silu else 0, out.data_ptr(), out.stride(2) * 4,
                                     out.stride(1) * 4, out.stride(0) * 4, nc, nr, n_t, n_s, _stream(stream))
    check(rc, "ssm_conv")
    return out


def configure(*, enabled=True, slots=-1, budget_gb=0.0, margin_gb=2.0, seed_path=None, max_promotions=48,
              verbose=False, async_promotions=False):
    cfg = Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb = int(enabled), slots, budget_gb, margin_gb
    cfg._seed = seed_path.encode() if seed_path else None
    cfg.seed_path = cfg._seed
    cfg.max_promotions, cfg.verbose = max_promotions, int(verbose)
    cfg.async_promotions = int(async_promotions)
    check(lib().ggml_hip_moe_cache_configure(C.byref(cfg)), "configure")


def check_status(stream=None) -> int:
    """0, or E_TIMEOUT when a fused gate/up launch on `stream` had a bounded wait give up (then cleared)."""
    return lib().ggml_hip_moe_check_status(_stream(stream))


def reset():
    check(lib().ggml_hip_moe_cache_reset(), "reset")


def step(stream=None):
    return check(lib().ggml_hip_moe_cache_step(_stream(stream)), "step")


def entry_info(i: int) -> EntryInfo:
    info = EntryInfo()
    check(lib().ggml_hip_moe_cache_entry_info(i, C.byref(info)), "entry_info")
    return info


def entry_state(i: int):
    import numpy as np
    info = entry_info(i)
    slot_of = np.empty(info.n_experts, dtype=np.int32)
    expert_of = np.empty(max(info.n_slots, 1), dtype=np.int32)
    table = np.empty(info.n_experts, dtype=np.int32)
    check(lib().ggml_hip_moe_cache_entry_slots(i, slot_of.ctypes.data, info.n_experts, expert_of.ctypes.data,
                                               info.n_slots), "entry_slots")
    check(lib().ggml_hip_moe_cache_entry_table(i, table.ctypes.data, info.n_experts), "entry_table")
    return {"info": info, "slot_of": slot_of, "expert_of": expert_of[:info.n_slots], "table": table}


def totals() -> Totals:
    t = Totals()
    check(lib().ggml_hip_moe_cache_totals(C.byref(t)), "totals")
    return t


def device_globals():
    s, c = C.c_void_p(), C.c_void_p()
    check(lib().ggml_hip_moe_cache_device_globals(C.byref(s), C.byref(c)), "device_globals")
    return s.value, c.value


def entry_device(i: int):
    t, s, p = C.c_void_p(), C.c_void_p(), C.c_void_p()
    check(lib().ggml_hip_moe_cache_entry_device(i, C.byref(t), C.byref(s), C.byref(p)), "entry_device")
    return t.value, s.value, p.value


def stats_snapshot(n_words: int = STATS_WORDS, stream=None):
    import numpy as np
    out = np.zeros(n_words, dtype=np.uint32)
    check(lib().ggml_hip_moe_cache_stats_snapshot(out.ctypes.data, n_words, _stream(stream)), "stats_snapshot")
    return out


def stamps_snapshot(i: int, stream=None):
    import numpy as np
    n = entry_info(i).n_experts
    out = np.zeros(n, dtype=np.uint32)
    check(lib().ggml_hip_moe_cache_stamps_snapshot(i, out.ctypes.data, n, _stream(stream)), "stamps_snapshot")
    return out


def combine_q8_1(o, w, shared=None, residual=None, x_out=None, y=None, rms_norm=False, norm_weight=None, eps=1e-6,
                 stream=None):
    """o: [n_tok, n_used, k] fp32, w: [n_tok, n_used] -> (x_out [n_tok, k], y q8_1 [n_tok, k/32*36]);
    with rms_norm, y holds q8_1((x * rms scale) * norm_weight)."""
    torch = _torch()
    _require_gpu(o, w, shared, residual, x_out, y, norm_weight)
    n_tok, n_used, k = o.shape
    if y is None:
        y = torch.empty((n_tok, k // 32 * 36), dtype=torch.uint8, device=o.device)
    check(lib().ggml_hip_moe_combine_q8_1(o.data_ptr(), o.stride(1), w.data_ptr(), n_used, _ptr(shared),
                                          shared.stride(0) if shared is not None else 0, _ptr(residual),
                                          _ptr(x_out), y.data_ptr(), y.stride(0) // 36, k, n_tok,
                                          int(bool(rms_norm)), _ptr(norm_weight), eps, _stream(stream)),
          "combine_q8_1")
    return x_out, y
