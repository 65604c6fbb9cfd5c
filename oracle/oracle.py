"""ctypes bindings of the CPU oracle (oracle/mc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libmc_oracle.so"

# ggml_type numbering
F32, F16, Q4_0, Q5_0, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 6, 8, 9, 10, 11, 12, 13, 14, 15
WEIGHT_TYPES = [Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]
TYPE_NAMES = {Q4_0: "q4_0", Q5_0: "q5_0", Q8_0: "q8_0", Q8_1: "q8_1", Q2_K: "q2_K", Q3_K: "q3_K",
              Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K"}
KQUANTS = {Q2_K, Q3_K, Q4_K, Q5_K, Q6_K}

ACT_CPU, ACT_Q8_1, ACT_Q8_0_AS_Q8_1 = 0, 1, 2
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_GEGLU_ERF, GLU_GEGLU_QUICK, GLU_SWIGLU_CLAMP = range(7)


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < max(
            (HERE / f).stat().st_mtime for f in ("mc_oracle.c", "mc_oracle.h", "Makefile")):
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    return LIB_PATH


class _MmidArgs(C.Structure):
    _fields_ = [
        ("type", C.c_int), ("ne00", C.c_int64), ("ne01", C.c_int64), ("n_as", C.c_int32),
        ("nb01", C.c_size_t), ("nb02", C.c_size_t), ("src0", C.c_void_p), ("gate", C.c_void_p),
        ("x_bias", C.c_void_p), ("gate_bias", C.c_void_p), ("bias_stride", C.c_int64),
        ("x_scale", C.c_void_p), ("gate_scale", C.c_void_p),
        ("glu_op", C.c_int32), ("glu_limit", C.c_float),
        ("sh_type", C.c_int32), ("sh_up", C.c_void_p), ("sh_gate", C.c_void_p), ("sh_dst", C.c_void_p),
        ("sh_stride_col_dst", C.c_int64), ("sh_act", C.c_void_p), ("sh_act_stride_col", C.c_size_t),
        ("ids", C.c_void_p), ("n_ids", C.c_int32), ("n_tok", C.c_int32), ("ids_stride", C.c_int64),
        ("act_kind", C.c_int32), ("act", C.c_void_p), ("nchannels_y", C.c_int64),
        ("act_stride_col", C.c_size_t), ("act_stride_channel", C.c_size_t),
        ("dst", C.c_void_p), ("dst_stride_col", C.c_int64), ("dst_stride_channel", C.c_int64),
        ("nthreads", C.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(str(LIB_PATH))
        vp, i64, sz = C.c_void_p, C.c_int64, C.c_size_t
        L.or_fp32_to_fp16.argtypes, L.or_fp32_to_fp16.restype = [C.c_float], C.c_uint16
        L.or_fp16_to_fp32.argtypes, L.or_fp16_to_fp32.restype = [C.c_uint16], C.c_float
        L.or_block_elems.argtypes, L.or_block_elems.restype = [C.c_int], C.c_int
        L.or_block_bytes.argtypes, L.or_block_bytes.restype = [C.c_int], sz
        L.or_row_bytes.argtypes, L.or_row_bytes.restype = [C.c_int, i64], sz
        for fn in ("or_dequantize_row", "or_quantize_row_weights"):
            getattr(L, fn).argtypes, getattr(L, fn).restype = [C.c_int, vp, vp, i64], None
        for fn in ("or_quantize_q8_1", "or_quantize_q8_0", "or_quantize_q8_0_as_q8_1", "or_quantize_q8_K"):
            getattr(L, fn).argtypes, getattr(L, fn).restype = [vp, vp, i64], None
        L.or_act_type.argtypes, L.or_act_type.restype = [C.c_int, C.c_int], C.c_int
        L.or_act_row_bytes.argtypes, L.or_act_row_bytes.restype = [C.c_int, C.c_int, i64], sz
        L.or_quantize_act_row.argtypes, L.or_quantize_act_row.restype = [C.c_int, C.c_int, vp, vp, i64], None
        L.or_vec_dot.argtypes, L.or_vec_dot.restype = [C.c_int, C.c_int, i64, vp, vp], C.c_float
        L.or_vec_dot_cpu.argtypes, L.or_vec_dot_cpu.restype = [C.c_int, i64, vp, vp], C.c_float
        L.or_set_simd.argtypes, L.or_set_simd.restype = [C.c_int], None
        L.or_block_isums.argtypes, L.or_block_isums.restype = [C.c_int, vp, vp, vp], C.c_int
        L.or_glu.argtypes, L.or_glu.restype = [C.c_int, C.c_float, C.c_float, C.c_float], C.c_float
        L.or_mul_mat_id.argtypes, L.or_mul_mat_id.restype = [C.POINTER(_MmidArgs)], C.c_int
        L.or_cpu_mul_mat_id_f32.argtypes = [C.c_int, i64, i64, C.c_int32, vp, sz, sz, vp, i64, i64, i64,
                                            vp, C.c_int32, C.c_int32, i64, vp, i64, i64, C.c_int32]
        L.or_cpu_mul_mat_id_f32.restype = C.c_int
        L.or_fill_normal.argtypes, L.or_fill_normal.restype = [C.c_uint64, C.c_float, C.c_float, vp, i64], None
        L.or_topk_uniform.argtypes, L.or_topk_uniform.restype = [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, vp], None
        L.or_omp_max_threads.argtypes, L.or_omp_max_threads.restype = [], C.c_int
        L.or_combine_q8_1.argtypes = [vp, i64, vp, C.c_int32, vp, i64, vp, vp, vp, i64, i64, C.c_int32, vp, C.c_float]
        L.or_rms_sum.argtypes, L.or_rms_sum.restype = [vp, i64], C.c_float
        L.or_combine_q8_1.restype = None
        L.or_ssm_conv_f32.argtypes = [vp, i64, i64, vp, C.c_int, i64, vp, C.c_int, vp, i64, i64, i64, i64, i64, i64]
        L.or_ssm_conv_f32.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def block_elems(t):
    return lib().or_block_elems(t)


def block_bytes(t):
    return lib().or_block_bytes(t)


def row_bytes(t, k):
    return lib().or_row_bytes(t, k)


def fill_normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().or_fill_normal(seed, mean, std, _p(out), n)
    return out


def topk_uniform(seed, n_experts, k, n_tok):
    ids = np.empty((n_tok, k), dtype=np.int32)
    lib().or_topk_uniform(seed, n_experts, k, n_tok, _p(ids))
    return ids


def quantize_weights(t, x):
    """x: float32 [rows, k] -> uint8 [rows, row_bytes]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    out = np.zeros((rows, row_bytes(t, k)), dtype=np.uint8)
    L = lib()
    flat = x.reshape(rows, k)
    for r in range(rows):
        L.or_quantize_row_weights(t, flat[r].ctypes.data, out[r].ctypes.data, k)
    return out


def quantize_weights_fast(t, x):
    """Same as quantize_weights, one call for the whole contiguous array (rows are independent)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    n = x.size
    out = np.zeros(n // k * row_bytes(t, k), dtype=np.uint8)
    lib().or_quantize_row_weights(t, x.ctypes.data, out.ctypes.data, n)
    return out.reshape(n // k, row_bytes(t, k))


def dequantize(t, q, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.size // row_bytes(t, k)
    out = np.empty((rows, k), dtype=np.float32)
    lib().or_dequantize_row(t, q.ctypes.data, out.ctypes.data, rows * k)
    return out


def quantize_act(wtype, act_kind, x):
    """x float32 [..., k] -> uint8 [..., act_row_bytes]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    L = lib()
    rb = L.or_act_row_bytes(wtype, act_kind, k)
    flat = x.reshape(-1, k)
    out = np.empty((flat.shape[0], rb), dtype=np.uint8)
    for r in range(flat.shape[0]):
        L.or_quantize_act_row(wtype, act_kind, flat[r].ctypes.data, out[r].ctypes.data, k)
    return out.reshape(x.shape[:-1] + (rb,))


def quantize_q8_1(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 36, dtype=np.uint8)
    lib().or_quantize_q8_1(x.ctypes.data, out.ctypes.data, x.size)
    return out


def quantize_q8_K(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 256 * 292, dtype=np.uint8)
    lib().or_quantize_q8_K(x.ctypes.data, out.ctypes.data, x.size)
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().or_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size)
    return out


def vec_dot(wtype, act_kind, k, wrow, arow):
    wrow = np.ascontiguousarray(wrow, dtype=np.uint8)
    arow = np.ascontiguousarray(arow, dtype=np.uint8)
    return lib().or_vec_dot(wtype, act_kind, k, wrow.ctypes.data, arow.ctypes.data)


def vec_dot_cpu(wtype, k, wrow, arow):
    """ggml-CPU vec_dot (q8_0 / q8_K activation row): AVX2 for Q2_K / Q4_K unless set_simd(False)."""
    wrow, arow = np.ascontiguousarray(wrow), np.ascontiguousarray(arow)
    return lib().or_vec_dot_cpu(wtype, k, wrow.ctypes.data, arow.ctypes.data)


def set_simd(on: bool):
    """AVX2 q8_K dots in the ggml-CPU MUL_MAT_ID restatement (default on) or the scalar path."""
    lib().or_set_simd(1 if on else 0)


def block_isums(wtype, wblock, q8):
    out = np.zeros(16, dtype=np.int32)
    wblock = np.ascontiguousarray(wblock, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    n = lib().or_block_isums(wtype, wblock.ctypes.data, q8.ctypes.data, out.ctypes.data)
    return out[:n]


def glu(op, g, up, limit=0.0):
    return lib().or_glu(op, g, up, limit)


def mul_mat_id(*, wtype, K, R, n_as, src0, ids, act, act_kind, gate=None, x_bias=None, gate_bias=None,
               x_scale=None, gate_scale=None, glu_op=GLU_SWIGLU, glu_limit=0.0, nchannels_y=1,
               sh_type=None, sh_up=None, sh_gate=None, sh_act=None, nthreads=None):
    """Oracle MUL_MAT_ID with fused post-ops.

    src0/gate: uint8 [n_as, R, row_bytes]; ids: int32 [n_tok, n_used];
    act: uint8 [n_tok, nchannels_y, act_row_bytes] (pre-quantized rows);
    returns dst float32 [n_tok, n_used, R] (and sh_dst [n_tok, R] when sh_up is given).
    """
    n_tok, n_used = ids.shape
    rb = row_bytes(wtype, K)
    src0 = np.ascontiguousarray(src0, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    act = np.ascontiguousarray(act, dtype=np.uint8)
    dst = np.zeros((n_tok, n_used, R), dtype=np.float32)
    a = _MmidArgs()
    a.type, a.ne00, a.ne01, a.n_as, a.nb01, a.nb02 = wtype, K, R, n_as, rb, rb * R
    a.src0 = src0.ctypes.data
    keep = [src0, ids, act, dst]
    if gate is not None:
        gate = np.ascontiguousarray(gate, dtype=np.uint8); keep.append(gate); a.gate = gate.ctypes.data
    for name, arr in (("x_bias", x_bias), ("gate_bias", gate_bias), ("x_scale", x_scale), ("gate_scale", gate_scale)):
        if arr is not None:
            arr = np.ascontiguousarray(arr, dtype=np.float32); keep.append(arr); setattr(a, name, arr.ctypes.data)
    a.bias_stride = R
    a.glu_op, a.glu_limit = glu_op, glu_limit
    sh_dst = None
    if sh_up is not None:
        sh_up = np.ascontiguousarray(sh_up, dtype=np.uint8); keep.append(sh_up)
        sh_dst = np.zeros((n_tok, R), dtype=np.float32); keep.append(sh_dst)
        a.sh_type, a.sh_up, a.sh_dst, a.sh_stride_col_dst = sh_type, sh_up.ctypes.data, sh_dst.ctypes.data, R
        if sh_gate is not None:
            sh_gate = np.ascontiguousarray(sh_gate, dtype=np.uint8); keep.append(sh_gate); a.sh_gate = sh_gate.ctypes.data
        if sh_act is not None:
            sh_act = np.ascontiguousarray(sh_act, dtype=np.uint8); keep.append(sh_act)
            a.sh_act, a.sh_act_stride_col = sh_act.ctypes.data, sh_act.shape[-1]
    a.ids, a.n_ids, a.n_tok, a.ids_stride = ids.ctypes.data, n_used, n_tok, n_used
    arb = act.shape[-1]
    a.act_kind, a.act, a.nchannels_y = act_kind, act.ctypes.data, nchannels_y
    a.act_stride_col, a.act_stride_channel = arb * nchannels_y, arb
    a.dst, a.dst_stride_col, a.dst_stride_channel = dst.ctypes.data, n_used * R, R
    a.nthreads = nthreads or lib().or_omp_max_threads()
    rc = lib().or_mul_mat_id(C.byref(a))
    if rc != 0:
        raise RuntimeError(f"or_mul_mat_id failed: {rc}")
    return (dst, sh_dst) if sh_up is not None else dst


def cpu_mul_mat_id_f32(*, wtype, K, R, n_as, src0, src1, ids, nthreads=None):
    """ggml-CPU MUL_MAT_ID restatement on fp32 src1 [n_tok, ne11, K] -> dst [n_tok, n_used, R]."""
    n_tok, n_used = ids.shape
    src1 = np.ascontiguousarray(src1, dtype=np.float32)
    if src1.ndim == 2:
        src1 = src1[:, None, :]
    ne11 = src1.shape[1]
    rb = row_bytes(wtype, K)
    src0 = np.ascontiguousarray(src0, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    dst = np.zeros((n_tok, n_used, R), dtype=np.float32)
    rc = lib().or_cpu_mul_mat_id_f32(wtype, K, R, n_as, src0.ctypes.data, rb, rb * R, src1.ctypes.data, ne11, K,
                                     ne11 * K, ids.ctypes.data, n_used, n_tok, n_used, dst.ctypes.data,
                                     n_used * R, R, nthreads or lib().or_omp_max_threads())
    if rc != 0:
        raise RuntimeError(f"or_cpu_mul_mat_id_f32 failed: {rc}")
    return dst


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def cpu_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except Exception:  # pragma: no cover
        return os.cpu_count() or 1


def combine_q8_1(o, w, shared=None, residual=None, rms_norm=False, norm_weight=None, eps=1e-6):
    """o [n_tok, n_used, k], w [n_tok, n_used] -> (x [n_tok, k], q8_1 bytes [n_tok, k/32*36]);
    with rms_norm the quantized row is (x * rms scale) * norm_weight."""
    o = np.ascontiguousarray(o, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n_tok, n_used, k = o.shape
    x = np.empty((n_tok, k), np.float32)
    y = np.empty((n_tok, k // 32 * 36), np.uint8)
    sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    nw = None if norm_weight is None else np.ascontiguousarray(norm_weight, dtype=np.float32)
    lib().or_combine_q8_1(o.ctypes.data, k, w.ctypes.data, n_used, _p(sh), k, _p(res), x.ctypes.data, y.ctypes.data,
                          k, n_tok, int(bool(rms_norm)), _p(nw), eps)
    return x, y


def ssm_conv(x, w, bias=None, silu=False):
    """SSM_CONV: x [n_s, nr, nc - 1 + n_t] float32, w [nr, nc] float32 or float16,
    bias [nr] (with silu) -> dst [n_s, n_t, nr] float32 (or_ssm_conv_f32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_s, nr, cols = x.shape
    f16 = np.asarray(w).dtype == np.float16
    w = np.ascontiguousarray(w, dtype=np.float16 if f16 else np.float32)
    nc = w.shape[1]
    n_t = cols - nc + 1
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    dst = np.empty((n_s, n_t, nr), np.float32)
    lib().or_ssm_conv_f32(x.ctypes.data, cols, nr * cols, w.ctypes.data, int(f16), nc, _p(b), int(bool(silu)),
                          dst.ctypes.data, nr, n_t * nr, nc, nr, n_t, n_s)
    return dst


def rms_sum(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().or_rms_sum(x.ctypes.data, x.size)
