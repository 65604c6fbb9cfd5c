"""CPU: the op-level MUL_MAT_ID entry's host half (ggml_hip_moe_mul_mat_id_workspace_bytes):
path choice and workspace size from the tensors, and refusal of tensors that are not a
supported MUL_MAT_ID.  No device call is made on these paths."""
import ctypes as C

import pytest


def _desc(mc, ggml_type, ne, nb, data=0):
    t = mc.Tensor()
    t.type = ggml_type
    t.ne[:] = list(ne) + [1] * (4 - len(ne))
    nbl = list(nb)
    while len(nbl) < 4:
        nbl.append(nbl[-1] * t.ne[len(nbl) - 1])
    t.nb[:] = nbl
    t.data = data
    t.has_buffer = 1
    return t


def _op(mc, wtype, K, R, E, n_tok, n_used, ne11=1, src1_type=0, ids_type=26, K1=None):
    src0 = mc.make_tensor(wtype, K, R, E, 0)
    K1 = K if K1 is None else K1
    s1 = _desc(mc, src1_type, [K1, ne11, n_tok], [4, 4 * K1, 4 * K1 * ne11])
    ids = _desc(mc, ids_type, [n_used, n_tok], [4, 4 * (n_used + 2)])
    return src0, s1, ids


def _ws(mc, src0, s1, ids, fusion=None):
    return int(mc.lib().ggml_hip_moe_mul_mat_id_workspace_bytes(C.byref(src0), C.byref(s1), C.byref(ids),
                                                                  C.byref(fusion) if fusion is not None else None))


def test_decode_workspace_is_the_q8_1_rows(mc):
    src0, s1, ids = _op(mc, mc.Q2_K, 4096, 768, 512, 2, 8)
    assert _ws(mc, src0, s1, ids) == 2 * 128 * 36          # 2 tokens x 128 q8_1 blocks


def test_prefill_workspace_is_q8_K_rows_plus_the_gemm_workspace(mc):
    src0, s1, ids = _op(mc, mc.Q4_K, 1024, 136, 24, 40, 6)
    rows = 40 * 4 * 292                                     # 40 tokens x 4 q8_K blocks
    gemm = int(mc.lib().ggml_hip_moe_mul_mat_q_workspace_bytes(1024, 24, 240))
    assert _ws(mc, src0, s1, ids) == (rows + 255) // 256 * 256 + gemm


def test_fused_bias_or_legacy_types_stay_on_the_gemv(mc):
    src0, s1, ids = _op(mc, mc.Q4_K, 1024, 136, 24, 40, 6)
    f = mc.Fusion()
    f.x_bias = 256                                          # any non-null bias pointer
    assert _ws(mc, src0, s1, ids, f) == 40 * 32 * 36
    src0, s1, ids = _op(mc, mc.Q4_0, 1024, 136, 24, 40, 6)
    assert _ws(mc, src0, s1, ids) == 40 * 32 * 36


@pytest.mark.parametrize("bad", ["src1_type", "ids_type", "K"])
def test_refuses_non_mul_mat_id_tensors(mc, bad):
    kw = {"src1_type": 1} if bad == "src1_type" else {"ids_type": 0} if bad == "ids_type" else {"K1": 512}
    src0, s1, ids = _op(mc, mc.Q4_K, 1024, 136, 24, 40, 6, **kw)
    assert _ws(mc, src0, s1, ids) == -1
    assert b"mul_mat_id" in mc.lib().ggml_hip_moe_last_error()
