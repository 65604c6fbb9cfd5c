"""GPU: the plain MUL_MAT_ID GEMV on rows of more than 64 lane units (legacy types above
K = 4096, K-quants above K = 16384), which it streams through LDS 64 units at a time,
against the oracle fed the same activation bytes (rel-L2 1e-5, the GEMV bar), with a fused
gate + GLU, fp32 activation rows (bit-identical to quantize-then-GEMV) and a wide shared
expert beside narrow routed experts.  The reference GEMV takes any row length
(kernels/moe-cache.cu:76-291 loops over the row's blocks)."""
import sys

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("wtype,K,act,gated", [
    (2, 5120, "q8_1", False),       # Q4_0, 80 units per row
    (8, 7168, "q8_1", True),        # Q8_0, 112 units, gate + SwiGLU
    (6, 8192, "f32", False),        # Q5_0, 128 units, fp32 rows
    (12, 16640, "q8_1", True),      # Q4_K, 65 super-blocks: a 1-unit last chunk
    (14, 16896, "q8_K", False),     # Q6_K, 66 super-blocks, q8_K activations
    (2, 16384, "f32", True),        # Q4_0, 256 units, fp32 rows (largest fp32 row), gated
])
def test_gemv_wide_rows_match_oracle(torch_gpu, mc, O, wtype, K, act, gated):
    torch = torch_gpu
    R, n_exp, n_used, n_tok = 21, 6, 3, 2
    _note(f"wide gemv type={wtype} K={K} act={act} gated={gated}")
    w = H.weights(wtype, n_exp, R, K, seed=3300 + wtype)
    gate = H.weights(wtype, n_exp, R, K, seed=3400 + wtype) if gated else None
    x = H.activations(n_tok, K, seed=3500 + K)
    ids = H.routing(n_tok, n_used, n_exp, seed=3600)
    xd = _dev(torch, x)
    if act == "q8_K":
        y, kind, okind = mc.quantize_q8_K(xd), mc.ACT_Q8_K, O.ACT_CPU
    else:
        y, kind, okind = mc.quantize_q8_1(xd), mc.ACT_Q8_1, O.ACT_Q8_1
    keep = []
    f = None
    if gated:
        gd = _dev(torch, gate)
        keep.append(gd)
        f = mc.make_fusion(glu_op=2)
        f.gate = gd.data_ptr()
    wd = _dev(torch, w)
    ids_d = _dev(torch, ids)
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_vec(wtype=wtype, weights=wd, ids=ids_d, y=y.view(n_tok, 1, -1), dst=dst, K=K, R=R, n_experts=n_exp,
                   act=kind, fusion=f)
    if act == "f32":
        # fp32 rows quantized inside the GEMV: bit-identical to the q8_1 path on the quantizer's bytes
        dst32 = torch.zeros_like(dst)
        mc.mul_mat_vec(wtype=wtype, weights=wd, ids=ids_d, y=xd.view(n_tok, 1, -1), dst=dst32, K=K, R=R,
                       n_experts=n_exp, act=mc.ACT_F32, fusion=f)
        torch.cuda.synchronize()
        assert torch.equal(dst32, dst)
    torch.cuda.synchronize()
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=w, gate=gate, ids=ids,
                        act=y.cpu().numpy().reshape(n_tok, 1, -1), act_kind=okind, glu_op=2)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME


def test_gemv_wide_shared_expert(torch_gpu, mc, O):
    """Routed Q4_K rows of 20 super-blocks (one step holds 3 rows) beside a Q4_0 shared expert
    whose rows are 80 units (one row per step, two chunks)."""
    torch = torch_gpu
    wtype, shtype, K, R, n_exp, n_used, n_tok = 12, 2, 5120, 30, 8, 4, 2
    up = H.weights(wtype, n_exp, R, K, seed=3701)
    gate = H.weights(wtype, n_exp, R, K, seed=3702)
    sh_up = H.weights(shtype, 1, R, K, seed=3703)[0]
    sh_gate = H.weights(shtype, 1, R, K, seed=3704)[0]
    x = H.activations(n_tok, K, seed=3705)
    ids = H.routing(n_tok, n_used, n_exp, seed=3706)
    yq = mc.quantize_q8_1(_dev(torch, x))
    sh_dst = torch.zeros((n_tok, R), dtype=torch.float32, device="cuda")
    su, sg, gd = _dev(torch, sh_up), _dev(torch, sh_gate), _dev(torch, gate)
    f = mc.make_fusion(glu_op=2, shared_up=su, shared_gate=sg, shared_dst=sh_dst, shared_type=shtype)
    f.gate = gd.data_ptr()
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_vec(wtype=wtype, weights=_dev(torch, up), ids=_dev(torch, ids), y=yq.view(n_tok, 1, -1), dst=dst,
                   K=K, R=R, n_experts=n_exp, act=mc.ACT_Q8_1, fusion=f)
    torch.cuda.synchronize()
    want, want_sh = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=up, gate=gate, ids=ids,
                                 act=yq.cpu().numpy().reshape(n_tok, 1, -1), act_kind=O.ACT_Q8_1, glu_op=2,
                                 sh_type=shtype, sh_up=sh_up, sh_gate=sh_gate)
    e1, e2 = O.rel_l2(dst.cpu().numpy(), want), O.rel_l2(sh_dst.cpu().numpy(), want_sh)
    _note(f"wide shared: routed rel_l2={e1:.3e} shared rel_l2={e2:.3e}")
    assert e1 <= H.TOL_SAME and e2 <= H.TOL_SAME


def test_gemv_row_length_limits(torch_gpu, mc):
    """Rows past the staged-activation limit (65536 values; 16384 for fp32 rows) are refused
    before any launch."""
    torch = torch_gpu
    for K, act, wtype in ((65536 + 256, mc.ACT_Q8_K, 12), (16384 + 64, mc.ACT_F32, 2)):
        w = torch.zeros(mc.row_bytes(wtype, K) * 2, dtype=torch.uint8, device="cuda")
        y = torch.zeros(K * 4, dtype=torch.uint8, device="cuda")
        ids = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
        dst = torch.zeros((1, 1, 2), dtype=torch.float32, device="cuda")
        with pytest.raises(mc.MoeError, match="exceeds the staged activation row"):
            mc.mul_mat_vec(wtype=wtype, weights=w, ids=ids, y=y.view(1, 1, -1), dst=dst, K=K, R=2, n_experts=1,
                           act=act)
