"""GPU: MUL_MAT_ID at the op level (ggml_hip_moe_mul_mat_id): strides derived from the
tensors, src1 quantized inside, then the GEMV (q8_1) or the grouped GEMM (q8_K), against
the CPU oracle on the same inputs, through the C ABI."""
import sys

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _ids_view(torch, ids, extra=3):
    """ids as the first n_used columns of a wider int32 matrix (ids_stride > n_used)."""
    n_tok, n_used = ids.shape
    wide = np.full((n_tok, n_used + extra), -7, np.int32)
    wide[:, :n_used] = ids
    return _dev(torch, wide)[:, :n_used]


@pytest.mark.parametrize("wtype", [10, 12, 2])
def test_decode_takes_the_gemv(torch_gpu, mc, O, wtype):
    """2 tokens, one activation row per token, ids and dst as strided views: the q8_1 GEMV."""
    torch = torch_gpu
    E, K, R, n_tok, n_used = 16, 2048, 96, 2, 8
    _note(f"mul_mat_id decode type={wtype}")
    w = H.weights(wtype, E, R, K, seed=1500 + wtype)
    x = H.activations(n_tok, K, seed=1501).reshape(n_tok, 1, K)
    ids = H.routing(n_tok, n_used, E, seed=1502)
    xd = _dev(torch, x)
    big = torch.full((n_tok, n_used, R + 16), -3.0, dtype=torch.float32, device="cuda")
    dst = big[:, :, :R]
    mc.mul_mat_id(wtype=wtype, weights=_dev(torch, w), x=xd, ids=_ids_view(torch, ids), dst=dst, K=K, R=R, n_experts=E)
    torch.cuda.synchronize()
    yq = mc.quantize_q8_1(xd.reshape(n_tok, K)).cpu().numpy().reshape(n_tok, 1, -1)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=E, src0=w, ids=ids, act=yq, act_kind=O.ACT_Q8_1)
    got = big.cpu().numpy()
    err = O.rel_l2(got[:, :, :R], want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME
    assert np.all(got[:, :, R:] == -3.0)


@pytest.mark.parametrize("wtype", [10, 11, 12, 14])
def test_prefill_takes_the_grouped_gemm(torch_gpu, mc, O, wtype):
    """40 tokens of K-quant experts: q8_K rows and the grouped GEMM (ggml-CPU semantics)."""
    torch = torch_gpu
    E, K, R, n_tok, n_used = 24, 1024, 136, 40, 6
    _note(f"mul_mat_id prefill type={wtype}")
    w = H.weights(wtype, E, R, K, seed=1600 + wtype)
    x = H.activations(n_tok, K, seed=1601).reshape(n_tok, 1, K)
    ids = H.routing(n_tok, n_used, E, seed=1602)
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_id(wtype=wtype, weights=_dev(torch, w), x=_dev(torch, x), ids=_ids_view(torch, ids), dst=dst, K=K, R=R,
                  n_experts=E)
    torch.cuda.synchronize()
    want = O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=E, src0=w, src1=x, ids=ids)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2 vs ggml-cpu={err:.3e}")
    assert err <= H.TOL_SAME


@pytest.mark.parametrize("wtype", [13, 2])
def test_per_slot_rows_with_padded_tokens(torch_gpu, mc, O, wtype):
    """Down-projection shape: one activation row per slot, tokens padded apart in src1
    (quantized token by token).  Q5_K takes the grouped GEMM, Q4_0 the GEMV."""
    torch = torch_gpu
    E, K, R, n_tok, n_used = 12, 768, 80, 20, 4
    _note(f"mul_mat_id per-slot rows type={wtype}")
    w = H.weights(wtype, E, R, K, seed=1700 + wtype)
    x = H.activations(n_tok * n_used, K, seed=1701).reshape(n_tok, n_used, K)
    ids = H.routing(n_tok, n_used, E, seed=1702)
    xpad = torch.zeros((n_tok, n_used + 1, K), dtype=torch.float32, device="cuda")
    xpad[:, :n_used] = _dev(torch, x)
    xv = xpad[:, :n_used]                          # token stride (n_used + 1) rows
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_id(wtype=wtype, weights=_dev(torch, w), x=xv, ids=_dev(torch, ids), dst=dst, K=K, R=R, n_experts=E)
    torch.cuda.synchronize()
    if wtype == 13:
        want = O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=E, src0=w, src1=x, ids=ids)
    else:
        yq = mc.quantize_q8_1(_dev(torch, x.reshape(-1, K))).cpu().numpy().reshape(n_tok, n_used, -1)
        want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=E, src0=w, ids=ids, act=yq, act_kind=O.ACT_Q8_1,
                            nchannels_y=n_used)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME


def test_prefill_gate_glu(torch_gpu, mc, O):
    torch = torch_gpu
    wtype, E, K, R, n_tok, n_used = 12, 16, 1024, 72, 32, 4
    _note("mul_mat_id prefill gate + SwiGLU")
    up = H.weights(wtype, E, R, K, seed=1801)
    gate = H.weights(wtype, E, R, K, seed=1802)
    x = H.activations(n_tok, K, seed=1803).reshape(n_tok, 1, K)
    ids = H.routing(n_tok, n_used, E, seed=1804)
    gd = _dev(torch, gate)
    f = mc.make_fusion(gate=gd, glu_op=O.GLU_SWIGLU)
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_id(wtype=wtype, weights=_dev(torch, up), x=_dev(torch, x), ids=_dev(torch, ids), dst=dst, K=K, R=R,
                  n_experts=E, fusion=f)
    torch.cuda.synchronize()
    act = np.stack([O.quantize_act(wtype, O.ACT_CPU, r) for r in x.reshape(n_tok, K)]).reshape(n_tok, 1, -1)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=E, src0=up, gate=gate, ids=ids, act=act, act_kind=O.ACT_CPU,
                        glu_op=O.GLU_SWIGLU)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME
