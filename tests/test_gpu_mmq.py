"""GPU: the prefill-shaped MUL_MAT_ID (expert-grouped int8 MFMA, q8_K activations)
against the CPU oracle's ggml-CPU MUL_MAT_ID restatement, through the C ABI."""
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


def _q8_K_rows(torch, mc, x):
    """q8_K rows of x packed back to back in a 256-byte aligned device buffer."""
    n, K = x.shape
    rb = K // 256 * 292
    buf = torch.zeros(n * rb + 256, dtype=torch.uint8, device="cuda")
    buf[:n * rb] = mc.quantize_q8_K(_dev(torch, x)).reshape(-1)
    return buf


@pytest.mark.parametrize("wtype", [10, 11, 12, 13, 14])
# (16, 768, 101, ...): three super-blocks per row and an odd row count, so Q3_K / Q6_K rows
# and experts alternate between 4-byte and 2-byte aligned starts
@pytest.mark.parametrize("E,K,R,n_tok,n_used", [(16, 512, 100, 40, 4), (16, 768, 101, 40, 4),
                                                (64, 4096, 256, 96, 8)])
def test_mul_mat_q_matches_ggml_cpu(torch_gpu, mc, O, wtype, E, K, R, n_tok, n_used):
    torch = torch_gpu
    _note(f"mul_mat_q type={wtype} E={E} K={K} R={R} tok={n_tok} used={n_used}")
    w = H.weights(wtype, E, R, K, seed=1100 + wtype)
    x = H.activations(n_tok, K, seed=1101)
    ids = H.routing(n_tok, n_used, E, seed=1102)
    if E == 16:
        ids[3, 1] = -1                    # skipped pick: its dst row stays untouched
        ids[7, 0] = E + 5
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    _note(f"  pairs per expert: min {counts.min()} max {counts.max()}")
    ycat = _q8_K_rows(torch, mc, x)
    sentinel = np.float32(-12345.0)
    dst = torch.full((n_tok, n_used, R), float(sentinel), dtype=torch.float32, device="cuda")
    ids_d = _dev(torch, ids)
    wd = _dev(torch, w)
    ws = torch.empty(int(mc.lib().ggml_hip_moe_mul_mat_q_workspace_bytes(K, E, n_tok * n_used)), dtype=torch.uint8,
                     device="cuda")
    mc.mul_mat_q(wtype=wtype, weights=wd, ids=ids_d, y=ycat, dst=dst, K=K, R=R, n_experts=E, workspace=ws)
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    want = O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=E, src0=w, src1=x, ids=np.clip(ids, 0, E - 1))
    valid = (ids >= 0) & (ids < E)
    err = O.rel_l2(got[valid], want[valid])
    _note(f"  rel_l2 vs ggml-cpu={err:.3e}")
    assert err <= H.TOL_SAME
    assert np.all(got[~valid] == sentinel)


@pytest.mark.parametrize("wtype", [10, 11, 12, 13, 14])
def test_mul_mat_q_many_pairs_per_expert(torch_gpu, mc, O, wtype):
    """Experts with many pairs: more than MMQ_FEW_PAIRS per expert on average selects the
    4-blocks-per-pass kernel, and expert 0 (every token's first slot) needs two passes."""
    torch = torch_gpu
    E, K, R, n_tok, n_used = 8, 1024, 136, 96, 2
    _note(f"mul_mat_q many pairs type={wtype}")
    w = H.weights(wtype, E, R, K, seed=1300 + wtype)
    x = H.activations(n_tok, K, seed=1301)
    ids = H.routing(n_tok, n_used, E, seed=1302)
    ids[:, 1] = np.where(ids[:, 0] == 0, ids[:, 1], ids[:, 0])
    ids[:, 1] = np.where(ids[:, 1] == 0, 1, ids[:, 1])
    ids[:, 0] = 0
    counts = np.bincount(ids.reshape(-1), minlength=E)
    _note(f"  pairs per expert: {counts.tolist()}")
    assert counts[0] == n_tok and counts.sum() == n_tok * n_used
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_q(wtype=wtype, weights=_dev(torch, w), ids=_dev(torch, ids), y=_q8_K_rows(torch, mc, x), dst=dst, K=K,
                 R=R, n_experts=E)
    torch.cuda.synchronize()
    want = O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=E, src0=w, src1=x, ids=ids)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2 vs ggml-cpu={err:.3e}")
    assert err <= H.TOL_SAME


@pytest.mark.parametrize("wtype,R", [(12, 136), (10, 100), (14, 72), (11, 80)])
def test_mul_mat_q_gate_glu(torch_gpu, mc, O, wtype, R):
    torch = torch_gpu
    E, K, n_tok, n_used = 24, 1024, 48, 6
    _note(f"mul_mat_q gate+GLU type={wtype} R={R}")
    up = H.weights(wtype, E, R, K, seed=1201)
    gate = H.weights(wtype, E, R, K, seed=1202)
    x = H.activations(n_tok, K, seed=1203)
    ids = H.routing(n_tok, n_used, E, seed=1204)
    ycat = _q8_K_rows(torch, mc, x)
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_q(wtype=wtype, weights=_dev(torch, up), gate=_dev(torch, gate), ids=_dev(torch, ids), y=ycat, dst=dst,
                 K=K, R=R, n_experts=E, glu_op=O.GLU_SWIGLU)
    torch.cuda.synchronize()
    act = np.stack([O.quantize_act(wtype, O.ACT_CPU, r) for r in x]).reshape(n_tok, 1, -1)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=E, src0=up, gate=gate, ids=ids, act=act, act_kind=O.ACT_CPU,
                        glu_op=O.GLU_SWIGLU)
    err = O.rel_l2(dst.cpu().numpy(), want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME
