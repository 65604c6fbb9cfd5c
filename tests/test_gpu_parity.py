"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle.

Bars: activation quantizers bit-exact; GEMV outputs within rel-L2 1e-5 of the
oracle fed the same activation bytes, and within 1e-3 of the ggml-CPU
MUL_MAT_ID restatement in CPU-compatible activation mode.
"""
import sys

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu

ALL_TYPES = [2, 6, 8, 10, 11, 12, 13, 14]


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("K", [256, 768, 4096])
def test_quantize_q8_1_bitexact(torch_gpu, mc, O, K):
    torch = torch_gpu
    _note(f"quantize_q8_1 K={K}")
    x = np.concatenate([H.activations(7, K, 11 + K), H.special_rows(K)])
    got = mc.quantize_q8_1(_dev(torch, x)).cpu().numpy()
    want = np.stack([O.quantize_q8_1(r) for r in x])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("K", [256, 4096])
def test_quantize_q8_K_bitexact(torch_gpu, mc, O, K):
    torch = torch_gpu
    _note(f"quantize_q8_K K={K}")
    x = np.concatenate([H.activations(5, K, 21 + K), H.special_rows(K)])
    got = mc.quantize_q8_K(_dev(torch, x)).cpu().numpy()
    want = np.stack([O.quantize_q8_K(r) for r in x])
    assert np.array_equal(got, want)


def test_quantize_q8_0_bitexact(torch_gpu, mc, O):
    torch = torch_gpu
    K = 1024
    x = np.concatenate([H.activations(5, K, 31), H.special_rows(K)])
    got = mc.quantize_q8_1(_dev(torch, x), kind="q8_0").cpu().numpy()
    want = np.stack([O.quantize_act(O.Q4_0, O.ACT_Q8_0_AS_Q8_1, r) for r in x])
    assert np.array_equal(got, want)


def _run_gemv(torch, mc, wtype, w, ids, y_bytes, K, R, n_exp, act, nchannels_y=1, fusion=None, gate=None):
    n_tok, n_used = ids.shape
    dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
    wd = _dev(torch, w)
    f = fusion
    keep = [wd]
    if gate is not None:
        gd = _dev(torch, gate)
        keep.append(gd)
        f = f if f is not None else mc.make_fusion()
        f.gate = gd.data_ptr()
    mc.mul_mat_vec(wtype=wtype, weights=wd, ids=_dev(torch, ids), y=_dev(torch, y_bytes), dst=dst, K=K, R=R,
                   n_experts=n_exp, act=act, fusion=f, nchannels_y=nchannels_y)
    torch.cuda.synchronize()
    return dst.cpu().numpy()


@pytest.mark.parametrize("wtype", ALL_TYPES)
@pytest.mark.parametrize("K,R,n_tok", [(4096, 40, 1), (768, 70, 2), (2048, 33, 3)])
def test_gemv_q8_1_matches_oracle(torch_gpu, mc, O, wtype, K, R, n_tok):
    torch = torch_gpu
    n_exp, n_used = 12, 4
    _note(f"gemv q8_1 type={wtype} K={K} R={R} tok={n_tok}")
    w = H.weights(wtype, n_exp, R, K, seed=100 + wtype)
    x = H.activations(n_tok, K, seed=200 + K)
    ids = H.routing(n_tok, n_used, n_exp, seed=300 + n_tok)
    yq = mc.quantize_q8_1(_dev(torch, x)).cpu().numpy().reshape(n_tok, 1, -1)
    got = _run_gemv(torch, mc, wtype, w, ids, yq, K, R, n_exp, mc.ACT_Q8_1)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=w, ids=ids, act=yq, act_kind=O.ACT_Q8_1)
    err = O.rel_l2(got, want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= H.TOL_SAME


@pytest.mark.parametrize("wtype", ALL_TYPES)
def test_gemv_cpu_mode_matches_ggml_cpu(torch_gpu, mc, O, wtype):
    """CPU-compatible activations (q8_K for K-quants, q8_0 rounding for legacy) vs ggml-CPU MUL_MAT_ID."""
    torch = torch_gpu
    K, R, n_exp, n_used, n_tok = 4096, 48, 16, 8, 2
    _note(f"gemv cpu-mode type={wtype}")
    w = H.weights(wtype, n_exp, R, K, seed=400 + wtype)
    x = H.activations(n_tok, K, seed=500)
    ids = H.routing(n_tok, n_used, n_exp, seed=600)
    xd = _dev(torch, x)
    if wtype in mc.KQUANTS:
        yq, act = mc.quantize_q8_K(xd), mc.ACT_Q8_K
    else:
        yq, act = mc.quantize_q8_1(xd, kind="q8_0"), mc.ACT_Q8_1
    got = _run_gemv(torch, mc, wtype, w, ids, yq.cpu().numpy().reshape(n_tok, 1, -1), K, R, n_exp, act)
    want = O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=n_exp, src0=w, src1=x, ids=ids)
    err = O.rel_l2(got, want)
    _note(f"  rel_l2 vs ggml-cpu={err:.3e}")
    assert err <= H.TOL_CPU
    # and the default q8_1 boundary format, beside it.  Legacy types: q8_1 codes equal ggml-CPU's q8_0
    # codes, so only the fp32 summation order differs.  K-quants: 32-value q8_1 scales against ggml-CPU's
    # one q8_K scale per 256 values, two independent 8-bit roundings of x; the oracle measures 7.9e-3 to
    # 8.2e-3 on these inputs for Q2_K..Q6_K.
    yq1 = mc.quantize_q8_1(xd).cpu().numpy().reshape(n_tok, 1, -1)
    got1 = _run_gemv(torch, mc, wtype, w, ids, yq1, K, R, n_exp, mc.ACT_Q8_1)
    err1 = O.rel_l2(got1, want)
    _note(f"  q8_1-mode rel_l2 vs ggml-cpu={err1:.3e}")
    assert err1 <= (H.TOL_Q8_1_VS_CPU if wtype in mc.KQUANTS else H.TOL_SAME)


@pytest.mark.parametrize("glu_op", [2, 0, 1, 3, 4, 5, 6])
def test_gemv_fused_glu_bias_scale(torch_gpu, mc, O, glu_op):
    torch = torch_gpu
    wtype, K, R, n_exp, n_used, n_tok = 10, 4096, 24, 10, 4, 2
    _note(f"gemv fused glu={glu_op}")
    up = H.weights(wtype, n_exp, R, K, seed=701)
    gate = H.weights(wtype, n_exp, R, K, seed=702)
    x = H.activations(n_tok, K, seed=703)
    ids = H.routing(n_tok, n_used, n_exp, seed=704)
    rng = np.random.default_rng(705)
    xb = (rng.standard_normal((n_exp, R)) * 0.1).astype(np.float32)
    gb = (rng.standard_normal((n_exp, R)) * 0.1).astype(np.float32)
    xs = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, n_exp).astype(np.float32)
    xd = _dev(torch, x)
    yq = mc.quantize_q8_1(xd).cpu().numpy().reshape(n_tok, 1, -1)
    t = [_dev(torch, a) for a in (xb, gb, xs, gs)]
    f = mc.make_fusion(x_bias=t[0], gate_bias=t[1], x_scale=t[2], gate_scale=t[3], glu_op=glu_op, glu_limit=0.7)
    got = _run_gemv(torch, mc, wtype, up, ids, yq, K, R, n_exp, mc.ACT_Q8_1, fusion=f, gate=gate)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=up, gate=gate, ids=ids, act=yq, act_kind=O.ACT_Q8_1,
                        x_bias=xb, gate_bias=gb, x_scale=xs, gate_scale=gs, glu_op=glu_op, glu_limit=0.7)
    err = O.rel_l2(got, want)
    _note(f"  rel_l2={err:.3e}")
    assert err <= 1e-5


@pytest.mark.parametrize("wtype,shtype", [(10, 12), (12, 12), (2, 10), (14, 11)])
def test_gemv_shared_expert(torch_gpu, mc, O, wtype, shtype):
    torch = torch_gpu
    K, R, n_exp, n_used, n_tok = 4096, 36, 8, 4, 2
    _note(f"gemv shared routed={wtype} shared={shtype}")
    up = H.weights(wtype, n_exp, R, K, seed=801)
    gate = H.weights(wtype, n_exp, R, K, seed=802)
    sh_up = H.weights(shtype, 1, R, K, seed=803)[0]
    sh_gate = H.weights(shtype, 1, R, K, seed=804)[0]
    x = H.activations(n_tok, K, seed=805)
    ids = H.routing(n_tok, n_used, n_exp, seed=806)
    xd = _dev(torch, x)
    yq = mc.quantize_q8_1(xd).cpu().numpy().reshape(n_tok, 1, -1)
    sh_dst = torch.zeros((n_tok, R), dtype=torch.float32, device="cuda")
    su, sg = _dev(torch, sh_up), _dev(torch, sh_gate)
    f = mc.make_fusion(glu_op=2, shared_up=su, shared_gate=sg, shared_dst=sh_dst, shared_type=shtype)
    got = _run_gemv(torch, mc, wtype, up, ids, yq, K, R, n_exp, mc.ACT_Q8_1, fusion=f, gate=gate)
    want, want_sh = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=up, gate=gate, ids=ids, act=yq,
                                 act_kind=O.ACT_Q8_1, glu_op=2, sh_type=shtype, sh_up=sh_up, sh_gate=sh_gate)
    e1, e2 = O.rel_l2(got, want), O.rel_l2(sh_dst.cpu().numpy(), want_sh)
    _note(f"  routed rel_l2={e1:.3e} shared rel_l2={e2:.3e}")
    assert e1 <= 1e-5 and e2 <= 1e-5


def test_gemv_down_projection_channels(torch_gpu, mc, O):
    """Down-projection shape: one activation row per slot (nchannels_y = n_used), K = 768."""
    torch = torch_gpu
    wtype, K, R, n_exp, n_used, n_tok = 10, 768, 200, 16, 8, 2
    w = H.weights(wtype, n_exp, R, K, seed=901)
    x = H.activations(n_tok * n_used, K, seed=902)
    ids = H.routing(n_tok, n_used, n_exp, seed=903)
    yq = mc.quantize_q8_1(_dev(torch, x)).cpu().numpy().reshape(n_tok, n_used, -1)
    got = _run_gemv(torch, mc, wtype, w, ids, yq, K, R, n_exp, mc.ACT_Q8_1, nchannels_y=n_used)
    want = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=w, ids=ids, act=yq, act_kind=O.ACT_Q8_1,
                        nchannels_y=n_used)
    err = O.rel_l2(got, want)
    _note(f"down rel_l2={err:.3e}")
    assert err <= 1e-5


@pytest.mark.parametrize("wtype,shtype,K,gated", [(10, 12, 768, False), (2, 10, 1024, True), (12, 12, 4096, True),
                                                   (14, 11, 512, False), (6, 8, 2048, False)])
def test_gemv_f32_activations_equal_q8_1_path(torch_gpu, mc, O, wtype, shtype, K, gated):
    """fp32 activation rows quantized inside the GEMV give bit-identical outputs to the
    q8_1 quantizer followed by the q8_1 GEMV (routed slots with one row each, plus the
    shared expert reading its own row)."""
    torch = torch_gpu
    R, n_exp, n_used, n_tok = 70, 12, 4, 2
    _note(f"gemv f32 act type={wtype} shared={shtype} K={K} gated={gated}")
    up = H.weights(wtype, n_exp, R, K, seed=1001 + wtype)
    gate = H.weights(wtype, n_exp, R, K, seed=1002 + wtype) if gated else None
    sh_up = H.weights(shtype, 1, R, K, seed=1003)[0]
    x = H.activations(n_tok * (n_used + 1), K, seed=1004 + K).reshape(n_tok, n_used + 1, K)
    x[0, 1] = 0.0                                         # an all-zero row: d = 0, codes 0
    ids = H.routing(n_tok, n_used, n_exp, seed=1005)
    xd = _dev(torch, x)
    ids_d = _dev(torch, ids)
    yq = mc.quantize_q8_1(xd.view(-1, K)).view(n_tok, n_used + 1, -1)
    sh_up_d = _dev(torch, sh_up)
    outs = []
    for act, y, sh_row, stride in ((mc.ACT_Q8_1, yq, yq[:, n_used], (n_used + 1) * K // 32),
                                   (mc.ACT_F32, xd, xd[:, n_used], (n_used + 1) * K)):
        sh_dst = torch.zeros((n_tok, R), dtype=torch.float32, device="cuda")
        dst = torch.zeros((n_tok, n_used, R), dtype=torch.float32, device="cuda")
        f = mc.make_fusion(glu_op=2, shared_up=sh_up_d, shared_dst=sh_dst, shared_type=shtype,
                           shared_src1=sh_row, shared_stride_col_y=stride)
        keep = [f]
        if gated:
            gd = _dev(torch, gate)
            keep.append(gd)
            f.gate = gd.data_ptr()
        wd = _dev(torch, up)
        blk = 32 if act == mc.ACT_Q8_1 else 1
        src0 = mc.make_tensor(wtype, K, R, n_exp, wd.data_ptr(), keep=keep)
        import ctypes as C
        rc = mc.lib().ggml_hip_moe_mul_mat_vec_ex(0, act, C.byref(src0), None, C.byref(f), y.data_ptr(),
                                                   ids_d.data_ptr(), dst.data_ptr(), K, R, n_exp, n_tok,
                                                   n_used + 1, n_used, (n_used + 1) * K // blk, n_used * R, K // blk, R,
                                                   n_used, None)
        mc.check(rc, "mul_mat_vec_ex")
        torch.cuda.synchronize()
        outs.append((dst.cpu().numpy(), sh_dst.cpu().numpy()))
    assert np.isfinite(outs[0][0]).all() and np.isfinite(outs[0][1]).all()
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    # and the q8_1 path itself against the oracle on the same bytes
    yq_np = yq.cpu().numpy()
    want, want_sh = O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_exp, src0=up, gate=gate, ids=ids, act=yq_np[:, :n_used],
                                 act_kind=O.ACT_Q8_1, nchannels_y=n_used, glu_op=2, sh_type=shtype, sh_up=sh_up,
                                 sh_act=yq_np[:, n_used])
    assert O.rel_l2(outs[0][0], want) <= 1e-5 and O.rel_l2(outs[0][1], want_sh) <= 1e-5
