"""GPU: the fusion that ggml_hip_moe_fusion_detect finds in a MoE FFN block's nodes,
run as ONE ggml_hip_moe_mul_mat_id call, equals the block's unfused op sequence
computed by the oracle op by op (up and gate MUL_MAT_IDs, MUL by the per-expert
scale, ADD_ID of the per-expert bias, the GLU, and the shared expert's two MUL_MATs
+ GLU), on the same activation bytes.  The fused epilogue order is the reference's
(kernels/moe-cache.cu:246-282)."""
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


def _node(mc, op, t, srcs, glu_op=0, glu_limit=0.0):
    n = mc.Node()
    n.op = op
    n.t = t
    for k in range(3):
        s = srcs[k] if k < len(srcs) else None
        if isinstance(s, int):
            n.src[k] = s
        else:
            n.src[k] = -1
            if s is not None:
                n.leaf[k] = s
    n.glu_op, n.glu_limit = glu_op, glu_limit
    return n


def _glu(O, op, g, u, limit):
    f = np.vectorize(lambda a, b: O.glu(op, float(a), float(b), limit), otypes=[np.float32])
    return f(g, u)


@pytest.mark.parametrize("wtype,op,bias,scale,shared,n_tok", [
    (12, 2, False, False, False, 2),      # Q4_K SWIGLU
    (10, 3, True, True, True, 1),         # Q2_K SWIGLU_OAI, biases, scales, shared expert
    (2, 1, True, False, True, 3),         # Q4_0 GEGLU, biases, shared expert
    (14, 6, False, True, False, 2),       # Q6_K SWIGLU_CLAMP, scales
    (12, 2, False, False, False, 24),     # Q4_K SWIGLU, 24 tokens: the grouped GEMM with the fused gate
])
def test_detected_fusion_equals_unfused_sequence(torch_gpu, mc, O, wtype, op, bias, scale, shared, n_tok):
    torch = torch_gpu
    E, K, R, n_used, limit = 16, 1024, 96, 4, 7.0
    _note(f"fusion_detect type={wtype} glu={op} bias={bias} scale={scale} shared={shared} n_tok={n_tok}")
    rng = np.random.default_rng(4100 + wtype + n_tok)
    w_up = H.weights(wtype, E, R, K, seed=4101 + wtype)
    w_gate = H.weights(wtype, E, R, K, seed=4102 + wtype)
    x = H.activations(n_tok, K, seed=4103).reshape(n_tok, 1, K)
    ids = H.routing(n_tok, n_used, E, seed=4104)
    xb = (rng.standard_normal((E, R)) * 0.05).astype(np.float32)
    gb = (rng.standard_normal((E, R)) * 0.05).astype(np.float32)
    xs = rng.uniform(0.5, 1.5, (E, 1)).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, (E, 1)).astype(np.float32)
    sh_up = H.weights(wtype, 1, R, K, seed=4105 + wtype)
    sh_gate = H.weights(wtype, 1, R, K, seed=4106 + wtype)

    wu_d, wg_d, x_d, ids_d = _dev(torch, w_up), _dev(torch, w_gate), _dev(torch, x), _dev(torch, ids)
    xb_d, gb_d, xs_d, gs_d = _dev(torch, xb), _dev(torch, gb), _dev(torch, xs), _dev(torch, gs)
    shu_d, shg_d = _dev(torch, sh_up), _dev(torch, sh_gate)
    keep = []
    F32, I32 = mc.GGML_F32, mc.GGML_I32
    desc = lambda t, ty=F32: mc.torch_tensor_desc(t, ty, keep=keep)   # noqa: E731
    inter = lambda: torch.empty((n_tok, n_used, R), dtype=torch.float32, device="cuda")   # noqa: E731
    tx, tids = desc(x_d), desc(ids_d, I32)

    # the block as ggml builds it: up path, gate path, GLU; the shared expert beside it
    nodes = []

    def add(*a, **k):
        nodes.append(_node(mc, *a, **k))
        return len(nodes) - 1

    def path(w_d):
        cur = add(mc.OP_MUL_MAT_ID, desc(inter()), [mc.make_tensor(wtype, K, R, E, w_d.data_ptr(), keep=keep), tx, tids])
        first = cur
        sc, bi = (xs_d, xb_d) if w_d is wu_d else (gs_d, gb_d)
        if scale:
            cur = add(mc.OP_MUL, desc(inter()), [cur, desc(sc), tids])
        if bias:
            cur = add(mc.OP_ADD_ID, desc(inter()), [cur, desc(bi), tids])
        return first, cur

    up, up_end = path(wu_d)
    gate, gate_end = path(wg_d)
    out = torch.full((n_tok, n_used, R), -9.0, dtype=torch.float32, device="cuda")
    k_glu = add(mc.OP_GLU, desc(out), [gate_end, up_end], glu_op=op, glu_limit=limit)
    expected_nodes = 3 + 2 * (int(scale) + int(bias))
    sh_out = None
    if shared:
        xsh = desc(x_d.reshape(n_tok, K))
        su = add(mc.OP_MUL_MAT, desc(torch.empty((n_tok, R), dtype=torch.float32, device="cuda")),
                 [mc.make_tensor(wtype, K, R, 1, shu_d.data_ptr(), keep=keep), xsh])
        sg = add(mc.OP_MUL_MAT, desc(torch.empty((n_tok, R), dtype=torch.float32, device="cuda")),
                 [mc.make_tensor(wtype, K, R, 1, shg_d.data_ptr(), keep=keep), xsh])
        sh_out = torch.full((n_tok, R), -9.0, dtype=torch.float32, device="cuda")
        add(mc.OP_GLU, desc(sh_out), [sg, su], glu_op=op, glu_limit=limit)
        expected_nodes += 3

    n_cov, f, gate_host, covered, out_node = mc.fusion_detect(nodes, up)
    assert gate_host is None and out_node == k_glu and n_cov == expected_nodes and all(covered)
    assert f.gate == wg_d.data_ptr() and f.glu_op == op
    assert bool(f.shared_up) == shared

    mc.mul_mat_id(wtype=wtype, weights=wu_d, x=x_d, ids=ids_d, dst=out, K=K, R=R, n_experts=E, fusion=f)
    torch.cuda.synchronize()

    # the unfused sequence, op by op, on the CPU
    if n_tok > 8:
        mm = lambda w, n_as, i: O.cpu_mul_mat_id_f32(wtype=wtype, K=K, R=R, n_as=n_as, src0=w, src1=x, ids=i)  # noqa: E731
    else:
        yq = mc.quantize_q8_1(x_d.reshape(n_tok, K)).cpu().numpy().reshape(n_tok, 1, -1)
        mm = lambda w, n_as, i: O.mul_mat_id(wtype=wtype, K=K, R=R, n_as=n_as, src0=w, ids=i, act=yq,  # noqa: E731
                                             act_kind=O.ACT_Q8_1)
    u, g = mm(w_up, E, ids), mm(w_gate, E, ids)
    if scale:
        u, g = u * xs[ids], g * gs[ids]
    if bias:
        u, g = u + xb[ids], g + gb[ids]
    want = _glu(O, op, g, u, limit)
    err = O.rel_l2(out.cpu().numpy(), want)
    _note(f"  routed rel_l2={err:.3e}")
    assert err <= H.TOL_SAME
    if shared:
        z = np.zeros((n_tok, 1), np.int32)
        su_v, sg_v = mm(sh_up, 1, z)[:, 0], mm(sh_gate, 1, z)[:, 0]
        sh_want = _glu(O, op, sg_v, su_v, limit)
        sh_err = O.rel_l2(sh_out.cpu().numpy(), sh_want)
        _note(f"  shared rel_l2={sh_err:.3e}")
        assert sh_err <= H.TOL_SAME
