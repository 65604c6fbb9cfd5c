"""GPU: the fused decode kernels (ggml_hip_moe_ffn_gate_up_norm and
ggml_hip_moe_ffn_down_combine) against the op-by-op path (combine + RMSNorm +
q8_1, then the MUL_MAT_ID GEMVs, then the weighted combine).  Both run the same
steps in the same arithmetic order, so every output must be bit-identical; the
op-by-op path is checked against the CPU oracle in test_gpu_decode.py and
test_gpu_parity.py, and the fused path is also checked against the oracle here
on its own intermediate bytes."""
import ctypes as C
from importlib import import_module

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SENTINEL = -7.25


def _note(msg):
    print(msg, flush=True)


def _stream(torch):
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _norm_q8_1(torch, mc, x, nw, eps):
    """q8_1((x * rms scale) * nw) of each row through the combine kernel (no expert terms)."""
    n_tok, K = x.shape
    y = torch.zeros((n_tok, K // 32 * 36), dtype=torch.uint8, device="cuda")
    mc.check(mc.lib().ggml_hip_moe_combine_q8_1(None, 0, None, 0, None, 0, x.data_ptr(), None, y.data_ptr(), K // 32,
                                                K, n_tok, 1, nw.data_ptr() if nw is not None else None, eps,
                                                _stream(torch)), "norm")
    return y


@pytest.mark.parametrize("wtype,sh_type,K,R,n_tok,with_nw,bad_id,sh_q8", [
    ("Q2_K", "Q4_K", 1024, 256, 1, True, False, True),
    ("Q2_K", "Q4_K", 4096, 96, 3, True, True, True),
    ("Q4_K", "Q6_K", 2048, 160, 2, False, False, True),
    ("Q3_K", None, 1024, 128, 1, True, False, True),
    ("Q6_K", "Q5_K", 1024, 64, 2, True, True, True),
    ("Q5_K", "Q2_K", 768, 200, 1, True, False, True),
    # rows longer than 16 chunks: eight chunks per prologue wave (no q8_1 copies: mixed workgroups,
    # each an even share of a token's routed and shared steps)
    ("Q2_K", "Q4_K", 6144, 96, 2, True, True, True),
    ("Q4_K", "Q2_K", 8192, 64, 1, False, False, True),
    ("Q2_K", "Q4_K", 6144, 200, 3, True, True, True),
    # routed q8_1 copies without the shared one: shared-expert workgroups sized by bytes
    ("Q2_K", "Q4_K", 4096, 768, 1, True, False, False),
    ("Q2_K", "Q6_K", 2048, 96, 3, True, True, False),
    ("Q4_K", "Q2_K", 1024, 256, 2, False, False, False),
])
def test_gate_up_norm_equals_norm_then_gemv(torch_gpu, mc, wtype, sh_type, K, R, n_tok, with_nw, bad_id, sh_q8):
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    _note(f"gate_up_norm {wtype}/{sh_type} K={K} R={R} tok={n_tok} nw={with_nw} bad_id={bad_id} sh_q8={sh_q8}")
    E, U, eps = 16, 4, 1e-6
    tw = getattr(mc, wtype)
    ts = getattr(mc, sh_type) if sh_type else None
    gen = torch.Generator(device="cuda")
    gen.manual_seed(K + R + n_tok)
    up = md.random_expert_tensor(torch, tw, E, R, K, gen)
    gate = md.random_expert_tensor(torch, tw, E, R, K, gen)
    sh_up = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    sh_gate = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    rng = np.random.default_rng(K * 7 + n_tok)
    x = torch.from_numpy(rng.standard_normal((n_tok, K)).astype(np.float32) * 3).cuda()
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).cuda() if with_nw else None
    ids_np = np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)
    if bad_id:
        ids_np[-1, 1] = -1
    ids = torch.from_numpy(ids_np).cuda()

    # op by op: RMSNorm + q8_1 through the combine kernel, then the q8_1 GEMV
    y_ref = _norm_q8_1(torch, mc, x, nw, eps)
    dst_ref = torch.full((n_tok, U, R), SENTINEL, dtype=torch.float32, device="cuda")
    sh_ref = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    f_ref = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, shared_up=sh_up, shared_gate=sh_gate,
                           shared_dst=sh_ref if ts else None, shared_type=ts if ts else -1)
    mc.mul_mat_vec(wtype=tw, weights=up, ids=ids, y=y_ref.view(n_tok, 1, -1), dst=dst_ref, K=K, R=R, n_experts=E,
                   fusion=f_ref)

    # fused
    dst = torch.full((n_tok, U, R), SENTINEL, dtype=torch.float32, device="cuda")
    sh = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    y_out = torch.zeros_like(y_ref)
    f = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, shared_up=sh_up, shared_gate=sh_gate,
                       shared_dst=sh if ts else None, shared_type=ts if ts else -1)
    q8 = R % 32 == 0 and K <= 4096            # q8_1 copies of the outputs need 32-row blocks
    dq = torch.zeros((n_tok, U, R // 32 * 36), dtype=torch.uint8, device="cuda") if q8 else None
    shq = torch.zeros((n_tok, R // 32 * 36), dtype=torch.uint8, device="cuda") if q8 and ts and sh_q8 else None
    mc.ffn_gate_up_norm(wtype=tw, weights=up, ids=ids, x=x, dst=dst, K=K, R=R, n_experts=E, norm_weight=nw, eps=eps,
                        fusion=f, y_out=y_out, dst_q8_1=dq, shared_dst_q8_1=shq)
    torch.cuda.synchronize()
    assert torch.equal(y_out, y_ref)
    assert torch.equal(dst, dst_ref)
    if ts:
        assert torch.equal(sh, sh_ref)
    if q8:
        # bit-identical to the q8_1 quantizer run on the fp32 outputs (skipped picks excepted)
        for ti in range(n_tok):
            for c in range(U):
                if ids_np[ti, c] >= 0:
                    assert torch.equal(dq[ti, c], mc.quantize_q8_1(dst[ti, c].view(1, R))[0]), (ti, c)
            if ts and sh_q8:
                assert torch.equal(shq[ti], mc.quantize_q8_1(sh[ti].view(1, R))[0])
    if bad_id:
        assert bool((dst[-1, 1] == SENTINEL).all())
    assert bool(torch.isfinite(dst[dst != SENTINEL]).all())


@pytest.mark.parametrize("wtype,sh_type,K,R,n_tok,U,act,residual,fuse_bias,bad_id", [
    ("Q2_K", "Q4_K", 768, 4096, 1, 8, "f32", True, False, False),
    ("Q2_K", "Q4_K", 512, 1024, 2, 4, "q8_1", True, False, True),
    # q8_1 routed rows, fp32 shared rows quantized by the shared wave
    ("Q2_K", "Q4_K", 768, 4096, 1, 8, "q8_1+shf32", True, False, False),
    ("Q3_K", "Q6_K", 512, 512, 3, 4, "q8_1+shf32", True, True, True),
    ("Q5_K", None, 768, 1280, 3, 6, "f32", False, True, False),      # 15-row tiles, the last one partial
    ("Q3_K", "Q6_K", 512, 512, 3, 4, "f32", True, True, True),
    ("Q6_K", "Q4_K", 1024, 512, 1, 11, "q8_1", True, False, False),   # 12 waves per workgroup
])
def test_down_combine_equals_gemv_then_combine(torch_gpu, mc, wtype, sh_type, K, R, n_tok, U, act, residual,
                                               fuse_bias, bad_id):
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    assert R % 256 == 0                       # the op-by-op combine works on 256-value chunks
    _note(f"down_combine {wtype}/{sh_type} K={K} R={R} tok={n_tok} U={U} act={act} res={residual} "
          f"bias={fuse_bias} bad_id={bad_id}")
    E = 16
    tw = getattr(mc, wtype)
    ts = getattr(mc, sh_type) if sh_type else None
    act_fmt = mc.ACT_F32 if act == "f32" else mc.ACT_Q8_1
    sh_f32 = act == "q8_1+shf32"
    gen = torch.Generator(device="cuda")
    gen.manual_seed(K + R + U)
    down = md.random_expert_tensor(torch, tw, E, R, K, gen)
    sh_down = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    rng = np.random.default_rng(R + n_tok)
    h_f = torch.from_numpy(rng.standard_normal((n_tok, U, K)).astype(np.float32)).cuda()
    hs_f = torch.from_numpy(rng.standard_normal((n_tok, K)).astype(np.float32)).cuda()
    if act_fmt == mc.ACT_F32:
        h, hs, sh_stride = h_f, hs_f, K
    else:
        h = mc.quantize_q8_1(h_f.view(n_tok * U, K)).view(n_tok, U, -1)
        hs = mc.quantize_q8_1(hs_f)
        sh_stride = K // 32
    x = torch.from_numpy(rng.standard_normal((n_tok, R)).astype(np.float32)).cuda() if residual else None
    w = torch.from_numpy(rng.dirichlet(np.ones(U), n_tok).astype(np.float32)).cuda()
    ids_np = np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)
    if bad_id:
        ids_np[0, U - 1] = E + 3
    ids = torch.from_numpy(ids_np).cuda()
    bias = torch.from_numpy(rng.standard_normal((E, R)).astype(np.float32) * 0.1).cuda() if fuse_bias else None
    scale = torch.from_numpy(rng.uniform(0.5, 1.5, E).astype(np.float32)).cuda() if fuse_bias else None

    # op by op: down GEMV (an out-of-range id leaves its rows at 0), then the combine
    o = torch.zeros((n_tok, U, R), dtype=torch.float32, device="cuda")
    o_sh = torch.zeros((n_tok, R), dtype=torch.float32, device="cuda")
    f_ref = mc.make_fusion(x_bias=bias, x_scale=scale, shared_up=sh_down, shared_dst=o_sh if ts else None,
                           shared_type=ts if ts else -1, shared_src1=hs if ts else None,
                           shared_stride_col_y=sh_stride, bias_stride=R)
    mc.mul_mat_vec(wtype=tw, weights=down, ids=ids, y=h, dst=o, K=K, R=R, n_experts=E, act=act_fmt, fusion=f_ref,
                   nchannels_y=U)
    x_ref = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    mc.combine_q8_1(o, w, shared=o_sh if ts else None, residual=x, x_out=x_ref)

    x_out = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    f = mc.make_fusion(x_bias=bias, x_scale=scale, shared_up=sh_down, shared_type=ts if ts else -1,
                       shared_src1=(hs_f if sh_f32 else hs) if ts else None,
                       shared_stride_col_y=K if sh_f32 else sh_stride, bias_stride=R)
    mc.ffn_down_combine(wtype=tw, weights=down, ids=ids, h=h, router_w=w, x_out=x_out, K=K, R=R, n_experts=E,
                        residual=x, act=act_fmt | (mc.ACT_SHARED_F32 if sh_f32 else 0), fusion=f)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(x_ref).all())
    assert torch.equal(x_out, x_ref)


def test_down_combine_in_place_residual(torch_gpu, mc):
    """residual == x_out: every row is read and written by the same lane."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    E, U, K, R = 8, 4, 512, 768
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    down = md.random_expert_tensor(torch, mc.Q2_K, E, R, K, gen)
    rng = np.random.default_rng(5)
    h = torch.from_numpy(rng.standard_normal((1, U, K)).astype(np.float32)).cuda()
    x = torch.from_numpy(rng.standard_normal((1, R)).astype(np.float32)).cuda()
    w = torch.from_numpy(rng.dirichlet(np.ones(U), 1).astype(np.float32)).cuda()
    ids = torch.from_numpy(rng.choice(E, (1, U), replace=False).astype(np.int32)).cuda()
    want = torch.empty_like(x)
    mc.ffn_down_combine(wtype=mc.Q2_K, weights=down, ids=ids, h=h, router_w=w, x_out=want, K=K, R=R, n_experts=E,
                        residual=x)
    got = x.clone()
    mc.ffn_down_combine(wtype=mc.Q2_K, weights=down, ids=ids, h=h, router_w=w, x_out=got, K=K, R=R, n_experts=E,
                        residual=got)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_fused_layer_against_oracle(torch_gpu, mc, O):
    """The fused pair on its own intermediate bytes: y_out against the oracle's RMSNorm + q8_1,
    the GLU rows against the oracle's MUL_MAT_ID on y, x_out against the oracle's down
    projection of q8_1(h) and combine."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    m = md.MoeDecodeModel(torch, n_layers=1, n_experts=16, hidden=1024, ffn=512, n_used=4, seed=9)
    H, F, U, E = m.H, m.F, m.U, m.E
    ids, w = md.make_routing(1, 1, E, U, seed=3)
    rng = np.random.default_rng(8)
    x0 = rng.standard_normal((1, H)).astype(np.float32) * 2
    m.x.copy_(torch.from_numpy(x0))
    m.set_routing(torch.from_numpy(ids[0]), torch.from_numpy(w[0]))
    y_out = torch.zeros((1, H // 32 * 36), dtype=torch.uint8, device="cuda")
    ly = m.layers[0]
    mc.check(mc.lib().ggml_hip_moe_ffn_gate_up_norm(0, C.byref(ly.t_up), None, C.byref(ly.f_gu), m.x.data_ptr(),
                                                    m.norm[0].data_ptr(), m.eps, m.ids[0].data_ptr(), m.h.data_ptr(),
                                                    H, F, E, 1, U, H, U * F, F, U, y_out.data_ptr(), H // 32,
                                                    m.hq.data_ptr(), (U + 1) * F // 32, F // 32,
                                                    m.hq[U:].data_ptr(), (U + 1) * F // 32, _stream(torch)),
             "gate_up_norm")
    torch.cuda.synchronize()
    nw = m.norm[0].cpu().numpy()
    _, want_y = O.combine_q8_1(np.zeros((1, 0, H), np.float32), np.zeros((1, 0), np.float32), residual=x0,
                               rms_norm=True, norm_weight=nw, eps=m.eps)
    y = y_out.cpu().numpy()
    assert np.array_equal(y, want_y)
    g, u, d = ly.gate.cpu().numpy(), ly.up.cpu().numpy(), ly.down.cpu().numpy()
    sg, su, sd = ly.sh_gate.cpu().numpy(), ly.sh_up.cpu().numpy(), ly.sh_down.cpu().numpy()
    lid = ids[0, 0].reshape(1, U)
    h = m.h.cpu().numpy()
    assert np.array_equal(m.hq.cpu().numpy(), np.stack([O.quantize_q8_1(r) for r in h]))   # q8_1 copy of h
    want_h, want_hs = O.mul_mat_id(wtype=m.wtype, K=H, R=F, n_as=E, src0=u, gate=g, ids=lid, act=y.reshape(1, 1, -1),
                                   act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU, sh_type=m.sh_type, sh_up=su, sh_gate=sg)
    assert O.rel_l2(h[:U], want_h[0]) <= 1e-5
    assert O.rel_l2(h[U], want_hs[0]) <= 1e-5
    m.launch_down_combine(0, m.x, m.x_next)
    torch.cuda.synchronize()
    hq = np.stack([O.quantize_q8_1(r) for r in h])
    want_o, want_osh = O.mul_mat_id(wtype=m.wtype, K=F, R=H, n_as=E, src0=d, ids=lid, act=hq[:U].reshape(1, U, -1),
                                    act_kind=O.ACT_Q8_1, nchannels_y=U, sh_type=m.sh_type, sh_up=sd,
                                    sh_act=hq[U:].reshape(1, -1))
    want_x, _ = O.combine_q8_1(want_o, w[0, 0].reshape(1, U), shared=want_osh, residual=x0)
    assert O.rel_l2(m.x_next.cpu().numpy(), want_x) <= 1e-5


@pytest.mark.parametrize("hand_off", ["q8_1", "f32"])
def test_fused_decode_equals_op_plan(torch_gpu, mc, hand_off):
    """Three tokens through the fused plan and through the op-by-op plan: identical
    residual streams after every token, eager and under graph replay.  hand_off f32: the
    gate/up launch writes only fp32 GLU rows and every down wave quantizes its row to q8_1."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    m = md.MoeDecodeModel(torch, n_layers=3, n_experts=16, hidden=1024, ffn=512, n_used=4, seed=5, fused=False)
    ids, w = md.make_routing(3, m.L, m.E, m.U, seed=21)
    ids_d, w_d = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    x0 = torch.from_numpy(np.random.default_rng(6).standard_normal((1, m.H)).astype(np.float32)).cuda()
    ref = []
    m.x.copy_(x0)
    for t in range(3):
        m.set_routing(ids_d[t], w_d[t])
        m.launch_token()
        torch.cuda.synchronize()
        ref.append(m.x.clone())
    m.fused = True
    m.hand_off = hand_off
    m.x.copy_(x0)
    for t in range(3):
        m.set_routing(ids_d[t], w_d[t])
        m.launch_token()
        torch.cuda.synchronize()
        assert torch.equal(m.x, ref[t]), f"fused token {t} differs"
    m.x.copy_(x0)
    m.set_routing(ids_d[0], w_d[0])
    m.capture()
    m.x.copy_(x0)
    for t in range(3):
        m.set_routing(ids_d[t], w_d[t])
        m.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.x, ref[t]), f"fused replay {t} differs"


def test_fused_block_through_the_cache(torch_gpu, mc):
    """Both fused launches on cache-managed experts (pinned host tensors behind LSB-tagged tables,
    promoted into the HBM pool by the step between tokens): outputs bit-identical to the same
    launches on device-resident copies, and the recorder counts every pick of the three tensors."""
    torch = torch_gpu
    import helpers as H
    E, U, H_, F, n_tok, slots = 16, 4, 1024, 256, 2, 6
    wt, st = mc.Q2_K, mc.Q4_K
    mc.reset()
    mc.configure(enabled=True, slots=slots)
    stream = _stream(torch)
    w_np = {r: H.weights(wt, E, F, H_, seed=40 + i) for i, r in enumerate(("gate", "up"))}
    w_np["down"] = H.weights(wt, E, H_, F, seed=43)
    host, dev, keep = {}, {}, []
    for r, arr in w_np.items():
        p = torch.empty(arr.size, dtype=torch.uint8, pin_memory=True)
        p.numpy()[:] = arr.reshape(-1)
        host[r], dev[r] = p, torch.from_numpy(arr).cuda()
    t_up = mc.make_tensor(wt, H_, F, E, host["up"].data_ptr(), name="blk.0.ffn_up_exps.weight", keep=keep)
    t_gate = mc.make_tensor(wt, H_, F, E, host["gate"].data_ptr(), name="blk.0.ffn_gate_exps.weight", keep=keep)
    t_down = mc.make_tensor(wt, F, H_, E, host["down"].data_ptr(), name="blk.0.ffn_down_exps.weight", keep=keep)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(12)
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    sh = {r: md.random_expert_tensor(torch, st, 1, rows, k, gen)[0]
          for r, rows, k in (("gate", F, H_), ("up", F, H_), ("down", H_, F))}
    rng = np.random.default_rng(31)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, H_).astype(np.float32)).cuda()
    ids = torch.zeros((n_tok, U), dtype=torch.int32, device="cuda")
    w = torch.zeros((n_tok, U), dtype=torch.float32, device="cuda")

    def block(use_cache, x):
        h = torch.zeros((n_tok, U + 1, F), dtype=torch.float32, device="cuda")
        hq = torch.zeros((n_tok, U + 1, F // 32 * 36), dtype=torch.uint8, device="cuda")
        out = torch.zeros_like(x)
        f_gu = mc.make_fusion(glu_op=mc.GLU_SWIGLU, shared_up=sh["up"], shared_gate=sh["gate"],
                              shared_dst=h[:, U], shared_type=st)
        f_gu.shared_stride_col_dst = (U + 1) * F
        if not use_cache:
            f_gu.gate = dev["gate"].data_ptr()
        src_up = t_up if use_cache else mc.make_tensor(wt, H_, F, E, dev["up"].data_ptr(), keep=keep)
        mc.check(mc.lib().ggml_hip_moe_ffn_gate_up_norm(
            1 if use_cache else 0, C.byref(src_up), C.byref(t_gate) if use_cache else None, C.byref(f_gu),
            x.data_ptr(), nw.data_ptr(), 1e-6, ids.data_ptr(), h.data_ptr(), H_, F, E, n_tok, U, H_,
            (U + 1) * F, F, U, None, 0, hq.data_ptr(), (U + 1) * F // 32, F // 32, hq[:, U].data_ptr(),
            (U + 1) * F // 32, stream), "gate_up_norm")
        f_dn = mc.make_fusion(shared_up=sh["down"], shared_type=st, shared_src1=hq[:, U],
                              shared_stride_col_y=(U + 1) * F // 32)
        src_dn = t_down if use_cache else mc.make_tensor(wt, F, H_, E, dev["down"].data_ptr(), keep=keep)
        mc.check(mc.lib().ggml_hip_moe_ffn_down_combine(
            1 if use_cache else 0, mc.ACT_Q8_1, C.byref(src_dn), C.byref(f_dn), hq.data_ptr(), ids.data_ptr(),
            w.data_ptr(), x.data_ptr(), out.data_ptr(), F, H_, E, n_tok, U, (U + 1) * F // 32, F // 32, H_, U,
            stream), "down_combine")
        return h, out

    x = torch.from_numpy(rng.standard_normal((n_tok, H_)).astype(np.float32)).cuda()
    for step in range(6):
        ids.copy_(torch.from_numpy(np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)))
        w.copy_(torch.from_numpy(rng.dirichlet(np.ones(U), n_tok).astype(np.float32)))
        h_c, x_c = block(True, x)
        stats = mc.stats_snapshot()
        h_r, x_r = block(False, x)
        torch.cuda.synchronize()
        assert torch.equal(h_c, h_r), f"step {step}: GLU rows differ between cache and resident paths"
        assert torch.equal(x_c, x_r), f"step {step}: residual differs between cache and resident paths"
        assert int(stats[0]) + int(stats[1]) == 3 * n_tok * U, (step, int(stats[0]), int(stats[1]))
        mc.step()
        x = x_c
    tot = mc.totals()
    assert tot.promotions > 0 and tot.hits > 0
    mc.reset()


def test_gate_up_norm_timeout_reports_status(torch_gpu, mc):
    """A bounded wait that gives up is reported, not silent: with the debug spin limit 0 every wait of the
    fused gate/up kernel gives up at once (every kernel still exits: the waits poll zero times), and
    ggml_hip_moe_check_status returns E_TIMEOUT once, then 0.  With the default limit the same launch
    matches the op-by-op path and reports nothing."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    _note("gate_up_norm timeout status")
    E, U, K, R, n_tok, eps = 8, 4, 1024, 64, 1, 1e-6
    gen = torch.Generator(device="cuda")
    gen.manual_seed(91)
    up = md.random_expert_tensor(torch, mc.Q2_K, E, R, K, gen)
    gate = md.random_expert_tensor(torch, mc.Q2_K, E, R, K, gen)
    rng = np.random.default_rng(92)
    x = torch.from_numpy(rng.standard_normal((n_tok, K)).astype(np.float32)).cuda()
    ids = torch.from_numpy(np.array([[0, 3, 5, 7]], np.int32)).cuda()
    f = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU)
    assert mc.check_status() == 0                      # nothing pending from earlier tests
    dst = torch.full((n_tok, U, R), SENTINEL, dtype=torch.float32, device="cuda")
    try:
        assert mc.lib().ggml_hip_moe_debug_set_spin_limit(0) == 0
        mc.ffn_gate_up_norm(wtype=mc.Q2_K, weights=up, ids=ids, x=x, dst=dst, K=K, R=R, n_experts=E, eps=eps,
                            fusion=f)
    finally:
        mc.lib().ggml_hip_moe_debug_set_spin_limit(-1)
    rc = mc.check_status()
    assert rc == mc.E_TIMEOUT, rc
    assert b"gave up" in mc.lib().ggml_hip_moe_last_error()
    assert bool((dst == SENTINEL).all())               # every step skipped its rows
    assert mc.check_status() == 0                      # cleared
    mc.ffn_gate_up_norm(wtype=mc.Q2_K, weights=up, ids=ids, x=x, dst=dst, K=K, R=R, n_experts=E, eps=eps, fusion=f)
    assert mc.check_status() == 0
    y_ref = _norm_q8_1(torch, mc, x, None, eps)
    dst_ref = torch.zeros_like(dst)
    mc.mul_mat_vec(wtype=mc.Q2_K, weights=up, ids=ids, y=y_ref.view(n_tok, 1, -1), dst=dst_ref, K=K, R=R,
                   n_experts=E, fusion=f)
    torch.cuda.synchronize()
    assert torch.equal(dst, dst_ref)


# ---------------------------------------------------------------------------
# q8_K mode: the dots on q8_K rows (ggml-CPU's MUL_MAT_ID activations for K-quant experts)
# ---------------------------------------------------------------------------

def _normalized(O, x, nw, eps):
    """(x * s) * nw with s = 1/sqrt(mean(x^2) + eps), the mean of squares in the canonical order."""
    K = x.shape[-1]
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        ss = np.float32(O.rms_sum(x[t]))
        s = np.float32(1.0) / np.sqrt(ss / np.float32(K) + np.float32(eps))
        v = (x[t] * s).astype(np.float32)
        out[t] = (v * nw).astype(np.float32) if nw is not None else v
    return out


@pytest.mark.parametrize("wtype,sh_type,K,R,n_tok,with_nw,bad_id", [
    ("Q2_K", "Q4_K", 4096, 768, 1, True, False),
    ("Q2_K", "Q4_K", 2048, 96, 3, True, True),
    ("Q4_K", "Q6_K", 1024, 160, 2, False, False),
    ("Q3_K", None, 1024, 128, 1, True, False),
    ("Q5_K", "Q2_K", 8192, 64, 1, True, False),
])
def test_gate_up_norm_q8K(torch_gpu, mc, O, wtype, sh_type, K, R, n_tok, with_nw, bad_id):
    """q8_K rows: y_out byte-identical to the oracle's q8_K of the normalized row, the outputs
    bit-identical to the q8_K GEMV on those rows and within fp32 summation order of the oracle."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    _note(f"gate_up_norm q8_K {wtype}/{sh_type} K={K} R={R} tok={n_tok} nw={with_nw} bad_id={bad_id}")
    E, U, eps = 16, 4, 1e-6
    tw = getattr(mc, wtype)
    ts = getattr(mc, sh_type) if sh_type else None
    gen = torch.Generator(device="cuda")
    gen.manual_seed(K + R + n_tok + 1)
    up = md.random_expert_tensor(torch, tw, E, R, K, gen)
    gate = md.random_expert_tensor(torch, tw, E, R, K, gen)
    sh_up = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    sh_gate = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    rng = np.random.default_rng(K * 5 + n_tok)
    x_np = (rng.standard_normal((n_tok, K)) * 3).astype(np.float32)
    nw_np = rng.uniform(0.5, 1.5, K).astype(np.float32) if with_nw else None
    ids_np = np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)
    if bad_id:
        ids_np[-1, 2] = E + 5
    x, ids = torch.from_numpy(x_np).cuda(), torch.from_numpy(ids_np).cuda()
    nw = torch.from_numpy(nw_np).cuda() if with_nw else None

    dst = torch.full((n_tok, U, R), SENTINEL, dtype=torch.float32, device="cuda")
    sh = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    y_out = torch.zeros((n_tok, K // 256 * 292), dtype=torch.uint8, device="cuda")
    f = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, shared_up=sh_up, shared_gate=sh_gate,
                       shared_dst=sh if ts else None, shared_type=ts if ts else -1)
    mc.ffn_gate_up_norm(wtype=tw, weights=up, ids=ids, x=x, dst=dst, K=K, R=R, n_experts=E, norm_weight=nw, eps=eps,
                        fusion=f, y_out=y_out, act=mc.ACT_Q8_K)
    torch.cuda.synchronize()
    want_y = np.stack([O.quantize_q8_K(r) for r in _normalized(O, x_np, nw_np, eps)])
    assert np.array_equal(y_out.cpu().numpy(), want_y)

    # the q8_K GEMV on the same rows: bit-identical
    dst_ref = torch.full((n_tok, U, R), SENTINEL, dtype=torch.float32, device="cuda")
    sh_ref = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    f_ref = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, shared_up=sh_up, shared_gate=sh_gate,
                           shared_dst=sh_ref if ts else None, shared_type=ts if ts else -1)
    mc.mul_mat_vec(wtype=tw, weights=up, ids=ids, y=y_out.view(n_tok, 1, -1), dst=dst_ref, K=K, R=R, n_experts=E,
                   act=mc.ACT_Q8_K, fusion=f_ref)
    torch.cuda.synchronize()
    assert torch.equal(dst, dst_ref)
    if ts:
        assert torch.equal(sh, sh_ref)
    # and the oracle
    ok = ids_np >= 0
    ok &= ids_np < E
    got = dst.cpu().numpy()
    kw = dict(sh_type=ts, sh_up=sh_up.cpu().numpy(), sh_gate=sh_gate.cpu().numpy()) if ts else {}
    res = O.mul_mat_id(wtype=tw, K=K, R=R, n_as=E, src0=up.cpu().numpy(), gate=gate.cpu().numpy(),
                       ids=np.where(ok, ids_np, 0).astype(np.int32), act=want_y.reshape(n_tok, 1, -1),
                       act_kind=O.ACT_CPU, glu_op=O.GLU_SWIGLU, **kw)
    want, want_sh = res if ts else (res, None)
    assert O.rel_l2(got[ok], want[ok]) <= 1e-5
    if bad_id:
        assert bool((dst[-1, 2] == SENTINEL).all())
    if ts:
        assert O.rel_l2(sh.cpu().numpy(), want_sh) <= 1e-5


@pytest.mark.parametrize("wtype,sh_type,K,R,n_tok,U,residual,bad_id", [
    ("Q2_K", "Q4_K", 768, 4096, 1, 8, True, False),
    ("Q3_K", "Q6_K", 512, 512, 3, 4, True, True),
    ("Q5_K", None, 768, 1280, 2, 6, False, False),
])
def test_down_combine_q8K(torch_gpu, mc, O, wtype, sh_type, K, R, n_tok, U, residual, bad_id):
    """fp32 rows quantized to q8_K in the launch: bit-identical to q8_K quantizer + q8_K GEMV +
    combine, and within fp32 summation order of the oracle."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    _note(f"down_combine q8_K {wtype}/{sh_type} K={K} R={R} tok={n_tok} U={U} res={residual} bad_id={bad_id}")
    E = 16
    tw = getattr(mc, wtype)
    ts = getattr(mc, sh_type) if sh_type else None
    gen = torch.Generator(device="cuda")
    gen.manual_seed(K + R + U + 3)
    down = md.random_expert_tensor(torch, tw, E, R, K, gen)
    sh_down = md.random_expert_tensor(torch, ts, 1, R, K, gen)[0] if ts else None
    rng = np.random.default_rng(R + n_tok + 1)
    h = torch.from_numpy(rng.standard_normal((n_tok, U, K)).astype(np.float32)).cuda()
    hs = torch.from_numpy(rng.standard_normal((n_tok, K)).astype(np.float32)).cuda()
    x = torch.from_numpy(rng.standard_normal((n_tok, R)).astype(np.float32)).cuda() if residual else None
    w = torch.from_numpy(rng.dirichlet(np.ones(U), n_tok).astype(np.float32)).cuda()
    ids_np = np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)
    if bad_id:
        ids_np[0, U - 1] = -2
    ids = torch.from_numpy(ids_np).cuda()

    # op by op: q8_K quantizer, q8_K GEMV, combine
    hq = mc.quantize_q8_K(h.view(n_tok * U, K)).view(n_tok, U, -1)
    hsq = mc.quantize_q8_K(hs)
    o = torch.zeros((n_tok, U, R), dtype=torch.float32, device="cuda")
    o_sh = torch.zeros((n_tok, R), dtype=torch.float32, device="cuda")
    f_ref = mc.make_fusion(shared_up=sh_down, shared_dst=o_sh if ts else None, shared_type=ts if ts else -1,
                           shared_src1=hsq if ts else None, shared_stride_col_y=K // 256)
    mc.mul_mat_vec(wtype=tw, weights=down, ids=ids, y=hq, dst=o, K=K, R=R, n_experts=E, act=mc.ACT_Q8_K,
                   fusion=f_ref, nchannels_y=U)
    x_ref = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    mc.combine_q8_1(o, w, shared=o_sh if ts else None, residual=x, x_out=x_ref)

    x_out = torch.full((n_tok, R), SENTINEL, dtype=torch.float32, device="cuda")
    f = mc.make_fusion(shared_up=sh_down, shared_type=ts if ts else -1, shared_src1=hs if ts else None,
                       shared_stride_col_y=K)
    mc.ffn_down_combine(wtype=tw, weights=down, ids=ids, h=h, router_w=w, x_out=x_out, K=K, R=R, n_experts=E,
                        residual=x, act=mc.ACT_F32 | mc.ACT_DOT_Q8_K, fusion=f)
    torch.cuda.synchronize()
    assert torch.equal(x_out, x_ref)
    # the oracle on the same q8_K bytes
    hq_np = hq.cpu().numpy()
    assert np.array_equal(hq_np.reshape(n_tok * U, -1), np.stack([O.quantize_q8_K(r) for r in h.cpu().numpy().reshape(-1, K)]))
    ok = (ids_np >= 0) & (ids_np < E)
    kw = dict(sh_type=ts, sh_up=sh_down.cpu().numpy(), sh_act=hsq.cpu().numpy()) if ts else {}
    res = O.mul_mat_id(wtype=tw, K=K, R=R, n_as=E, src0=down.cpu().numpy(), ids=np.where(ok, ids_np, 0).astype(np.int32),
                       act=hq_np, act_kind=O.ACT_CPU, nchannels_y=U, **kw)
    want_o, want_sh = res if ts else (res, None)
    want_o = np.where(ok[:, :, None], want_o, 0.0).astype(np.float32)
    want_x, _ = O.combine_q8_1(want_o, w.cpu().numpy(), shared=want_sh, residual=x.cpu().numpy() if residual else None)
    assert O.rel_l2(x_out.cpu().numpy(), want_x) <= 1e-5


@pytest.mark.parametrize("n_layers,mix", [(2, "pure"), (8, "q2_K_s")])
def test_fused_q8K_decode_against_ggml_cpu(torch_gpu, mc, O, n_layers, mix):
    """The headline decode block in q8_K mode against the ggml-CPU MUL_MAT_ID restatement
    (fp32 src1 quantized to q8_K inside, K-quant x q8_K dots), op by op: RMSNorm, gate/up +
    SwiGLU, down, router-weighted combine with the shared expert and the residual.  q2_K_s:
    the first n_layers / 8 layers' down experts in Q4_K."""
    torch = torch_gpu
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    _note(f"q8_K decode {n_layers} layers, mix {mix}")
    m = md.MoeDecodeModel(torch, n_layers=n_layers, n_experts=32, hidden=2048, ffn=768, n_used=8, seed=12, act="q8_K",
                          mix=mix)
    if mix == "q2_K_s":
        assert m.down_types[0] == mc.Q4_K and m.down_types[1] == m.wtype
    H, F, U, E = m.H, m.F, m.U, m.E
    ids, w = md.make_routing(1, m.L, E, U, seed=4)
    x0 = (np.random.default_rng(13).standard_normal((1, H)) * 2).astype(np.float32)
    m.x.copy_(torch.from_numpy(x0))
    m.set_routing(torch.from_numpy(ids[0]), torch.from_numpy(w[0]))
    m.launch_token()
    torch.cuda.synchronize()
    got = m.x.cpu().numpy()
    x = x0.copy()
    for l in range(m.L):
        ly = m.layers[l]
        lid = ids[0, l].reshape(1, U)
        y = _normalized(O, x, m.norm[l].cpu().numpy(), m.eps).reshape(1, 1, H)
        cpu = lambda wt, t, K, R, n_as, src1, i: O.cpu_mul_mat_id_f32(wtype=wt, K=K, R=R, n_as=n_as,  # noqa: E731
                                                                      src0=t.cpu().numpy().reshape(n_as, R, -1),
                                                                      src1=src1, ids=i)
        g = cpu(m.wtype, ly.gate, H, F, E, y, lid)
        u = cpu(m.wtype, ly.up, H, F, E, y, lid)
        z = np.zeros((1, 1), np.int32)
        sg = cpu(m.sh_type, ly.sh_gate, H, F, 1, y, z)
        su = cpu(m.sh_type, ly.sh_up, H, F, 1, y, z)
        glu = np.vectorize(lambda a, b: O.glu(O.GLU_SWIGLU, float(a), float(b), 0.0), otypes=[np.float32])
        hh = glu(g, u).reshape(1, U, F)
        hs = glu(sg, su).reshape(1, 1, F)
        o = cpu(ly.down_type, ly.down, F, H, E, hh, lid)
        osh = cpu(m.sh_type, ly.sh_down, F, H, 1, hs, z).reshape(1, H)
        x, _ = O.combine_q8_1(o.reshape(1, U, H), w[0, l].reshape(1, U), shared=osh, residual=x)
    err = O.rel_l2(got, x)
    _note(f"  q8_K decode vs ggml-CPU rel_l2={err:.3e}")
    assert err <= 1e-3
