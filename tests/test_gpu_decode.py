"""GPU: the synthetic MoE decode step (the benchmark's workload), stage by stage
against the CPU oracle on the GPU's own intermediate bytes, and graph replay
against eager launches."""
from importlib import import_module

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_model(torch_gpu, mc):
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    torch = torch_gpu
    m = md.MoeDecodeModel(torch, n_layers=3, n_experts=16, hidden=1024, ffn=512, n_used=4, seed=5)
    ids, w = md.make_routing(4, m.L, m.E, m.U, seed=11)
    return md, m, ids, w


def test_decode_layer_stagewise(torch_gpu, mc, O, small_model):
    torch = torch_gpu
    md, m, ids, w = small_model
    H, F, U, E = m.H, m.F, m.U, m.E
    x0 = np.random.default_rng(2).standard_normal((1, H)).astype(np.float32)
    m.x.copy_(torch.from_numpy(x0))
    m.set_routing(torch.from_numpy(ids[0]), torch.from_numpy(w[0]))
    mc.quantize_q8_1(m.x, out=m.y)
    ly = m.layers[0]
    g, u, d = ly.gate.cpu().numpy(), ly.up.cpu().numpy(), ly.down.cpu().numpy()
    sg, su, sd = ly.sh_gate.cpu().numpy(), ly.sh_up.cpu().numpy(), ly.sh_down.cpu().numpy()
    lid = ids[0, 0].reshape(1, U)

    y = m.y.cpu().numpy()
    assert np.array_equal(y[0], O.quantize_q8_1(x0[0]))
    m.launch_gate_up(0)
    torch.cuda.synchronize()
    h = m.h.cpu().numpy()
    want_h, want_hs = O.mul_mat_id(wtype=m.wtype, K=H, R=F, n_as=E, src0=u, gate=g, ids=lid, act=y.reshape(1, 1, -1),
                                   act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU, sh_type=m.sh_type, sh_up=su, sh_gate=sg)
    assert O.rel_l2(h[:U], want_h[0]) <= 1e-5
    assert O.rel_l2(h[U], want_hs[0]) <= 1e-5

    # the down GEMV quantizes the fp32 GLU rows itself: its input is q8_1 of the GPU's h bytes
    hq = np.stack([O.quantize_q8_1(r) for r in h])

    m.launch_down(0)
    torch.cuda.synchronize()
    o, osh = m.o.cpu().numpy(), m.o_sh.cpu().numpy()
    want_o, want_osh = O.mul_mat_id(wtype=m.wtype, K=F, R=H, n_as=E, src0=d, ids=lid, act=hq[:U].reshape(1, U, -1),
                                    act_kind=O.ACT_Q8_1, nchannels_y=U, sh_type=m.sh_type, sh_up=sd,
                                    sh_act=hq[U:].reshape(1, -1))
    assert O.rel_l2(o, want_o[0]) <= 1e-5
    assert O.rel_l2(osh, want_osh) <= 1e-5

    nw = m.norm[1]
    for norm, weight in ((False, None), (True, None), (True, nw)):
        m.x_next.zero_()
        m.y.zero_()
        mc.combine_q8_1(m.o.view(1, U, H), m.w[0], shared=m.o_sh, residual=m.x, x_out=m.x_next, y=m.y,
                        rms_norm=norm, norm_weight=weight, eps=1e-6)
        torch.cuda.synchronize()
        wx, wy = O.combine_q8_1(o.reshape(1, U, H), w[0, 0].reshape(1, U), shared=osh, residual=x0, rms_norm=norm,
                                norm_weight=None if weight is None else weight.cpu().numpy(), eps=1e-6)
        assert np.array_equal(m.x_next.cpu().numpy(), wx)
        assert np.array_equal(m.y.cpu().numpy(), wy), (norm, weight is not None)


def test_decode_graph_replay_matches_eager(torch_gpu, mc, small_model):
    torch = torch_gpu
    md, m, ids, w = small_model
    x0 = torch.from_numpy(np.random.default_rng(4).standard_normal((1, m.H)).astype(np.float32)).cuda()
    ids_d, w_d = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    eager = []
    m.x.copy_(x0)
    for t in range(3):
        m.set_routing(ids_d[t], w_d[t])
        m.launch_token()
        torch.cuda.synchronize()
        eager.append(m.x.clone())
    assert all(bool(torch.isfinite(e).all()) for e in eager)
    m.x.copy_(x0)
    m.set_routing(ids_d[0], w_d[0])
    m.capture()                               # runs one eager token first, then captures
    m.x.copy_(x0)
    for t in range(3):
        m.set_routing(ids_d[t], w_d[t])
        m.replay()
        torch.cuda.synchronize()              # eager host work between replays
        assert torch.equal(m.x, eager[t]), f"replay {t} differs from eager"
