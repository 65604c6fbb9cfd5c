"""GPU parity at the benchmark workloads' own shapes (the other GPU tests use
reduced shapes), through the C ABI, against the CPU oracle:

  * one decode MUL_MAT_ID: 64 experts, Q4_0 [1024 x 2048], batch 1, top-8;
  * one MoE layer of 512 experts, hidden 4096, expert ffn 768, top-8, Q2_K
    gate/up/down with a Q4_K shared expert: the plain GEMVs and the fused
    decode pair, each on its own intermediate bytes;
  * the type x batch sweep on that layer: Q4_0, Q5_0, Q8_0, Q3_K, Q4_K, Q5_K,
    Q6_K at 1, 2, 4 and 8 tokens, per-expert bias and scale fused;
  * the 512-token prefill over 512 Q4_K experts (expert-grouped int8 MFMA);
  * the 48-layer decode step (Q2_K routed + Q4_K shared, every layer resident);
  * the pointer-table cache at the layer shape: 435 of 512 slots seeded from a
    seed file, Zipf(1.1) routing, recorder and LRU state against the cache model.

Expert tensors of 512 experts are random valid blocks on the GPU, with the
experts a test routes to (and the shared experts) replaced by N(0, 0.02)
weights quantized by the oracle where the workload says so; the oracle reads
the GPU's own bytes of every expert it needs.
"""
import ctypes as C
from importlib import import_module

import numpy as np
import pytest

import cache_scenario as S
import helpers as H

pytestmark = pytest.mark.gpu

E512, HID, FFN, TOPK = 512, 4096, 768, 8


def _note(msg):
    print(msg, flush=True)


def _md():
    return import_module("a6000_custom_kernels_amd.moe_decode")


def _softmax(rng, n_tok, k):
    z = rng.standard_normal((n_tok, k)).astype(np.float32)
    w = np.exp(z - z.max(-1, keepdims=True))
    return (w / w.sum(-1, keepdims=True)).astype(np.float32)


def _tensor_with(torch, md, wtype, E, R, K, seed, fill=None):
    """Random valid blocks [E, R, row_bytes] on the GPU; fill: {expert: uint8 [R, row_bytes]} replaces those experts."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    w = md.random_expert_tensor(torch, wtype, E, R, K, gen)
    for e, q in (fill or {}).items():
        w[e].copy_(torch.from_numpy(q))
    return w


def _normal_experts(wtype, experts, R, K, seed):
    """N(0, 0.02) weights quantized by the oracle, one [R, row_bytes] array per expert."""
    return {int(e): H.weights(wtype, 1, R, K, seed=seed * 7919 + int(e))[0] for e in experts}


def _sub(torch, w, ids, *per_expert):
    """The GPU bytes of the experts ids reference, with ids renumbered into that subset (-1 stays -1);
    per-expert arrays (bias [E, R], scale [E]) are cut the same way."""
    uniq = np.unique(ids[ids >= 0])
    remap = np.full(w.shape[0], -1, np.int64)
    remap[uniq] = np.arange(len(uniq))
    rid = np.where(ids >= 0, remap[np.maximum(ids, 0)], -1).astype(np.int32)
    sub = w[torch.from_numpy(uniq.astype(np.int64)).cuda()].cpu().numpy()
    return (sub, rid) + tuple(a[uniq] for a in per_expert)


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ---------------------------------------------------------------------------
# one decode MUL_MAT_ID: 64 experts, Q4_0 [1024 x 2048], batch 1, top-8
# ---------------------------------------------------------------------------

def test_decode_q4_0_64_experts_1024x2048_top8(torch_gpu, mc, O):
    torch = torch_gpu
    E, R, K, U = 64, 1024, 2048, 8
    _note(f"decode MUL_MAT_ID Q4_0 {E} x [{R} x {K}] top-{U} B=1")
    w = H.weights(O.Q4_0, E, R, K, seed=11)                       # N(0, 0.02), quantized by the oracle
    x = H.activations(1, K, seed=12)
    ids = H.routing(1, U, E, seed=13)
    wd, xd, idd = _dev(torch, w), _dev(torch, x), _dev(torch, ids)
    yq = mc.quantize_q8_1(xd)
    dst = torch.zeros((1, U, R), dtype=torch.float32, device="cuda")
    mc.mul_mat_vec(wtype=mc.Q4_0, weights=wd, ids=idd, y=yq.view(1, 1, -1), dst=dst, K=K, R=R, n_experts=E)
    # the op-level entry (src1 fp32, quantized inside) on the same tensors
    dst_op = torch.zeros_like(dst)
    mc.mul_mat_id(wtype=mc.Q4_0, weights=wd, x=xd.view(1, 1, K), ids=idd, dst=dst_op, K=K, R=R, n_experts=E)
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    assert np.array_equal(yq.cpu().numpy()[0], O.quantize_q8_1(x[0]))
    want = O.mul_mat_id(wtype=O.Q4_0, K=K, R=R, n_as=E, src0=w, ids=ids, act=yq.cpu().numpy().reshape(1, 1, -1),
                        act_kind=O.ACT_Q8_1)
    e_same = O.rel_l2(got, want)
    e_cpu = O.rel_l2(got, O.cpu_mul_mat_id_f32(wtype=O.Q4_0, K=K, R=R, n_as=E, src0=w, src1=x, ids=ids))
    _note(f"  rel_l2 vs oracle {e_same:.2e}, vs ggml-CPU {e_cpu:.2e}")
    assert e_same <= H.TOL_SAME and e_cpu <= H.TOL_SAME       # Q4_0: q8_1 codes equal ggml-CPU's q8_0 codes
    assert torch.equal(dst_op, dst)


# ---------------------------------------------------------------------------
# one 512-expert layer: Q2_K gate/up/down, Q4_K shared expert, SwiGLU, top-8
# ---------------------------------------------------------------------------

class Layer512:
    def __init__(self, torch, O, seed, n_tok=1):
        md = _md()
        rng = np.random.default_rng(seed)
        self.ids = np.stack([rng.choice(E512, TOPK, replace=False) for _ in range(n_tok)]).astype(np.int32)
        self.w = _softmax(rng, n_tok, TOPK)
        self.x = rng.standard_normal((n_tok, HID)).astype(np.float32)
        used = np.unique(self.ids)
        self.gate = _tensor_with(torch, md, O.Q2_K, E512, FFN, HID, seed + 1, _normal_experts(O.Q2_K, used, FFN, HID, seed + 1))
        self.up = _tensor_with(torch, md, O.Q2_K, E512, FFN, HID, seed + 2, _normal_experts(O.Q2_K, used, FFN, HID, seed + 2))
        self.down = _tensor_with(torch, md, O.Q2_K, E512, HID, FFN, seed + 3, _normal_experts(O.Q2_K, used, HID, FFN, seed + 3))
        self.sh = {k: H.weights(O.Q4_K, 1, r, c, seed=seed + 10 + i)[0]
                   for i, (k, r, c) in enumerate((("gate", FFN, HID), ("up", FFN, HID), ("down", HID, FFN)))}
        self.sh_dev = {k: _dev(torch, v) for k, v in self.sh.items()}


def test_layer_512_experts_q2K_plain_gemvs(torch_gpu, mc, O):
    """gate/up GEMV (SwiGLU + shared expert) -> q8_1 of the GLU rows -> down GEMV (+ shared), each stage
    against the oracle on the GPU's own input bytes, and against ggml-CPU in q8_K mode."""
    torch = torch_gpu
    _note("512-expert layer Q2_K + Q4_K shared, plain GEMVs")
    L = Layer512(torch, O, seed=100)
    U, n_tok = TOPK, 1
    xd, idd = _dev(torch, L.x), _dev(torch, L.ids)
    y = mc.quantize_q8_1(xd)
    h = torch.zeros((n_tok, U, FFN), dtype=torch.float32, device="cuda")
    h_sh = torch.zeros((n_tok, FFN), dtype=torch.float32, device="cuda")
    f = mc.make_fusion(gate=L.gate, glu_op=mc.GLU_SWIGLU, shared_up=L.sh_dev["up"], shared_gate=L.sh_dev["gate"],
                       shared_dst=h_sh, shared_type=mc.Q4_K)
    mc.mul_mat_vec(wtype=mc.Q2_K, weights=L.up, ids=idd, y=y.view(n_tok, 1, -1), dst=h, K=HID, R=FFN, n_experts=E512,
                   fusion=f)
    hq = mc.quantize_q8_1(h.view(n_tok * U, FFN)).view(n_tok, U, -1)
    hq_sh = mc.quantize_q8_1(h_sh)
    o = torch.zeros((n_tok, U, HID), dtype=torch.float32, device="cuda")
    o_sh = torch.zeros((n_tok, HID), dtype=torch.float32, device="cuda")
    fd = mc.make_fusion(shared_up=L.sh_dev["down"], shared_dst=o_sh, shared_type=mc.Q4_K, shared_src1=hq_sh,
                        shared_stride_col_y=FFN // 32)
    mc.mul_mat_vec(wtype=mc.Q2_K, weights=L.down, ids=idd, y=hq, dst=o, K=FFN, R=HID, n_experts=E512, fusion=fd,
                   nchannels_y=U)
    torch.cuda.synchronize()
    gsub, rid = _sub(torch, L.gate, L.ids)
    usub, _ = _sub(torch, L.up, L.ids)
    dsub, _ = _sub(torch, L.down, L.ids)
    yb = y.cpu().numpy().reshape(n_tok, 1, -1)
    want_h, want_hsh = O.mul_mat_id(wtype=O.Q2_K, K=HID, R=FFN, n_as=len(usub), src0=usub, gate=gsub, ids=rid, act=yb,
                                    act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU, sh_type=O.Q4_K, sh_up=L.sh["up"],
                                    sh_gate=L.sh["gate"])
    e1, e2 = O.rel_l2(h.cpu().numpy(), want_h), O.rel_l2(h_sh.cpu().numpy(), want_hsh)
    want_o, want_osh = O.mul_mat_id(wtype=O.Q2_K, K=FFN, R=HID, n_as=len(dsub), src0=dsub, ids=rid,
                                    act=hq.cpu().numpy(), act_kind=O.ACT_Q8_1, nchannels_y=U, sh_type=O.Q4_K,
                                    sh_up=L.sh["down"], sh_act=hq_sh.cpu().numpy())
    e3, e4 = O.rel_l2(o.cpu().numpy(), want_o), O.rel_l2(o_sh.cpu().numpy(), want_osh)
    _note(f"  gate/up {e1:.2e} shared {e2:.2e}; down {e3:.2e} shared {e4:.2e}")
    assert max(e1, e2, e3, e4) <= H.TOL_SAME
    # q8_K activations (ggml-CPU's vec_dot_type) vs the ggml-CPU restatement of the up projection
    yk = mc.quantize_q8_K(xd)
    up_k = torch.zeros((n_tok, U, FFN), dtype=torch.float32, device="cuda")
    mc.mul_mat_vec(wtype=mc.Q2_K, weights=L.up, ids=idd, y=yk.view(n_tok, 1, -1), dst=up_k, K=HID, R=FFN,
                   n_experts=E512, act=mc.ACT_Q8_K)
    torch.cuda.synchronize()
    want_cpu = O.cpu_mul_mat_id_f32(wtype=O.Q2_K, K=HID, R=FFN, n_as=len(usub), src0=usub, src1=L.x, ids=rid)
    e5 = O.rel_l2(up_k.cpu().numpy(), want_cpu)
    _note(f"  q8_K mode vs ggml-CPU {e5:.2e}")
    assert e5 <= H.TOL_CPU


def test_layer_512_experts_q2K_fused_pair(torch_gpu, mc, O):
    """The two-launch decode block at the layer shape: gate/up with the RMSNorm + q8_1 prologue (checked on
    its own normalized row y_out), then down + weighted combine (checked on its own q8_1 GLU rows)."""
    torch = torch_gpu
    _note("512-expert layer Q2_K + Q4_K shared, fused decode pair")
    L = Layer512(torch, O, seed=200)
    U, n_tok, eps = TOPK, 1, 1e-6
    rng = np.random.default_rng(201)
    nw = rng.uniform(0.5, 1.5, HID).astype(np.float32)
    xd, idd, nwd, wd = _dev(torch, L.x), _dev(torch, L.ids), _dev(torch, nw), _dev(torch, L.w)
    h = torch.zeros((n_tok, U, FFN), dtype=torch.float32, device="cuda")
    h_sh = torch.zeros((n_tok, FFN), dtype=torch.float32, device="cuda")
    y_out = torch.zeros((n_tok, HID // 32 * 36), dtype=torch.uint8, device="cuda")
    hq = torch.zeros((n_tok, U, FFN // 32 * 36), dtype=torch.uint8, device="cuda")
    hq_sh = torch.zeros((n_tok, FFN // 32 * 36), dtype=torch.uint8, device="cuda")
    f = mc.make_fusion(gate=L.gate, glu_op=mc.GLU_SWIGLU, shared_up=L.sh_dev["up"], shared_gate=L.sh_dev["gate"],
                       shared_dst=h_sh, shared_type=mc.Q4_K)
    mc.ffn_gate_up_norm(wtype=mc.Q2_K, weights=L.up, ids=idd, x=xd, dst=h, K=HID, R=FFN, n_experts=E512,
                        norm_weight=nwd, eps=eps, fusion=f, y_out=y_out, dst_q8_1=hq, shared_dst_q8_1=hq_sh)
    x_out = torch.zeros((n_tok, HID), dtype=torch.float32, device="cuda")
    fd = mc.make_fusion(shared_up=L.sh_dev["down"], shared_type=mc.Q4_K, shared_src1=hq_sh,
                        shared_stride_col_y=FFN // 32)
    mc.ffn_down_combine(wtype=mc.Q2_K, weights=L.down, ids=idd, h=hq, router_w=wd, x_out=x_out, K=FFN, R=HID,
                        n_experts=E512, act=mc.ACT_Q8_1, fusion=fd)
    assert mc.check_status() == 0
    torch.cuda.synchronize()
    # the prologue's row equals the combine kernel's RMSNorm + q8_1 (oracle restatement, bit-exact)
    _, y_ref = O.combine_q8_1(np.zeros((n_tok, 0, HID), np.float32), np.zeros((n_tok, 0), np.float32),
                              residual=L.x, rms_norm=True, norm_weight=nw, eps=eps)
    assert np.array_equal(y_out.cpu().numpy(), y_ref)
    gsub, rid = _sub(torch, L.gate, L.ids)
    usub, _ = _sub(torch, L.up, L.ids)
    dsub, _ = _sub(torch, L.down, L.ids)
    want_h, want_hsh = O.mul_mat_id(wtype=O.Q2_K, K=HID, R=FFN, n_as=len(usub), src0=usub, gate=gsub, ids=rid,
                                    act=y_ref.reshape(n_tok, 1, -1), act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU,
                                    sh_type=O.Q4_K, sh_up=L.sh["up"], sh_gate=L.sh["gate"])
    hg, hshg = h.cpu().numpy(), h_sh.cpu().numpy()
    e1, e2 = O.rel_l2(hg, want_h), O.rel_l2(hshg, want_hsh)
    # the q8_1 copies are the quantizer's bytes of the fp32 outputs
    assert np.array_equal(hq.cpu().numpy().reshape(U, -1), np.stack([O.quantize_q8_1(r) for r in hg[0]]))
    assert np.array_equal(hq_sh.cpu().numpy()[0], O.quantize_q8_1(hshg[0]))
    o, o_sh = O.mul_mat_id(wtype=O.Q2_K, K=FFN, R=HID, n_as=len(dsub), src0=dsub, ids=rid, act=hq.cpu().numpy(),
                           act_kind=O.ACT_Q8_1, nchannels_y=U, sh_type=O.Q4_K, sh_up=L.sh["down"],
                           sh_act=hq_sh.cpu().numpy())
    want_x, _ = O.combine_q8_1(o, L.w, shared=o_sh)
    e3 = O.rel_l2(x_out.cpu().numpy(), want_x)
    _note(f"  gate/up {e1:.2e} shared {e2:.2e}; down+combine {e3:.2e}")
    assert max(e1, e2, e3) <= H.TOL_SAME


# ---------------------------------------------------------------------------
# type x batch sweep on the 512-expert layer, bias + scale fused
# ---------------------------------------------------------------------------

@pytest.mark.timeout(300)
@pytest.mark.parametrize("tname", ["Q4_0", "Q5_0", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_layer_512_experts_type_batch_sweep(torch_gpu, mc, O, tname):
    torch = torch_gpu
    md = _md()
    t = getattr(mc, tname)
    _note(f"512-expert layer {tname}: B in 1, 2, 4, 8 with bias + scale")
    seed = 300 + t
    gate = _tensor_with(torch, md, t, E512, FFN, HID, seed + 1)
    up = _tensor_with(torch, md, t, E512, FFN, HID, seed + 2)
    down = _tensor_with(torch, md, t, E512, HID, FFN, seed + 3)
    rng = np.random.default_rng(seed)
    xb = (rng.standard_normal((E512, FFN)) * 0.1).astype(np.float32)
    gb = (rng.standard_normal((E512, FFN)) * 0.1).astype(np.float32)
    db = (rng.standard_normal((E512, HID)) * 0.1).astype(np.float32)
    xs = rng.uniform(0.5, 1.5, E512).astype(np.float32)
    gs = rng.uniform(0.5, 1.5, E512).astype(np.float32)
    ds = rng.uniform(0.5, 1.5, E512).astype(np.float32)
    dv = {k: _dev(torch, v) for k, v in dict(xb=xb, gb=gb, db=db, xs=xs, gs=gs, ds=ds).items()}
    for B in (1, 2, 4, 8):
        ids = np.stack([rng.choice(E512, TOPK, replace=False) for _ in range(B)]).astype(np.int32)
        x = rng.standard_normal((B, HID)).astype(np.float32)
        idd = _dev(torch, ids)
        y = mc.quantize_q8_1(_dev(torch, x))
        h = torch.zeros((B, TOPK, FFN), dtype=torch.float32, device="cuda")
        f = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, x_bias=dv["xb"], gate_bias=dv["gb"], x_scale=dv["xs"],
                           gate_scale=dv["gs"])
        mc.mul_mat_vec(wtype=t, weights=up, ids=idd, y=y.view(B, 1, -1), dst=h, K=HID, R=FFN, n_experts=E512, fusion=f)
        hq = mc.quantize_q8_1(h.view(B * TOPK, FFN)).view(B, TOPK, -1)
        o = torch.zeros((B, TOPK, HID), dtype=torch.float32, device="cuda")
        fd = mc.make_fusion(x_bias=dv["db"], x_scale=dv["ds"])
        mc.mul_mat_vec(wtype=t, weights=down, ids=idd, y=hq, dst=o, K=FFN, R=HID, n_experts=E512, fusion=fd,
                       nchannels_y=TOPK)
        torch.cuda.synchronize()
        gsub, rid, xb_s, gb_s, xs_s, gs_s = _sub(torch, gate, ids, xb, gb, xs, gs)
        usub, _ = _sub(torch, up, ids)
        dsub, _, db_s, ds_s = _sub(torch, down, ids, db, ds)
        want_h = O.mul_mat_id(wtype=t, K=HID, R=FFN, n_as=len(usub), src0=usub, gate=gsub, ids=rid,
                              act=y.cpu().numpy().reshape(B, 1, -1), act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU,
                              x_bias=xb_s, gate_bias=gb_s, x_scale=xs_s, gate_scale=gs_s)
        want_o = O.mul_mat_id(wtype=t, K=FFN, R=HID, n_as=len(dsub), src0=dsub, ids=rid, act=hq.cpu().numpy(),
                              act_kind=O.ACT_Q8_1, nchannels_y=TOPK, x_bias=db_s, x_scale=ds_s)
        e1, e2 = O.rel_l2(h.cpu().numpy(), want_h), O.rel_l2(o.cpu().numpy(), want_o)
        _note(f"  B={B} unique experts {len(usub)}: gate/up {e1:.2e} down {e2:.2e}")
        assert e1 <= H.TOL_SAME and e2 <= H.TOL_SAME


# ---------------------------------------------------------------------------
# prefill: 512 tokens x top-8 over 512 Q4_K experts, expert-grouped int8 MFMA
# ---------------------------------------------------------------------------

def test_prefill_512_tokens_q4K_512_experts(torch_gpu, mc, O):
    """Every pair of 16 sampled experts (about 128 of the 4,096 pairs) is checked: gate/up + SwiGLU against the
    oracle on the GPU's own q8_K rows, the down projection against the ggml-CPU restatement on the fp32 GLU
    rows.  The other pairs run as well (the GEMM sees the full routing)."""
    torch = torch_gpu
    md = _md()
    n_tok, E, U = 512, E512, TOPK
    _note(f"prefill {n_tok} tokens x top-{U} over {E} Q4_K experts")
    rng = np.random.default_rng(500)
    ids = np.stack([rng.choice(E, U, replace=False) for _ in range(n_tok)]).astype(np.int32)
    sample = rng.choice(np.unique(ids), 16, replace=False)
    gate = _tensor_with(torch, md, mc.Q4_K, E, FFN, HID, 501, _normal_experts(mc.Q4_K, sample, FFN, HID, 501))
    up = _tensor_with(torch, md, mc.Q4_K, E, FFN, HID, 502, _normal_experts(mc.Q4_K, sample, FFN, HID, 502))
    down = _tensor_with(torch, md, mc.Q4_K, E, HID, FFN, 503, _normal_experts(mc.Q4_K, sample, HID, FFN, 503))
    x = rng.standard_normal((n_tok, HID)).astype(np.float32)
    idd = _dev(torch, ids)
    yk = mc.quantize_q8_K(_dev(torch, x))
    h = torch.zeros((n_tok, U, FFN), dtype=torch.float32, device="cuda")
    mc.mul_mat_q(wtype=mc.Q4_K, weights=up, ids=idd, y=yk.view(n_tok, 1, -1), dst=h, K=HID, R=FFN, n_experts=E,
                 gate=gate, glu_op=mc.GLU_SWIGLU)
    hk = mc.quantize_q8_K(h.view(n_tok * U, FFN)).view(n_tok, U, -1)
    o = torch.zeros((n_tok, U, HID), dtype=torch.float32, device="cuda")
    mc.mul_mat_q(wtype=mc.Q4_K, weights=down, ids=idd, y=hk, dst=o, K=FFN, R=HID, n_experts=E, nchannels_y=U)
    torch.cuda.synchronize()
    sel = np.isin(ids, sample)
    ids_s = np.where(sel, ids, -1).astype(np.int32)
    gsub, rid = _sub(torch, gate, ids_s)
    usub, _ = _sub(torch, up, ids_s)
    dsub, _ = _sub(torch, down, ids_s)
    want_h = O.mul_mat_id(wtype=O.Q4_K, K=HID, R=FFN, n_as=len(usub), src0=usub, gate=gsub, ids=rid,
                          act=yk.cpu().numpy().reshape(n_tok, 1, -1), act_kind=O.ACT_CPU, glu_op=O.GLU_SWIGLU)
    hg = h.cpu().numpy()
    e1 = O.rel_l2(hg[sel], want_h[sel])
    want_o = O.cpu_mul_mat_id_f32(wtype=O.Q4_K, K=FFN, R=HID, n_as=len(dsub), src0=dsub, src1=hg, ids=rid)
    e2 = O.rel_l2(o.cpu().numpy()[sel], want_o[sel])
    _note(f"  {int(sel.sum())} pairs of 16 experts: gate/up {e1:.2e}, down vs ggml-CPU {e2:.2e}")
    assert e1 <= H.TOL_SAME and e2 <= H.TOL_SAME
    assert bool(torch.isfinite(h).all()) and bool(torch.isfinite(o).all())


# ---------------------------------------------------------------------------
# 48-layer decode step, every layer resident
# ---------------------------------------------------------------------------

@pytest.mark.timeout(600)
def test_decode_48_layers_q2K(torch_gpu, mc, O):
    """The benchmark's decode model: two tokens through 48 layers with the fused plan equal the op-by-op plan
    bit for bit, graph replay equals eager, outputs stay finite, and layer 0 of the fused plan matches the
    oracle on its own intermediate bytes."""
    torch = torch_gpu
    md = _md()
    L = 48
    _note(f"decode {L} layers Q2_K + Q4_K shared (allocating ~71 GiB)")
    model = md.MoeDecodeModel(torch, n_layers=L, fused=True)
    ids_np, w_np = md.make_routing(2, L, model.E, model.U, seed=21)
    x0 = torch.from_numpy(np.random.default_rng(22).standard_normal((1, model.H)).astype(np.float32)).cuda()

    def run(fused, graph=False):
        model.fused = fused
        model.x.copy_(x0)
        outs = []
        if graph:
            model.set_routing(_dev(torch, ids_np[0]), _dev(torch, w_np[0]))
            model.capture()
            model.x.copy_(x0)
        for t in range(2):
            model.set_routing(_dev(torch, ids_np[t]), _dev(torch, w_np[t]))
            if graph:
                model.replay()
            else:
                model.launch_token()
            torch.cuda.synchronize()
            outs.append(model.x.clone())
        return outs

    fused = run(True)
    ops = run(False)
    replay = run(True, graph=True)
    assert mc.check_status() == 0
    for t in range(2):
        assert bool(torch.isfinite(fused[t]).all())
        assert torch.equal(fused[t], ops[t]), f"token {t}: fused plan != op-by-op plan"
        assert torch.equal(fused[t], replay[t]), f"token {t}: graph replay != eager"
    _note("  fused == ops == replay for 2 tokens")
    # layer 0 of the fused plan against the oracle on its own bytes
    model.fused = True
    model.x.copy_(x0)
    model.set_routing(_dev(torch, ids_np[0]), _dev(torch, w_np[0]))
    y_out = torch.zeros((1, model.H // 32 * 36), dtype=torch.uint8, device="cuda")
    ly = model.layers[0]
    U, F, Hd = model.U, model.F, model.H
    f = mc.make_fusion(gate=ly.gate, glu_op=mc.GLU_SWIGLU, shared_up=ly.sh_up, shared_gate=ly.sh_gate,
                       shared_dst=model.h[U:], shared_type=mc.Q4_K)
    mc.ffn_gate_up_norm(wtype=mc.Q2_K, weights=ly.up, ids=model.ids[0], x=model.x, dst=model.h[:U].view(1, U, F),
                        K=Hd, R=F, n_experts=model.E, norm_weight=model.norm[0], eps=model.eps, fusion=f, y_out=y_out,
                        dst_q8_1=model.hq[:U].view(1, U, -1), shared_dst_q8_1=model.hq[U:])
    model.residual = False                # x_next = shared + sum_j w_j o_j alone: the MoE terms are what is checked
    model.launch_down_combine(0, model.x, model.x_next)
    model.residual = True
    torch.cuda.synchronize()
    ids0 = ids_np[0, 0].reshape(1, U)
    gsub, rid = _sub(torch, ly.gate, ids0)
    usub, _ = _sub(torch, ly.up, ids0)
    dsub, _ = _sub(torch, ly.down, ids0)
    sh = {k: getattr(ly, k).cpu().numpy() for k in ("sh_gate", "sh_up", "sh_down")}
    want_h, want_hsh = O.mul_mat_id(wtype=O.Q2_K, K=Hd, R=F, n_as=len(usub), src0=usub, gate=gsub, ids=rid,
                                    act=y_out.cpu().numpy().reshape(1, 1, -1), act_kind=O.ACT_Q8_1,
                                    glu_op=O.GLU_SWIGLU, sh_type=O.Q4_K, sh_up=sh["sh_up"], sh_gate=sh["sh_gate"])
    e1 = O.rel_l2(model.h[:U].cpu().numpy()[None], want_h)
    e2 = O.rel_l2(model.h[U:].cpu().numpy(), want_hsh)
    hq = model.hq.cpu().numpy()
    o, o_sh = O.mul_mat_id(wtype=O.Q2_K, K=F, R=Hd, n_as=len(dsub), src0=dsub, ids=rid, act=hq[:U][None],
                           act_kind=O.ACT_Q8_1, nchannels_y=U, sh_type=O.Q4_K, sh_up=sh["sh_down"], sh_act=hq[U:])
    want_x, _ = O.combine_q8_1(o, w_np[0, 0].reshape(1, U), shared=o_sh)
    e3 = O.rel_l2(model.x_next.cpu().numpy(), want_x)
    _note(f"  layer 0: gate/up {e1:.2e} shared {e2:.2e}, down+combine {e3:.2e}")
    assert max(e1, e2, e3) <= H.TOL_SAME
    del model
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# pointer-table cache at the layer shape
# ---------------------------------------------------------------------------

@pytest.mark.timeout(600)
def test_cache_layer_shape_zipf_435_slots(torch_gpu, mc, O, tmp_path):
    """4 layers of Q2_K gate/up/down (512 experts each) in pinned host memory, a pool of 435 slots per tensor
    seeded from a seed file (the head of a per-layer permutation), Gumbel-top-8 Zipf(1.1) routing over that
    permutation, 64 tokens with the cache step between them.  After every token: the stats words (counts and
    miss log), the stamps, and after every step the slot maps and tables equal the cache model's.  The
    layer-0 outputs of the first and last token equal the resident path's."""
    from oracle.cache_model import CacheModel, parse_seed_file
    torch = torch_gpu
    md = _md()
    layers, n_tok, POOL, U = 4, 64, 435, TOPK
    t = mc.Q2_K
    eb = mc.row_bytes(t, HID) * FFN
    _note(f"cache at the layer shape: {layers} layers x 3 tensors, {POOL}/{E512} slots, {n_tok} tokens")
    rng = np.random.default_rng(600)
    perms = [rng.permutation(E512) for _ in range(layers)]
    seed_path = tmp_path / "moe_seed.txt"
    with open(seed_path, "w") as fh:
        for l in range(layers):
            head = ",".join(str(int(e)) for e in perms[l][:POOL])
            for role in ("gate", "up", "down"):
                fh.write(f"blk.{l}.ffn_{role}_exps.weight {head}\n")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(601)
    keep, host, tens = [], {}, {}
    for l in range(layers):
        for role, rows, k in (("gate", FFN, HID), ("up", FFN, HID), ("down", HID, FFN)):
            dev = md.random_expert_tensor(torch, t, E512, rows, k, gen)
            p = torch.empty(E512 * eb, dtype=torch.uint8, pin_memory=True)
            p.copy_(dev.view(-1))
            if l == 0:
                host[role] = dev                       # resident copy for the output check
            else:
                del dev
            keep.append(p)
            tens[(l, role)] = mc.make_tensor(t, k, rows, E512, p.data_ptr(), name=f"blk.{l}.ffn_{role}_exps.weight",
                                             keep=keep)
    torch.cuda.synchronize()
    logp = -1.1 * np.log(np.arange(1, E512 + 1))
    routes = np.empty((n_tok, layers, U), np.int32)
    for i in range(n_tok):
        for l in range(layers):
            routes[i, l] = perms[l][np.argpartition(-(logp + rng.gumbel(size=E512)), U)[:U]]
    lib = mc.lib()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    mc.reset()
    mc.configure(enabled=True, slots=POOL, budget_gb=0.0, margin_gb=2.0, seed_path=str(seed_path), max_promotions=48)
    free_b = torch.cuda.mem_get_info()[0]
    model = CacheModel(slots=POOL, budget_bytes=0, margin_bytes=2 << 30, max_promotions=48,
                       seed=parse_seed_file(seed_path))
    x = torch.from_numpy(rng.standard_normal((1, HID)).astype(np.float32)).cuda()
    y = mc.quantize_q8_1(x)
    h = torch.zeros((1, U, FFN), dtype=torch.float32, device="cuda")
    o = torch.zeros((1, U, HID), dtype=torch.float32, device="cuda")
    ids_dev = torch.zeros((layers, 1, U), dtype=torch.int32, device="cuda")
    ar = HID // 32
    ents = {}
    for i in range(n_tok):
        ids_dev.copy_(torch.from_numpy(routes[i][:, None, :]))
        for l in range(layers):
            mc.check(lib.ggml_hip_moe_cache_mul_mat_vec_q(
                C.byref(tens[(l, "up")]), C.byref(tens[(l, "gate")]), None, y.data_ptr(), ids_dev[l].data_ptr(),
                h.data_ptr(), HID, FFN, E512, 1, 1, HID // 256, eb, eb * E512, 1, U, ar, U * FFN, ar, FFN, U, stream),
                "gate/up")
            if l == 0 and i in (0, n_tok - 1):
                torch.cuda.synchronize()
                ref = torch.zeros_like(h)
                mc.mul_mat_vec(wtype=t, weights=host["up"], ids=ids_dev[0], y=y.view(1, 1, -1), dst=ref, K=HID, R=FFN,
                               n_experts=E512, fusion=mc.make_fusion(gate=host["gate"], glu_op=mc.GLU_SWIGLU))
                torch.cuda.synchronize()
                assert torch.equal(h, ref), f"token {i}: cache gate/up != resident"
            mc.check(lib.ggml_hip_moe_mul_mat_vec_ex(
                1, mc.ACT_F32, C.byref(tens[(l, "down")]), None, None, h.data_ptr(), ids_dev[l].data_ptr(),
                o.data_ptr(), FFN, HID, E512, 1, U, U, U * FFN, U * HID, FFN, HID, U, stream), "down")
            if i == 0:
                for role in ("up", "gate", "down"):
                    ents[(l, role)] = model.register(tens[(l, role)].data, tens[(l, role)].name.decode(), E512, eb,
                                                     free_b)
            model.record(ents[(l, "up")], ents[(l, "gate")], routes[i, l][None].tolist())
            model.record(ents[(l, "down")], None, routes[i, l][None].tolist())
        S.check_recorder(lib, stream, model, f"token {i} recorder")
        if i == 0:
            S.compare_state(mc, lib, model, "after registration")
        assert lib.ggml_hip_moe_cache_step(stream) == 0, lib.ggml_hip_moe_last_error()
        model.step()
        S.compare_state(mc, lib, model, f"token {i} after step")
    tot = mc.totals()
    hit_rate = tot.hits / max(tot.hits + tot.misses, 1)
    _note(f"  hits {tot.hits} misses {tot.misses} (hit rate {hit_rate:.4f}), promotions {tot.promotions}, "
          f"evictions {tot.evictions}")
    assert tot.promotions == model.promotions and tot.evictions == model.evictions
    assert 0.9 < hit_rate < 1.0
    torch.cuda.synchronize()
    mc.reset()
