"""GPU: pointer-table cache path -- pinned host experts (LSB=1, zero-copy PCIe
reads), HBM pool slots (LSB=0), device recorder and the LRU step, all checked
against oracle/cache_model.py; outputs checked against the resident path and
the CPU oracle."""
import ctypes as C
import sys

import numpy as np
import pytest

import cache_scenario as S
import helpers as H

pytestmark = pytest.mark.gpu


class GpuBackend:
    def __init__(self, torch, mc, O, n_experts, R, K, wtype, seed, gate_mode="cache", shared_bias=False):
        self.torch, self.mc, self.O = torch, mc, O
        self.K, self.R, self.wtype, self.n_experts = K, R, wtype, n_experts
        self.gate_mode, self.shared_bias = gate_mode, shared_bias
        self.w = {"up": H.weights(wtype, n_experts, R, K, seed=seed),
                  "gate": H.weights(wtype, n_experts, R, K, seed=seed + 1)}
        self.stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.keep = []
        if shared_bias:
            rng = np.random.default_rng(seed + 2)
            self.sh_type = 12                                  # Q4_K shared expert
            self.sh_up = H.weights(self.sh_type, 1, R, K, seed=seed + 3)[0]
            self.sh_gate = H.weights(self.sh_type, 1, R, K, seed=seed + 4)[0]
            self.bias = rng.normal(0.0, 0.1, (n_experts, R)).astype(np.float32)

    def host_tensor(self, nbytes, role):
        t = self.torch.empty(nbytes, dtype=self.torch.uint8, pin_memory=True)
        t.numpy()[:] = self.w[role].reshape(-1)
        self.keep.append(t)
        return t.data_ptr(), t

    def device_tensor(self, nbytes, role):
        t = self.torch.from_numpy(self.w[role].reshape(-1)).cuda()
        self.keep.append(t)
        return t.data_ptr(), t

    def fusion_extra(self):
        torch = self.torch
        self.d_bias = torch.from_numpy(self.bias).cuda()
        self.d_sh_up = torch.from_numpy(self.sh_up).cuda()
        self.d_sh_gate = torch.from_numpy(self.sh_gate).cuda()
        self.sh_dst = torch.zeros((8, self.R), dtype=torch.float32, device="cuda")     # up to 8 tokens
        f = {"x_bias": self.d_bias.data_ptr(), "shared_up": self.d_sh_up.data_ptr(), "shared_type": self.sh_type,
             "shared_dst": self.sh_dst.data_ptr(), "shared_stride_col_dst": self.R}
        if self.gate_mode != "none":
            f["shared_gate"] = self.d_sh_gate.data_ptr()
        return f

    def ids_buffer(self, n_tok, n_used):
        self.ids = self.torch.zeros((n_tok, n_used), dtype=self.torch.int32, device="cuda")
        return self.ids.data_ptr(), lambda ids: self.ids.copy_(self.torch.from_numpy(ids))

    def act_buffer(self, n_tok, K):
        self.x = H.activations(n_tok, K, seed=77)
        self.y = self.mc.quantize_q8_1(self.torch.from_numpy(self.x).cuda())
        return self.y.data_ptr()

    def dst_buffer(self, n_tok, n_used, R):
        self.dst = self.torch.zeros((n_tok, n_used, R), dtype=self.torch.float32, device="cuda")
        return self.dst.data_ptr()

    def check_outputs(self, step, ids):
        torch, mc, O = self.torch, self.mc, self.O
        torch.cuda.synchronize()
        got = self.dst.cpu().numpy()
        got_sh = self.sh_dst.cpu().numpy()[:ids.shape[0]] if self.shared_bias else None
        # the same weights resident in device memory, through the no-cache entry point
        ref = torch.zeros_like(self.dst)
        up_d = torch.from_numpy(self.w["up"]).cuda()
        has_gate = self.gate_mode != "none"
        gate_d = torch.from_numpy(self.w["gate"]).cuda() if has_gate else None
        kw = {}
        if self.shared_bias:
            ref_sh = torch.zeros_like(self.sh_dst)
            kw = dict(x_bias=self.d_bias, shared_up=self.d_sh_up, shared_gate=self.d_sh_gate if has_gate else None,
                      shared_dst=ref_sh, shared_type=self.sh_type)
        f = mc.make_fusion(gate=gate_d, glu_op=mc.GLU_SWIGLU, **kw)
        mc.mul_mat_vec(wtype=self.wtype, weights=up_d, ids=self.ids, y=self.y, dst=ref, K=self.K, R=self.R,
                       n_experts=self.n_experts, fusion=f)
        torch.cuda.synchronize()
        assert np.array_equal(got, ref.cpu().numpy()), f"step {step}: cache path != resident path"
        if self.shared_bias:
            assert np.array_equal(got_sh, ref_sh.cpu().numpy()[:ids.shape[0]]), f"step {step}: shared expert differs"
        yb = self.y.cpu().numpy().reshape(ids.shape[0], 1, -1)
        okw = {}
        if self.shared_bias:
            okw = dict(x_bias=self.bias, sh_type=self.sh_type, sh_up=self.sh_up,
                       sh_gate=self.sh_gate if has_gate else None)
        want = O.mul_mat_id(wtype=self.wtype, K=self.K, R=self.R, n_as=self.n_experts, src0=self.w["up"],
                            gate=self.w["gate"] if has_gate else None, ids=ids, act=yb, act_kind=O.ACT_Q8_1,
                            glu_op=O.GLU_SWIGLU, **okw)
        if self.shared_bias:
            want, want_sh = want
            # the shared expert takes no routed bias (the reference's shared row indexes expert 0's bias,
            # kernels/moe-cache.cu:244 with :143)
            assert O.rel_l2(got_sh, want_sh) <= H.TOL_SAME
        assert O.rel_l2(got, want) <= H.TOL_SAME


@pytest.mark.parametrize("wtype,slots,seeded", [(10, 5, True), (14, 3, False), (2, 16, False)])
def test_cache_scenario_gpu(torch_gpu, mc, O, tmp_path, wtype, slots, seeded):
    torch = torch_gpu
    print(f"cache scenario type={wtype} slots={slots} seeded={seeded}", flush=True)
    n_experts, R, K = 16, 40, 4096 if wtype != 2 else 2048
    seed_path = None
    if seeded:
        seed_path = str(tmp_path / "seed.txt")
        with open(seed_path, "w") as f:
            f.write(f"{S.UP_NAME} 3,1,3,99,-2,0,7,8,9\n{S.GATE_NAME} 2,5\nother.weight 1,2\n")
    be = GpuBackend(torch, mc, O, n_experts, R, K, wtype, seed=900 + wtype)
    free_b = torch.cuda.mem_get_info()[0]
    model, keep = S.run_scenario(mc, mc.lib(), be, n_experts=n_experts, R=R, K=K, wtype=wtype, slots=slots,
                                 steps=10, seed_path=seed_path, free_bytes=free_b, check_outputs=be.check_outputs)
    assert model.promotions > 0
    if slots < n_experts:
        assert model.evictions > 0
    torch.cuda.synchronize()
    assert mc.lib().ggml_hip_moe_cache_reset() == 0


@pytest.mark.parametrize("wtype,slots,n_tok", [(10, 5, 2), (12, 3, 3)])
def test_cache_async_promotions_gpu(torch_gpu, mc, O, wtype, slots, n_tok):
    """Promotion copies on the library's second stream: outputs against the resident path and the
    oracle every step; with a device-wide synchronize after each step (so the next GEMV sees every
    promotion) the recorder and LRU state follow the cache model exactly."""
    torch = torch_gpu
    print(f"cache async promotions type={wtype} slots={slots} n_tok={n_tok}", flush=True)
    n_experts, R, K = 16, 64, 4096
    be = GpuBackend(torch, mc, O, n_experts, R, K, wtype, seed=970 + wtype)
    free_b = torch.cuda.mem_get_info()[0]
    model, keep = S.run_scenario(mc, mc.lib(), be, n_experts=n_experts, R=R, K=K, wtype=wtype, slots=slots, steps=10,
                                 n_tok=n_tok, n_used=4, free_bytes=free_b, check_outputs=be.check_outputs,
                                 rng_seed=23 + n_tok, async_promotions=True, after_step=torch.cuda.synchronize)
    assert model.promotions > 0 and model.evictions > 0
    torch.cuda.synchronize()
    assert mc.lib().ggml_hip_moe_cache_reset() == 0


@pytest.mark.parametrize("gate_mode,shared_bias", [("device", False), ("device_host_desc", False), ("none", False),
                                                    ("cache", True), ("device", True)])
def test_cache_gate_modes_gpu(torch_gpu, mc, O, gate_mode, shared_bias):
    """Host-resident up with a gate the cache does not manage (device memory as fusion->gate, or a
    device tensor given as the host-side gate, which wants() refuses): the gate leaves no stamps, hits or
    misses (kernels/moe-cache.cu:178-201, :804) and is addressed per expert (the reference reads expert 0's
    gate there, :199-201).  With a shared expert and a routed bias, the shared expert takes no bias.
    Recorder and LRU state vs the cache model; outputs vs the resident path and the oracle."""
    torch = torch_gpu
    print(f"cache gate mode {gate_mode} shared_bias={shared_bias}", flush=True)
    n_experts, R, K, wtype = 16, 64, 2048, 10
    be = GpuBackend(torch, mc, O, n_experts, R, K, wtype, seed=950, gate_mode=gate_mode, shared_bias=shared_bias)
    free_b = torch.cuda.mem_get_info()[0]
    model, keep = S.run_scenario(mc, mc.lib(), be, n_experts=n_experts, R=R, K=K, wtype=wtype, slots=5, steps=8,
                                 n_tok=2, n_used=4, free_bytes=free_b, check_outputs=be.check_outputs, rng_seed=17,
                                 gate_mode=gate_mode, shared_bias=shared_bias)
    assert model.promotions > 0
    torch.cuda.synchronize()
    assert mc.lib().ggml_hip_moe_cache_reset() == 0


def test_cache_refuses_device_memory_and_views(torch_gpu, mc):
    torch = torch_gpu
    mc.reset()
    mc.configure(enabled=True)
    w = torch.zeros(8 * 4 * mc.row_bytes(mc.Q2_K, 256), dtype=torch.uint8, device="cuda")
    keep = []
    t = mc.make_tensor(mc.Q2_K, 256, 4, 8, w.data_ptr(), keep=keep)
    assert mc.lib().ggml_hip_moe_cache_wants(C.byref(t)) == 0         # device memory: not the cache path
    p = torch.zeros(8 * 4 * mc.row_bytes(mc.Q2_K, 256), dtype=torch.uint8, pin_memory=True)
    t = mc.make_tensor(mc.Q2_K, 256, 4, 8, p.data_ptr(), keep=keep)
    assert mc.lib().ggml_hip_moe_cache_wants(C.byref(t)) == 1
    assert mc.lib().ggml_hip_moe_cache_pin_host(C.byref(t)) == 1
    t.is_view = 1
    assert mc.lib().ggml_hip_moe_cache_wants(C.byref(t)) == 0
    t.is_view = 0
    t.ne[2] = 1
    assert mc.lib().ggml_hip_moe_cache_wants(C.byref(t)) == 0
    mc.reset()
