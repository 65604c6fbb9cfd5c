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
    def __init__(self, torch, mc, O, n_experts, R, K, wtype, seed):
        self.torch, self.mc, self.O = torch, mc, O
        self.K, self.R, self.wtype, self.n_experts = K, R, wtype, n_experts
        self.w = {"up": H.weights(wtype, n_experts, R, K, seed=seed),
                  "gate": H.weights(wtype, n_experts, R, K, seed=seed + 1)}
        self.stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.keep = []

    def host_tensor(self, nbytes, role):
        t = self.torch.empty(nbytes, dtype=self.torch.uint8, pin_memory=True)
        t.numpy()[:] = self.w[role].reshape(-1)
        self.keep.append(t)
        return t.data_ptr(), t

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
        # the same weights resident in device memory, through the no-cache entry point
        ref = torch.zeros_like(self.dst)
        up_d = torch.from_numpy(self.w["up"]).cuda()
        gate_d = torch.from_numpy(self.w["gate"]).cuda()
        f = mc.make_fusion(gate=gate_d, glu_op=mc.GLU_SWIGLU)
        mc.mul_mat_vec(wtype=self.wtype, weights=up_d, ids=self.ids, y=self.y, dst=ref, K=self.K, R=self.R,
                       n_experts=self.n_experts, fusion=f)
        torch.cuda.synchronize()
        assert np.array_equal(got, ref.cpu().numpy()), f"step {step}: cache path != resident path"
        yb = self.y.cpu().numpy().reshape(ids.shape[0], 1, -1)
        want = O.mul_mat_id(wtype=self.wtype, K=self.K, R=self.R, n_as=self.n_experts, src0=self.w["up"],
                            gate=self.w["gate"], ids=ids, act=yb, act_kind=O.ACT_Q8_1, glu_op=O.GLU_SWIGLU)
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
