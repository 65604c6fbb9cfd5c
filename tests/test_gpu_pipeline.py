"""GPU: the host-side sequences around the pointer-table path, end to end on pinned tensors.

- The scheduler claims (results/final.patch:13-54 with kernels/moe-cache.cu:365-405): enabled() claims
  the MUL_MAT_ID, pin_host() accepts GPU-readable host memory (and refuses device and pageable
  memory without registering anything), wants() selects the cache path, the first MUL_MAT_ID
  registers the tensor (active() turns 1), and the step runs between tokens.
- The seed pipeline (patches/trace-hook/ggml-cpu.c:1597-1617, tools/make_seed.py:30-51,
  kernels/moe-cache.cu:587-609): routing ids read back from the GPU are appended to a trace with
  ggml_hip_moe_trace_append, make_seed ranks them into a seed file, and a seeded registration
  fills the pool with the most frequent experts.
Outputs are checked bit for bit against the device-resident GEMV on the same weights."""
import ctypes as C
import sys
from importlib import import_module

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _gemv_args(K, R, E, eb, n_tok, n_used):
    ar = K // 32
    return (K, R, E, 1, n_tok, K // 256, eb, eb * E, 1, n_used, ar, n_used * R, ar, R, n_used)


def test_scheduler_claims_sequence(torch_gpu, mc):
    torch = torch_gpu
    lib = mc.lib()
    E, R, K, U, n_tok, wtype = 32, 64, 2048, 4, 1, mc.Q2_K
    eb = mc.row_bytes(wtype, K) * R
    w = H.weights(wtype, E, R, K, seed=3100)
    keep = []
    mc.reset()
    mc.configure(enabled=True, slots=6, max_promotions=8)
    assert lib.ggml_hip_moe_cache_enabled() == 1           # the offload hook claims MUL_MAT_ID
    assert lib.ggml_hip_moe_cache_active() == 0

    host = torch.empty(w.size, dtype=torch.uint8, pin_memory=True)
    host.numpy()[:] = w.reshape(-1)
    t_host = mc.make_tensor(wtype, K, R, E, host.data_ptr(), name="blk.0.ffn_up_exps.weight", keep=keep)
    dev_w = torch.from_numpy(w.reshape(-1)).cuda()
    t_dev = mc.make_tensor(wtype, K, R, E, dev_w.data_ptr(), name="dev", keep=keep)
    pageable = np.zeros(w.size + 4096, np.uint8)
    t_page = mc.make_tensor(wtype, K, R, E, pageable.ctypes.data, name="pageable", keep=keep)

    # buffer claims: pinned host memory is GPU-readable as it is; device memory is not the cache's;
    # pageable memory is refused (registration is off) with the reason
    assert lib.ggml_hip_moe_cache_pin_host(C.byref(t_host)) == 1
    assert lib.ggml_hip_moe_cache_pin_host(C.byref(t_dev)) == 0
    assert lib.ggml_hip_moe_cache_pin_host(C.byref(t_page)) == 0
    assert b"GPU-readable" in lib.ggml_hip_moe_last_error()
    assert lib.ggml_hip_moe_cache_wants(C.byref(t_host)) == 1
    assert lib.ggml_hip_moe_cache_wants(C.byref(t_dev)) == 0
    assert lib.ggml_hip_moe_cache_wants(C.byref(t_page)) == 0
    assert lib.ggml_hip_moe_cache_active() == 0            # nothing registered by the claims

    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((n_tok, K)).astype(np.float32)).cuda()
    y = mc.quantize_q8_1(x)
    ids = torch.zeros((n_tok, U), dtype=torch.int32, device="cuda")
    dst = torch.zeros((n_tok, U, R), dtype=torch.float32, device="cuda")
    ref = torch.zeros_like(dst)
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    tot0 = mc.totals()
    for tok in range(12):
        ids.copy_(torch.from_numpy(rng.choice(12, (n_tok, U), replace=False).astype(np.int32).reshape(n_tok, U)))
        mc.check(lib.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t_host), None, None, y.data_ptr(), ids.data_ptr(),
                                                      dst.data_ptr(), *_gemv_args(K, R, E, eb, n_tok, U), s), "gemv")
        if tok == 0:
            assert lib.ggml_hip_moe_cache_active() == 1
            assert lib.ggml_hip_moe_cache_num_entries() == 1
        mc.mul_mat_vec(wtype=wtype, weights=dev_w, ids=ids, y=y.view(n_tok, 1, -1), dst=ref, K=K, R=R, n_experts=E)
        torch.cuda.synchronize()
        assert torch.equal(dst, ref), tok
        mc.check(lib.ggml_hip_moe_cache_step(s), "step")
    tot = mc.totals()
    assert tot.steps - tot0.steps == 12 and tot.promotions > 0
    assert tot.hits + tot.misses - tot0.hits - tot0.misses == 12 * n_tok * U
    torch.cuda.synchronize()
    mc.reset()
    assert lib.ggml_hip_moe_cache_active() == 0


def test_seed_pipeline(torch_gpu, mc, tmp_path):
    torch = torch_gpu
    lib = mc.lib()
    seed_mod = import_module("a6000_custom_kernels_amd.seed")
    E, R, K, U, wtype, slots = 64, 32, 1024, 6, mc.Q4_K, 9
    names = ("blk.0.ffn_up_exps.weight", "blk.1.ffn_up_exps.weight")
    eb = mc.row_bytes(wtype, K) * R
    ws = [H.weights(wtype, E, R, K, seed=3200 + i) for i in range(2)]
    keep = []
    rng = np.random.default_rng(9)
    p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
    p /= p.sum()
    perms = [rng.permutation(E) for _ in names]

    # 1. a routed run on the device (resident experts); its ids read back and traced per tensor
    trace = str(tmp_path / "trace.bin")
    dev = [torch.from_numpy(w.reshape(-1)).cuda() for w in ws]
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).cuda()
    y = mc.quantize_q8_1(x)
    ids = torch.zeros((1, U), dtype=torch.int32, device="cuda")
    out = torch.zeros((1, U, R), dtype=torch.float32, device="cuda")
    counts = [np.zeros(E, np.int64) for _ in names]
    for tok in range(40):
        for i, name in enumerate(names):
            ids.copy_(torch.from_numpy(perms[i][rng.choice(E, U, replace=False, p=p)].astype(np.int32)).view(1, U))
            mc.mul_mat_vec(wtype=wtype, weights=dev[i], ids=ids, y=y.view(1, 1, -1), dst=out, K=K, R=R, n_experts=E)
            ids_h = ids.cpu().numpy().astype(np.int32)            # the intercept's copy, outside capture
            counts[i][ids_h.reshape(-1)] += 1
            mc.check(lib.ggml_hip_moe_trace_append(trace.encode(), name.encode(), ids_h.ctypes.data, U, 1, E),
                     "trace")
    assert lib.ggml_hip_moe_trace_close() == 0

    # 2. make_seed: every tensor's experts ranked by count (ties in first-seen order)
    seed_path = str(tmp_path / "seed.txt")
    n_rec, got_counts = seed_mod.make_seed(trace, seed_path)
    assert n_rec == 80
    seeds = seed_mod.read_seed(seed_path)
    for i, name in enumerate(names):
        want_counts = {int(e): int(c) for e, c in enumerate(counts[i]) if c}
        assert dict(got_counts[name]) == want_counts
        assert sorted(seeds[name]) == sorted(want_counts)
        assert all(counts[i][a] >= counts[i][b] for a, b in zip(seeds[name], seeds[name][1:]))

    # 3. a seeded registration: slot k holds the k-th most frequent expert, its table entry points at the pool
    mc.reset()
    mc.configure(enabled=True, slots=slots, seed_path=seed_path)
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, name in enumerate(names):
        host = torch.empty(ws[i].size, dtype=torch.uint8, pin_memory=True)
        host.numpy()[:] = ws[i].reshape(-1)
        keep.append(host)
        t = mc.make_tensor(wtype, K, R, E, host.data_ptr(), name=name, keep=keep)
        ids.copy_(torch.from_numpy(np.array(seeds[name][:U], np.int32)).view(1, U))
        mc.check(lib.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, y.data_ptr(), ids.data_ptr(),
                                                      out.data_ptr(), *_gemv_args(K, R, E, eb, 1, U), s), "gemv")
        ref = torch.zeros_like(out)
        mc.mul_mat_vec(wtype=wtype, weights=dev[i], ids=ids, y=y.view(1, 1, -1), dst=ref, K=K, R=R, n_experts=E)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        slot_of = np.empty(E, np.int32)
        expert_of = np.empty(slots, np.int32)
        assert lib.ggml_hip_moe_cache_entry_slots(i, slot_of.ctypes.data, E, expert_of.ctypes.data, slots) == 0
        assert expert_of.tolist() == seeds[name][:slots]
        table = np.empty(E, np.int32)                        # decoded: pool slot, or -1 for host memory
        assert lib.ggml_hip_moe_cache_entry_table(i, table.ctypes.data, E) == 0
        want_tbl = np.full(E, -1, np.int32)
        want_tbl[seeds[name][:slots]] = np.arange(slots)
        assert np.array_equal(table, want_tbl), name
        _note(f"seeded {name}: slots {expert_of.tolist()}")
    # the seeded experts hit from the first token
    mc.check(lib.ggml_hip_moe_cache_step(s), "step")
    tot = mc.totals()
    assert tot.last_step_hits == 2 * U and tot.last_step_misses == 0
    torch.cuda.synchronize()
    mc.reset()
