"""ggml_hip_moe_mul_mat_id_noalloc: the op-level MUL_MAT_ID for callers that cannot
allocate, with the library's per-GPU device scratch as its workspace.

GPU: through the C ABI, two calls in a row (the second smaller) give the same
bytes as ggml_hip_moe_mul_mat_id with a caller workspace, on the grouped-GEMM
path and the GEMV path; a call whose workspace would exceed the scratch is
refused with a clear error.  CPU (simulated device): the refusals, and no
device allocation on the way to the first launch.
"""
import ctypes as C
from importlib import import_module
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
SCRATCH_BYTES = 64 << 20


def _note(msg):
    print(msg, flush=True)


def _problem(torch, mc, wtype, E, R, K, n_tok, n_used, seed, gate):
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    w = md.random_expert_tensor(torch, wtype, E, R, K, gen)
    g = md.random_expert_tensor(torch, wtype, E, R, K, gen) if gate else None
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((n_tok, 1, K)).astype(np.float32)).cuda()
    ids_np = np.stack([rng.choice(E, n_used, replace=False) for _ in range(n_tok)]).astype(np.int32)
    ids = torch.from_numpy(ids_np).cuda()
    return w, g, x, ids


def _descs(mc, wtype, w, x, ids, dst, K, R, E, keep):
    src0 = mc.make_tensor(wtype, K, R, E, w.data_ptr(), keep=keep)
    return src0, mc.torch_tensor_desc(x, mc.GGML_F32), mc.torch_tensor_desc(ids, mc.GGML_I32), \
        mc.torch_tensor_desc(dst, mc.GGML_F32)


def _noalloc(torch, mc, wtype, w, x, ids, dst, K, R, E, fusion):
    keep = []
    s0, s1, it, dt = _descs(mc, wtype, w, x, ids, dst, K, R, E, keep)
    fp = C.byref(fusion) if fusion is not None else None
    return mc.lib().ggml_hip_moe_mul_mat_id_noalloc(C.byref(s0), C.byref(s1), C.byref(it), C.byref(dt), fp,
                                                    C.c_void_p(torch.cuda.current_stream().cuda_stream))


# first call, then a smaller second call: (type, experts, rows, K, tokens, slots, gate)
SEQUENCES = [
    (("Q4_K", 64, 256, 2048, 64, 8, True), ("Q4_K", 64, 256, 2048, 5, 8, True)),     # grouped GEMM, then GEMV
    (("Q2_K", 512, 768, 4096, 512, 8, True), ("Q2_K", 512, 768, 4096, 96, 8, True)),  # prefill-sized grouped GEMMs
    (("Q2_K", 32, 128, 4096, 6, 4, False), ("Q2_K", 32, 128, 4096, 1, 4, False)),     # GEMV twice
    (("Q4_0", 16, 64, 1024, 3, 2, True), ("Q4_0", 16, 64, 1024, 2, 2, True)),         # legacy-type GEMV
]


@pytest.mark.gpu
@pytest.mark.parametrize("seq", SEQUENCES, ids=lambda s: f"{s[0][0]}-{s[0][4]}tok-then-{s[1][4]}tok")
def test_noalloc_matches_mul_mat_id(torch_gpu, mc, seq):
    torch = torch_gpu
    for i, (tname, E, R, K, n_tok, n_used, gate) in enumerate(seq):
        t = getattr(mc, tname)
        _note(f"noalloc call {i}: {tname} E={E} R={R} K={K} tokens={n_tok} slots={n_used} gate={gate}")
        w, g, x, ids = _problem(torch, mc, t, E, R, K, n_tok, n_used, seed=1000 * i + E + n_tok, gate=gate)
        f = mc.make_fusion(gate=g, glu_op=mc.GLU_SWIGLU) if gate else None
        ref = torch.full((n_tok, n_used, R), -3.5, dtype=torch.float32, device="cuda")
        mc.mul_mat_id(wtype=t, weights=w, x=x, ids=ids, dst=ref, K=K, R=R, n_experts=E, fusion=f)
        dst = torch.full_like(ref, -3.5)
        rc = _noalloc(torch, mc, t, w, x, ids, dst, K, R, E, f)
        assert rc == 0, mc.lib().ggml_hip_moe_last_error()
        torch.cuda.synchronize()
        assert torch.equal(dst, ref), f"call {i}: no-alloc entry != ggml_hip_moe_mul_mat_id"
        assert bool(torch.isfinite(dst).all())


@pytest.mark.gpu
def test_noalloc_refuses_beyond_scratch(torch_gpu, mc):
    """2048 tokens x top-8 over 512 Q4_K experts of 4096 columns needs ~110 MB of grouped-GEMM workspace: refused
    before anything is launched (the buffers are real, full-size tensors all the same)."""
    torch = torch_gpu
    E, R, K, n_tok, U = 512, 64, 4096, 2048, 8
    w, _, x, ids = _problem(torch, mc, mc.Q4_K, E, R, K, n_tok, U, seed=7, gate=False)
    dst = torch.full((n_tok, U, R), -3.5, dtype=torch.float32, device="cuda")
    keep = []
    s0, s1, it, _ = _descs(mc, mc.Q4_K, w, x, ids, dst, K, R, E, keep)
    need = mc.lib().ggml_hip_moe_mul_mat_id_workspace_bytes(C.byref(s0), C.byref(s1), C.byref(it), None)
    assert need > SCRATCH_BYTES
    rc = _noalloc(torch, mc, mc.Q4_K, w, x, ids, dst, K, R, E, None)
    assert rc == mc.E_UNSUPPORTED
    assert b"scratch holds" in mc.lib().ggml_hip_moe_last_error()
    torch.cuda.synchronize()
    assert bool((dst == -3.5).all())


# ---------------------------------------------------------------------------
# CPU: simulated device
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def sim(mc):
    import importlib.util
    spec = importlib.util.spec_from_file_location("mc_build", ROOT / "a6000-custom-kernels_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    lib = mc.bind(b.build_hostsim())
    for n, r, a in (("mc_sim_host_alloc", C.c_void_p, [C.c_uint64]), ("mc_sim_dev_alloc", C.c_void_p, [C.c_uint64]),
                    ("mc_sim_alloc_count", C.c_longlong, [])):
        fn = getattr(lib, n)
        fn.restype, fn.argtypes = r, a
    return lib


def _sim_call(mc, sim, data, n_tok, K=256, R=8, E=8, U=2):
    x = np.zeros((n_tok, 1, K), np.float32)
    ids = np.zeros((n_tok, U), np.int32)
    dst = np.zeros((n_tok, U, R), np.float32)
    keep = []
    s0 = mc.make_tensor(mc.Q2_K, K, R, E, data, keep=keep)

    def desc(a, t):
        d = mc.Tensor()
        ne = list(a.shape)[::-1] + [1] * (4 - a.ndim)
        nb = [st for st in a.strides[::-1]]
        while len(nb) < 4:
            nb.append(nb[-1] * ne[len(nb) - 1])
        d.type, d.ne[:], d.nb[:], d.data, d.has_buffer = t, ne, nb, a.ctypes.data, 1
        return d
    s1, it, dt = desc(x, mc.GGML_F32), desc(ids, mc.GGML_I32), desc(dst, mc.GGML_F32)
    rc = sim.ggml_hip_moe_mul_mat_id_noalloc(C.byref(s0), C.byref(s1), C.byref(it), C.byref(dt), None, None)
    return rc, sim.ggml_hip_moe_last_error()


def test_noalloc_sim_refusals_allocate_nothing(sim, mc):
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.max_promotions = 1, 4, 48
    assert sim.ggml_hip_moe_cache_reset() == 0
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    eb = mc.row_bytes(mc.Q2_K, 256) * 8
    dev_w = sim.mc_sim_dev_alloc(eb * 8)
    host_w = sim.mc_sim_host_alloc(eb * 8)
    n0 = sim.mc_sim_alloc_count()
    # host-resident experts: the cache path would register (allocate)
    rc, msg = _sim_call(mc, sim, host_w, 2)
    assert rc == mc.E_UNSUPPORTED and b"device-resident" in msg
    # the simulated scratch holds 1 MiB: 4096 tokens of q8_1 rows of 256 values need 1.2 MB
    rc, msg = _sim_call(mc, sim, dev_w, 4096)
    assert rc == mc.E_UNSUPPORTED and b"scratch holds" in msg
    # within the scratch: the call reaches the quantize launch (which the simulation does not run)
    rc, msg = _sim_call(mc, sim, dev_w, 3)
    assert rc == mc.E_DEVICE and b"quantize" in msg
    assert sim.mc_sim_alloc_count() == n0
    assert sim.ggml_hip_moe_cache_num_entries() == 0
