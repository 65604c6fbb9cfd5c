"""CPU: the product's registry / recorder contract / LRU step code (mc_host.cpp),
linked against the test-only simulated device, driven through the C ABI and
checked step by step against oracle/cache_model.py."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import cache_scenario as S
from oracle.cache_model import CacheModel

ROOT = Path(__file__).resolve().parent.parent
SEED_FIXTURE = ROOT / "tests" / "golden" / "moe_seed.txt"


class SimBackend:
    def __init__(self, lib):
        self.lib = lib
        self.stream = C.c_void_p(0)

    def host_tensor(self, nbytes, role):
        p = self.lib.mc_sim_host_alloc(nbytes)
        assert p
        return p, p

    def device_tensor(self, nbytes, role):
        p = self.lib.mc_sim_dev_alloc(nbytes)
        assert p
        return p, p

    def fusion_extra(self):
        R = 64
        bias = self.lib.mc_sim_dev_alloc(4 * R * 64)
        sh = self.lib.mc_sim_dev_alloc(1 << 16)
        sh_dst = self.lib.mc_sim_dev_alloc(4 * R * 8)
        return {"x_bias": bias, "shared_up": sh, "shared_gate": sh, "shared_dst": sh_dst, "shared_type": 12,
                "shared_stride_col_dst": R}

    def ids_buffer(self, n_tok, n_used):
        self.ids = np.zeros((n_tok, n_used), np.int32)

        def setter(ids):
            self.ids[:] = ids
        return self.ids.ctypes.data, setter

    def act_buffer(self, n_tok, K):
        self.y = np.zeros(n_tok * K, np.uint8)
        return self.y.ctypes.data

    def dst_buffer(self, n_tok, n_used, R):
        self.dst = np.zeros(n_tok * n_used * R, np.float32)
        return self.dst.ctypes.data


@pytest.mark.parametrize("slots,steps,n_tok,n_used,max_promo,rseed", [
    (5, 30, 2, 4, 48, 1), (3, 25, 4, 8, 2, 2), (16, 10, 1, 8, 48, 3), (0, 8, 2, 4, 48, 4), (1, 40, 3, 6, 5, 5)])
def test_sim_scenario_matches_model(sim, mc, tmp_path, slots, steps, n_tok, n_used, max_promo, rseed):
    seed_path = str(tmp_path / "seed.txt")
    with open(seed_path, "w") as f:
        f.write(f"{S.UP_NAME} 4,4,1,2\n{S.GATE_NAME} 9,15,17,-1\n")
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    model, keep = S.run_scenario(mc, sim, SimBackend(sim), n_experts=16, R=8, K=256, wtype=10, slots=slots,
                                 steps=steps, n_tok=n_tok, n_used=n_used, seed_path=seed_path, free_bytes=64 << 30,
                                 max_promotions=max_promo, rng_seed=rseed)
    if slots:
        assert model.promotions > 0


@pytest.mark.parametrize("gate_mode,shared_bias", [("device", False), ("device_host_desc", False), ("none", False),
                                                    ("cache", True), ("device", True)])
def test_sim_gate_modes_match_model(sim, mc, gate_mode, shared_bias):
    """A gate the cache does not manage (device memory as fusion->gate, or a device tensor that wants()
    refuses) and no gate at all leave no gate stamps, hits or misses (kernels/moe-cache.cu:178-201, :804):
    the model records the up tensor only.  A shared expert with a routed bias changes nothing recorded."""
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    model, keep = S.run_scenario(mc, sim, SimBackend(sim), n_experts=16, R=8, K=256, wtype=10, slots=5, steps=20,
                                 n_tok=2, n_used=4, free_bytes=64 << 30, rng_seed=11, gate_mode=gate_mode,
                                 shared_bias=shared_bias)
    assert len(model.entries) == (2 if gate_mode == "cache" else 1)
    assert model.promotions > 0 and model.evictions > 0


@pytest.mark.parametrize("slots,n_tok,max_promo,rseed,gate_mode", [
    (5, 2, 48, 21, "cache"), (3, 4, 2, 22, "cache"), (1, 3, 5, 23, "device")])
def test_sim_async_promotions_match_model(sim, mc, slots, n_tok, max_promo, rseed, gate_mode):
    """Promotion copies on the second stream: the simulated device completes every copy when it is
    issued, so the registry, tables, pools and counters must follow the model step for step; the
    stream and events go away with reset."""
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    model, keep = S.run_scenario(mc, sim, SimBackend(sim), n_experts=16, R=8, K=256, wtype=10, slots=slots, steps=25,
                                 n_tok=n_tok, n_used=4, free_bytes=64 << 30, max_promotions=max_promo, rng_seed=rseed,
                                 gate_mode=gate_mode, async_promotions=True)
    assert model.promotions > 0 and (slots >= 16 or model.evictions > 0)
    se = (C.c_longlong * 2)()
    sim.mc_sim_live_streams_events(se)
    assert se[0] == 1 and se[1] == 2                 # one copy stream, its two events
    assert sim.ggml_hip_moe_cache_reset() == 0
    sim.mc_sim_live_streams_events(se)
    assert se[0] == 0 and se[1] == 0


def test_sim_step_reads_stamps_in_one_batch(sim, mc):
    """A step that evicts in several tensors reads their stamps with one wait, not one per tensor."""
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    cnt = (C.c_longlong * 5)()
    before, after = [], []

    def pre(step, ids):                              # called right before each step
        sim.mc_sim_counters(cnt)
        before.append(cnt[3])

    def post():
        sim.mc_sim_counters(cnt)
        after.append(cnt[3])
    model, keep = S.run_scenario(mc, sim, SimBackend(sim), n_experts=16, R=8, K=256, wtype=10, slots=2, steps=12,
                                 n_tok=3, n_used=4, free_bytes=64 << 30, rng_seed=31, gate_mode="cache",
                                 check_outputs=pre, after_step=post)
    # each step: the stats wait and at most one stamps wait, though both tensors (up, gate) evict
    per_step = np.array(after) - np.array(before)
    assert model.evictions > 4 and per_step.max() == 2, per_step


@pytest.mark.parametrize("fail_after,what", [(4, b"table upload"), (2, b"seed copy")])
def test_sim_failed_registration_leaves_nothing(sim, mc, tmp_path, fail_after, what):
    """A failing seed copy or table upload frees the pool, table and stamps and registers nothing, so a
    later call registers the tensor afresh (never an entry whose device table was not written)."""
    be = SimBackend(sim)
    assert sim.ggml_hip_moe_cache_reset() == 0
    seed_path = str(tmp_path / "seed.txt")
    with open(seed_path, "w") as f:
        f.write("x 3,1,2,0\n")
    cfg = mc.Config()
    sp = seed_path.encode()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb, cfg.seed_path, cfg.max_promotions = 1, 4, 0.0, 0.0, sp, 48
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    K, R, n = 256, 8, 8
    eb = mc.row_bytes(mc.Q2_K, K) * R
    keep = []
    p = be.host_tensor(eb * n, "up")[0]
    t = mc.make_tensor(mc.Q2_K, K, R, n, p, name="x", keep=keep)
    ids_p, set_ids = be.ids_buffer(1, 2)
    set_ids(np.array([[0, 1]], np.int32))
    y, d = be.act_buffer(1, K), be.dst_buffer(1, 2, R)
    args = (K, R, n, 1, 1, 1, eb, eb * n, 1, 2, 8, 2 * R, 8, R, 2, be.stream)
    # the first call creates the globals (stats, clock, pinned stats, stamps arenas); measure after that
    assert sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, y, ids_p, d, *args) == 0
    assert sim.ggml_hip_moe_cache_reset() == 0
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    base = sim.mc_sim_live_regions()
    # the registration's H2D copies are seed 3, seed 1, seed 2, seed 0, then the table: fail_after of
    # them succeed and the next one fails
    sim.mc_sim_fail_h2d_after(fail_after)
    rc = sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, y, ids_p, d, *args)
    sim.mc_sim_fail_h2d_after(-1)
    assert rc < 0 and what in sim.ggml_hip_moe_last_error()
    assert sim.ggml_hip_moe_cache_num_entries() == 0
    # stats/clock/pinned stats and the stamps arena (device + pinned) remain; nothing of the failed entry does
    assert sim.mc_sim_live_regions() == base + 5
    assert sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, y, ids_p, d, *args) == 0
    assert sim.ggml_hip_moe_cache_num_entries() == 1
    expert_of = np.empty(4, np.int32)
    assert sim.ggml_hip_moe_cache_entry_slots(0, None, 0, expert_of.ctypes.data, 4) == 0
    assert expert_of.tolist() == [3, 1, 2, 0]
    assert sim.ggml_hip_moe_cache_reset() == 0
    assert sim.mc_sim_live_regions() == base


def test_sim_budget_and_free_memory_clamp(sim, mc):
    """slots = min(SLOTS, budget_left/eb, (free - margin)/eb, n_experts) (kernels/moe-cache.cu:542-561)."""
    be = SimBackend(sim)
    K, R, n = 256, 8, 64
    eb = mc.row_bytes(mc.Q2_K, K) * R          # 672 bytes
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb, cfg.seed_path, cfg.max_promotions = 1, 40, 30 * eb / (1 << 30), 0.0, None, 48
    assert sim.ggml_hip_moe_cache_reset() == 0
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    sim.mc_sim_set_mem_info(12 * eb, 1 << 30)    # free memory binds for the 2nd tensor
    keep = []
    ids_p, set_ids = be.ids_buffer(1, 2)
    set_ids(np.array([[0, 1]], np.int32))
    got = []
    for i in range(3):
        p = be.host_tensor(eb * n, "up")[0]
        t = mc.make_tensor(mc.Q2_K, K, R, n, p, name=f"t{i}", keep=keep)
        rc = sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, be.act_buffer(1, K), ids_p,
                                                   be.dst_buffer(1, 2, R), K, R, n, 1, 1, 1, eb, eb * n, 1, 2, 8, 2 * R,
                                                   8, R, 2, be.stream)
        assert rc == 0, sim.ggml_hip_moe_last_error()
        info = mc.EntryInfo()
        sim.ggml_hip_moe_cache_entry_info(i, C.byref(info))
        got.append(info.n_slots)
    # tensor 0: min(40, budget 30, free 12) = 12; tensor 1: min(40, 18, 12) = 12; tensor 2: min(40, 6, 12) = 6
    model = CacheModel(slots=40, budget_bytes=int(30 * eb / (1 << 30) * (1 << 30)), margin_bytes=0)
    want = [model.register(i, f"t{i}", n, eb, 12 * eb).n_slots for i in range(3)]
    assert got == want == [12, 12, 6]
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)


def test_sim_alloc_failure_is_an_error_not_an_abort(sim, mc):
    be = SimBackend(sim)
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb, cfg.seed_path, cfg.max_promotions = 1, 4, 0.0, 0.0, None, 48
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    K, R, n = 256, 8, 8
    eb = mc.row_bytes(mc.Q2_K, K) * R
    keep = []
    p = be.host_tensor(eb * n, "up")[0]
    t = mc.make_tensor(mc.Q2_K, K, R, n, p, name="x", keep=keep)
    ids_p, set_ids = be.ids_buffer(1, 2)
    set_ids(np.array([[0, 1]], np.int32))
    sim.mc_sim_fail_alloc_after(3)   # stats, pinned stats, clock succeed; the table allocation fails
    rc = sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, be.act_buffer(1, K), ids_p, be.dst_buffer(1, 2, R),
                                               K, R, n, 1, 1, 1, eb, eb * n, 1, 2, 8, 2 * R, 8, R, 2, be.stream)
    sim.mc_sim_fail_alloc_after(-1)
    assert rc < 0
    assert b"alloc" in sim.ggml_hip_moe_last_error()
    assert sim.ggml_hip_moe_cache_num_entries() == 0


def test_sim_rejects_unsupported(sim, mc):
    be = SimBackend(sim)
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb, cfg.seed_path, cfg.max_promotions = 1, 4, 0.0, 0.0, None, 48
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    keep = []
    p = be.host_tensor(1 << 16, "up")[0]
    t = mc.make_tensor(mc.Q2_K, 256, 8, 8, p, name="x", keep=keep)
    assert sim.ggml_hip_moe_cache_wants(C.byref(t)) == 1
    t.type = 3                                     # Q4_1: not on the path
    assert sim.ggml_hip_moe_cache_wants(C.byref(t)) == 0
    t.type = mc.Q2_K
    t.nb[1] += 4                                   # non-contiguous rows
    assert sim.ggml_hip_moe_cache_wants(C.byref(t)) == 0
    t = mc.make_tensor(mc.Q2_K, 256, 8, 8, sim.mc_sim_plain_alloc(1 << 16), name="y", keep=keep)
    assert sim.ggml_hip_moe_cache_wants(C.byref(t)) == 0       # not GPU-readable host memory
    assert sim.ggml_hip_moe_cache_pin_host(C.byref(t)) == 0    # registration not allowed by default
    t = mc.make_tensor(mc.Q2_K, 256, 8, 8, sim.mc_sim_dev_alloc(1 << 16), name="z", keep=keep)
    assert sim.ggml_hip_moe_cache_wants(C.byref(t)) == 0       # device memory
    # an unsupported type through the GEMV entry is an error code, not an abort
    t = mc.make_tensor(mc.Q2_K, 256, 8, 8, p, name="x", keep=keep)
    t.type = 3
    ids_p, set_ids = be.ids_buffer(1, 2)
    rc = sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, be.act_buffer(1, 256), ids_p, be.dst_buffer(1, 2, 8),
                                               256, 8, 8, 1, 1, 1, 0, 0, 1, 2, 8, 16, 8, 8, 2, be.stream)
    assert rc < 0


def test_sim_disabled_by_default(sim, mc):
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled = 0
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    assert sim.ggml_hip_moe_cache_enabled() == 0
    assert sim.ggml_hip_moe_cache_step(None) == 0      # no-op
    assert sim.ggml_hip_moe_cache_active() == 0


def test_sim_seed_fixture_registration(sim, mc):
    """Registration with the reference's own seed file: slots 0..k-1 follow the file's order."""
    from oracle.cache_model import parse_seed_file
    seed = parse_seed_file(SEED_FIXTURE)
    name = "blk.47.ffn_gate_exps.weight"
    be = SimBackend(sim)
    assert sim.ggml_hip_moe_cache_reset() == 0
    cfg = mc.Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb, cfg.max_promotions = 1, 100, 0.0, 0.0, 48
    sp = str(SEED_FIXTURE).encode()
    cfg.seed_path = sp
    assert sim.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0
    sim.mc_sim_set_mem_info(64 << 30, 64 << 30)
    K, R, n = 256, 2, 512
    eb = mc.row_bytes(mc.Q2_K, K) * R
    keep = []
    p = be.host_tensor(eb * n, "up")[0]
    t = mc.make_tensor(mc.Q2_K, K, R, n, p, name=name, keep=keep)
    ids_p, set_ids = be.ids_buffer(1, 1)
    set_ids(np.array([[0]], np.int32))
    rc = sim.ggml_hip_moe_cache_mul_mat_vec_q(C.byref(t), None, None, be.act_buffer(1, K), ids_p, be.dst_buffer(1, 1, R),
                                               K, R, n, 1, 1, 1, eb, eb * n, 1, 1, 8, R, 8, R, 1, be.stream)
    assert rc == 0, sim.ggml_hip_moe_last_error()
    expert_of = np.empty(100, np.int32)
    assert sim.ggml_hip_moe_cache_entry_slots(0, None, 0, expert_of.ctypes.data, 100) == 0
    assert expert_of[:5].tolist() == [333, 183, 357, 241, 146]
    assert expert_of.tolist() == seed[name][:100]
