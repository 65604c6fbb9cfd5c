"""A cache scenario driven through the C ABI and checked against oracle/cache_model.py.

The same driver runs against the product library on the GPU (pinned host
experts read zero-copy, HBM pool, real kernels) and against the test-only
host-memory simulated device (CPU), so the registry / recorder / LRU contract
is checked identically on both.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from oracle.cache_model import CacheModel, parse_seed_file

UP_NAME = "blk.7.ffn_up_exps.weight"
GATE_NAME = "blk.7.ffn_gate_exps.weight"


def skewed_ids(rng, n_tok, n_used, n_experts, s=1.1):
    """top-n_used picks per token from a Zipf-like distribution (without replacement)."""
    p = 1.0 / np.arange(1, n_experts + 1) ** s
    p /= p.sum()
    return np.stack([rng.choice(n_experts, size=n_used, replace=False, p=p) for _ in range(n_tok)]).astype(np.int32)


def compare_state(mc_mod, lib, model: CacheModel, tag: str):
    n = lib.ggml_hip_moe_cache_num_entries()
    assert n == len(model.entries), (tag, n, len(model.entries))
    for e in model.entries:
        info = mc_mod.EntryInfo()
        assert lib.ggml_hip_moe_cache_entry_info(e.id, C.byref(info)) == 0
        assert info.n_slots == e.n_slots and info.n_experts == e.n_experts, (tag, info.n_slots, e.n_slots)
        slot_of = np.empty(e.n_experts, np.int32)
        expert_of = np.empty(max(e.n_slots, 1), np.int32)
        table = np.empty(e.n_experts, np.int32)
        assert lib.ggml_hip_moe_cache_entry_slots(e.id, slot_of.ctypes.data, e.n_experts, expert_of.ctypes.data,
                                                  e.n_slots) == 0
        assert lib.ggml_hip_moe_cache_entry_table(e.id, table.ctypes.data, e.n_experts) == 0
        assert slot_of.tolist() == e.slot_of, (tag, e.name, slot_of.tolist(), e.slot_of)
        assert expert_of[:e.n_slots].tolist() == e.expert_of, (tag, e.name)
        assert table.tolist() == e.table(), (tag, e.name)


def check_recorder(lib, stream, model: CacheModel, tag: str):
    stats = np.zeros(2 + 8190, np.uint32)
    assert lib.ggml_hip_moe_cache_stats_snapshot(stats.ctypes.data, stats.size, stream) == 0
    assert int(stats[0]) == model.count, (tag, int(stats[0]), model.count)
    assert int(stats[1]) == model.hits, (tag, int(stats[1]), model.hits)
    n = min(model.count, 8190)
    assert stats[2:2 + n].tolist() == model.log[:n], tag
    for e in model.entries:
        st = np.zeros(e.n_experts, np.uint32)
        assert lib.ggml_hip_moe_cache_stamps_snapshot(e.id, st.ctypes.data, e.n_experts, stream) == 0
        assert st.tolist() == e.stamps, (tag, e.name)


def fusion_from_ptrs(mc_mod, **ptrs):
    """ggml_hip_moe_fusion from raw addresses (ints); glu_op SWIGLU unless given."""
    f = mc_mod.Fusion()
    f.glu_op = ptrs.pop("glu_op", 2)
    f.shared_type = ptrs.pop("shared_type", -1)
    for k, v in ptrs.items():
        setattr(f, k, v)
    return f


GATE_MODES = ("cache", "device", "device_host_desc", "none")


def run_scenario(mc_mod, lib, backend, *, n_experts=16, R=40, K=4096, wtype=10, slots=5, steps=12, n_tok=2,
                 n_used=4, seed_path=None, free_bytes, max_promotions=48, check_outputs=None, rng_seed=1234,
                 gate_mode="cache", shared_bias=False, async_promotions=False, after_step=None):
    """backend: object with
         host_tensor(nbytes, role) -> (ptr, keepalive)  GPU-readable host memory holding the weights of `role`
         device_tensor(nbytes, role) -> (ptr, keepalive) device memory holding the weights of `role`
         fusion_extra() -> dict of fusion fields (x_bias, shared_up, shared_gate, shared_dst, shared_type,
                           shared_stride_col_dst) as addresses: a shared expert and a routed bias
         ids_buffer(n_tok, n_used) -> (ptr, setter)     device-visible ids
         act_buffer(n_tok, K), dst_buffer(n_tok, n_used, R) -> ptr
         stream -> c_void_p
       gate_mode: "cache"  the gate is a host tensor the cache manages (its own entry, stamps and misses);
                  "device" the gate is device memory passed as fusion->gate;
                  "device_host_desc" the gate is device memory passed as the host-side gate tensor, which
                           wants() refuses;
                  "none"   no gate.
       Only a cache-managed gate is recorded (kernels/moe-cache.cu:178-201, :804): the model sees gate=None
       otherwise.  check_outputs(step, ids) is called after each GEMV when given (GPU backend).
       async_promotions: the step's promotion copies go on the library's second stream; after_step()
       (e.g. a device-wide synchronize) runs after each step, before the state is compared, so the
       next GEMV sees every promotion, as the model assumes."""
    assert gate_mode in GATE_MODES, gate_mode
    rng = np.random.default_rng(rng_seed)
    cfg = mc_mod.Config()
    cfg.enabled, cfg.slots, cfg.budget_gb, cfg.margin_gb = 1, slots, 0.0, 2.0
    sp = seed_path.encode() if seed_path else None
    cfg.seed_path = sp
    cfg.max_promotions, cfg.verbose = max_promotions, 0
    cfg.async_promotions = int(async_promotions)
    assert lib.ggml_hip_moe_cache_reset() == 0
    assert lib.ggml_hip_moe_cache_configure(C.byref(cfg)) == 0, lib.ggml_hip_moe_last_error()

    rb = mc_mod.row_bytes(wtype, K)
    eb = rb * R
    up_ptr, up_keep = backend.host_tensor(eb * n_experts, "up")
    keep = []
    up_t = mc_mod.make_tensor(wtype, K, R, n_experts, up_ptr, name=UP_NAME, keep=keep)
    gate_t, gate_keep, fptrs = None, None, {}
    if gate_mode == "cache":
        gate_ptr, gate_keep = backend.host_tensor(eb * n_experts, "gate")
        gate_t = mc_mod.make_tensor(wtype, K, R, n_experts, gate_ptr, name=GATE_NAME, keep=keep)
    elif gate_mode == "device_host_desc":
        gate_ptr, gate_keep = backend.device_tensor(eb * n_experts, "gate")
        gate_t = mc_mod.make_tensor(wtype, K, R, n_experts, gate_ptr, name=GATE_NAME, keep=keep)
        assert lib.ggml_hip_moe_cache_wants(C.byref(gate_t)) == 0
    elif gate_mode == "device":
        gate_ptr, gate_keep = backend.device_tensor(eb * n_experts, "gate")
        fptrs["gate"] = gate_ptr
    if shared_bias:
        fptrs.update(backend.fusion_extra())
    fusion = fusion_from_ptrs(mc_mod, **fptrs) if fptrs else None
    assert lib.ggml_hip_moe_cache_wants(C.byref(up_t)) == 1, lib.ggml_hip_moe_last_error()
    assert lib.ggml_hip_moe_cache_active() == 0

    model = CacheModel(slots=slots, budget_bytes=0, margin_bytes=2 << 30, max_promotions=max_promotions,
                       seed=parse_seed_file(seed_path) if seed_path else None)
    ids_ptr, set_ids = backend.ids_buffer(n_tok, n_used)
    y_ptr = backend.act_buffer(n_tok, K)
    dst_ptr = backend.dst_buffer(n_tok, n_used, R)
    stream = backend.stream
    act_row = K // 32
    gate_e = None
    for step in range(steps):
        ids = skewed_ids(rng, n_tok, n_used, n_experts)
        set_ids(ids)
        rc = lib.ggml_hip_moe_cache_mul_mat_vec_q(
            C.byref(up_t), C.byref(gate_t) if gate_t is not None else None,
            C.byref(fusion) if fusion is not None else None, y_ptr, ids_ptr, dst_ptr,
            K, R, n_experts, 1, n_tok, K // mc_mod.BLOCK[wtype][0], eb, eb * n_experts,
            1, n_used, act_row, n_used * R, act_row, R, n_used, stream)
        assert rc == 0, lib.ggml_hip_moe_last_error()
        if step == 0:
            up_e = model.register(up_ptr, UP_NAME, n_experts, eb, free_bytes)
            if gate_mode == "cache":
                gate_e = model.register(gate_ptr, GATE_NAME, n_experts, eb, free_bytes)
            assert lib.ggml_hip_moe_cache_active() == 1
            compare_state(mc_mod, lib, model, "after registration")
        model.record(up_e, gate_e, ids.tolist())
        check_recorder(lib, stream, model, f"step {step} recorder")
        if check_outputs is not None:
            check_outputs(step, ids)
        assert lib.ggml_hip_moe_cache_step(stream) == 0, lib.ggml_hip_moe_last_error()
        if after_step is not None:
            after_step()
        model.step()
        compare_state(mc_mod, lib, model, f"step {step} after promotion")
        tot = mc_mod.Totals()
        assert lib.ggml_hip_moe_cache_totals(C.byref(tot)) == 0
        assert (tot.last_step_misses, tot.last_step_hits) == model.last, (step, tot.last_step_misses, model.last)
        assert tot.promotions == model.promotions and tot.evictions == model.evictions and tot.clock == model.clock
    return model, (up_keep, gate_keep, keep, sp, fusion)
