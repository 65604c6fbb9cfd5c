#!/usr/bin/env python3
"""Benchmark: pointer-table quantized MoE GEMV on one MI355X.

Workload (one "step" = one decode token): the MoE block of a 48-layer model
shaped like the reference's (512 experts, hidden 4096, expert FFN 768, top-8
routing with softmax router weights, llama.cpp's Q2_K_S expert mix (Q2_K, the
first 6 layers' ffn_down in Q4_K), one always-on Q4_K shared expert, fused
SwiGLU), batch 1, every layer with its own weights (73 GiB resident in HBM, so
the 256 MB MALL cannot serve repeat reads).  One
token = 2 launches per layer through the C ABI (--plan fused: gate/up GEMV with
the RMSNorm + q8_1 of its input in the same launch, then the down GEMV with the
weighted combine), or 3 per layer (--plan ops: gate/up, down, combine),
captured once as a hipGraph.

value = achieved HBM GB/s of the whole step = algorithmic bytes per token
(unique expert matrices read + activations + outputs) x tokens/s.  The
roofline object prices the dominant kernel (the gate/up GEMV) with HIP events
on its own stream.  cpu_baseline times the CPU oracle's ggml-CPU
MUL_MAT_ID restatement on this host's cores over a bounded sample of the same
layer shape (its weights copied from the GPU).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "a6000-custom-kernels_amd"
PEAK_HBM_GBS = 8000.0
PEAK_INT8_OPS = 5.0e15        # MI355X dense int8 MFMA
METRIC = "MoE GEMV achieved HBM GB/s (% of peak) + 48-layer MoE decode tok/s"


def load_package():
    name = "a6000_custom_kernels_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_kernel(torch, model, launch, n_rounds):
    """Average duration of one launch of `launch(l)` over all layers: the L launches are
    captured as one graph (so host launch latency is excluded) and replayed n_rounds
    times between two events recorded on the stream the kernels run on."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for l in range(model.L):
                launch(l)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(n_rounds):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    n = n_rounds * model.L
    return e0.elapsed_time(e1) / n, n


def gate_up_launcher(model):
    """launch(l) of the plan's gate/up kernel (the fused plan normalizes model.x)."""
    if model.fused:
        return lambda l: model.launch_gate_up_norm(l, model.x)
    return model.launch_gate_up


def down_launcher(model):
    if model.fused:
        return lambda l: model.launch_down_combine(l, model.x, model.x_next)
    return model.launch_down


def copy_calibration(torch):
    """Three device copies of 1 GiB (known traffic: 1 GiB read, 1 GiB written): the scale of the
    FETCH_SIZE / WRITE_SIZE counters."""
    n = 1 << 28
    a, b = torch.empty(n, dtype=torch.float32, device="cuda"), torch.empty(n, dtype=torch.float32, device="cuda")
    a.fill_(1.0)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    return 4 * n


def traffic_probe(torch, model, md):
    """Kernels whose per-dispatch FETCH_SIZE / WRITE_SIZE a counter run reads: three copies of
    1 GiB (known traffic: 1 GiB read, 1 GiB written) and two gate/up GEMV launches per layer."""
    n = copy_calibration(torch) // 4
    ids_np, w_np = md.make_routing(1, model.L, model.E, model.U, seed=7)
    model.set_routing(torch.from_numpy(ids_np[0]).cuda(), torch.from_numpy(w_np[0]).cuda())
    model.launch_token()                     # builds every device table
    torch.cuda.synchronize()
    launch = gate_up_launcher(model)
    for _ in range(2):
        for l in range(model.L):
            launch(l)
    torch.cuda.synchronize()
    log(f"traffic probe done: copy {4 * n} bytes x3, gate/up GEMV x{2 * model.L}")


def read_floor(torch, model, md, rounds):
    """The cost of one fused gate/up launch's bytes with nothing else in the way (bench_floor.hip): every
    layer's GEMV steps (the same spans, routing, step list and 8-wave workgroups as the gate/up launch) only
    streamed into LDS; the same steps in one-wave workgroups; an empty launch of the same grid.  One graph
    of the model's layers each, timed like the kernels."""
    import numpy as np
    lib = C.CDLL(str(ROOT / "bench_floor.so"))
    lib.floor_launch.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_uint, C.c_uint, C.c_void_p, C.c_void_p]
    lib.floor_launch_empty.argtypes = [C.c_uint, C.c_uint, C.c_void_p]
    ids_np, _ = md.make_routing(1, model.L, model.E, model.U, seed=7)
    step_t = np.dtype([("gate", np.uint64), ("up", np.uint64), ("bytes", np.uint32), ("pad", np.uint32)])
    F, H = model.F, model.H
    rb, rbs = md.row_bytes(model.wtype, H), md.row_bytes(model.sh_type, H)
    rps, sh_rps = 4, 4                                   # the q8_1 hand-off's 32-row workgroups of 8 steps
    steps, nbytes = [], 0
    for l, ly in enumerate(model.layers):
        st = []
        for r0 in range(0, F, sh_rps):
            st.append((ly.sh_gate.data_ptr() + r0 * rbs, ly.sh_up.data_ptr() + r0 * rbs, sh_rps * rbs, 0))
        eb = rb * F
        for e in ids_np[0, l]:
            for r0 in range(0, F, rps):
                st.append((ly.gate.data_ptr() + int(e) * eb + r0 * rb, ly.up.data_ptr() + int(e) * eb + r0 * rb,
                           rps * rb, 0))
        a = np.array(st, dtype=step_t)
        nbytes = int(2 * a["bytes"].astype(np.int64).sum())
        steps.append(torch.from_numpy(a.view(np.uint8).copy()).cuda())
    max_bytes = max(sh_rps * rbs, rps * rb)
    region = 2 * (((max_bytes + 1024) + 1023) // 1024 * 1024)
    out = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    n_steps = steps[0].numel() // step_t.itemsize
    res = {"workload": f"bytes of one gate/up launch ({model.L} layers' own spans, {n_steps} GEMV steps of 4 rows, "
                       "gate + up each): buffer->LDS DMA with the non-temporal policy, then a wait; nothing else",
           "bytes_per_launch": nbytes}

    def launch(l, wpw):
        sp = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.floor_launch(steps[l].data_ptr(), n_steps, wpw, region, max_bytes, out.data_ptr(), sp)
        assert rc == 0, f"floor_launch returned {rc}"

    for wpw, key in ((8, "fused_layout"), (1, "one_wave_workgroups")):
        ms = graph_ms(torch, [lambda l=l, w=wpw: launch(l, w) for l in range(model.L)], rounds) / model.L
        res[key] = {"waves_per_workgroup": wpw, "workgroups": (n_steps + wpw - 1) // wpw, **_rate(nbytes, ms)}
    grid = (n_steps + 7) // 8

    def empty():
        rc = lib.floor_launch_empty(grid, 768, C.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, f"floor_launch_empty returned {rc}"
    res["empty_launch_us"] = round(graph_ms(torch, [empty] * model.L, rounds) / model.L * 1000, 3)
    return res


TRAFFIC_FILES = {True: "ffn_gate_up_norm_q2K_traffic.json", False: "gemv_gate_up_q2K_traffic.json"}
KERNEL_NAMES = {True: ("mc_ffn_gate_up_kernel<q2_K, q4_K shared> (RMSNorm + q8_1 of x, gate/up + SwiGLU)",
                       "mc_ffn_down_combine_kernel<q2_K, q4_K shared, q8_1> (down + weighted combine)"),
                False: ("mc_gemv_kernel<q2_K, q4_K shared, q8_1> (fused gate/up + SwiGLU)",
                        "mc_gemv_kernel<q2_K, q4_K shared, f32> (down)")}


def load_traffic(fused):
    """Per-launch HBM traffic of the plan's gate/up kernel from the committed counter summary, or None."""
    p = ROOT / "profiles" / TRAFFIC_FILES[fused]
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
        return int(d["hbm_bytes_per_launch"])
    except (ValueError, KeyError):
        return None


def cpu_baseline(torch, model, ids, w, budget_s=10.0, budget_1t_s=4.0, budget_scalar_s=4.0):
    """ggml-CPU MUL_MAT_ID restatement (oracle) over the last layer's weights (the mix's majority types), on
    this host's cores: AVX2 q8_K vec_dot (bit-identical to the scalar restatement) on all of them, then on one
    thread, then the scalar vec_dot on all of them."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    nth = int(os.environ.get("OMP_NUM_THREADS", "0")) or O.cpu_cores()
    li = model.L - 1
    ly = model.layers[li]
    mats = tuple(t.cpu().numpy() for t in (ly.gate, ly.up, ly.down, ly.sh_gate, ly.sh_up, ly.sh_down))
    layer_bytes = model.gate_up_bytes() + model.down_bytes(li) + model.combine_bytes()
    O.set_simd(True)
    n, el = _cpu_layer_loop(O, model, mats, ids, w, nth, budget_s)
    n1, el1 = _cpu_layer_loop(O, model, mats, ids, w, 1, budget_1t_s)
    O.set_simd(False)
    ns, els = _cpu_layer_loop(O, model, mats, ids, w, nth, budget_scalar_s)
    O.set_simd(True)
    gbs = lambda k, t: round(k * layer_bytes / t / 1e9, 3)
    return {"value": gbs(n, el), "unit": "GB/s", "cores": nth, "kind": "port",
            "sample": f"{n} layer-tokens of one MoE layer (512 experts Q2_K gate/up/down + Q4_K shared, B=1, "
                      f"fresh top-8 routing each) through the oracle's ggml-CPU MUL_MAT_ID restatement: q8_K "
                      f"activations, AVX2 vec_dot (bit-identical to the scalar restatement), chunked rows over "
                      f"{nth} OpenMP threads, GLU/combine unfused; {el:.1f} s",
            "layer_tok_per_s": round(n / el, 3),
            "one_thread": {"value": gbs(n1, el1), "unit": "GB/s", "cores": 1, "layer_tok_per_s": round(n1 / el1, 3),
                           "sample": f"{n1} layer-tokens, AVX2 vec_dot, one thread; {el1:.1f} s"},
            "scalar": {"value": gbs(ns, els), "unit": "GB/s", "cores": nth, "layer_tok_per_s": round(ns / els, 3),
                       "sample": f"{ns} layer-tokens, scalar vec_dot, {nth} threads; {els:.1f} s"}}


def _cpu_layer_loop(O, model, mats, ids, w, nth, budget_s):
    """Layer-tokens through the CPU restatement on nth threads until budget_s has passed:
    returns (layer-tokens, seconds)."""
    import numpy as np
    gate, up, down, sg, su, sd = mats
    H, F, U, E = model.H, model.F, model.U, model.E
    x = np.random.default_rng(1).standard_normal((1, H)).astype(np.float32)
    t0 = time.perf_counter()
    n = 0
    while True:
        tid = ids[n % len(ids), 0].reshape(1, U)
        g = O.cpu_mul_mat_id_f32(wtype=model.wtype, K=H, R=F, n_as=E, src0=gate, src1=x, ids=tid, nthreads=nth)
        u = O.cpu_mul_mat_id_f32(wtype=model.wtype, K=H, R=F, n_as=E, src0=up, src1=x, ids=tid, nthreads=nth)
        one = np.zeros((1, 1), np.int32)
        shg = O.cpu_mul_mat_id_f32(wtype=model.sh_type, K=H, R=F, n_as=1, src0=sg[None], src1=x, ids=one, nthreads=nth)
        shu = O.cpu_mul_mat_id_f32(wtype=model.sh_type, K=H, R=F, n_as=1, src0=su[None], src1=x, ids=one, nthreads=nth)
        hh = (u / (1.0 + np.exp(-g)) * g).reshape(1, U, F).astype(np.float32)        # SwiGLU up*silu(gate)
        hs = (shu / (1.0 + np.exp(-shg)) * shg).reshape(1, F).astype(np.float32)
        o = O.cpu_mul_mat_id_f32(wtype=model.down_types[-1], K=F, R=H, n_as=E, src0=down, src1=hh, ids=tid,
                                 nthreads=nth)
        os_ = O.cpu_mul_mat_id_f32(wtype=model.sh_type, K=F, R=H, n_as=1, src0=sd[None], src1=hs, ids=one, nthreads=nth)
        x = (x + os_[:, 0] + (w[n % len(w), 0][None, :, None] * o).sum(1)).astype(np.float32)
        x /= max(1.0, float(np.abs(x).max()))
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return n, el


def graph_ms(torch, launches, rounds):
    """Mean ms of one pass over `launches` (callables issuing kernels), captured as one graph and replayed
    `rounds` times between two events on the replay stream (host launch cost excluded)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in launches:                    # first use builds every device table
            f()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for f in launches:
                f()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(rounds):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / rounds


def _rate(nbytes, ms):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1000, 3), "bytes": int(nbytes), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}


def wl_decode_q4_0(torch, mc, md, rounds, cpu_s=3.0):
    """One decode MUL_MAT_ID: 64 experts Q4_0 [1024 x 2048], batch 1, top-8, q8_1 activations, all resident.
    16 copies of the 75 MB expert tensor rotate (1.2 GB) so the 256 MB MALL cannot serve repeat reads."""
    import numpy as np
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    E, K, R, U, copies = 64, 2048, 1024, 8, 16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    ws = [md.random_expert_tensor(torch, mc.Q4_0, E, R, K, gen) for _ in range(copies)]
    eb = mc.row_bytes(mc.Q4_0, K) * R
    x = torch.randn((1, K), generator=gen, device="cuda")
    y = mc.quantize_q8_1(x)
    ids_np, _ = md.make_routing(copies, 1, E, U, seed=12)
    ids = [torch.from_numpy(ids_np[i]).cuda() for i in range(copies)]
    dst = torch.zeros((1, U, R), dtype=torch.float32, device="cuda")
    launches = [lambda i=i: mc.mul_mat_vec(wtype=mc.Q4_0, weights=ws[i], ids=ids[i], y=y, dst=dst, K=K, R=R,
                                           n_experts=E) for i in range(copies)]
    ms = graph_ms(torch, launches, rounds) / copies
    nbytes = U * eb + y.numel() + U * R * 4
    out = {"workload": "decode MUL_MAT_ID GEMV, 64 experts Q4_0 [1024 x 2048], B=1, top-8, q8_1, resident",
           "kernel": "mc_gemv_kernel<q4_0, none, q8_1>", **_rate(nbytes, ms)}
    if cpu_s > 0:
        nth = int(os.environ.get("OMP_NUM_THREADS", "0")) or O.cpu_cores()
        w0, xs = ws[0].cpu().numpy(), x.cpu().numpy()
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < cpu_s:
            O.cpu_mul_mat_id_f32(wtype=mc.Q4_0, K=K, R=R, n_as=E, src0=w0, src1=xs, ids=ids_np[n % copies],
                                 nthreads=nth)
            n += 1
        el = (time.perf_counter() - t0) / n
        out["cpu_baseline"] = {"us_per_call": round(el * 1e6, 1), "GB/s": round(nbytes / el / 1e9, 2), "cores": nth,
                               "kind": "port", "sample": f"{n} calls of the oracle's ggml-CPU MUL_MAT_ID (AVX2 Q4_0 x q8_0 vec_dot) on copy 0"}
    del ws
    torch.cuda.empty_cache()
    return out


def wl_type_batch(torch, mc, md, rounds, batches=(1, 8)):
    """The 512-expert layer (hidden 4096, ffn 768, top-8) for Q4_0, Q5_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K experts at
    `batches` tokens: gate/up GEMV (SwiGLU, per-expert bias and scale on both projections) + down GEMV (bias and
    scale) from the fp32 GLU rows, 16 seeded routings per point.  Bytes = unique experts x (gate + up + down) +
    activations + outputs."""
    import numpy as np
    E, H, F, U, sets = 512, 4096, 768, 8, 16
    types = [("q4_0", mc.Q4_0), ("q5_0", mc.Q5_0), ("q8_0", mc.Q8_0), ("q3_K", mc.Q3_K), ("q4_K", mc.Q4_K),
             ("q5_K", mc.Q5_K), ("q6_K", mc.Q6_K)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    rng = np.random.default_rng(22)
    dev = lambda a: torch.from_numpy(a.astype(np.float32)).cuda()
    xb, gb = dev(rng.standard_normal((E, F)) * 0.1), dev(rng.standard_normal((E, F)) * 0.1)
    xs, gs = dev(rng.uniform(0.5, 1.5, E)), dev(rng.uniform(0.5, 1.5, E))
    db, ds = dev(rng.standard_normal((E, H)) * 0.1), dev(rng.uniform(0.5, 1.5, E))
    rows = []
    for name, t in types:
        gate = md.random_expert_tensor(torch, t, E, F, H, gen)
        up = md.random_expert_tensor(torch, t, E, F, H, gen)
        down = md.random_expert_tensor(torch, t, E, H, F, gen)
        eb_gu, eb_dn = mc.row_bytes(t, H) * F, mc.row_bytes(t, F) * H
        for B in batches:
            ids_np, _ = md.make_routing(sets * B, 1, E, U, seed=100 + B)
            ids_np = ids_np.reshape(sets, B, U)
            x = torch.randn((B, H), generator=gen, device="cuda")
            y = mc.quantize_q8_1(x)
            h = torch.zeros((B, U, F), dtype=torch.float32, device="cuda")
            o = torch.zeros((B, U, H), dtype=torch.float32, device="cuda")
            f_gu = mc.make_fusion(gate=gate, glu_op=mc.GLU_SWIGLU, x_bias=xb, gate_bias=gb, x_scale=xs, gate_scale=gs)
            f_dn = mc.make_fusion(x_bias=db, x_scale=ds)
            ids = [torch.from_numpy(np.ascontiguousarray(ids_np[i])).cuda() for i in range(sets)]

            def step(i):
                mc.mul_mat_vec(wtype=t, weights=up, ids=ids[i], y=y, dst=h, K=H, R=F, n_experts=E, fusion=f_gu)
                mc.mul_mat_vec(wtype=t, weights=down, ids=ids[i], y=h, dst=o, K=F, R=H, n_experts=E, fusion=f_dn,
                               act=mc.ACT_F32, nchannels_y=U)

            ms = graph_ms(torch, [lambda i=i: step(i) for i in range(sets)], rounds) / sets
            uniq = float(np.mean([len(np.unique(ids_np[i])) for i in range(sets)]))
            nbytes = uniq * (2 * eb_gu + eb_dn) + y.numel() + h.numel() * 8 + o.numel() * 4
            rows.append({"type": name, "batch": B, "unique_experts": round(uniq, 2), **_rate(nbytes, ms)})
            log(f"  type x batch: {name} B={B}: {rows[-1]['us']} us per layer, {rows[-1]['GB/s']} GB/s")
        del gate, up, down
        torch.cuda.empty_cache()
    return {"workload": "512-expert layer (hidden 4096, ffn 768, top-8), gate/up + SwiGLU + bias/scale GEMV and "
                        "down + bias/scale GEMV, per type and batch; us/bytes per layer",
            "points": rows}


def wl_prefill(torch, mc, md, rounds, wtype=None):
    """512 tokens x top-8 over 512 Q4_K experts (hidden 4096, ffn 768): q8_K of x, grouped int8-MFMA gate/up GEMM
    with SwiGLU, q8_K of the GLU rows, grouped down GEMM."""
    wtype = wtype if wtype is not None else mc.Q4_K
    E, H, F, U, T = 512, 4096, 768, 8, 512
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    gate = md.random_expert_tensor(torch, wtype, E, F, H, gen)
    up = md.random_expert_tensor(torch, wtype, E, F, H, gen)
    down = md.random_expert_tensor(torch, wtype, E, H, F, gen)
    ids_np, _ = md.make_routing(T, 1, E, U, seed=32)
    ids = torch.from_numpy(ids_np.reshape(T, U)).cuda()
    x = torch.randn((T, H), generator=gen, device="cuda")
    yx = torch.zeros(T * H // 256 * 292 + 256, dtype=torch.uint8, device="cuda")
    h = torch.zeros((T, U, F), dtype=torch.float32, device="cuda")
    yh = torch.zeros(T * U * F // 256 * 292 + 256, dtype=torch.uint8, device="cuda")
    o = torch.zeros((T, U, H), dtype=torch.float32, device="cuda")
    nws = max(int(mc.lib().ggml_hip_moe_mul_mat_q_workspace_bytes(H, E, T * U)),
              int(mc.lib().ggml_hip_moe_mul_mat_q_workspace_bytes(F, E, T * U)))
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    s = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def q_x():
        mc.check(mc.lib().ggml_hip_quantize_q8_K(x.data_ptr(), yx.data_ptr(), H, T, H, H // 256, s()), "q8_K x")

    def gu():
        mc.mul_mat_q(wtype=wtype, weights=up, gate=gate, ids=ids, y=yx, dst=h, K=H, R=F, n_experts=E, workspace=ws)

    def q_h():
        mc.check(mc.lib().ggml_hip_quantize_q8_K(h.data_ptr(), yh.data_ptr(), F, T * U, F, F // 256, s()), "q8_K h")

    def dn():
        mc.mul_mat_q(wtype=wtype, weights=down, ids=ids, y=yh, dst=o, K=F, R=H, n_experts=E, nchannels_y=U,
                     workspace=ws)

    ms_all = graph_ms(torch, [q_x, gu, q_h, dn], rounds)
    ms_gu = graph_ms(torch, [gu], rounds)
    ms_dn = graph_ms(torch, [dn], rounds)
    eb = mc.row_bytes(wtype, H) * F
    touched = len(set(ids_np.reshape(-1).tolist()))
    wbytes = touched * 3 * eb
    ops = 2 * T * U * 3 * F * H
    out = {"workload": f"prefill FFN, {T} tokens x top-{U} of {E} experts ({mc.TYPE_NAMES[wtype]}, hidden {H}, "
                       f"ffn {F}): q8_K activations, grouped int8-MFMA GEMMs; us/bytes per layer",
           **_rate(wbytes, ms_all), "us_gate_up": round(ms_gu * 1000, 1), "us_down": round(ms_dn * 1000, 1),
           "experts_touched": touched, "int8_ops": ops, "TOP/s": round(ops / (ms_all * 1e-3) / 1e12, 2),
           "mfma_frac": round(ops / (ms_all * 1e-3) / PEAK_INT8_OPS, 4), "tok_per_s": round(T / (ms_all * 1e-3), 1)}
    del gate, up, down, ws
    torch.cuda.empty_cache()
    return out


def wl_table_gate_up(torch, mc, md, rounds, layers=8, routings=4):
    """The pointer-table GEMV itself (ggml_hip_moe_cache_mul_mat_vec_q): gate/up + SwiGLU over 512 Q2_K experts
    (hidden 4096, ffn 768), top-8, B=1, every table entry LSB=0 (the pool holds every expert, seeded), the pick
    recorder on.  `layers` layers of gate/up tensors in pinned host memory, `routings` routings per layer, one
    graph of layers x routings launches (~530 MB of distinct expert reads per replay, past the MALL)."""
    import numpy as np
    import tempfile
    E, H, F, U = 512, 4096, 768, 8
    t = mc.Q2_K
    eb = mc.row_bytes(t, H) * F
    gen = torch.Generator(device="cuda")
    gen.manual_seed(51)
    keep, tens = [], {}
    seed_path = os.path.join(tempfile.mkdtemp(), "moe_seed_all.txt")
    all_ids = ",".join(str(e) for e in range(E))
    with open(seed_path, "w") as f:
        for l in range(layers):
            for role in ("gate", "up"):
                f.write(f"blk.{l}.ffn_{role}_exps.weight {all_ids}\n")
    for l in range(layers):
        for role in ("gate", "up"):
            dev = md.random_expert_tensor(torch, t, E, F, H, gen)
            p = torch.empty(E * eb, dtype=torch.uint8, pin_memory=True)
            p.copy_(dev.view(-1))
            del dev
            keep.append(p)
            tens[(l, role)] = mc.make_tensor(t, H, F, E, p.data_ptr(), name=f"blk.{l}.ffn_{role}_exps.weight", keep=keep)
    mc.reset()
    mc.configure(enabled=True, slots=-1, budget_gb=0.0, margin_gb=2.0, seed_path=seed_path, max_promotions=48)
    ids_np, _ = md.make_routing(routings, layers, E, U, seed=52)
    ids = torch.from_numpy(ids_np).cuda()                      # [routings, layers, U]
    x = torch.randn((1, H), generator=gen, device="cuda")
    y = mc.quantize_q8_1(x)
    h = torch.zeros((1, U, F), dtype=torch.float32, device="cuda")
    lib, ar = mc.lib(), H // 32

    def launch(r, l):
        sp = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        mc.check(lib.ggml_hip_moe_cache_mul_mat_vec_q(
            C.byref(tens[(l, "up")]), C.byref(tens[(l, "gate")]), None, y.data_ptr(), ids[r, l].data_ptr(),
            h.data_ptr(), H, F, E, 1, 1, H // 256, eb, eb * E, 1, U, ar, U * F, ar, F, U, sp), "table gate/up")

    ms = graph_ms(torch, [lambda r=r, l=l: launch(r, l) for r in range(routings) for l in range(layers)],
                  rounds) / (routings * layers)
    stats = mc.stats_snapshot(2)
    assert int(stats[0]) == 0, f"all-hit run recorded {int(stats[0])} misses"
    nbytes = 2 * U * eb + y.numel() + U * F * 4
    out = {"workload": "pointer-table GEMV (cache path), gate/up + SwiGLU, 512 Q2_K experts [768 x 4096], top-8, "
                       "B=1, every table entry in the HBM pool (LSB=0), pick recorder on",
           "kernel": "mc_gemv_kernel<q2_K, none, q8_1> with tbl/tbl_gate, stamps and stats",
           **_rate(nbytes, ms), "misses": int(stats[0]), "hits_recorded": int(stats[1])}
    mc.reset()
    del keep
    torch.cuda.empty_cache()
    return out


def wl_cache_mixed(torch, mc, md, rounds, layers=40, tokens=128, calib_tokens=16):
    """The pointer-table cache under mixed residency (bench_configs.cfg3_runs): Q2_K gate/up/down experts of up
    to 40 layers (as many as the host lets the GPU map) in pinned host memory, a 435/512 HBM pool per tensor,
    Zipf(1.1) routing, the cache step between tokens; all-hit and all-miss calibrations beside it."""
    sys.path.insert(0, str(ROOT))
    from bench_configs import cfg3_runs
    hit, miss, mix = cfg3_runs(torch, mc, md, tokens=tokens, calib_tokens=calib_tokens, layers=layers,
                               async_run=False)
    torch.cuda.empty_cache()
    keys = ("tokens", "hit_rate", "promotions", "us_per_token_gpu", "us_per_token_step", "us_per_token_wall",
            "tok_per_s_gpu", "tok_per_s_with_step", "HBM_GB/s_hits", "PCIe_GB/s_misses", "us_per_layer_gpu")
    return {"workload": f"pointer-table cache under mixed residency: {mix['layers']} layers of 512 Q2_K gate/up/down "
                        "experts (hidden 4096, ffn 768) in pinned host memory, 435/512 per tensor in the HBM pool "
                        "(seeded), Zipf(1.1) top-8 routing, B=1, miss log + LRU step (48 promotions) between tokens",
            "layers": mix["layers"], **{k: mix[k] for k in keys},
            "calibration": {"all_hit_HBM_GB/s": hit["HBM_GB/s"], "all_hit_us_per_token": hit["us_per_token_gpu"],
                            "all_miss_PCIe_GB/s": miss["PCIe_GB/s"], "all_miss_us_per_token": miss["us_per_token_gpu"]}}


WORKLOADS = {"decode_q4_0": wl_decode_q4_0, "type_batch": wl_type_batch, "prefill": wl_prefill,
             "cache_mixed": wl_cache_mixed, "table_gate_up": wl_table_gate_up}


def run_workloads(torch, mc, md, names, args):
    """The secondary workloads, each as one entry: us / bytes / GB/s / frac of its dominant unit."""
    res = {}
    for name in names:
        t0 = time.perf_counter()
        fn = WORKLOADS[name]
        res[name] = fn(torch, mc, md, args.kernel_rounds) if name != "decode_q4_0" else \
            fn(torch, mc, md, args.kernel_rounds, cpu_s=0.0 if args.no_cpu else 3.0)
        r = res[name]
        log(f"workload {name}: " + (f"{r['us']} us, {r['GB/s']} GB/s" if "us" in r else
                                     f"hit rate {r['hit_rate']}, {r['us_per_token_wall']} us/token with the step"
                                     if "hit_rate" in r else "done") +
            f" ({time.perf_counter() - t0:.1f}s)")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-rounds", type=int, default=10)
    ap.add_argument("--plan", choices=("fused", "ops"), default="fused",
                    help="fused: 2 launches per layer (default); ops: gate/up, down, combine launches")
    ap.add_argument("--shared-rows", choices=("q8_1", "f32"), default="q8_1",
                    help="fused plan: the gate/up launch writes the shared expert's q8_1 row (q8_1), or only its "
                         "fp32 row, quantized by the down launch, with byte-balanced shared workgroups (f32)")
    ap.add_argument("--mix", choices=("q2_K_s", "pure"), default="q2_K_s",
                    help="routed expert types: llama.cpp's Q2_K_S mix (the first n_layer/8 layers' ffn_down in "
                         "Q4_K, the rest Q2_K; default) or Q2_K everywhere")
    ap.add_argument("--act", choices=("q8_1", "q8_K"), default="q8_1",
                    help="fused plan: the dots' activations, q8_1 (ggml-CUDA MMVQ, the reference's path) or q8_K "
                         "(ggml-CPU MUL_MAT_ID for K-quant experts)")
    ap.add_argument("--hand-off", choices=("q8_1", "f32"), default="q8_1",
                    help="fused plan, q8_1 dots: the gate/up launch hands the GLU rows to the down launch as q8_1 "
                         "blocks (default) or as fp32 rows that every down wave quantizes to q8_1")
    ap.add_argument("--read-floor", action="store_true",
                    help="time the gate/up launch's bytes alone (bench_floor.hip: the same spans and workgroups, "
                         "DMA only) and an empty launch, then exit")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: a 1 GiB copy (the counter calibration) and the gate/up "
                         "GEMV of every layer, then exit")
    ap.add_argument("--workloads", default="all",
                    help="secondary workloads measured after the decode step, comma-separated from "
                         f"{','.join(WORKLOADS)} (default all; none: skip)")
    ap.add_argument("--skip-decode", action="store_true",
                    help="measure only the secondary workloads (for per-kernel profiles); prints their JSON")
    args = ap.parse_args()
    wl_names = [] if args.workloads == "none" else list(WORKLOADS) if args.workloads == "all" else \
        [w for w in args.workloads.split(",") if w]
    for w in wl_names:
        if w not in WORKLOADS:
            ap.error(f"unknown workload {w!r}")
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not run "
              "(the multi-GPU sharding is a design note, not a measured configuration)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    mc = load_package()
    from importlib import import_module
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    assert torch.cuda.is_available(), "bench.py needs a HIP device"

    if args.skip_decode:
        if args.traffic_probe:                # counter calibration first: 1 GiB copies of known traffic
            copy_calibration(torch)
        print(json.dumps({"workloads": run_workloads(torch, mc, md, wl_names, args)}), flush=True)
        return
    t0 = time.perf_counter()
    fused = args.plan == "fused"
    model = md.MoeDecodeModel(torch, n_layers=args.layers, fused=fused, shared_q8=args.shared_rows == "q8_1",
                              act=args.act if fused else "q8_1", mix=args.mix, hand_off=args.hand_off)
    torch.cuda.synchronize()
    log(f"weights ready: {args.layers} layers in {time.perf_counter() - t0:.1f}s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")
    if args.traffic_probe:
        traffic_probe(torch, model, md)
        return
    if args.read_floor:
        print(json.dumps({"read_floor": read_floor(torch, model, md, args.kernel_rounds)}), flush=True)
        return
    n_tok_routes = max(64, args.warmup + args.steps)
    ids_np, w_np = md.make_routing(n_tok_routes, model.L, model.E, model.U, seed=7)
    ids_dev = torch.from_numpy(ids_np).cuda()
    w_dev = torch.from_numpy(w_np).cuda()
    x0 = torch.from_numpy(np.random.default_rng(3).standard_normal((1, model.H)).astype(np.float32)).cuda()

    model.x.copy_(x0)
    model.set_routing(ids_dev[0], w_dev[0])
    model.capture()
    for i in range(args.warmup):
        model.set_routing(ids_dev[i % n_tok_routes], w_dev[i % n_tok_routes])
        model.replay()
    torch.cuda.synchronize()
    assert torch.isfinite(model.x).all() and torch.isfinite(model.x_next).all(), "non-finite residual stream"

    # timed region: K tokens
    s = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    ev0.record(s)
    for i in range(args.steps):
        j = (args.warmup + i) % n_tok_routes
        model.set_routing(ids_dev[j], w_dev[j])
        model.replay()
    ev1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_total = ev0.elapsed_time(ev1)
    ms_per_tok = ms_total / args.steps
    tok_s = 1000.0 / ms_per_tok
    bpt = model.bytes_per_token()
    gbs = bpt * tok_s / 1e9
    log(f"decode: {ms_per_tok * 1000:.1f} us/token, {tok_s:.1f} tok/s, {gbs:.1f} GB/s (wall {wall:.2f}s)")

    # dominant kernel: the gate/up GEMV (+ shared gate/up), per-launch events on its stream
    gu_ms, n_launch = time_kernel(torch, model, gate_up_launcher(model), args.kernel_rounds)
    dn_ms, _ = time_kernel(torch, model, down_launcher(model), args.kernel_rounds)
    gu_bytes, dn_bytes = model.gate_up_bytes(), model.down_bytes()
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    dn_gbs = dn_bytes / (dn_ms * 1e-3) / 1e9
    log(f"gate/up: {gu_ms * 1000:.2f} us/launch ({n_launch} launches), {gu_gbs:.0f} GB/s; "
        f"down: {dn_ms * 1000:.2f} us/launch, {dn_gbs:.0f} GB/s")

    # the other activation format of the fused plan, on the same weights and routes
    modes = {}
    if fused:
        main = (model.act, model.hand_off if model.act == "q8_1" else "f32")
        for name, act, hand_off in (("q8_1", "q8_1", "q8_1"), ("q8_K", "q8_K", "f32"),
                                    ("q8_1, fp32 hand-off", "q8_1", "f32")):
            if (act, hand_off) == main:
                continue
            model.act, model.hand_off = act, hand_off
            model.x.copy_(x0)
            model.set_routing(ids_dev[0], w_dev[0])
            model.capture()
            for i in range(args.warmup):
                model.set_routing(ids_dev[i % n_tok_routes], w_dev[i % n_tok_routes])
                model.replay()
            n2 = max(1, args.steps // 2)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for i in range(n2):
                j = (args.warmup + i) % n_tok_routes
                model.set_routing(ids_dev[j], w_dev[j])
                model.replay()
            e1.record(s)
            torch.cuda.synchronize()
            ms2 = e0.elapsed_time(e1) / n2
            g2, _ = time_kernel(torch, model, gate_up_launcher(model), args.kernel_rounds)
            d2, _ = time_kernel(torch, model, down_launcher(model), args.kernel_rounds)
            modes[name] = {"ms_per_step": round(ms2, 4), "tok_per_s": round(1000.0 / ms2, 2), "steps": n2,
                          "gate_up_us_per_launch": round(g2 * 1000, 3), "down_us_per_launch": round(d2 * 1000, 3),
                          "gate_up_bytes_per_launch": model.gate_up_bytes(),
                          "down_bytes_per_launch": model.down_bytes()}
            log(f"{name}: {ms2 * 1000:.1f} us/token, gate/up {g2 * 1000:.2f} us, down {d2 * 1000:.2f} us")
        model.act = main[0]
        model.hand_off = main[1] if main[0] == "q8_1" else args.hand_off

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, model, ids_np, w_np)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads (AVX2), "
            f"{cpu['one_thread']['value']} GB/s on 1 thread, scalar {cpu['scalar']['value']} GB/s")

    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_tok, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random valid Q2_K/Q4_K blocks, N(0,1) input, uniform top-8, softmax router weights)",
        "config": {"workload": f"{model.L}-layer MoE decode step, B=1: 512 experts, hidden 4096, expert ffn 768, "
                               "top-8, " + ("Q2_K_S expert mix (Q2_K gate/up, Q2_K down except the first "
                                            f"{model.L // 8} layers' in Q4_K)" if model.mix == "q2_K_s" else
                                            "Q2_K routed gate/up/down") +
                               " + Q4_K shared expert, fused SwiGLU, all resident",
                   "mix": model.mix,
                   "layers": model.L, "experts": model.E, "hidden": model.H, "ffn": model.F, "top_k": model.U,
                   "routed_type": "q2_K", "shared_type": "q4_K", "batch": 1,
                   "plan": f"{args.plan}: {2 if fused else 3} launches per layer",
                   "shared_rows": args.shared_rows, "activations": model.act,
                   "hand_off": "fp32 rows" if model.f32_rows else "q8_1 rows"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "tok_per_s": round(tok_s, 2),
        "bytes_per_step": bpt,
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": load_traffic(fused),
                     "kernel": KERNEL_NAMES[fused][0],
                     "bytes_per_launch": gu_bytes, "us_per_launch": round(gu_ms * 1000, 3)},
        "kernels": {"down": {"kernel": KERNEL_NAMES[fused][1], "bytes_per_launch": dn_bytes,
                             "us_per_launch": round(dn_ms * 1000, 3), "GB/s": round(dn_gbs, 1)}},
        "cpu_baseline": cpu,
    }
    if modes:
        out["other_activation_modes"] = modes
    if wl_names:
        del model                             # 71 GiB of decode weights are not needed below
        torch.cuda.empty_cache()
        out["workloads"] = run_workloads(torch, mc, md, wl_names, args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
