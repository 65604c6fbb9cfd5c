#!/usr/bin/env python3
"""Benchmark: pointer-table quantized MoE GEMV on one MI355X.

Workload (one "step" = one decode token): the MoE block of a 48-layer model
shaped like the reference's (512 experts, hidden 4096, expert FFN 768, top-8
routing with softmax router weights, Q2_K routed experts, one always-on Q4_K
shared expert, fused SwiGLU), batch 1, every layer with its own weights
(~76 GB resident in HBM, so the 256 MB MALL cannot serve repeat reads).  One
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
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "a6000-custom-kernels_amd"
PEAK_HBM_GBS = 8000.0
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


def traffic_probe(torch, model, md):
    """Kernels whose per-dispatch FETCH_SIZE / WRITE_SIZE a counter run reads: three copies of
    1 GiB (known traffic: 1 GiB read, 1 GiB written) and two gate/up GEMV launches per layer."""
    n = 1 << 28
    a, b = torch.empty(n, dtype=torch.float32, device="cuda"), torch.empty(n, dtype=torch.float32, device="cuda")
    a.fill_(1.0)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
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


def cpu_baseline(torch, model, ids, w, budget_s=12.0, budget_1t_s=6.0):
    """ggml-CPU MUL_MAT_ID restatement (oracle) over layer 0's weights, on this host's cores
    (all of them, then one thread)."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    nth = int(os.environ.get("OMP_NUM_THREADS", "0")) or O.cpu_cores()
    ly = model.layers[0]
    mats = tuple(t.cpu().numpy() for t in (ly.gate, ly.up, ly.down, ly.sh_gate, ly.sh_up, ly.sh_down))
    layer_bytes = model.bytes_per_token() / model.L
    n, el = _cpu_layer_loop(O, model, mats, ids, w, nth, budget_s)
    n1, el1 = _cpu_layer_loop(O, model, mats, ids, w, 1, budget_1t_s)
    return {"value": round(n * layer_bytes / el / 1e9, 3), "unit": "GB/s", "cores": nth, "kind": "port",
            "sample": f"{n} layer-tokens of the same MoE layer (512 experts Q2_K gate/up/down + Q4_K shared, "
                      f"B=1, fresh top-8 routing each) through the oracle's ggml-CPU MUL_MAT_ID restatement "
                      f"(q8_K activations, scalar vec_dot, OpenMP rows), GLU/combine unfused; {el:.1f} s",
            "layer_tok_per_s": round(n / el, 3),
            "one_thread": {"value": round(n1 * layer_bytes / el1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                           "layer_tok_per_s": round(n1 / el1, 3),
                           "sample": f"{n1} layer-tokens of the same layer and routing stream; {el1:.1f} s"}}


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
        o = O.cpu_mul_mat_id_f32(wtype=model.wtype, K=F, R=H, n_as=E, src0=down, src1=hh, ids=tid, nthreads=nth)
        os_ = O.cpu_mul_mat_id_f32(wtype=model.sh_type, K=F, R=H, n_as=1, src0=sd[None], src1=hs, ids=one, nthreads=nth)
        x = (x + os_[:, 0] + (w[n % len(w), 0][None, :, None] * o).sum(1)).astype(np.float32)
        x /= max(1.0, float(np.abs(x).max()))
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return n, el


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
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: a 1 GiB copy (the counter calibration) and the gate/up "
                         "GEMV of every layer, then exit")
    args = ap.parse_args()
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

    t0 = time.perf_counter()
    fused = args.plan == "fused"
    model = md.MoeDecodeModel(torch, n_layers=args.layers, fused=fused)
    torch.cuda.synchronize()
    log(f"weights ready: {args.layers} layers in {time.perf_counter() - t0:.1f}s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")
    if args.traffic_probe:
        traffic_probe(torch, model, md)
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

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, model, ids_np, w_np)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads, "
            f"{cpu['one_thread']['value']} GB/s on 1 thread")

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
                               "top-8, Q2_K routed gate/up/down + Q4_K shared expert, fused SwiGLU, all resident",
                   "layers": model.L, "experts": model.E, "hidden": model.H, "ffn": model.F, "top_k": model.U,
                   "routed_type": "q2_K", "shared_type": "q4_K", "batch": 1,
                   "plan": f"{args.plan}: {2 if fused else 3} launches per layer"},
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
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
