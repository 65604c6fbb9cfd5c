#!/usr/bin/env python3
"""Measurements of the secondary MoE workloads on one MI355X, one JSON line each.

  cfg1   one decode MUL_MAT_ID: 64 experts, Q4_0 [1024 x 2048], batch 1, top-8,
         q8_1 activations, all resident, no cache (16 copies of the expert tensor
         rotate so that the 256 MB MALL cannot serve repeat reads);
  cfg4   the 512-expert, hidden 4096, ffn 768 layer at batch 1/2/4/8 for Q4_0,
         Q5_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K: fused gate/up GEMV (SwiGLU, per-expert
         bias and scale on both projections) + down GEMV (bias and scale), 16
         seeded routings per point;
  cfg5a  the prefill-shaped FFN: 512 tokens x top-8 over 512 Q4_K experts through
         the expert-grouped int8-MFMA path (q8_K of x, gate/up + SwiGLU, q8_K of
         the GLU rows, down).

Kernel times come from graph replays timed with HIP events on the replay
stream, so host launch cost is excluded.  Bytes are algorithmic: the unique
expert matrices a launch touches plus activations and outputs.  cpu_baseline
(cfg1) is the CPU oracle's ggml-CPU MUL_MAT_ID restatement on this host.

Usage: python bench_configs.py [--configs cfg1,cfg4,cfg5a] [--rounds N]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from importlib import import_module
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
from bench import PEAK_HBM_GBS, load_package, log  # noqa: E402

PEAK_INT8_OPS = 5.0e15        # MI355X dense int8 MFMA


def graph_ms(torch, launches, rounds):
    """Mean ms of one pass over all of `launches` (callables issuing kernels), replayed as one graph."""
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


def emit(obj):
    print(json.dumps(obj), flush=True)


def cfg1(torch, mc, md, rounds):
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
    gbs = nbytes / (ms * 1e-3) / 1e9
    # CPU: the oracle's ggml-CPU MUL_MAT_ID on copy 0 (weights copied to the host), all cores
    nth = int(os.environ.get("OMP_NUM_THREADS", "0")) or O.cpu_cores()
    w0 = ws[0].cpu().numpy()
    xs = x.cpu().numpy()
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < 5.0:
        O.cpu_mul_mat_id_f32(wtype=mc.Q4_0, K=K, R=R, n_as=E, src0=w0, src1=xs, ids=ids_np[n % copies], nthreads=nth)
        n += 1
    cpu_s = (time.perf_counter() - t0) / n
    emit({"config": "cfg1", "workload": "MUL_MAT_ID decode, 64 experts Q4_0 [1024 x 2048], B=1, top-8, q8_1, resident",
          "us_per_launch": round(ms * 1000, 3), "bytes_per_launch": nbytes, "GB/s": round(gbs, 1),
          "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
          "cpu_baseline": {"us_per_call": round(cpu_s * 1e6, 1), "GB/s": round(nbytes / cpu_s / 1e9, 2),
                           "cores": nth, "kind": "port", "sample": f"{n} calls on copy 0"}})


def cfg4(torch, mc, md, rounds):
    import numpy as np
    E, H, F, U, sets = 512, 4096, 768, 8, 16
    types = [("q4_0", mc.Q4_0), ("q5_0", mc.Q5_0), ("q8_0", mc.Q8_0), ("q3_K", mc.Q3_K), ("q4_K", mc.Q4_K),
             ("q5_K", mc.Q5_K), ("q6_K", mc.Q6_K)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    rng = np.random.default_rng(22)
    xb = torch.from_numpy((rng.standard_normal((E, F)) * 0.1).astype(np.float32)).cuda()
    gb = torch.from_numpy((rng.standard_normal((E, F)) * 0.1).astype(np.float32)).cuda()
    xs = torch.from_numpy(rng.uniform(0.5, 1.5, E).astype(np.float32)).cuda()
    gs = torch.from_numpy(rng.uniform(0.5, 1.5, E).astype(np.float32)).cuda()
    db = torch.from_numpy((rng.standard_normal((E, H)) * 0.1).astype(np.float32)).cuda()
    ds = torch.from_numpy(rng.uniform(0.5, 1.5, E).astype(np.float32)).cuda()
    for name, t in types:
        gate = md.random_expert_tensor(torch, t, E, F, H, gen)
        up = md.random_expert_tensor(torch, t, E, F, H, gen)
        down = md.random_expert_tensor(torch, t, E, H, F, gen)
        eb_gu, eb_dn = mc.row_bytes(t, H) * F, mc.row_bytes(t, F) * H
        for B in (1, 2, 4, 8):
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
            uniq = np.mean([len(np.unique(ids_np[i])) for i in range(sets)])
            nbytes = uniq * (2 * eb_gu + eb_dn) + y.numel() + h.numel() * 8 + o.numel() * 4
            gbs = nbytes / (ms * 1e-3) / 1e9
            emit({"config": "cfg4", "type": name, "batch": B, "unique_experts": round(float(uniq), 2),
                  "us_per_layer": round(ms * 1000, 3), "bytes_per_layer": int(nbytes), "GB/s": round(gbs, 1),
                  "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2)})
        del gate, up, down
        torch.cuda.empty_cache()


def cfg5a(torch, mc, md, rounds):
    E, H, F, U, T = 512, 4096, 768, 8, 512
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    gate = md.random_expert_tensor(torch, mc.Q4_K, E, F, H, gen)
    up = md.random_expert_tensor(torch, mc.Q4_K, E, F, H, gen)
    down = md.random_expert_tensor(torch, mc.Q4_K, E, H, F, gen)
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
        mc.mul_mat_q(wtype=mc.Q4_K, weights=up, gate=gate, ids=ids, y=yx, dst=h, K=H, R=F, n_experts=E, workspace=ws)

    def q_h():
        mc.check(mc.lib().ggml_hip_quantize_q8_K(h.data_ptr(), yh.data_ptr(), F, T * U, F, F // 256, s()),
                 "q8_K h")

    def dn():
        mc.mul_mat_q(wtype=mc.Q4_K, weights=down, ids=ids, y=yh, dst=o, K=F, R=H, n_experts=E, nchannels_y=U,
                     workspace=ws)

    ms_all = graph_ms(torch, [q_x, gu, q_h, dn], rounds)
    ms_gu = graph_ms(torch, [gu], rounds)
    ms_dn = graph_ms(torch, [dn], rounds)
    eb = mc.row_bytes(mc.Q4_K, H) * F
    touched = len(set(ids_np.reshape(-1).tolist()))
    wbytes = touched * 3 * eb
    ops = 2 * T * U * 3 * F * H
    gbs = wbytes / (ms_all * 1e-3) / 1e9
    emit({"config": "cfg5a", "workload": "prefill FFN, 512 tokens x top-8 of 512 Q4_K experts (hidden 4096, ffn 768), "
                                         "q8_K activations, int8 MFMA grouped GEMM",
          "us_per_layer": round(ms_all * 1000, 1), "us_gate_up": round(ms_gu * 1000, 1),
          "us_down": round(ms_dn * 1000, 1), "experts_touched": touched, "weight_bytes": wbytes,
          "GB/s": round(gbs, 1), "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
          "int8_ops": ops, "TOP/s": round(ops / (ms_all * 1e-3) / 1e12, 2),
          "mfma_frac": round(ops / (ms_all * 1e-3) / PEAK_INT8_OPS, 4),
          "tok_per_s": round(T / (ms_all * 1e-3), 1)})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="cfg1,cfg4,cfg5a")
    ap.add_argument("--rounds", type=int, default=10)
    args = ap.parse_args()
    import torch
    mc = load_package()
    md = import_module("a6000_custom_kernels_amd.moe_decode")
    assert torch.cuda.is_available(), "bench_configs.py needs a HIP device"
    for name in args.configs.split(","):
        log(f"running {name}")
        {"cfg1": cfg1, "cfg4": cfg4, "cfg5a": cfg5a}[name](torch, mc, md, args.rounds)


if __name__ == "__main__":
    main()
