#!/usr/bin/env python3
"""
Benchmark: int4 MoE-layer decode tok/s + % of HBM roofline, OLMoE shape, bs=1, one MI355X.

Workload (the OLMoE-shaped 16-layer MoE stack at batch 1, all experts int4 gs64 and resident):
d_model 2048, 64 experts per layer, softmax router top-8 without renormalisation, SwiGLU d_ff
1024, router weights and expert weights N(0, 0.02) (experts quantised int4 gs64 absmax on the
GPU with moelab's packing), fp16 hidden states N(0, 1), one seeded state per (token, layer).
A step = one decode token through the 16 MoE layers: per layer router -> HOBBIT table ->
kernel A -> kernel B -> combine, all on the GPU, replayed as one HIP graph per token. 16 x 64 int4
records = 3.42 GB, far above the 256 MB Infinity Cache, and each token routes differently.

Roofline: the dominant kernel is kernel A (gate/up GEMV over the 8 routed records); its
algorithmic bytes per launch = 8 x (gate_up.q + gate_up.s) + x + h, its duration is measured live
with HIP events on the stream it runs on, over launches that rotate through all layers.

CPU baseline: the oracle's restatement of moelab's CPU expert branch (dequantise to fp32,
F.linear-equivalent matvecs, weighted sum) on a bounded sample of the same workload, host cores.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "moe-offload-lab_amd"))

H, I, E, K_TOP, L = 2048, 1024, 64, 8, 16
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_workload(dev, n_tokens: int, seed: int = 0):
    import torch

    from moelab_hip.layer import MoEDecoder, ResidentStore
    from moelab_hip.policy import PrecisionPolicy
    from moelab_hip.store import record_layout

    g = torch.Generator(device=dev).manual_seed(seed)
    lay = record_layout("int4", H, I, 64, scale="absmax")
    store = ResidentStore({"int4": lay}, L, E, dev)
    t0 = time.time()
    store.fill_synthetic(g, std=0.02)
    torch.cuda.synchronize()
    log(f"[bench] encoded {L * E} int4 records ({store.bytes_resident / 1e9:.2f} GB) in {time.time() - t0:.1f} s")
    Wr = [(torch.randn(E, H, device=dev, generator=g) * 0.02).half() for _ in range(L)]
    xs = torch.randn(n_tokens, L, 1, H, device=dev, generator=g).half()
    dec = MoEDecoder(store, K_TOP, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    return store, dec, xs, Wr, lay


def gpu_bench(args):
    import torch

    from moelab_hip import _lib
    from moelab_hip.kernels import _Plan

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    S = args.tokens
    store, dec, xs, Wr, lay = build_workload(dev, S)
    outs = torch.zeros(S, L, 1, H, dtype=torch.float16, device=dev)

    def token(s):
        for l in range(L):
            dec.layer(l, xs[s, l], outs[s, l])

    # eager run of every token, then one graph per token
    for s in range(S):
        token(s)
    torch.cuda.synchronize()
    graphs = []
    for s in range(S):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            token(s)
        graphs.append(gr)
    torch.cuda.synchronize()
    ref_out = outs.clone()
    for s in range(S):
        graphs[s].replay()
    torch.cuda.synchronize()
    if not torch.equal(outs, ref_out):
        raise RuntimeError("graph replay differs from the eager run")
    if dec.miss.item() != 0:
        raise RuntimeError("experts missing from the resident store")

    for i in range(args.warmup):
        graphs[i % S].replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    for i in range(args.steps):
        graphs[i % S].replay()
    b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = a.elapsed_time(b)
    ms_step = ms_total / args.steps
    log(f"[bench] {args.steps} tokens x {L} layers: {ms_step * 1000:.1f} us/token ({wall:.2f} s wall)")

    # --- dominant kernel (A) timed live with HIP events on its stream -------------------
    # routing tables for every (token, layer) are prepared first, then kernel A alone is
    # launched back to back, rotating over tokens and layers, between two events.
    plan: _Plan = dec.plans[0]
    tabs, wts = [], []
    for s in range(S):
        for l in range(L):
            dec.layer(l, xs[s, l], outs[s, l])
            tabs.append(dec.tab[0].clone())
            wts.append(dec.wtab[0].clone())
    torch.cuda.synchronize()
    h = torch.empty(K_TOP, I, dtype=torch.float32, device=dev)
    acc = torch.empty(H, dtype=torch.float32, device=dev)
    nA = len(tabs)
    reps = max(1, args.kernel_launches // nA)
    st = torch.cuda.current_stream(dev)
    for j in range(nA):
        plan.up(K_TOP, tabs[j], wts[j], xs[j // L, j % L], h, acc, zero=False)
    ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ea.record(st)
    for _ in range(reps):
        for j in range(nA):
            plan.up(K_TOP, tabs[j], wts[j], xs[j // L, j % L], h, acc, zero=False)
    eb.record(st)
    torch.cuda.synchronize()
    upA_us = ea.elapsed_time(eb) * 1000 / (reps * nA)
    # kernel B (+ its ordered reduce) the same way
    part = plan.partial(K_TOP, dev)
    ea.record(st)
    for _ in range(reps):
        for j in range(nA):
            plan.down(K_TOP, tabs[j], wts[j], h, acc)
    eb.record(st)
    torch.cuda.synchronize()
    downB_us = ea.elapsed_time(eb) * 1000 / (reps * nA)

    gu_bytes = 2 * I * (H // 2) + 2 * I * (H // 64) * 2  # gate_up.q + gate_up.s of one record
    dn_bytes = H * (I // 2) + H * (I // 64) * 2
    rec_bytes = gu_bytes + dn_bytes
    bytes_A = K_TOP * gu_bytes + H * 2 + K_TOP * I * 4
    layer_alg = K_TOP * rec_bytes + E * H * 2 + 2 * H * 2  # experts + router + x/out
    achieved_A = bytes_A / (upA_us * 1e-6) / 1e9
    tok_s = 1000.0 / ms_step
    layer_us = ms_step * 1000 / L
    return {
        "tok_s": tok_s, "ms_step": ms_step, "layer_us": layer_us,
        "layer_tok_s": tok_s * L,
        "expert_gbs": K_TOP * rec_bytes / (layer_us * 1e-6) / 1e9,
        "layer_alg_gbs": layer_alg / (layer_us * 1e-6) / 1e9,
        "kernelA_us": upA_us, "kernelB_us": downB_us,
        "kernelA_bytes": bytes_A, "kernelA_gbs": achieved_A,
        "kernelB_gbs": (K_TOP * dn_bytes + K_TOP * I * 4 + K_TOP * H * 4) / (downB_us * 1e-6) / 1e9,
        "layer_bytes": layer_alg, "record_bytes": rec_bytes,
    }


def cpu_baseline(seconds: float):
    """The oracle's CPU expert path (moelab/runtime.py:646-702) on a bounded sample."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    import oracle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max([t.get("num_threads", 1) for t in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        threads = 1
    rng = np.random.default_rng(0)
    lay = O.record_layout("int4", H, I, 64, scale="absmax")
    n_rec = 8
    t0 = time.time()
    blobs = [O.encode_record(lay, (rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32),
                             (rng.standard_normal((H, I)) * 0.02).astype(np.float32), "absmax") for _ in range(n_rec)]
    log(f"[bench] cpu baseline: {n_rec} records encoded in {time.time() - t0:.1f} s")
    x = rng.standard_normal((1, H)).astype(np.float16).astype(np.float32)
    ents = [("int4", blobs[j], 0.125) for j in range(K_TOP)]
    O.cpu_expert_path(x, ents[:1], {"int4": lay})  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        O.cpu_expert_path(x, ents, {"int4": lay})
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    per_layer = el / n
    return {"value": 1.0 / per_layer, "unit": "layer-tok/s", "cores": int(threads), "kind": "port",
            "sample": f"{n} token-layers (OLMoE layer, 8 int4 experts each) in {el:.1f} s; "
                      f"{K_TOP * lay['record_bytes'] * n / el / 1e9:.3f} GB/s of records; stack tok/s = "
                      f"{1.0 / per_layer / L:.3f}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--tokens", type=int, default=16, help="distinct decode tokens (one graph each)")
    ap.add_argument("--kernel-launches", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE-layer path here runs on a single MI355X "
              "(multi-GPU sharding is described, not run). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    r = gpu_bench(args)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": "int4 MoE-layer decode tok/s + % HBM roofline, OLMoE shape, bs=1, 1 GPU",
        "value": round(r["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic",
        "config": {
            "workload": "OLMoE-shaped 16-layer MoE stack, decode bs=1, int4 gs64 (absmax) experts, all resident",
            "d_model": H, "experts": E, "top_k": K_TOP, "d_ff": I, "layers": L, "batch": 1,
            "activations": "fp16", "accumulate": "fp32", "router": "softmax top-8, no renorm",
        },
        "layer_tok_s": round(r["layer_tok_s"], 1),
        "layer_us": round(r["layer_us"], 3),
        "expert_gbs_ref_definition": round(r["expert_gbs"], 1),
        "layer_alg_gbs": round(r["layer_alg_gbs"], 1),
        "kernels_us": {"A_gate_up": round(r["kernelA_us"], 3), "B_down_plus_reduce": round(r["kernelB_us"], 3)},
        "roofline": {
            "bound": "hbm", "achieved": round(r["kernelA_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r["kernelA_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_up<int4> (grouped gate/up GEMV, 8 records)", "bytes_per_launch": r["kernelA_bytes"],
        },
        "cpu_baseline": cpu,
        "torch": torch.__version__,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
