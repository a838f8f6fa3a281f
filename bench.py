#!/usr/bin/env python3
"""
Benchmark: int4 MoE-layer decode tok/s + % of HBM roofline, OLMoE shape, bs=1, one MI355X.

Workload (the OLMoE-shaped 16-layer MoE stack at batch 1, all experts int4 gs64 and resident):
d_model 2048, 64 experts per layer, softmax router top-8 without renormalisation, SwiGLU d_ff
1024, router weights and expert weights N(0, 0.02) (experts quantised int4 gs64 absmax on the
GPU with moelab's packing), fp16 hidden states N(0, 1), one seeded state per (token, layer).
A step = one decode token through the 16 MoE layers: per layer ONE launch of the fused kernel
(router -> routing and HOBBIT decision -> gate/up rows -> down rows -> combine; the XCD-local
kernel k_decode_xcd), replayed as one HIP graph per token. 16 x 64 int4
records = 3.42 GB, far above the 256 MB Infinity Cache, and each token routes differently.

Roofline: the dominant (only) kernel is the fused decode-layer kernel, one launch per layer; its
algorithmic bytes per launch = 8 routed int4 records (3,342,336 B each: gate_up.q/.s, down.q/.s)
+ router weights (64 x 2048 fp16) + x and out (fp16) = 27,009,024 B; its duration is measured
live with HIP events on the stream it runs on, over launches that rotate through all tokens and
layers.

HBM traffic per launch (roofline.traffic) is read from the committed rocprofv3 counter summary
profiles/k_decode_xcd_olmoe_int4_bs1.md (FETCH_SIZE + WRITE_SIZE of this kernel, scaled by the
same counters on a plain copy of known size, `--copy-calibration`); null when that file is absent.
The prefill layer's comes from profiles/k_gemm_qwen3_30b_prefill_t512.md the same way.

CPU baseline: the oracle's restatement of moelab's CPU expert branch (dequantise to fp32,
F.linear-equivalent matvecs, weighted sum) on a bounded sample of the same workload, host cores.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
    python bench.py --copy-calibration 256     # a plain 256 MiB device copy, 20 times (counter scale)
    python bench.py --workload qwen3-30b-prefill   # the grouped-GEMM path: one Qwen3-30B-shaped
                                                   # layer on a 512-token bf16 chunk (own JSON line)
    python bench.py --workload qwen3-next-offload  # offloaded decode, records in pinned host memory
    python bench.py --workload dense-int8          # one-token int8 GEMVs of the dense part (LM head)
    python bench.py --workload disk-tier           # offloaded decode served from an expert store on disk
    python bench.py --workload stream-floor        # the dependency-free read of one decode layer's bytes
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
PROFILE = ROOT / "profiles" / "k_decode_xcd_olmoe_int4_bs1.md"
PREFILL_PROFILE = ROOT / "profiles" / "k_gemm_qwen3_30b_prefill_t512.md"
BATCH_PROFILE = ROOT / "profiles" / "k_gemv_batched_decode.md"
SHAPES_PROFILE = ROOT / "profiles" / "k_decode_xcd_bs1_other_shapes.md"
STREAM_PROFILE = ROOT / "profiles" / "k_stream_read_olmoe_layer.md"


def measured_traffic(profile: Path = PROFILE, workload: str | None = None):
    """HBM bytes per launch from a committed counter summary (its `traffic_bytes_per_launch:`
    line, or `traffic_bytes_per_layer[workload]:` for a summary that covers several workloads),
    or None."""
    key = "traffic_bytes_per_launch:" if workload is None else f"traffic_bytes_per_layer[{workload}]:"
    try:
        for line in profile.read_text().splitlines():
            if line.strip().startswith(key):
                return int(float(line.split(":", 1)[1].split()[0]))
    except (OSError, ValueError):
        pass
    return None


def copy_calibration(mib: int):
    """A plain device-to-device copy of `mib` MiB, 20 times: the bytes per launch are known
    exactly (read mib MiB, write mib MiB), so counters read on it scale the kernel's counters."""
    import torch

    n = mib * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 20}), flush=True)


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


# stamps of the XCD decode kernel's traced launches (index: stage reached)
XC_STAGES = {1: "router rows done", 2: "logits polled", 3: "experts ranked", 4: "softmax (routing wave)",
             5: "levels decided (routing wave)", 6: "routing known (workgroup)", 7: "up weights requested",
             8: "up data in / down weights requested", 9: "h stored", 10: "segment's h in (down items)",
             11: "down products", 12: "combined (combiners)", 13: "item(s) done", 14: "end"}


def layer_reference_check(store, lay, dec, xs, Wr, outs, token=0, dims=None, renorm=False, shared=None):
    """Before timing: token `token`'s layers against a torch fp32 reference of the MoE layer on
    the same int4 records (nibbles - 8 times the fp16 group scales), with the kernel's routing
    (its experts must be a top-k of the fp32 router logits, its weights their softmax within
    2^-9 relative for fp16 logits, 2^-6 for bf16). Raises unless each layer's output is within max-abs 2e-2 and mean-rel 1e-3."""
    import torch

    from moelab_hip.store import _nibble_table, views

    table = _nibble_table(outs.device)
    H, I, K_TOP, L = dims or (globals()["H"], globals()["I"], globals()["K_TOP"], globals()["L"])

    def deq(v, name, rows, cols):
        q = table[v[f"{name}.q"].long()].reshape(rows, cols).float()
        sc = v[f"{name}.s"].float()
        return q * sc.repeat_interleave(cols // sc.shape[1], dim=1)

    worst_abs, worst_rel = 0.0, 0.0
    for l in range(L):
        x = xs[token, l]
        dec.layer(l, x, outs[token, l])
        torch.cuda.synchronize()
        idx = dec.idx.view(-1).tolist()
        w = dec.w32.view(-1).float()
        xf = x.view(-1).float()
        logits = (Wr[l].float() @ xf).to(x.dtype).float()  # the router's logits are rounded to the dtype
        prob = torch.softmax(logits, dim=0)
        kth = torch.topk(logits, K_TOP + 1).values
        chosen = logits[idx]
        if chosen.min() < kth[K_TOP - 1] - 1e-3 or len(set(idx)) != K_TOP:
            raise RuntimeError(f"layer {l}: routed experts {idx} are not a top-{K_TOP} of the fp32 router logits")
        pw = prob[idx] / prob[idx].sum() if renorm else prob[idx]
        # one unit in the last place of a 16-bit logit moves its weight by about that much: the
        # kernel's and torch's fp32 sums may round to neighbouring logits
        wtol = 2.0 ** -9 if x.dtype == torch.float16 else 2.0 ** -6
        if not torch.allclose(w, pw, rtol=wtol, atol=1e-6):
            raise RuntimeError(f"layer {l}: routed weights differ from the softmax of the fp32 logits")
        y = torch.zeros(H, device=x.device)
        # the weights in the activation dtype, as the model's routing hands them over
        wd = w.to(x.dtype).float()
        rows = [(wd[j], store.blob("int4", l, e)) for j, e in enumerate(idx)]
        if shared is not None:  # the shared expert, weighted by the sigmoid of its gate's logit
            sg = (shared[l]["gate"].float() @ xf).to(x.dtype).float()
            rows.append((torch.sigmoid(sg).to(x.dtype).float(), shared[l]["rec"]["int4"]))
        for wj, blob in rows:
            v = views(lay, blob)
            gu = deq(v, "gate_up", 2 * I, H)
            dn = deq(v, "down", H, I)
            gate, up = gu[:I] @ xf, gu[I:] @ xf
            y += wj * (dn @ (torch.nn.functional.silu(gate) * up))
        got = outs[token, l].view(-1).float()
        ref = y.to(outs.dtype).float()
        d = (got - ref).abs()
        mabs, mrel = float(d.max()), float(d.mean() / ref.abs().mean())
        if mabs > 2e-2 or mrel > 1e-3:
            raise RuntimeError(f"layer {l}: output off the fp32 reference (max-abs {mabs:.3g}, mean-rel {mrel:.3g})")
        worst_abs, worst_rel = max(worst_abs, mabs), max(worst_rel, mrel)
    log(f"[bench] parity: token {token}, {L} layers against a torch fp32 reference: max-abs {worst_abs:.2e}, "
        f"mean-rel {worst_rel:.2e} (bars 2e-2, 1e-3)")
    return {"layers": L, "max_abs": worst_abs, "mean_rel": worst_rel}


def gpu_bench(args):
    import torch

    from moelab_hip import _lib

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
    parity = layer_reference_check(store, lay, dec, xs, Wr, outs)
    if not torch.equal(outs, ref_out):
        raise RuntimeError("the checked eager layers differ from the graph replay")

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

    # --- the layer kernel timed live with HIP events on its stream -----------------------
    # one fused launch per layer: back-to-back eager launches rotating over every (token,
    # layer), bracketed by two events on the stream the kernel runs on.
    st = torch.cuda.current_stream(dev)
    nA = S * L
    reps = max(1, args.kernel_launches // nA)
    for j in range(nA):
        dec.layer(j % L, xs[j // L, j % L], outs[j // L, j % L])
    kernel_name = _lib.last_decode_kernel()  # the kernel these launches ran (the library's readout)
    torch.cuda.synchronize()
    ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ea.record(st)
    for _ in range(reps):
        for j in range(nA):
            dec.layer(j % L, xs[j // L, j % L], outs[j // L, j % L])
    eb.record(st)
    torch.cuda.synchronize()
    kern_us = ea.elapsed_time(eb) * 1000 / (reps * nA)
    dec.check_error()

    # the expert phase of the launch (first weight request to the last down product, per-workgroup
    # real-time stamps of a traced launch), over a few (token, layer) launches
    phases, stages = [], []
    tr = torch.zeros(16 * 4096, dtype=torch.int64, device=dev)
    for j in range(min(nA, 12)):
        dec.grid, dec.trace = -1, tr
        tr.zero_()
        dec.layer(j % L, xs[j // L, j % L], outs[j // L, j % L])
        torch.cuda.synchronize()
        dec.grid, dec.trace = 0, None
        t = tr.view(-1, 16).cpu()
        t = t[t[:, 0] > 0]
        done = t[:, 11][t[:, 11] > 0]
        if len(t) and len(done):
            phases.append(float(done.max() - t[:, 6].min()) * 10 / 1000)
            stages.append(t)
    dec.check_error()
    if getattr(args, "stage_stamps", False) and stages:
        # every stage's time over all workgroups of these launches: median / max in us from the
        # launch's first workgroup start (a stage a workgroup does not pass reads 0 and is left out)
        for i, name in XC_STAGES.items():
            vals = []
            for t in stages:
                s0 = int(t[:, 0].min())
                col = t[:, i]
                vals += [(int(v) - s0) * 10 / 1000 for v in col[col > 0]]
            if vals:
                vals.sort()
                log(f"[bench] stage {i:2d} {name:<34s} median {vals[len(vals) // 2]:6.2f} us  max {vals[-1]:6.2f} us")
    phases.sort()
    expert_phase_us = phases[len(phases) // 2] if phases else None

    gu_bytes = 2 * I * (H // 2) + 2 * I * (H // 64) * 2  # gate_up.q + gate_up.s of one record
    dn_bytes = H * (I // 2) + H * (I // 64) * 2
    rec_bytes = gu_bytes + dn_bytes
    layer_alg = K_TOP * rec_bytes + E * H * 2 + 2 * H * 2  # experts + router + x/out
    tok_s = 1000.0 / ms_step
    layer_us = ms_step * 1000 / L
    return {
        "parity": parity,
        "tok_s": tok_s, "ms_step": ms_step, "layer_us": layer_us,
        "layer_tok_s": tok_s * L,
        "expert_gbs": K_TOP * rec_bytes / (layer_us * 1e-6) / 1e9,
        "layer_alg_gbs": layer_alg / (layer_us * 1e-6) / 1e9,
        "kernel_us": kern_us, "kernel_bytes": layer_alg,
        "kernel_gbs": layer_alg / (kern_us * 1e-6) / 1e9,
        "record_bytes": rec_bytes, "fused": dec.fused, "kernel": kernel_name,
        "expert_phase_us": expert_phase_us,
        "expert_phase_gbs": (K_TOP * rec_bytes / (expert_phase_us * 1e-6) / 1e9) if expert_phase_us else None,
    }


# Qwen3-30B-A3B-shaped prefill chunk (the grouped-GEMM path)
QH, QI, QE, QK, QT, QL = 2048, 768, 128, 8, 512, 8
MFMA_PEAK_TFS = 2500.0  # dense fp16/bf16 MFMA


def prefill_bench(args):
    """One Qwen3-30B-shaped MoE layer on a 512-token bf16 chunk in one moehip_prefill_layer call
    (router logits -> top-k with expert buckets -> placement -> gate/up GEMM -> down GEMM ->
    combine), rotating over QL layers of int4 records (8 x 128 x 2.5 MB = 2.6 GB, far above the
    Infinity Cache)."""
    import torch

    from moelab_hip import _lib
    from moelab_hip.layer import ResidentStore
    from moelab_hip.prefill import GroupedTokens
    from moelab_hip.store import record_layout

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    lay = record_layout("int4", QH, QI, 64, scale="absmax")
    store = ResidentStore({"int4": lay}, QL, QE, dev)
    t0 = time.time()
    store.fill_synthetic(g, std=0.02)
    torch.cuda.synchronize()
    log(f"[bench] encoded {QL * QE} int4 records ({store.bytes_resident / 1e9:.2f} GB) in {time.time() - t0:.1f} s")
    Wr = [(torch.randn(QE, QH, device=dev, generator=g) * 0.02).bfloat16() for _ in range(QL)]
    xs = torch.randn(QL, QT, QH, device=dev, generator=g).bfloat16()
    outs = torch.zeros(QL, QT, QH, dtype=torch.bfloat16, device=dev)
    gt = GroupedTokens(lay, QE, QK, QT, dev)
    tabs = [gt.table(store.rtab[l, 0]) for l in range(QL)]
    distinct = []
    for l in range(QL):
        _, idx, _, _ = gt.route(xs[l], Wr[l], True)
        distinct.append(int(torch.unique(idx).numel()))
    st = torch.cuda.current_stream(dev)

    def one(l):
        gt.layer(xs[l], Wr[l], True, tabs[l], outs[l])

    for i in range(max(args.warmup // 20, QL)):
        one(i % QL)
    torch.cuda.synchronize()
    n = max(QL, args.steps // 10)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for i in range(n):
        one(i % QL)
    b.record(st)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000 / n
    rec = lay["record_bytes"]
    nd = sum(distinct) / QL
    alg = nd * rec + QE * QH * 2 + 2 * QT * QH * 2  # distinct experts + router + x/out
    flops = 2 * QT * QK * 3 * QH * QI + 2 * QT * QE * QH
    log(f"[bench] prefill layer: {us:.1f} us, {nd:.1f} distinct experts, {alg / us / 1e3:.0f} GB/s, "
        f"{flops / us / 1e6:.1f} TFLOP/s")
    return {"us": us, "n": n, "alg": alg, "flops": flops, "distinct": nd}


def prefill_line(args):
    r = prefill_bench(args)
    gbs = r["alg"] / (r["us"] * 1e-6) / 1e9
    tfs = r["flops"] / (r["us"] * 1e-6) / 1e12
    return {
        "metric": "int4 MoE-layer prefill tok/s, Qwen3-30B shape, 512-token chunk, 1 GPU",
        "value": round(QT / (r["us"] * 1e-6), 1), "unit": "tok/s", "n_gpus": 1, "steps": r["n"],
        "warmup": max(args.warmup // 20, QL), "ms_per_step": round(r["us"] / 1000, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int4", "data": "synthetic",
        "config": {"workload": "Qwen3-30B-A3B-shaped MoE layer, 512-token bf16 prefill chunk, int4 gs64 experts",
                   "d_model": QH, "experts": QE, "top_k": QK, "d_ff": QI, "layers_rotated": QL, "tokens": QT,
                   "router": "softmax top-8, renormalised", "distinct_experts": r["distinct"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(PREFILL_PROFILE),
                     "kernel": "whole layer: router logits + k_route_post + k_route_place + k_gemm_up + k_gemm_down + k_combine_pairs",
                     "bytes_per_launch": int(r["alg"])},
        "mfma": {"achieved": round(tfs, 1), "peak": MFMA_PEAK_TFS, "unit": "TFLOP/s", "frac": round(tfs / MFMA_PEAK_TFS, 4),
                 "flops_per_launch": r["flops"]},
        "cpu_baseline": None if args.no_cpu else prefill_cpu_baseline(args.cpu_seconds),
    }


def prefill_cpu_baseline(seconds: float):
    """moelab's prefill expert path on the host (runtime.py:418-436, 352-353: per expert materialize,
    F.linear, index_add_) restated in torch fp32 (oracle/cpu_path.py), on a bounded sample of
    experts of the chunk's average token count."""
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_path

    r = cpu_path.time_prefill_layer(seconds, QH, QI, QE, QK, QT)
    log(f"[bench] prefill cpu baseline: {r['n']} experts in {r['seconds']:.1f} s on {r['threads']} threads "
        f"({r['cpu_model']}): {r['layer_s'] * 1000:.1f} ms per layer")
    return {"value": round(QT / r["layer_s"], 1), "unit": "tok/s", "cores": r["threads"], "kind": "port",
            "host_cpus": r["host_cpus"], "cpu_model": r["cpu_model"],
            "sample": f"{r['n']} experts of {r['tokens_per_expert']} tokens (int4 gs64 records, torch fp32 "
                      f"dequantize + F.linear + index_add_) in {r['seconds']:.1f} s on {r['threads']} threads; "
                      f"layer = {QE} experts x {r['expert_s'] * 1000:.2f} ms"}


# The dense part in int8 (moelab/denseq.py), one token: the LM heads and an attention projection
DENSE_SHAPES = {"olmoe-lm-head": (50304, 2048), "qwen3-next-lm-head": (151936, 2048), "attention-proj": (2048, 2048)}


def dense_line(args):
    """One-token int8 GEMVs at the dense part's shapes (moehip_dense_gemv_int8 behind QLinear), each
    timed with HIP events around one HIP graph of back-to-back launches that rotate over enough
    weight copies to exceed the 256 MB Infinity Cache; the headline is the OLMoE LM head."""
    import torch

    from moelab_hip import _lib
    from moelab_hip import denseq as D

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    st = torch.cuda.current_stream(dev)
    res = {}
    for name, (O_, K) in DENSE_SHAPES.items():
        nb = O_ * K + O_ * (K // 64) * 2
        copies = max(3, -(-768 * 2**20 // nb))
        g = torch.Generator(device=dev).manual_seed(O_)
        mats = []
        for _ in range(copies):
            q, s = D.quantize_int8(torch.randn(O_, K, device=dev, generator=g) * 0.02, 64)
            mats.append((q, s))
        x = torch.randn(K, device=dev, generator=g).bfloat16()
        for i in range(2 * copies):
            D.gemv_int8(*mats[i % copies], x, 64)
        torch.cuda.synchronize()
        # the launches replayed as one HIP graph (the host's per-call cost stays out of the figure)
        n = max(4 * copies, args.kernel_launches // 4)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(n):
                D.gemv_int8(*mats[i % copies], x, 64)
        gr.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream(dev)
        a.record(st)
        gr.replay()
        b.record(st)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1000 / n
        del gr
        res[name] = {"O": O_, "K": K, "bytes": nb + 2 * K + 2 * O_, "us": round(us, 3),
                     "gbs": round((nb + 2 * K + 2 * O_) / (us * 1e-6) / 1e9, 1), "copies": copies, "launches": n}
        log(f"[bench] dense int8 GEMV {name} {O_}x{K}: {us:.2f} us, {res[name]['gbs']:.0f} GB/s")
        del mats
        torch.cuda.empty_cache()
    h = res["olmoe-lm-head"]
    return {
        "metric": "dense-part int8 GEMV GB/s (one token), OLMoE LM head, 1 GPU",
        "value": h["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": h["launches"], "warmup": 2 * h["copies"],
        "ms_per_step": round(h["us"] / 1000, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "one-token int8 gs64 GEMVs of the dense part (QLinear), bf16 activations",
                   "shapes": {k: [v["O"], v["K"]] for k, v in res.items()}},
        "roofline": {"bound": "hbm", "achieved": h["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(h["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(ROOT / "profiles" / "k_gemv8_dense_int8.md", "olmoe-lm-head"),
                     "kernel": "k_gemv8<bf16> (moehip_dense_gemv_int8)", "bytes_per_launch": h["bytes"]},
        "shapes": res,
        "cpu_baseline": None,
    }


# More decode configurations through the same fused kernel (their own JSON lines): the OLMoE stack
# with two record precisions per expert (a weight-threshold precision rule), and the Qwen3-30B-A3B /
# Qwen3-Next-80B-A3B layer shapes at batch 1.
DECODE_SPECS = {
    "olmoe-mixed-decode": dict(H=2048, I=1024, E=64, k=8, L=16, precs=["fp16", "int4"], dtype="float16",
                               renorm=False, shared=False, policy=("weight", 0.15),
                               desc="OLMoE-shaped 16-layer MoE stack, decode bs=1, each routed expert in fp16 "
                                    "if its gate weight >= 0.15, else int4 gs64; fp16 and int4 records of "
                                    "every expert resident"),
    "qwen3-30b-decode": dict(H=2048, I=768, E=128, k=8, L=8, precs=["int4"], dtype="bfloat16", renorm=True,
                             shared=False, policy=("lo",),
                             desc="Qwen3-30B-A3B-shaped MoE layer, decode bs=1, int4 gs64 experts, 8 layers "
                                  "rotated"),
    "qwen3-next-decode-int4": dict(H=2048, I=512, E=512, k=10, L=8, precs=["int4"], dtype="bfloat16",
                                   renorm=True, shared=True, policy=("lo",),
                                   desc="Qwen3-Next-80B-A3B-shaped MoE layer, decode bs=1, 512 int4 gs64 experts "
                                        "top-10 + sigmoid-gated shared expert, 8 layers rotated"),
    "qwen3-next-decode-fp8": dict(H=2048, I=512, E=512, k=10, L=8, precs=["fp8"], dtype="bfloat16",
                                  renorm=True, shared=True, policy=("lo",),
                                  desc="Qwen3-Next-80B-A3B-shaped MoE layer, decode bs=1, 512 FP8 e4m3 experts "
                                       "(128x128 block scales) top-10 + sigmoid-gated shared expert, 8 layers "
                                       "rotated"),
}

# batched decode (T > 1 tokens per step): the grouped path over the resident store
BATCH_SPECS = {
    "olmoe-mixed-decode-bs8": dict(DECODE_SPECS["olmoe-mixed-decode"], batch=8,
                                   desc="OLMoE-shaped 16-layer MoE stack, decode bs=8, each (token, expert) "
                                        "requesting fp16 if its gate weight >= 0.15, else int4 gs64, one "
                                        "precision per expert by vote; fp16 and int4 records of every expert "
                                        "resident"),
    "qwen3-next-decode-int4-bs32": dict(DECODE_SPECS["qwen3-next-decode-int4"], batch=32,
                                        desc="Qwen3-Next-80B-A3B-shaped MoE layer, decode bs=32, 512 int4 gs64 "
                                             "experts top-10 + sigmoid-gated shared expert, 8 layers rotated"),
    "qwen3-next-decode-fp8-bs32": dict(DECODE_SPECS["qwen3-next-decode-fp8"], batch=32,
                                       desc="Qwen3-Next-80B-A3B-shaped MoE layer, decode bs=32, 512 FP8 e4m3 "
                                            "experts (128x128 block scales) top-10 + sigmoid-gated shared "
                                            "expert, 8 layers rotated"),
}


def _decode_setup(sp, name):
    """Resident store of L layers x E experts in each precision of the spec (synthetic N(0, 0.02)
    weights), router weights, shared experts and the precision policy."""
    import torch

    from moelab_hip import _lib
    from moelab_hip.layer import ResidentStore
    from moelab_hip.policy import PrecisionPolicy
    from moelab_hip.store import encode_record_, record_layout

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    H_, I_, E_, L_ = sp["H"], sp["I"], sp["E"], sp["L"]
    dt = getattr(torch, sp["dtype"])
    g = torch.Generator(device=dev).manual_seed(0)
    lays = {p: record_layout(p, H_, I_, 64, scale="absmax" if p in ("int4", "int8") else None) for p in sp["precs"]}
    store = ResidentStore(lays, L_, E_, dev)
    t0 = time.time()
    store.fill_synthetic(g, std=0.02)
    torch.cuda.synchronize()
    log(f"[bench] {name}: {store.bytes_resident / 1e9:.2f} GB of records encoded in {time.time() - t0:.1f} s")
    Wr = [(torch.randn(E_, H_, device=dev, generator=g) * 0.02).to(dt) for _ in range(L_)]
    shared = None
    if sp["shared"]:
        shared = []
        for _ in range(L_):
            rec = {}
            for p, lay in lays.items():
                blob = torch.zeros(lay["record_bytes"], dtype=torch.uint8, device=dev)
                encode_record_(lay, blob, torch.randn(2 * I_, H_, device=dev, generator=g) * 0.02,
                               torch.randn(H_, I_, device=dev, generator=g) * 0.02)
                rec[p] = blob
            shared.append({"gate": (torch.randn(H_, device=dev, generator=g) * 0.05).to(dt), "rec": rec})
    # upgrade=False: a level-2 request runs the int4 record even though the fp16 one is resident
    pol = (PrecisionPolicy(sp["policy"][0], t1=sp["policy"][1], upgrade=False) if len(sp["policy"]) > 1
           else PrecisionPolicy(sp["policy"][0]))
    return dev, dt, g, lays, store, Wr, shared, pol


def decode_line(args, name):
    """One decode configuration: a HIP graph per token over L layers (fused kernel), 16 tokens;
    algorithmic bytes per launch = the records the launch ran (from the kernel's per-row readout)
    + router + shared gate + x/out."""
    import torch

    from moelab_hip import _lib
    from moelab_hip.layer import MoEDecoder

    sp = DECODE_SPECS[name]
    H_, I_, E_, k_, L_ = sp["H"], sp["I"], sp["E"], sp["k"], sp["L"]
    dev, dt, g, lays, store, Wr, shared, pol = _decode_setup(sp, name)
    dec = MoEDecoder(store, k_, pol, dt, router_weights=Wr, renorm=sp["renorm"], shared=shared)
    S = 16
    xs = torch.randn(S, L_, 1, H_, device=dev, generator=g).to(dt)
    outs = torch.zeros(S, L_, 1, H_, dtype=dt, device=dev)
    # bytes each launch ran: one eager pass, reading the per-row readout after every layer
    precs = store.precisions
    run_bytes = 0
    for s_ in range(S):
        for l in range(L_):
            dec.layer(l, xs[s_, l], outs[s_, l])
            kernel_name = _lib.last_decode_kernel()
            info = dec.info[l].cpu()
            for j in range(k_):
                c = int(info[1, j])
                if c >= 0:
                    run_bytes += lays[precs[c]]["record_bytes"]
    if sp["shared"]:
        run_bytes += S * L_ * lays[precs[0]]["record_bytes"]
    alg = run_bytes / (S * L_) + E_ * H_ * 2 + (H_ * 2 if sp["shared"] else 0) + 2 * H_ * 2
    if dec.miss.item() != 0:
        raise RuntimeError("experts missing from the resident store")
    parity = None
    if precs == ["int4"]:
        parity = layer_reference_check(store, lays["int4"], dec, xs, Wr, outs, dims=(H_, I_, k_, L_),
                                       renorm=sp["renorm"], shared=shared)

    def token(s_):
        for l in range(L_):
            dec.layer(l, xs[s_, l], outs[s_, l])

    graphs = []
    for s_ in range(S):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            token(s_)
        graphs.append(gr)
    for i in range(max(S, args.warmup // 4)):
        graphs[i % S].replay()
    torch.cuda.synchronize()
    steps = max(S, args.steps // 4)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        graphs[i % S].replay()
    b.record()
    torch.cuda.synchronize()
    dec.check_error()
    ms = a.elapsed_time(b) / steps
    layer_us = ms * 1000 / L_
    gbs = alg / (layer_us * 1e-6) / 1e9
    log(f"[bench] {name}: {layer_us:.2f} us per layer, {alg / 1e6:.2f} MB per launch, {gbs:.0f} GB/s")
    return {
        "metric": f"MoE-layer decode tok/s + % HBM roofline, {name}, bs=1, 1 GPU",
        "value": round(1000.0 / ms, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": max(S, args.warmup // 4),
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "+".join(sp["precs"]), "data": "synthetic",
        "config": {"workload": sp["desc"], "d_model": H_, "experts": E_, "top_k": k_, "d_ff": I_, "layers": L_,
                   "batch": 1, "activations": sp["dtype"], "shared_expert": sp["shared"]},
        "layer_us": round(layer_us, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(SHAPES_PROFILE, name),
                     "kernel": f"{kernel_name} (one launch per layer, HIP graph per token)",
                     "bytes_per_launch": int(alg)},
        "cpu_baseline": (decode_cpu_baseline(args.cpu_seconds, H_, I_, k_ + (1 if sp["shared"] else 0), L_)
                         if not args.no_cpu and sp["precs"] == ["int4"] else None),
        "parity": None if parity is None else {
            "checked": f"token 0, {parity['layers']} layers, torch fp32 reference before timing",
            "max_abs": float(f"{parity['max_abs']:.3g}"), "mean_rel": float(f"{parity['mean_rel']:.3g}")},
    }


def decode_cpu_baseline(seconds: float, H_: int, I_: int, n_exp: int, L_: int):
    """moelab's CPU expert branch (runtime.py:646-702) restated in torch (oracle/cpu_path.py) on one
    layer of this workload's shape: n_exp int4 gs64 records (the routed experts, plus the shared
    one where the model has it), one token, the host's cores."""
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_path

    r = cpu_path.time_olmoe_layer(seconds, H_, I_, n_exp)
    log(f"[bench] cpu baseline: {r['n']} layers in {r['seconds']:.1f} s on {r['threads']} threads")
    return {"value": round(1.0 / r["layer_s"] / L_, 3), "unit": "tok/s", "cores": r["threads"], "kind": "port",
            "host_cpus": r["host_cpus"], "cpu_model": r["cpu_model"],
            "sample": f"{r['n']} token-layers ({n_exp} int4 gs64 records of H={H_}, I={I_}, torch fp32 dequantize + "
                      f"F.linear on {r['threads']} threads) in {r['seconds']:.1f} s; tok/s over the {L_}-layer stack"}


def batch_cpu_baseline(seconds: float, H_: int, I_: int, n_exp: float, B: int, L_: int):
    """moelab's CPU expert branch (runtime.py:646-702, oracle/cpu_path.py) for a batch: each distinct
    expert of the layer is dequantised once and run on its tokens. Timed on 8 int4 gs64 records
    with one token each; the layer time is the per-record time times the layer's distinct experts
    (a record's dequantisation dominates: its 1-2 tokens' products are left out, which favours the
    CPU)."""
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_path

    r = cpu_path.time_olmoe_layer(seconds, H_, I_, 8)
    layer_s = r["layer_s"] / 8 * n_exp
    log(f"[bench] cpu baseline: {r['n']} 8-record layers in {r['seconds']:.1f} s on {r['threads']} threads")
    return {"value": round(B / (layer_s * L_), 3), "unit": "tok/s", "cores": r["threads"], "kind": "port",
            "host_cpus": r["host_cpus"], "cpu_model": r["cpu_model"],
            "sample": f"{r['n']} x 8 int4 gs64 records of H={H_}, I={I_} (torch fp32 dequantize + F.linear, one "
                      f"token each, {r['threads']} threads) in {r['seconds']:.1f} s; scaled to {n_exp:.1f} "
                      f"distinct experts per layer, {B} tokens, {L_} layers"}


def batch_line(args, name):
    """Batched decode: B tokens per step through L layers on the grouped path (GroupedLayer: router,
    levels, dispatch, per-expert vote, grouped GEMMs per precision, ordered combine), a HIP graph
    per step, 8 distinct batches. Algorithmic bytes per layer = the distinct (expert, precision)
    records the layer ran (from the vote's readout) + shared record + router + shared gate +
    B x (x + out)."""
    import torch

    from moelab_hip.prefill import GroupedLayer

    sp = BATCH_SPECS[name]
    H_, I_, E_, k_, L_, B = sp["H"], sp["I"], sp["E"], sp["k"], sp["L"], sp["batch"]
    dev, dt, g, lays, store, Wr, shared, pol = _decode_setup(sp, name)
    gl = GroupedLayer(store, k_, B, pol, dt, router_weights=Wr, renorm=sp["renorm"], shared=shared)
    S = 8
    xs = torch.randn(S, L_, B, H_, device=dev, generator=g).to(dt)
    outs = torch.zeros(S, L_, B, H_, dtype=dt, device=dev)
    precs = store.precisions
    run_bytes, distinct = 0, 0
    for s_ in range(S):
        for l in range(L_):
            gl.layer(l, xs[s_, l], outs[s_, l])
            info = gl.info[l].cpu()
            for e in range(info.numel()):
                c = int(info[e])
                if c >= 0:
                    run_bytes += lays[precs[c]]["record_bytes"]
                    distinct += 1 if e < E_ else 0
    if gl.miss.item() != 0:
        raise RuntimeError("experts missing from the resident store")
    alg = run_bytes / (S * L_) + E_ * H_ * 2 + (H_ * 2 if sp["shared"] else 0) + B * 2 * H_ * 2

    def step(s_):
        for l in range(L_):
            gl.layer(l, xs[s_, l], outs[s_, l])

    graphs = []
    for s_ in range(S):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            step(s_)
        graphs.append(gr)
    warm = max(S, args.warmup // 8)
    for i in range(warm):
        graphs[i % S].replay()
    torch.cuda.synchronize()
    steps = max(S, args.steps // 8)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        graphs[i % S].replay()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    layer_us = ms * 1000 / L_
    gbs = alg / (layer_us * 1e-6) / 1e9
    log(f"[bench] {name}: {layer_us:.2f} us per layer, {alg / 1e6:.2f} MB per layer, {gbs:.0f} GB/s, "
        f"{distinct / (S * L_):.1f} distinct routed experts per layer")
    return {
        "metric": f"MoE-layer decode tok/s + % HBM roofline, {name}, bs={B}, 1 GPU",
        "value": round(B * 1000.0 / ms, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "+".join(sp["precs"]), "data": "synthetic",
        "config": {"workload": sp["desc"], "d_model": H_, "experts": E_, "top_k": k_, "d_ff": I_, "layers": L_,
                   "batch": B, "activations": sp["dtype"], "shared_expert": sp["shared"],
                   "distinct_experts_per_layer": round(distinct / (S * L_), 2)},
        "layer_us": round(layer_us, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(BATCH_PROFILE, name),
                     "traffic_scope": "k_gemv_up + k_gemv_down per layer (FETCH_SIZE, WRITE_SIZE)",
                     "kernel": "whole layer: router logits + top-k / shared slot + levels, dispatch, vote and "
                               "work list + k_gemv_up/down per precision + combine (HIP graph per step)",
                     "bytes_per_launch": int(alg)},
        "cpu_baseline": (None if args.no_cpu else
                         batch_cpu_baseline(args.cpu_seconds, H_, I_, distinct / (S * L_) + (1 if sp["shared"] else 0),
                                            B, L_)),
    }


# Qwen3-Next-80B-A3B-shaped offloaded decode
NH, NI, NE, NK = 2048, 512, 512, 10


def residual_stream(dev, steps: int, L: int, E: int, H: int, seed: int, rho: float = 0.6, alpha: float = 0.35,
                    pop: float = 1.0):
    """A synthetic decode: per layer a router (E, H) and per (token, layer) a hidden state, bf16.
    Routers: N(0, 1/H) rows plus a popularity term pop * -log(rank + 1) (a random rank order per
    layer) along a direction u that every hidden state carries, so the logits are a Zipf-like
    per-expert bias plus N(0, 1) noise. Hidden states: x = u + z, z of unit variance per coordinate;
    token t's first z is rho-correlated with token t-1's (experts recur from token to token), and
    each layer adds alpha * N(0, 1) (a residual stream: the next layer's gate on this layer's
    state predicts that layer's routing imperfectly)."""
    import math

    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    u = torch.randn(H, device=dev, generator=g)
    u /= u.norm()
    Ws = []
    for _ in range(L):
        rank = torch.randperm(E, device=dev, generator=g).float()
        bias = -pop * torch.log(rank + 1.0)
        W = torch.randn(E, H, device=dev, generator=g) / math.sqrt(H) + bias[:, None] * u[None, :]
        Ws.append(W.bfloat16().contiguous())
    xs = torch.empty(steps, L, 1, H, dtype=torch.bfloat16, device=dev)
    z = torch.randn(H, device=dev, generator=g)
    for t in range(steps):
        z = rho * z + math.sqrt(1.0 - rho * rho) * torch.randn(H, device=dev, generator=g)
        zl = z.clone()
        for l in range(L):
            xs[t, l, 0] = (u + zl).bfloat16()
            zl = zl + alpha * torch.randn(H, device=dev, generator=g)
    return Ws, xs


def staging_peak(dev, lay, mode: str, reps: int = 5):
    """GB/s of one staging batch of 32 records (pinned host -> device slots)."""
    import torch

    from moelab_hip.offload import DevicePool, Stager

    rb = lay["record_bytes"]
    host = torch.empty(32 * rb, dtype=torch.uint8).pin_memory()
    st = Stager(dev, DevicePool({"int4": rb}, 40 * rb, dev), mode=mode)
    items = [(host[i * rb:(i + 1) * rb], "int4") for i in range(32)]
    best = 0.0
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st.copy_stream)
        dsts, _ = st.stage(items)
        b.record(st.copy_stream)
        b.synchronize()
        for d in dsts:
            st.pool.release(d, "int4")
        best = max(best, 32 * rb / (a.elapsed_time(b) * 1e-3) / 1e9)
    return best


def offload_bench(args):
    """Qwen3-Next-shaped offloaded decode at bs=1: every int4 record in pinned host memory
    (HostPool slots), a 16 GB device budget under the LRFU cache, Zipf(1.1) routing with 40 %
    token-to-token reuse, misses staged on demand and the next layer's experts staged ahead."""
    import numpy as np
    import torch

    from moelab_hip import _lib
    from moelab_hip.layer import ResidentStore
    from moelab_hip.offload import HostPool, OffloadDecoder
    from moelab_hip.policy import PrecisionPolicy
    from moelab_hip.store import record_layout

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    L = args.offload_layers
    lay = record_layout("int4", NH, NI, 64, scale="absmax")
    rb = lay["record_bytes"]
    t0 = time.time()
    pool = HostPool({"int4": rb}, int(L * NE * rb * 1.25) + (64 << 20), pin=True, log=log)
    tmp = ResidentStore({"int4": lay}, 1, NE, dev)
    g = torch.Generator(device=dev).manual_seed(0)
    host = {}
    for l in range(L):
        tmp.fill_synthetic(g, std=0.02)
        for e in range(NE):
            slot = pool.acquire("int4")
            slot.copy_(tmp.blob("int4", 0, e), non_blocking=True)
            host[(l, e)] = slot
        torch.cuda.synchronize()
    del tmp
    log(f"[bench] {L * NE} int4 records ({L * NE * rb / 1e9:.1f} GB) in pinned host memory in "
        f"{time.time() - t0:.1f} s ({pool.describe()}, {pool.fallbacks} outside the pool)")
    peaks = {m: staging_peak(dev, lay, m) for m in ("kernel", "sdma")}
    big = torch.empty(256 << 20, dtype=torch.uint8).pin_memory()
    bigd = torch.empty_like(big, device=dev)
    ta = time.perf_counter()
    for _ in range(4):
        bigd.copy_(big, non_blocking=True)
    torch.cuda.synchronize()
    copy_peak = 4 * big.numel() / (time.perf_counter() - ta) / 1e9
    del big, bigd
    log(f"[bench] staging batch of 32 records: kernel {peaks['kernel']:.1f} GB/s, sdma {peaks['sdma']:.1f} GB/s; "
        f"torch pinned copy {copy_peak:.1f} GB/s")
    mode = max(peaks, key=peaks.get) if args.stage_mode == "auto" else args.stage_mode
    steps, warm = args.offload_steps, args.offload_warmup
    Wr, xs = residual_stream(dev, warm + steps, L, NE, NH, seed=1)
    # 16 GB for the 48-layer model by default: the same resident fraction (39 %)
    budget = int(args.offload_budget_gb * 10**9) * L // 48
    off = OffloadDecoder({"int4": lay}, L, NE, NK, lambda l, e, p: host[(l, e)], budget, dev, PrecisionPolicy("lo"),
                         torch.bfloat16, router_weights=Wr, renorm=True, mode=mode, predictor="gate",
                         prefetch_mode=args.prefetch_mode, prefetch_mass=args.prefetch_mass)
    out = torch.zeros(1, NH, dtype=torch.bfloat16, device=dev)
    # the routing every layer will get (the same router kernel on the same states), for the
    # ground-truth predictor run only
    truth = torch.zeros(warm + steps, L, NK, dtype=torch.int64, device=dev)
    dec = off.dec
    for t in range(warm + steps):
        for l in range(L):
            dec.route(l, xs[t, l])
            truth[t, l] = dec.idx[0]
    truth = truth.cpu().numpy()
    distinct = float(np.mean([len(np.unique(truth[:, l])) for l in range(L)]))
    reuse = float(np.mean([len(set(truth[t, l]) & set(truth[t - 1, l])) / NK
                           for t in range(1, warm + steps) for l in range(L)]))
    log(f"[bench] routing: {distinct:.0f} distinct experts per layer over {warm + steps} tokens, "
        f"{reuse:.2f} of a token's experts also used by the previous token")

    def token(t, how):
        for l in range(L):
            if how == "truth" and l + 1 < L:
                off.layer(l, xs[t, l], out, predict={int(e): "int4" for e in truth[t, l + 1]})
            else:
                off.layer(l, xs[t, l], out)
        off.tick()

    res = {}
    for how in ("gate", "truth", "none"):
        off.predictor = "gate" if how == "gate" else "none"
        off.cache.clear()
        off.stats = {k: 0 for k in off.stats}
        for t in range(warm):
            token(t, how)
        torch.cuda.synchronize()
        s0 = dict(off.stats)
        b0 = off.stager.bytes_h2d
        t0 = time.perf_counter()
        for t in range(warm, warm + steps):
            token(t, how)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        ds = {k: off.stats[k] - s0[k] for k in s0}
        h2d = off.stager.bytes_h2d - b0
        hit = ds["hits"] / max(1, ds["hits"] + ds["misses"])
        res[how] = {"tok_s": steps / dt, "ms_per_token": dt * 1000 / steps, "hit_rate": hit,
                    "h2d_gb_per_token": h2d / steps / 1e9, "h2d_gbs": h2d / dt / 1e9,
                    "prefetch_hits": ds["prefetch_hits"], "prefetch_issued": ds["prefetch_issued"],
                    "predictor_recall": ds["pred_hits"] / max(1, ds["pred_total"])}
        off.dec.check_error()
        if off.dec.miss.item() != 0:
            raise RuntimeError("offloaded decode ran an expert that was not resident")
        log(f"[bench] offload predictor={how}: {res[how]}")
    return {"res": res, "peaks": peaks, "copy_peak": copy_peak, "mode": mode, "prefetch_mode": args.prefetch_mode,
            "prefetch_mass": args.prefetch_mass,
            "L": L, "steps": steps, "warm": warm,
            "records_host_gb": L * NE * rb / 1e9, "budget_gb": budget / 1e9, "distinct": distinct, "reuse": reuse}


def offload_line(args):
    r = offload_bench(args)
    p = r["res"]["gate"]
    peak = max(r["peaks"].values())
    side = lambda d: {k: round(v, 4) if isinstance(v, float) else v for k, v in d.items()}  # noqa: E731
    return {
        "metric": "offloaded int4 MoE decode tok/s + H2D GB/s, Qwen3-Next shape, bs=1, 1 GPU",
        "value": round(p["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": r["steps"], "warmup": r["warm"],
        "ms_per_step": round(p["ms_per_token"], 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4", "data": "synthetic",
        "config": {"workload": "Qwen3-Next-shaped offloaded decode, int4 gs64 records in pinned host memory, "
                               "16 GB device budget, LRFU, routing by each layer's router on a synthetic "
                               "residual stream (Zipf-like expert popularity, token-to-token correlation), bs=1",
                   "d_model": NH, "experts": NE, "top_k": NK, "d_ff": NI, "layers": r["L"],
                   "records_host_gb": round(r["records_host_gb"], 1), "device_budget_gb": r["budget_gb"],
                   "staging": r["mode"], "prefetch_staging": r["prefetch_mode"], "prefetch_mass": r["prefetch_mass"],
                   "prefetch": "the next layer's gate on the current hidden state, on the GPU (read back with "
                               "the current routing)",
                   "distinct_experts_per_layer": round(r["distinct"], 1), "token_reuse": round(r["reuse"], 3),
                   "shared_expert": "not included"},
        "hit_rate": round(p["hit_rate"], 4), "predictor_recall": round(p["predictor_recall"], 4),
        "h2d_gb_per_token": round(p["h2d_gb_per_token"], 4),
        "roofline": {"bound": "host link", "achieved": round(p["h2d_gbs"], 2), "peak": round(peak, 2), "unit": "GB/s",
                     "frac": round(p["h2d_gbs"] / peak, 4), "traffic": None,
                     "peak_is": "best measured staging batch (32 records) over kernel and sdma modes"},
        "staging_gbs": {k: round(v, 2) for k, v in r["peaks"].items()}, "torch_pinned_copy_gbs": round(r["copy_peak"], 2),
        "ground_truth_predictor": side(r["res"]["truth"]),
        "no_prefetch": side(r["res"]["none"]),
        "cpu_baseline": None,
    }


def _drop_cache(paths) -> None:
    """Evict the files' pages from the page cache (fsync + POSIX_FADV_DONTNEED: the next reads
    come from the disk)."""
    for f in paths:
        fd = os.open(f, os.O_RDONLY)
        try:
            os.fsync(fd)
            os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
        finally:
            os.close(fd)


def disk_bench(args):
    """The disk tier at the Qwen3-Next shape: args.disk_layers layers of int4 records (512 per
    layer) written as a store on the box's disk, then (1) record reads straight from the disk
    (page cache dropped before each mode): O_DIRECT into page-aligned pageable buffers with 1, 4
    and 8 ranges in flight, and ordinary reads into pinned buffers with 4; (2) the offloaded
    decode served from that store through DiskTier (RAM tier a quarter of the store, VRAM budget a
    tenth), gate predictor on."""
    import numpy as np
    import torch

    from moelab_hip import _lib
    from moelab_hip.diskstore import DiskTier, ExpertStore, write_store
    from moelab_hip.layer import ResidentStore
    from moelab_hip.offload import OffloadDecoder
    from moelab_hip.policy import PrecisionPolicy
    from moelab_hip.store import record_layout

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    L = args.disk_layers
    lay = record_layout("int4", NH, NI, 64, scale="absmax")
    rb = lay["record_bytes"]
    root = Path(args.store_dir or os.environ.get("TMPDIR", "/tmp")) / f"moehip_store_{os.getpid()}"
    tmp = ResidentStore({"int4": lay}, 1, NE, dev)
    g = torch.Generator(device=dev).manual_seed(0)
    cur = {}

    def record(li, e, prec):
        if cur.get("l") != li:
            tmp.fill_synthetic(g, std=0.02)
            cur["l"], cur["host"] = li, tmp.arena["int4"].cpu().numpy()
        return cur["host"][e * rb:(e + 1) * rb]

    t0 = time.time()
    write_store(root, [lay], [f"model.layers.{i}.mlp" for i in range(L)], NE, NH, NI, record, model_type="qwen3_next")
    files = sorted(root.glob("layer*.bin"))
    _drop_cache(files)
    log(f"[bench] store of {L * NE} int4 records ({L * NE * rb / 1e9:.2f} GB) written to {root} in {time.time() - t0:.1f} s")
    del tmp
    try:
        st = ExpertStore(root)
        rng = np.random.default_rng(0)
        n = min(args.disk_reads, L * NE)
        picks = [divmod(int(i), NE) for i in rng.choice(L * NE, n, replace=False)]
        raw = torch.empty(rb + 4096, dtype=torch.uint8)
        off = (-raw.data_ptr()) % 4096
        pageable = raw[off:off + rb]
        pinned = torch.empty(rb, dtype=torch.uint8).pin_memory()
        reads = {}
        for name, direct, parts, buf in (("direct_p1", True, 1, pageable), ("direct_p4", True, 4, pageable),
                                         ("direct_p8", True, 8, pageable), ("pinned_p4", False, 4, pinned)):
            _drop_cache(files)
            st.direct = direct
            st.direct_reads = st.direct_fallbacks = 0
            ta = time.perf_counter()
            for li, e in picks:
                st.read(li, e, "int4", out=buf, parts=parts)
            dt = time.perf_counter() - ta
            reads[name] = {"gbs": n * rb / dt / 1e9, "ms_per_record": dt * 1000 / n,
                           "direct_share": st.direct_reads / n if direct else 0.0}
            log(f"[bench] disk read {name}: {reads[name]}")
        st.close()
        # the offloaded decode from disk
        steps, warm = args.disk_steps, max(4, args.disk_steps // 8)
        Wr, xs = residual_stream(dev, warm + steps, L, NE, NH, seed=1)
        _drop_cache(files)
        tier = DiskTier(ExpertStore(root), L * NE * rb // 4, pin=True, parts=4, direct=False)
        off = OffloadDecoder({"int4": lay}, L, NE, NK, tier, L * NE * rb // 10, dev, PrecisionPolicy("lo"),
                             torch.bfloat16, router_weights=Wr, renorm=True, mode="kernel", predictor="gate")
        out = torch.zeros(1, NH, dtype=torch.bfloat16, device=dev)
        for t in range(warm):
            for li in range(L):
                off.layer(li, xs[t, li], out)
            off.tick()
        torch.cuda.synchronize()
        s0, d0, b0 = dict(off.stats), dict(tier.stats), tier.store.bytes_read
        ta = time.perf_counter()
        for t in range(warm, warm + steps):
            for li in range(L):
                off.layer(li, xs[t, li], out)
            off.tick()
        torch.cuda.synchronize()
        dt = time.perf_counter() - ta
        off.dec.check_error()
        if off.dec.miss.item() != 0:
            raise RuntimeError("offloaded decode ran an expert that was not resident")
        ds = {k: off.stats[k] - s0[k] for k in s0}
        dd = {k: tier.stats[k] - d0[k] for k in d0}
        dec = {"tok_s": steps / dt, "ms_per_token": dt * 1000 / steps,
               "vram_hit_rate": ds["hits"] / max(1, ds["hits"] + ds["misses"]),
               "ram_hit_rate": dd["host_hits"] / max(1, dd["host_hits"] + dd["disk_reads"]),
               "disk_reads_per_token": dd["disk_reads"] / steps,
               "disk_gbs": (tier.store.bytes_read - b0) / dt / 1e9}
        log(f"[bench] offload from disk: {dec}")
        tier.close()
    finally:
        for f in root.glob("*"):
            f.unlink()
        root.rmdir()
    return {"reads": reads, "dec": dec, "L": L, "steps": steps, "warm": warm, "store_gb": L * NE * rb / 1e9,
            "n_reads": n, "rb": rb}


def disk_line(args):
    r = disk_bench(args)
    d = r["dec"]
    peak = max(v["gbs"] for v in r["reads"].values())
    side = lambda d_: {k: round(v, 4) if isinstance(v, float) else v for k, v in d_.items()}  # noqa: E731
    return {
        "metric": "offloaded int4 MoE decode tok/s from an expert store on disk, Qwen3-Next shape, bs=1, 1 GPU",
        "value": round(d["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": r["steps"], "warmup": r["warm"],
        "ms_per_step": round(d["ms_per_token"], 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4", "data": "synthetic",
        "config": {"workload": f"Qwen3-Next-shaped offloaded decode over {r['L']} layers whose int4 gs64 records "
                               f"({r['store_gb']:.2f} GB) are a store on the box's disk: RAM tier 1/4 of it (pinned "
                               "pool, LRFU), VRAM budget 1/10, gate predictor, bs=1",
                   "d_model": NH, "experts": NE, "top_k": NK, "d_ff": NI, "layers": r["L"],
                   "record_bytes": r["rb"]},
        "vram_hit_rate": round(d["vram_hit_rate"], 4), "ram_hit_rate": round(d["ram_hit_rate"], 4),
        "disk_reads_per_token": round(d["disk_reads_per_token"], 2),
        "roofline": {"bound": "disk", "achieved": round(d["disk_gbs"], 3), "peak": round(peak, 3), "unit": "GB/s",
                     "frac": round(d["disk_gbs"] / peak, 4), "traffic": None,
                     "peak_is": f"best record-read rate measured on this disk ({r['n_reads']} random records)"},
        "disk_reads": {k: side(v) for k, v in r["reads"].items()},
        "cpu_baseline": None,
    }


def stream_floor(dev, arena: "torch.Tensor", routers: list, rec_bytes: int, n_rec: int, grids: list,
                 launches: int = 2048, seed: int = 0, stamp_grid: int | None = None) -> dict:
    """The dependency-free floor of one launch that reads one decode layer's bytes (n_rec records
    chosen at random per launch among the arena's, plus one layer's router matrix) with
    moehip_stream_read, per grid: us per launch from HIP events over back-to-back launches on
    the stream they run on, rotating over 256 (layer, token) choices so that the records come
    from HBM. With stamp_grid, also the per-workgroup stamps of 12 launches at that grid."""
    import ctypes

    import torch

    from moelab_hip import _lib

    lib = _lib.load()
    n_all = arena.numel() // rec_bytes
    g = torch.Generator().manual_seed(seed)
    choices = []
    for j in range(256):
        recs = torch.randperm(n_all, generator=g)[:n_rec].tolist()
        bases = (ctypes.c_int64 * n_rec)(*[arena.data_ptr() + r * rec_bytes for r in recs])
        choices.append((bases, routers[j % len(routers)]))
    sink = torch.zeros(max(grids + [stamp_grid or 0]), dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev)
    rb = routers[0].numel() * routers[0].element_size()
    out = {}
    for grid in grids:
        def launch(j, stamps=None):
            bases, wr = choices[j % len(choices)]
            _lib.call("moehip_stream_read", bases, n_rec, rec_bytes, wr.data_ptr(), rb, grid, sink.data_ptr(),
                      _lib.ptr(stamps), st.cuda_stream)
        for j in range(256):
            launch(j)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for j in range(launches):
            launch(j)
        b.record(st)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1000 / launches
        out[grid] = us
        if grid == stamp_grid:
            ends, durs = [], []
            stamps = torch.zeros(2 * grid, dtype=torch.int64, device=dev)
            for j in range(12):
                launch(j)  # an untraced launch first: the traced one starts behind a busy GPU
                stamps.zero_()
                launch(j + 1, stamps)
                torch.cuda.synchronize()
                t = stamps.view(-1, 2).cpu()
                t0 = int(t[:, 0].min())
                ends += [(int(v) - t0) * 10 / 1000 for v in t[:, 1]]
                durs += [(int(e) - int(s_)) * 10 / 1000 for s_, e in t.tolist()]
            ends.sort()
            durs.sort()
            out["stamps"] = {"grid": grid, "data_in_median_us": ends[len(ends) // 2], "data_in_max_us": ends[-1],
                             "per_workgroup_median_us": durs[len(durs) // 2]}
    return out


def stream_line(args):
    """The read floor behind the headline: one launch reading what one OLMoE decode layer reads
    (8 int4 records of 3,342,336 B drawn from 16 x 64 of them, 3.42 GB, and the layer's 262,144 B
    router), without the dependencies of the decode (no routing before the record reads, no h
    exchange): us per launch at several grids, the decode kernel's own grid (768) among them."""
    import torch

    from moelab_hip import _lib

    dev = torch.device("cuda:0")
    _lib.check_device(dev)
    rec = 3_342_336
    arena = torch.ones(L * E * rec, dtype=torch.uint8, device=dev)
    routers = [torch.ones(E, H, dtype=torch.float16, device=dev) for _ in range(L)]
    grids = [256, 512, 768, 1024, 1536, 2048, 3072]
    r = stream_floor(dev, arena, routers, rec, K_TOP, grids, stamp_grid=768)
    nbytes = K_TOP * rec + E * H * 2
    per = {str(gd): {"us": round(r[gd], 3), "gbs": round(nbytes / (r[gd] * 1e-6) / 1e9, 1)} for gd in grids}
    best = min(grids, key=lambda gd: r[gd])
    # more bytes per launch: the launch's fixed costs against the transfer
    more = {}
    for n in (16, 32):
        rr = stream_floor(dev, arena, routers, rec, n, [1536, 3072])
        nb = n * rec + E * H * 2
        gd = min(rr, key=rr.get)
        more[f"{n}_records"] = {"bytes": nb, "grid": gd, "us": round(rr[gd], 3), "gbs": round(nb / (rr[gd] * 1e-6) / 1e9, 1)}
    log(f"[bench] stream floor, {nbytes} B per launch: " + ", ".join(f"grid {gd}: {r[gd]:.2f} us" for gd in grids))
    return {
        "metric": "dependency-free read floor of one OLMoE decode layer's bytes in one launch, 1 GPU",
        "value": round(nbytes / (r[768] * 1e-6) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": 2048, "warmup": 256,
        "ms_per_step": round(r[768] / 1000, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "8 int4 records (3,342,336 B) drawn at random per launch from 16 x 64 (3.42 GB) + "
                               "one 64 x 2048 fp16 router, read once by moehip_stream_read", "bytes_per_launch": nbytes},
        "per_grid": per, "best_grid": best, "stamps_grid_768": r.get("stamps"), "more_bytes": more,
        "roofline": {"bound": "hbm", "achieved": round(nbytes / (r[768] * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(nbytes / (r[768] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(STREAM_PROFILE),
                     "kernel": "k_stream_read (moehip_stream_read), grid 768"},
        "cpu_baseline": None,
    }


def cpu_baseline(seconds: float):
    """moelab's CPU expert branch (runtime.py:646-702: fp32 dequantize, F.linear, silu, add_ with
    alpha = w) restated in torch (oracle/cpu_path.py), on one OLMoE layer of 8 int4 records, all
    the cores this process may use (torch.set_num_threads), timed as hw.py:45-55 times it."""
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_path

    r = cpu_path.time_olmoe_layer(seconds, H, I, K_TOP)
    log(f"[bench] cpu baseline: {r['n']} layers in {r['seconds']:.1f} s on {r['threads']} threads ({r['cpu_model']})")
    return {"value": 1.0 / r["layer_s"], "unit": "layer-tok/s", "cores": r["threads"], "kind": "port",
            "host_cpus": r["host_cpus"], "cpu_model": r["cpu_model"],
            "sample": f"{r['n']} token-layers (OLMoE layer, 8 int4 gs64 records, torch fp32 dequantize + F.linear "
                      f"on {r['threads']} threads) in {r['seconds']:.1f} s; "
                      f"{r['k'] * r['record_bytes'] * r['n'] / r['seconds'] / 1e9:.3f} GB/s of records; "
                      f"16-layer stack tok/s = {1.0 / r['layer_s'] / L:.3f}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--tokens", type=int, default=16, help="distinct decode tokens (one graph each)")
    ap.add_argument("--kernel-launches", type=int, default=4096)
    ap.add_argument("--stage-stamps", action="store_true",
                    help="log each stage of the headline kernel's traced launches (median / max us)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    ap.add_argument("--workload", choices=["olmoe-decode-bs1", "qwen3-30b-prefill", "qwen3-next-offload", "dense-int8",
                                           "disk-tier", "stream-floor",
                                           *DECODE_SPECS, *BATCH_SPECS],
                    default="olmoe-decode-bs1")
    ap.add_argument("--offload-layers", type=int, default=48)
    ap.add_argument("--offload-steps", type=int, default=256)
    ap.add_argument("--offload-warmup", type=int, default=32)
    ap.add_argument("--offload-budget-gb", type=float, default=16.0,
                    help="offload: device budget of the 48-layer model (scaled to --offload-layers)")
    ap.add_argument("--stage-mode", choices=["auto", "kernel", "sdma"], default="auto")
    ap.add_argument("--prefetch-mass", type=float, default=None,
                    help="offload: stage the predicted experts up to this probability mass (at most 2k)")
    ap.add_argument("--prefetch-mode", choices=["kernel", "sdma"], default="sdma",
                    help="offload: how predicted experts are staged while the decode kernel runs")
    ap.add_argument("--disk-layers", type=int, default=4)
    ap.add_argument("--disk-reads", type=int, default=512)
    ap.add_argument("--disk-steps", type=int, default=64)
    ap.add_argument("--store-dir", default=None, help="where the disk-tier workload writes its store")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE-layer path here runs on a single MI355X "
              "(multi-GPU sharding is described, not run). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.workload == "qwen3-30b-prefill":
        print(json.dumps(prefill_line(args)), flush=True)
        return
    if args.workload == "qwen3-next-offload":
        print(json.dumps(offload_line(args)), flush=True)
        return
    if args.workload == "dense-int8":
        print(json.dumps(dense_line(args)), flush=True)
        return
    if args.workload == "disk-tier":
        print(json.dumps(disk_line(args)), flush=True)
        return
    if args.workload == "stream-floor":
        print(json.dumps(stream_line(args)), flush=True)
        return
    if args.workload in DECODE_SPECS:
        print(json.dumps(decode_line(args, args.workload)), flush=True)
        return
    if args.workload in BATCH_SPECS:
        print(json.dumps(batch_line(args, args.workload)), flush=True)
        return
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
        "kernel_us": round(r["kernel_us"], 3),
        "expert_phase": {"us": r["expert_phase_us"] and round(r["expert_phase_us"], 3),
                         "gbs": r["expert_phase_gbs"] and round(r["expert_phase_gbs"], 1),
                         "is": "8 records' bytes over the time from the first weight request to the last down "
                               "product inside a launch (per-workgroup stamps of traced launches)"},
        "roofline": {
            "bound": "hbm", "achieved": round(r["kernel_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": f"{r['kernel']} (router + routing + 8 int4 experts + combine, one launch per layer)",
            "bytes_per_launch": r["kernel_bytes"],
        },
        "cpu_baseline": cpu,
        "torch": torch.__version__,
    }
    line["parity"] = {"checked": f"token 0, {r['parity']['layers']} layers, torch fp32 reference before timing",
                      "max_abs": float(f"{r['parity']['max_abs']:.3g}"),
                      "mean_rel": float(f"{r['parity']['mean_rel']:.3g}")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
