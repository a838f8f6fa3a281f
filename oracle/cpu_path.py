"""
Torch restatement (CPU) of moelab's CPU expert branch — the reported CPU baseline of bench.py.

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ use it; the product never imports
it. It restates, in torch on the host cores:
  - quant.py:191-205 `dequantize` (int4: low nibble = even column, value - 8; times the group's
    fp16 scale, in the compute dtype) and store.py:164-174 `materialize`;
  - runtime.py:165-168 `expert_ffn` (F.linear to gate/up, silu(gate) * up, F.linear to down);
  - runtime.py:682-697 the decode branch: out_cpu (T, H) zeros, then out_cpu.add_(y, alpha=w) per
    expert, in the order given;
  - hw.py:45-55 `measure_host_compute`'s timing (one warm call, then n timed calls).
Record bytes come from oracle.moe_ref's record_layout (the store's layout, store.py:76-115).
"""

from __future__ import annotations

import os
import platform
import time

import numpy as np
import torch
import torch.nn.functional as F

from . import moe_ref as O


def dequantize(q: torch.Tensor, s: torch.Tensor, bits: int, dtype=torch.float32) -> torch.Tensor:
    """quant.py:191-205."""
    rows = q.shape[0]
    if bits == 8:
        vals = q.to(dtype)
    else:
        vals = torch.stack((q & 0x0F, q >> 4), dim=-1).reshape(rows, 2 * q.shape[1]).to(dtype) - 8
    cols = vals.shape[1]
    gs = cols // s.shape[1]
    return (vals.reshape(rows, cols // gs, gs) * s.to(dtype).unsqueeze(-1)).reshape(rows, cols)


def materialize(layout: dict, blob: torch.Tensor, dtype=torch.float32):
    """store.py:164-174 for int4 / int8 / float records: (gate_up, down) in `dtype`."""
    v = {}
    for name, shape, dt, off in layout["fields"]:
        nb = O.ELEM_SIZE[dt] * int(np.prod(shape))
        tdt = {"uint8": torch.uint8, "int8": torch.int8, "float16": torch.float16, "bfloat16": torch.bfloat16,
               "float32": torch.float32}[dt]
        v[name] = blob[off:off + nb].view(tdt).view(*shape)
    prec = layout["precision"]
    if prec in ("int4", "int8"):
        bits = 4 if prec == "int4" else 8
        return (dequantize(v["gate_up.q"], v["gate_up.s"], bits, dtype),
                dequantize(v["down.q"], v["down.s"], bits, dtype))
    return v["gate_up"].to(dtype), v["down"].to(dtype)


def expert_ffn(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """runtime.py:165-168 with act_fn = silu."""
    gate, up = F.linear(x, gate_up).chunk(2, dim=-1)
    return F.linear(F.silu(gate) * up, down)


def cpu_layer(x: torch.Tensor, entries, layouts: dict, dtype=torch.float32) -> torch.Tensor:
    """runtime.py:682-697 (decode): x (1, H); entries [(precision, record uint8 tensor, weight)]."""
    xc = x.to("cpu", dtype)
    out = torch.zeros(xc.shape[0], xc.shape[1], dtype=dtype)
    for prec, blob, w in entries:
        out.add_(expert_ffn(xc, *materialize(layouts[prec], blob, dtype)), alpha=w)
    return out


def host_threads() -> int:
    """The cores this process may use: its CPU affinity, capped by OMP_NUM_THREADS when set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def time_olmoe_layer(seconds: float, H: int = 2048, I: int = 1024, k: int = 8, seed: int = 0) -> dict:
    """One OLMoE layer on the CPU path: k int4 gs64 absmax records of N(0, 0.02) weights (the
    oracle's encoder: moelab's packing and fp16 scales), x (1, H) ~ N(0, 1) rounded to fp16, weight
    1/k each; one warm call, then timed calls for about `seconds`."""
    threads = host_threads()
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    lay = O.record_layout("int4", H, I, 64, scale="absmax")
    blobs = [torch.from_numpy(O.encode_record(lay, (rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32),
                                              (rng.standard_normal((H, I)) * 0.02).astype(np.float32), "absmax"))
             for _ in range(k)]
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float16))
    entries = [("int4", b, 1.0 / k) for b in blobs]
    cpu_layer(x, entries, {"int4": lay})  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        cpu_layer(x, entries, {"int4": lay})
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"layer_s": el / n, "n": n, "seconds": el, "threads": threads, "host_cpus": os.cpu_count(),
            "cpu_model": cpu_model(), "record_bytes": lay["record_bytes"], "k": k}


def time_prefill_layer(seconds: float, H: int = 2048, I: int = 768, E: int = 128, k: int = 8, T: int = 512,
                       seed: int = 0) -> dict:
    """A prefill chunk on the CPU path (runtime.py:418-436 `_run_grouped_tokens` with the experts on
    the host: per expert the rows of its tokens, `materialize`, `expert_ffn`, then
    out.index_add_(0, rows, y * w) as runtime.py:352-353), fp32, on a bounded sample: experts of
    T * k / E tokens each (the chunk's average), as many as fit in about `seconds`; the layer time is
    the per-expert time times E."""
    threads = host_threads()
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    lay = O.record_layout("int4", H, I, 64, scale="absmax")
    n_rec = 4
    blobs = [torch.from_numpy(O.encode_record(lay, (rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32),
                                              (rng.standard_normal((H, I)) * 0.02).astype(np.float32), "absmax"))
             for _ in range(n_rec)]
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32))
    per = max(1, T * k // E)
    out = torch.zeros(T, H)

    def one(i):
        rows = torch.from_numpy(rng.choice(T, per, replace=False))
        w = torch.from_numpy(rng.random(per).astype(np.float32))
        gu, dn = materialize(lay, blobs[i % n_rec], torch.float32)
        y = expert_ffn(x.index_select(0, rows), gu, dn)
        out.index_add_(0, rows, y * w[:, None])

    one(0)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        one(n)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"expert_s": el / n, "layer_s": el / n * E, "n": n, "seconds": el, "threads": threads,
            "tokens_per_expert": per, "host_cpus": os.cpu_count(), "cpu_model": cpu_model()}
