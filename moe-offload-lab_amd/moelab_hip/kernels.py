"""
Drop-in replacement for moelab's `kernels` module (moelab/kernels.py), backed by hand-written
HIP kernels for gfx950 (libmoehip.so) instead of Triton.

Same names and semantics as the names moelab's runtime imports (runtime.py:34-35,
fullgraph.py:38, profiling.py:134-158):

- gemv_int4, expert_ffn_int4                      (kernels.py:60-74)
- grouped_ffn_int4 / grouped_ffn_int8 / grouped_ffn_float: out (1, H) += sum_e w_e * expert_e(x)
                                                  (kernels.py:834-891, 747-769)
- grouped_ffn_fp8                                 (new: block-scaled fp8 records)
- _Plan(layout, version).up / .down / .offs / .I / .H   (kernels.py:772-831)
- GroupedGraph(layouts, x, out, k, version, capture) with .run(items, cpu_out), .supports
                                                  (kernels.py:909-984), captured in a HIP graph
- pick_int4_version, grouped_graph_gpu_ms, triton_usable, _pow2_groups, _pow2_groups8, _even,
  _tuned, _table, HAVE_TRITON, INTERPRET          (kernels bookkeeping names)

Differences, all deliberate:
- there is one kernel family; `version` is accepted and ignored (pick_int4_version returns 2);
- kernel B combines experts in table order (deterministic), not with fp32 atomics;
- the grouped kernels take any even group size, so `_pow2_groups*` only reject odd sizes;
- errors raise RuntimeError (the runtime's existing try/except fallbacks still apply) and there
  is no silent CPU path: on a machine without a gfx950 GPU `triton_usable` is False.
"""

from __future__ import annotations

import torch

from . import _lib
from .store import dims, field_offsets, group_size_of

HAVE_TRITON = False  # no Triton behind this module (kept so `from kernels import HAVE_TRITON` works)
INTERPRET = False
HAVE_HIP = _lib.available()


def triton_usable(device) -> bool:
    """The runtime's "fast kernels usable on this device" predicate (kernels.py:77-82): True on
    a gfx950 GPU with libmoehip loaded."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return False
    try:
        _lib.check_device(dev)
    except RuntimeError:
        return False
    return True


def _tuned(key, restore=None):
    """No autotuner: launch shapes are fixed per shape class in the HIP host code."""
    return lambda f: f


def _even(*pairs) -> bool:
    return all(d % m == 0 for d, m in pairs)


def _pow2_groups(groups: dict) -> bool:
    """Grouped int4 kernels support these group sizes (any even size here)."""
    return all(g > 0 and g % 2 == 0 for g in (groups["gate_up"], groups["down"]))


def _pow2_groups8(groups: dict) -> bool:
    return _pow2_groups(groups)


def _check_x(x: torch.Tensor) -> None:
    if x.device.type != "cuda":
        raise RuntimeError("moehip kernels run on the GPU; got a tensor on " + str(x.device))
    _lib.check_device(x.device)


# ---------------------------------------------------------------------------------------
# single-matrix GEMV and one-expert FFN
# ---------------------------------------------------------------------------------------
def gemv_int4(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor, group_size: int) -> torch.Tensor:
    """y = W @ x with W int4 (q (O, I/2) u8, s (O, I/gs) f16); x (I,); returns (O,) in x.dtype."""
    _check_x(x)
    O, P = q.shape
    I = 2 * P
    if q.stride(-1) != 1 or s.stride(-1) != 1 or q.stride(0) != P or s.stride(0) != I // group_size:
        q, s = q.contiguous(), s.contiguous()
    x = x.reshape(-1).contiguous()
    if x.numel() != I:
        raise ValueError(f"x has {x.numel()} values, W has {I} columns")
    y = torch.empty(O, dtype=x.dtype, device=x.device)
    _lib.call("moehip_gemv_int4", q.data_ptr(), s.data_ptr(), x.data_ptr(), y.data_ptr(), O, I, group_size,
              _lib.dt_code(x.dtype), _lib.stream_of(x.device))
    return y


def expert_ffn_int4(x_row: torch.Tensor, v: dict, groups: dict, act_fn) -> torch.Tensor:
    """One int4 expert for ONE token: down(act(gate x) * up x) without dequantising (kernels.py:70-74)."""
    h = gemv_int4(v["gate_up.q"], v["gate_up.s"], x_row.reshape(-1), groups["gate_up"])
    gate, up = h.chunk(2)
    return gemv_int4(v["down.q"], v["down.s"], act_fn(gate) * up, groups["down"]).reshape(1, -1)


# ---------------------------------------------------------------------------------------
# tables
# ---------------------------------------------------------------------------------------
class _Staging:
    """Pinned host ring for table uploads without a host sync (kernels.py:195-224)."""

    def __init__(self, slots: int = 32, nbytes: int = 4096):
        self.nbytes = nbytes
        self.bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(slots)]
        self.events: list = [None] * slots
        self.i = 0

    def send(self, host: torch.Tensor, device) -> torch.Tensor:
        n = host.numel()
        if n > self.nbytes:
            return host.to(device)
        i = self.i
        self.i = (i + 1) % len(self.bufs)
        if self.events[i] is not None:
            self.events[i].synchronize()
        buf = self.bufs[i][:n]
        buf.copy_(host)
        dev = torch.empty(n, dtype=torch.uint8, device=device)
        dev.copy_(buf, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.events[i] = ev
        return dev


_staging: _Staging | None = None


def _table(entries, keys, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Address table (n, 4) int64 + weights (n,) fp32 on `device`, one async upload (kernels.py:230-244)."""
    global _staging
    n = len(entries)
    buf = torch.empty(n * 36, dtype=torch.uint8)
    buf[: n * 32].view(torch.int64).copy_(
        torch.tensor([[v[k].data_ptr() for k in keys] for v, _ in entries], dtype=torch.int64).reshape(-1))
    buf[n * 32:].view(torch.float32).copy_(torch.tensor([float(w) for _, w in entries], dtype=torch.float32))
    if torch.device(device).type == "cuda":
        if _staging is None:
            _staging = _Staging()
        dev = _staging.send(buf, device)
    else:
        dev = buf.to(device)
    return dev[: n * 32].view(torch.int64).view(n, 4), dev[n * 32:].view(torch.float32)


# ---------------------------------------------------------------------------------------
# plans: the two launches of one precision
# ---------------------------------------------------------------------------------------
class _Plan:
    """Dimensions and launches of kernels A/B for one record layout (kernels.py:772-831)."""

    def __init__(self, layout: dict, version: int = 2):
        self.layout = layout
        self.prec = layout["precision"]
        self.code = _lib.prec_code(self.prec)
        self.kind = self.prec if self.prec in ("int4", "int8", "fp8") else "float"
        self.H, self.I = dims(layout)
        self.g_up, self.g_dn = group_size_of(layout)
        self.offs = field_offsets(layout)
        self.version = version
        self._partial: dict = {}

    def partial(self, n: int, device) -> torch.Tensor:
        key = (n, torch.device(device))
        p = self._partial.get(key)
        if p is None:
            p = torch.empty(max(1, n * self.H), dtype=torch.float32, device=device)
            self._partial[key] = p
        return p

    def up(self, n, tab, w, x, h, acc, zero: bool):
        """h[e] = silu(gate_e x) * (up_e x) for the n table rows; acc zeroed first if `zero`."""
        _lib.call("moehip_grouped_up", self.code, tab.data_ptr(), w.data_ptr(), x.data_ptr(),
                  _lib.dt_code(x.dtype), h.data_ptr(), acc.data_ptr() if zero else None, n, self.I, self.H,
                  self.g_up, _lib.stream_of(x.device))

    def down(self, n, tab, w, h, acc):
        """acc += sum_e w_e * (down_e h[e]), experts added in table order."""
        part = self.partial(n, h.device)
        _lib.call("moehip_grouped_down", self.code, tab.data_ptr(), w.data_ptr(), h.data_ptr(), acc.data_ptr(),
                  n, self.H, self.I, self.g_dn, part.data_ptr(), _lib.stream_of(h.device))


def _combine(acc: torch.Tensor, out: torch.Tensor, add: torch.Tensor | None = None, accumulate: bool = True):
    T = out.numel() // acc.shape[-1] if out.dim() > 1 else 1
    _lib.call("moehip_combine", acc.data_ptr(), add.data_ptr() if add is not None else None, out.data_ptr(), T,
              acc.shape[-1], _lib.dt_code(out.dtype), 1 if accumulate else 0, _lib.stream_of(out.device))


def _grouped(x_row: torch.Tensor, entries: list, layout: dict, out: torch.Tensor) -> None:
    _check_x(x_row)
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    plan = _Plan(layout)
    n = len(entries)
    dev = x_row.device
    keys = ("gate_up.q", "gate_up.s", "down.q", "down.s") if plan.kind != "float" else ("gate_up", "gate_up", "down", "down")
    tab, w = _table(entries, keys, dev)
    h = torch.empty(n, plan.I, dtype=torch.float32, device=dev)
    acc = torch.empty(plan.H, dtype=torch.float32, device=dev)
    x = x_row.reshape(-1).contiguous()
    plan.up(n, tab, w, x, h, acc, zero=True)
    plan.down(n, tab, w, h, acc)
    _combine(acc, out, accumulate=True)


def _layout_from_views(v: dict, prec: str) -> dict:
    from .store import record_layout
    if prec == "int4":
        two_i, ph = v["gate_up.q"].shape
        H, pi = v["down.q"].shape
        gs_up = 2 * ph // v["gate_up.s"].shape[1]
        gs_dn = 2 * pi // v["down.s"].shape[1]
        lay = record_layout("int4", H, two_i // 2, max(gs_up, gs_dn))
        lay["group_sizes"] = {"gate_up": gs_up, "down": gs_dn}
        return lay
    if prec == "int8":
        two_i, H = v["gate_up.q"].shape
        gs_up = H // v["gate_up.s"].shape[1]
        gs_dn = v["down.q"].shape[1] // v["down.s"].shape[1]
        lay = record_layout("int8", H, two_i // 2, max(gs_up, gs_dn))
        lay["group_sizes"] = {"gate_up": gs_up, "down": gs_dn}
        return lay
    if prec == "fp8":
        two_i, H = v["gate_up.q"].shape
        return record_layout("fp8", H, two_i // 2)
    two_i, H = v["gate_up"].shape
    name = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[v["gate_up"].dtype]
    return record_layout(name, H, two_i // 2)


def grouped_ffn_int4(x_row: torch.Tensor, entries: list, groups: dict, out: torch.Tensor, version: int = 2) -> None:
    """out (1, H) += sum of the int4 experts; entries = [(views(record), router weight)] (kernels.py:834-872)."""
    lay = _layout_from_views(entries[0][0], "int4")
    lay["group_sizes"] = dict(groups)
    _grouped(x_row, entries, lay, out)


def grouped_ffn_int8(x_row: torch.Tensor, entries: list, layout: dict, out: torch.Tensor) -> None:
    """out (1, H) += sum of the int8 experts (kernels.py:747-769)."""
    _grouped(x_row, entries, layout, out)


def grouped_ffn_float(x_row: torch.Tensor, entries: list, out: torch.Tensor) -> None:
    """Same for fp16 / bf16 / fp32 records (kernels.py:875-891)."""
    _grouped(x_row, entries, _layout_from_views(entries[0][0], "float"), out)


def grouped_ffn_fp8(x_row: torch.Tensor, entries: list, out: torch.Tensor) -> None:
    """Same for block-scaled fp8 records (the checkpoint format of moelab/quant.py:208-219)."""
    _grouped(x_row, entries, _layout_from_views(entries[0][0], "fp8"), out)


# ---------------------------------------------------------------------------------------
# per-layer graph (kernels.py:909-984)
# ---------------------------------------------------------------------------------------
class GroupedGraph:
    """The grouped computation of one MoE layer replayed as one HIP graph: pinned host table ->
    device table copy, kernels A then B for each precision, out = acc + cpu_part. Per token the
    host writes k addresses and k weights per precision and replays (one launch)."""

    def __init__(self, layouts: dict, x: torch.Tensor, out: torch.Tensor, k: int, version: int = 2,
                 capture: bool = True):
        self.dev = x.device
        self.x, self.out, self.k, self.version = x.reshape(-1), out, k, version
        self.plans: dict[str, _Plan] = {p: _Plan(lay, version) for p, lay in layouts.items()}
        H = out.shape[-1]
        pin = self.dev.type == "cuda"
        self.tabs = {}
        for p, plan in self.plans.items():
            host = torch.zeros(k * 36, dtype=torch.uint8, pin_memory=pin)
            dev = torch.empty_like(host, device=self.dev)
            self.tabs[p] = {
                "host": host, "dev": dev,
                "tab_np": host[: k * 32].view(torch.int64).numpy(), "w_np": host[k * 32:].view(torch.float32).numpy(),
                "tab": dev[: k * 32].view(torch.int64), "w": dev[k * 32:].view(torch.float32),
                "h": torch.empty(k, plan.I, dtype=torch.float32, device=self.dev),
            }
            plan.partial(k, self.dev)
        self.acc = torch.empty(H, dtype=torch.float32, device=self.dev)
        self.cpu_part = torch.zeros_like(out)
        self.cpu_dirty = False
        self.capture = capture and self.dev.type == "cuda"
        self.graph = None
        self.replays = 0
        self.runs = 0

    def supports(self, prec: str) -> bool:
        return prec in self.plans

    def _sequence(self) -> None:
        for t in self.tabs.values():
            t["dev"].copy_(t["host"], non_blocking=True)
        first = True
        for p, plan in self.plans.items():
            t = self.tabs[p]
            plan.up(self.k, t["tab"], t["w"], self.x, t["h"], self.acc, zero=first)
            first = False
        for p, plan in self.plans.items():
            t = self.tabs[p]
            plan.down(self.k, t["tab"], t["w"], t["h"], self.acc)
        _combine(self.acc, self.out, self.cpu_part, accumulate=False)

    def run(self, items: dict, cpu_out: torch.Tensor | None = None) -> None:
        """items: {precision: [(record on the GPU, weight), ...]}; cpu_out: sum of the CPU-computed experts."""
        self.runs += 1
        for p, t in self.tabs.items():
            tab, w = t["tab_np"], t["w_np"]
            tab[:] = 0
            w[:] = 0.0
            offs = self.plans[p].offs
            rows = items.get(p, ())
            if len(rows) > self.k:
                raise ValueError(f"{len(rows)} {p} experts for a table of {self.k} rows")
            for j, (blob, wt) in enumerate(rows):
                base = blob.data_ptr()
                tab[4 * j: 4 * j + 4] = [base + o for o in offs]
                w[j] = wt
        if cpu_out is not None:
            self.cpu_part.copy_(cpu_out)
            self.cpu_dirty = True
        elif self.cpu_dirty:
            self.cpu_part.zero_()
            self.cpu_dirty = False
        if not self.capture:
            self._sequence()
            return
        if self.graph is not None:
            self.graph.replay()
            self.replays += 1
            return
        self._sequence()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._sequence()
        self.graph = g
        torch.cuda.synchronize()


def grouped_graph_gpu_ms(layout: dict, x, out, k: int, version: int, items: dict, repeat: int = 50) -> float:
    """GPU time of one grouped computation (k experts) replayed as a graph (kernels.py:590-602)."""
    gg = GroupedGraph({layout["precision"]: layout}, x, out, k, version=version)
    gg.run(items)
    gg.run(items)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(repeat):
        gg.graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / repeat


AUTO_CANDIDATES = (2,)


def pick_int4_version(layout: dict, device, k: int = 8) -> int:
    """One HIP kernel family: always 2 (the name is kept for the runtime, kernels.py:611-642)."""
    return 2
