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

import ctypes

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
def _table(entries, keys, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Address table (n, 4) int64 + weights (n,) fp32 of [(views, weight)] on `device`
    (kernels.py:230-244): one host buffer from torch's pinned-memory cache, one asynchronous copy
    (the cache keeps the buffer until the copy has run, so nothing waits here)."""
    n = len(entries)
    dev = torch.device(device)
    host = torch.empty(n * 36, dtype=torch.uint8, pin_memory=dev.type == "cuda")
    host[: n * 32].view(torch.int64).numpy().reshape(n, 4)[:] = [[v[key].data_ptr() for key in keys] for v, _ in entries]
    host[n * 32:].view(torch.float32).numpy()[:] = [float(w) for _, w in entries]
    out = host.to(dev, non_blocking=True)
    return out[: n * 32].view(torch.int64).view(n, 4), out[n * 32:].view(torch.float32)


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
def _fused_ok(layouts: dict, dtype) -> bool:
    """The layouts the one-launch layer kernel takes (16-bit or fp32 activations, no fp32 records,
    d_model and d_ff <= 2048 and multiples of 32)."""
    for lay in layouts.values():
        H, I = dims(lay)
        if lay["precision"] == "fp32" or H > 2048 or I > 2048 or H % 32 or I % 32:
            return False
    return dtype in _lib.DT_CODES


class GroupedGraph:
    """One MoE layer's grouped expert computation for one decode token, replayed as a HIP graph
    (interface of kernels.py:909-984: GroupedGraph(layouts, x, out, k, version, capture),
    .run(items, cpu_out), .supports(prec); attributes graph / runs / replays / out / x / k /
    version).

    Per token the host writes one request block: for every precision p (layouts' order) k rows of
    (record base address int64, router weight fp32), 12 bytes a row, unused rows 0 (the field
    offsets are static and applied on the device). The block travels in ONE host-to-device copy,
    then ONE launch of the layer kernel on explicit rows (moehip_decode_rows) runs every row's
    gate/up and down products and writes out = sum of the rows in table order + cpu_part. Two
    request blocks alternate, each with its own graph and the event of its last copy: the host
    waits on that event before rewriting a block, so it never overwrites a block whose copy is
    still queued. Layouts the layer kernel does not take (fp32 records, d_model or d_ff above
    2048) run kernels A and B per precision instead, from the same request block."""

    NBLOCKS = 2

    def __init__(self, layouts: dict, x: torch.Tensor, out: torch.Tensor, k: int, version: int = 2,
                 capture: bool = True):
        self.dev = x.device
        self.x, self.out, self.k, self.version = x.reshape(-1), out, k, version
        self.precs = list(layouts)
        self.layouts = dict(layouts)
        self.plans: dict[str, _Plan] = {p: _Plan(lay, version) for p, lay in layouts.items()}
        P = len(self.precs)
        cuda = self.dev.type == "cuda"
        self.blocks = []
        for _ in range(self.NBLOCKS):
            host = torch.zeros(P * k * 12, dtype=torch.uint8, pin_memory=cuda)
            devb = torch.zeros_like(host, device=self.dev)
            self.blocks.append({
                "host": host, "dev": devb, "event": None, "graph": None,
                "bases": host[: P * k * 8].view(torch.int64).numpy().reshape(P, k),
                "weights": host[P * k * 8:].view(torch.float32).numpy().reshape(P, k),
                "dev_bases": devb[: P * k * 8].view(torch.int64), "dev_weights": devb[P * k * 8:].view(torch.float32),
            })
        self.cpu_part = torch.zeros_like(out)
        self.cpu_dirty = False
        self.fused = cuda and _fused_ok(self.layouts, self.x.dtype) and self.out.is_contiguous()
        if self.fused:
            self.desc = self._desc()
            n = _lib.load().moehip_decode_rows_workspace_bytes(P, k, self.desc.H, self.desc.I)
            self.ws = torch.zeros(n, dtype=torch.uint8, device=self.dev)
        else:
            H = out.shape[-1]
            self.offs = torch.tensor([field_offsets(self.layouts[p]) for p in self.precs], dtype=torch.int64,
                                     device=self.dev)
            self.h = {p: torch.empty(k, plan.I, dtype=torch.float32, device=self.dev) for p, plan in self.plans.items()}
            self.acc = torch.empty(H, dtype=torch.float32, device=self.dev)
            self.tabs = torch.zeros(P, k, 4, dtype=torch.int64, device=self.dev)
            for plan in self.plans.values():
                plan.partial(k, self.dev)
        self.capture = capture and cuda
        self.replays = 0
        self.runs = 0
        self._last = None

    @property
    def graph(self):
        """The graph of the block the last run used (None before the first capture)."""
        return None if self._last is None else self._last["graph"]

    def supports(self, prec: str) -> bool:
        return prec in self.plans

    def _desc(self) -> _lib.LayerDesc:
        d = _lib.LayerDesc()
        d.P, d.E, d.k = len(self.precs), 1, self.k
        d.H, d.I = self.plans[self.precs[0]].H, self.plans[self.precs[0]].I
        d.dtype = _lib.dt_code(self.x.dtype)
        for pi, p in enumerate(self.precs):
            plan = self.plans[p]
            if (plan.H, plan.I) != (d.H, d.I):
                raise ValueError("GroupedGraph: every layout must have the same d_model and d_ff")
            d.prec[pi] = plan.code
            d.gs_up[pi], d.gs_dn[pi] = plan.g_up, plan.g_dn
            d.planned[pi] = 1
            for f, o in enumerate(plan.offs):
                d.offs[pi][f] = o
        return d

    def _launches(self, blk: dict) -> None:
        """What one replay enqueues: the request copy, then the layer."""
        blk["dev"].copy_(blk["host"], non_blocking=True)
        stream = _lib.stream_of(self.dev)
        if self.fused:
            _lib.call("moehip_decode_rows", ctypes.byref(self.desc), self.x.data_ptr(), blk["dev_bases"].data_ptr(),
                      blk["dev_weights"].data_ptr(), self.out.data_ptr(), self.cpu_part.data_ptr(), 0,
                      self.ws.data_ptr(), self.ws.numel(), stream)
            return
        bases = blk["dev_bases"].view(len(self.precs), self.k, 1)
        torch.mul(bases + self.offs.view(-1, 1, 4), (bases != 0).to(torch.int64), out=self.tabs)
        w = blk["dev_weights"].view(len(self.precs), self.k)
        for pi, p in enumerate(self.precs):
            self.plans[p].up(self.k, self.tabs[pi], w[pi], self.x, self.h[p], self.acc, zero=pi == 0)
        for pi, p in enumerate(self.precs):
            self.plans[p].down(self.k, self.tabs[pi], w[pi], self.h[p], self.acc)
        _combine(self.acc, self.out, self.cpu_part, accumulate=False)

    def run(self, items: dict, cpu_out: torch.Tensor | None = None) -> None:
        """items: {precision: [(record on the GPU, weight), ...]} (at most k per precision);
        cpu_out: the sum of the experts computed on the CPU, added to the result."""
        self.runs += 1
        blk = self.blocks[self.runs % self.NBLOCKS]
        if blk["event"] is not None:
            blk["event"].synchronize()  # that block's previous copy has run (long ago, in practice)
        bases, weights = blk["bases"], blk["weights"]
        bases[:] = 0
        weights[:] = 0.0
        for p, rows in items.items():
            if p not in self.plans:
                raise ValueError(f"GroupedGraph: no layout for precision {p}")
            if len(rows) > self.k:
                raise ValueError(f"{len(rows)} {p} experts for a table of {self.k} rows")
            pi = self.precs.index(p)
            for j, (blob, wt) in enumerate(rows):
                bases[pi, j] = blob.data_ptr()
                weights[pi, j] = wt
        if cpu_out is not None:
            self.cpu_part.copy_(cpu_out)
            self.cpu_dirty = True
        elif self.cpu_dirty:
            self.cpu_part.zero_()
            self.cpu_dirty = False
        self._last = blk
        if not self.capture:
            self._launches(blk)
        elif blk["graph"] is not None:
            blk["graph"].replay()
            self.replays += 1
        else:  # first token: run it, then capture every block's launches for the later tokens
            self._launches(blk)
            torch.cuda.synchronize(self.dev)
            for b in self.blocks:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._launches(b)
                b["graph"] = g
        if self.dev.type == "cuda":
            ev = torch.cuda.Event()
            ev.record()
            blk["event"] = ev


def grouped_graph_gpu_ms(layout: dict, x, out, k: int, version: int, items: dict, repeat: int = 50) -> float:
    """GPU milliseconds of one grouped computation of k experts as a graph replay (kernels.py:
    590-602): both request blocks are captured, then `repeat` replays alternate between them."""
    gg = GroupedGraph({layout["precision"]: layout}, x, out, k, version=version)
    for _ in range(GroupedGraph.NBLOCKS):  # both request blocks hold the same rows
        gg.run(items)
    graphs = [b["graph"] for b in gg.blocks]
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(repeat):
        graphs[i % len(graphs)].replay()
    t1.record()
    t1.synchronize()
    return t0.elapsed_time(t1) / repeat


AUTO_CANDIDATES = (2,)


def pick_int4_version(layout: dict, device, k: int = 8) -> int:
    """One HIP kernel family: always 2 (the name is kept for the runtime, kernels.py:611-642)."""
    return 2
