"""
Device-resident experts and the whole-layer decode pipeline on the GPU.

`ResidentStore` keeps every record of L layers x E experts of each precision in HBM: one arena
per precision (record (l, e) at (l*E + e) * record_bytes, 4096-B aligned) and a device table
rtab (L, P, E) int64 of record base addresses, 0 = not resident (moelab/fullgraph.py:43-98;
layer-major so that one layer's (P, E) slice is contiguous for the decision kernel).

`MoEDecoder.layer(l, x)` runs one MoE layer for one decode token entirely on the GPU with no
host round trip, so a whole token can be captured in one HIP graph (moelab/fullgraph.py:117-192).
By default it is ONE launch of the fused decode-layer kernel (moehip_decode_layer): router,
softmax/top-k/renorm, HOBBIT levels + resident copy + tables, kernel-A and kernel-B rows and the
table-order combine. With fused=False the same steps run as separate launches:
  1. router: logits, softmax, top-k, renorm            (moehip_router_topk)
  2. HOBBIT levels + resident copy + kernel tables      (moehip_decide_table)
  3. kernel A per planned precision (acc zeroed by the first)   (moehip_grouped_up)
  4. kernel B per planned precision, table-order combine        (moehip_grouped_down)
  5. out = acc (+ cpu part), cast to the model dtype             (moehip_combine)
`miss` counts experts that were requested but had no usable resident copy, like FullMoE.flag.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kernels import _Plan, _combine
from .policy import PrecisionPolicy, level_to_precision
from .store import encode_record_, group_size_of, record_layout


class ResidentStore:
    def __init__(self, layouts: dict, num_layers: int, num_experts: int, device, precisions: list | None = None):
        self.device = torch.device(device)
        self.precisions = list(precisions or layouts)  # most precise first
        self.layouts = {p: layouts[p] for p in self.precisions}
        self.L, self.E = num_layers, num_experts
        self.arena = {}
        for p in self.precisions:
            rb = self.layouts[p]["record_bytes"]
            self.arena[p] = torch.zeros(num_layers * num_experts * rb, dtype=torch.uint8, device=self.device)
        self.present = torch.zeros(len(self.precisions), num_layers, num_experts, dtype=torch.bool)
        self.rtab = torch.zeros(num_layers, len(self.precisions), num_experts, dtype=torch.int64, device=self.device)

    def record_bytes(self, p: str) -> int:
        return self.layouts[p]["record_bytes"]

    def blob(self, p: str, layer: int, expert: int) -> torch.Tensor:
        rb = self.record_bytes(p)
        o = (layer * self.E + expert) * rb
        return self.arena[p][o:o + rb]

    def set_present(self, p: str, layer: int, expert: int, on: bool = True) -> None:
        pi = self.precisions.index(p)
        self.present[pi, layer, expert] = on
        self.rtab[layer, pi, expert] = self.blob(p, layer, expert).data_ptr() if on else 0

    def encode(self, p: str, layer: int, expert: int, gate_up: torch.Tensor, down: torch.Tensor) -> None:
        encode_record_(self.layouts[p], self.blob(p, layer, expert), gate_up, down)
        self.set_present(p, layer, expert)

    def fill_synthetic(self, generator: torch.Generator | None = None, std: float = 0.02,
                       precisions: list | None = None) -> None:
        """Random N(0, std) experts, quantised on the GPU with the store's packing."""
        for p in precisions or self.precisions:
            H, I = _dims(self.layouts[p])
            for l in range(self.L):
                for e in range(self.E):
                    gu = torch.randn(2 * I, H, device=self.device, generator=generator) * std
                    dn = torch.randn(H, I, device=self.device, generator=generator) * std
                    self.encode(p, l, e, gu, dn)

    @property
    def bytes_resident(self) -> int:
        return sum(int(self.present[i].sum()) * self.record_bytes(p) for i, p in enumerate(self.precisions))


def _dims(layout):
    from .store import dims
    return dims(layout)


class MoEDecoder:
    """One decode token through the MoE layers, all on the GPU (capturable)."""

    def __init__(self, store: ResidentStore, k: int, policy: PrecisionPolicy | None = None, dtype=torch.float16,
                 router_weights: list | None = None, renorm: bool = False, planned: list | None = None,
                 fused: bool = True, grid: int = 0, shared: list | None = None, one_token_rule: bool = False):
        """shared: per layer None or {"gate": (H,) tensor in dtype, "rec": {precision: record blob}}
        for a Qwen3-Next shared expert (out += sigmoid(x . gate) * FFN_s(x)); fused path only.
        one_token_rule: HOBBIT levels by the float64 rule of PrecisionPolicy.levels_one (moelab's
        default decode path, runtime.py:494-517) instead of the tensor rule of gpu_levels (the
        whole-token graph, fullgraph.py:101-114)."""
        self.store = store
        self.shared = shared
        self.k = k
        self.policy = policy or PrecisionPolicy("lo")
        self.dtype = dtype
        self.renorm = renorm
        self.router_weights = router_weights  # per layer (E, H) tensors in dtype, or None
        dev = store.device
        precs = store.precisions
        self.P = len(precs)
        planned = set(planned if planned is not None else precs)
        self.plans = {pi: _Plan(store.layouts[p]) for pi, p in enumerate(precs) if p in planned}
        H = _dims(store.layouts[precs[0]])[0]
        self.H = H
        E = store.E
        self.tab = torch.zeros(self.P, k, 4, dtype=torch.int64, device=dev)
        self.wtab = torch.zeros(self.P, k, dtype=torch.float32, device=dev)
        self.h = {pi: torch.empty(k, pl.I, dtype=torch.float32, device=dev) for pi, pl in self.plans.items()}
        for pl in self.plans.values():
            pl.partial(k, dev)
        self.offs = torch.tensor([_offs(store.layouts[p]) for p in precs], dtype=torch.int64, device=dev)
        self.planned_dev = torch.tensor([1 if pi in self.plans else 0 for pi in range(self.P)], dtype=torch.int32,
                                        device=dev)
        self.lv2p = (ctypes.c_int * 3)(*[precs.index(level_to_precision(v, precs)) for v in range(3)])
        self.acc = torch.zeros(H, dtype=torch.float32, device=dev)
        self.logits = torch.empty(1, E, dtype=dtype, device=dev)
        self.idx = torch.zeros(1, k, dtype=torch.int64, device=dev)
        self.w = torch.zeros(1, k, dtype=dtype, device=dev)
        self.w32 = torch.zeros(1, k, dtype=torch.float32, device=dev)
        self.info = torch.zeros(store.L, 3, k, dtype=torch.float32, device=dev)
        self.miss = torch.zeros(1, dtype=torch.float32, device=dev)
        self._pols = [self.policy.device_policy(l, one_token=one_token_rule) for l in range(store.L)]
        self.grid = grid
        self.trace = None  # optional int64 device tensor of 3 * (items + 3) + 8 * items: per-item stamps
        self.fused = fused and all(store.layouts[p]["precision"] != "fp32" for p in precs) and H <= 2048 \
            and _dims(store.layouts[precs[0]])[1] <= 2048
        if shared is not None and not self.fused:
            raise RuntimeError("MoEDecoder: the shared expert runs in the fused decode kernel only")
        if self.fused:
            self._descs = [self._desc(l) for l in range(store.L)]
            rows = k + (1 if shared is not None and any(s is not None for s in shared) else 0)
            nbytes = _lib.load().moehip_decode_layer_workspace_bytes(self.P, rows, E, H, self._descs[0].I)
            self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
            self.err = torch.zeros(1, dtype=torch.int32, device=dev)

    def _desc(self, layer: int) -> _lib.LayerDesc:
        st = self.store
        d = _lib.LayerDesc()
        d.P, d.E, d.k = self.P, st.E, self.k
        d.H, d.I = _dims(st.layouts[st.precisions[0]])
        d.dtype = _lib.dt_code(self.dtype)
        d.renorm = 1 if self.renorm else 0
        for pi, p in enumerate(st.precisions):
            lay = st.layouts[p]
            d.prec[pi] = _lib.prec_code(lay["precision"])
            gu, gd = group_size_of(lay)
            d.gs_up[pi], d.gs_dn[pi] = gu, gd
            d.planned[pi] = 1 if pi in self.plans else 0
            for f, o in enumerate(_offs(lay)):
                d.offs[pi][f] = o
        for v in range(3):
            d.lv2p[v] = self.lv2p[v]
        d.pol = self._pols[layer]
        sh = self.shared[layer] if self.shared is not None else None
        if sh is not None:
            g = sh["gate"]
            if g.dtype != self.dtype or g.numel() != d.H or not g.is_contiguous() or g.device != st.device:
                raise RuntimeError(f"shared gate of layer {layer}: ({d.H},) {self.dtype} contiguous on {st.device}")
            d.shared_gate = g.data_ptr()
            for pi, p in enumerate(st.precisions):
                blob = sh["rec"].get(p)
                d.shared_rec[pi] = 0 if blob is None else blob.data_ptr()
        return d

    def work_items(self) -> int:
        """Number of work items of one fused launch (router rows, up blocks, down blocks)."""
        n = _lib.load().moehip_decode_layer_work_items(ctypes.byref(self._descs[0]),
                                                        1 if self.router_weights is not None else 0)
        if n < 0:
            raise RuntimeError("moehip_decode_layer_work_items: bad layer description")
        return n

    def check_error(self) -> None:
        """Raise if a bounded wait inside the fused kernel expired on this decoder's workspace."""
        if self.fused:
            _lib.call("moehip_decode_layer_error", self.ws.data_ptr(), self.err.data_ptr(), _lib.stream_of(self.ws.device))
            if int(self.err.item()) != 0:
                raise RuntimeError("fused decode-layer kernel: a bounded wait expired (workspace error flag set)")

    def route(self, layer: int, x: torch.Tensor) -> None:
        Wr = self.router_weights[layer]
        E = self.store.E
        _lib.call("moehip_router_topk", x.data_ptr(), Wr.data_ptr(), 1, self.H, E, self.k, 1 if self.renorm else 0,
                  _lib.dt_code(self.dtype), self.logits.data_ptr(), self.idx.data_ptr(), self.w.data_ptr(),
                  self.w32.data_ptr(), _lib.stream_of(x.device))

    def decide(self, layer: int, idx: torch.Tensor, w32: torch.Tensor) -> None:
        st = self.store
        _lib.call("moehip_decide_table", idx.data_ptr(), w32.data_ptr(), self.k, ctypes.byref(self._pols[layer]),
                  self.lv2p, st.rtab[layer].data_ptr(),
                  self.P, st.E, self.offs.data_ptr(), self.planned_dev.data_ptr(), self.tab.data_ptr(),
                  self.wtab.data_ptr(), self.info[layer].data_ptr(), self.miss.data_ptr(), _lib.stream_of(idx.device))

    def experts(self, x: torch.Tensor, out: torch.Tensor, cpu_part: torch.Tensor | None = None,
                accumulate: bool = False) -> None:
        first = True
        for pi, plan in self.plans.items():
            plan.up(self.k, self.tab[pi], self.wtab[pi], x, self.h[pi], self.acc, zero=first)
            first = False
        if not self.plans:
            self.acc.zero_()
        for pi, plan in self.plans.items():
            plan.down(self.k, self.tab[pi], self.wtab[pi], self.h[pi], self.acc)
        _combine(self.acc, out, cpu_part, accumulate=accumulate)

    def layer(self, layer: int, x: torch.Tensor, out: torch.Tensor, idx: torch.Tensor | None = None,
              w32: torch.Tensor | None = None, cpu_part: torch.Tensor | None = None,
              accumulate: bool = False) -> torch.Tensor:
        """out (1, H) = MoE layer `layer` applied to x (1, H) (+ out if accumulate) (+ cpu_part, the
        partial of experts run elsewhere), summed in fp32 in that order. With idx/w32 given, the
        router is skipped."""
        if self.fused:
            st = self.store
            Wr = None if idx is not None else self.router_weights[layer]
            _lib.call("moehip_decode_layer", ctypes.byref(self._descs[layer]), x.data_ptr(), _lib.ptr(Wr),
                      _lib.ptr(idx), _lib.ptr(w32), st.rtab[layer].data_ptr(), out.data_ptr(), _lib.ptr(cpu_part),
                      1 if accumulate else 0,
                      self.logits.data_ptr(), self.idx.data_ptr() if idx is None else None,
                      self.w.data_ptr() if idx is None else None, self.w32.data_ptr() if idx is None else None,
                      self.info[layer].data_ptr(), self.miss.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                      self.grid, _lib.ptr(self.trace), _lib.stream_of(x.device))
            return out
        if idx is None:
            self.route(layer, x)
            idx, w32 = self.idx, self.w32
        self.decide(layer, idx, w32)
        self.experts(x, out, cpu_part, accumulate)
        return out


def _offs(layout):
    from .store import field_offsets
    return field_offsets(layout)


def olmoe_layouts(H: int = 2048, I: int = 1024, precs=("int4",)) -> dict:
    return {p: record_layout(p, H, I, 64, scale="absmax" if p in ("int4", "int8") else None) for p in precs}
