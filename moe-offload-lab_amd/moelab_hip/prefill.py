"""
T > 1 tokens through one layer's experts on the GPU (prefill chunks, batched decode).

Replaces moelab/runtime.py:418-436 (`_run_grouped_tokens`: per expert, expert_ffn on the
expert's tokens) and runtime.py:352-353 (`out.index_add_(0, tok, y * w)`) for int4 gs64 records:
moehip_dispatch sorts the (token, slot) pairs by expert (stable, as runtime.py:459-492), then
moehip_grouped_gemm runs the gate/up and down GEMMs of every routed expert on MFMA and sums each
token's slots in slot order. Everything is on the device and capturable; nothing is copied to
the host.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .store import dims, field_offsets, group_size_of


class GroupedTokens:
    """Per-layer runner for up to `max_tokens` tokens with top-`k` routing over `num_experts`
    experts stored in `layout` (int4 gs64)."""

    def __init__(self, layout: dict, num_experts: int, k: int, max_tokens: int, device):
        if layout["precision"] != "int4" or group_size_of(layout) != (64, 64):
            raise RuntimeError("GroupedTokens runs int4 gs64 records")
        self.layout = layout
        self.H, self.I = dims(layout)
        self.E, self.k, self.max_tokens = num_experts, k, max_tokens
        self.device = torch.device(device)
        _lib.check_device(self.device)
        lib = _lib.load()
        n = lib.moehip_grouped_gemm_workspace_bytes(max_tokens, k, self.H, self.I)
        self.ws = torch.empty(n, dtype=torch.uint8, device=self.device)
        self.counts = torch.empty(num_experts, dtype=torch.int32, device=self.device)
        self.offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=self.device)
        self.sorted_pos = torch.empty(max_tokens * k, dtype=torch.int32, device=self.device)
        self.rank = torch.empty(max_tokens * k, dtype=torch.int32, device=self.device)
        self.offs = torch.tensor(field_offsets(layout), dtype=torch.int64, device=self.device)
        self._route_bufs = None
        # the one-call layer (moehip_prefill_layer): its own workspace, zeroed once (routing counters)
        n = lib.moehip_prefill_layer_workspace_bytes(max_tokens, k, self.H, self.I, num_experts)
        self.ws_layer = torch.zeros(n, dtype=torch.uint8, device=self.device)

    def route(self, x: torch.Tensor, Wr: torch.Tensor, renorm: bool):
        """Router for the T rows of x (moehip_router_topk): returns (logits, idx, w, w32) views of
        preallocated buffers (valid until the next call). Replaces the model's gate call on a
        prefill chunk (transformers Qwen3MoeTopKRouter / OlmoeTopKRouter.forward, called by moelab
        at runtime.py:909)."""
        T = x.shape[0]
        if T > self.max_tokens or Wr.shape != (self.E, self.H) or Wr.dtype != x.dtype:
            raise RuntimeError(f"GroupedTokens.route: x {tuple(x.shape)} Wr {tuple(Wr.shape)} {Wr.dtype}")
        if self._route_bufs is None or self._route_bufs[0].dtype != x.dtype:
            n, E, k, d = self.max_tokens, self.E, self.k, self.device
            self._route_bufs = (torch.empty(n, E, dtype=x.dtype, device=d), torch.empty(n, k, dtype=torch.int64, device=d),
                                torch.empty(n, k, dtype=x.dtype, device=d), torch.empty(n, k, dtype=torch.float32, device=d))
        logits, idx, w, w32 = (b[:T] for b in self._route_bufs)
        _lib.call("moehip_router_topk", x.data_ptr(), Wr.data_ptr(), T, self.H, self.E, self.k, 1 if renorm else 0,
                  _lib.dt_code(x.dtype), logits.data_ptr(), idx.data_ptr(), w.data_ptr(), w32.data_ptr(),
                  _lib.stream_of(self.device))
        return logits, idx, w, w32

    def layer(self, x: torch.Tensor, Wr: torch.Tensor, renorm: bool, tab: torch.Tensor, out: torch.Tensor,
              add: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
        """One MoE layer on a chunk: router logits, top-k with the expert buckets (and the fp16 copy
        of bf16 activations), grouped GEMMs, ordered combine (moehip_prefill_layer, four launches).
        The routing it used is left in the route buffers (`route_out`)."""
        T = x.shape[0]
        if T > self.max_tokens or x.shape[1] != self.H or Wr.shape != (self.E, self.H) or Wr.dtype != x.dtype:
            raise RuntimeError(f"GroupedTokens.layer: x {tuple(x.shape)} Wr {tuple(Wr.shape)} {Wr.dtype}")
        for t, name in ((x, "x"), (Wr, "Wr"), (tab, "tab"), (out, "out")):
            if not t.is_contiguous() or t.device != self.device:
                raise RuntimeError(f"GroupedTokens.layer: {name} must be a contiguous tensor on {self.device}")
        if tab.dtype != torch.int64 or out.dtype != x.dtype or out.shape != x.shape:
            raise RuntimeError("GroupedTokens.layer: tab int64, out like x")
        if self._route_bufs is None or self._route_bufs[0].dtype != x.dtype:
            n, E, k, d = self.max_tokens, self.E, self.k, self.device
            self._route_bufs = (torch.empty(n, E, dtype=x.dtype, device=d), torch.empty(n, k, dtype=torch.int64, device=d),
                                torch.empty(n, k, dtype=x.dtype, device=d), torch.empty(n, k, dtype=torch.float32, device=d))
        logits, idx, w, w32 = (b[:T] for b in self._route_bufs)
        _lib.call("moehip_prefill_layer", _lib.prec_code("int4"), tab.data_ptr(), x.data_ptr(), Wr.data_ptr(),
                  _lib.dt_code(x.dtype), T, self.H, self.I, self.k, self.E, 64, 1 if renorm else 0, logits.data_ptr(),
                  idx.data_ptr(), w.data_ptr(), w32.data_ptr(), out.data_ptr(), _lib.ptr(add), 1 if accumulate else 0,
                  self.ws_layer.data_ptr(), self.ws_layer.numel(), _lib.stream_of(self.device))
        self.route_out = (logits, idx, w, w32)
        return out

    def table(self, bases: torch.Tensor) -> torch.Tensor:
        """(E, 4) field-address table from the (E,) record base addresses (0 = not resident)."""
        b = bases.to(torch.int64).view(-1, 1)
        return torch.where(b != 0, b + self.offs.view(1, 4), torch.zeros_like(b))

    def run(self, x: torch.Tensor, idx: torch.Tensor, w32: torch.Tensor, tab: torch.Tensor, out: torch.Tensor,
            skip: torch.Tensor | None = None, accumulate: bool = False, add: torch.Tensor | None = None) -> torch.Tensor:
        """out (T, H) = sum over each token's routed experts (in slot order) of w * expert(x).
        x (T, H) fp16/bf16, idx (T, k) int64, w32 (T, k) fp32, tab (E, 4) from `table`,
        skip (T, k) uint8 or None."""
        T = x.shape[0]
        if T > self.max_tokens or x.shape[1] != self.H or idx.shape != (T, self.k) or w32.shape != (T, self.k):
            raise RuntimeError(f"GroupedTokens.run: shapes x {tuple(x.shape)} idx {tuple(idx.shape)} "
                               f"w {tuple(w32.shape)} (max_tokens {self.max_tokens}, k {self.k}, H {self.H})")
        for t, name in ((x, "x"), (idx, "idx"), (w32, "w32"), (tab, "tab"), (out, "out")):
            if not t.is_contiguous() or t.device != self.device:
                raise RuntimeError(f"GroupedTokens.run: {name} must be a contiguous tensor on {self.device}")
        if idx.dtype != torch.int64 or w32.dtype != torch.float32 or tab.dtype != torch.int64 or out.dtype != x.dtype:
            raise RuntimeError("GroupedTokens.run: dtypes (idx int64, w32 float32, tab int64, out like x)")
        stream = _lib.stream_of(self.device)
        _lib.call("moehip_dispatch", idx.data_ptr(), _lib.ptr(skip), T, self.k, self.E, self.counts.data_ptr(),
                  self.offsets.data_ptr(), self.sorted_pos.data_ptr(), self.rank.data_ptr(), stream)
        _lib.call("moehip_grouped_gemm", _lib.prec_code("int4"), tab.data_ptr(), x.data_ptr(), _lib.dt_code(x.dtype), T,
                  self.H, self.I, self.k, self.E, 64, self.offsets.data_ptr(), self.sorted_pos.data_ptr(),
                  self.rank.data_ptr(), w32.data_ptr(), out.data_ptr(), _lib.ptr(add), 1 if accumulate else 0,
                  self.ws.data_ptr(), self.ws.numel(), stream)
        return out


class GroupedLayer:
    """T > 1 tokens (batched decode of a few tokens, prefill chunks) through the MoE layers of a
    `ResidentStore` on the GPU, any record precision and one precision per expert.

    Replaces moelab/runtime.py:459-492 (`_decide_general`: per-token HOBBIT levels and skip,
    stable expert sort, one precision per expert by `expert_level` vote, policy.py:148-154) and
    runtime.py:418-436 (`_run_grouped_tokens`) for every precision the store holds. Per layer, all
    on the device and capturable (no host round trip):
      1. router on the T rows (moehip_router_topk), unless idx / w32 are given
      2. Qwen3-Next shared expert as slot k of every token (moehip_shared_slot), when present
      3. levels and skip per (token, slot)            (moehip_batch_levels)
      4. expert-sorted dispatch of the kept pairs     (moehip_dispatch)
      5. vote, resident copy, per-precision tables    (moehip_batch_vote)
         with fused_decide (the default): 3-5 in one launch (moehip_batch_decide), and, when the
         router runs here on up to route_fused_tokens 16-bit tokens, the top-k, 2, 3-5 and the
         GEMVs' work list in one launch after the logits (moehip_router_logits +
         moehip_batch_route_decide)
      6. expert products per precision + ordered combine: batched dequant GEMVs for up to
         `gemv_tokens` tokens (moehip_grouped_gemv_multi), MFMA tiles beyond
         (moehip_grouped_gemm_multi)
    `shared`: per layer None or {"gate": (H,) tensor in dtype, "rec": {precision: record blob}}
    (the same form as MoEDecoder's). `info[layer]` (E + 1) holds the precision index each expert
    ran at (-1 missing, -2 no pairs); `miss` counts pairs of experts with no usable copy."""

    def __init__(self, store, k: int, max_tokens: int, policy=None, dtype=torch.float16,
                 router_weights: list | None = None, renorm: bool = False, shared: list | None = None,
                 planned: list | None = None, gemv_tokens: int = 64, fused_decide: bool = True,
                 route_fused_tokens: int = 16):
        from .policy import PrecisionPolicy, level_to_precision

        self.gemv_tokens = gemv_tokens
        self.fused_decide = fused_decide
        # up to this many tokens the top-k, shared slot, decision and work list run in the one
        # workgroup of moehip_batch_route_decide; beyond, the top-k and shared slot spread over one
        # wave per token in launches of their own
        self.route_fused_tokens = route_fused_tokens

        self.store, self.k, self.max_tokens = store, k, max_tokens
        self.policy = policy or PrecisionPolicy("lo")
        self.dtype, self.renorm, self.router_weights = dtype, renorm, router_weights
        self.shared = shared
        precs = store.precisions
        self.P = len(precs)
        if self.P > 4:
            raise RuntimeError("GroupedLayer: at most 4 record precisions")
        self.H, self.I = dims(store.layouts[precs[0]])
        for p in precs:
            lay = store.layouts[p]
            if dims(lay) != (self.H, self.I):
                raise RuntimeError(f"GroupedLayer: precision {p} has dims {dims(lay)} != {(self.H, self.I)}")
            if lay["precision"] not in ("int4", "int8", "fp8", "fp16", "bf16"):
                raise RuntimeError(f"GroupedLayer: {lay['precision']} records are not supported (int4/int8/fp8/fp16/bf16)")
            if lay["precision"] in ("int4", "int8") and group_size_of(lay) != (64, 64):
                raise RuntimeError(f"GroupedLayer: {p} records need group size 64, got {group_size_of(lay)}")
        self.device = store.device
        _lib.check_device(self.device)
        lib = _lib.load()
        d, E = self.device, store.E
        self.E = E
        self.has_shared = shared is not None and any(s is not None for s in shared)
        ks = k + (1 if self.has_shared else 0)
        EA = E + (1 if self.has_shared else 0)
        self.ks_max, self.EA_max = ks, EA
        n = max_tokens
        self.logits = torch.empty(n, E, dtype=dtype, device=d)
        self.idx = torch.empty(n, k, dtype=torch.int64, device=d)
        self.w = torch.empty(n, k, dtype=dtype, device=d)
        self.w32 = torch.empty(n, k, dtype=torch.float32, device=d)
        self.idx_ext = torch.empty(n, ks, dtype=torch.int64, device=d)
        self.w_ext = torch.empty(n, ks, dtype=torch.float32, device=d)
        self.levels = torch.empty(n, ks, dtype=torch.int32, device=d)
        self.skip = torch.empty(n, ks, dtype=torch.uint8, device=d)
        self.counts = torch.empty(EA, dtype=torch.int32, device=d)
        self.offsets = torch.empty(EA + 1, dtype=torch.int32, device=d)
        self.sorted_pos = torch.empty(n * ks, dtype=torch.int32, device=d)
        self.rank = torch.empty(n * ks, dtype=torch.int32, device=d)
        self.tabs = torch.zeros(self.P, EA, 4, dtype=torch.int64, device=d)
        self.items = torch.empty(self.P * (n * ks + 1), dtype=torch.int32, device=d)  # a work list per precision
        self.info = torch.zeros(store.L, EA, dtype=torch.float32, device=d)
        self.miss = torch.zeros(1, dtype=torch.float32, device=d)
        self.offs = torch.tensor([field_offsets(store.layouts[p]) for p in precs], dtype=torch.int64, device=d)
        planned = set(planned if planned is not None else precs)
        self.planned_dev = torch.tensor([1 if p in planned else 0 for p in precs], dtype=torch.int32, device=d)
        self.lv2p = (ctypes.c_int * 3)(*[precs.index(level_to_precision(v, precs)) for v in range(3)])
        self.precs_arr = (ctypes.c_int * self.P)(*[_lib.prec_code(store.layouts[p]["precision"]) for p in precs])
        self._pols = [self.policy.device_policy(l) for l in range(store.L)]
        self._srec = []
        for l in range(store.L):
            sh = shared[l] if shared is not None else None
            if sh is None:
                self._srec.append(None)
                continue
            g = sh["gate"]
            if g.dtype != dtype or g.numel() != self.H or not g.is_contiguous() or g.device != d:
                raise RuntimeError(f"shared gate of layer {l}: ({self.H},) {dtype} contiguous on {d}")
            self._srec.append((ctypes.c_int64 * self.P)(*[0 if sh["rec"].get(p) is None else sh["rec"][p].data_ptr()
                                                          for p in precs]))
        nbytes = lib.moehip_grouped_gemm_workspace_bytes(max_tokens, ks, self.H, self.I)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=d)

    def layer(self, layer: int, x: torch.Tensor, out: torch.Tensor, idx: torch.Tensor | None = None,
              w32: torch.Tensor | None = None, add: torch.Tensor | None = None) -> torch.Tensor:
        """out (T, H) = MoE layer `layer` on x (T, H) (+ add). With idx (T, k) int64 / w32 (T, k)
        fp32 given, the router is skipped."""
        T, k, st = x.shape[0], self.k, self.store
        if T > self.max_tokens or x.shape[1] != self.H or x.dtype != self.dtype or not x.is_contiguous():
            raise RuntimeError(f"GroupedLayer.layer: x {tuple(x.shape)} {x.dtype} (max_tokens {self.max_tokens}, "
                               f"H {self.H}, {self.dtype}, contiguous)")
        if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise RuntimeError("GroupedLayer.layer: out must be a contiguous tensor like x")
        stream = _lib.stream_of(self.device)
        srec = self._srec[layer]
        if idx is None and self.fused_decide and x.dtype in (torch.float16, torch.bfloat16):
            return self._layer_routed(layer, x, out, add, srec, stream)
        if idx is None:
            Wr = self.router_weights[layer]
            _lib.call("moehip_router_topk", x.data_ptr(), Wr.data_ptr(), T, self.H, self.E, k,
                      1 if self.renorm else 0, _lib.dt_code(x.dtype), self.logits.data_ptr(), self.idx.data_ptr(),
                      self.w.data_ptr(), self.w32.data_ptr(), stream)
            idx, w32 = self.idx[:T], self.w32[:T]
        elif idx.shape != (T, k) or w32.shape != (T, k) or idx.dtype != torch.int64 or w32.dtype != torch.float32 \
                or not idx.is_contiguous() or not w32.is_contiguous():
            raise RuntimeError("GroupedLayer.layer: idx (T, k) int64 and w32 (T, k) float32, contiguous")
        if srec is not None:
            g = self.shared[layer]["gate"]
            _lib.call("moehip_shared_slot", x.data_ptr(), g.data_ptr(), T, self.H, _lib.dt_code(x.dtype),
                      idx.data_ptr(), w32.data_ptr(), k, self.E, self.idx_ext.data_ptr(), self.w_ext.data_ptr(), stream)
            pidx, pw, ks, EA = self.idx_ext, self.w_ext, k + 1, self.E + 1
        else:
            pidx, pw, ks, EA = idx, w32, k, self.E
        gemv = T <= self.gemv_tokens
        items = None
        if self.fused_decide:
            items = self.items.data_ptr() if gemv else None
            self._decide(layer, pw, pidx, T, ks, srec, items, stream)
        else:
            _lib.call("moehip_batch_levels", pw.data_ptr(), T, k, ks, ctypes.byref(self._pols[layer]),
                      self.levels.data_ptr(), self.skip.data_ptr(), stream)
            _lib.call("moehip_dispatch", pidx.data_ptr(), self.skip.data_ptr(), T, ks, EA, self.counts.data_ptr(),
                      self.offsets.data_ptr(), self.sorted_pos.data_ptr(), self.rank.data_ptr(), stream)
            _lib.call("moehip_batch_vote", self.levels.data_ptr(), self.E, 1 if srec is not None else 0,
                      self.offsets.data_ptr(), self.sorted_pos.data_ptr(), float(self.policy.hi_vote),
                      ctypes.byref(self._pols[layer]), self.lv2p, st.rtab[layer].data_ptr(), srec, self.P,
                      self.offs.data_ptr(), self.planned_dev.data_ptr(), self.tabs.data_ptr(), self.rank.data_ptr(),
                      self.info[layer].data_ptr(), self.miss.data_ptr(), stream)
        args = (self.P, self.precs_arr, self.tabs.data_ptr(), x.data_ptr(), _lib.dt_code(x.dtype), T, self.H,
                self.I, ks, EA, 64, self.offsets.data_ptr(), self.sorted_pos.data_ptr(), self.rank.data_ptr(),
                pw.data_ptr(), out.data_ptr(), _lib.ptr(add), 0, self.ws.data_ptr(), self.ws.numel())
        if gemv:  # without a work list from the decision it is built there
            _lib.call("moehip_grouped_gemv_multi", *args, items, stream)
        else:
            _lib.call("moehip_grouped_gemm_multi", *args, stream)
        return out

    def _decide(self, layer, pw, pidx, T, ks, srec, items, stream):
        _lib.call("moehip_batch_decide", pw.data_ptr(), pidx.data_ptr(), T, self.k, ks,
                  ctypes.byref(self._pols[layer]), self.levels.data_ptr(), self.skip.data_ptr(), self.E,
                  1 if srec is not None else 0, self.counts.data_ptr(), self.offsets.data_ptr(),
                  self.sorted_pos.data_ptr(), self.rank.data_ptr(), float(self.policy.hi_vote), self.lv2p,
                  self.store.rtab[layer].data_ptr(), srec, self.P, self.offs.data_ptr(), self.planned_dev.data_ptr(),
                  self.tabs.data_ptr(), self.info[layer].data_ptr(), self.miss.data_ptr(), items, stream)

    def _layer_routed(self, layer, x, out, add, srec, stream):
        """The layer with the router run here: logits, then one launch from the logits to the work
        list of the GEMVs (moehip_batch_route_decide) for up to route_fused_tokens tokens, else the
        per-token routing over many workgroups (moehip_route_tokens) and the decision with the work
        list (moehip_batch_decide); then the expert products."""
        T, k, st = x.shape[0], self.k, self.store
        shared = srec is not None
        ks, EA = (k + 1, self.E + 1) if shared else (k, self.E)
        Wr = self.router_weights[layer]
        dt = _lib.dt_code(x.dtype)
        _lib.call("moehip_router_logits", x.data_ptr(), Wr.data_ptr(), T, self.H, self.E, dt, self.logits.data_ptr(),
                  stream)
        g = self.shared[layer]["gate"] if shared else None
        gemv = T <= self.gemv_tokens
        if T > self.route_fused_tokens:
            _lib.call("moehip_route_tokens", self.logits.data_ptr(), dt, T, self.E, k, 1 if self.renorm else 0,
                      x.data_ptr(), _lib.ptr(g), self.H, self.idx.data_ptr(), self.w.data_ptr(), self.w32.data_ptr(),
                      self.idx_ext.data_ptr(), self.w_ext.data_ptr(), stream)
            pidx, pw = (self.idx_ext, self.w_ext) if shared else (self.idx, self.w32)
            self._decide(layer, pw, pidx, T, ks, srec, self.items.data_ptr() if gemv else None, stream)
        else:
            _lib.call("moehip_batch_route_decide", self.logits.data_ptr(), dt, T, self.E, k, 1 if self.renorm else 0,
                      x.data_ptr(), _lib.ptr(g), self.H, self.idx.data_ptr(), self.w.data_ptr(), self.w32.data_ptr(),
                      self.idx_ext.data_ptr(), self.w_ext.data_ptr(), ctypes.byref(self._pols[layer]),
                      self.levels.data_ptr(), self.skip.data_ptr(), self.counts.data_ptr(), self.offsets.data_ptr(),
                      self.sorted_pos.data_ptr(), self.rank.data_ptr(), float(self.policy.hi_vote), self.lv2p,
                      st.rtab[layer].data_ptr(), srec, self.P, self.offs.data_ptr(), self.planned_dev.data_ptr(),
                      self.tabs.data_ptr(), self.info[layer].data_ptr(), self.miss.data_ptr(),
                      self.items.data_ptr() if gemv else None, stream)
        pw = self.w_ext if shared else self.w32
        args = (self.P, self.precs_arr, self.tabs.data_ptr(), x.data_ptr(), dt, T, self.H, self.I, ks, EA, 64,
                self.offsets.data_ptr(), self.sorted_pos.data_ptr(), self.rank.data_ptr(), pw.data_ptr(),
                out.data_ptr(), _lib.ptr(add), 0, self.ws.data_ptr(), self.ws.numel())
        if gemv:
            _lib.call("moehip_grouped_gemv_multi", *args, self.items.data_ptr(), stream)
        else:
            _lib.call("moehip_grouped_gemm_multi", *args, stream)
        return out
