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
              add: torch.Tensor | None = None) -> torch.Tensor:
        """One MoE layer on a chunk: router, expert-sorted dispatch, grouped GEMMs, ordered combine."""
        _, idx, _, w32 = self.route(x, Wr, renorm)
        return self.run(x, idx, w32, tab, out, add=add)

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
