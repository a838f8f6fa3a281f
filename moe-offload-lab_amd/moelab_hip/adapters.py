"""
The fast MoE-layer paths behind moelab's own layer signatures.

moelab enters an MoE layer in two ways, and each has a drop-in here:

1. The experts module of a transformers decoder layer (OlmoeExperts, Qwen3MoeExperts,
   Qwen3NextExperts) is replaced by one whose forward(hidden_states (T, H), top_k_index (T, k)
   int64, top_k_weights (T, k) in the model dtype) -> (T, H) calls
   MoERuntime.run_layer(layer, x, top_k_index, top_k_weights, act_fn, out=None, packed=None)
   (moelab/runtime.py:1093-1112, 523-531). `HipMoE.run_layer` is that call for experts resident
   in a ResidentStore: T = 1 goes to the one-launch decode kernel (moehip_decode_layer with the
   routing given, HOBBIT by the float64 one-token rule of runtime.py:494-517), T > 1 to the
   batched layer (GroupedLayer: per-token levels by the tensor rule, dispatch, vote, GEMVs or
   MFMA tiles, runtime.py:459-492 + 418-436). `ResidentExperts` is the nn.Module to put in place
   of a model's experts module.
2. During the whole-token graph capture, moelab calls FullMoE.layer(layer, x, idx, w, call)
   (moelab/fullgraph.py:149-188) with `call(fn)` launching fn inside the capture or the recorder.
   `FullMoEHip.layer` has that signature: the routing is copied into fixed buffers (recorded torch
   ops), the one-launch decode kernel goes through `call`, HOBBIT by the tensor rule (gpu_levels,
   fullgraph.py:101-114), and `readout()` returns [missing experts] + info (L, 3, k) like
   FullMoE.readout.

The kernels compute silu(gate) * up: any other activation is refused with RuntimeError, as moelab's
runtime routes such layers away from its fused kernels (runtime.py:160-162).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .layer import MoEDecoder
from .policy import PrecisionPolicy
from .prefill import GroupedLayer


def is_silu(act_fn) -> bool:
    """The activation the kernels compute (runtime.py:160-162 `_is_silu`)."""
    return act_fn is F.silu or type(act_fn).__name__ in ("SiLU", "SiLUActivation")


class HipMoE:
    """MoE layers of a ResidentStore behind MoERuntime.run_layer's signature (routing given by the
    model's router, as moelab's runtime receives it)."""

    def __init__(self, store, k: int, policy: PrecisionPolicy | None = None, dtype=torch.bfloat16,
                 max_tokens: int = 512, gemv_tokens: int = 64):
        self.store, self.k, self.dtype = store, k, dtype
        self.policy = policy or PrecisionPolicy("lo")
        self.max_tokens = max_tokens
        self.decoder = MoEDecoder(store, k, self.policy, dtype, one_token_rule=True)
        self.grouped = GroupedLayer(store, k, max_tokens, self.policy, dtype, gemv_tokens=gemv_tokens)
        self.capture_hook = None  # moelab's graph capture sets this on its runtime (runtime.py:1108-1110)

    @property
    def miss(self) -> float:
        """Experts requested but without a usable resident copy, over every call so far."""
        return float(self.decoder.miss.item() + self.grouped.miss.item())

    @torch.no_grad()
    def run_layer(self, layer: int, x: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor,
                  act_fn, out: torch.Tensor | None = None, packed: torch.Tensor | None = None) -> torch.Tensor:
        """out (T, H) = sum over each token's routed experts of weight * expert(x) (runtime.py:523-531).
        `packed` (the routing gathered for one host readback, graphs.py:252-263) is not needed: the
        decisions are made on the device."""
        if not is_silu(act_fn):
            raise RuntimeError(f"moehip kernels compute silu(gate) * up, not {type(act_fn).__name__}")
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        T = x2.shape[0]
        if x2.dtype != self.dtype:
            raise RuntimeError(f"run_layer: activations {x2.dtype}, the layer was set up for {self.dtype}")
        x2 = x2.contiguous()
        idx = top_k_index.reshape(T, -1).to(torch.int64).contiguous()
        w32 = top_k_weights.reshape(T, -1).to(torch.float32).contiguous()
        if idx.shape[1] != self.k:
            raise RuntimeError(f"run_layer: top-{idx.shape[1]} routing for a top-{self.k} layer")
        res = out.reshape(T, shape[-1]) if out is not None else torch.empty_like(x2)
        if T == 1:
            self.decoder.layer(layer, x2, res, idx=idx.view(-1), w32=w32.view(-1))
        else:
            for t0 in range(0, T, self.max_tokens):
                t1 = min(T, t0 + self.max_tokens)
                self.grouped.layer(layer, x2[t0:t1], res[t0:t1], idx[t0:t1], w32[t0:t1])
        return res.view(shape) if out is None else out


class ResidentExperts(nn.Module):
    """In place of a transformers MoE block's `experts` module (the call moelab/runtime.py:
    1093-1112 `OffloadedExperts` receives): forward(hidden_states, top_k_index, top_k_weights)."""

    def __init__(self, moe: HipMoE, layer: int, act_fn: nn.Module, num_experts: int):
        super().__init__()
        self.moe, self.layer, self.act_fn, self.num_experts = moe, layer, act_fn, num_experts

    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor):
        if self.moe.capture_hook is not None:
            return self.moe.capture_hook(self, hidden_states, top_k_index, top_k_weights)
        return self.moe.run_layer(self.layer, hidden_states, top_k_index, top_k_weights, self.act_fn)


class FullMoEHip:
    """The MoE layers inside moelab's whole-token graph (fullgraph.py:117-192 `FullMoE`): layer(layer,
    x, idx, w, call) -> the layer's output in x's dtype, readout() -> [missing] + info."""

    def __init__(self, store, k: int, x: torch.Tensor, policy: PrecisionPolicy | None = None):
        self.store, self.k = store, k
        self.dev = x.device
        self.dec = MoEDecoder(store, k, policy or PrecisionPolicy("lo"), x.dtype)
        self.idx = torch.zeros(k, dtype=torch.int64, device=self.dev)
        self.w32 = torch.zeros(k, dtype=torch.float32, device=self.dev)
        self.flag = self.dec.miss          # (1,) missing experts, as FullMoE.flag
        self.info = self.dec.info          # (L, 3, k): expert, chosen precision (-2 skipped), level
        self.used = False

    def layer(self, layer: int, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, call) -> torch.Tensor:
        if idx.shape[-1] != self.k:
            raise RuntimeError(f"top-{idx.shape[-1]} routing for a top-{self.k} layer")
        self.idx.copy_(idx.reshape(-1))
        self.w32.copy_(w.reshape(-1))
        xc = x.reshape(1, -1).contiguous()
        out = torch.empty_like(xc)

        def launch():
            self.dec.layer(layer, xc, out, idx=self.idx, w32=self.w32)

        call(launch)
        return out.view_as(x)

    def readout(self) -> list:
        """One host readback per token: missing experts, then the info of every layer."""
        return torch.cat((self.flag, self.info.reshape(-1))).tolist()
