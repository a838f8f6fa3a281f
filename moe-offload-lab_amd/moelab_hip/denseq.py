"""The dense part in int8 (moelab/denseq.py): attention projections, shared experts and the LM
head as int8 weights in groups of 64 with fp16 scales, read directly by a gfx950 GEMV for one
token, dequantised in row blocks for several.

Same names and meaning as moelab's module: `gemv_int8(q, s, x, group_size)`, `QLinear` (a
drop-in for nn.Linear: `QLinear(q, s, group_size, bias, out_dtype)` and
`QLinear.from_linear(lin, device, group_size=64)`), `quantizable`, `linear_bytes` and
`quantize_dense`. The weights live on the GPU; a module whose input is not on the GPU, or whose
in_features is not a multiple of 16, raises instead of computing elsewhere.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .store import pick_group_size

__all__ = ["gemv_int8", "dequantize_rows", "quantize_int8", "QLinear", "quantizable", "linear_bytes",
           "quantize_dense"]

_DEQUANT_BLOCK_BYTES = 64 << 20  # rows dequantised at a time in the multi-token path (moelab's bound)


def quantize_int8(w: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(q (O, K) int8, s (O, K/gs) fp16) of a GPU matrix, symmetric per group (moelab/quant.py:129-170
    with bits=8, the store's quantiser)."""
    wf = w.float().contiguous()
    O, K = wf.shape
    q = torch.empty(O, K, dtype=torch.int8, device=w.device)
    s = torch.empty(O, K // group_size, dtype=torch.float16, device=w.device)
    _lib.call("moehip_quantize", wf.data_ptr(), O, K, 8, group_size, q.data_ptr(), s.data_ptr(),
              _lib.stream_of(w.device))
    return q, s


def gemv_int8(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor, group_size: int) -> torch.Tensor:
    """y = (q * s) @ x for ONE vector x (K,); q (O, K) int8, s (O, K/gs) fp16; y (O,) in x's dtype
    (moelab/denseq.py:59-66)."""
    O, K = q.shape
    if not (q.is_cuda and x.is_cuda):
        raise RuntimeError("gemv_int8 runs on the GPU (moehip_dense_gemv_int8)")
    q, s, x = q.contiguous(), s.contiguous(), x.contiguous()
    y = torch.empty(O, dtype=x.dtype, device=x.device)
    _lib.call("moehip_dense_gemv_int8", q.data_ptr(), s.data_ptr(), x.data_ptr(), y.data_ptr(), O, K, group_size,
              _lib.dt_code(x.dtype), _lib.stream_of(x.device))
    return y


def dequantize_rows(q: torch.Tensor, s: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """q * s for rows of an int8 matrix, in `dtype` (moelab/quant.py:191-205 `dequantize(q, s, 8, dtype)`)."""
    rows, K = q.shape
    q, s = q.contiguous(), s.contiguous()
    w = torch.empty(rows, K, dtype=dtype, device=q.device)
    _lib.call("moehip_dense_dequant_int8", q.data_ptr(), s.data_ptr(), rows, K, K // s.shape[1], _lib.dt_code(dtype),
              w.data_ptr(), _lib.stream_of(q.device))
    return w


class QLinear(nn.Module):
    """nn.Linear with int8 group-quantised weights (weights only; arithmetic in float), as moelab's
    QLinear (denseq.py:69-109): one token -> the int8 GEMV, several -> row blocks dequantised to the
    activation dtype, then F.linear."""

    def __init__(self, q: torch.Tensor, s: torch.Tensor, group_size: int, bias: torch.Tensor | None, out_dtype):
        super().__init__()
        self.register_buffer("q", q, persistent=False)
        self.register_buffer("s", s, persistent=False)
        self.bias = None if bias is None else nn.Parameter(bias, requires_grad=False)
        self.group_size = group_size
        self.in_features, self.out_features = q.shape[1], q.shape[0]
        self.out_dtype = out_dtype
        # the GEMV takes K % 32 == 0 and groups of a multiple of 16 values; the row-block path K % 16
        self.kernel = self.in_features % 32 == 0 and group_size % 16 == 0

    @classmethod
    def from_linear(cls, lin: nn.Linear, device, group_size: int = 64) -> "QLinear":
        w = lin.weight.data
        gs = pick_group_size(w.shape[1], group_size)
        q, s = quantize_int8(w.to(device), gs)
        bias = None if lin.bias is None else lin.bias.data.to(device)
        return cls(q, s, gs, bias, w.dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("QLinear runs on the GPU: move the input to the weights' device")
        if self.in_features % 16:
            raise RuntimeError(f"QLinear: in_features {self.in_features} is not a multiple of 16")
        lead = x.shape[:-1]
        n = x.numel() // self.in_features
        if n == 1 and self.kernel:
            y = gemv_int8(self.q, self.s, x.reshape(-1), self.group_size).reshape(*lead, -1)
        else:
            # several tokens: row blocks of the weights dequantised (bounded temporary memory)
            step = max(1, _DEQUANT_BLOCK_BYTES // (self.in_features * x.element_size()))
            parts = []
            for o in range(0, self.out_features, step):
                w = dequantize_rows(self.q[o: o + step], self.s[o: o + step], x.dtype)
                parts.append(F.linear(x, w))
            y = torch.cat(parts, dim=-1) if len(parts) > 1 else parts[0]
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, int8 gs{self.group_size}"


def quantizable(model: nn.Module, min_out: int = 64) -> list[tuple[str, nn.Linear]]:
    """The dense nn.Linear layers to put in int8: at least `min_out` outputs, even in_features
    (so not the small heads such as a shared-expert gate), moelab/denseq.py:112-115."""
    return [(n, m) for n, m in model.named_modules()
            if isinstance(m, nn.Linear) and m.out_features >= min_out and m.weight.dim() == 2 and m.in_features % 2 == 0]


def linear_bytes(model: nn.Module, min_out: int = 64) -> int:
    return sum(m.weight.numel() * m.weight.element_size() for _, m in quantizable(model, min_out))


@torch.no_grad()
def quantize_dense(model: nn.Module, device, log=print) -> dict:
    """Swap every quantizable nn.Linear for a QLinear, one at a time (peak memory: one matrix),
    moelab/denseq.py:122-142. Returns the counts and bytes before / after."""
    before = after = n = 0
    for name, lin in quantizable(model):
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        before += lin.weight.numel() * lin.weight.element_size()
        ql = QLinear.from_linear(lin, device)
        after += ql.q.numel() + ql.s.numel() * 2
        setattr(parent, attr, ql)
        n += 1
        del lin
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    log(f"  dense part in int8: {n} Linear layers, {before / 2**30:.2f} -> {after / 2**30:.2f} GiB")
    return {"layers": n, "bytes_before": before, "bytes_after": after}
