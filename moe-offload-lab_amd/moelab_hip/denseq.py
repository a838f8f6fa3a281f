"""The dense part in int8 (moelab/denseq.py): attention projections, shared experts and the LM
head as int8 weights in groups of 64 with fp16 scales, read directly by a gfx950 GEMV for one
token, dequantised one block of rows at a time into a scratch matrix for several.

Same names and meaning as moelab's module: `gemv_int8(q, s, x, group_size)`, `QLinear` (a
drop-in for nn.Linear: `QLinear(q, s, group_size, bias, out_dtype)` and
`QLinear.from_linear(lin, device, group_size=64)`), `quantizable`, `linear_bytes` and
`quantize_dense`. The weights live on the GPU; a module whose input is not on the GPU, or whose
in_features is not a multiple of 16, raises instead of computing elsewhere.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .store import pick_group_size

__all__ = ["gemv_int8", "dequantize_rows", "quantize_int8", "QLinear", "quantizable", "linear_bytes",
           "quantize_dense"]

# Rows of W dequantised per step of the multi-token path: a multiple of 256 rows (whole row blocks
# of the dequantisation kernel on every XCD) holding at most this many bytes of temporary weights.
_ROWS_BUDGET_BYTES = 32 << 20


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
    """nn.Linear with int8 weights in groups (fp16 scale per group; arithmetic in the activation
    dtype), keeping moelab's QLinear interface (denseq.py:69-109: `QLinear(q, s, group_size, bias,
    out_dtype)`, `from_linear`, the `q` / `s` buffers, `in_features` / `out_features`).

    One token streams the int8 rows through moehip_dense_gemv_int8 (the bias added in place).
    Several tokens compute the transposed product yT (out_features, tokens) one block of rows at
    a time: each block of W is dequantised into one reusable scratch matrix in the activation
    dtype (moehip_dense_dequant_int8, bit-identical to moelab's dequantize) and multiplied into
    its contiguous rows of yT by addmm with the bias folded in, so no partial results are
    concatenated and the temporary weights never exceed one block."""

    def __init__(self, q: torch.Tensor, s: torch.Tensor, group_size: int, bias: torch.Tensor | None, out_dtype):
        super().__init__()
        out_f, in_f = q.shape
        if s.shape != (out_f, in_f // group_size) or in_f % group_size:
            raise ValueError(f"QLinear: scales {tuple(s.shape)} do not match q {tuple(q.shape)} in groups of {group_size}")
        self.register_buffer("q", q, persistent=False)
        self.register_buffer("s", s, persistent=False)
        self.bias = None if bias is None else nn.Parameter(bias, requires_grad=False)
        self.group_size = group_size
        self.in_features, self.out_features = in_f, out_f
        self.out_dtype = out_dtype
        # moehip_dense_gemv_int8 takes rows of 32-value multiples and groups of 16-value multiples
        self.kernel = in_f % 32 == 0 and group_size % 16 == 0
        self._rows = max(256, _ROWS_BUDGET_BYTES // (2 * in_f) // 256 * 256)

    @classmethod
    def from_linear(cls, lin: nn.Linear, device, group_size: int = 64) -> "QLinear":
        """The int8 form of an nn.Linear, quantised on `device` by the library's absmax quantiser
        (moelab quant.py with bits = 8), the group size chosen as moelab's pick_group_size does."""
        weight = lin.weight.detach()
        gs = pick_group_size(weight.shape[1], group_size)
        q, s = quantize_int8(weight.to(device), gs)
        bias = lin.bias.detach().to(device) if lin.bias is not None else None
        return cls(q, s, gs, bias, weight.dtype)

    def _one_token(self, x: torch.Tensor) -> torch.Tensor:
        y = gemv_int8(self.q, self.s, x.reshape(self.in_features), self.group_size)
        if self.bias is not None:
            y.add_(self.bias.to(y.dtype))
        return y

    def _tokens(self, x2: torch.Tensor) -> torch.Tensor:
        n = x2.shape[0]
        xt = x2.t()
        yt = torch.empty(self.out_features, n, dtype=x2.dtype, device=x2.device)
        rows = min(self._rows, self.out_features)
        scratch = torch.empty(rows, self.in_features, dtype=x2.dtype, device=x2.device)
        lib = _lib.load()
        bias = None if self.bias is None else self.bias.to(x2.dtype).unsqueeze(1)
        for r0 in range(0, self.out_features, rows):
            r1 = min(r0 + rows, self.out_features)
            w = scratch[:r1 - r0]
            rc = lib.moehip_dense_dequant_int8(self.q[r0:r1].data_ptr(), self.s[r0:r1].data_ptr(), r1 - r0,
                                               self.in_features, self.group_size, _lib.dt_code(x2.dtype), w.data_ptr(),
                                               _lib.stream_of(x2.device))
            if rc != 0:
                raise RuntimeError(f"moehip_dense_dequant_int8 failed ({rc}): {lib.moehip_last_error().decode()}")
            if bias is None:
                torch.mm(w, xt, out=yt[r0:r1])
            else:
                torch.addmm(bias[r0:r1], w, xt, out=yt[r0:r1])
        return yt.t()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("QLinear runs on the GPU: move the input to the weights' device")
        if self.in_features % 16:
            raise RuntimeError(f"QLinear: in_features {self.in_features} is not a multiple of 16")
        *lead, k_in = x.shape
        if k_in != self.in_features:
            raise RuntimeError(f"QLinear: input of {k_in} features, {self.in_features} expected")
        x2 = x.reshape(-1, k_in)
        if x2.shape[0] == 1 and self.kernel:
            y = self._one_token(x2.contiguous())
        else:
            y = self._tokens(x2.contiguous())
        return y.reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        return (f"{self.in_features} -> {self.out_features}, int8 weights, groups of {self.group_size}, "
                f"bias={self.bias is not None}")


def quantizable(model: nn.Module, min_out: int = 64) -> list[tuple[str, nn.Linear]]:
    """The dense nn.Linear layers to put in int8 (moelab's rule, denseq.py:112-115, kept so that a
    model selects the same layers): at least `min_out` outputs and an even in_features, which
    leaves out small heads such as a shared-expert gate."""
    picked = []
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and mod.weight.dim() == 2 and mod.out_features >= min_out \
                and mod.in_features % 2 == 0:
            picked.append((name, mod))
    return picked


def linear_bytes(model: nn.Module, min_out: int = 64) -> int:
    """Bytes of the weights `quantizable` would take."""
    total = 0
    for _, mod in quantizable(model, min_out):
        total += mod.weight.numel() * mod.weight.element_size()
    return total


@torch.no_grad()
def quantize_dense(model: nn.Module, device, log=print) -> dict:
    """Replace the quantizable nn.Linear layers by QLinear modules (moelab's entry point,
    denseq.py:122-142), layer by layer, so that at most one matrix exists in both forms at a time.
    Returns {"layers", "bytes_before", "bytes_after"}."""
    targets = quantizable(model)
    modules = dict(model.named_modules())
    stats = {"layers": 0, "bytes_before": 0, "bytes_after": 0}
    for name, lin in targets:
        owner_name, attr = name.rsplit(".", 1) if "." in name else ("", name)
        owner = modules[owner_name]
        ql = QLinear.from_linear(lin, device)
        stats["bytes_before"] += lin.weight.numel() * lin.weight.element_size()
        stats["bytes_after"] += ql.q.numel() * ql.q.element_size() + ql.s.numel() * ql.s.element_size()
        owner.register_module(attr, ql)
        stats["layers"] += 1
    targets.clear()  # the last references to the float layers: their weights can go
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    log(f"  int8 dense layers: {stats['layers']} nn.Linear replaced, "
        f"{stats['bytes_before'] / 2**30:.2f} GiB of weights -> {stats['bytes_after'] / 2**30:.2f} GiB")
    return stats
