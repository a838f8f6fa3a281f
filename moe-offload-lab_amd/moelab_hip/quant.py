"""
Store-side quantisation on the GPU (moelab/quant.py): `quantize` (absmax or mse scales, the
store's packing) and `gptq_quantize` (GPTQ against a layer's input Hessian), with moelab's
signatures and return values: (q, scales), q int4-packed uint8 (out, in/2) or int8 (out, in),
scales fp16 (out, in/group_size).

The kernels are the moehip quantisers (moehip_quantize, moehip_quantize_mse) and the GPTQ column
sweep (moehip_gptq_block). GPTQ's Hessian preparation and Cholesky factors (quant.py:151-166)
and the product that carries a block's errors to the columns on its right (quant.py:187) are
library linear algebra on the same device (torch.linalg / the float32 GEMM).
"""

from __future__ import annotations

import torch

from . import _lib

QMAX = {8: 127, 4: 7}
SCALE_METHODS = ("absmax", "mse")


def _check(w: torch.Tensor, bits: int, group_size: int, method: str) -> None:
    if bits not in QMAX:
        raise ValueError(f"bits must be 4 or 8, not {bits}")
    if method not in SCALE_METHODS:
        raise ValueError(f"unknown scale method {method!r} (choices: {', '.join(SCALE_METHODS)})")
    if w.dim() != 2:
        raise ValueError("w must be (out, in)")
    if w.shape[1] % group_size:
        raise ValueError(f"in_features={w.shape[1]} is not divisible by group_size={group_size}")
    if w.device.type != "cuda":
        raise RuntimeError("the moehip quantisers run on the GPU; w must be a device tensor")


def _buffers(out_f: int, in_f: int, bits: int, group_size: int, device):
    q = torch.empty((out_f, in_f // 2 if bits == 4 else in_f), dtype=torch.uint8 if bits == 4 else torch.int8,
                    device=device)
    s = torch.empty((out_f, in_f // group_size), dtype=torch.float16, device=device)
    return q, s


def quantize(w: torch.Tensor, bits: int, group_size: int, method: str = "absmax") -> tuple[torch.Tensor, torch.Tensor]:
    """quant.py:104-127 on the GPU: bit-exact scales and packed values (the mse errors summed in
    numpy's pairwise order)."""
    _check(w, bits, group_size, method)
    if group_size > 64 or group_size % 2:
        raise ValueError(f"group_size {group_size}: even and <= 64")
    _lib.check_device(w.device)
    wf = w.float().contiguous()
    out_f, in_f = wf.shape
    q, s = _buffers(out_f, in_f, bits, group_size, w.device)
    _lib.call("moehip_quantize_mse" if method == "mse" else "moehip_quantize", wf.data_ptr(), out_f, in_f, bits,
              group_size, q.data_ptr(), s.data_ptr(), _lib.stream_of(w.device))
    return q, s


def hessian_inverse_factor(hessian: torch.Tensor, damp: float = 0.01):
    """quant.py:151-166: dead columns (zero diagonal) get H[d, d] = 1, then damp * mean(diag) on
    the diagonal, again after each failed factorisation (6 tries). Returns (Hinv, dead): Hinv the
    upper Cholesky factor of H^-1 (float32), None when every try failed."""
    H = hessian.float().clone()
    dead = torch.diag(H) == 0
    H[dead, dead] = 1.0
    H.diagonal().add_(damp * torch.mean(torch.diag(H)))
    for _ in range(6):
        L, info = torch.linalg.cholesky_ex(H)
        if int(info) == 0:
            U, info2 = torch.linalg.cholesky_ex(torch.cholesky_inverse(L), upper=True)
            if int(info2) == 0 and bool(torch.isfinite(U).all()):
                return U.contiguous(), dead
        H.diagonal().add_(damp * torch.mean(torch.diag(H)))
    return None, dead


def gptq_quantize(w: torch.Tensor, hessian: torch.Tensor, bits: int, group_size: int, method: str = "mse",
                  damp: float = 0.01, block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """GPTQ (Frantar et al., 2023) in the store's format, quant.py:130-188: columns quantised left
    to right, each one's error carried to the columns not yet quantised through the inverse
    Hessian; a group's scale chosen (`method`) at its first column from the corrected weights.
    w (out, in), hessian (in, in) = sum of x x^T over the layer's real inputs, both on the GPU.
    Falls back to `quantize` when the damped Hessian cannot be factorised (as the reference)."""
    _check(w, bits, group_size, method)
    if group_size not in (32, 64):
        raise ValueError(f"group_size {group_size}: the GPTQ sweep takes 32 or 64")
    if block % group_size or not 0 < block <= 128:
        raise ValueError(f"block={block} must be a multiple of group_size={group_size}, at most 128")
    if hessian.shape != (w.shape[1], w.shape[1]):
        raise ValueError(f"hessian must be ({w.shape[1]}, {w.shape[1]}), got {tuple(hessian.shape)}")
    _lib.check_device(w.device)
    Hinv, dead = hessian_inverse_factor(hessian.to(w.device), damp)
    if Hinv is None:
        return quantize(w, bits, group_size, method)
    W = w.float().clone()
    W[:, dead] = 0.0
    out_f, in_f = W.shape
    q, s = _buffers(out_f, in_f, bits, group_size, w.device)
    E = torch.empty((out_f, block), dtype=torch.float32, device=w.device)
    st = _lib.stream_of(w.device)
    code = 1 if method == "mse" else 0
    for i1 in range(0, in_f, block):
        i2 = min(i1 + block, in_f)
        nb = i2 - i1
        _lib.call("moehip_gptq_block", W.data_ptr(), in_f, Hinv.data_ptr(), in_f, out_f, i1, nb, bits, group_size, code,
                  q.data_ptr(), q.shape[1], s.data_ptr(), s.shape[1], E.data_ptr(), block, st)
        if i2 < in_f:
            W[:, i2:] -= E[:, :nb] @ Hinv[i1:i2, i2:]
    return q, s
