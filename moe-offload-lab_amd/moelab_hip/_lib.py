"""
ctypes binding of libmoehip.so (declared in include/moehip.h).

The library is loaded lazily on first use and there is no fallback: if it is missing or was
built for another GPU, every call raises RuntimeError with the reason.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("MOEHIP_LIB", Path(__file__).resolve().parent / "libmoehip.so"))

ABI_VERSION = 4
PREC_CODES = {"int4": 0, "int8": 1, "fp16": 2, "bf16": 3, "fp32": 4, "fp8": 5}
DT_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


class Policy(ctypes.Structure):
    """moehip_policy: HOBBIT parameters for one layer (thresholds include the +1e-6 of policy.py:120-122)."""

    _fields_ = [("mode", _i), ("t1", _f), ("t_mid", _f), ("t2", _f), ("protect", _i), ("upgrade", _i),
                ("f64", _i), ("e3", _i), ("t1_64", ctypes.c_double), ("t_mid_64", ctypes.c_double),
                ("t2_64", ctypes.c_double), ("miss_t1_64", ctypes.c_double)]


class LayerDesc(ctypes.Structure):
    """moehip_layer_desc: static description of one MoE layer for the fused decode kernel."""

    _fields_ = [("P", _i), ("E", _i), ("k", _i), ("H", _i), ("I", _i), ("dtype", _i), ("renorm", _i),
                ("prec", _i * 4), ("gs_up", _i * 4), ("gs_dn", _i * 4), ("planned", _i * 4), ("lv2p", _i * 3),
                ("offs", (ctypes.c_int64 * 4) * 4), ("pol", Policy), ("shared_gate", _vp),
                ("shared_rec", ctypes.c_int64 * 4)]


class Copy(ctypes.Structure):
    """moehip_copy: one host -> device record copy."""

    _fields_ = [("src", _vp), ("dst", _vp), ("bytes", ctypes.c_uint64)]


_SIGS = {
    "moehip_abi_version": ([], _i),
    "moehip_layer_desc_bytes": ([], ctypes.c_size_t),
    "moehip_last_error": ([], ctypes.c_char_p),
    "moehip_device_check": ([_i], _i),
    "moehip_gemv_int4": ([_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "moehip_dense_gemv_int8": ([_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "moehip_dense_dequant_int8": ([_vp, _vp, _i, _i, _i, _i, _vp, _vp], _i),
    "moehip_grouped_up": ([_i, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "moehip_grouped_down": ([_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp], _i),
    "moehip_down_workspace_floats": ([_i, _i], ctypes.c_size_t),
    "moehip_combine": ([_vp, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "moehip_router_topk": ([_vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_decide_table": ([_vp, _vp, _i, ctypes.POINTER(Policy), _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp,
                             _vp, _vp], _i),
    "moehip_dispatch": ([_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_quantize": ([_vp, _i, _i, _i, _i, _vp, _vp, _vp], _i),
    "moehip_quantize_mse": ([_vp, _i, _i, _i, _i, _vp, _vp, _vp], _i),
    "moehip_disk_read": ([_i, _i, ctypes.c_int64, _vp, ctypes.c_size_t, _i, _vp, _vp], _i),
    "moehip_gptq_block": ([_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp], _i),
    "moehip_quantize_fp8_block": ([_vp, _i, _i, _vp, _vp, _vp], _i),
    "moehip_decode_layer": ([ctypes.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                             _vp, _vp, _vp, ctypes.c_size_t, _i, _vp, _vp], _i),
    "moehip_decode_layer_workspace_bytes": ([_i, _i, _i, _i, _i], ctypes.c_size_t),
    "moehip_decode_layer_noalloc": ([ctypes.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _vp], _i),
    "moehip_decode_layer_work_items": ([ctypes.POINTER(LayerDesc), _i], _i),
    "moehip_decode_rows": ([ctypes.POINTER(LayerDesc), _vp, _vp, _vp, _vp, _vp, _i, _vp, ctypes.c_size_t, _vp], _i),
    "moehip_decode_rows_workspace_bytes": ([_i, _i, _i, _i], ctypes.c_size_t),
    "moehip_decode_layer_error": ([_vp, _vp, _vp], _i),
    "moehip_decode_last_kernel": ([], _i),
    "moehip_decode_kernel_name": ([_i], ctypes.c_char_p),
    "moehip_stream_read": ([ctypes.POINTER(ctypes.c_int64), _i, ctypes.c_int64, _vp, ctypes.c_int64, _i, _vp, _vp,
                            _vp], _i),
    "moehip_grouped_gemm": ([_i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                             ctypes.c_size_t, _vp], _i),
    "moehip_grouped_gemm_workspace_bytes": ([_i, _i, _i, _i], ctypes.c_size_t),
    "moehip_prefill_layer": ([_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                              ctypes.c_size_t, _vp], _i),
    "moehip_prefill_layer_workspace_bytes": ([_i, _i, _i, _i, _i], ctypes.c_size_t),
    "moehip_grouped_gemm_multi": ([_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                   _vp, ctypes.c_size_t, _vp], _i),
    "moehip_grouped_gemv_multi": ([_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                   _vp, ctypes.c_size_t, _vp, _vp], _i),
    "moehip_router_logits": ([_vp, _vp, _i, _i, _i, _i, _vp, _vp], _i),
    "moehip_batch_route_decide": ([_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp,
                                   ctypes.POINTER(Policy), _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_double, _vp, _vp,
                                   _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_batch_levels": ([_vp, _i, _i, _i, ctypes.POINTER(Policy), _vp, _vp, _vp], _i),
    "moehip_batch_vote": ([_vp, _i, _i, _vp, _vp, ctypes.c_double, ctypes.POINTER(Policy), _vp, _vp, _vp, _i, _vp,
                           _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_batch_decide": ([_vp, _vp, _i, _i, _i, ctypes.POINTER(Policy), _vp, _vp, _i, _i, _vp, _vp, _vp, _vp,
                             ctypes.c_double, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_route_tokens": ([_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "moehip_shared_slot": ([_vp, _vp, _i, _i, _i, _vp, _vp, _i, _i, _vp, _vp, _vp], _i),
    "moehip_stage_records": ([ctypes.POINTER(Copy), _i, _i, _vp], _i),
    "moehip_table_set": ([_vp, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64), _i,
                          _vp], _i),
}

EXPORTED = tuple(_SIGS)
_lib = None
_checked_devices: set[int] = set()


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load libmoehip.so (no device access). Raises RuntimeError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"libmoehip.so not found at {p}: build it with `python -m moelab_hip.build` "
                           "(or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.moehip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libmoehip ABI {lib.moehip_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check_device(device: torch.device | int | str | None = None) -> None:
    """Raise unless `device` is a gfx950 GPU the library can run on."""
    lib = load()
    if not torch.cuda.is_available():
        raise RuntimeError("no ROCm GPU visible: the moehip kernels need a gfx950 device")
    dev = torch.device(device) if device is not None and not isinstance(device, int) else None
    idx = (device if isinstance(device, int) else (dev.index if dev is not None and dev.index is not None
                                                     else torch.cuda.current_device()))
    if idx in _checked_devices:
        return
    rc = lib.moehip_device_check(idx)
    if rc != 0:
        raise RuntimeError(lib.moehip_last_error().decode())
    _checked_devices.add(idx)


def call(name: str, *args) -> None:
    """Call an entry point; a non-zero return raises RuntimeError with the library's message."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc}): {lib.moehip_last_error().decode()}")


def last_decode_kernel() -> str:
    """Name of the decode kernel the calling thread's last moehip_decode_layer(_noalloc) or
    moehip_decode_rows call launched: "k_decode_xcd", "k_decode_xcd (two passes)", "k_decode_tok",
    "k_decode_layer", or "none"."""
    lib = load()
    return lib.moehip_decode_kernel_name(lib.moehip_decode_last_kernel()).decode()


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def prec_code(prec: str) -> int:
    try:
        return PREC_CODES[prec]
    except KeyError:
        raise RuntimeError(f"unsupported record precision {prec!r}") from None


def dt_code(dtype: torch.dtype) -> int:
    try:
        return DT_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported activation dtype {dtype}") from None
