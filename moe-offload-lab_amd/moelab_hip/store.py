"""
Expert record format (moelab/store.py:36-115) and its device-side encoding.

A record holds everything one expert needs: gate_up (2I, H) and down (H, I), quantised or not,
each field 64-B aligned inside a 4096-B aligned record, so one record = one contiguous copy.
`record_layout` produces the same dict as the reference (same field names, shapes, dtypes,
offsets, record_bytes, group_sizes, scale), so stores and manifests are interchangeable.

This module adds one record kind the reference does not have: "fp8" (checkpoint-format e4m3fn
weights with fp32 128x128 block scales, the `weight_scale_inv` of moelab/quant.py:208-219),
laid out with the same alignment rules.

Encoding runs on the GPU (`encode_record_`): absmax or mse int4/int8 through the moehip quantisers
(bit-exact with moelab/quant.py's absmax path), fp8 through the moehip block quantiser (amax/448 scales,
round-to-nearest-even e4m3fn codes), float records by casting.
"""

from __future__ import annotations

import math

import torch

from . import _lib

ALIGN = 4096  # store.py:36
FIELD_ALIGN = 64  # store.py:37
FP8_BLOCK = 128

PRECISIONS = {  # store.py:39-45, plus fp8
    "fp32": {"kind": "float", "dtype": "float32"},
    "fp16": {"kind": "float", "dtype": "float16"},
    "bf16": {"kind": "float", "dtype": "bfloat16"},
    "int8": {"kind": "int", "bits": 8},
    "int4": {"kind": "int", "bits": 4},
    "fp8": {"kind": "fp8"},
}

TORCH_DTYPES = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "int8": torch.int8,
    "uint8": torch.uint8,
}
ELEM_SIZE = {"float32": 4, "float16": 2, "bfloat16": 2, "int8": 1, "uint8": 1}


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def pick_group_size(in_features: int, preferred: int = 64) -> int:
    """Largest even group size <= preferred dividing in_features (moelab/quant.py:49-54)."""
    for gs in range(min(preferred, in_features), 1, -1):
        if in_features % gs == 0 and gs % 2 == 0:
            return gs
    raise ValueError(f"no even group size divides {in_features}")


def record_layout(prec: str, hidden: int, inter: int, group_size: int = 64, scale: str | None = None) -> dict:
    """Layout of one expert record (moelab/store.py:76-115)."""
    spec = PRECISIONS[prec]
    if spec["kind"] == "int" and scale is None:
        scale = "mse" if spec["bits"] == 4 else "absmax"
    mats = {"gate_up": (2 * inter, hidden), "down": (hidden, inter)}
    raw: list[tuple[str, tuple[int, ...], str]] = []
    groups: dict[str, int] = {}
    if spec["kind"] == "float":
        for name, shape in mats.items():
            raw.append((name, shape, spec["dtype"]))
    elif spec["kind"] == "fp8":
        for name, (o, i) in mats.items():
            raw.append((f"{name}.q", (o, i), "uint8"))
            raw.append((f"{name}.s", (math.ceil(o / FP8_BLOCK), math.ceil(i / FP8_BLOCK)), "float32"))
    else:
        bits = spec["bits"]
        for name, (o, i) in mats.items():
            gs = pick_group_size(i, group_size)
            groups[name] = gs
            raw.append((f"{name}.q", (o, i) if bits == 8 else (o, i // 2), "int8" if bits == 8 else "uint8"))
            raw.append((f"{name}.s", (o, i // gs), "float16"))
    fields, off = [], 0
    for name, shape, dtype in raw:
        nbytes = ELEM_SIZE[dtype] * math.prod(shape)
        fields.append([name, list(shape), dtype, off])
        off = _align(off + nbytes, FIELD_ALIGN)
    lay = {"precision": prec, "fields": fields, "record_bytes": _align(off, ALIGN), "group_sizes": groups}
    if spec["kind"] == "int":
        lay["scale"] = scale
    return lay


def field_offsets(layout: dict) -> list[int]:
    """Byte offsets of the four table entries [gate_up.q, gate_up.s, down.q, down.s]
    (float records repeat [gate_up, gate_up, down, down], moelab/kernels.py:782-797)."""
    f = {name: off for name, _, _, off in layout["fields"]}
    if PRECISIONS[layout["precision"]]["kind"] == "float":
        return [f["gate_up"], f["gate_up"], f["down"], f["down"]]
    return [f["gate_up.q"], f["gate_up.s"], f["down.q"], f["down.s"]]


def dims(layout: dict) -> tuple[int, int]:
    """(H, I) of a layout."""
    f = {name: shape for name, shape, _, _ in layout["fields"]}
    if "gate_up" in f:
        two_i, H = f["gate_up"]
    elif layout["precision"] == "int4":
        two_i, H = f["gate_up.q"][0], f["gate_up.q"][1] * 2
    else:
        two_i, H = f["gate_up.q"]
    return H, two_i // 2


def group_size_of(layout: dict) -> tuple[int, int]:
    """(gate_up group size, down group size); 0 for non-int records."""
    g = layout.get("group_sizes") or {}
    return int(g.get("gate_up", 0)), int(g.get("down", 0))


def views(layout: dict, blob: torch.Tensor) -> dict[str, torch.Tensor]:
    """Typed zero-copy views into a record (moelab/store.py:153-161)."""
    out = {}
    for name, shape, dtype, off in layout["fields"]:
        nbytes = ELEM_SIZE[dtype] * math.prod(shape)
        part = blob[off:off + nbytes]
        if dtype != "uint8":
            part = part.view(TORCH_DTYPES[dtype])
        out[name] = part.view(shape)
    return out


def encode_record_(layout: dict, blob: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """Write one record into `blob` (uint8 device tensor of record_bytes) from float weights on
    the same device. int4/int8: the layout's scale method ("absmax" or "mse", moelab/quant.py:64-93)
    through the moehip quantisers (identical bytes to moelab/store.py:122-150); float: cast; fp8:
    per-128x128-block amax/448 scales and round-to-nearest-even e4m3fn codes."""
    prec = layout["precision"]
    spec = PRECISIONS[prec]
    if blob.numel() != layout["record_bytes"] or blob.dtype != torch.uint8:
        raise ValueError("blob must be a uint8 tensor of record_bytes")
    blob.zero_()
    v = views(layout, blob)
    mats = {"gate_up": gate_up, "down": down}
    if spec["kind"] == "float":
        for name, w in mats.items():
            v[name].copy_(w)
        return blob
    if blob.device.type != "cuda":
        raise RuntimeError("encode_record_ quantises on the GPU; blob must be a device tensor")
    _lib.check_device(blob.device)
    if spec["kind"] == "fp8":
        for name, w in mats.items():
            wf = w.float().contiguous()
            O, I = wf.shape
            _lib.call("moehip_quantize_fp8_block", wf.data_ptr(), O, I, v[f"{name}.q"].data_ptr(),
                      v[f"{name}.s"].data_ptr(), _lib.stream_of(blob.device))
        return blob
    bits = spec["bits"]
    method = layout.get("scale") or "absmax"
    if method not in ("absmax", "mse"):
        raise ValueError(f"unknown scale method {method!r} (absmax, mse)")
    entry = "moehip_quantize_mse" if method == "mse" else "moehip_quantize"
    for name, w in mats.items():
        wf = w.float().contiguous()
        O, I = wf.shape
        gs = layout["group_sizes"][name]
        _lib.call(entry, wf.data_ptr(), O, I, bits, gs, v[f"{name}.q"].data_ptr(),
                  v[f"{name}.s"].data_ptr(), _lib.stream_of(blob.device))
    return blob


def unpacked_layout(layout: dict) -> dict | None:
    """The "unpacked" form of an int4 record (moelab/store.py:177-189, `fast_int4_unpacked`): the
    int8 layout of the same shapes and groups, one int4 value per byte. None for other records,
    or when the int8 layout cannot keep the int4 groups."""
    if layout["precision"] != "int4":
        return None
    H, I = dims(layout)
    l8 = record_layout("int8", H, I, max(layout["group_sizes"].values()))
    return l8 if l8["group_sizes"] == layout["group_sizes"] else None


_NIBBLE_TABLES: dict = {}


def _nibble_table(device) -> torch.Tensor:
    """(256, 2) int8 on `device`: byte b -> (low nibble - 8, high nibble - 8), the even and the odd
    value of moelab's packing (quant.py:96-101)."""
    key = str(device)
    if key not in _NIBBLE_TABLES:
        b = torch.arange(256, dtype=torch.int16)
        _NIBBLE_TABLES[key] = torch.stack([(b & 15) - 8, (b >> 4) - 8], dim=1).to(torch.int8).to(device)
    return _NIBBLE_TABLES[key]


def unpack_int4_record(blob: torch.Tensor, layout4: dict, layout8: dict) -> torch.Tensor:
    """An int4 record rewritten in its unpacked int8 layout (moelab/store.py:192-203): the same
    values one per byte and the same scales, on the device of `blob` (padding bytes zero).
    moelab's int8 kernels then run it (grouped_ffn_int8, runtime.py:230-240, 405)."""
    table = _nibble_table(blob.device)
    out = torch.zeros(layout8["record_bytes"], dtype=torch.uint8, device=blob.device)
    src, dst = views(layout4, blob), views(layout8, out)
    for name in ("gate_up", "down"):
        packed = src[f"{name}.q"]
        dst[f"{name}.q"].copy_(table[packed.long()].reshape(packed.shape[0], -1))
        dst[f"{name}.s"].copy_(src[f"{name}.s"])
    return out
