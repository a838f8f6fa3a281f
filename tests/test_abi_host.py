"""CPU tests: the C-ABI library loads and exports what include/moehip.h declares; argument
validation works without touching a GPU; host-side layout and policy logic match the oracle."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest
import torch

import oracle as O
from conftest import ROOT
from moelab_hip import _lib
from moelab_hip.policy import PrecisionPolicy, level_to_precision
from moelab_hip.store import dims, field_offsets, group_size_of, record_layout, unpack_int4_record, unpacked_layout

HEADER = ROOT / "include" / "moehip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(moehip_\w+)\s*\(", text)) - {"moehip_policy"})


def test_header_declares_the_bound_entry_points():
    assert set(_declared()) == set(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.moehip_abi_version() == _lib.ABI_VERSION == 4
    assert lib.moehip_layer_desc_bytes() == ctypes.sizeof(_lib.LayerDesc)


def test_argument_validation_without_gpu():
    lib = _lib.load()
    # null pointers / bad sizes are rejected before any HIP call
    assert lib.moehip_grouped_up(0, None, None, None, 0, None, None, 8, 1024, 2048, 64, None) == 1
    assert b"null" in lib.moehip_last_error()
    assert lib.moehip_grouped_down(9, None, None, None, None, 8, 2048, 1024, 64, None, None) == 1
    assert lib.moehip_quantize(None, 4, 64, 3, 64, None, None, None) == 1
    assert lib.moehip_router_topk(None, None, 1, 64, 2048, 8, 0, 0, None, None, None, None, None) == 1
    assert lib.moehip_dispatch(None, None, 1, 8, 64, None, None, None, None, None) == 1
    assert lib.moehip_down_workspace_floats(8, 2048) == 8 * 2048
    with pytest.raises(RuntimeError, match="grouped_up"):
        _lib.call("moehip_grouped_up", 0, None, None, None, 0, None, None, 8, 1024, 2048, 64, None)


def test_policy_struct_layout():
    assert ctypes.sizeof(_lib.Policy) == 64
    assert _lib.Policy.miss_t1_64.offset == 56


def test_device_policy_cache_miss_rule():
    """miss_t1 (E3, runtime.py:600-615) reaches the kernels only through the one-token rule, with
    the +1e-6 slack in float64; mode "lo" never allows upgrades (policy.py:176-185)."""
    p = PrecisionPolicy("hobbit", t1=0.6, miss_t1=0.2)
    one, many = p.device_policy(0, one_token=True), p.device_policy(0)
    assert one.e3 == 1 and one.f64 == 1 and one.miss_t1_64 == 0.2 + 1e-6
    assert many.e3 == 0
    assert PrecisionPolicy("hobbit").device_policy(0, one_token=True).e3 == 0
    assert PrecisionPolicy("lo", upgrade=True).device_policy(0, one_token=True).upgrade == 0
    assert PrecisionPolicy("hobbit", upgrade=False).device_policy(0).upgrade == 0


@pytest.mark.parametrize("prec", ["fp32", "fp16", "bf16", "int8", "int4", "fp8"])
@pytest.mark.parametrize("H,I", [(2048, 1024), (2048, 768), (2048, 512), (64, 32), (96, 48), (512, 256)])
def test_record_layout_matches_oracle(prec, H, I):
    mine = record_layout(prec, H, I, 64)
    ref = O.record_layout(prec, H, I, 64)
    assert mine == ref
    assert dims(mine) == (H, I)
    offs = field_offsets(mine)
    assert len(offs) == 4 and all(o % 64 == 0 for o in offs)
    if prec in ("int4", "int8"):
        assert group_size_of(mine) == (O.pick_group_size(H), O.pick_group_size(I))


def test_policy_levels_match_oracle():
    g = torch.Generator().manual_seed(1)
    pols = [dict(mode="hobbit", t1=0.3, t_mid=0.7), dict(mode="hobbit", t1=0.5, t_mid=0.6, t2=0.9),
            dict(mode="hobbit", t1=0.6, t1_layers={1: 0.2, 3: 0.9}), dict(mode="hi"), dict(mode="lo"),
            dict(mode="hobbit", protect_layers={2})]
    for kw in pols:
        mine, ref = PrecisionPolicy(**kw), O.Policy(**kw)
        for layer in range(4):
            w = torch.rand(20, 8, generator=g) ** 2
            l1, s1 = mine.levels(layer, w)
            l2, s2 = ref.levels(layer, w.numpy())
            assert np.array_equal(l1.numpy(), l2) and np.array_equal(s1.numpy(), s2)
            for t in range(4):
                lo, so, _ = mine.levels_one(layer, w[t].tolist())
                assert lo == l1[t].tolist() and so == s1[t].tolist()


def test_device_policy_thresholds():
    p = PrecisionPolicy("hobbit", t1=0.6, t2=0.9, t1_layers={3: 0.2}, protect_layers={5})
    d = p.device_policy(3)
    assert d.mode == 0 and d.t1 == float(np.float32(0.2 + 1e-6)) and d.t2 == float(np.float32(0.9 + 1e-6))
    assert d.t_mid == -1.0 and d.protect == 0 and d.upgrade == 1
    assert p.device_policy(5).protect == 1
    assert PrecisionPolicy("lo").device_policy(0).upgrade == 0
    assert d.f64 == 0 and d.t1_64 == 0.2 + 1e-6 and d.t2_64 == 0.9 + 1e-6 and d.t_mid_64 == -1.0
    assert p.device_policy(3, one_token=True).f64 == 1
    assert [level_to_precision(v, ["fp16", "int4"]) for v in (0, 1, 2)] == ["fp16", "int4", "int4"]


@pytest.mark.parametrize("H,I", [(2048, 1024), (2048, 512), (256, 128)])
def test_unpacked_int4_record_dequantizes_identically(H, I):
    """The reference's check (test_optim.py:86-98): an int4 record rewritten in its unpacked int8
    layout materialises to exactly the same weights; the layout is moelab's int8 one, larger."""
    l4 = record_layout("int4", H, I, 64, scale="absmax")
    l8 = unpacked_layout(l4)
    assert l8 == O.record_layout("int8", H, I, 64) and l8["record_bytes"] > l4["record_bytes"]
    assert unpacked_layout(record_layout("fp16", H, I)) is None
    g = torch.Generator().manual_seed(H + I)
    gu, dn = (torch.randn(2 * I, H, generator=g) * 0.05).numpy(), (torch.randn(H, I, generator=g) * 0.05).numpy()
    blob = O.encode_record(l4, gu, dn, "absmax")
    off = O.field(l4, "gate_up.q")[2]
    blob[off:off + 256] = np.arange(256, dtype=np.uint8)  # every byte value once
    b8 = unpack_int4_record(torch.from_numpy(blob), l4, l8).numpy()
    a, b = O.materialize(l4, blob), O.materialize(l8, b8)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
