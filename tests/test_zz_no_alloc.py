"""GPU: moehip_decode_layer_noalloc (the library's own scratch array: no workspace argument, no
allocation) against moehip_decode_layer on a caller workspace, through the C ABI. The same kernels
run on the same inputs, so outputs and readouts must be identical (bit for bit), on two calls in a
row, the second on a smaller layer; a layer whose workspace exceeds the array is refused."""

from __future__ import annotations

import ctypes

import pytest
import torch

from moelab_hip import _lib
from moelab_hip.layer import MoEDecoder, ResidentStore
from moelab_hip.policy import PrecisionPolicy
from moelab_hip.store import record_layout

pytestmark = pytest.mark.gpu


def _layer(dev, H, I, E, k, seed):
    store = ResidentStore({"int4": record_layout("int4", H, I, 64, scale="absmax")}, 1, E, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    store.fill_synthetic(g, std=0.02)
    Wr = [(torch.randn(E, H, device=dev, generator=g) * 0.05).half()]
    dec = MoEDecoder(store, k, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    assert dec.fused
    x = torch.randn(1, H, device=dev, generator=g).half()
    return store, dec, Wr[0], x


def _readouts(dev, E, k):
    return {"logits": torch.zeros(E, dtype=torch.float16, device=dev),
            "idx": torch.full((k,), -1, dtype=torch.int64, device=dev),
            "w": torch.zeros(k, dtype=torch.float16, device=dev),
            "w32": torch.zeros(k, dtype=torch.float32, device=dev),
            "info": torch.zeros(3, k, dtype=torch.float32, device=dev),
            "miss": torch.zeros(1, dtype=torch.float32, device=dev)}


def _call(name, dec, store, Wr, x, out, r, extra):
    _lib.call(name, ctypes.byref(dec._descs[0]), x.data_ptr(), Wr.data_ptr(), None, None, store.rtab[0].data_ptr(),
              out.data_ptr(), None, 0, r["logits"].data_ptr(), r["idx"].data_ptr(), r["w"].data_ptr(),
              r["w32"].data_ptr(), r["info"].data_ptr(), r["miss"].data_ptr(), *extra, _lib.stream_of(x.device))


@pytest.mark.parametrize("shapes", [((2048, 1024, 64, 8), (512, 256, 16, 4))])
def test_noalloc_matches_workspace_entry(dev, shapes):
    for n, (H, I, E, k) in enumerate(shapes):
        print(f"noalloc call {n}: H={H} I={I} E={E} k={k}", flush=True)
        store, dec, Wr, x = _layer(dev, H, I, E, k, seed=11 + n)
        out_ws = torch.zeros(1, H, dtype=torch.float16, device=dev)
        out_na = torch.full((1, H), float("nan"), dtype=torch.float16, device=dev)
        r_ws, r_na = _readouts(dev, E, k), _readouts(dev, E, k)
        for _ in range(2):  # twice each: the second launch of a shape reuses the array's state
            _call("moehip_decode_layer", dec, store, Wr, x, out_ws, r_ws, (dec.ws.data_ptr(), dec.ws.numel(), 0, None))
            _call("moehip_decode_layer_noalloc", dec, store, Wr, x, out_na, r_na, ())
            torch.cuda.synchronize()
            assert torch.equal(out_na, out_ws)
            assert not torch.isnan(out_na.float()).any()
            for key in r_ws:
                if key != "miss":
                    assert torch.equal(r_na[key], r_ws[key]), key
            assert r_na["miss"].item() == r_ws["miss"].item() == 0
        dec.check_error()
        # the scratch array's own error word (no workspace pointer): clear after these calls
        flag = torch.full((1,), 7, dtype=torch.int32, device=dev)
        _lib.call("moehip_decode_layer_error", None, flag.data_ptr(), _lib.stream_of(dev))
        torch.cuda.synchronize()
        assert flag.item() == 0


def test_noalloc_refuses_an_oversized_layer(dev):
    d = _lib.LayerDesc()
    d.P, d.k, d.E, d.H, d.I = 4, 32, 1024, 2048, 2048  # a 4.26 MB workspace: above the 2 MiB array
    lib = _lib.load()
    need = lib.moehip_decode_layer_workspace_bytes(4, 32, 1024, 2048, 2048)
    assert need > (2 << 20)
    rc = lib.moehip_decode_layer_noalloc(ctypes.byref(d), None, None, None, None, None, None, None, 0, None, None, None,
                                         None, None, None, _lib.stream_of(dev))
    assert rc == 1  # MOEHIP_EINVAL
    assert "scratch array holds" in lib.moehip_last_error().decode()
