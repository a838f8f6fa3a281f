"""
GPU tests of the offload staging path: moehip_stage_records (gather kernel and SDMA) copies
records byte for byte, moehip_table_set writes the record table, and a decode through
OffloadDecoder (LRFU cache smaller than the working set, misses staged on demand, next-layer
predictions staged in the background, evicted slots reused) gives exactly the outputs of the
same fused kernel with every record resident.
"""

import ctypes

import pytest
import torch

from moelab_hip import _lib
from moelab_hip.layer import MoEDecoder, ResidentStore
from moelab_hip.offload import OffloadDecoder, Stager, DevicePool
from moelab_hip.policy import PrecisionPolicy
from moelab_hip.store import record_layout

pytestmark = pytest.mark.gpu


def _items(srcs, dsts):
    arr = (_lib.Copy * len(srcs))()
    for j, (s, d) in enumerate(zip(srcs, dsts)):
        arr[j].src, arr[j].dst, arr[j].bytes = s.data_ptr(), d.data_ptr(), s.numel()
    return arr


@pytest.mark.parametrize("mode", [0, 1])
def test_stage_records_bit_exact(dev, mode):
    g = torch.Generator().manual_seed(mode)
    sizes = [1_671_168, 4096, 65536 + 16, 3_342_336, 16, 200_000]
    host = [torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g).pin_memory() for n in sizes]
    dst = [torch.zeros(n, dtype=torch.uint8, device=dev) for n in sizes]
    s = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    print(f"stage_records mode {mode}: {len(sizes)} records", flush=True)
    _lib.call("moehip_stage_records", _items(host, dst), len(sizes), mode, s.cuda_stream)
    s.synchronize()
    for h, d in zip(host, dst):
        assert torch.equal(h, d.cpu())


def test_stage_records_checks_on_host(dev):
    """Bad batches are refused before any launch: pageable sources for the gather kernel, more
    than 32 records, misaligned sizes."""
    pageable = torch.zeros(4096, dtype=torch.uint8)
    pinned = torch.zeros(4096, dtype=torch.uint8).pin_memory()
    d = torch.zeros(4096, dtype=torch.uint8, device=dev)
    lib = _lib.load()
    assert lib.moehip_stage_records(_items([pageable], [d]), 1, 0, None) == 1
    assert b"pinned" in lib.moehip_last_error()
    assert lib.moehip_stage_records(_items([pinned] * 33, [d] * 33), 33, 0, None) == 1
    odd = _items([pinned], [d])
    odd[0].bytes = 4095
    assert lib.moehip_stage_records(odd, 1, 1, None) == 1
    with pytest.raises(RuntimeError):
        Stager(dev, DevicePool({"int4": 4096}, 1 << 20, dev), mode="kernel").stage([(pageable, "int4")])


def test_table_set(dev):
    tab = torch.zeros(100, dtype=torch.int64, device=dev)
    idx = (ctypes.c_int64 * 3)(3, 97, 50)
    val = (ctypes.c_int64 * 3)(1 << 40, -5, 7)
    _lib.call("moehip_table_set", tab.data_ptr(), 100, idx, val, 3, None)
    torch.cuda.synchronize()
    ref = torch.zeros(100, dtype=torch.int64)
    ref[3], ref[97], ref[50] = 1 << 40, -5, 7
    assert torch.equal(tab.cpu(), ref)
    bad = (ctypes.c_int64 * 1)(100)
    assert _lib.load().moehip_table_set(tab.data_ptr(), 100, bad, val, 1, None) == 1


def _setup(dev, H, I, E, L, k, seed):
    lay = record_layout("int4", H, I, 64, scale="absmax")
    store = ResidentStore({"int4": lay}, L, E, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    store.fill_synthetic(g, std=0.05)
    Wr = [(torch.randn(E, H, device=dev, generator=g) * 0.05).half() for _ in range(L)]
    rb = lay["record_bytes"]
    host = torch.empty(L * E * rb, dtype=torch.uint8).pin_memory()
    host.copy_(store.arena["int4"].cpu())

    def host_record(l, e, p):
        o = (l * E + e) * rb
        return host[o:o + rb]

    return lay, store, Wr, host_record


@pytest.mark.parametrize("mode", ["kernel", "sdma"])
@pytest.mark.parametrize("routed", [True, False])
def test_offload_decoder_matches_resident(dev, mode, routed):
    H, I, E, L, k, T = 512, 256, 32, 3, 4, 10
    lay, store, Wr, host_record = _setup(dev, H, I, E, L, k, 3)
    rb = lay["record_bytes"]
    ref_dec = MoEDecoder(store, k, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    # 13 records: one token's 12 fit, the working set (3 layers x 32 experts) does not
    off = OffloadDecoder({"int4": lay}, L, E, k, host_record, 13 * rb, dev, PrecisionPolicy("lo"), torch.float16,
                         router_weights=Wr, mode=mode)
    g = torch.Generator().manual_seed(5)
    xs = torch.randn(T, L, 1, H, generator=g).half()
    xs[4:] = xs[torch.arange(4, T) % 3]  # later tokens repeat earlier ones: their experts may still be resident
    xs = xs.to(dev)
    idx = torch.stack([torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(L)]) for _ in range(T)])
    idx[4:] = idx[torch.arange(4, T) % 3]
    w = torch.rand(T, L, k, generator=g) + 0.05
    idx_d, w_d = idx.to(dev), w.to(dev)
    got = torch.zeros(T, L, 1, H, dtype=torch.float16, device=dev)
    ref = torch.zeros_like(got)
    print(f"offload decode mode {mode} routed {routed}: {T} tokens x {L} layers", flush=True)
    for t in range(T):
        for l in range(L):
            if routed:  # the same router kernel as OffloadDecoder.layer, then the experts
                ref_dec.route(l, xs[t, l])
                ref_dec.layer(l, xs[t, l], ref[t, l], idx=ref_dec.idx, w32=ref_dec.w32)
                nxt = None
            else:
                ref_dec.layer(l, xs[t, l], ref[t, l], idx=idx_d[t, l:l + 1], w32=w_d[t, l:l + 1])
                nxt = ({int(e): "int4" for e in idx[t, l + 1]} if (t % 2 == 0 and l + 1 < L) else None)
            if routed:
                off.layer(l, xs[t, l], got[t, l])
            else:
                off.layer(l, xs[t, l], got[t, l], idx=idx_d[t, l:l + 1], w32=w_d[t, l:l + 1], predict=nxt)
        off.tick()
    torch.cuda.synchronize()
    assert off.dec.miss.item() == 0
    assert torch.equal(got, ref)
    st = off.cache.stats
    assert st.evictions > 0 and off.cache.used <= off.cache.budget
    assert off.stats["misses"] > 0 and off.stats["hits"] > 0
    if not routed:
        assert off.stats["prefetch_hits"] > 0
    # every slot handed out is either resident or free again
    pages = (rb + 4095) // 4096
    assert len(off.pool.lent) == len(off.cache.entries)
    assert off.pool.free_pages() + pages * len(off.pool.lent) == off.pool.allocated // 4096


@pytest.mark.parametrize("mode", ["kernel", "sdma"])
@pytest.mark.parametrize("prefetch_mode", ["sdma", "kernel"])
def test_offload_gate_predictor(dev, mode, prefetch_mode):
    """The gate predictor (the next layer's router on the current state, on the GPU, read back with
    the current routing) stages layer l + 1's predicted experts while layer l runs: outputs stay
    identical to the resident decoder's, predictions are counted, and the states that repeat
    (a layer's state fed to the next layer unchanged) are predicted exactly. Misses and
    prefetches are staged by either mode (prefetches by SDMA unless told otherwise)."""
    H, I, E, L, k, T = 512, 256, 32, 4, 4, 8
    lay, store, Wr, host_record = _setup(dev, H, I, E, L, k, 7)
    rb = lay["record_bytes"]
    ref_dec = MoEDecoder(store, k, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    off = OffloadDecoder({"int4": lay}, L, E, k, host_record, 3 * k * rb, dev, PrecisionPolicy("lo"), torch.float16,
                         router_weights=Wr, mode=mode, predictor="gate", prefetch_mode=prefetch_mode)
    g = torch.Generator().manual_seed(11)
    xs = torch.randn(T, 1, 1, H, generator=g).half().repeat(1, L, 1, 1).to(dev)  # one state through every layer
    got = torch.zeros(T, L, 1, H, dtype=torch.float16, device=dev)
    ref = torch.zeros_like(got)
    print(f"offload gate predictor mode {mode} prefetch {prefetch_mode}", flush=True)
    for t in range(T):
        for l in range(L):
            ref_dec.route(l, xs[t, l])
            ref_dec.layer(l, xs[t, l], ref[t, l], idx=ref_dec.idx, w32=ref_dec.w32)
            off.layer(l, xs[t, l], got[t, l])
        off.tick()
    torch.cuda.synchronize()
    assert off.dec.miss.item() == 0
    assert torch.equal(got, ref)
    st = off.stats
    assert st["pred_total"] == T * (L - 1) * k
    assert st["pred_hits"] == st["pred_total"]  # the same state: the gate predicts exactly
    assert st["prefetch_issued"] > 0 and st["prefetch_hits"] > 0


@pytest.mark.parametrize("direct,parts", [(True, 4), (False, 1)])
def test_offload_decoder_from_disk_matches_resident(dev, tmp_path, direct, parts):
    """The disk tier under the offloaded decoder: records written to a store directory, read back
    (O_DIRECT + split reads, or plain reads) into pinned pool buffers through a RAM cache smaller
    than the working set, staged to the device: the outputs are exactly the resident decode's, and
    RAM and VRAM both evict and re-read."""
    from moelab_hip.diskstore import DiskTier, ExpertStore, write_store

    H, I, E, L, k, T = 512, 256, 32, 3, 4, 8
    lay, store, Wr, host_record = _setup(dev, H, I, E, L, k, 7)
    rb = lay["record_bytes"]
    write_store(tmp_path / "store", [lay], [f"model.layers.{i}.mlp" for i in range(L)], E, H, I,
                lambda l, e, p: host_record(l, e, p))
    tier = DiskTier(ExpertStore(tmp_path / "store"), 20 * rb, pin=True, parts=parts, direct=direct)
    ref_dec = MoEDecoder(store, k, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    off = OffloadDecoder({"int4": lay}, L, E, k, tier, 13 * rb, dev, PrecisionPolicy("lo"), torch.float16,
                         router_weights=Wr, mode="kernel")
    g = torch.Generator().manual_seed(8)
    xs = (torch.randn(T, L, 1, H, generator=g).half()).to(dev)
    got = torch.zeros(T, L, 1, H, dtype=torch.float16, device=dev)
    ref = torch.zeros_like(got)
    print(f"offload decode from disk direct={direct} parts={parts}: {T} tokens x {L} layers", flush=True)
    for t in range(T):
        for l in range(L):
            ref_dec.route(l, xs[t, l])
            ref_dec.layer(l, xs[t, l], ref[t, l], idx=ref_dec.idx, w32=ref_dec.w32)
            off.layer(l, xs[t, l], got[t, l])
        off.tick()
    torch.cuda.synchronize()
    assert off.dec.miss.item() == 0
    assert torch.equal(got, ref)
    assert tier.stats["disk_reads"] > 0 and tier.cache.stats.evictions > 0 and tier.stats["host_hits"] > 0
    assert off.cache.stats.evictions > 0
    if direct:
        assert tier.store.direct_reads + tier.store.direct_fallbacks == tier.stats["disk_reads"]
    tier.close()


@pytest.mark.parametrize("mass", [0.5, 0.95])
def test_offload_gate_predictor_mass(dev, mass):
    """Score-mass prefetch (moelab prefetch_mass): the predicted experts up to mass m, at most 2k,
    are staged ahead; the outputs stay identical to the resident decoder's."""
    H, I, E, L, k, T = 512, 256, 32, 4, 4, 6
    lay, store, Wr, host_record = _setup(dev, H, I, E, L, k, 9)
    rb = lay["record_bytes"]
    ref_dec = MoEDecoder(store, k, PrecisionPolicy("lo"), torch.float16, router_weights=Wr)
    off = OffloadDecoder({"int4": lay}, L, E, k, host_record, 4 * k * rb, dev, PrecisionPolicy("lo"), torch.float16,
                         router_weights=Wr, predictor="gate", prefetch_mass=mass)
    g = torch.Generator().manual_seed(13)
    xs = torch.randn(T, 1, 1, H, generator=g).half().repeat(1, L, 1, 1).to(dev)
    got = torch.zeros(T, L, 1, H, dtype=torch.float16, device=dev)
    ref = torch.zeros_like(got)
    print(f"offload gate predictor mass {mass}", flush=True)
    for t in range(T):
        for l in range(L):
            ref_dec.route(l, xs[t, l])
            ref_dec.layer(l, xs[t, l], ref[t, l], idx=ref_dec.idx, w32=ref_dec.w32)
            off.layer(l, xs[t, l], got[t, l])
        off.tick()
    torch.cuda.synchronize()
    assert off.dec.miss.item() == 0
    assert torch.equal(got, ref)
    assert off.stats["prefetch_issued"] > 0 and off.stats["prefetch_hits"] > 0
    with pytest.raises(ValueError):
        OffloadDecoder({"int4": lay}, L, E, k, host_record, 4 * k * rb, dev, router_weights=Wr, prefetch_mass=0.0)
