"""
The disk tier on the host (no GPU): the store directory format (moelab/store.py:466-561), record
reads through the library's native reader (store.py:378-445: ordinary, O_DIRECT and split
reads, the "truncated read" error), the hot store (store.py:331-356) and the RAM tier in front
of the disk (DiskTier with pageable buffers). Records are random bytes of the layouts' sizes:
the reader moves bytes, so equality with what was written is the whole check.
"""

from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

from moelab_hip import _lib
from moelab_hip.diskstore import DiskTier, ExpertStore, json_ident, write_store
from moelab_hip.store import record_layout

pytestmark = pytest.mark.skipif(not _lib.available(), reason="libmoehip.so not built")

L, E, H, I = 3, 6, 256, 128


def _layouts():
    return [record_layout("fp16", H, I), record_layout("int4", H, I, 64, scale="mse")]


def _record(li, e, prec, rb):
    rng = np.random.default_rng(1000 * li + 10 * e + (prec == "int4"))
    return rng.integers(0, 256, rb, dtype=np.uint8)


@pytest.fixture()
def store_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("store")
    lays = _layouts()
    rbs = {l["precision"]: l["record_bytes"] for l in lays}
    write_store(d, lays, [f"model.layers.{i}.mlp" for i in range(L)], E, H, I,
                lambda li, e, p: _record(li, e, p, rbs[p]), model_type="olmoe")
    return d


def _aligned(n):
    """A page-aligned uint8 host tensor of n bytes (what a pool buffer is)."""
    raw = torch.empty(n + 4096, dtype=torch.uint8)
    off = (-raw.data_ptr()) % 4096
    return raw[off:off + n]


def test_manifest_format_and_store_id(store_dir):
    m = json.loads((store_dir / "manifest.json").read_text())
    assert m["format"] == "moelab-expert-store" and m["version"] == 1 and m["complete"]
    assert m["layers"] == [f"model.layers.{i}.mlp" for i in range(L)]
    assert (m["num_experts"], m["hidden"], m["inter"]) == (E, H, I)
    # store.py:444-447: precisions named with their int scale method unless absmax
    ident = json_ident("olmoe", m["layers"], E, H, I, m["layouts"])
    assert json.loads(ident)[-1] == ["fp16", "int4:mse"]
    assert m["store_id"] == hashlib.sha1(ident.encode()).hexdigest()[:12]
    st = ExpertStore(store_dir)
    assert st.precisions == ["fp16", "int4"] and st.hi == "fp16" and st.lo == "int4" and st.rank("int4") == 1
    assert st.file(2, "int4").name == "layer002.int4.bin"
    assert st.total_bytes("int4") == L * E * st.record_bytes("int4")


@pytest.mark.parametrize("parts", [1, 3, 8])
@pytest.mark.parametrize("direct", [False, True])
def test_read_records(store_dir, parts, direct):
    st = ExpertStore(store_dir)
    st.direct = direct
    for li in range(L):
        for e in range(E):
            for p in st.precisions:
                rb = st.record_bytes(p)
                out = _aligned(rb) if e % 2 == 0 else _aligned(rb + 64)[64:]  # page-aligned or not
                st.read(li, e, p, out=out, parts=parts)
                assert np.array_equal(out.numpy(), _record(li, e, p, rb)), (li, e, p)
    assert st.bytes_read == L * E * sum(st.record_bytes(p) for p in st.precisions)
    if direct:
        # page-aligned buffers take the direct path (records and offsets are 4096-aligned), the
        # others cannot: both kinds are counted (all fall back where the file system has no
        # direct reads)
        assert st.direct_reads + st.direct_fallbacks == L * E * 2
        if st._direct_error is None:
            assert st.direct_reads == L * E and st.direct_fallbacks == L * E
    st.close()


def test_truncated_store_is_an_error(store_dir):
    f = store_dir / "layer001.int4.bin"
    data = f.read_bytes()
    f.write_bytes(data[:-100])
    st = ExpertStore(store_dir)
    st.read(1, 0, "int4")  # an intact record still reads
    with pytest.raises(RuntimeError, match="truncated"):
        st.read(1, E - 1, "int4", parts=4)


def test_incomplete_store_refused(tmp_path):
    (tmp_path / "manifest.json").write_text(json.dumps({"complete": False}))
    with pytest.raises(RuntimeError, match="incomplete"):
        ExpertStore(tmp_path)
    with pytest.raises(FileNotFoundError):
        ExpertStore(tmp_path / "nothing")


def test_hot_store(store_dir, tmp_path):
    st = ExpertStore(store_dir)
    rb = st.record_bytes("int4")
    hot = tmp_path / "hot"
    hot.mkdir()
    # slot 0: (layer 2, expert 5); slot 1: (layer 0, expert 1), as a hot-store build would copy them
    (hot / "hot.int4.bin").write_bytes(_record(2, 5, "int4", rb).tobytes() + _record(0, 1, "int4", rb).tobytes())
    (hot / "hot.json").write_text(json.dumps({"store_id": st.store_id, "experts": {"int4": {"2:5": 0, "0:1": 1}}}))
    assert st.attach_hot(hot) == 2
    for li, e in ((2, 5), (0, 1), (1, 1)):
        out = st.read(li, e, "int4")
        assert np.array_equal(out.numpy(), _record(li, e, "int4", rb))
    assert st.hot_reads == 2
    (hot / "hot.json").write_text(json.dumps({"store_id": "other", "experts": {}}))
    with pytest.raises(ValueError):
        ExpertStore(store_dir).attach_hot(hot)


def test_disk_tier_ram_cache(store_dir):
    st = ExpertStore(store_dir)
    rb4 = st.record_bytes("int4")
    tier = DiskTier(st, host_budget_bytes=4 * rb4, pin=False, parts=2)
    got = tier.many([(0, 1, "int4"), (0, 2, "int4"), (0, 1, "int4")])
    assert got[0] is got[2] and tier.stats["disk_reads"] == 2
    for (li, e), b in zip(((0, 1), (0, 2)), got):
        assert np.array_equal(b.numpy(), _record(li, e, "int4", rb4))
    again = tier(0, 2, "int4")
    assert again is got[1] and tier.stats["host_hits"] == 1
    # past the budget the coldest records leave RAM and are read again when needed
    for e in range(E):
        tier(1, e, "int4")
    assert tier.cache.used <= 4 * rb4
    b = tier(0, 1, "int4")
    assert np.array_equal(b.numpy(), _record(0, 1, "int4", rb4))
    assert tier.stats["disk_reads"] == 2 + E + 1
    with pytest.raises(RuntimeError, match="host cache"):
        tier.many([(2, e, "int4") for e in range(5)])  # one batch larger than the budget
    tier.close()


def test_disk_tier_failed_reads_return_their_buffers(store_dir):
    """A batch with a truncated record raises, and no pool buffer is lost: the failed read gives
    its buffer back, the batch's good reads are cached, and every buffer the pool has lent out is
    held by a cache entry."""
    f = store_dir / "layer002.int4.bin"
    f.write_bytes(f.read_bytes()[:-100])  # the last expert of layer 2 is cut short
    st = ExpertStore(store_dir)
    rb4 = st.record_bytes("int4")
    tier = DiskTier(st, host_budget_bytes=8 * rb4, pin=False, parts=2)
    batch = [(2, e, "int4") for e in range(E)]
    for _ in range(2):
        with pytest.raises(RuntimeError, match="truncated"):
            tier.many(batch)
        held = {ent.blob.data_ptr() for ent in tier.cache.entries.values()}
        assert set(tier.pool._lent) == held
        assert len(held) == E - 1  # the intact records of the batch stay cached
    for e in range(E - 1):
        assert np.array_equal(tier(2, e, "int4").numpy(), _record(2, e, "int4", rb4))
    tier.close()
