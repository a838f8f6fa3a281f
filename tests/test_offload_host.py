"""
Host-side offload logic (no GPU): the LRFU TierCache and the HostPool against the behaviour
moelab's own unit tests fix (moelab tests/test_units.py:88-152, 253-291, 376-413 and
tests/test_a5.py:109-125), the LRFU closed form, and heap victims against a brute-force sort.
"""

import random

import pytest
import torch

from moelab_hip.offload import HostPool, TierCache

RANK = {"fp16": 0, "int8": 1, "int4": 2}.get


def blob(n):
    return torch.zeros(n, dtype=torch.uint8)


def test_lrfu_score_closed_form():
    """f after touches at clocks t_i, read at clock T: sum_i gamma^(T - t_i)."""
    c = TierCache("t", "cpu", 1000, RANK, half_life=3.0)
    e = c.insert((0, 0, "fp16"), blob(10))  # touch at 0
    c.tick(2)
    c.touch(e)  # at 2
    c.tick(3)
    c.touch(e)  # at 5
    c.tick(4)   # read at 9
    g = 0.5 ** (1 / 3.0)
    assert c.score(e) == pytest.approx(g ** 9 + g ** 7 + g ** 4, rel=1e-12)
    # half-life: with no touches the score halves every half_life ticks
    s0 = c.score(e)
    c.tick(3)
    assert c.score(e) == pytest.approx(s0 / 2, rel=1e-12)


def test_lrfu_evicts_coldest():
    c = TierCache("t", "cpu", 300, RANK, half_life=4)
    for e in range(3):
        c.insert((0, e, "fp16"), blob(100))
    for _ in range(3):
        c.tick()
        c.touch(c.entries[(0, 0, "fp16")])
    c.tick()
    c.insert((0, 9, "fp16"), blob(100))
    assert (0, 0, "fp16") in c.entries and (0, 9, "fp16") in c.entries
    assert len(c.entries) == 3 and c.stats.evictions == 1


def test_lrfu_recency_beats_old_frequency():
    c = TierCache("t", "cpu", 200, RANK, half_life=1)
    c.insert((0, 0, "fp16"), blob(100))
    for _ in range(3):
        c.touch(c.entries[(0, 0, "fp16")])
    c.clock += 20
    c.insert((0, 1, "fp16"), blob(100))
    c.insert((0, 2, "fp16"), blob(100))
    assert (0, 0, "fp16") not in c.entries


def test_precision_substitution():
    c = TierCache("t", "cpu", 1000, RANK)
    c.insert((2, 7, "fp16"), blob(10))
    assert c.lookup(2, 7, "int4").key[2] == "fp16"  # a more precise copy serves
    c2 = TierCache("t", "cpu", 1000, RANK)
    c2.insert((2, 7, "int4"), blob(10))
    assert c2.lookup(2, 7, "fp16") is None  # a less precise one does not
    assert c2.lookup(2, 7, "int4", exact=True) is not None
    assert c2.stats.hits == 1 and c2.stats.misses == 1
    c2.lookup(2, 8, "int4", count=False)
    assert c2.stats.misses == 1


def test_pins_and_protect():
    c = TierCache("t", "cpu", 300, RANK, pin_fraction=0.5)
    c.insert((0, 0, "fp16"), blob(100), pinned=True)
    c.insert((0, 1, "fp16"), blob(100))
    c.insert((0, 2, "fp16"), blob(100))
    assert c.insert((0, 3, "fp16"), blob(100), protect=frozenset({(0, 1, "fp16"), (0, 2, "fp16")})) is None
    assert c.insert((0, 3, "fp16"), blob(100)) is not None
    assert (0, 0, "fp16") in c.entries
    assert c.insert((0, 4, "fp16"), blob(400)) is None
    assert c.stats.rejected == 2


def test_repin_hysteresis_and_max_swaps():
    c = TierCache("t", "cpu", 10_000, RANK, pin_fraction=0.5, half_life=1000)
    for e in range(5):
        c.insert((0, e, "fp16"), blob(1000), pinned=True)
    for e in range(5, 10):
        c.insert((0, e, "fp16"), blob(1000))
    for e in range(5, 10):
        for _ in range(3):
            c.touch(c.entries[(0, e, "fp16")])
    swaps = c.repin(hysteresis=0.25, max_swaps=4)
    assert len(swaps) == 4
    assert sum(ent.pinned for ent in c.entries.values()) == 5
    d = TierCache("t", "cpu", 2000, RANK, pin_fraction=0.5, half_life=1000)
    d.insert((0, 0, "fp16"), blob(1000), pinned=True)
    d.insert((0, 1, "fp16"), blob(1000))
    d.entries[(0, 0, "fp16")].f = 10.0
    d.entries[(0, 1, "fp16")].f = 11.0  # only 10 % hotter: no swap
    assert d.repin() == []


def test_heap_victims_match_sorted_scores():
    """Brute force: every eviction removes an entry of the lowest score among the unpinned,
    unprotected ones (the heap gives the same victims as a full sort)."""
    rnd = random.Random(0)
    c = TierCache("t", "cpu", 40 * 64, {"a": 0}.get, half_life=8.0, pin_fraction=0.25)
    checked = 0
    for step in range(3000):
        r = rnd.random()
        if r < 0.5:
            key = (rnd.randrange(4), rnd.randrange(60), "a")
            if key in c.entries:
                c.touch(c.entries[key])
                continue
            protect = frozenset(rnd.sample(list(c.entries), min(3, len(c.entries)))) if c.entries else frozenset()
            expect = None
            if c.used + 64 > c.budget:
                cands = sorted((e for e in c.entries.values() if not e.pinned and e.key not in protect), key=c.score)
                expect = [round(c.score(cands[0]), 9)] if cands else None
            before = {k: c.score(e) for k, e in c.entries.items()}
            c.insert(key, blob(64), protect=protect, pinned=rnd.random() < 0.05)
            gone = [k for k in before if k not in c.entries]
            if expect is not None:
                assert sorted(round(before[k], 9) for k in gone) == expect, step
                assert not set(gone) & protect
                # the victim walk dropped the stale pairs it passed: the top pair was current or held
                top = c._heap.a[0] if c._heap.a else None
                assert top is None or c._heap._current(top) or top[1].key in gone
                checked += 1
        elif r < 0.8:
            c.tick()
        elif r < 0.9 and c.entries:
            c.unpin(rnd.choice(list(c.entries)))
        elif c.entries:
            c.pin(rnd.choice(list(c.entries)))
        if step % 97 == 0:  # the whole candidate order, and the stale pairs kept bounded
            order = [e.key for e in c._heap.ascending()]
            c._heap.restore()
            assert order == [e.key for e in sorted((e for e in c.entries.values() if not e.pinned), key=lambda e: e.rank)]
            assert len(c._heap) == len(order) and len(c._heap.a) <= 2 * len(order) + 64
    assert checked > 500 and c.used <= c.budget


def test_stale_eviction_protects_current_pass():
    for policy, victim in (("lrfu", (0, 1, "a")), ("stale", (0, 0, "a"))):
        c = TierCache("t", "cpu", 3 * 64, {"a": 0}.get, eviction=policy)
        old = c.insert((0, 0, "a"), blob(64))
        for _ in range(5):  # old but much used: high LRFU score
            c.touch(old)
        c.tick()
        c.insert((0, 1, "a"), blob(64))  # this pass
        c.insert((0, 2, "a"), blob(64))
        c.touch(c.entries[(0, 2, "a")])
        c.insert((0, 3, "a"), blob(64))
        assert {(0, 0, "a"), (0, 1, "a"), (0, 2, "a")} - set(c.entries) == {victim}, policy
    with pytest.raises(ValueError):
        TierCache("t", "cpu", 64, {"a": 0}.get, eviction="fifo")


def test_listener_and_on_evict():
    seen, freed = [], []

    class L:
        def added(self, e):
            seen.append(("+", e.key))

        def removed(self, e):
            seen.append(("-", e.key))

    c = TierCache("t", "cpu", 200, RANK, on_evict=freed.append)
    c.listener = L()
    a = blob(100)
    c.insert((0, 0, "int4"), a)
    c.insert((0, 1, "int4"), blob(100))
    c.tick(5)
    c.touch(c.entries[(0, 1, "int4")])
    c.insert((0, 2, "int4"), blob(100))
    assert seen == [("+", (0, 0, "int4")), ("+", (0, 1, "int4")), ("-", (0, 0, "int4")), ("+", (0, 2, "int4"))]
    assert len(freed) == 1 and freed[0] is a
    assert c.by_expert == {(0, 1): {"int4"}, (0, 2): {"int4"}}
    c.clear()
    assert c.used == 0 and not c.entries and not c.by_expert


def test_host_pool_exact_slots_cap_and_quarantine():
    """moelab tests/test_units.py:252-267: exact-size buffers, a double release ignored, a released
    buffer unavailable until the next layer, the cap respected with ordinary buffers beyond it."""
    pool = HostPool({"fp16": 3000, "int4": 800}, cap_bytes=64 * 1024, pin=False, log=lambda *a: None)
    a = pool.acquire("fp16")
    assert a.numel() == 3000 and pool.is_pooled(a) and a.data_ptr() % 4096 == 0
    pool.release(a)
    pool.release(a)  # double release ignored
    b = pool.acquire("fp16")
    assert b.data_ptr() != a.data_ptr()  # quarantined until the next layer
    pool.advance()
    assert pool.acquire("fp16").data_ptr() == a.data_ptr()  # reusable now, and taken first
    blobs = [pool.acquire("int4") for _ in range(200)]
    assert pool.allocated <= pool.cap and pool.fallbacks > 0
    assert all(x.numel() == 800 for x in blobs)
    assert not pool.is_pooled(blobs[-1]) and pool.is_pooled(blobs[0])


def test_host_pool_event_gates_reuse():
    class Ev:
        def __init__(self):
            self.done = False

        def query(self):
            return self.done

    pool = HostPool({"int4": 4096}, cap_bytes=16 * 4096, pin=False, log=lambda *a: None)
    slots = [pool.acquire("int4") for _ in range(16)]
    assert all(pool.is_pooled(x) for x in slots) and pool.allocated == pool.cap
    ev = Ev()
    pool.release(slots[0], ev)
    pool.advance()
    extra = pool.acquire("int4")
    assert not pool.is_pooled(extra) and pool.fallbacks == 1  # the copy reading slot 0 is in flight
    ev.done = True
    assert pool.acquire("int4").data_ptr() == slots[0].data_ptr()


def test_host_pool_space_freed_by_one_precision_serves_another():
    """moelab tests/test_units.py:270-291 (a `lo` run fills the pool with int4, a `hobbit` run then
    needs int8 buffers): freed neighbouring extents merge, so the larger records fit without any
    new allocation."""
    pool = HostPool({"int8": 8192, "int4": 4096}, cap_bytes=4 * 65536, pin=False, log=lambda *a: None)
    lo = []
    while True:
        b = pool.acquire("int4")
        if not pool.is_pooled(b):
            break
        lo.append(b)
    assert pool.allocated == pool.cap and len(lo) == pool.cap // 4096 and pool.fallbacks == 1
    for b in lo:
        pool.release(b)
    pool.advance()
    hi = [pool.acquire("int8") for _ in range(20)]
    assert all(pool.is_pooled(x) for x in hi) and pool.fallbacks == 1
    assert pool.allocated == pool.cap
    assert len({x.data_ptr() for x in hi}) == 20
    spans = sorted((x.data_ptr(), x.data_ptr() + x.numel()) for x in hi)
    assert all(e0 <= s1 for (_, e0), (s1, _) in zip(spans, spans[1:]))  # no overlap
    pool.close()
    assert pool.allocated == 0 and "0.00" in pool.describe()


def test_host_pool_arena_rule():
    """Arenas of 256 MiB (or the room left under the cap, if smaller), at least one record; a
    Qwen3-Next-shaped int4 record takes exactly its pages."""
    rb = 1_671_168  # 408 pages
    pool = HostPool({"int4": rb}, cap_bytes=1 << 30, pin=False, log=lambda *a: None)
    x = pool.acquire("int4")
    assert pool.allocated == 256 << 20 and x.numel() == rb
    assert pool.free_bytes == (256 << 20) - rb
    small = HostPool({"int4": rb}, cap_bytes=5 * rb + 100, pin=False, log=lambda *a: None)
    ys = [small.acquire("int4") for _ in range(6)]
    assert small.allocated == 5 * rb and small.fallbacks == 1 and sum(small.is_pooled(y) for y in ys) == 5


class _Ev:
    """Stands in for a device event: done or not."""

    def __init__(self, done=False):
        self.done = done

    def query(self):
        return self.done


def test_device_pool_pages():
    """The device record pool (on host memory here: the bookkeeping is what is tested) carves
    slots of every precision from the same pages: the pages of a freed slot serve the other
    precision, neighbours coalesce, pending events travel with the pages, and the cap holds."""
    from moelab_hip.offload import DevicePool

    rb = {"fp16": 3 * 4096 + 100, "int4": 4096}
    pool = DevicePool(rb, 9 * 4096, "cpu")
    a, ea = pool.acquire("fp16")            # pages 0-3
    b, _ = pool.acquire("int4")             # page 4
    c, _ = pool.acquire("fp16")             # pages 5-8
    assert ea == [] and a.numel() == rb["fp16"] and a.data_ptr() % 4096 == 0
    assert pool.allocated == 9 * 4096 and pool.free_pages() == 0
    with pytest.raises(RuntimeError, match="pool full"):
        pool.acquire("int4")
    pending = _Ev()
    pool.release(a, "fp16", pending)        # pages 0-3 free once `pending` has passed
    ints = [pool.acquire("int4") for _ in range(4)]  # the fp16 slot's pages serve four int4 records
    assert all(evs == [pending] for _, evs in ints)
    assert {t.data_ptr() for t, _ in ints} == {a.data_ptr() + i * 4096 for i in range(4)}
    for t, _ in ints:
        pool.release(t, "int4")
    pool.release(b, "int4")
    assert pool.free_pages() == 5 and len(pool.free_ext[0]) == 1  # pages 0-4 coalesced
    pending.done = True
    d, evs = pool.acquire("fp16")           # done events are dropped
    assert evs == [] and d.data_ptr() == a.data_ptr()
    pool.release(c, "fp16")
    pool.release(d, "fp16")
    assert pool.free_pages() == 9 and pool.free_ext[0] == [[0, 9, []]] and not pool.lent


def test_device_pool_holds_cap_over_record_size_records(monkeypatch):
    """Slabs are cut to a whole number of the largest records, so a pool whose slab size is not a
    multiple of the record size still holds cap // record_bytes records (a Qwen3-Next int4
    record is 408 pages: 160 of them leave 256 pages of a 65,536-page slab, which no record fits)."""
    import moelab_hip.offload as off

    monkeypatch.setattr(off, "SLAB_BYTES", 64 * 4096)  # 64 pages: 6 records of 10 pages + 4 left
    rb = {"int4": 10 * 4096}
    pool = off.DevicePool(rb, 60 * 10 * 4096, "cpu")
    got = [pool.acquire("int4") for _ in range(60)]
    assert len({t.data_ptr() for t, _ in got}) == 60 and pool.allocated == 60 * 10 * 4096
    with pytest.raises(RuntimeError, match="pool full"):
        pool.acquire("int4")


def test_mass_prediction():
    """moelab's score-mass prefetch (runtime.py:851-870): the most probable experts while the mass
    before each is below m, at most 2k; j < k pairs with the router's j-th weight."""
    from moelab_hip.offload import mass_prediction

    confident = [10.0] + [0.0] * 15
    assert mass_prediction(confident, [0.9, 0.05], 0.8) == [(0, 0)]  # one expert holds the mass
    flat = [0.0] * 8
    assert mass_prediction(flat, [0.5, 0.5], 0.8) == [(0, 0), (1, 1), (2, 2), (3, 3)]  # capped at 2k
    assert mass_prediction(flat, [0.5, 0.5], 0.3) == [(0, 0), (1, 1), (2, 2)]  # 0, 1/8, 2/8 < 0.3
    assert mass_prediction([0.0, 3.0, 1.0], [0.8, 0.2], 1.0) == [(1, 0), (2, 1), (0, 2)]  # kp = E = 3
    rnd = torch.Generator().manual_seed(3)
    for _ in range(20):  # against the softmax / topk / cumsum of the reference's tensor form
        lg = torch.randn(64, generator=rnd) * 2
        m = float(torch.rand(1, generator=rnd)) * 0.9 + 0.05
        pv, pi = torch.softmax(lg, 0).topk(16)
        keep = ((pv.cumsum(0) - pv) < m).tolist()
        want = [(int(pi[j]), j) for j in range(16) if keep[j]]
        assert mass_prediction(lg.tolist(), [0.0] * 8, m) == want


def test_mass_wants_precisions():
    """The score-mass prediction's precisions (moelab runtime.py:872-890): experts within the
    router's top k take the one-token rule's precision (skipped ones are dropped), the experts
    beyond it the lowest precision."""
    from types import SimpleNamespace

    from moelab_hip.offload import OffloadDecoder
    from moelab_hip.policy import PrecisionPolicy

    lg = torch.tensor([0.0, 4.0, 3.0, 2.0, 1.0, -5.0], dtype=torch.float16)
    fake = SimpleNamespace(policy=PrecisionPolicy("weight", t1=0.5, upgrade=False), precisions=["fp16", "int4"],
                           rb_logits=lg, prefetch_mass=0.999)
    want = OffloadDecoder._mass_wants(fake, 0, [0.7, 0.3])  # k = 2: kp = 4 most probable experts
    assert list(want) == [1, 2, 3, 4]
    assert want[1][0] == "fp16" and want[2][0] == "int4"     # weight rule: 0.7 >= 0.5, 0.3 < 0.5
    assert want[3] == ("int4", 2, 0.0) and want[4] == ("int4", 2, 0.0)  # beyond the top k: lowest
    fake.prefetch_mass = 0.8  # p = 0.636, 0.234, 0.086, ...: the mass before expert 3 is 0.870
    assert list(OffloadDecoder._mass_wants(fake, 0, [0.7, 0.3])) == [1, 2]
    fake.prefetch_mass = 0.5
    assert list(OffloadDecoder._mass_wants(fake, 0, [0.7, 0.3])) == [1]
