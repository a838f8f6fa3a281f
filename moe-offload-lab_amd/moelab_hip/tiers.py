"""
Host-side tiers of the offload path: the pool of host record buffers and the LRFU expert cache.

Both keep the public interface of moelab's runtime objects (moelab/hostpool.py:52-185 `HostPool`,
moelab/cache.py:78-311 `TierCache`: names, constructor arguments, methods, attributes the runtime
reads, and the eviction semantics), so code written against them runs on these. The insides are
built differently:

HostPool    one or a few large page-aligned arenas (pinned when asked) handed out as page
            extents of exactly one record; free space is an address-ordered extent list per arena,
            coalesced on return, so space freed by one precision serves any other directly (no
            per-precision slabs to re-cut). A returned extent waits in quarantine until its event
            has passed and `advance()` was called (a copy or the CPU branch may still read it).
TierCache   LRFU (Lee et al. 2001): an entry accessed at clocks t_i scores sum_i gamma^(clock - t_i),
            gamma = 0.5^(1/half_life). The ranking key log f - t log gamma does not depend on the
            clock, so the eviction candidates live in an indexed binary min-heap keyed
            (log f - t log gamma, sequence) whose entries know their own position: a touched entry
            is re-keyed in place and an evicted or pinned one removed in place, in O(log n), and
            victims that must be skipped (protected keys) are stepped over by a best-first walk of
            the heap tree without popping anything.
"""

from __future__ import annotations

import heapq
import math
import threading
from bisect import bisect_left
from dataclasses import dataclass, field

import torch

PAGE = 4096
ARENA_BYTES = 256 << 20


# ---------------------------------------------------------------------------------------------
# host record buffers
# ---------------------------------------------------------------------------------------------
class HostPool:
    """Bounded pool of host record buffers (interface of moelab/hostpool.py:52-185).

    acquire(prec) -> uint8 tensor of exactly record_bytes[prec], page-aligned; past `cap_bytes` of
    arenas (or once the system refuses to pin more) an ordinary buffer, counted in `fallbacks`.
    release(blob, event=None) -> the extent is reusable once `event` has passed AND advance() has
    been called (the next layer). Thread-safe (disk reader threads acquire)."""

    def __init__(self, record_bytes: dict, cap_bytes: int, pin: bool, log=print):
        self.record_bytes = dict(record_bytes)
        self.cap = int(cap_bytes)
        self.pin = pin
        self.log = log
        self.lock = threading.Lock()
        self.arenas: list[torch.Tensor] = []
        self.allocated = 0
        self._holes: list[list[list[int]]] = []  # per arena: sorted [first page, pages] of free space
        self._lent: dict[int, tuple] = {}        # data_ptr -> (arena, first page, pages)
        self._waiting: list[tuple] = []          # (arena, first page, pages, event, epoch)
        self.epoch = 0
        self.exhausted = False
        self.fallbacks = 0
        self.reclaims = 0  # kept for callers that print it: extents never need re-cutting here

    @staticmethod
    def _pages(nbytes: int) -> int:
        return (nbytes + PAGE - 1) // PAGE

    def _new_arena(self, need_pages: int) -> bool:
        room = (self.cap - self.allocated) // PAGE
        if room < need_pages:
            return False
        pages = min(room, max(need_pages, ARENA_BYTES // PAGE))
        try:
            if self.pin:
                buf = torch.empty(pages * PAGE, dtype=torch.uint8, pin_memory=True)
            else:
                raw = torch.empty(pages * PAGE + PAGE, dtype=torch.uint8)
                o = (-raw.data_ptr()) % PAGE
                buf = raw[o:o + pages * PAGE]
        except RuntimeError as exc:  # the system refused to pin more
            self.exhausted = True
            self.log(f"host pool: pinning refused after {self.allocated / 2**30:.2f} GiB ({type(exc).__name__}); "
                     "ordinary buffers from now on")
            return False
        self.arenas.append(buf)
        self._holes.append([[0, pages]])
        self.allocated += pages * PAGE
        return True

    def _carve(self, need: int):
        """First fit over the arenas in order: (arena, first page) or None."""
        for a, holes in enumerate(self._holes):
            for i, h in enumerate(holes):
                if h[1] >= need:
                    first = h[0]
                    if h[1] == need:
                        holes.pop(i)
                    else:
                        h[0] += need
                        h[1] -= need
                    return a, first
        return None

    def _give_back(self, a: int, first: int, pages: int) -> None:
        holes = self._holes[a]
        i = bisect_left(holes, [first, 0])
        if i > 0 and holes[i - 1][0] + holes[i - 1][1] == first:  # merge with the hole before
            i -= 1
            holes[i][1] += pages
        else:
            holes.insert(i, [first, pages])
        if i + 1 < len(holes) and holes[i][0] + holes[i][1] == holes[i + 1][0]:  # and the one after
            holes[i][1] += holes.pop(i + 1)[1]

    def _drain(self) -> None:
        still = []
        for a, first, pages, ev, epoch in self._waiting:
            if epoch < self.epoch and (ev is None or ev.query()):
                self._give_back(a, first, pages)
            else:
                still.append((a, first, pages, ev, epoch))
        self._waiting = still

    def acquire(self, prec: str) -> torch.Tensor:
        rb = self.record_bytes[prec]
        need = self._pages(rb)
        with self.lock:
            if self._waiting:  # recently freed extents first (low addresses, warm pages)
                self._drain()
            got = self._carve(need)
            if got is None and not self.exhausted and self._new_arena(need):
                got = self._carve(need)
            if got is not None:
                a, first = got
                blob = self.arenas[a][first * PAGE:first * PAGE + rb]
                self._lent[blob.data_ptr()] = (a, first, need)
                return blob
            self.fallbacks += 1
        return torch.empty(rb, dtype=torch.uint8)

    def release(self, blob: torch.Tensor, event=None) -> None:
        """Ignored for buffers from outside the pool and for a second release of the same one."""
        with self.lock:
            ext = self._lent.pop(blob.data_ptr(), None)
            if ext is not None:
                self._waiting.append((*ext, event, self.epoch))

    def advance(self) -> None:
        """Start of a layer: extents released before it become reusable once their event passed."""
        with self.lock:
            self.epoch += 1

    def is_pooled(self, blob: torch.Tensor) -> bool:
        p = blob.data_ptr()
        return any(a.data_ptr() <= p < a.data_ptr() + a.numel() for a in self.arenas)

    @property
    def free_bytes(self) -> int:
        return PAGE * sum(h[1] for holes in self._holes for h in holes)

    def describe(self) -> str:
        s = (f"host pool ({'pinned' if self.pin else 'pageable'}): {self.allocated / 2**30:.2f}/"
             f"{self.cap / 2**30:.2f} GiB in {len(self.arenas)} arenas, {self.free_bytes / 2**20:.0f} MiB free")
        if self.fallbacks:
            s += f", {self.fallbacks} buffers outside the pool"
        return s

    def close(self) -> None:
        with self.lock:
            self.arenas.clear()
            self._holes.clear()
            self._lent.clear()
            self._waiting.clear()
            self.allocated = 0


# ---------------------------------------------------------------------------------------------
# LRFU cache
# ---------------------------------------------------------------------------------------------
@dataclass
class Entry:
    key: tuple
    blob: torch.Tensor
    nbytes: int
    f: float = 0.0
    t: int = 0
    pinned: bool = False
    event: object = None       # copy to this tier still in flight
    waited: object = None      # the stream (handle) that has already waited for `event`
    prefetched: bool = False   # staged ahead and not used yet
    rank: tuple = (0.0, 0)     # (log f - t log gamma, sequence): the eviction order
    slot: int = field(default=-1, repr=False)  # 0 while in the victim heap, -1 = not in it


@dataclass
class TierStats:
    hits: int = 0
    misses: int = 0
    inserts: int = 0
    evictions: int = 0
    rejected: int = 0
    bytes_in: int = 0


class _VictimHeap:
    """Min-heap of entries by Entry.rank with lazy removal (heapq on (rank, entry) pairs; ranks
    are unique, so entries are never compared). A re-ranked entry gets a new pair and its old one
    stays behind, stale: its rank is no longer the entry's, or the entry has left (slot -1). The
    candidate walk pops pairs in rank order, dropping stale ones for good and handing live ones
    back afterwards (restore); the array is also rebuilt from the live pairs once stale ones
    outnumber them. Entry.slot is 0 while the entry is in the heap."""

    def __init__(self):
        self.a: list[tuple] = []
        self.live = 0
        self._held: list[tuple] = []

    def __len__(self):
        return self.live

    @staticmethod
    def _current(item) -> bool:
        r, e = item
        return e.slot >= 0 and e.rank is r

    def _compact(self) -> None:
        if len(self.a) > 2 * self.live + 64:
            self.a = [it for it in self.a if self._current(it)]
            heapq.heapify(self.a)

    def add(self, e: Entry) -> None:
        e.slot = 0
        self.live += 1
        heapq.heappush(self.a, (e.rank, e))
        self._compact()

    def rekey(self, e: Entry) -> None:
        heapq.heappush(self.a, (e.rank, e))
        self._compact()

    def drop(self, e: Entry) -> None:
        e.slot = -1
        self.live -= 1

    def ascending(self):
        """Entries in increasing rank, popped: stale pairs are dropped, live ones held until
        restore() puts them back (call it once the walk is over, however far it went)."""
        a = self.a
        while a:
            it = heapq.heappop(a)
            if self._current(it):
                self._held.append(it)
                yield it[1]

    def restore(self) -> None:
        for it in self._held:
            heapq.heappush(self.a, it)
        self._held.clear()


class TierCache:
    """One memory tier's expert cache (interface of moelab/cache.py:78-311): key (layer, expert,
    precision); a touch sets f <- score + 1 at the current clock; eviction takes unpinned,
    unprotected entries in increasing score (ties: the earlier re-keyed first), or with
    eviction="stale" the entries not touched in the current pass first; pinned entries stay within
    pin_fraction of the budget; repin swaps cold pinned entries for hotter unpinned ones with
    hysteresis. `listener.added/removed(entry)` follow every insertion and eviction, `on_evict(blob)`
    gets every evicted buffer back."""

    def __init__(self, name: str, device, budget_bytes: int, rank_of, half_life: float = 32.0,
                 pin_fraction: float = 0.5, on_evict=None, eviction: str = "lrfu"):
        if eviction not in ("lrfu", "stale"):
            raise ValueError(f"unknown eviction policy {eviction} (lrfu or stale)")
        self.name = name
        self.device = torch.device(device)
        self.budget = int(budget_bytes)
        self.rank_of = rank_of
        self.gamma = 0.5 ** (1.0 / half_life)
        self._log_gamma = math.log(self.gamma)
        self.pin_budget = int(self.budget * pin_fraction)
        self.on_evict = on_evict
        self.eviction = eviction
        self.listener = None
        self.entries: dict[tuple, Entry] = {}
        self.by_expert: dict[tuple, set] = {}
        self.used = 0
        self.pinned_bytes = 0
        self.clock = 0
        self.stats = TierStats()
        self._heap = _VictimHeap()
        self._seq = 0

    # -- scores ----------------------------------------------------------------------------
    def score(self, e: Entry) -> float:
        return e.f * self.gamma ** (self.clock - e.t)

    def _rank(self, e: Entry) -> None:
        """Give e a fresh eviction rank and put it in place among the candidates (pinned: none)."""
        self._seq += 1
        e.rank = (math.log(e.f) - e.t * self._log_gamma, self._seq)
        if e.pinned:
            if e.slot >= 0:
                self._heap.drop(e)
        elif e.slot >= 0:
            self._heap.rekey(e)
        else:
            self._heap.add(e)

    def touch(self, e: Entry) -> None:
        e.f = self.score(e) + 1.0
        e.t = self.clock
        if self.entries.get(e.key) is e:
            self._rank(e)

    def tick(self, n: int = 1) -> None:
        self.clock += n

    # -- lookup ----------------------------------------------------------------------------
    def lookup(self, layer: int, expert: int, need: str, exact: bool = False, count: bool = True) -> Entry | None:
        """The most precise resident copy of (layer, expert) at least as precise as `need` (only
        `need` itself with exact=True); count=False checks without counting a hit or miss."""
        have = self.by_expert.get((layer, expert), ())
        if exact:
            best = need if need in have else None
        else:
            limit = self.rank_of(need)
            best = min((p for p in have if self.rank_of(p) <= limit), key=self.rank_of, default=None)
        if best is None:
            self.stats.misses += count
            return None
        self.stats.hits += count
        return self.entries[(layer, expert, best)]

    def contains(self, key: tuple) -> bool:
        return key in self.entries

    # -- insertion and eviction -------------------------------------------------------------
    def _pick(self, need: int, protect) -> list | None:
        """Entries whose eviction frees room for `need` more bytes, or None (then none is taken)."""
        over = self.used + need - self.budget
        if over <= 0:
            return []
        if self.eviction == "stale":
            order = sorted((e for e in self.entries.values() if not e.pinned and e.key not in protect),
                           key=lambda e: (e.t >= self.clock, self.score(e)))
        else:
            order = (e for e in self._heap.ascending() if e.key not in protect)
        out, freed = [], 0
        try:
            for e in order:
                out.append(e)
                freed += e.nbytes
                if freed >= over:
                    return out
            return None
        finally:
            if self.eviction != "stale":
                self._heap.restore()

    def insert(self, key: tuple, blob: torch.Tensor, pinned: bool = False, protect: frozenset = frozenset(),
               event=None) -> Entry | None:
        """Add an entry, evicting the lowest-ranked unpinned, unprotected ones when needed; None
        when no such room can be made (nothing is evicted then). An existing key is touched."""
        old = self.entries.get(key)
        if old is not None:
            self.touch(old)
            return old
        nbytes = blob.numel() * blob.element_size()
        if pinned and self.pinned_bytes + nbytes > self.pin_budget:
            pinned = False
        victims = None if nbytes > self.budget - self.pinned_bytes else self._pick(nbytes, protect)
        if victims is None:
            self.stats.rejected += 1
            return None
        for v in victims:
            self.evict(v.key)
        e = Entry(key, blob, nbytes, pinned=pinned, event=event)
        e.f, e.t = 1.0, self.clock
        self.entries[key] = e
        self._rank(e)
        self.by_expert.setdefault(key[:2], set()).add(key[2])
        self.used += nbytes
        self.pinned_bytes += nbytes if pinned else 0
        self.stats.inserts += 1
        self.stats.bytes_in += nbytes
        if self.listener is not None:
            self.listener.added(e)
        return e

    def evict(self, key: tuple) -> None:
        e = self.entries.pop(key)
        if e.slot >= 0:
            self._heap.drop(e)
        if e.event is not None and self.device.type == "cuda":
            # a copy into this buffer may still be in flight: later work waits for it
            torch.cuda.current_stream(self.device).wait_event(e.event)
        have = self.by_expert[key[:2]]
        have.discard(key[2])
        if not have:
            del self.by_expert[key[:2]]
        self.used -= e.nbytes
        self.pinned_bytes -= e.nbytes if e.pinned else 0
        self.stats.evictions += 1
        if self.listener is not None:
            self.listener.removed(e)
        if self.on_evict is not None:
            self.on_evict(e.blob)

    def clear(self) -> None:
        for key in list(self.entries):
            self.evict(key)
        self.stats = TierStats()

    # -- pins ------------------------------------------------------------------------------
    def pin(self, key: tuple) -> bool:
        e = self.entries.get(key)
        if e is None:
            return False
        if e.pinned:
            return True
        if self.pinned_bytes + e.nbytes > self.pin_budget:
            return False
        e.pinned = True
        self.pinned_bytes += e.nbytes
        if e.slot >= 0:
            self._heap.drop(e)
        return True

    def unpin(self, key: tuple) -> None:
        e = self.entries.get(key)
        if e is not None and e.pinned:
            e.pinned = False
            self.pinned_bytes -= e.nbytes
            self._rank(e)

    def repin(self, hysteresis: float = 0.25, max_swaps: int = 4) -> list:
        """Pin the hottest unpinned entries: into free pin budget, or in place of a colder pinned
        entry when the candidate scores more than (1 + hysteresis) times it; at most max_swaps
        changes. Returns [(pinned key, unpinned key or None)]."""
        hot = sorted((e for e in self.entries.values() if not e.pinned), key=self.score, reverse=True)
        cold = iter(sorted((e for e in self.entries.values() if e.pinned), key=self.score))
        done: list = []
        victim = None
        for c in hot:
            if len(done) >= max_swaps:
                break
            if self.pinned_bytes + c.nbytes <= self.pin_budget:
                self.pin(c.key)
                done.append((c.key, None))
                continue
            if victim is None or not victim.pinned:
                victim = next((v for v in cold if v.pinned), None)
            if victim is None or self.score(c) <= self.score(victim) * (1.0 + hysteresis):
                break  # the remaining candidates are colder still
            self.unpin(victim.key)
            if not self.pin(c.key):
                self.pin(victim.key)
                break
            done.append((c.key, victim.key))
            victim = None
        return done

    def describe(self) -> str:
        return (f"{self.name}: {self.used / 2**20:.0f}/{self.budget / 2**20:.0f} MiB, {len(self.entries)} entries "
                f"({self.pinned_bytes / 2**20:.0f} MiB pinned)")
