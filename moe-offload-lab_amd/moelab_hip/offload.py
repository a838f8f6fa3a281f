"""
Expert offload for decode: every record lives in pinned host memory, a bounded set of them is
resident in device memory under an LRFU cache, and the records a layer needs are staged on a
copy stream before its experts run, next-layer predictions in the background.

The host-side objects keep the names, arguments and semantics of moelab's offload runtime, so
code written against those objects works on these:
  HostPool     moelab/hostpool.py:52-185   (tiers.py) page extents of pinned arenas
  TierCache    moelab/cache.py:78-311      (tiers.py) LRFU (Lee et al. 2001), indexed victim heap
  Stager       moelab/runtime.py:186 (copy_stream), 310-326 (`_to_fast`), 328-333 (`_ready`)
  DeviceTable  moelab/fullgraph.py:43-98   TierCache listener keeping the device record table
Stager takes any pinned uint8 record buffer, so the reference's own HostPool slots and TierCache
entries can drive it unchanged.
What changes is the device side: a layer's records are staged by ONE moehip_stage_records call
(a gather kernel reading pinned host memory directly, or SDMA copies) into slots of a fixed
device pool (no allocator traffic), and table entries are written on the copy stream after
the bytes (moehip_table_set), so a non-zero entry always points at a complete record.

Slot reuse is stream-ordered: an evicted record's table entry is cleared on the compute stream,
an event recorded after that clear travels with the freed slot, and the copy stream waits on it
before writing the slot again. Nothing here synchronises the host except the routing readback
of `OffloadDecoder.layer` (the host must know which experts to stage).
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import torch

from . import _lib
from .layer import MoEDecoder
from .policy import PrecisionPolicy, level_to_precision
from .tiers import HostPool, TierCache  # noqa: F401  (re-exported: the runtime imports them from here)

SLAB_BYTES = 256 << 20
STAGE_MAX = 32   # records per moehip_stage_records call
TABLE_MAX = 64   # entries per moehip_table_set call
STAGE_MODES = {"kernel": 0, "sdma": 1}


# ---------------------------------------------------------------------------------------------
# Device tier
# ---------------------------------------------------------------------------------------------
class DevicePool:
    """Fixed device memory for resident records, shared by every record precision: slabs
    (<= 256 MiB, allocated once, up to the cap, never returned to the allocator) cut into 4096-B
    pages; a record slot is a run of pages taken first-fit from a slab's free extents, and a
    released slot's pages rejoin their neighbours. Each free extent carries the events after
    which its pages may be overwritten (the copy stream waits on them), so records of any
    precision can reuse any freed space: a two-precision cache never strands one precision's
    slots while the other runs out."""

    PAGE = 4096

    def __init__(self, record_bytes: dict, cap_bytes: int, device):
        self.record_bytes = dict(record_bytes)
        self.cap = int(cap_bytes)
        self.device = torch.device(device)
        self.slabs: list[torch.Tensor] = []
        self.free_ext: list[list] = []   # per slab: sorted [first page, pages, [events]]
        self.allocated = 0
        self.lent: dict[int, tuple] = {}  # slot address -> (slab, first page, pages)

    def _pages(self, prec: str) -> int:
        return (self.record_bytes[prec] + self.PAGE - 1) // self.PAGE

    def _new_slab(self, pages: int) -> bool:
        room = (self.cap - self.allocated) // self.PAGE
        if room < pages:
            return False
        # a whole number of the largest records per slab: a slab's tail shorter than a record
        # would be capacity the cap counts but no record of that size can use
        unit = max(self._pages(p) for p in self.record_bytes)
        n = min(max(pages, SLAB_BYTES // self.PAGE // unit * unit), room)
        slab = torch.empty(n * self.PAGE + self.PAGE, dtype=torch.uint8, device=self.device)
        off = (-slab.data_ptr()) % self.PAGE
        self.slabs.append(slab[off:off + n * self.PAGE])
        self.free_ext.append([[0, n, []]])
        self.allocated += n * self.PAGE
        return True

    def _carve(self, pages: int):
        for si, exts in enumerate(self.free_ext):
            for ei, ext in enumerate(exts):
                if ext[1] >= pages:
                    first, events = ext[0], ext[2]
                    if ext[1] == pages:
                        exts.pop(ei)
                    else:
                        ext[0] += pages
                        ext[1] -= pages
                        ext[2] = list(events)
                    return si, first, [e for e in events if not e.query()]
        return None

    def acquire(self, prec: str):
        """(slot, events to wait on before writing it); raises when the cap is reached."""
        pages = self._pages(prec)
        got = self._carve(pages)
        if got is None and self._new_slab(pages):
            got = self._carve(pages)
        if got is None:
            raise RuntimeError(f"device record pool full ({self.allocated / 2**30:.2f} GiB, cap "
                               f"{self.cap / 2**30:.2f} GiB): raise the budget margin")
        si, first, events = got
        slot = self.slabs[si][first * self.PAGE:first * self.PAGE + self.record_bytes[prec]]
        self.lent[slot.data_ptr()] = (si, first, pages)
        return slot, events

    def release(self, slot: torch.Tensor, prec: str, event=None) -> None:
        """Return a slot; its pages are reusable once `event` (if any) has passed on the device."""
        si, first, pages = self.lent.pop(slot.data_ptr())
        exts = self.free_ext[si]
        ev = [event] if event is not None else []
        i = 0
        while i < len(exts) and exts[i][0] < first:
            i += 1
        exts.insert(i, [first, pages, ev])
        # merge with the extent after, then with the one before
        if i + 1 < len(exts) and exts[i][0] + exts[i][1] == exts[i + 1][0]:
            nxt = exts.pop(i + 1)
            exts[i][1] += nxt[1]
            exts[i][2] = exts[i][2] + nxt[2]
        if i > 0 and exts[i - 1][0] + exts[i - 1][1] == exts[i][0]:
            cur = exts.pop(i)
            exts[i - 1][1] += cur[1]
            exts[i - 1][2] = exts[i - 1][2] + cur[2]
            i -= 1
        exts[i][2] = [e for e in exts[i][2] if not e.query()]

    def free_pages(self) -> int:
        return sum(e[1] for exts in self.free_ext for e in exts)


class DeviceTable:
    """Listener of the device TierCache (moelab/fullgraph.py:43-98): the record table rtab
    (L, P, E) int64 on the device, layer-major as the decode kernels read it.

    added(e): an entry whose copy is in flight (e.event set) is written by the next `flush_adds`
    on the copy stream, i.e. after its bytes; one already complete is written at once on the
    compute stream. removed(e): cleared at once on the compute stream, after every kernel
    already enqueued there; `removal_event` marks that point (freed slots wait on it)."""

    def __init__(self, num_layers: int, precisions: list, num_experts: int, device):
        self.precs = list(precisions)
        self.L, self.P, self.E = num_layers, len(self.precs), num_experts
        self.device = torch.device(device)
        self.dev = torch.zeros(num_layers, self.P, num_experts, dtype=torch.int64, device=self.device)
        self.pending: list[tuple[int, int]] = []
        self.removal_event = None
        self.adds_before = None  # event the next add flush waits on (last removal)
        self.launches = 0

    def _index(self, key) -> int:
        l, x, p = key
        return (l * self.P + self.precs.index(p)) * self.E + x

    def _set(self, pairs: list, stream) -> None:
        for i in range(0, len(pairs), TABLE_MAX):
            part = pairs[i:i + TABLE_MAX]
            idx = (ctypes.c_int64 * len(part))(*[a for a, _ in part])
            val = (ctypes.c_int64 * len(part))(*[b for _, b in part])
            _lib.call("moehip_table_set", self.dev.data_ptr(), self.dev.numel(), idx, val, len(part),
                      stream.cuda_stream)
            self.launches += 1

    def added(self, e) -> None:
        pair = (self._index(e.key), e.blob.data_ptr())
        if e.event is None:
            self._set([pair], torch.cuda.current_stream(self.device))
        else:
            self.pending.append(pair)

    def removed(self, e) -> None:
        idx = self._index(e.key)
        self.pending = [p for p in self.pending if p[0] != idx]
        cur = torch.cuda.current_stream(self.device)
        self._set([(idx, 0)], cur)
        ev = torch.cuda.Event()
        ev.record(cur)
        self.removal_event = ev
        self.adds_before = ev

    def flush_adds(self, copy_stream) -> None:
        if not self.pending:
            return
        if self.adds_before is not None:
            copy_stream.wait_event(self.adds_before)
            self.adds_before = None
        self._set(self.pending, copy_stream)
        self.pending = []


class Stager:
    """Host record -> device slot copies on a dedicated copy stream (default priority).

    `stage(items)` stages a batch [(host_blob, precision)] with one moehip_stage_records call
    per 32 records (mode "kernel": a gather kernel reading the pinned host records directly;
    "sdma": one hipMemcpyAsync each), flushes the table entries after them and records one
    event. `to_fast(blob, prec)` and `ready(blob, ev)` keep the reference signatures
    (runtime.py:310-333)."""

    def __init__(self, device, pool: DevicePool, table: DeviceTable | None = None, mode: str = "kernel"):
        if mode not in STAGE_MODES:
            raise ValueError(f"staging mode {mode} (kernel or sdma)")
        self.device = torch.device(device)
        self.pool, self.table, self.mode = pool, table, mode
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self._inflight: list[tuple] = []  # (event, host blobs) kept alive until the copy is done
        self.bytes_h2d = 0
        self.batches = 0

    def _prune(self) -> None:
        self._inflight = [(ev, b) for ev, b in self._inflight if not ev.query()]

    def stage(self, items: list, mode: str | None = None) -> tuple[list, object]:
        """[(host_blob, prec)] -> ([device slot], event after the copies and table entries);
        mode overrides the stager's own ("kernel" or "sdma") for this batch."""
        if not items:
            return [], None
        mode = self.mode if mode is None else mode
        if mode not in STAGE_MODES:
            raise ValueError(f"staging mode {mode} (kernel or sdma)")
        self._prune()
        dsts, waits = [], []
        for blob, prec in items:
            if blob.dtype != torch.uint8 or not blob.is_contiguous() or blob.numel() != self.pool.record_bytes[prec]:
                raise RuntimeError(f"stage: host record of {blob.numel()} B for {prec} "
                                   f"({self.pool.record_bytes[prec]} B expected)")
            if mode == "kernel" and not blob.is_pinned():
                raise RuntimeError("stage: kernel staging reads pinned host memory; this record is pageable")
            slot, evs = self.pool.acquire(prec)
            dsts.append(slot)
            waits.extend(evs)
        cs = self.copy_stream
        for ev in waits:
            cs.wait_event(ev)
        code = STAGE_MODES[mode]
        for i in range(0, len(items), STAGE_MAX):
            part = list(zip(items[i:i + STAGE_MAX], dsts[i:i + STAGE_MAX]))
            arr = (_lib.Copy * len(part))()
            for j, ((blob, _), dst) in enumerate(part):
                arr[j].src, arr[j].dst, arr[j].bytes = blob.data_ptr(), dst.data_ptr(), blob.numel()
            _lib.call("moehip_stage_records", arr, len(part), code, cs.cuda_stream)
        self.bytes_h2d += sum(b.numel() for b, _ in items)
        self.batches += 1
        done = torch.cuda.Event()
        done.record(cs)
        self._inflight.append((done, [b for b, _ in items]))
        return dsts, done

    def flush_table(self):
        """Write the pending table entries on the copy stream (after the staged bytes); returns the
        event that covers bytes and entries."""
        if self.table is None:
            return None
        self.table.flush_adds(self.copy_stream)
        ev = torch.cuda.Event()
        ev.record(self.copy_stream)
        return ev

    def to_fast(self, blob: torch.Tensor, prec: str):
        """One record to the device (runtime.py:310-326): (device slot, event)."""
        dsts, ev = self.stage([(blob, prec)])
        return dsts[0], ev

    @staticmethod
    def ready(blob: torch.Tensor, ev) -> None:
        """Before the compute stream reads a staged record (runtime.py:328-333). Slots belong to
        the pool and are never freed to the allocator, so no record_stream is needed."""
        if ev is not None:
            torch.cuda.current_stream(blob.device).wait_event(ev)


def mass_prediction(logits, weights: list, mass: float) -> list[tuple[int, int]]:
    """moelab's score-mass prefetch (runtime.py:851-870, 872-890, prefetch_mass = m): the router's
    most probable experts, in decreasing probability of the softmax over all E logits, while the
    probability before each is below m, at most 2k of them (kp = min(E, 2k)). Returns
    [(expert, j)]: j < k pairs the j-th most probable expert with the router's j-th top-k weight
    (`weights`, decreasing), j >= k marks an expert beyond the router's top-k."""
    import numpy as np

    lg = np.asarray(logits, dtype=np.float32).reshape(-1)
    k = len(weights)
    kp = min(lg.size, 2 * k)
    e = np.exp(lg - lg.max())
    probs = (e / e.sum()).astype(np.float32)
    order = np.argsort(-probs, kind="stable")[:kp]
    pv = probs[order]
    chosen = (np.cumsum(pv) - pv) < mass
    return [(int(order[j]), j) for j in range(kp) if chosen[j]]


# ---------------------------------------------------------------------------------------------
# Offloaded decode
# ---------------------------------------------------------------------------------------------
class OffloadDecoder:
    """Decode with experts offloaded to pinned host memory (moelab/runtime.py:523-750 decode
    path, fast tier only): per layer, route on the GPU, read the k choices back, look them up in
    the device TierCache, stage the misses on the copy stream (one batch), make the compute
    stream wait for every needed record, run the fused experts kernel on the resident table,
    then stage the next layer's predicted experts in the background (runtime.py:899-951).

    host_record(layer, expert, prec) -> pinned uint8 tensor of the record (the host tier): a
    callable over records in host memory, or a `diskstore.DiskTier` (RAM cache over a store on
    disk, which also offers `many` for a batch and `copied` for the copies' completion).
    fast_budget_bytes bounds the resident records (the TierCache budget); the device pool holds
    that plus `margin_records` slots of headroom for copies in flight. `mode` stages the misses
    (the compute stream waits for them); `prefetch_mode` ("sdma" by default) stages the
    predicted experts, which copy while the decode kernel runs: a gather kernel there would hold
    CU slots that the decode kernel's grid (every workgroup resident at once) waits for.
    `prefetch_mass` m (moelab's S3, runtime.py:79, 851-890): the gate predictor stages the next
    layer's most probable experts up to probability mass m (at most 2k; those within the router's
    top k at their policy precision, the others at the lowest one) instead of its top k."""

    def __init__(self, layouts: dict, num_layers: int, num_experts: int, k: int, host_record, fast_budget_bytes: int,
                 device, policy: PrecisionPolicy | None = None, dtype=torch.float16, router_weights: list | None = None,
                 renorm: bool = False, mode: str = "kernel", half_life: float = 32.0, eviction: str = "lrfu",
                 margin_records: int | None = None, predictor: str = "none", prefetch_mode: str = "sdma",
                 prefetch_mass: float | None = None):
        if prefetch_mode not in STAGE_MODES:
            raise ValueError(f"prefetch staging mode {prefetch_mode} (kernel or sdma)")
        if prefetch_mass is not None and not 0.0 < prefetch_mass <= 1.0:
            raise ValueError(f"prefetch_mass {prefetch_mass}: in (0, 1] or None")
        self.prefetch_mode = prefetch_mode
        self.prefetch_mass = prefetch_mass
        self.device = torch.device(device)
        _lib.check_device(self.device)
        self.precisions = list(layouts)
        self.layouts = dict(layouts)
        self.L, self.E, self.k = num_layers, num_experts, k
        self.host_record = host_record
        self.policy = policy or PrecisionPolicy("lo")
        rbs = {p: lay["record_bytes"] for p, lay in layouts.items()}
        rank = {p: i for i, p in enumerate(self.precisions)}
        margin = (2 * k + 2 if margin_records is None else margin_records) * max(rbs.values())
        self.pool = DevicePool(rbs, fast_budget_bytes + margin, self.device)
        self.table = DeviceTable(num_layers, self.precisions, num_experts, self.device)
        self.cache = TierCache("VRAM", self.device, fast_budget_bytes, rank.get, half_life, pin_fraction=0.0,
                               on_evict=self._evicted, eviction=eviction)
        self.cache.listener = self.table
        self.stager = Stager(self.device, self.pool, self.table, mode)
        view = SimpleNamespace(device=self.device, precisions=self.precisions, layouts=self.layouts, L=num_layers,
                               E=num_experts, rtab=self.table.dev)
        # the host decides what to stage with levels_one, so the kernel uses the same float64 rule
        self.dec = MoEDecoder(view, k, self.policy, dtype, router_weights=router_weights, renorm=renorm,
                              one_token_rule=True)
        self._blob_prec: dict[int, str] = {}
        if predictor not in ("none", "gate"):
            raise ValueError(f"predictor {predictor!r}: 'none' or 'gate'")
        if predictor == "gate" and router_weights is None:
            raise ValueError("the gate predictor needs the layers' router weights")
        self.predictor = predictor
        self.renorm = renorm
        # the next layer's gate on the current state (moelab graphs.py:252-263): its own buffers
        self.p_logits = torch.empty(1, num_experts, dtype=dtype, device=self.device)
        self.p_idx = torch.zeros(1, k, dtype=torch.int64, device=self.device)
        self.p_w = torch.zeros(1, k, dtype=dtype, device=self.device)
        self.p_w32 = torch.zeros(1, k, dtype=torch.float32, device=self.device)
        # one pinned readback per layer: the current routing and the prediction for the next layer
        self.rb = torch.empty(2, k, dtype=torch.float32, pin_memory=True)      # weights: current, predicted
        self.rb_idx = torch.empty(2, k, dtype=torch.int64, pin_memory=True)    # experts: current, predicted
        self.rb_logits = torch.empty(num_experts, dtype=dtype, pin_memory=True)  # predicted logits (mass)
        self._predicted: tuple[int, frozenset] | None = None
        self.stats = {"hits": 0, "misses": 0, "prefetch_issued": 0, "prefetch_hits": 0, "skipped": 0,
                      "pred_hits": 0, "pred_total": 0, "miss_downgrades": 0}

    def _evicted(self, blob: torch.Tensor) -> None:
        prec = self._blob_prec.pop(blob.data_ptr())
        self.pool.release(blob, prec, self.table.removal_event)

    def _wants(self, layer: int, idx: list, w: list) -> dict:
        """{expert: (precision, level, s)} of one token's non-skipped slots: the one-token rule
        (levels_one, policy.py:125-137; the kernel uses the same float64 rule) and level ->
        precision (policy.py:188-192)."""
        levels, skip, s = self.policy.levels_one(layer, w)
        return {e: (level_to_precision(levels[j], self.precisions), levels[j], s[j])
                for j, e in enumerate(idx) if not skip[j]}

    def _mass_wants(self, layer: int, weights: list) -> dict:
        """{expert: (precision, level, s)} of a score-mass prediction (runtime.py:872-890): the
        experts paired with the router's top-k weights take the one-token rule's precision unless
        skipped, the further ones the lowest precision."""
        levels, skip, s = self.policy.levels_one(layer, weights)
        low = self.precisions[-1]
        want = {}
        for e, j in mass_prediction(self.rb_logits.float().numpy(), weights, self.prefetch_mass):
            if j < len(weights):
                if not skip[j]:
                    want[e] = (level_to_precision(levels[j], self.precisions), levels[j], s[j])
            else:
                want.setdefault(e, (low, 2, 0.0))
        return want

    def _stage_missing(self, layer: int, want: dict, protect: frozenset, prefetch: bool, stream=None):
        """Look the wanted records of `layer` up in the device cache as moelab's decode does
        (runtime.py:587-615) and stage the misses; returns (events the compute stream must wait
        on, the keys this layer uses: its hits and its staged records). `stream` (the compute
        stream's handle) has already waited for an entry's copy event once it is the entry's
        `waited`: such a hit adds no wait (the stream's later work is ordered after that wait).

        The lookup takes a more precise resident copy only when the policy allows upgrades
        (`allow_upgrade`: never in mode "lo"), as the kernel's copy choice does. With `miss_t1`
        set, a level-0 request that misses and whose unimportance s exceeds miss_t1 + 1e-6 is
        looked up again at level 1 and, if still absent, staged at level 1 (E3; the kernel
        applies the same rule to the table it finds). Prefetches take neither step (moelab's
        background prefetch stages what it is given)."""
        exact = not self.policy.allow_upgrade
        e3 = not prefetch and self.policy.miss_t1 is not None
        count = not prefetch
        waits, todo, used = [], [], set()
        for e, (prec, level, s) in want.items():
            ent = self.cache.lookup(layer, e, prec, exact=exact, count=count)
            if ent is None and e3 and level == 0 and s > self.policy.miss_t1 + 1e-6:
                prec = level_to_precision(1, self.precisions)
                self.stats["miss_downgrades"] += 1
                ent = self.cache.lookup(layer, e, prec, exact=exact, count=count)
            if ent is not None:
                used.add(ent.key)
                if not prefetch:
                    self.cache.touch(ent)
                    self.stats["hits"] += 1
                    if ent.prefetched:
                        self.stats["prefetch_hits"] += 1
                        ent.prefetched = False
                    if ent.event is not None and ent.waited != stream:
                        waits.append(ent.event)
                        ent.waited = stream
                continue
            todo.append((e, prec))
            used.add((layer, e, prec))
        used = frozenset(used) | protect
        if not todo:
            return waits, used
        if not prefetch:
            self.stats["misses"] += len(todo)
        else:
            self.stats["prefetch_issued"] += len(todo)
        many = getattr(self.host_record, "many", None)  # a host tier that reads a batch at once
        srcs = many([(layer, e, p) for e, p in todo]) if many else [self.host_record(layer, e, p) for e, p in todo]
        # a prefetch batch runs beside the next kernels: it goes by SDMA, since the gather kernel's
        # workgroups would take CU slots the decode kernel's co-resident grid needs
        dsts, ev = self.stager.stage([(src, p) for src, (_, p) in zip(srcs, todo)],
                                     mode=self.prefetch_mode if prefetch else None)
        copied = getattr(self.host_record, "copied", None)  # its buffers are reusable after `ev`
        if copied:
            copied(srcs, ev)
        added = []
        for (e, p), dst in zip(todo, dsts):
            self._blob_prec[dst.data_ptr()] = p
            ent = self.cache.insert((layer, e, p), dst, protect=used, event=ev)
            if ent is None or ent.blob is not dst:
                self._blob_prec.pop(dst.data_ptr(), None)
                self.pool.release(dst, p, ev)
                if not prefetch:
                    raise RuntimeError(f"device expert cache cannot hold layer {layer}'s experts "
                                       f"({self.cache.describe()}): raise fast_budget_bytes")
                continue
            ent.prefetched = prefetch
            added.append(ent)
        tab_ev = self.stager.flush_table()
        for ent in added:  # usable once bytes AND table entry are in place
            ent.event = tab_ev
            ent.waited = None if prefetch else stream
        if not prefetch:
            waits.append(tab_ev)
        return list({id(ev): ev for ev in waits}.values()), used

    def _gate_predict(self, layer: int, x: torch.Tensor) -> None:
        """Layer `layer`'s router on x into the prediction buffers (the next layer's gate applied
        to the current hidden state, moelab runtime.py:851-869 with prefetch_mass None)."""
        Wr = self.dec.router_weights[layer]
        _lib.call("moehip_router_topk", x.data_ptr(), Wr.data_ptr(), 1, x.shape[-1], self.E, self.k,
                  1 if self.renorm else 0, _lib.dt_code(x.dtype), self.p_logits.data_ptr(), self.p_idx.data_ptr(),
                  self.p_w.data_ptr(), self.p_w32.data_ptr(), _lib.stream_of(x.device))

    def layer(self, layer: int, x: torch.Tensor, out: torch.Tensor, idx: torch.Tensor | None = None,
              w32: torch.Tensor | None = None, predict: dict | None = None) -> torch.Tensor:
        """out (1, H) = MoE layer `layer` on x (1, H). idx/w32 (device, (1, k)) skip the router.
        predict {expert: precision} for layer + 1 is staged in the background afterwards; without
        it, the gate predictor (predictor='gate') predicts layer + 1's experts from x with that
        layer's router, read back with this layer's routing (one host wait per layer)."""
        cur = torch.cuda.current_stream(self.device)
        if idx is None:
            self.dec.route(layer, x)
            idx, w32 = self.dec.idx, self.dec.w32
        gate = predict is None and self.predictor == "gate" and layer + 1 < self.L
        if gate:
            self._gate_predict(layer + 1, x)
        self.rb_idx[0].copy_(idx.view(-1), non_blocking=True)
        self.rb[0].copy_(w32.view(-1), non_blocking=True)
        if gate:
            self.rb_idx[1].copy_(self.p_idx.view(-1), non_blocking=True)
            self.rb[1].copy_(self.p_w32.view(-1), non_blocking=True)
            if self.prefetch_mass is not None:
                self.rb_logits.copy_(self.p_logits.view(-1), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(cur)
        ev.synchronize()
        ids = self.rb_idx[0].tolist()
        ws = self.rb[0].tolist()
        if self._predicted is not None and self._predicted[0] == layer:
            self.stats["pred_total"] += len(ids)
            self.stats["pred_hits"] += sum(1 for e in ids if e in self._predicted[1])
        self._predicted = None
        if gate:
            pids = self.rb_idx[1].tolist()
            if self.prefetch_mass is None:
                predict = self._wants(layer + 1, pids, self.rb[1].tolist())
            else:
                predict = self._mass_wants(layer + 1, self.rb[1].tolist())
        elif predict:
            predict = {e: (p, 0, 0.0) for e, p in predict.items()}
        if predict and layer + 1 < self.L:
            self._predicted = (layer + 1, frozenset(predict))
        want = self._wants(layer, ids, ws)
        waits, used = self._stage_missing(layer, want, frozenset(), prefetch=False, stream=cur.cuda_stream)
        for wev in waits:
            cur.wait_event(wev)
        self.dec.layer(layer, x, out, idx=idx, w32=w32)
        if predict and layer + 1 < self.L:
            self._stage_missing(layer + 1, predict, used, prefetch=True)
        return out

    def tick(self) -> None:
        """End of a decode token (the LRFU clock)."""
        self.cache.tick()
