"""
The disk tier: an expert store on disk (moelab/store.py:264-445 `ExpertStore`, the directory
format of store.py:466-561 `build_store`) and the host tier that serves the offloaded decoder
from it.

Directory format (kept identical, so stores built by either side open on the other):
`manifest.json` (format "moelab-expert-store", version 1, store_id, source, model_type, layers,
num_experts, hidden, inter, layouts, complete) and one file per (layer, precision),
`layer{L:03d}.{prec}.bin`, holding the E records of the layer back to back (record e at
e * record_bytes). An optional hot store (`hot.json` + `hot.{prec}.bin`, store.py:331-356) holds
copies of chosen experts on a faster disk.

Reads go through the library's native reader (moehip_disk_read): one descriptor per file, opened
once and shared by every thread (positional reads), plus an O_DIRECT descriptor when `direct` is
on; a record is read as `read_parts` ranges in flight at once on the library's reader threads.

`DiskTier` is the host tier the offloaded decoder takes as its `host_record`: a RAM TierCache over
a HostPool of pinned record buffers in front of the store; the records a layer misses are read
concurrently, and a buffer evicted from RAM goes back to the pool only once the copies that read
it have completed.
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import ctypes
import torch

from . import _lib
from .tiers import HostPool, TierCache

ALIGN = 4096
FORMAT = "moelab-expert-store"


def json_ident(model_type: str, layers: list, E: int, H: int, I: int, layouts: list) -> str:
    """What identifies a store's contents (store.py:444-447): model, shapes, precisions and the
    int scale method ("int4:mse"; plain name for absmax or float formats)."""
    precs = [l["precision"] if l.get("scale") in (None, "absmax") else f"{l['precision']}:{l['scale']}" for l in layouts]
    return json.dumps([model_type, layers, E, H, I, precs])


def write_store(path, layouts: list, layer_names: list, num_experts: int, hidden: int, inter: int, record,
                model_type: str = "synthetic", source: str = "") -> dict:
    """Write a complete store: `record(layer, expert, prec)` gives each record's bytes (a uint8
    tensor or array of record_bytes). Layouts are the store's, most precise first. Returns the
    manifest."""
    out = Path(path)
    out.mkdir(parents=True, exist_ok=True)
    ident = json_ident(model_type, layer_names, num_experts, hidden, inter, layouts)
    manifest = {"format": FORMAT, "version": 1, "store_id": hashlib.sha1(ident.encode()).hexdigest()[:12],
                "source": source, "model_type": model_type, "layers": list(layer_names), "num_experts": num_experts,
                "hidden": hidden, "inter": inter, "layouts": list(layouts), "complete": False}
    (out / "manifest.json").write_text(json.dumps(manifest, indent=1), encoding="utf-8")
    for li in range(len(layer_names)):
        for lay in layouts:
            prec, rb = lay["precision"], lay["record_bytes"]
            with open(out / f"layer{li:03d}.{prec}.bin", "wb") as f:
                for e in range(num_experts):
                    blob = record(li, e, prec)
                    data = blob.cpu().numpy().tobytes() if isinstance(blob, torch.Tensor) else bytes(blob)
                    if len(data) != rb:
                        raise ValueError(f"record ({li}, {e}, {prec}) has {len(data)} bytes, the layout {rb}")
                    f.write(data)
    manifest["complete"] = True
    (out / "manifest.json").write_text(json.dumps(manifest, indent=1), encoding="utf-8")
    return manifest


class ExpertStore:
    """Read access to a store on disk (the interface of moelab/store.py:264-445). Thread-safe."""

    def __init__(self, path):
        self.path = Path(path)
        mpath = self.path / "manifest.json"
        if not mpath.exists():
            raise FileNotFoundError(f"no manifest.json in {self.path} (was the store built?)")
        self.manifest = json.loads(mpath.read_text(encoding="utf-8"))
        if not self.manifest.get("complete"):
            raise RuntimeError(f"the store {self.path} is incomplete (its build did not finish)")
        self.layers: list[str] = self.manifest["layers"]
        self.num_experts: int = self.manifest["num_experts"]
        self.hidden: int = self.manifest["hidden"]
        self.inter: int = self.manifest["inter"]
        self.layouts: dict[str, dict] = {l["precision"]: l for l in self.manifest["layouts"]}
        self.precisions: list[str] = [l["precision"] for l in self.manifest["layouts"]]
        self.direct = False          # O_DIRECT reads (set by the caller; off when the system refuses)
        self.read_parts = 1          # ranges in flight per record
        self.bytes_read = 0
        self.read_seconds = 0.0
        self.direct_reads = 0        # records read with at least one direct range
        self.direct_fallbacks = 0    # records read without one although `direct` was on
        self.hot: dict[str, dict[tuple[int, int], int]] = {}
        self.hot_path: Path | None = None
        self.hot_reads = 0
        self._direct_error: str | None = None
        self._fds: dict[Path, int] = {}
        self._dfds: dict[Path, int] = {}
        self._lock = threading.Lock()

    # -- the manifest ----------------------------------------------------------------------
    @property
    def hi(self) -> str:
        return self.precisions[0]

    @property
    def lo(self) -> str:
        return self.precisions[-1]

    @property
    def store_id(self) -> str:
        return self.manifest["store_id"]

    def rank(self, prec: str) -> int:
        """0 = the most precise; a lower rank may serve a request for a higher one."""
        return self.precisions.index(prec)

    def record_bytes(self, prec: str) -> int:
        return self.layouts[prec]["record_bytes"]

    def layer_index(self, prefix: str) -> int:
        return self.layers.index(prefix)

    def file(self, layer: int, prec: str) -> Path:
        return self.path / f"layer{layer:03d}.{prec}.bin"

    def total_bytes(self, prec: str) -> int:
        return self.record_bytes(prec) * self.num_experts * len(self.layers)

    def summary(self) -> str:
        parts = [f"{p}: {self.record_bytes(p) / 2**20:.2f} MiB/expert, {self.total_bytes(p) / 2**30:.2f} GiB in all"
                 for p in self.precisions]
        return (f"store {self.path}: {len(self.layers)} MoE layers x {self.num_experts} experts "
                f"(H={self.hidden}, I={self.inter}); " + "; ".join(parts))

    # -- hot store -------------------------------------------------------------------------
    def attach_hot(self, hot_dir) -> int:
        """Serve the experts of a hot store (a copy of chosen records on a faster disk) from
        there; returns how many it holds."""
        hot_dir = Path(hot_dir)
        meta = json.loads((hot_dir / "hot.json").read_text(encoding="utf-8"))
        if meta.get("store_id") != self.store_id:
            raise ValueError(f"the hot store {hot_dir} was built for another store")
        self.hot = {p: {tuple(int(v) for v in k.split(":")): int(slot) for k, slot in m.items()}
                    for p, m in meta["experts"].items()}
        self.hot_path = hot_dir
        return sum(len(m) for m in self.hot.values())

    def _locate(self, layer: int, expert: int, prec: str) -> tuple[Path, int]:
        rb = self.record_bytes(prec)
        slot = self.hot.get(prec, {}).get((layer, expert))
        if slot is not None:
            return self.hot_path / f"hot.{prec}.bin", slot * rb
        return self.file(layer, prec), expert * rb

    # -- reads -----------------------------------------------------------------------------
    def _descriptors(self, path: Path) -> tuple[int, int]:
        with self._lock:
            fd = self._fds.get(path)
            if fd is None:
                fd = self._fds[path] = os.open(path, os.O_RDONLY)
            dfd = -1
            if self.direct and self._direct_error is None:
                dfd = self._dfds.get(path, -1)
                if dfd < 0:
                    try:
                        dfd = self._dfds[path] = os.open(path, os.O_RDONLY | getattr(os, "O_DIRECT", 0))
                    except OSError as e:  # a file system without direct reads: ordinary ones
                        self._direct_error = f"{e.__class__.__name__}: {e}"
                        dfd = -1
            return fd, dfd

    def read(self, layer: int, expert: int, prec: str, out: torch.Tensor | None = None,
             parts: int | None = None) -> torch.Tensor:
        """Read one record from disk into `out` (a contiguous uint8 host tensor of record_bytes,
        e.g. a pinned pool buffer; a new one when None); `parts` ranges in flight (default
        read_parts)."""
        rb = self.record_bytes(prec)
        if out is None:
            out = torch.empty(rb, dtype=torch.uint8)
        if out.device.type != "cpu" or out.dtype != torch.uint8 or out.numel() != rb or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous uint8 host tensor of {rb} bytes")
        path, offset = self._locate(layer, expert, prec)
        fd, dfd = self._descriptors(path)
        parts = self.read_parts if parts is None else parts
        parts = max(1, min(int(parts), 64)) if rb >= 2 * ALIGN else 1
        nd, nf = ctypes.c_int(0), ctypes.c_int(0)
        t0 = time.perf_counter()
        _lib.call("moehip_disk_read", fd, dfd, offset, out.data_ptr(), rb, parts, ctypes.byref(nd), ctypes.byref(nf))
        dt = time.perf_counter() - t0
        with self._lock:
            self.bytes_read += rb
            self.read_seconds += dt
            if self.hot_path is not None and path.parent == self.hot_path:
                self.hot_reads += 1
            if self.direct:
                if nd.value > 0:
                    self.direct_reads += 1
                else:
                    self.direct_fallbacks += 1
                if nf.value > 0 and self._direct_error is None:
                    self._direct_error = "a direct read was refused (EINVAL: the file system; EFAULT: the buffer)"
        return out

    def close(self) -> None:
        with self._lock:
            for fd in list(self._fds.values()) + list(self._dfds.values()):
                os.close(fd)
            self._fds.clear()
            self._dfds.clear()


class DiskTier:
    """The host tier of the offloaded decoder over a store on disk (moelab/runtime.py:250-333:
    RAM cache in front of disk reads into pool buffers). Call it as `host_record(layer, expert,
    prec)`; `many(items)` serves a layer's batch with the missing records read concurrently;
    `copied(blobs, event)` tells it which copy last read each buffer, so an eviction returns the
    buffer to the pool only after that copy."""

    def __init__(self, store: ExpertStore, host_budget_bytes: int, pin: bool = True, parts: int | None = None,
                 direct: bool = False, half_life: float = 32.0, readers: int = 8, log=lambda *a: None):
        self.store = store
        store.direct = direct
        if parts is not None:
            store.read_parts = parts
        rbs = {p: store.record_bytes(p) for p in store.precisions}
        rank = {p: i for i, p in enumerate(store.precisions)}
        # headroom for one batch in flight beyond the cache budget
        self.pool = HostPool(rbs, host_budget_bytes + 32 * max(rbs.values()), pin, log=log)
        self.cache = TierCache("RAM", "cpu", host_budget_bytes, rank.get, half_life, pin_fraction=0.0,
                               on_evict=self._evicted)
        self._last_copy: dict[int, object] = {}
        self._io = ThreadPoolExecutor(max_workers=readers, thread_name_prefix="moehip-disk")
        self.stats = {"host_hits": 0, "disk_reads": 0, "bytes_disk": 0}

    def _evicted(self, blob: torch.Tensor) -> None:
        self.pool.release(blob, self._last_copy.pop(blob.data_ptr(), None))

    def _read(self, key: tuple) -> torch.Tensor:
        """One record into a pool buffer; the buffer goes back to the pool if the read fails."""
        layer, e, prec = key
        buf = self.pool.acquire(prec)
        try:
            return self.store.read(layer, e, prec, out=buf)
        except BaseException:
            self.pool.release(buf)
            raise

    def many(self, items: list) -> list:
        """Pinned record buffers for [(layer, expert, prec), ...]: RAM hits as they are, the
        misses read from disk at once; every record of the batch stays cached until the next."""
        self.pool.advance()
        keys = [tuple(k) for k in items]
        protect = frozenset(keys)
        out: dict[tuple, torch.Tensor] = {}
        todo = []
        for k in keys:
            ent = self.cache.entries.get(k)
            if ent is not None:
                self.cache.touch(ent)
                self.stats["host_hits"] += 1
                out[k] = ent.blob
            elif k not in todo:
                todo.append(k)
        # every read of the batch runs to its end before anything is raised: a failed read has
        # released its own buffer, the others' buffers are cached (or released) as usual
        futures = [self._io.submit(self._read, k) for k in todo]
        first_error = None
        for k, fut in zip(todo, futures):
            try:
                blob = fut.result()
            except Exception as exc:  # noqa: BLE001  (re-raised below, after the batch is settled)
                first_error = first_error or exc
                continue
            self.stats["disk_reads"] += 1
            self.stats["bytes_disk"] += blob.numel()
            ent = self.cache.insert(k, blob, protect=protect)
            if ent is None or ent.blob is not blob:
                self.pool.release(blob)
                first_error = first_error or RuntimeError(
                    f"the host cache cannot hold the batch ({self.cache.describe()}): raise host_budget_bytes")
                continue
            out[k] = blob
        if first_error is not None:
            raise first_error
        return [out[k] for k in keys]

    def __call__(self, layer: int, expert: int, prec: str) -> torch.Tensor:
        return self.many([(layer, expert, prec)])[0]

    def copied(self, blobs: list, event) -> None:
        for b in blobs:
            self._last_copy[b.data_ptr()] = event

    def close(self) -> None:
        self._io.shutdown(wait=True)
        self.store.close()
        self.pool.close()
