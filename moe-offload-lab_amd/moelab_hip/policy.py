"""
HOBBIT precision policy (moelab/policy.py), host side.

Same dataclass fields and rules as the reference; `device_policy(layer)` packs the parameters
for the on-GPU decision kernel (moehip_decide_table), with the reference's +1e-6 threshold
slack folded in and rounded to fp32 the way the reference's tensor comparisons round it
(policy.py:120-122, fullgraph.py:110-113).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ._lib import Policy

MODES = ("hi", "lo", "hobbit", "weight")


@dataclass
class PrecisionPolicy:
    """policy.py:20-58. mode "weight" (not in moelab) is the benchmark configurations' rule: an
    expert is served at level 0 (the most precise record) when its own routed weight is >= t1, else
    at level 2; no skipping."""

    mode: str = "hobbit"
    t1: float = 0.6
    t2: float | None = None
    protect_layers: frozenset = field(default_factory=frozenset)
    hi_vote: float = 0.5
    upgrade: bool = True
    t_mid: float | None = None
    t1_layers: dict | None = None
    miss_t1: float | None = None

    def __post_init__(self):
        if self.mode not in MODES:
            raise ValueError(f"unknown mode {self.mode} (choices: {', '.join(MODES)})")
        self.protect_layers = frozenset(self.protect_layers)
        if self.t2 is not None and self.t2 < self.t1:
            raise ValueError("t2 must be >= t1")
        if self.t_mid is not None and self.t_mid < self.t1:
            raise ValueError("t_mid must be >= t1")
        if self.t1_layers is not None:
            self.t1_layers = {int(k): float(v) for k, v in self.t1_layers.items()}

    def t1_for(self, layer: int) -> float:
        return self.t1_layers.get(layer, self.t1) if self.t1_layers else self.t1

    def _fixed(self, layer: int) -> int | None:
        if self.mode == "hi" or layer in self.protect_layers:
            return 0
        if self.mode == "lo":
            return 2
        return None

    @staticmethod
    def unimportance(weights: torch.Tensor) -> torch.Tensor:
        """policy.py:77-87 (torch, any device)."""
        w = weights.float()
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
        sw, order = w.sort(dim=-1, descending=True, stable=True)
        s_sorted = sw.cumsum(dim=-1) - sw
        return torch.empty_like(s_sorted).scatter_(-1, order, s_sorted)

    @staticmethod
    def unimportance_one(weights: list) -> list:
        """policy.py:89-98 (pure Python, one token)."""
        total = sum(weights) or 1e-12
        s = [0.0] * len(weights)
        acc = 0.0
        for j in sorted(range(len(weights)), key=lambda j: -weights[j]):
            s[j] = acc
            acc += weights[j] / total
        return s

    def levels(self, layer: int, weights: torch.Tensor):
        """policy.py:110-123 -> (level (T,k) int8, skip (T,k) bool)."""
        T, k = weights.shape
        none = torch.zeros(T, k, dtype=torch.bool)
        fixed = self._fixed(layer)
        if fixed is not None:
            return torch.full((T, k), fixed, dtype=torch.int8), none
        if self.mode == "weight":  # level 0 when the expert's own weight reaches t1 (no skip)
            w = weights.cpu().float()
            return torch.where(w >= self.t1, 0, 2).to(torch.int8), none
        s = self.unimportance(weights.cpu())
        lvl = torch.full((T, k), 2, dtype=torch.int8)
        if self.t_mid is not None:
            lvl[s <= self.t_mid + 1e-6] = 1
        lvl[s <= self.t1_for(layer) + 1e-6] = 0
        skip = (s > self.t2 + 1e-6) & (lvl != 0) if self.t2 is not None else none
        return lvl, skip

    def levels_one(self, layer: int, weights: list):
        """policy.py:125-137 -> (levels, skip, s) for one token."""
        k = len(weights)
        fixed = self._fixed(layer)
        if fixed is not None:
            return [fixed] * k, [False] * k, [0.0] * k
        if self.mode == "weight":
            f32 = lambda v: float(torch.tensor(v, dtype=torch.float32))  # noqa: E731
            return [0 if f32(w) >= f32(self.t1) else 2 for w in weights], [False] * k, [0.0] * k
        s = self.unimportance_one(weights)
        t1 = self.t1_for(layer) + 1e-6
        tm = None if self.t_mid is None else self.t_mid + 1e-6
        lvl = [0 if v <= t1 else (1 if tm is not None and v <= tm else 2) for v in s]
        if self.t2 is None:
            return lvl, [False] * k, s
        return lvl, [v > self.t2 + 1e-6 and lv != 0 for v, lv in zip(s, lvl)], s

    def expert_level(self, token_levels: torch.Tensor) -> int:
        """policy.py:148-154 (T > 1 vote)."""
        n = token_levels.numel()
        for level in (0, 1):
            if (token_levels <= level).sum().item() >= (self.hi_vote - 1e-9) * n:
                return level
        return 2

    @property
    def allow_upgrade(self) -> bool:
        """policy.py:176-185."""
        return self.upgrade and self.mode != "lo"

    def device_policy(self, layer: int, one_token: bool = False) -> Policy:
        """Parameters of the decision kernels for `layer`. one_token=True selects, for the
        one-token kernels, the float64 rule of `levels_one` (moelab's default decode path,
        runtime.py:494-517); otherwise the tensor rule of `levels` / `gpu_levels` (the T > 1 path
        and the whole-token graph, fullgraph.py:101-114). Both threshold forms are packed."""
        mode = {"hobbit": 0, "hi": 1, "lo": 2, "weight": 3}[self.mode]
        f32 = lambda v: float(torch.tensor(v, dtype=torch.float32))  # noqa: E731
        prot = 1 if layer in self.protect_layers else 0
        upg = 1 if self.allow_upgrade else 0
        # the cache-miss rule (runtime.py:600-615) belongs to the one-token path only
        e3 = 1 if one_token and self.miss_t1 is not None else 0
        mt = self.miss_t1 + 1e-6 if e3 else 0.0
        if self.mode == "weight":
            return Policy(mode=mode, t1=f32(self.t1), t_mid=-1.0, t2=-1.0, protect=prot, upgrade=upg,
                          f64=1 if e3 else 0, e3=e3, t1_64=-1.0, t_mid_64=-1.0, t2_64=-1.0, miss_t1_64=mt)
        t1 = self.t1_for(layer) + 1e-6
        tm = None if self.t_mid is None else self.t_mid + 1e-6
        t2 = None if self.t2 is None else self.t2 + 1e-6
        return Policy(mode=mode, t1=f32(t1), t_mid=-1.0 if tm is None else f32(tm), t2=-1.0 if t2 is None else f32(t2),
                      protect=prot, upgrade=upg, f64=1 if one_token else 0, e3=e3, t1_64=t1,
                      t_mid_64=-1.0 if tm is None else tm, t2_64=-1.0 if t2 is None else t2, miss_t1_64=mt)


def level_to_precision(level: int, precisions: list) -> str:
    """policy.py:188-192."""
    if len(precisions) >= 3:
        return precisions[min(level, len(precisions) - 1)]
    return precisions[0] if level == 0 else precisions[-1]
