"""
GPU tests of the offloaded decoder over a two-precision store (fp16 + int4 records of every
expert in pinned host memory): which resident copy serves each routed expert must follow
moelab's one-token decode (runtime.py:587-615):

- the lookup takes a more precise resident copy only when `allow_upgrade` holds
  (policy.py:176-185: `upgrade` and a mode other than "lo"), else exactly the requested one;
- with `miss_t1` set (E3), a level-0 request that misses and whose unimportance s exceeds
  miss_t1 + 1e-6 is looked up again at level 1 and, still absent, staged at level 1.

The expected choice of every slot is restated here from those lines against the device cache's
content before each call; the kernel's own readout (chosen precision and level per slot) must
equal it, the host's hit and stage counts must equal the restatement's, no expert may be
missing, and the output must match the oracle's layer on the chosen records.
"""

import numpy as np
import pytest
import torch

import oracle as O
from moelab_hip.offload import OffloadDecoder
from moelab_hip.policy import PrecisionPolicy
from test_gpu_parity import _Stack, assert_layer_close

pytestmark = pytest.mark.gpu

PRECS = ["fp16", "int4"]


def _lookup(resident, layer, e, need, exact):
    """cache.py:134-154: the most precise resident copy at least as precise as `need` (exact:
    `need` only), or None."""
    have = {p for (l, x, p) in resident if l == layer and x == e}
    if exact:
        return need if need in have else None
    ok = [p for p in have if PRECS.index(p) <= PRECS.index(need)]
    return min(ok, key=PRECS.index) if ok else None


def _expected(pol, resident, layer, idx, w):
    """runtime.py:587-615 for one token: [(precision index used, level, hit)] per slot."""
    ref = O.Policy(pol.mode, t1=pol.t1, t2=pol.t2, t_mid=pol.t_mid)
    lv, skip, s = ref.levels_one(layer, np.asarray(w, np.float32))
    exact = not (pol.upgrade and pol.mode != "lo")
    out = []
    for j, e in enumerate(idx):
        if skip[j]:
            out.append((-2, lv[j], None))
            continue
        level = lv[j]
        need = O.level_to_precision(level, PRECS)
        got = _lookup(resident, layer, e, need, exact)
        if got is None and pol.miss_t1 is not None and level == 0 and s[j] > pol.miss_t1 + 1e-6:
            level, need = 1, O.level_to_precision(1, PRECS)
            got = _lookup(resident, layer, e, need, exact)
        out.append((PRECS.index(got or need), level, got is not None))
    return out


CASES = {
    # mode "lo" never upgrades: an fp16 copy already resident does not serve an int4 request
    "lo_fp16_resident": dict(mode="lo"),
    # hobbit with upgrades: resident fp16 copies serve int4 requests
    "hobbit_upgrade": dict(mode="hobbit", t1=0.6, upgrade=True),
    # hobbit without upgrades: only the requested precision serves
    "hobbit_exact": dict(mode="hobbit", t1=0.6, upgrade=False),
    # E3: level-0 misses with s > 0.2 drop to int4
    "hobbit_miss_t1": dict(mode="hobbit", t1=0.6, upgrade=True, miss_t1=0.2),
    "hobbit_miss_t1_exact": dict(mode="hobbit", t1=0.6, upgrade=False, miss_t1=0.2),
}


@pytest.mark.parametrize("case", list(CASES))
def test_offload_two_precision_store_follows_moelab_lookup(dev, case):
    H, I, E, L, k, T = 512, 256, 16, 2, 4, 10
    dtype = torch.float16
    S = _Stack(dev, H, I, E, L, PRECS, 31, std=0.05)
    host, rb = {}, {}
    for p in PRECS:
        rb[p] = S.store.layouts[p]["record_bytes"]
        host[p] = torch.empty(L * E * rb[p], dtype=torch.uint8).pin_memory()
        host[p].copy_(S.store.arena[p].cpu())

    def host_record(l, e, p):
        o = (l * E + e) * rb[p]
        return host[p][o:o + rb[p]]

    pol = PrecisionPolicy(**CASES[case])
    off = OffloadDecoder(S.store.layouts, L, E, k, host_record, 6 * rb["fp16"], dev, pol, dtype, mode="kernel")
    g = torch.Generator().manual_seed(77)
    # weights with s = [0, 0.5, 0.8, 0.95] in a token-dependent slot order: levels 0, 0, 2, 2 at t1 0.6
    base = torch.tensor([0.5, 0.3, 0.15, 0.05])
    xs = torch.randn(T, L, 1, H, generator=g).to(dtype)
    idx = torch.stack([torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(L)]) for _ in range(T)])
    idx[5:] = idx[torch.arange(5, T) % 4]  # repeated routings: records already resident serve them
    w = torch.stack([torch.stack([base[torch.randperm(k, generator=g)] for _ in range(L)]) for _ in range(T)])
    xs_d, idx_d, w_d = xs.to(dev), idx.to(dev), w.to(dev)
    hits = misses = 0
    upgraded = downgraded = beside = 0
    print(f"offload two-precision store, case {case}: {T} tokens x {L} layers", flush=True)
    for t in range(T):
        for l in range(L):
            # every other token, layer 0 prefetches fp16 copies of layer 1's experts (the next
            # token's routing of layer 1), so fp16 copies sit in the cache beside int4 requests
            predict = None
            if l == 0 and t % 2 == 0 and t + 1 < T:
                predict = {int(e): "fp16" for e in idx[t + 1, 1]}
            resident = set(off.cache.entries)
            exp = _expected(pol, resident, l, [int(e) for e in idx[t, l]], w[t, l].tolist())
            h0, m0 = off.stats["hits"], off.stats["misses"]
            out = torch.zeros(1, H, dtype=dtype, device=dev)
            off.layer(l, xs_d[t, l], out, idx=idx_d[t, l:l + 1], w32=w_d[t, l:l + 1], predict=predict)
            torch.cuda.synchronize()
            info = off.dec.info[l].cpu().numpy()
            assert info[1].tolist() == [float(c) for c, _, _ in exp], (t, l, info, exp)
            assert info[2].tolist() == [float(v) for _, v, _ in exp], (t, l, info, exp)
            n_hit = sum(1 for _, _, h in exp if h)
            assert off.stats["hits"] - h0 == n_hit
            assert off.stats["misses"] - m0 == len(exp) - n_hit
            hits += n_hit
            misses += len(exp) - n_hit
            lv_req = O.Policy(pol.mode, t1=pol.t1).levels_one(l, w[t, l].numpy())[0]
            upgraded += sum(1 for (c, _, h), r in zip(exp, lv_req) if h and c < PRECS.index(O.level_to_precision(r, PRECS)))
            downgraded += sum(1 for (_, v, _), r in zip(exp, lv_req) if v != r)
            chosen = {int(e): PRECS[c] for e, (c, _, _) in zip(idx[t, l], exp)}
            beside += sum(1 for e, p in chosen.items() if p == "int4" and (l, e, "fp16") in resident)
            ref = O.moe_layer(xs[t, l].float().numpy(), idx[t, l:l + 1].numpy(), w[t, l:l + 1].numpy(),
                              lambda e: S.mats(l, e, chosen[e]))
            assert_layer_close(out.float().cpu().numpy(), ref, dtype)
        off.tick()
    assert off.dec.miss.item() == 0
    off.dec.check_error()
    assert hits > 0 and misses > 0
    # the cases reach the branches they are named for
    if case == "lo_fp16_resident":  # int4 served while an fp16 copy of the expert was resident
        assert beside > 0 and upgraded == 0
    if case == "hobbit_upgrade":
        assert upgraded > 0
    if case == "hobbit_exact":
        assert beside > 0 and upgraded == 0
    if case.startswith("hobbit_miss_t1"):
        assert downgraded > 0 and off.stats["miss_downgrades"] >= downgraded
