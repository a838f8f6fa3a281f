"""
GPU parity of the T > 1 path (prefill chunks, batched decode): moehip_dispatch + the MFMA grouped
GEMM against the oracle's expert-by-expert layer (oracle.moe_layer_grouped, pinned against
transformers' OlmoeExperts in test_oracle.py), within the north-star tolerance.
"""

import numpy as np
import pytest
import torch

import oracle as O
from moelab_hip import _lib
from moelab_hip.layer import ResidentStore
from moelab_hip.prefill import GroupedTokens
from moelab_hip.store import record_layout
from test_gpu_parity import assert_layer_close

pytestmark = pytest.mark.gpu


class _Experts:
    """E int4 experts of N(0, std) weights (each regenerated from its own seed), encoded on the
    GPU, with the oracle's float view built on demand."""

    def __init__(self, dev, H, I, E, seed, std=0.02):
        self.H, self.I, self.E, self.seed, self.std = H, I, E, seed, std
        self.store = ResidentStore({"int4": record_layout("int4", H, I, 64, scale="absmax")}, 1, E, dev)
        for e in range(E):
            gu, dn = self.weights(e)
            self.store.encode("int4", 0, e, gu.to(dev), dn.to(dev))
        self._mats = {}

    def weights(self, e):
        g = torch.Generator().manual_seed(self.seed * 7919 + e)
        return (torch.randn(2 * self.I, self.H, generator=g) * self.std,
                torch.randn(self.H, self.I, generator=g) * self.std)

    def mats(self, e):
        if e not in self._mats:
            gu, dn = self.weights(e)
            lay = O.record_layout("int4", self.H, self.I, 64, scale="absmax")
            self._mats[e] = O.materialize(lay, O.encode_record(lay, gu.numpy(), dn.numpy(), "absmax"))
        return self._mats[e]

    def bases(self):
        return self.store.rtab[0, 0].clone()


def _routing(T, E, k, seed, renorm):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g) + 0.05
    if renorm:
        w = w / w.sum(1, keepdim=True)
    return idx, w.float()


def _run(dev, ex, x, idx, w, dtype, skip=None, missing=()):
    T, k = idx.shape
    gt = GroupedTokens(ex.store.layouts["int4"], ex.E, k, T, dev)
    bases = ex.bases()
    for e in missing:
        bases[e] = 0
    tab = gt.table(bases)
    xd, idxd, wd = x.to(dev).contiguous(), idx.to(dev).contiguous(), w.to(dev).contiguous()
    out = torch.zeros(T, ex.H, dtype=dtype, device=dev)
    sk = None if skip is None else torch.from_numpy(skip.astype(np.uint8)).to(dev)
    gt.run(xd, idxd, wd, tab, out, skip=sk)
    torch.cuda.synchronize()
    keep = np.zeros(idx.shape, bool) if skip is None else skip.copy()
    for e in missing:
        keep |= idx.numpy() == e
    ref = O.moe_layer_grouped(x.float().numpy(), idx.numpy(), w.numpy().astype(np.float64), ex.mats, skip=keep)
    return out.float().cpu().numpy(), ref


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_grouped_gemm_small(dev, dtype):
    H, I, E, k, T = 256, 128, 8, 2, 40
    ex = _Experts(dev, H, I, E, 1)
    idx, w = _routing(T, E, k, 2, False)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(dtype)
    got, ref = _run(dev, ex, x, idx, w, dtype)
    assert_layer_close(got, ref, dtype)


def test_grouped_gemm_many_tokens_per_expert_skip_and_missing(dev):
    """> 64 tokens per expert (several passes), skipped pairs and a non-resident expert."""
    H, I, E, k, T = 512, 256, 4, 2, 200
    dtype = torch.float16
    ex = _Experts(dev, H, I, E, 4)
    idx, w = _routing(T, E, k, 5, True)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(dtype)
    skip = np.zeros((T, k), bool)
    skip[::5, 0] = True
    got, ref = _run(dev, ex, x, idx, w, dtype, skip=skip, missing=(2,))
    assert_layer_close(got, ref, dtype)


def test_grouped_gemm_large_activations_bf16(dev):
    """bf16 activations far outside fp16's range: the per-token power-of-two scaling keeps them."""
    H, I, E, k, T = 256, 128, 4, 2, 24
    dtype = torch.bfloat16
    ex = _Experts(dev, H, I, E, 7)
    idx, w = _routing(T, E, k, 8, False)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9))
    x[::2] *= 3.0e5  # |x| ~ 1e6 on even tokens
    x[1::4] *= 1.0e-6
    x = x.to(dtype)
    got, ref = _run(dev, ex, x, idx, w, dtype)
    # relative to each token's largest output: bf16 output rounding alone is up to 2^-9 of it;
    # an overflow or a flush to zero of the huge or tiny rows would be ~1
    scale = np.abs(ref).max(axis=1, keepdims=True)
    err = np.abs(got - ref) / scale
    assert err.max() < 2.0 ** -7, err.max()
    assert np.isfinite(got).all() and (np.abs(got[1::4]).max(axis=1) > 0).all()


def test_grouped_gemm_qwen3_30b_prefill_shape(dev):
    """Qwen3-30B-A3B MoE layer: d_model 2048, 128 experts, top-8 renormalised, d_ff 768, a
    512-token bf16 prefill chunk."""
    H, I, E, k, T = 2048, 768, 128, 8, 512
    dtype = torch.bfloat16
    ex = _Experts(dev, H, I, E, 10)
    idx, w = _routing(T, E, k, 11, True)
    w = O.round_to(w.numpy(), "bfloat16").astype(np.float32)  # weights in the model dtype
    w = torch.from_numpy(w)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(12)).to(dtype)
    got, ref = _run(dev, ex, x, idx, w, dtype)
    assert_layer_close(got, ref, dtype)


def test_persistent_ffn_matches_the_separate_launches(dev, monkeypatch):
    """The persistent up + down kernel (MOEHIP_GEMM_FUSED: per-XCD tile queues, 16 x 16 x 32 MFMA
    tiles, fp16 h with a power of two per (pair, up tile), rescaled while staged) against the
    default separate up / h / down launches (32 x 32 x 16 tiles), on a Qwen3-30B-shaped layer
    with several passes for some experts and a missing expert: both within the oracle's bar, and
    within one bf16 rounding of the output of each other (the two tile shapes sum a row's
    products in different orders)."""
    H, I, E, k, T = 2048, 768, 32, 8, 320
    dtype = torch.bfloat16
    ex = _Experts(dev, H, I, E, 13)
    g = torch.Generator().manual_seed(14)
    # skewed routing: experts 0..3 get most tokens (several 64-token passes each)
    pref = torch.tensor([8.0] * 4 + [1.0] * (E - 4))
    idx = torch.stack([torch.multinomial(pref, k, replacement=False, generator=g) for _ in range(T)])
    w = torch.rand(T, k, generator=g).float() + 0.05
    x = torch.randn(T, H, generator=g).to(dtype)
    monkeypatch.setenv("MOEHIP_GEMM_FUSED", "1")
    fused, ref = _run(dev, ex, x, idx, w, dtype, missing=(5,))
    monkeypatch.delenv("MOEHIP_GEMM_FUSED")
    sep, _ = _run(dev, ex, x, idx, w, dtype, missing=(5,))
    assert_layer_close(fused, ref, dtype)
    assert_layer_close(sep, ref, dtype)
    scale = np.abs(ref).max(axis=1, keepdims=True)
    assert (np.abs(fused - sep) / scale).max() < 2.0 ** -7


@pytest.mark.parametrize("dtype,renorm", [(torch.bfloat16, True), (torch.float16, False)])
def test_prefill_layer_one_call_matches_route_then_run(dev, dtype, renorm):
    """moehip_prefill_layer (logits, one launch for top-k + expert buckets + fp16 copy of x,
    grouped GEMMs, combine) against moehip_router_topk + moehip_dispatch + moehip_grouped_gemm
    (GroupedTokens.route + run): the same routing bit for bit, the same output bit for bit (the
    pairs' order within an expert differs, the products and sums do not), repeatably (the routing
    counters are left at zero), for a full chunk and a shorter one in between; and the oracle's
    layer on that routing."""
    H, I, E, k, T = 2048, 768, 64, 8, 192
    ex = _Experts(dev, H, I, E, 21)
    gt = GroupedTokens(ex.store.layouts["int4"], E, k, T, dev)
    tab = gt.table(ex.bases())
    g = torch.Generator().manual_seed(22)
    Wr = (torch.randn(E, H, generator=g) * 0.05).to(dtype).to(dev)
    x = torch.randn(T, H, generator=g).to(dtype).to(dev)
    outs = []
    for T_ in (T, 37, T):
        out = torch.zeros(T_, H, dtype=dtype, device=dev)
        gt.layer(x[:T_].contiguous(), Wr, renorm, tab, out)
        torch.cuda.synchronize()
        if T_ == T:
            outs.append((out.clone(), [b.clone() for b in gt.route_out]))
    (o1, r1), (o2, r2) = outs
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)
    _, idx, _, w32 = (b.clone() for b in gt.route(x, Wr, renorm))
    for a, b in ((idx, r1[1]), (w32, r1[3])):
        assert torch.equal(a, b)
    ref_out = torch.zeros(T, H, dtype=dtype, device=dev)
    gt.run(x, idx, w32, tab, ref_out)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), ref_out.view(torch.int16))
    ref = O.moe_layer_grouped(x.float().cpu().numpy(), idx.cpu().numpy(), w32.cpu().numpy().astype(np.float64), ex.mats)
    assert_layer_close(o1.float().cpu().numpy(), ref, dtype)


def test_prefill_layer_refused_call_leaves_the_workspace_clean(dev):
    """A call refused for its record precision or group size launches nothing (the routing
    counters in the workspace stay zero): the next valid call on the same workspace equals a
    call on a fresh one, bit for bit."""
    H, I, E, k, T = 2048, 768, 64, 8, 64
    dtype = torch.bfloat16
    ex = _Experts(dev, H, I, E, 23)
    g = torch.Generator().manual_seed(24)
    Wr = (torch.randn(E, H, generator=g) * 0.05).to(dtype).to(dev)
    x = torch.randn(T, H, generator=g).to(dtype).to(dev)
    outs = []
    for refuse in (False, True):
        gt = GroupedTokens(ex.store.layouts["int4"], E, k, T, dev)
        tab = gt.table(ex.bases())
        out = torch.zeros(T, H, dtype=dtype, device=dev)
        if refuse:
            lib = _lib.load()
            logits, idx, w, w32 = gt.route(x, Wr, True)
            for prec, gs in ((_lib.prec_code("fp32"), 64), (_lib.prec_code("int4"), 32)):
                rc = lib.moehip_prefill_layer(prec, tab.data_ptr(), x.data_ptr(), Wr.data_ptr(), _lib.dt_code(dtype), T,
                                              H, I, k, E, gs, 1, logits.data_ptr(), idx.data_ptr(), w.data_ptr(),
                                              w32.data_ptr(), out.data_ptr(), None, 0, gt.ws_layer.data_ptr(),
                                              gt.ws_layer.numel(), _lib.stream_of(dev))
                assert rc == 1, lib.moehip_last_error()
            torch.cuda.synchronize()
            assert int(gt.ws_layer.count_nonzero()) == 0
        gt.layer(x, Wr, True, tab, out)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
