"""
GPU parity of the T > 1 layer over a ResidentStore (GroupedLayer: per-token levels, dispatch,
per-expert precision vote, grouped GEMMs for every record precision, the shared expert, ordered
combine) against the oracle: the decision against oracle.decide_general (runtime.py:459-492),
the output against oracle.moe_layer on the float view of the very records the kernels read,
within the north-star tolerance.
"""

import numpy as np
import pytest
import torch

import oracle as O
from moelab_hip.layer import ResidentStore
from moelab_hip.policy import PrecisionPolicy
from moelab_hip.prefill import GroupedLayer
from moelab_hip.store import encode_record_, record_layout
from test_gpu_parity import assert_layer_close

pytestmark = pytest.mark.gpu


def _layout(prec, H, I):
    return record_layout(prec, H, I, 64, scale="absmax")


def _store(dev, precs, H, I, E, seed, L=1, std=0.02):
    st = ResidentStore({p: _layout(p, H, I) for p in precs}, L, E, dev)
    for l in range(L):
        for e in range(E):
            g = torch.Generator().manual_seed(seed * 7919 + l * 1009 + e)
            gu = (torch.randn(2 * I, H, generator=g) * std).to(dev)
            dn = (torch.randn(H, I, generator=g) * std).to(dev)
            for p in precs:
                st.encode(p, l, e, gu, dn)
    return st


def _mats(st, p, l, e):
    """The oracle's float view of the record the kernels read."""
    return O.materialize(st.layouts[p], st.blob(p, l, e).cpu().numpy())


def _routing(T, E, k, seed, renorm=False):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g) + 0.02
    if renorm:
        w = w / w.sum(1, keepdim=True)
    return idx, w.float()


# GEMV: batched dequant GEMVs (the path for few tokens per expert); MFMA: the grouped GEMM tiles
PATHS = {"gemv": 64, "mfma": 0}


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("prec", ["int4", "int8", "fp8", "fp16", "bf16"])
def test_grouped_layer_each_record_precision(dev, prec, dtype, path):
    """One record precision (T = 24 tokens, top-2 of 8: ~6 tokens per expert, more than one
    4-token pass of the GEMV path)."""
    H, I, E, k, T = 512, 256, 8, 2, 24
    st = _store(dev, [prec], H, I, E, 1)
    gl = GroupedLayer(st, k, T, PrecisionPolicy("hi"), dtype, gemv_tokens=PATHS[path])
    idx, w = _routing(T, E, k, 2)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(dtype)
    out = torch.zeros(T, H, dtype=dtype, device=dev)
    print(f"grouped layer {prec} {dtype} {path}", flush=True)
    gl.layer(0, x.to(dev), out, idx.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = O.moe_layer(x.float().numpy(), idx.numpy(), w.numpy().astype(np.float64), lambda e: _mats(st, prec, 0, e))
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    info = gl.info[0].cpu().numpy()
    used = set(idx.numpy().reshape(-1).tolist())
    assert all(info[e] == (0 if e in used else -2) for e in range(E))
    assert gl.miss.item() == 0


@pytest.mark.parametrize("fused_decide", [True, False])
@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("mode", ["weight", "hobbit"])
def test_grouped_layer_mixed_precision_vote(dev, mode, path, fused_decide):
    """OLMoE-shaped batched decode, 8 tokens, fp16 + int4 records: the per-token rule (weight
    threshold at the median routed weight, or HOBBIT t1 = 0.6 with t2 = 0.8, which always skips
    each token's last expert), the vote per expert (hi_vote 0.5), and each expert's tokens computed
    at its voted precision."""
    H, I, E, k, T = 2048, 1024, 64, 8, 8
    dtype = torch.float16
    precs = ["fp16", "int4"]
    st = _store(dev, precs, H, I, E, 4)
    Wr = (torch.randn(E, H, generator=torch.Generator().manual_seed(5)) * 0.02).to(dtype)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(dtype)
    logits, idx, w, _ = O.router(x.float().numpy(), Wr.float().numpy(), k, False, "float16")
    if mode == "weight":
        t1 = float(np.median(w))
        pol, opol = PrecisionPolicy("weight", t1=t1, upgrade=False), O.Policy("weight", t1=t1)
    else:
        pol, opol = PrecisionPolicy("hobbit", t1=0.6, t2=0.8, upgrade=False), O.Policy("hobbit", t1=0.6, t2=0.8)
    gl = GroupedLayer(st, k, T, pol, dtype, router_weights=[Wr.to(dev)], gemv_tokens=PATHS[path],
                      fused_decide=fused_decide)
    out = torch.zeros(T, H, dtype=dtype, device=dev)
    print(f"mixed vote {mode} {path}", flush=True)
    gl.layer(0, x.to(dev), out)
    torch.cuda.synchronize()
    idx_d = gl.idx[:T].cpu().numpy()
    clear = O.topk_margin(logits, k) > 0
    assert (idx_d[clear] == idx[clear]).all()
    w_d = gl.w32[:T].cpu().numpy()
    assert np.allclose(w_d[clear], w[clear], rtol=2.0 ** -10, atol=0)
    skip, dec = O.decide_general(opol, 0, idx_d, w_d, precs)
    info = gl.info[0].cpu().numpy()
    for e in range(E):
        want = precs.index(dec[e][1]) if e in dec else -2
        assert info[e] == want, (e, info[e], want)
    assert {p for _, p in dec.values()} == set(precs), "both record kinds should run"
    ref = O.moe_layer(x.float().numpy(), idx_d, w_d.astype(np.float64), lambda e: _mats(st, dec[e][1], 0, e), skip=skip)
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    assert skip.any() == (mode == "hobbit")


@pytest.mark.parametrize("fused_decide", [True, False])
@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("prec", ["int4", "fp8"])
def test_grouped_layer_qwen3next_shared_expert(dev, prec, path, fused_decide):
    """Qwen3-Next-shaped batched decode, 32 tokens: routed top-10 of 512 (renormalised) plus the
    sigmoid-gated shared expert, bf16; gate logit and sigmoid rounded to bf16 as the module does
    (modeling_qwen3_next.py:786-797)."""
    H, I, E, k, T = 2048, 512, 512, 10, 32
    dtype = torch.bfloat16
    st = _store(dev, [prec], H, I, E, 8)
    lay = st.layouts[prec]
    g = torch.Generator().manual_seed(9)
    gu_s, dn_s = torch.randn(2 * I, H, generator=g) * 0.02, torch.randn(H, I, generator=g) * 0.02
    sh_blob = torch.zeros(lay["record_bytes"], dtype=torch.uint8, device=dev)
    encode_record_(lay, sh_blob, gu_s.to(dev), dn_s.to(dev))
    gate = (torch.randn(H, generator=g) * 0.05).to(dtype)
    Wr = (torch.randn(E, H, generator=g) * 0.02).to(dtype)
    gl = GroupedLayer(st, k, T, PrecisionPolicy("hi"), dtype, router_weights=[Wr.to(dev)], renorm=True,
                      shared=[{"gate": gate.to(dev), "rec": {prec: sh_blob}}], gemv_tokens=PATHS[path],
                      fused_decide=fused_decide)
    x = torch.randn(T, H, generator=g).to(dtype)
    out = torch.zeros(T, H, dtype=dtype, device=dev)
    print(f"shared expert batch {prec} {path}", flush=True)
    gl.layer(0, x.to(dev), out)
    torch.cuda.synchronize()
    logits, idx, w, _ = O.router(x.float().numpy(), Wr.float().numpy(), k, True, "bfloat16")
    clear = O.topk_margin(logits, k) > 0
    assert (gl.idx[:T].cpu().numpy()[clear] == idx[clear]).all()
    idx_d = gl.idx[:T].cpu().numpy()
    w_d = gl.w32[:T].cpu().numpy().astype(np.float64)
    xf = x.float().numpy().astype(np.float64)
    ref = O.moe_layer(xf, idx_d, w_d, lambda e: _mats(st, prec, 0, e))
    logit = O.round_to((xf @ gate.float().numpy().astype(np.float64)).astype(np.float32), "bfloat16")
    gs = O.round_to((1.0 / (1.0 + np.exp(-logit.astype(np.float64)))).astype(np.float32), "bfloat16")
    ref = ref + gs.astype(np.float64)[:, None] * O.expert_ffn(xf, *O.materialize(lay, sh_blob.cpu().numpy()))
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    assert gl.info[0, E].item() == 0 and gl.miss.item() == 0


def test_grouped_layer_missing_copy_and_graph(dev):
    """An expert whose voted precision has no resident copy contributes nothing and counts its
    pairs in miss (upgrade off); the layer captured in a HIP graph replays to the eager result."""
    H, I, E, k, T = 512, 256, 8, 2, 16
    dtype = torch.float16
    precs = ["fp16", "int4"]
    st = _store(dev, precs, H, I, E, 11)
    st.set_present("fp16", 0, 3, False)
    st.set_present("int4", 0, 3, False)
    gl = GroupedLayer(st, k, T, PrecisionPolicy("lo", upgrade=False), dtype)
    idx, w = _routing(T, E, k, 12)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(13)).to(dtype)
    xd, idxd, wd = x.to(dev), idx.to(dev), w.to(dev)
    out = torch.zeros(T, H, dtype=dtype, device=dev)
    gl.layer(0, xd, out, idxd, wd)
    torch.cuda.synchronize()
    n3 = int((idx.numpy() == 3).sum())
    assert n3 > 0 and gl.miss.item() == n3 and gl.info[0, 3].item() == -1
    ref = O.moe_layer(x.float().numpy(), idx.numpy(), w.numpy().astype(np.float64),
                      lambda e: _mats(st, "int4", 0, e), skip=idx.numpy() == 3)
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    out2 = torch.zeros_like(out)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gl.layer(0, xd, out2, idxd, wd)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        gl.layer(0, xd, out2, idxd, wd)
    for r in range(3):
        out2.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, eager), r


@pytest.mark.parametrize("T", [16, 40])
def test_grouped_layer_routed_graph_replays(dev, T):
    """The router-to-work-list launch (moehip_batch_route_decide; above 16 tokens moehip_route_tokens
    + moehip_batch_decide with the work list) and the GEMVs captured in a HIP graph: every replay
    equals the eager layer, and the eager layer equals the unfused steps."""
    H, I, E, k = 2048, 512, 512, 10
    dtype = torch.bfloat16
    st = _store(dev, ["int4"], H, I, E, 14)
    lay = st.layouts["int4"]
    g = torch.Generator().manual_seed(15)
    sh_blob = torch.zeros(lay["record_bytes"], dtype=torch.uint8, device=dev)
    encode_record_(lay, sh_blob, (torch.randn(2 * I, H, generator=g) * 0.02).to(dev),
                   (torch.randn(H, I, generator=g) * 0.02).to(dev))
    gate = (torch.randn(H, generator=g) * 0.05).to(dtype).to(dev)
    Wr = (torch.randn(E, H, generator=g) * 0.02).to(dtype).to(dev)
    shared = [{"gate": gate, "rec": {"int4": sh_blob}}]
    x = torch.randn(T, H, generator=g).to(dtype).to(dev)
    fused = GroupedLayer(st, k, T, PrecisionPolicy("hi"), dtype, router_weights=[Wr], renorm=True, shared=shared)
    steps = GroupedLayer(st, k, T, PrecisionPolicy("hi"), dtype, router_weights=[Wr], renorm=True, shared=shared,
                         fused_decide=False)
    eager = torch.zeros(T, H, dtype=dtype, device=dev)
    ref = torch.zeros_like(eager)
    fused.layer(0, x, eager)
    steps.layer(0, x, ref)
    torch.cuda.synchronize()
    assert torch.equal(fused.idx[:T], steps.idx[:T]) and torch.equal(fused.w32[:T], steps.w32[:T])
    assert torch.equal(fused.info[0], steps.info[0])
    # the same products and combine order; the gate dot product may round differently by one ulp
    assert (eager.float() - ref.float()).abs().max().item() <= 2e-2
    out2 = torch.zeros_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused.layer(0, x, out2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fused.layer(0, x, out2)
    for r in range(3):
        out2.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, eager), r


@pytest.mark.parametrize("E,shared,T", [(64, False, 40), (512, True, 40), (800, False, 40), (1023, True, 40),
                                         (64, False, 8), (16, False, 4), (63, True, 6), (200, False, 128),
                                         (1023, True, 113), (1023, True, 120)])
@pytest.mark.parametrize("mode", ["hobbit", "weight"])
def test_batch_decide_matches_steps(dev, E, shared, T, mode):
    """moehip_batch_decide (one launch: levels, dispatch, vote from per-expert tallies, work list)
    against moehip_batch_levels + moehip_dispatch + moehip_batch_vote: every output bit-exact, up to
    1023 experts + the shared one (the largest LDS), with skipped pairs (HOBBIT t2) and experts
    without a resident copy (their pairs ranked -1 and counted in miss); the work list against the
    offsets. T * ks <= 64 pairs over at most 64 experts take the one-wave dispatch and work list; up
    to 1024 pairs the LDS counting sort (1024 and 1017 pairs here), beyond it the per-wave column
    dispatch (1080 pairs)."""
    import ctypes
    from moelab_hip import _lib
    k, P = 8, 2
    ks, EA = (k + 1, E + 1) if shared else (k, E)
    g = np.random.default_rng(E + (7 if shared else 0))
    idx = np.stack([g.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = (g.random((T, k)) ** 2 + 0.01).astype(np.float32)
    if shared:  # the shared expert (id E) as slot k with its own weight
        idx = np.concatenate([idx, np.full((T, 1), E, np.int64)], 1)
        w = np.concatenate([w, g.random((T, 1)).astype(np.float32)], 1)
    pol = PrecisionPolicy("hobbit", t1=0.5, t2=0.85) if mode == "hobbit" else PrecisionPolicy("weight", t1=0.3)
    cpol = pol.device_policy(0)
    resident = g.random((P, E)) < 0.8
    rtab = torch.from_numpy(np.where(resident, (np.arange(P * E).reshape(P, E) + 1) * 4096, 0).astype(np.int64)).to(dev)
    srec = (ctypes.c_int64 * P)(*[(1 << 40) + 4096 * p for p in range(P)])
    offs = torch.tensor([[0, 8, 16, 24], [0, 64, 128, 192]], dtype=torch.int64, device=dev)
    planned = torch.tensor([1, 1], dtype=torch.int32, device=dev)
    lv2p = (ctypes.c_int * 3)(0, 1, 1)
    idx_d, w_d = torch.from_numpy(idx).to(dev), torch.from_numpy(w).to(dev)
    st = _lib.stream_of(dev)

    def bufs():
        return dict(levels=torch.full((T * ks,), -7, dtype=torch.int32, device=dev),
                    skip=torch.full((T * ks,), 9, dtype=torch.uint8, device=dev),
                    counts=torch.full((EA,), -7, dtype=torch.int32, device=dev),
                    offsets=torch.full((EA + 1,), -7, dtype=torch.int32, device=dev),
                    sorted_pos=torch.full((T * ks,), -7, dtype=torch.int32, device=dev),
                    rank=torch.full((T * ks,), -7, dtype=torch.int32, device=dev),
                    tabs=torch.full((P, EA, 4), -7, dtype=torch.int64, device=dev),
                    info=torch.full((EA,), -7.0, device=dev), miss=torch.zeros(1, device=dev))

    a, b = bufs(), bufs()
    items = torch.full((P * (T * ks + 1),), -7, dtype=torch.int32, device=dev)
    print(f"batch decide E={E} shared={shared} {mode}", flush=True)
    _lib.call("moehip_batch_decide", w_d.data_ptr(), idx_d.data_ptr(), T, k, ks, ctypes.byref(cpol),
              a["levels"].data_ptr(), a["skip"].data_ptr(), E, 1 if shared else 0, a["counts"].data_ptr(),
              a["offsets"].data_ptr(), a["sorted_pos"].data_ptr(), a["rank"].data_ptr(), float(pol.hi_vote), lv2p,
              rtab.data_ptr(), srec, P, offs.data_ptr(), planned.data_ptr(), a["tabs"].data_ptr(),
              a["info"].data_ptr(), a["miss"].data_ptr(), items.data_ptr(), st)
    _lib.call("moehip_batch_levels", w_d.data_ptr(), T, k, ks, ctypes.byref(cpol), b["levels"].data_ptr(),
              b["skip"].data_ptr(), st)
    _lib.call("moehip_dispatch", idx_d.data_ptr(), b["skip"].data_ptr(), T, ks, EA, b["counts"].data_ptr(),
              b["offsets"].data_ptr(), b["sorted_pos"].data_ptr(), b["rank"].data_ptr(), st)
    _lib.call("moehip_batch_vote", b["levels"].data_ptr(), E, 1 if shared else 0, b["offsets"].data_ptr(),
              b["sorted_pos"].data_ptr(), float(pol.hi_vote), ctypes.byref(cpol), lv2p, rtab.data_ptr(), srec, P,
              offs.data_ptr(), planned.data_ptr(), b["tabs"].data_ptr(), b["rank"].data_ptr(), b["info"].data_ptr(),
              b["miss"].data_ptr(), st)
    torch.cuda.synchronize()
    for name in a:
        assert torch.equal(a[name], b[name]), name
    sk = a["skip"].cpu().numpy()
    big = T == 40
    if big:
        assert (sk == 1).any() == (mode == "hobbit")
        assert a["miss"].item() > 0  # some chosen experts have no copy
    off = a["offsets"].cpu().numpy()
    ch = a["info"].cpu().numpy()
    it = items.cpu().numpy().reshape(P, T * ks + 1)
    for p in range(P):  # one work list per record precision: the experts voted to it
        exp = [(e << 8) | z for e in range(EA) if ch[e] == p for z in range(off[e + 1] - off[e])]
        assert it[p, T * ks] == len(exp) and it[p, :len(exp)].tolist() == exp, p
    if big:
        assert (ch == 0).any() and (ch == 1).any()
