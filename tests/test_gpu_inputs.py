"""
GPU parity for input classes the other files leave out: the float64 one-token HOBBIT rule next to
the tensor rule at a threshold, the Qwen3-30B decode shape in the fused kernel (I = 768: 24
chunks per down row), records quantised with moelab's store default (mse scales, some of them
negative) through every expert-product path, and the offloaded decoder at the Qwen3-Next shape.
Bars as in test_gpu_parity.py (indices and levels exact, outputs within max-abs 2e-2 and
mean-rel 1e-3 in fp16 / bf16).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from moelab_hip import _lib
from moelab_hip import kernels as K
from moelab_hip.layer import MoEDecoder, ResidentStore
from moelab_hip.offload import OffloadDecoder
from moelab_hip.policy import PrecisionPolicy
from moelab_hip.prefill import GroupedLayer
from moelab_hip.store import record_layout, views
from test_gpu_parity import NPDT, _Stack, assert_layer_close

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------------------
# HOBBIT: tensor rule (gpu_levels) and float64 one-token rule (levels_one) at a threshold
# ---------------------------------------------------------------------------------------
T1_EDGE = 0.5 - 1e-6 - 1e-9  # fp32(t1 + 1e-6) == 0.5 but t1 + 1e-6 < 0.5 in float64
W_EDGE = [0.5, 0.25, 0.25]   # s = [0, 0.5, 0.75] exactly in both rules


@pytest.mark.parametrize("one_token", [False, True])
def test_decide_table_levels_rule_at_threshold(dev, one_token):
    k, E, P = 3, 8, 2
    pol = PrecisionPolicy("hobbit", t1=T1_EDGE, upgrade=False)
    ref = O.Policy("hobbit", t1=T1_EDGE)
    w = np.array(W_EDGE, np.float32)
    exp = ref.levels_one(0, w)[0] if one_token else ref.levels(0, w[None])[0][0].tolist()
    assert exp == ([0, 2, 2] if one_token else [0, 0, 2])
    rtab = torch.full((P, E), 1 << 30, dtype=torch.int64, device=dev)
    offs = torch.zeros(P, 4, dtype=torch.int64, device=dev)
    planned = torch.ones(P, dtype=torch.int32, device=dev)
    lv2p = (ctypes.c_int * 3)(0, 1, 1)
    idx = torch.tensor([2, 5, 7], device=dev)
    wd = torch.from_numpy(w).to(dev)
    tab = torch.zeros(P, k, 4, dtype=torch.int64, device=dev)
    wtab = torch.zeros(P, k, device=dev)
    info = torch.zeros(3, k, device=dev)
    miss = torch.zeros(1, device=dev)
    _lib.call("moehip_decide_table", idx.data_ptr(), wd.data_ptr(), k, ctypes.byref(pol.device_policy(0, one_token)),
              lv2p, rtab.data_ptr(), P, E, offs.data_ptr(), planned.data_ptr(), tab.data_ptr(), wtab.data_ptr(),
              info.data_ptr(), miss.data_ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    assert info[2].cpu().tolist() == [float(v) for v in exp]
    assert info[1].cpu().tolist() == [0.0 if v == 0 else 1.0 for v in exp]


@pytest.mark.parametrize("one_token", [False, True])
def test_fused_levels_rule_at_threshold(dev, one_token):
    """The fused kernel with external routing (fp16 + int4 records, upgrade off): the slot the two
    rules disagree on runs from the record its rule picks."""
    H, I, E, k = 512, 256, 8, 3
    S = _Stack(dev, H, I, E, 1, ["fp16", "int4"], 21)
    pol = PrecisionPolicy("hobbit", t1=T1_EDGE, upgrade=False)
    dec = MoEDecoder(S.store, k, pol, torch.float16, one_token_rule=one_token)
    x = torch.randn(1, H, generator=S.g).half()
    idx = torch.tensor([[2, 5, 7]])
    w = torch.tensor([W_EDGE], dtype=torch.float32)
    out = torch.zeros(1, H, dtype=torch.float16, device=dev)
    idx_d, w_d = idx.to(dev), w.to(dev)
    dec.layer(0, x.to(dev), out, idx=idx_d.view(-1), w32=w_d.view(-1))
    torch.cuda.synchronize()
    ref_pol = O.Policy("hobbit", t1=T1_EDGE)
    lvl = ref_pol.levels_one(0, W_EDGE)[0] if one_token else ref_pol.levels(0, w.numpy())[0][0].tolist()
    assert dec.info[0, 2].cpu().tolist() == [float(v) for v in lvl]
    prec_of = {int(e): O.level_to_precision(int(v), ["fp16", "int4"]) for e, v in zip(idx[0], lvl)}
    ref = O.moe_layer(x.float().numpy(), idx.numpy(), w.numpy(), lambda e: S.mats(0, e, prec_of[e]))
    assert_layer_close(out.float().cpu().numpy(), ref, torch.float16)
    dec.check_error()


# ---------------------------------------------------------------------------------------
# Qwen3-30B-A3B decode shape in the fused kernel
# ---------------------------------------------------------------------------------------
def test_fused_qwen3_30b_decode(dev):
    """d_model 2048, 128 experts, top-8 renormalised, d_ff 768 (24 chunks per int4 down row, padded
    to 32 lanes), int4 gs64, bf16, with the router, three tokens."""
    H, I, E, k = 2048, 768, 128, 8
    dtype = torch.bfloat16
    S = _Stack(dev, H, I, E, 1, ["int4"], 31, dtype=dtype)
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), dtype, router_weights=[S.Wr[0].to(dev)], renorm=True)
    for t in range(3):
        x = torch.randn(1, H, generator=S.g).to(dtype)
        out = torch.zeros(1, H, dtype=dtype, device=dev)
        print(f"qwen3-30b decode token {t}", flush=True)
        dec.layer(0, x.to(dev), out)
        assert _lib.last_decode_kernel() == "k_decode_xcd"
        torch.cuda.synchronize()
        lo, idx, w, ref = S.reference(0, x, k, True, O.Policy("lo"))
        assert dec.idx.cpu().numpy().tolist() == idx.tolist()
        assert np.allclose(dec.w32.cpu().numpy(), w, rtol=2.0 ** -7, atol=0)
        assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    assert dec.miss.item() == 0
    dec.check_error()


# ---------------------------------------------------------------------------------------
# mse-quantised records (moelab's int4 store default, store.py:84-85), negative scales included
# ---------------------------------------------------------------------------------------
def _planted(std, H, I, g):
    """gate_up (2I, H) and down (H, I) of N(0, std) weights with the known-answer group of
    moelab tests/test_requant.py:35-42 (8, 1, 2, 3, -4, zeros; scaled) planted in gate_up row 0 and
    down row 3: its mse scale is negative (the largest weight lands on -8)."""
    gu = (torch.randn(2 * I, H, generator=g) * std).numpy()
    dn = (torch.randn(H, I, generator=g) * std).numpy()
    grp = np.zeros(64, np.float32)
    grp[:5] = np.array([8.0, 1.0, 2.0, 3.0, -4.0], np.float32) / 16  # exact in fp16 with scale -1/16
    gu[0, :64] = grp
    dn[3, 64:128] = -grp
    return gu, dn


class _MseStore:
    """L x E int4 records quantised with mse scales by the oracle's encoder (the store builder's
    method), written into a ResidentStore; the float view of each record for the reference."""

    def __init__(self, dev, H, I, E, L, seed, std=0.05):
        self.lay = O.record_layout("int4", H, I, 64, scale="mse")
        self.store = ResidentStore({"int4": record_layout("int4", H, I, 64, scale="mse")}, L, E, dev)
        assert self.store.layouts["int4"]["record_bytes"] == self.lay["record_bytes"]
        g = torch.Generator().manual_seed(seed)
        self.mats, self.neg = {}, 0
        for l in range(L):
            for e in range(E):
                gu, dn = _planted(std, H, I, g)
                blob = O.encode_record(self.lay, gu, dn, method="mse")
                v = O.views(self.lay, blob)
                self.neg += int((v["gate_up.s"] < 0).sum() + (v["down.s"] < 0).sum())
                self.store.blob("int4", l, e).copy_(torch.from_numpy(blob))
                self.store.set_present("int4", l, e)
                self.mats[(l, e)] = O.materialize(self.lay, blob)
        g2 = torch.Generator().manual_seed(seed + 1)
        self.Wr = [(torch.randn(E, H, generator=g2) * 0.05) for _ in range(L)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mse_records_fused_kernel(dev, dtype):
    H, I, E, k, L = 512, 256, 16, 4, 2
    ms = _MseStore(dev, H, I, E, L, 41)
    assert ms.neg > 0
    Wr = [w.to(dtype) for w in ms.Wr]
    dec = MoEDecoder(ms.store, k, PrecisionPolicy("lo"), dtype, router_weights=[w.to(dev) for w in Wr])
    g = torch.Generator().manual_seed(42)
    for l in range(L):
        x = torch.randn(1, H, generator=g).to(dtype)
        out = torch.zeros(1, H, dtype=dtype, device=dev)
        print(f"mse fused {dtype} layer {l} (router)", flush=True)
        dec.layer(l, x.to(dev), out)
        torch.cuda.synchronize()
        _, idx, w, _ = O.router(x.float().numpy(), Wr[l].float().numpy(), k, False, NPDT[dtype])
        assert dec.idx.cpu().numpy().tolist() == idx.tolist()
        ref = O.moe_layer(x.float().numpy(), idx, w, lambda e: ms.mats[(l, e)])
        assert_layer_close(out.float().cpu().numpy(), ref, dtype)
        # external routing that includes the planted expert 0
        idx0 = torch.tensor([[0, 3, 9, 14]])
        w0 = torch.tensor([[0.4, 0.3, 0.2, 0.1]])
        out2 = torch.zeros(1, H, dtype=dtype, device=dev)
        i0, w0d = idx0.to(dev), w0.to(dev)
        dec.layer(l, x.to(dev), out2, idx=i0.view(-1), w32=w0d.view(-1))
        torch.cuda.synchronize()
        ref2 = O.moe_layer(x.float().numpy(), idx0.numpy(), w0.numpy(), lambda e: ms.mats[(l, e)])
        assert_layer_close(out2.float().cpu().numpy(), ref2, dtype)
    dec.check_error()


def test_mse_records_grouped_ffn_int4(dev):
    H, I, E = 512, 256, 4
    ms = _MseStore(dev, H, I, E, 1, 43)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(44)).half()
    ws = [0.4, 0.3, 0.2, 0.1]
    entries = [(views(ms.store.layouts["int4"], ms.store.blob("int4", 0, e)), ws[e]) for e in range(E)]
    out = torch.full((1, H), 0.5, dtype=torch.float16, device=dev)
    K.grouped_ffn_int4(x.to(dev), entries, {"gate_up": 64, "down": 64}, out)
    torch.cuda.synchronize()
    ref = 0.5 + O.moe_layer(x.float().numpy(), np.arange(E)[None], np.array([ws]), lambda e: ms.mats[(0, e)])
    assert_layer_close(out.float().cpu().numpy(), ref, torch.float16)


@pytest.mark.parametrize("path,T", [("gemv", 8), ("mfma", 96)])
def test_mse_records_grouped_layer(dev, path, T):
    """The batched GEMV (few tokens per expert) and the MFMA grouped GEMM on mse records; every
    token routes to the planted expert 0 in slot 0."""
    H, I, E, k = 512, 256, 8, 3
    ms = _MseStore(dev, H, I, E, 1, 45)
    gl = GroupedLayer(ms.store, k, T, PrecisionPolicy("lo"), torch.bfloat16, gemv_tokens=64 if path == "gemv" else 0)
    g = torch.Generator().manual_seed(46)
    idx = torch.stack([torch.cat([torch.tensor([0]), torch.randperm(E - 1, generator=g)[:k - 1] + 1]) for _ in range(T)])
    w = (torch.rand(T, k, generator=g) + 0.05).float()
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    out = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    print(f"mse grouped layer {path} T={T}", flush=True)
    gl.layer(0, x.to(dev), out, idx.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = O.moe_layer(x.float().numpy(), idx.numpy(), w.numpy().astype(np.float64), lambda e: ms.mats[(0, e)])
    assert_layer_close(out.float().cpu().numpy(), ref, torch.bfloat16)
    assert gl.miss.item() == 0


# ---------------------------------------------------------------------------------------
# offloaded decode at the Qwen3-Next shape
# ---------------------------------------------------------------------------------------
def test_offload_decoder_qwen3next_shape(dev):
    """d_model 2048, 512 experts, top-10 renormalised, d_ff 512, bf16, int4 records in pinned host
    memory, a device budget of 25 records (one token touches 30 over the 3 layers): outputs
    bit-identical to the same fused kernel with every record resident."""
    H, I, E, L, k, T = 2048, 512, 512, 3, 10, 8
    dtype = torch.bfloat16
    lay = record_layout("int4", H, I, 64, scale="absmax")
    store = ResidentStore({"int4": lay}, L, E, dev)
    g = torch.Generator(device=dev).manual_seed(51)
    store.fill_synthetic(g, std=0.02)
    Wr = [(torch.randn(E, H, device=dev, generator=g) * 0.05).to(dtype) for _ in range(L)]
    rb = lay["record_bytes"]
    host = torch.empty(L * E * rb, dtype=torch.uint8).pin_memory()
    host.copy_(store.arena["int4"].cpu())

    def host_record(l, e, p):
        o = (l * E + e) * rb
        return host[o:o + rb]

    ref_dec = MoEDecoder(store, k, PrecisionPolicy("lo"), dtype, router_weights=Wr, renorm=True)
    off = OffloadDecoder({"int4": lay}, L, E, k, host_record, 25 * rb, dev, PrecisionPolicy("lo"), dtype,
                         router_weights=Wr, renorm=True)
    gx = torch.Generator().manual_seed(52)
    xs = torch.randn(T, L, 1, H, generator=gx).to(dtype)
    xs[5:] = xs[:3]  # repeated tokens: some experts are still resident
    xs = xs.to(dev)
    got = torch.zeros(T, L, 1, H, dtype=dtype, device=dev)
    ref = torch.zeros_like(got)
    print(f"offload qwen3-next shape: {T} tokens x {L} layers", flush=True)
    for t in range(T):
        for l in range(L):
            ref_dec.route(l, xs[t, l])
            ref_dec.layer(l, xs[t, l], ref[t, l], idx=ref_dec.idx, w32=ref_dec.w32)
            off.layer(l, xs[t, l], got[t, l])
        off.tick()
    torch.cuda.synchronize()
    assert off.dec.miss.item() == 0
    assert torch.equal(got, ref)
    assert off.cache.stats.evictions > 0 and off.cache.used <= off.cache.budget
    assert off.stats["misses"] > 0 and off.stats["hits"] > 0


# ---------------------------------------------------------------------------------------
# the shared expert's record choice with a two-precision store (one-token and T > 1 paths agree)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("path", ["gemv", "mfma", "fused"])
def test_shared_expert_only_less_precise_copy(dev, path):
    """Store [fp16, int4], HOBBIT with upgrade off, the shared expert's record present in int4
    only: every path runs the shared expert from that copy (its most precise present one) and
    counts no miss for it."""
    from test_gpu_batch import _store as batch_store
    H, I, E, k = 512, 256, 16, 4
    T = 1 if path == "fused" else 24
    dtype = torch.bfloat16
    precs = ["fp16", "int4"]
    st = batch_store(dev, precs, H, I, E, 61)
    lay4 = st.layouts["int4"]
    g = torch.Generator().manual_seed(62)
    gu_s, dn_s = torch.randn(2 * I, H, generator=g) * 0.02, torch.randn(H, I, generator=g) * 0.02
    sh_blob = torch.zeros(lay4["record_bytes"], dtype=torch.uint8, device=dev)
    from moelab_hip.store import encode_record_
    encode_record_(lay4, sh_blob, gu_s.to(dev), dn_s.to(dev))
    gate = (torch.randn(H, generator=g) * 0.05).to(dtype)
    Wr = (torch.randn(E, H, generator=g) * 0.05).to(dtype)
    pol, opol = PrecisionPolicy("hobbit", t1=0.5, upgrade=False), O.Policy("hobbit", t1=0.5)
    shared = [{"gate": gate.to(dev), "rec": {"int4": sh_blob}}]
    x = torch.randn(T, H, generator=g).to(dtype)
    out = torch.zeros(T, H, dtype=dtype, device=dev)
    print(f"shared expert, int4 copy only, {path}", flush=True)
    if path == "fused":
        dec = MoEDecoder(st, k, pol, dtype, router_weights=[Wr.to(dev)], renorm=True, shared=shared)
        dec.layer(0, x.to(dev), out)
        torch.cuda.synchronize()
        idx_d, w_d = dec.idx.cpu().numpy(), dec.w32.cpu().numpy()
        miss = dec.miss.item()
    else:
        gl = GroupedLayer(st, k, T, pol, dtype, router_weights=[Wr.to(dev)], renorm=True, shared=shared,
                          gemv_tokens=64 if path == "gemv" else 0)
        gl.layer(0, x.to(dev), out)
        torch.cuda.synchronize()
        idx_d, w_d = gl.idx[:T].cpu().numpy(), gl.w32[:T].cpu().numpy()
        assert gl.info[0, E].item() == 1  # precision index of int4
        miss = gl.miss.item()
    assert miss == 0
    xf = x.float().numpy().astype(np.float64)
    if path == "fused":
        lvl = opol.levels(0, w_d)[0]
        prec_of = {int(e): precs[0] if int(v) == 0 else precs[1] for e, v in zip(idx_d[0], lvl[0])}
        ref = O.moe_layer(xf, idx_d, w_d.astype(np.float64),
                          lambda e: O.materialize(st.layouts[prec_of[e]], st.blob(prec_of[e], 0, e).cpu().numpy()))
    else:
        skip, decs = O.decide_general(opol, 0, idx_d, w_d, precs)
        ref = O.moe_layer(xf, idx_d, w_d.astype(np.float64),
                          lambda e: O.materialize(st.layouts[decs[e][1]], st.blob(decs[e][1], 0, e).cpu().numpy()),
                          skip=skip)
    logit = O.round_to((xf @ gate.float().numpy().astype(np.float64)).astype(np.float32), "bfloat16")
    gs = O.round_to((1.0 / (1.0 + np.exp(-logit.astype(np.float64)))).astype(np.float32), "bfloat16")
    ref = ref + gs.astype(np.float64)[:, None] * O.expert_ffn(xf, *O.materialize(lay4, sh_blob.cpu().numpy()))
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)


# ---------------------------------------------------------------------------------------
# the fast paths behind moelab's layer signatures (adapters.py)
# ---------------------------------------------------------------------------------------
def _olmoe_block(dev, H, I, E, k, dtype, precs, seed):
    """A transformers OlmoeSparseMoeBlock (its router on the GPU, in `dtype`) and a ResidentStore
    holding its experts in every precision of `precs` (records built from the block's weights)."""
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeSparseMoeBlock

    torch.manual_seed(seed)
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k, norm_topk_prob=False)
    blk = OlmoeSparseMoeBlock(cfg)
    with torch.no_grad():
        blk.gate.weight.normal_(0, 0.05)
        blk.experts.gate_up_proj.normal_(0, 0.02)
        blk.experts.down_proj.normal_(0, 0.02)
    st = ResidentStore({p: record_layout(p, H, I, 64, scale="absmax") for p in precs}, 1, E, dev)
    for e in range(E):
        for p in precs:
            st.encode(p, 0, e, blk.experts.gate_up_proj[e].detach().to(dev), blk.experts.down_proj[e].detach().to(dev))
    return blk.to(dev, dtype), st


@pytest.mark.parametrize("T", [1, 5, 70])
def test_experts_module_signature(dev, T):
    """transformers' OLMoE MoE block with its `experts` module swapped for ResidentExperts (the call
    moelab's OffloadedExperts.forward receives, runtime.py:1108-1112): bf16 hidden states, the
    block's own router, fp16 + int4 records and HOBBIT t1 = 0.5 (upgrade off). T = 1 takes the
    decode kernel (float64 one-token rule), T = 5 the batched GEMVs, T = 70 the MFMA tiles (tensor
    rule, per-expert vote); each checked against the oracle on the float view of the records."""
    from moelab_hip.adapters import HipMoE, ResidentExperts

    H, I, E, k = 512, 256, 16, 4
    dtype = torch.bfloat16
    precs = ["fp16", "int4"]
    blk, st = _olmoe_block(dev, H, I, E, k, dtype, precs, 71)
    pol = PrecisionPolicy("hobbit", t1=0.5, upgrade=False)
    moe = HipMoE(st, k, pol, dtype, max_tokens=128)
    seen = {}
    blk.experts = ResidentExperts(moe, 0, blk.experts.act_fn, E)
    blk.experts.register_forward_pre_hook(lambda m, a: seen.__setitem__("args", tuple(t.clone() for t in a)))
    x = torch.randn(1, T, H, generator=torch.Generator().manual_seed(72)).to(dev, dtype)
    print(f"experts-module binding T={T}", flush=True)
    with torch.no_grad():
        got = blk(x)
    torch.cuda.synchronize()
    hs, idx, w = (t.cpu() for t in seen["args"])
    assert got.shape == x.shape and got.dtype == dtype
    w32 = w.float().numpy()
    opol = O.Policy("hobbit", t1=0.5)
    mats = lambda p, e: O.materialize(st.layouts[p], st.blob(p, 0, e).cpu().numpy())  # noqa: E731
    xf = hs.float().numpy()
    if T == 1:
        lvl = opol.levels_one(0, w32[0])[0]
        prec_of = {int(e): precs[0] if v == 0 else precs[1] for e, v in zip(idx[0].tolist(), lvl)}
        ref = O.moe_layer(xf, idx.numpy(), w32.astype(np.float64), lambda e: mats(prec_of[e], e))
    else:
        skip, decs = O.decide_general(opol, 0, idx.numpy(), w32, precs)
        ref = O.moe_layer(xf, idx.numpy(), w32.astype(np.float64), lambda e: mats(decs[e][1], e), skip=skip)
    assert_layer_close(got.reshape(T, H).float().cpu().numpy(), ref, dtype)
    assert moe.miss == 0


def test_run_layer_refuses_other_activations(dev):
    from moelab_hip.adapters import HipMoE

    st = ResidentStore({"int4": record_layout("int4", 512, 256, 64, scale="absmax")}, 1, 8, dev)
    moe = HipMoE(st, 2, dtype=torch.float16, max_tokens=8)
    x = torch.zeros(1, 512, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="silu"):
        moe.run_layer(0, x, torch.zeros(1, 2, dtype=torch.int64, device=dev), torch.zeros(1, 2, device=dev),
                      torch.nn.GELU())


@pytest.mark.parametrize("graph", [False, True])
def test_fullmoe_layer_signature(dev, graph):
    """FullMoE.layer(layer, x, idx, w, call) (fullgraph.py:149-188) on FullMoEHip: eagerly, and
    captured in a HIP graph with `call` launching inside the capture, replayed on new routing;
    readout() = [missing] + info, HOBBIT by the tensor rule."""
    from moelab_hip.adapters import FullMoEHip

    H, I, E, k, L = 512, 256, 16, 4, 2
    dtype = torch.float16
    S = _Stack(dev, H, I, E, L, ["fp16", "int4"], 81)
    x = torch.zeros(1, H, dtype=dtype, device=dev)
    idx = torch.zeros(1, k, dtype=torch.int64, device=dev)
    w = torch.zeros(1, k, dtype=dtype, device=dev)
    fm = FullMoEHip(S.store, k, x, PrecisionPolicy("hobbit", t1=0.6, upgrade=False))
    outs = []

    def token():
        outs.clear()
        for l in range(L):
            outs.append(fm.layer(l, x, idx, w, lambda fn: fn()))

    g = None
    if graph:
        token()  # eager warm-up, then capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            token()
    rng = np.random.default_rng(82)
    for step in range(3):
        xi = torch.randn(1, H, generator=S.g).to(dtype)
        ii = torch.from_numpy(rng.choice(E, k, replace=False)).view(1, k)
        wi = torch.from_numpy(rng.random((1, k)).astype(np.float32)).to(dtype)
        x.copy_(xi.to(dev))
        idx.copy_(ii.to(dev))
        w.copy_(wi.to(dev))
        print(f"fullmoe binding graph={graph} step {step}", flush=True)
        if graph:
            g.replay()
        else:
            token()
        torch.cuda.synchronize()
        ro = fm.readout()
        assert ro[0] == 0.0
        info = np.array(ro[1:]).reshape(L, 3, k)
        w32 = wi.float().numpy()
        lvl = O.Policy("hobbit", t1=0.6).levels(0, w32)[0][0]
        for l in range(L):
            prec_of = {int(e): "fp16" if v == 0 else "int4" for e, v in zip(ii[0].tolist(), lvl)}
            ref = O.moe_layer(xi.float().numpy(), ii.numpy(), w32.astype(np.float64),
                              lambda e: S.mats(l, e, prec_of[e]))
            assert_layer_close(outs[l].float().cpu().numpy(), ref, dtype)
            assert info[l, 0].tolist() == ii[0].float().tolist() and info[l, 2].tolist() == lvl.astype(float).tolist()


def test_grouped_graph_fp32_records(dev):
    """GroupedGraph on fp32 records (outside the one-launch kernel): kernels A and B per precision
    from the same request block, replayed."""
    H, I, k = 256, 128, 3
    from test_gpu_parity import make_records, to_dev
    lay32, b32, m32 = make_records("fp32", H, I, 5, 91)
    r32 = to_dev(b32, dev)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(92)).to(dev)
    out = torch.zeros(1, H, device=dev)
    gg = K.GroupedGraph({"fp32": lay32}, x, out, k)
    assert not gg.fused
    rng = np.random.default_rng(93)
    for step in range(4):
        e = rng.choice(5, k, replace=False)
        wv = rng.random(k).astype(np.float32)
        gg.run({"fp32": [(r32[i], float(v)) for i, v in zip(e, wv)]})
        torch.cuda.synchronize()
        ref = O.moe_layer(x.cpu().numpy(), np.array([list(e)]), np.array([wv]), lambda i: m32[i])
        assert np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max() < 1e-4
    assert gg.replays == 3


# ---------------------------------------------------------------------------------------
# an expired bounded wait, forced from the host: NaN output and the error flag, every workgroup
# exits, and the next launch on the same workspace is exact again
# ---------------------------------------------------------------------------------------
XC_TEST_WORD, ERR_WORD = 576, 512  # header words of the decode-layer workspace (uint32 index)

# (record precisions, grid, the kernel that runs): the XCD kernel, the one-item kernel (a grid at
# least the layer's item count), the item loop (a smaller grid), and the item loop on two record
# precisions (mixed launches never run the XCD kernel)
FORCED = {"xcd": (["int4"], 0, "k_decode_xcd"), "one_item": (["int4"], 1 << 20, "k_decode_tok"),
          "item_loop": (["int4"], 64, "k_decode_layer"), "two_precisions": (["fp16", "int4"], 0, "k_decode_layer")}


@pytest.mark.parametrize("kernel", list(FORCED))
def test_forced_expired_wait_poisons_output_and_sets_the_flag(dev, kernel):
    precs, grid, name = FORCED[kernel]
    H, I, E, k = 2048, 1024, 64, 8
    S = _Stack(dev, H, I, E, 1, precs, 31)
    pol = PrecisionPolicy("hobbit", t1=0.5, upgrade=False) if len(precs) > 1 else PrecisionPolicy("lo")
    dec = MoEDecoder(S.store, k, pol, torch.float16, router_weights=[S.Wr[0].to(dev)], grid=grid)
    assert dec.fused
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(5)).half().to(dev)
    ref = torch.zeros(1, H, dtype=torch.float16, device=dev)
    dec.layer(0, x, ref)
    assert _lib.last_decode_kernel() == name
    torch.cuda.synchronize()
    dec.check_error()
    words = dec.ws.view(torch.int32)
    print(f"forced expiry ({name}): test word set", flush=True)
    words[XC_TEST_WORD] = 1
    out = torch.zeros(1, H, dtype=torch.float16, device=dev)
    dec.layer(0, x, out)
    assert _lib.last_decode_kernel() == name
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    with pytest.raises(RuntimeError, match="bounded wait expired"):
        dec.check_error()
    print(f"forced expiry ({name}): cleared, normal launch", flush=True)
    words[XC_TEST_WORD] = 0
    words[ERR_WORD] = 0
    out2 = torch.zeros(1, H, dtype=torch.float16, device=dev)
    for _ in range(2):
        dec.layer(0, x, out2)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref)
    dec.check_error()
