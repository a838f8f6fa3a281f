"""
GPU parity: every HIP entry point against the oracle on the same seeded inputs.

Bars (the reference's north-star bar): integer / byte / index work bit-exact; layer outputs in
fp16/bf16 within max-abs 2e-2 and mean-rel 1e-3 of the reference path's output in that dtype, where
mean-rel = mean|got - ref| / mean|ref| and the reference output is the exact (float64) result of the
dequantise-then-matmul path rounded once to the output dtype; fp32 activations within the
reference's own kernel-test bound (rel-err < 1e-4 of max|ref|, moelab tests/test_kernels.py:49-50).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from moelab_hip import _lib
from moelab_hip import kernels as K
from moelab_hip.layer import MoEDecoder, ResidentStore
from moelab_hip.store import unpack_int4_record, unpacked_layout
from moelab_hip.policy import PrecisionPolicy
from moelab_hip.store import encode_record_, record_layout, views

pytestmark = pytest.mark.gpu

NPDT = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def mean_rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30))


def assert_layer_close(got, ref, dtype):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if dtype == torch.float32:
        err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 1e-4, err
    else:
        ref_d = O.round_to(ref.astype(np.float32), NPDT[dtype]).astype(np.float64)
        assert np.abs(got - ref).max() <= 2e-2, np.abs(got - ref).max()
        assert mean_rel(got, ref_d) <= 1e-3, mean_rel(got, ref_d)


def make_records(prec, H, I, n, seed, std=0.1):
    g = torch.Generator().manual_seed(seed)
    lay = O.record_layout(prec, H, I, 64, scale="absmax")
    blobs, mats = [], []
    for _ in range(n):
        gu = (torch.randn(2 * I, H, generator=g) * std).numpy()
        dn = (torch.randn(H, I, generator=g) * std).numpy()
        b = O.encode_record(lay, gu, dn, method="absmax")
        blobs.append(b)
        mats.append(O.materialize(lay, b, "float32"))
    return lay, blobs, mats


def to_dev(blobs, dev):
    return [torch.from_numpy(b.copy()).to(dev) for b in blobs]


# ---------------------------------------------------------------------------------------
# store encoding (quantiser) — bit-exact
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("O_,I_,gs", [(256, 512, 64), (64, 96, 48), (33, 128, 32), (2048, 1024, 64)])
def test_quantize_bit_exact(dev, bits, O_, I_, gs):
    g = torch.Generator().manual_seed(O_ + I_ + bits)
    w = torch.randn(O_, I_, generator=g) * 0.02
    w[0, :gs] = 0.0  # zero group -> fp16(1e-7) scale
    w[1, :gs] = torch.arange(gs) - gs / 2  # exact halves: ties to even
    if O_ > 2:
        w[2, :gs] = torch.linspace(-1e-9, 1e-9, gs)  # tiny group: scale clamped at 1e-7
    q_ref, s_ref = O.quantize(w.numpy(), bits, gs)
    wd = w.to(dev)
    q = torch.empty(q_ref.shape, dtype=torch.uint8 if bits == 4 else torch.int8, device=dev)
    s = torch.empty(s_ref.shape, dtype=torch.float16, device=dev)
    _lib.call("moehip_quantize", wd.data_ptr(), O_, I_, bits, gs, q.data_ptr(), s.data_ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(q.cpu().numpy().view(np.uint8), q_ref.view(np.uint8))


def _mse_groups(O_, I_, gs, seed):
    """N(0, 0.02) weights with planted groups: all zero (fp16(1e-7) scale), exact halves (ties to
    even), tiny (the clamp), the largest magnitude on a negative weight (max / -8 > 0), two
    weights of equal magnitude and opposite signs (the first index wins the argmax), one positive
    outlier 30x the rest (a negative int4 scale, max / -8), and a row of duplicated groups (the
    same choice in every group)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(O_, I_, generator=g) * 0.02
    w[0, :gs] = 0.0
    w[1, :gs] = torch.arange(gs) - gs / 2
    w[2, :gs] = torch.linspace(-1e-9, 1e-9, gs)
    w[3, :gs] = torch.linspace(-0.9, 0.5, gs)
    w[4, :gs] = torch.randn(gs, generator=g) * 0.01
    w[4, 1], w[4, gs - 1] = 0.3, -0.3
    w[5, :gs] = torch.randn(gs, generator=g) * 0.01
    w[5, gs // 2] = 0.3
    w[6, :] = w[6, :gs].repeat(I_ // gs)
    return w


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("O_,I_,gs", [(64, 128, 64), (2048, 768, 64), (40, 96, 48), (16, 96, 32), (12, 60, 10),
                                      (12, 36, 6)])
def test_quantize_mse_bit_exact(dev, bits, O_, I_, gs):
    """moehip_quantize_mse against the oracle's mse restatement (quant.py:64-93): scales and
    packed values bit for bit, planted groups included, group sizes with and without a
    remainder below 8 (numpy's pairwise order for the error sums)."""
    print(f"quantize mse bits={bits} O={O_} I={I_} gs={gs}", flush=True)
    w = _mse_groups(O_, I_, gs, O_ + I_ + gs + bits)
    q_ref, s_ref = O.quantize(w.numpy(), bits, gs, "mse")
    if bits == 4:
        assert (s_ref.astype(np.float32) < 0).any()  # the negative scales are exercised
    wd = w.to(dev)
    q = torch.empty(q_ref.shape, dtype=torch.uint8 if bits == 4 else torch.int8, device=dev)
    s = torch.empty(s_ref.shape, dtype=torch.float16, device=dev)
    _lib.call("moehip_quantize_mse", wd.data_ptr(), O_, I_, bits, gs, q.data_ptr(), s.data_ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(q.cpu().numpy().view(np.uint8), q_ref.view(np.uint8))


@pytest.mark.parametrize("prec", ["int4", "int8"])
def test_encode_record_mse_bit_exact(dev, prec):
    """A record of an mse layout (the int4 store default) encoded on the GPU: the same bytes as
    the oracle's encoder (store.py:122-150 with scale="mse")."""
    H, I = 512, 256
    g = torch.Generator().manual_seed(8)
    gu, dn = torch.randn(2 * I, H, generator=g) * 0.05, torch.randn(H, I, generator=g) * 0.05
    lay = record_layout(prec, H, I, 64, scale="mse")
    blob = torch.empty(lay["record_bytes"], dtype=torch.uint8, device=dev)
    encode_record_(lay, blob, gu.to(dev), dn.to(dev))
    ref = O.encode_record(O.record_layout(prec, H, I, 64, scale="mse"), gu.numpy(), dn.numpy(), method="mse")
    assert np.array_equal(blob.cpu().numpy(), ref)


@pytest.mark.parametrize("prec", ["int4", "int8", "fp16", "bf16", "fp32", "fp8"])
def test_encode_record_bit_exact(dev, prec):
    H, I = 256, 128
    g = torch.Generator().manual_seed(7)
    gu, dn = torch.randn(2 * I, H, generator=g) * 0.05, torch.randn(H, I, generator=g) * 0.05
    lay = record_layout(prec, H, I, 64, scale="absmax")
    blob = torch.empty(lay["record_bytes"], dtype=torch.uint8, device=dev)
    encode_record_(lay, blob, gu.to(dev), dn.to(dev))
    ref = O.encode_record(O.record_layout(prec, H, I, 64, scale="absmax"), gu.numpy(), dn.numpy(), method="absmax")
    assert np.array_equal(blob.cpu().numpy(), ref)


# ---------------------------------------------------------------------------------------
# single-matrix GEMV
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("O_,I_", [(64, 128), (96, 192), (2048, 2048), (100, 96)])
def test_gemv_int4(dev, dtype, O_, I_):
    g = torch.Generator().manual_seed(O_ * I_)
    gs = O.pick_group_size(I_)
    w = torch.randn(O_, I_, generator=g)
    q, s = O.quantize(w.numpy(), 4, gs)
    x = torch.randn(I_, generator=g).to(dtype)
    ref = O.dequantize(q, s, 4, "float32").astype(np.float64) @ x.double().numpy()
    y = K.gemv_int4(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), x.to(dev), gs)
    assert y.dtype == dtype and y.shape == (O_,)
    got = y.float().cpu().numpy()
    tol = 1e-4 if dtype == torch.float32 else (2e-3 if dtype == torch.float16 else 1e-2)
    assert np.abs(got - ref).max() / np.abs(ref).max() < tol


# ---------------------------------------------------------------------------------------
# grouped kernels through the moelab.kernels API (the reference's kernel test shapes)
# ---------------------------------------------------------------------------------------
SHAPES = [(64, 32), (96, 48), (512, 256), (256, 128)]


@pytest.mark.parametrize("prec", ["int4", "int8", "fp16", "bf16", "fp32", "fp8"])
@pytest.mark.parametrize("H,I", SHAPES)
def test_grouped_ffn_matches_oracle_fp32(dev, prec, H, I):
    """moelab tests/test_kernels.py:16-51: 3 experts, weights 0.5/0.3/0.2, out pre-filled 0.5
    (the kernels ADD), fp32 activations, rel-err < 1e-4."""
    lay, blobs, mats = make_records(prec, H, I, 3, H + I)
    ws = [0.5, 0.3, 0.2]
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(H + I))
    ref = O.moe_layer(x.numpy(), np.array([[0, 1, 2]]), np.array([ws]), lambda e: mats[e])
    recs = to_dev(blobs, dev)
    ents = [(views(lay, b), w) for b, w in zip(recs, ws)]
    out = torch.full((1, H), 0.5, device=dev)
    if prec == "int4":
        K.grouped_ffn_int4(x.to(dev), ents, lay["group_sizes"], out)
    elif prec == "int8":
        K.grouped_ffn_int8(x.to(dev), ents, lay, out)
    elif prec == "fp8":
        K.grouped_ffn_fp8(x.to(dev), ents, out)
    else:
        K.grouped_ffn_float(x.to(dev), ents, out)
    got = out.cpu().numpy() - 0.5
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-4, (prec, H, I, err)


@pytest.mark.parametrize("prec", ["int4", "int8", "fp16", "fp8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_grouped_olmoe_shape(dev, prec, dtype):
    """scripts/check_setup.py:88-126 case: 8 experts at OLMoE dims (H=2048, I=1024),
    W ~ 0.02 N(0,1), weights 0.125, x ~ N(0,1) in the model dtype."""
    H, I, n = 2048, 1024, 8
    lay, blobs, mats = make_records(prec, H, I, n, 11, std=0.02)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(12)).to(dtype)
    ref = O.moe_layer(x.float().numpy(), np.array([list(range(n))]), np.full((1, n), 0.125), lambda e: mats[e])
    recs = to_dev(blobs, dev)
    ents = [(views(lay, b), 0.125) for b in recs]
    out = torch.zeros(1, H, dtype=dtype, device=dev)
    if prec == "int4":
        K.grouped_ffn_int4(x.to(dev), ents, lay["group_sizes"], out)
    elif prec == "int8":
        K.grouped_ffn_int8(x.to(dev), ents, lay, out)
    elif prec == "fp8":
        K.grouped_ffn_fp8(x.to(dev), ents, out)
    else:
        K.grouped_ffn_float(x.to(dev), ents, out)
    assert_layer_close(out.float().cpu().numpy(), ref, dtype)


def test_grouped_weight_zero_rows_skipped_and_deterministic(dev):
    H, I = 512, 256
    lay, blobs, mats = make_records("int4", H, I, 4, 3)
    recs = to_dev(blobs, dev)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(1)).to(dev)
    ws = [0.4, 0.0, 0.35, 0.25]
    ents = [(views(lay, b), w) for b, w in zip(recs, ws)]
    outs = []
    for _ in range(3):
        out = torch.zeros(1, H, device=dev)
        K.grouped_ffn_int4(x, ents, lay["group_sizes"], out)
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])  # bitwise: table-order combine
    ref = O.moe_layer(x.cpu().numpy(), np.array([[0, 2, 3]]), np.array([[0.4, 0.35, 0.25]]), lambda e: mats[e])
    assert np.abs(outs[0].numpy() - ref).max() / np.abs(ref).max() < 1e-4


def test_expert_ffn_int4(dev):
    H, I = 256, 128
    lay, blobs, mats = make_records("int4", H, I, 1, 5)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(2))
    ref = O.expert_ffn(x.numpy(), *mats[0])
    y = K.expert_ffn_int4(x.to(dev), views(lay, to_dev(blobs, dev)[0]), lay["group_sizes"], torch.nn.functional.silu)
    assert np.abs(y.cpu().numpy() - ref).max() / np.abs(ref).max() < 1e-4


def test_grouped_graph_replays(dev):
    """GroupedGraph captured once, replayed with different tables: every replay equals the
    eager result, with eager work and syncs between replays."""
    H, I, k = 512, 256, 4
    lay4, b4, m4 = make_records("int4", H, I, 6, 21)
    lay16, b16, m16 = make_records("fp16", H, I, 6, 22)
    r4, r16 = to_dev(b4, dev), to_dev(b16, dev)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(3)).to(dev)
    out = torch.zeros(1, H, device=dev)
    gg = K.GroupedGraph({"fp16": lay16, "int4": lay4}, x, out, k)
    rng = np.random.default_rng(0)
    for step in range(5):
        e16 = rng.choice(6, 1 + step % 2, replace=False)
        e4 = rng.choice(6, 2, replace=False)
        w16 = rng.random(len(e16)).astype(np.float32)
        w4 = rng.random(2).astype(np.float32)
        cpu = torch.randn(1, H, generator=torch.Generator().manual_seed(step)).to(dev) if step % 2 else None
        gg.run({"fp16": [(r16[e], float(w)) for e, w in zip(e16, w16)],
                "int4": [(r4[e], float(w)) for e, w in zip(e4, w4)]}, cpu)
        torch.cuda.synchronize()
        ref = O.moe_layer(x.cpu().numpy(), np.array([list(e16)]), np.array([w16]), lambda e: m16[e])
        ref += O.moe_layer(x.cpu().numpy(), np.array([list(e4)]), np.array([w4]), lambda e: m4[e])
        if cpu is not None:
            ref += cpu.cpu().numpy()
        err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
        assert err < 1e-4, (step, err)
        _ = (x * 2).sum().item()  # eager work + sync between replays
    assert gg.graph is not None and gg.replays == 4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_unpacked_int4_records_through_the_int8_kernels(dev, dtype):
    """moelab's unpacked int4 form (store.py:177-203; runtime.py:230-240 runs it with
    grouped_ffn_int8): int4 records rewritten in the int8 layout on the GPU hold exactly the
    oracle's weights, and grouped_ffn_int8 and a GroupedGraph of that layout (first run and
    replays) give the packed records' result: the same weights, so equal up to the fp32 sums'
    order, and the oracle's layer within the north-star tolerance."""
    H, I, n = 2048, 1024, 8
    lay4, blobs, mats = make_records("int4", H, I, n, 41, std=0.02)
    lay8 = unpacked_layout(lay4)
    r4 = to_dev(blobs, dev)
    r8 = [unpack_int4_record(b, lay4, lay8) for b in r4]
    olay8 = O.record_layout("int8", H, I, 64)
    for e in range(2):
        m8 = O.materialize(olay8, r8[e].cpu().numpy())
        assert all(np.array_equal(a, b) for a, b in zip(m8, mats[e]))
    rng = np.random.default_rng(7)
    for step in range(3):
        x = torch.randn(1, H, generator=torch.Generator().manual_seed(40 + step)).to(dtype).to(dev)
        w = rng.random(n).astype(np.float32)
        ref = O.moe_layer(x.float().cpu().numpy(), np.arange(n)[None], w[None], lambda e: mats[e])
        out4 = torch.zeros(1, H, dtype=dtype, device=dev)
        out8 = torch.zeros(1, H, dtype=dtype, device=dev)
        K.grouped_ffn_int4(x, [(views(lay4, b), float(v)) for b, v in zip(r4, w)], lay4["group_sizes"], out4)
        K.grouped_ffn_int8(x, [(views(lay8, b), float(v)) for b, v in zip(r8, w)], lay8, out8)
        if step == 0:
            g4 = torch.zeros(1, H, dtype=dtype, device=dev)
            g8 = torch.zeros(1, H, dtype=dtype, device=dev)
            gg4 = K.GroupedGraph({"int4": lay4}, x, g4, n)
            gg8 = K.GroupedGraph({"int4": lay8}, x, g8, n)  # the fast tier keeps the store's name
            xg = x
        xg.copy_(x)
        gg4.run({"int4": [(b, float(v)) for b, v in zip(r4, w)]})
        gg8.run({"int4": [(b, float(v)) for b, v in zip(r8, w)]})
        torch.cuda.synchronize()
        scale = np.abs(ref).max()
        for got in (out4, out8, g4, g8):
            assert_layer_close(got.float().cpu().numpy(), ref, dtype)
        ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7  # relative spacing of the output dtype
        for a, b in ((out8, out4), (g8, g4)):  # at most one rounding step apart
            assert np.abs(a.float().cpu().numpy() - b.float().cpu().numpy()).max() / scale <= 2 * ulp
    assert gg8.replays == 2 and gg4.replays == 2


# ---------------------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,E,k,renorm", [(1, 64, 8, False), (33, 64, 8, False), (8, 128, 8, True),
                                          (32, 512, 10, True), (5, 16, 4, True), (7, 200, 6, False),
                                          (6, 256, 8, True), (9, 1024, 8, False)])
def test_router_topk(dev, dtype, T, E, k, renorm):
    # (E picks the top-k's key slots per lane: 1 up to 64 experts, then 2, 4, 8, 16 up to 1024)
    H = 2048
    g = torch.Generator().manual_seed(T * E + k)
    x = torch.randn(T, H, generator=g).to(dtype)
    W = (torch.randn(E, H, generator=g) * 0.02).to(dtype)
    lo, oi, ow, _ = O.router(x.float().numpy(), W.float().numpy(), k, renorm, NPDT[dtype])
    xd, Wd = x.to(dev), W.to(dev)
    logits = torch.empty(T, E, dtype=dtype, device=dev)
    idx = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=dtype, device=dev)
    w32 = torch.empty(T, k, dtype=torch.float32, device=dev)
    _lib.call("moehip_router_topk", xd.data_ptr(), Wd.data_ptr(), T, H, E, k, int(renorm), _lib.dt_code(dtype),
              logits.data_ptr(), idx.data_ptr(), w.data_ptr(), w32.data_ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    gl = logits.float().cpu().numpy()
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    # logits: one rounding of an fp32 sum vs one rounding of the exact sum: within one dtype ulp
    # plus the fp32 accumulation error (bounded here by 8 sqrt(H) u sum|x w|, u = 2^-24)
    accb = 8 * np.sqrt(H) * 2.0 ** -24 * (np.abs(x.float().numpy()) @ np.abs(W.float().numpy()).T)
    bound = ulp * np.exp2(np.floor(np.log2(np.abs(lo) + 1e-30))) + accb + 1e-7
    assert np.all(np.abs(gl - lo) <= bound + ulp * np.exp2(np.floor(np.log2(accb + 1e-30))))
    same_logits = np.array_equal(gl, lo)
    gi = idx.cpu().numpy()
    clear = O.topk_margin(lo, k) > 2 * bound.max(axis=-1)
    for t in range(T):
        if same_logits or clear[t]:
            assert gi[t].tolist() == oi[t].tolist(), t  # bit-exact indices, same order
    if same_logits:
        assert np.array_equal(gi, oi)
    gw = w32.cpu().numpy()
    assert np.allclose(gw[clear], ow[clear], rtol=2 * ulp, atol=1e-6)
    assert np.array_equal(w.float().cpu().numpy(), gw)


def test_router_planted_ties(dev):
    """Equal logits: the lowest expert index wins, as in the oracle."""
    H, E = 64, 16
    W = torch.zeros(E, H)
    W[:, 0] = torch.tensor([0.1, 0.9, 0.5, 0.2, 0.3, 0.5, 0.4, 0.4, 0.0, 0.5, 0.1, 0.2, 0.3, 0.4, 0.9, 0.0])
    x = torch.zeros(1, H)
    x[0, 0] = 1.0
    for k in (2, 3, 4, 6):
        _, oi, _, _ = O.router(x.numpy(), W.numpy(), k, False, "float16")
        logits = torch.empty(1, E, dtype=torch.float16, device=dev)
        idx = torch.empty(1, k, dtype=torch.int64, device=dev)
        w32 = torch.empty(1, k, device=dev)
        xd, Wd = x.half().to(dev), W.half().to(dev)  # held until the kernel ran
        _lib.call("moehip_router_topk", xd.data_ptr(), Wd.data_ptr(), 1, H, E, k, 0, 0,
                  logits.data_ptr(), idx.data_ptr(), None, w32.data_ptr(), _lib.stream_of(dev))
        torch.cuda.synchronize()
        assert idx.cpu().numpy()[0].tolist() == oi[0].tolist()


# ---------------------------------------------------------------------------------------
# HOBBIT decision + table, dispatch
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("pol_kw", [dict(mode="hobbit", t1=0.6), dict(mode="hobbit", t1=0.3, t_mid=0.7, t2=0.9),
                                    dict(mode="hi"), dict(mode="lo"), dict(mode="hobbit", t1=0.5, upgrade=False),
                                    dict(mode="weight", t1=0.3), dict(mode="weight", t1=0.3, upgrade=False)])
def test_decide_table_matches_policy(dev, pol_kw):
    precs = ["fp16", "int8", "int4"]
    P, E, k = 3, 32, 8
    g = np.random.default_rng(5)
    pol = PrecisionPolicy(**pol_kw)
    ref = O.Policy(**{kk: v for kk, v in pol_kw.items() if kk != "upgrade"})
    resident = g.random((P, E)) < 0.7
    rtab = torch.from_numpy(np.where(resident, (np.arange(P * E).reshape(P, E) + 1) * 4096 * 1024, 0).astype(np.int64))
    offs = torch.tensor([[0, 8, 16, 24], [0, 64, 128, 192], [0, 32, 64, 96]], dtype=torch.int64)
    planned = torch.tensor([1, 1, 1], dtype=torch.int32)
    lv2p = (ctypes.c_int * 3)(0, 1, 2)
    rtab_d, offs_d, planned_d = rtab.to(dev), offs.to(dev), planned.to(dev)
    for trial in range(20):
        idx = g.choice(E, k, replace=False)
        w = (g.random(k) ** 2).astype(np.float32)
        tab = torch.zeros(P, k, 4, dtype=torch.int64, device=dev)
        wtab = torch.zeros(P, k, device=dev)
        info = torch.zeros(3, k, device=dev)
        miss = torch.zeros(1, device=dev)
        idx_d, w_d = torch.from_numpy(idx).to(dev), torch.from_numpy(w).to(dev)  # held until the kernel ran
        _lib.call("moehip_decide_table", idx_d.data_ptr(), w_d.data_ptr(), k, ctypes.byref(pol.device_policy(2)),
                  lv2p, rtab_d.data_ptr(), P, E, offs_d.data_ptr(), planned_d.data_ptr(), tab.data_ptr(),
                  wtab.data_ptr(), info.data_ptr(), miss.data_ptr(), _lib.stream_of(dev))
        torch.cuda.synchronize()
        lvl, skip = ref.levels(2, w[None])
        lvl, skip = lvl[0], skip[0]
        exp_ch = []
        for j in range(k):
            req = lvl[j]
            ch = -1
            for pi in reversed(range(P)):
                if resident[pi, idx[j]] and ((req >= pi) if pol.allow_upgrade else (req == pi)):
                    ch = pi
            exp_ch.append(ch)
        inf = info.cpu().numpy()
        assert inf[0].tolist() == idx.astype(np.float32).tolist()
        assert inf[2].tolist() == lvl.astype(np.float32).tolist()
        assert inf[1].tolist() == [(-2.0 if skip[j] else float(exp_ch[j])) for j in range(k)]
        assert miss.item() == sum(1 for j in range(k) if not skip[j] and exp_ch[j] < 0)
        tb, wt = tab.cpu().numpy(), wtab.cpu().numpy()
        for j in range(k):
            for pi in range(P):
                sel = exp_ch[j] == pi and not skip[j]
                exp_row = (rtab[pi, idx[j]].item() + offs[pi]).numpy() if sel else np.zeros(4, np.int64)
                assert np.array_equal(tb[pi, j], exp_row)
                assert wt[pi, j] == (w[j] if sel else 0.0)


@pytest.mark.parametrize("T,k,E,with_skip", [(1, 8, 64, False), (8, 8, 64, True), (32, 10, 512, False),
                                             (512, 8, 128, True), (1000, 8, 1024, False), (3, 2, 4, True)])
def test_dispatch_bit_exact(dev, T, k, E, with_skip):
    g = np.random.default_rng(T + k + E)
    idx = np.stack([g.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    skip = (g.random((T, k)) < 0.25) if with_skip else None
    se, sp, counts, offsets = O.dispatch(idx, E, skip)
    NP = T * k
    c = torch.empty(E, dtype=torch.int32, device=dev)
    o = torch.empty(E + 1, dtype=torch.int32, device=dev)
    s = torch.empty(NP, dtype=torch.int32, device=dev)
    r = torch.empty(NP, dtype=torch.int32, device=dev)
    sk = torch.from_numpy(skip.astype(np.uint8)).to(dev) if skip is not None else None
    idx_d = torch.from_numpy(idx).to(dev)  # held until the kernel ran
    _lib.call("moehip_dispatch", idx_d.data_ptr(), _lib.ptr(sk), T, k, E, c.data_ptr(),
              o.data_ptr(), s.data_ptr(), r.data_ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), counts)
    assert np.array_equal(o.cpu().numpy(), offsets)
    got_s = s.cpu().numpy()
    assert np.array_equal(got_s[:len(sp)], sp) and (got_s[len(sp):] == -1).all()
    rank = r.cpu().numpy()
    exp_rank = np.full(NP, -1)
    exp_rank[sp] = np.arange(len(sp))
    assert np.array_equal(rank, exp_rank)


# ---------------------------------------------------------------------------------------
# the whole decode layer (router -> HOBBIT -> kernels -> combine)
# ---------------------------------------------------------------------------------------
class _Stack:
    """L layers x E experts of random N(0, std) weights, encoded on the GPU in every precision,
    with the oracle's float view of each (layer, expert, precision) built on demand."""

    def __init__(self, dev, H, I, E, L, precs, seed, std=0.02, dtype=torch.float16):
        self.H, self.I, self.E, self.L, self.precs, self.dtype = H, I, E, L, precs, dtype
        self.seed, self.std = seed, std
        self.store = ResidentStore({p: record_layout(p, H, I, 64, scale="absmax") for p in precs}, L, E, dev)
        for l in range(L):
            for e in range(E):
                gu, dn = self.weights(l, e)
                gu_d, dn_d = gu.to(dev), dn.to(dev)
                for p in precs:
                    self.store.encode(p, l, e, gu_d, dn_d)
        g = torch.Generator().manual_seed(seed)
        self.Wr = [(torch.randn(E, H, generator=g) * std).to(dtype) for _ in range(L)]
        self.g = g
        self._mats = {}

    def weights(self, l, e):
        """(gate_up, down) of expert e of layer l, regenerated from its own seed."""
        g = torch.Generator().manual_seed(self.seed * 1_000_003 + l * 4099 + e)
        return (torch.randn(2 * self.I, self.H, generator=g) * self.std,
                torch.randn(self.H, self.I, generator=g) * self.std)

    def mats(self, l, e, p):
        key = (l, e, p)
        if key not in self._mats:
            gu, dn = self.weights(l, e)
            lay = O.record_layout(p, self.H, self.I, 64, scale="absmax")
            self._mats[key] = O.materialize(lay, O.encode_record(lay, gu.numpy(), dn.numpy(), "absmax"))
        return self._mats[key]

    def reference(self, l, x, k, renorm, pol, planned=None):
        dt = NPDT[self.dtype]
        lo, idx, w, _ = O.router(x.float().numpy(), self.Wr[l].float().numpy(), k, renorm, dt)
        lvl, skip = pol.levels(l, w)
        prec_of = {}
        for j in range(k):
            prec_of[int(idx[0, j])] = O.level_to_precision(int(lvl[0, j]), self.precs)
        ref = O.moe_layer(x.float().numpy(), idx, w, lambda e: self.mats(l, e, prec_of[e]), skip=skip)
        return lo, idx, w, ref


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mode", ["lo", "hobbit", "weight"])
def test_decoder_layer_olmoe(dev, mode, fused):
    """OLMoE layers; hobbit / weight: fp16 and int4 records of every expert, the level picks the
    record (the weight rule with a threshold that splits this seed's top-8 into both kinds)."""
    H, I, E, k, L = 2048, 1024, 64, 8, 2
    dtype = torch.float16
    precs = ["fp16", "int4"] if mode in ("hobbit", "weight") else ["int4"]
    S = _Stack(dev, H, I, E, L, precs, 100)
    xs = [torch.randn(1, H, generator=S.g).to(dtype) for _ in range(L)]
    t1 = 0.5
    if mode == "weight":  # the median routed weight of these tokens: both record kinds run
        ws = [O.router(xs[l].float().numpy(), S.Wr[l].float().numpy(), k, False, "float16")[2] for l in range(L)]
        t1 = float(np.median(np.concatenate([w.ravel() for w in ws])))
    pol = PrecisionPolicy(mode, t1=t1, upgrade=False)
    dec = MoEDecoder(S.store, k, pol, dtype, router_weights=[w.to(dev) for w in S.Wr], fused=fused)
    assert dec.fused == fused
    for l in range(L):
        x = xs[l]
        out = torch.zeros(1, H, dtype=dtype, device=dev)
        dec.layer(l, x.to(dev), out)
        if fused:  # the kernel that produced this output: one record kind -> the XCD kernel
            assert _lib.last_decode_kernel() == ("k_decode_xcd" if len(precs) == 1 else "k_decode_layer")
        torch.cuda.synchronize()
        lo, idx, w, ref = S.reference(l, x, k, False, O.Policy(mode, t1=t1))
        assert dec.idx.cpu().numpy().tolist() == idx.tolist()
        if mode == "weight" and l == 0:  # the rows really split between the two record kinds
            ch = dec.info[l, 1].cpu().numpy()
            assert (ch == 0).any() and (ch == 1).any(), ch
        assert np.allclose(dec.w32.cpu().numpy(), w, rtol=2.0 ** -10, atol=0)
        assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    assert dec.miss.item() == 0
    dec.check_error()


def test_fused_repeated_launches_and_graph_replays(dev):
    """Counters reset after every launch: many launches in a row, then the same layers captured
    in a HIP graph and replayed with new inputs written between replays; every output checked."""
    H, I, E, k, L = 1024, 512, 32, 4, 3
    dtype = torch.bfloat16
    S = _Stack(dev, H, I, E, L, ["int4"], 7, dtype=dtype)
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), dtype, router_weights=[w.to(dev) for w in S.Wr])
    xs = torch.randn(6, L, 1, H, generator=S.g).to(dtype)
    outs = torch.zeros(L, 1, H, dtype=dtype, device=dev)
    xbuf = torch.zeros(L, 1, H, dtype=dtype, device=dev)
    pol = O.Policy("lo")
    for t in range(3):  # eager
        xbuf.copy_(xs[t].to(dev))
        for l in range(L):
            dec.layer(l, xbuf[l], outs[l])
        got = outs.float().cpu().numpy()
        for l in range(L):
            assert_layer_close(got[l], S.reference(l, xs[t, l], k, False, pol)[3], dtype)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for l in range(L):
            dec.layer(l, xbuf[l], outs[l])
    for t in range(3, 6):  # replays
        xbuf.copy_(xs[t].to(dev))
        gr.replay()
        torch.cuda.synchronize()
        got = outs.float().cpu().numpy()
        for l in range(L):
            assert_layer_close(got[l], S.reference(l, xs[t, l], k, False, pol)[3], dtype)
        _ = (xbuf.float() * 2).sum().item()  # eager work between replays
    dec.check_error()


@pytest.mark.parametrize("fused", [True, False])
def test_layer_add_and_accumulate(dev, fused):
    """The optional output terms: out = layer(x) (+ out if accumulate) (+ cpu_part, the partial of
    experts run elsewhere: the offload path's CPU experts), summed in fp32 in that order."""
    H, I, E, k = 1024, 512, 32, 4
    dtype = torch.float16
    S = _Stack(dev, H, I, E, 1, ["int4"], 11)
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), dtype, router_weights=[w.to(dev) for w in S.Wr],
                     fused=fused)
    x = torch.randn(1, H, generator=S.g).to(dtype)
    ref = S.reference(0, x, k, False, O.Policy("lo"))[3]
    scale = float(np.abs(ref).max())
    add = (torch.randn(1, H, generator=S.g) * scale).to(dtype)
    o0 = (torch.randn(1, H, generator=S.g) * scale).to(dtype)
    for acc_flag, with_add in [(False, True), (True, False), (True, True)]:
        out = o0.to(dev) if acc_flag else torch.zeros(1, H, dtype=dtype, device=dev)
        dec.layer(0, x.to(dev), out, cpu_part=add.to(dev) if with_add else None, accumulate=acc_flag)
        torch.cuda.synchronize()
        exp = ref.astype(np.float64)
        if acc_flag:
            exp = exp + o0.double().numpy()
        if with_add:
            exp = exp + add.double().numpy()
        assert_layer_close(out.float().cpu().numpy(), exp, dtype)
    dec.check_error()


def test_fused_external_routing(dev):
    """Router skipped: idx / w32 given (the experts-module call of moelab/runtime.py:1108)."""
    H, I, E, k = 512, 256, 16, 4
    S = _Stack(dev, H, I, E, 1, ["int8", "int4"], 3)
    dec = MoEDecoder(S.store, k, PrecisionPolicy("hobbit", t1=0.6, upgrade=False), torch.float16,
                     router_weights=[w.to(dev) for w in S.Wr])
    x = torch.randn(1, H, generator=S.g).half()
    idx = torch.tensor([[3, 11, 0, 7]])
    w = torch.tensor([[0.4, 0.3, 0.2, 0.1]], dtype=torch.float32)
    out = torch.zeros(1, H, dtype=torch.float16, device=dev)
    idx_d, w_d = idx.to(dev), w.to(dev)
    dec.layer(0, x.to(dev), out, idx=idx_d.view(-1), w32=w_d.view(-1))
    torch.cuda.synchronize()
    lvl, _ = O.Policy("hobbit", t1=0.6).levels(0, w.numpy())
    prec_of = {int(e): O.level_to_precision(int(v), ["int8", "int4"]) for e, v in zip(idx[0], lvl[0])}
    ref = O.moe_layer(x.float().numpy(), idx.numpy(), w.numpy(), lambda e: S.mats(0, e, prec_of[e]))
    assert_layer_close(out.float().cpu().numpy(), ref, torch.float16)
    info = dec.info[0].cpu().numpy()
    assert info[0].tolist() == [3, 11, 0, 7] and info[2].tolist() == lvl[0].astype(np.float32).tolist()


@pytest.mark.parametrize("prec", ["int4", "fp8"])
def test_fused_qwen3next_shape(dev, prec):
    """Qwen3-Next routed experts: d_model 2048, 512 experts, top-10 renormalised, d_ff 512, bf16."""
    H, I, E, k = 2048, 512, 512, 10
    dtype = torch.bfloat16
    S = _Stack(dev, H, I, E, 1, [prec], 11, dtype=dtype)
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), dtype, router_weights=[S.Wr[0].to(dev)], renorm=True)
    for t in range(2):
        x = torch.randn(1, H, generator=S.g).to(dtype)
        out = torch.zeros(1, H, dtype=dtype, device=dev)
        dec.layer(0, x.to(dev), out)
        # fp8 rows make more items than resident workgroups: the two-pass instantiation
        assert _lib.last_decode_kernel() == ("k_decode_xcd" if prec == "int4" else "k_decode_xcd (two passes)")
        torch.cuda.synchronize()
        lo, idx, w, ref = S.reference(0, x, k, True, O.Policy("lo"))
        assert dec.idx.cpu().numpy().tolist() == idx.tolist()
        assert_layer_close(out.float().cpu().numpy(), ref, dtype)
    dec.check_error()


@pytest.mark.parametrize("E", [16, 128, 256, 1024])
@pytest.mark.parametrize("k", [2, 3, 6, 13])
def test_fused_router_planted_ties(dev, k, E):
    """Fused router on tied logits (including -0 against +0): equal logits go to the lowest
    expert index, in the oracle's order. E = 16: one key per lane, ranked by counting; E = 128:
    the candidate filter (keys at or above the k-th largest of the lanes' largest keys, ranked
    among themselves); E = 256 and 1024: the same with the router rows split over the XCDs and
    the logits relayed between them. The pattern repeats so that ties span far-apart indices."""
    H, I = 512, 256
    S = _Stack(dev, H, I, E, 1, ["int4"], 5)
    col = torch.tensor([0.1, 0.9, 0.5, -0.0, 0.3, 0.5, 0.4, 0.4, 0.0, 0.5, 0.1, -0.2, 0.3, 0.4, 0.9, 0.0]).repeat(E // 16)
    W = torch.zeros(E, H)
    W[:, 0] = col
    S.Wr[0] = W.half()
    x = torch.zeros(1, H, dtype=torch.float16)
    x[0, 0] = 1.0
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), torch.float16, router_weights=[S.Wr[0].to(dev)])
    assert dec.fused
    out = torch.zeros(1, H, dtype=torch.float16, device=dev)
    dec.layer(0, x.to(dev), out)
    torch.cuda.synchronize()
    lo, idx, w, ref = S.reference(0, x, k, False, O.Policy("lo"))
    assert dec.idx.cpu().numpy().tolist() == idx.tolist()
    assert np.allclose(dec.w32.cpu().numpy(), w, rtol=2.0 ** -10, atol=0)
    assert_layer_close(out.float().cpu().numpy(), ref, torch.float16)
    dec.check_error()


@pytest.mark.parametrize("prec", ["int4", "fp8"])
@pytest.mark.parametrize("routed", [True, False])
def test_fused_qwen3next_shared_expert(dev, prec, routed):
    """Qwen3-Next layer with its shared expert in the same launch: routed top-10 of 512
    (renormalised) + sigmoid(x . g) * FFN_s(x), bf16; the gate logit and the sigmoid rounded to
    bf16 as the module computes them (modeling_qwen3_next.py:786-797)."""
    H, I, E, k = 2048, 512, 512, 10
    dtype = torch.bfloat16
    S = _Stack(dev, H, I, E, 1, [prec], 12, dtype=dtype)
    lay = S.store.layouts[prec]
    g = torch.Generator().manual_seed(77)
    gu_s, dn_s = torch.randn(2 * I, H, generator=g) * 0.02, torch.randn(H, I, generator=g) * 0.02
    sh_blob = torch.zeros(lay["record_bytes"], dtype=torch.uint8, device=dev)
    encode_record_(lay, sh_blob, gu_s.to(dev), dn_s.to(dev))
    gate = (torch.randn(H, generator=g) * 0.05).to(dtype)
    olay = O.record_layout(prec, H, I, 64, scale="absmax")
    mats_s = O.materialize(olay, O.encode_record(olay, gu_s.numpy(), dn_s.numpy(), "absmax"))
    dec = MoEDecoder(S.store, k, PrecisionPolicy("lo"), dtype, router_weights=[S.Wr[0].to(dev)] if routed else None,
                     renorm=True, shared=[{"gate": gate.to(dev), "rec": {prec: sh_blob}}])
    for t in range(3):
        x = torch.randn(1, H, generator=g).to(dtype)
        out = torch.zeros(1, H, dtype=dtype, device=dev)
        print(f"shared expert {prec} routed={routed} token {t}", flush=True)
        if routed:
            dec.layer(0, x.to(dev), out)
            _, idx, w, ref = S.reference(0, x, k, True, O.Policy("lo"))
        else:
            idx = torch.randperm(E, generator=g)[:k].view(1, k).numpy()
            w = O.round_to(np.random.default_rng(t).random((1, k)).astype(np.float32), "bfloat16")
            dec.layer(0, x.to(dev), out, idx=torch.from_numpy(idx).to(dev),
                      w32=torch.from_numpy(w.astype(np.float32)).to(dev))
            ref = O.moe_layer(x.float().numpy(), idx, w.astype(np.float64), lambda e: S.mats(0, e, prec))
        assert _lib.last_decode_kernel() == ("k_decode_xcd" if prec == "int4" else "k_decode_xcd (two passes)")
        torch.cuda.synchronize()
        xf = x.float().numpy().astype(np.float64)
        logit = O.round_to((xf @ gate.float().numpy().astype(np.float64)).astype(np.float32), "bfloat16")
        gs = O.round_to((1.0 / (1.0 + np.exp(-logit.astype(np.float64)))).astype(np.float32), "bfloat16")
        ref = ref + gs.astype(np.float64)[:, None] * O.expert_ffn(xf, *mats_s)
        if routed:
            assert dec.idx.cpu().numpy().tolist() == idx.tolist()
        assert_layer_close(out.float().cpu().numpy(), ref, dtype)
        assert dec.miss.item() == 0
    dec.check_error()
