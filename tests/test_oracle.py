"""
Pins the oracle (oracle/moe_ref.py) against the reference's own known answers and tolerances,
closed forms, invariants, brute force, and the upstream library code the reference calls
(transformers' routers and experts). CPU only.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O


# -- quant.py ---------------------------------------------------------------------------
def test_int4_packing_order_known_answer():
    """tests/test_units.py:33-38: w=[7,-7] -> byte (7+8) | ((-7+8) << 4), dequantised exactly."""
    w = np.zeros((1, 64), np.float32)
    w[0, 0], w[0, 1] = 7.0, -7.0
    q, s = O.quantize(w, 4, 64)
    assert int(q[0, 0]) == (7 + 8) | ((-7 + 8) << 4) == 0x1F
    assert np.array_equal(O.dequantize(q, s, 4, "float32")[0, :2], np.array([7.0, -7.0], np.float32))


@pytest.mark.parametrize("bits,tol", [(8, 0.008), (4, 0.12)])
def test_quant_roundtrip_reference_tolerance(bits, tol):
    """tests/test_units.py:19-30 on the same torch-seeded input."""
    torch.manual_seed(0)
    w = torch.randn(96, 256).numpy()
    q, s = O.quantize(w, bits, 64)
    assert s.shape == (96, 4) and s.dtype == np.float16
    assert q.shape == ((96, 256) if bits == 8 else (96, 128))
    back = O.dequantize(q, s, bits, "float32")
    rel = np.linalg.norm(back - w) / np.linalg.norm(w)
    assert rel < tol, rel


def test_zero_group_and_group_size_known_answers():
    """tests/test_units.py:41-45."""
    q, s = O.quantize(np.zeros((4, 64), np.float32), 4, 64)
    assert np.array_equal(O.dequantize(q, s, 4, "float32"), np.zeros((4, 64), np.float32))
    assert s[0, 0] == np.float16(1e-7)  # never a zero scale (quant.py:57-61)
    assert O.pick_group_size(1024) == 64 and O.pick_group_size(32) == 32 and O.pick_group_size(768) == 64
    assert O.pick_group_size(96) == 48 and O.pick_group_size(512) == 64
    assert O.bits_per_weight(4, 64) == 4.25


def test_int4_pack_unpack_all_pairs():
    """Every (even, odd) pair of values in [-8, 7] survives pack -> unpack; bytes are distinct."""
    a, b = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    q = np.stack([a.reshape(-1), b.reshape(-1)], axis=1).astype(np.int16)  # (256, 2)
    packed = O.pack(q, 4)
    assert packed.shape == (256, 1) and len(np.unique(packed)) == 256
    assert np.array_equal(O.unpack_int4(packed).astype(np.int16), q)
    # low nibble holds the even column: value 7 at column 0, -8 at column 1 -> 0x0F
    assert int(O.pack(np.array([[7, -8]], np.int16), 4)[0, 0]) == 0x0F


def test_absmax_closed_forms():
    w = np.zeros((2, 64), np.float32)
    w[0, :8] = [7, -7, 3.5, 1, 0, -2, 6, 5]  # absmax 7 -> scale exactly 1 -> q = round-half-even(w)
    w[1, 0] = -1.27e2  # int8: scale 1.0
    q4, s4 = O.quantize(w[:1], 4, 64)
    assert s4[0, 0] == np.float16(1.0)
    assert np.array_equal(O.unpack_int4(q4)[0, :8], np.array([7, -7, 4, 1, 0, -2, 6, 5], np.int8))  # 3.5 -> 4
    q8, s8 = O.quantize(w[1:], 8, 64)
    assert s8[0, 0] == np.float16(1.0) and q8[0, 0] == -127
    # scale is rounded to fp16 BEFORE quantising (quant.py:68-69): absmax 0.7 -> fp16(0.1)
    g = np.full((1, 64), 0.05, np.float32)
    g[0, 0] = 0.7
    _, s = O.quantize(g, 4, 64)
    assert s[0, 0] == np.float16(np.float32(0.7) / np.float32(7))


def test_mse_known_answer_negative_scale():
    """tests/test_requant.py:35-42: the largest weight lands on -8 with a negative scale."""
    w = np.zeros((2, 64), np.float32)
    w[0, 0] = 8.0
    w[0, 1:5] = [1.0, 2.0, 3.0, -4.0]
    q, s = O.quantize(w, 4, 64, "mse")
    back = O.dequantize(q, s, 4, "float32")
    assert np.allclose(back[0, :5], w[0, :5]) and float(s[0, 0]) == -1.0
    assert np.array_equal(back[1], np.zeros(64, np.float32))


def test_mse_never_worse_than_absmax():
    """tests/test_requant.py:21-33 (Student-t weights, torch seed 0)."""
    torch.manual_seed(0)
    w = torch.distributions.StudentT(4).sample((256, 512)).numpy()

    def err(q, s):
        return float(((O.dequantize(q, s, 4, "float32") - w) ** 2).mean())

    e_abs = err(*O.quantize(w, 4, 64, "absmax"))
    e_mse = err(*O.quantize(w, 4, 64, "mse"))
    assert e_mse < 0.8 * e_abs, (e_abs, e_mse)
    g = w.reshape(256, 8, 64)
    sa = O.choose_scales(g, 4, "absmax").astype(np.float32)
    sm = O.choose_scales(g, 4, "mse").astype(np.float32)
    ea = ((np.clip(np.rint(g / sa), -8, 7) * sa - g) ** 2).sum(-1)
    em = ((np.clip(np.rint(g / sm), -8, 7) * sm - g) ** 2).sum(-1)
    assert bool((em <= ea + 1e-6).all())


def _gptq_case(seed=1, O_=64, I_=256):
    """The reference's GPTQ test set-up (tests/test_requant.py:45-51), numpy-seeded: N(0, 0.05)
    weights, correlated inputs X = N(0, 1) (1 + 0.4 N / sqrt(I)) with 8 columns scaled by 6."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((O_, I_)) * 0.05).astype(np.float32)
    X = (rng.standard_normal((2048, I_)) @ (np.eye(I_) + 0.4 * rng.standard_normal((I_, I_)) / I_ ** 0.5))
    X = X.astype(np.float32)
    X[:, :8] *= 6
    return w, X, (X.T @ X).astype(np.float32)


def test_gptq_reduces_output_error():
    """tests/test_requant.py:45-60: GPTQ's output error on the calibration inputs is at least 15 %
    below mse quantisation's; shapes and dtypes of the store's format."""
    w, X, H = _gptq_case()

    def out_err(q, s):
        return float(((X @ (O.dequantize(q, s, 4, "float32") - w).T) ** 2).mean())

    e_mse = out_err(*O.quantize(w, 4, 64, "mse"))
    q, s = O.gptq_quantize(w, H, 4, 64)
    assert out_err(q, s) < 0.85 * e_mse
    assert q.shape == (64, 128) and q.dtype == np.uint8 and s.shape == (64, 4) and s.dtype == np.float16


@pytest.mark.parametrize("bits,method", [(4, "mse"), (8, "mse"), (4, "absmax")])
def test_gptq_diagonal_hessian_is_plain_quantisation(bits, method):
    """Uncorrelated inputs (a diagonal Hessian): Hinv is diagonal, no error is carried to other
    columns, and GPTQ gives exactly the plain quantisation of the same method."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((48, 384)) * 0.05).astype(np.float32)
    H = np.diag(rng.uniform(0.5, 3.0, 384)).astype(np.float32)
    q, s = O.gptq_quantize(w, H, bits, 64, method)
    q2, s2 = O.quantize(w, bits, 64, method)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint16), s2.view(np.uint16))


def test_gptq_dead_columns_and_hinv():
    """Columns the calibration never excited (zero Hessian row and column: quant.py:153-155) are
    quantised as zeros; Hinv is upper triangular with Hinv^T Hinv = (H + damp)^-1."""
    w, X, H = _gptq_case(3, 32, 128)
    dead = [5, 70, 71]
    H[dead, :] = 0.0
    H[:, dead] = 0.0
    U, d = O.gptq_hinv(H)
    assert d.sum() == 3 and np.allclose(U, np.triu(U))
    Hd = H.astype(np.float64).copy()
    Hd[dead, dead] = 1.0
    Hd[np.diag_indices_from(Hd)] += 0.01 * np.mean(np.diag(Hd))
    ref = np.linalg.inv(Hd)
    assert np.abs(U.astype(np.float64).T @ U - ref).max() < 1e-4 * np.abs(ref).max()
    q, s = O.gptq_quantize(w, H, 4, 64)
    vals = O.unpack_int4(q)
    assert (vals[:, dead] == 0).all()


def test_dequantize_fp16_rounds_product():
    """quant.py:199-204 in float16: (q-8) and the scale are fp16, their product rounds to fp16."""
    q = np.array([[0x0F | (0x0 << 4)]], np.uint8)  # values +7, -8
    s = np.array([[np.float16(0.3)]], np.float16)
    out = O.dequantize(q, s, 4, "float16")
    exp = np.array([np.float16(7) * np.float16(0.3), np.float16(-8) * np.float16(0.3)], np.float16)
    assert np.array_equal(out[0].astype(np.float16), exp)


def test_fp8_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    mine = O.fp8_e4m3fn_to_f32(codes)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(mine), nan)
    assert np.array_equal(mine[~nan], ref[~nan])
    assert O.fp8_e4m3fn_to_f32(np.array([0x7E]))[0] == 448.0


def test_fp8_encode_matches_torch_cast():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(4096, generator=g) * 100).clamp(-448, 448)
    mine = O.f32_to_fp8_e4m3fn(x.numpy())
    ref = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_fp8_block_dequant_multiplies():
    """quant.py:208-219: weight_scale_inv multiplies; block (r//128, c//128)."""
    code = np.full((130, 129), 0x38, np.uint8)  # 1.0
    sc = np.array([[2.0, 3.0], [5.0, 7.0]], np.float32)
    w = O.dequantize_fp8_block(code, sc)
    assert w[0, 0] == 2.0 and w[0, 128] == 3.0 and w[128, 0] == 5.0 and w[129, 128] == 7.0
    with pytest.raises(ValueError):
        O.dequantize_fp8_block(code, sc[:1])


# -- store.py ---------------------------------------------------------------------------
RECORD_SIZES = {  # computed by hand from store.py:76-115 for the three model shapes
    ("int4", 2048, 1024): 3_342_336, ("int8", 2048, 1024): 6_488_064, ("fp16", 2048, 1024): 12_582_912,
    ("int4", 2048, 768): 2_506_752, ("int8", 2048, 768): 4_866_048, ("fp16", 2048, 768): 9_437_184,
    ("int4", 2048, 512): 1_671_168, ("int8", 2048, 512): 3_244_032, ("fp16", 2048, 512): 6_291_456,
}


@pytest.mark.parametrize("key", list(RECORD_SIZES))
def test_record_sizes_known(key):
    prec, H, I = key
    assert O.record_layout(prec, H, I)["record_bytes"] == RECORD_SIZES[key]


def test_olmoe_int4_field_offsets():
    lay = O.record_layout("int4", 2048, 1024)
    assert [f[3] for f in lay["fields"]] == [0, 2_097_152, 2_228_224, 3_276_800]
    assert [f[0] for f in lay["fields"]] == ["gate_up.q", "gate_up.s", "down.q", "down.s"]
    assert lay["group_sizes"] == {"gate_up": 64, "down": 64} and lay["scale"] == "mse"


@pytest.mark.parametrize("prec", ["fp32", "fp16", "bf16", "int8", "int4", "fp8"])
def test_record_roundtrip(prec):
    """tests/test_units.py:49-60 (fp8: the checkpoint fixture's 7 % bound, test_qwen3next.py:38-45)."""
    torch.manual_seed(1)
    H, I = 128, 64
    gu, dn = torch.randn(2 * I, H).numpy(), torch.randn(H, I).numpy()
    lay = O.record_layout(prec, H, I)
    assert lay["record_bytes"] % 4096 == 0
    for _, _, _, off in lay["fields"]:
        assert off % 64 == 0
    blob = O.encode_record(lay, gu, dn, method="absmax")
    g2, d2 = O.materialize(lay, blob, "float32")
    tol = {"fp32": 0, "fp16": 1e-3, "bf16": 1e-2, "int8": 1e-2, "int4": 0.12, "fp8": 0.07}[prec]
    assert np.linalg.norm(g2 - gu) / np.linalg.norm(gu) <= tol
    assert np.linalg.norm(d2 - dn) / np.linalg.norm(dn) <= tol


# -- policy.py ---------------------------------------------------------------------------
def test_hobbit_known_answer_docs06():
    """tests/test_units.py:168-176."""
    w = np.array([[0.1345, 0.1063, 0.0921, 0.0855, 0.0829, 0.0705, 0.0682, 0.0214]], np.float32)
    pol = O.Policy("hobbit", t1=0.6, t2=0.9)
    s = O.unimportance(w)[0]
    assert np.allclose(s, [0.0, 0.2034, 0.3641, 0.5034, 0.6327, 0.7580, 0.8646, 0.9677], atol=2e-4)
    lvl, skip = pol.levels(0, w)
    assert (lvl[0] == 0).tolist() == [True] * 4 + [False] * 4
    assert skip[0].tolist() == [False] * 7 + [True]


def test_hobbit_order_independent_and_modes():
    """tests/test_units.py:179-187."""
    w = np.array([[0.05, 0.6, 0.35]], np.float32)
    assert (O.Policy("hobbit", t1=0.6).levels(3, w)[0][0] == 0).tolist() == [False, True, True]
    assert (O.Policy("hi").levels(0, w)[0] == 0).all()
    assert not (O.Policy("lo").levels(0, w)[0] == 0).any()
    assert (O.Policy("hobbit", protect_layers={3}).levels(3, w)[0] == 0).all()
    pol = O.Policy("hobbit")
    assert pol.expert_level([0, 2]) == 0 and pol.expert_level([0, 2, 2]) == 2


def test_per_layer_t1_and_level_to_precision():
    """tests/test_optim.py:129-136."""
    pol = O.Policy("hobbit", t1=0.6, t1_layers={1: 0.0})
    w = np.array([[0.5, 0.3, 0.2]], np.float32)
    assert pol.levels(1, w)[0][0].tolist() == [0, 2, 2]
    assert pol.levels(0, w)[0][0].tolist() == [0, 0, 2]
    assert [O.level_to_precision(v, ["fp16", "int4"]) for v in (0, 1, 2)] == ["fp16", "int4", "int4"]
    assert [O.level_to_precision(v, ["fp16", "int8", "int4"]) for v in (0, 1, 2)] == ["fp16", "int8", "int4"]


def test_decide_general_vote_by_hand():
    """runtime.py:459-492 on three tokens worked by hand. With t1 = 0.6 each token's best expert has
    s = 0 (level 0) and the others s >= 0.6 (level 2); t2 = 0.9 skips s > 0.9 at level 2.
    token 0: w [0.7, 0.2, 0.1] -> s [0, .7, .9]    -> levels [0, 2, 2], no skip (.9 is not > .9 + 1e-6)
    token 1: w [0.5, 0.45, 0.05] -> s [0, .5, .95] -> levels [0, 0, 2], skip slot 2
    token 2: w [0.4, 0.35, 0.25] -> s [0, .4, .75] -> levels [0, 0, 2]
    idx: e3 gets (t0 lvl 0, t1 lvl 0) -> 0; e5 gets (t0 lvl 2, t2 lvl 0) -> 0 (1 of 2 >= 0.5);
    e7 gets (t0 lvl 2, t2 lvl 2) -> 2; e1 gets (t1 lvl 0, t2 lvl 0) -> 0; e9 only the skipped pair."""
    pol = O.Policy("hobbit", t1=0.6, t2=0.9)
    idx = np.array([[3, 5, 7], [1, 3, 9], [5, 1, 7]])
    w = np.array([[0.7, 0.2, 0.1], [0.5, 0.45, 0.05], [0.4, 0.35, 0.25]], np.float32)
    skip, dec = O.decide_general(pol, 0, idx, w, ["fp16", "int4"])
    assert skip.tolist() == [[False, False, False], [False, False, True], [False, False, False]]
    assert dec == {1: (0, "fp16"), 3: (0, "fp16"), 5: (0, "fp16"), 7: (2, "int4")}
    # a stricter vote: e5 (1 of 2 at level 0) no longer reaches 0.75
    pol.hi_vote = 0.75
    assert O.decide_general(pol, 0, idx, w, ["fp16", "int4"])[1][5] == (2, "int4")


def test_mse_planted_negative_scale_group():
    """The known answer of tests/test_requant.py:35-42 scaled by 1/16 inside random rows: the
    group's mse scale is -1/16 (the largest weight on -8), the negated group's is +1/16, and both
    dequantise exactly; the GPU parity tests plant the same groups in their mse records."""
    rng = np.random.default_rng(0)
    gu = (rng.standard_normal((256, 128)) * 0.05).astype(np.float32)
    dn = (rng.standard_normal((128, 128)) * 0.05).astype(np.float32)
    grp = np.zeros(64, np.float32)
    grp[:5] = np.array([8.0, 1.0, 2.0, 3.0, -4.0], np.float32) / 16
    gu[0, :64], dn[3, 64:128] = grp, -grp
    lay = O.record_layout("int4", 128, 128, 64, scale="mse")
    blob = O.encode_record(lay, gu, dn, method="mse")
    v = O.views(lay, blob)
    assert float(v["gate_up.s"][0, 0]) == -0.0625 and float(v["down.s"][3, 1]) == 0.0625
    g2, d2 = O.materialize(lay, blob)
    assert np.array_equal(g2[0, :64], gu[0, :64]) and np.array_equal(d2[3, 64:128], dn[3, 64:128])


def test_levels_one_known_answers():
    """The one-token float64 rule gives the reference's known answers too (tests/test_units.py:
    168-176, 364-373: levels_one == levels there; tests/test_optim.py:129-136 per-layer t1)."""
    w = [0.1345, 0.1063, 0.0921, 0.0855, 0.0829, 0.0705, 0.0682, 0.0214]
    lvl, skip, s = O.Policy("hobbit", t1=0.6, t2=0.9).levels_one(0, w)
    assert np.allclose(s, [0.0, 0.2034, 0.3641, 0.5034, 0.6327, 0.7580, 0.8646, 0.9677], atol=2e-4)
    assert [v == 0 for v in lvl] == [True] * 4 + [False] * 4 and skip == [False] * 7 + [True]
    pol = O.Policy("hobbit", t1=0.6, t1_layers={1: 0.0})
    assert pol.levels_one(1, [0.5, 0.3, 0.2])[0] == [0, 2, 2]
    assert pol.levels_one(0, [0.5, 0.3, 0.2])[0] == [0, 0, 2]
    assert O.Policy("hobbit", t1=0.3, t_mid=0.85, t2=0.9).levels_one(0, [0.5, 0.3, 0.15, 0.05])[:2] == \
        ([0, 1, 1, 2], [False, False, False, True])


def test_levels_one_differs_from_levels_at_a_threshold():
    """Weights that are exact binary fractions give s = [0, 0.5, 0.75] exactly in both rules. With
    t1 = 0.5 - 1e-6 - 1e-9 the float64 threshold t1 + 1e-6 = 0.499999999 lies below s = 0.5, but
    rounded to float32 (the tensor rule compares fp32 s against fp32(t1 + 1e-6)) it is 0.5: the
    tensor rule serves slot 1 at level 0 and the float64 rule at level 2."""
    t1 = 0.5 - 1e-6 - 1e-9
    assert np.float32(t1 + 1e-6) == np.float32(0.5) and t1 + 1e-6 < 0.5
    pol = O.Policy("hobbit", t1=t1)
    w = np.array([[0.5, 0.25, 0.25]], np.float32)
    assert pol.levels(0, w)[0][0].tolist() == [0, 0, 2]
    lvl, _, s = pol.levels_one(0, w[0])
    assert s == [0.0, 0.5, 0.75] and lvl == [0, 2, 2]


def test_t_mid_levels():
    w = np.array([[0.5, 0.3, 0.15, 0.05]], np.float32)  # s = 0, .5, .8, .95
    lvl, skip = O.Policy("hobbit", t1=0.3, t_mid=0.85, t2=0.9).levels(0, w)
    assert lvl[0].tolist() == [0, 1, 1, 2] and skip[0].tolist() == [False, False, False, True]


# -- router (transformers) ---------------------------------------------------------------
def _router_case(cls_name, dtype, renorm, E, k, H=64, T=256, seed=0):
    from transformers import OlmoeConfig, Qwen3NextConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeTopKRouter
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextTopKRouter

    if cls_name == "olmoe":
        cfg = OlmoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, norm_topk_prob=renorm)
        r = OlmoeTopKRouter(cfg)
    else:
        cfg = Qwen3NextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, norm_topk_prob=renorm)
        r = Qwen3NextTopKRouter(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        r.weight.copy_(torch.randn(E, H, generator=g) * 0.02)
    r = r.to(dtype)
    x = torch.randn(T, H, generator=g).to(dtype)
    with torch.no_grad():
        logits, scores, idx = r(x)
    return x, r.weight.detach(), logits, scores, idx


@pytest.mark.parametrize("cls_name,dtype,renorm,E,k", [
    ("olmoe", torch.float32, False, 64, 8), ("olmoe", torch.bfloat16, False, 64, 8),
    ("qwen3next", torch.float32, True, 512, 10), ("qwen3next", torch.bfloat16, True, 128, 8),
])
def test_router_matches_transformers(cls_name, dtype, renorm, E, k):
    x, W, logits, scores, idx = _router_case(cls_name, dtype, renorm, E, k)
    dn = {torch.float32: "float32", torch.bfloat16: "bfloat16"}[dtype]
    lo, oi, ow, _ = O.router(x.float().numpy(), W.float().numpy(), k, renorm, dn)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -20
    # logits agree to one rounding of the dtype (sum order differs)
    assert np.allclose(lo, logits.float().numpy(), rtol=ulp, atol=ulp)
    kth = -np.sort(-lo, axis=-1)[:, k - 1]
    ulp_k = np.exp2(np.floor(np.log2(np.abs(kth) + 1e-30))) * ulp  # one dtype ulp at the k-th logit
    clear = O.topk_margin(lo, k) > 2 * ulp_k
    assert clear.mean() > 0.5
    ti = idx.numpy()
    # same expert sets (torch.topk over probabilities may order equal values either way)
    for t in np.nonzero(clear)[0]:
        assert sorted(oi[t]) == sorted(ti[t]), t
        m = {int(e): float(v) for e, v in zip(ti[t], scores[t].float())}
        assert np.allclose([m[int(e)] for e in oi[t]], ow[t], rtol=ulp * 4, atol=1e-6)


def test_router_ties_lowest_index_first():
    """Planted ties: experts 2 and 5 (and 6, 7) have identical rows; the lower index wins."""
    H, E = 16, 8
    W = np.zeros((E, H), np.float32)
    W[:, 0] = [0.1, 0.9, 0.5, 0.2, 0.3, 0.5, 0.4, 0.4]
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 1.0
    _, idx, w, w32 = O.router(x, W, 3, False, "float32")
    assert idx[0].tolist() == [1, 2, 5]
    _, idx, _, _ = O.router(x, W, 2, False, "float32")
    assert idx[0].tolist() == [1, 2]
    _, idx, _, _ = O.router(x, W, 5, True, "float32")
    assert idx[0].tolist() == [1, 2, 5, 6, 7]
    p = np.exp(W[:, 0] - W[:, 0].max())
    p /= p.sum()
    _, _, _, w32 = O.router(x, W, 3, False, "float32")
    assert np.allclose(w32[0], p[[1, 2, 5]], rtol=1e-6)


# -- dispatch -----------------------------------------------------------------------------
def _dispatch_brute(idx, E, skip):
    T, k = idx.shape
    se, sp = [], []
    for e in range(E):
        for t in range(T):
            for j in range(k):
                if idx[t, j] == e and not (skip is not None and skip[t, j]):
                    se.append(e)
                    sp.append(t * k + j)
    return np.array(se, np.int64), np.array(sp, np.int64)


@pytest.mark.parametrize("T,k,E,with_skip", [(1, 8, 64, False), (8, 8, 64, True), (37, 3, 8, True), (5, 4, 16, False)])
def test_dispatch_matches_brute_force(T, k, E, with_skip):
    g = np.random.default_rng(T * 100 + k)
    idx = np.stack([g.choice(E, k, replace=False) for _ in range(T)])
    skip = g.random((T, k)) < 0.3 if with_skip else None
    se, sp, counts, offsets = O.dispatch(idx, E, skip)
    be, bp = _dispatch_brute(idx, E, skip)
    assert np.array_equal(se, be) and np.array_equal(sp, bp)
    assert counts.sum() == len(se) and offsets[-1] == len(se)
    assert np.array_equal(np.diff(offsets), counts)


# -- expert FFN + combine (transformers experts) ------------------------------------------
def _tiny_store(prec, H, I, E, seed):
    g = torch.Generator().manual_seed(seed)
    lay = O.record_layout(prec, H, I)
    blobs, mats = [], []
    for _ in range(E):
        gu = (torch.randn(2 * I, H, generator=g) * 0.1).numpy()
        dn = (torch.randn(H, I, generator=g) * 0.1).numpy()
        b = O.encode_record(lay, gu, dn, method="absmax")
        blobs.append(b)
        mats.append(O.materialize(lay, b, "float32"))
    return lay, blobs, mats


def test_moe_layer_matches_olmoe_experts():
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts

    H, I, E, k, T = 64, 32, 8, 3, 12
    lay, blobs, mats = _tiny_store("int4", H, I, E, 5)
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k)
    ex = OlmoeExperts(cfg).double()
    with torch.no_grad():
        for e in range(E):
            ex.gate_up_proj[e].copy_(torch.from_numpy(mats[e][0]))
            ex.down_proj[e].copy_(torch.from_numpy(mats[e][1]))
    g = torch.Generator().manual_seed(9)
    x = torch.randn(T, H, generator=g, dtype=torch.float64)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g, dtype=torch.float64)
    with torch.no_grad():
        ref = ex(x, idx, w).numpy()
    mine = O.moe_layer(x.numpy(), idx.numpy(), w.numpy(), lambda e: mats[e])
    assert np.allclose(mine, ref, rtol=1e-10, atol=1e-12)


def test_moe_layer_shared_expert_matches_qwen3next_block():
    from transformers import Qwen3NextConfig
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextSparseMoeBlock

    H, I, E, k, T = 64, 32, 16, 4, 10
    cfg = Qwen3NextConfig(hidden_size=H, moe_intermediate_size=I, shared_expert_intermediate_size=I, num_experts=E,
                          num_experts_per_tok=k, norm_topk_prob=True)
    blk = Qwen3NextSparseMoeBlock(cfg).double()
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float64) * 0.1)
    x = torch.randn(1, T, H, generator=g, dtype=torch.float64)
    with torch.no_grad():
        ref = blk(x)[0].numpy()
    Wr = blk.gate.weight.detach().numpy()
    _, idx, w, _ = O.router(x[0].numpy(), Wr, k, True, "float32")
    gu = blk.experts.gate_up_proj.detach().numpy()
    dn = blk.experts.down_proj.detach().numpy()
    se = blk.shared_expert
    shared = (np.concatenate([se.gate_proj.weight.detach().numpy(), se.up_proj.weight.detach().numpy()]),
              se.down_proj.weight.detach().numpy(), blk.shared_expert_gate.weight.detach().numpy()[0])
    # the module's softmax runs in float32 (dtype=torch.float), so weights agree to ~1e-7
    mine = O.moe_layer(x[0].numpy(), idx, w, lambda e: (gu[e], dn[e]), shared=shared)
    assert np.allclose(mine, ref, rtol=1e-5, atol=1e-7)


def test_cpu_expert_path_matches_float64_layer():
    H, I, E = 128, 64, 6
    lay, blobs, mats = _tiny_store("int4", H, I, E, 2)
    x = np.random.default_rng(1).standard_normal((1, H)).astype(np.float32)
    ws = [0.4, 0.3, 0.2, 0.1]
    got = O.cpu_expert_path(x, [("int4", blobs[e], ws[e]) for e in range(4)], {"int4": lay})
    ref = O.moe_layer(x, np.array([[0, 1, 2, 3]]), np.array([ws]), lambda e: mats[e])
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_moe_layer_grouped_matches_olmoe_experts():
    """The expert-by-expert evaluation (prefill order) against transformers' OlmoeExperts, with
    skipped pairs excluded like moe_layer."""
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts

    H, I, E, k, T = 64, 32, 8, 3, 20
    lay, blobs, mats = _tiny_store("int4", H, I, E, 6)
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k)
    ex = OlmoeExperts(cfg).double()
    with torch.no_grad():
        for e in range(E):
            ex.gate_up_proj[e].copy_(torch.from_numpy(mats[e][0]))
            ex.down_proj[e].copy_(torch.from_numpy(mats[e][1]))
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, H, generator=g, dtype=torch.float64)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g, dtype=torch.float64)
    with torch.no_grad():
        ref = ex(x, idx, w).numpy()
    mine = O.moe_layer_grouped(x.numpy(), idx.numpy(), w.numpy(), lambda e: mats[e])
    assert np.allclose(mine, ref, rtol=1e-10, atol=1e-12)
    skip = np.zeros((T, k), bool)
    skip[::3, 1] = True
    a = O.moe_layer_grouped(x.numpy(), idx.numpy(), w.numpy(), lambda e: mats[e], skip=skip)
    b = O.moe_layer(x.numpy(), idx.numpy(), w.numpy(), lambda e: mats[e], skip=skip)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-14)


def test_weight_threshold_rule():
    """The benchmark configurations' rule (fp16 if the gate weight is >= 0.15, else int4): level 0
    exactly at and above the threshold in fp32, never a skip; the host policy agrees, one token and
    batched, and packs the threshold without the HOBBIT slack."""
    import torch

    from moelab_hip.policy import PrecisionPolicy

    w = np.array([[0.3, np.float32(0.15), np.nextafter(np.float32(0.15), np.float32(0)), 0.0, 1.0]], np.float32)
    lvl, skip = O.Policy("weight", t1=0.15).levels(0, w)
    assert lvl.tolist() == [[0, 0, 2, 2, 0]] and not skip.any()
    pol = PrecisionPolicy("weight", t1=0.15)
    hl, hs = pol.levels(0, torch.from_numpy(w))
    assert hl.tolist() == lvl.tolist() and not hs.any()
    l1, s1, _ = pol.levels_one(0, w[0].tolist())
    assert l1 == lvl[0].tolist() and not any(s1)
    dp = pol.device_policy(3)
    assert dp.mode == 3 and dp.t1 == float(np.float32(0.15)) and dp.t2 < 0


# -- the CPU baseline's torch restatement (oracle/cpu_path.py) -------------------------------
def test_cpu_path_matches_the_oracle():
    """The torch restatement of the CPU expert branch dequantises byte-identically to the oracle
    and gives the oracle's layer output (fp32 vs float64 accumulation)."""
    import torch

    from oracle import cpu_path as C

    rng = np.random.default_rng(3)
    for prec in ("int4", "int8", "fp16"):
        lay = O.record_layout(prec, 256, 128, 64, scale="absmax" if prec != "fp16" else None)
        blobs, mats = [], []
        for _ in range(3):
            b = O.encode_record(lay, (rng.standard_normal((256, 256)) * 0.02).astype(np.float32),
                                (rng.standard_normal((256, 128)) * 0.02).astype(np.float32))
            blobs.append(b)
            mats.append(O.materialize(lay, b))
            g, d = C.materialize(lay, torch.from_numpy(b))
            assert np.array_equal(g.numpy(), mats[-1][0]) and np.array_equal(d.numpy(), mats[-1][1])
        x = rng.standard_normal((1, 256)).astype(np.float16)
        w = [0.5, 0.3, 0.2]
        got = C.cpu_layer(torch.from_numpy(x), [(prec, torch.from_numpy(b), wi) for b, wi in zip(blobs, w)], {prec: lay})
        ref = O.moe_layer(x.astype(np.float32), np.array([[0, 1, 2]]), np.array([w]), lambda e: mats[e])
        assert np.abs(got.numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
