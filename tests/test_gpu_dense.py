"""
GPU parity of the dense-part int8 path (moelab/denseq.py): the one-token GEMV against the oracle's
dequantise-then-matvec in float64, the row-block dequantisation bit-exact against the oracle's
`dequantize(q, s, 8, dtype)`, and QLinear / quantize_dense through nn.Linear-shaped modules.

Shapes: OLMoE attention projections (2048 x 2048) and LM head (50304 x 2048), Qwen3-Next's LM head
(151936 x 2048), attention output (2048 x 4096: two row segments) and shared expert (gate_up
1024 x 2048, down 2048 x 512), plus ragged ones (rows not a multiple of a block, K = 96, groups of 48).
Bars: fp32 outputs within 1e-4 of max|ref| (the reference kernel test's bound), fp16 2e-3, bf16
1e-2 (one rounding of the output); the dequantised weights bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
from moelab_hip import denseq as D

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 1e-2}
NP = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _weights(O_, K, gs, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(O_, K, generator=g) * 0.02
    q, s = O.quantize(w.numpy(), 8, gs)
    return q, s


def _ref(q, s, x):
    return O.dequantize(q, s, 8, "float32").astype(np.float64) @ x.double().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("O_,K,gs", [(2048, 2048, 64), (50304, 2048, 64), (1024, 2048, 64), (2048, 512, 64),
                                     (2048, 4096, 64), (100, 96, 48), (33, 2048, 32)])
def test_dense_gemv_int8(dev, dtype, O_, K, gs):
    print(f"dense gemv O={O_} K={K} gs={gs} {dtype}", flush=True)
    q, s = _weights(O_, K, gs, O_ + K)
    x = torch.randn(K, generator=torch.Generator().manual_seed(K)).to(dtype)
    y = D.gemv_int8(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), x.to(dev), gs)
    assert y.dtype == dtype and y.shape == (O_,)
    ref = _ref(q, s, x)
    got = y.float().cpu().numpy()
    assert np.abs(got - ref).max() / np.abs(ref).max() < TOL[dtype]


def test_dense_gemv_int8_qwen3next_lm_head(dev):
    O_, K, gs = 151936, 2048, 64
    q, s = _weights(O_, K, gs, 3)
    x = torch.randn(K, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    y = D.gemv_int8(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), x.to(dev), gs)
    ref = _ref(q, s, x)
    assert np.abs(y.float().cpu().numpy() - ref).max() / np.abs(ref).max() < TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("O_,K,gs", [(300, 2048, 64), (64, 96, 48), (17, 512, 32)])
def test_dense_dequant_int8_bit_exact(dev, dtype, O_, K, gs):
    q, s = _weights(O_, K, gs, 9 + O_)
    w = D.dequantize_rows(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), dtype)
    ref = O.dequantize(q, s, 8, NP[dtype])
    got = w.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 7])
@pytest.mark.parametrize("bias", [False, True])
def test_qlinear_from_linear(dev, dtype, T, bias):
    g = torch.Generator().manual_seed(T)
    lin = nn.Linear(2048, 1536, bias=bias).to(dtype)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(1536, 2048, generator=g) * 0.02).to(dtype))
        if bias:
            lin.bias.copy_((torch.randn(1536, generator=g) * 0.1).to(dtype))
    ql = D.QLinear.from_linear(lin, dev)
    assert ql.group_size == 64 and ql.q.dtype == torch.int8 and ql.s.dtype == torch.float16
    q_ref, s_ref = O.quantize(lin.weight.detach().float().numpy(), 8, 64)
    assert np.array_equal(ql.q.cpu().numpy(), q_ref.view(np.int8))
    assert np.array_equal(ql.s.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    x = (torch.randn(1, T, 2048, generator=g)).to(dtype)
    y = ql(x.to(dev))
    assert y.shape == (1, T, 1536) and y.dtype == dtype
    wdq = O.dequantize(q_ref, s_ref, 8, "float32").astype(np.float64)
    ref = x.double().numpy() @ wdq.T
    if bias:
        ref = ref + lin.bias.detach().double().numpy()
    got = y.float().cpu().numpy()
    # T > 1: weights rounded to the activation dtype before F.linear, as the reference's prefill does
    tol = TOL[dtype] if T == 1 else 2e-2
    assert np.abs(got - ref).max() / np.abs(ref).max() < tol


def test_quantize_dense_swaps_the_dense_layers(dev):
    g = torch.Generator().manual_seed(0)
    model = nn.Sequential(nn.Linear(512, 1024), nn.GELU(), nn.Linear(1024, 512, bias=False), nn.Linear(512, 8))
    with torch.no_grad():
        for m in model:
            if isinstance(m, nn.Linear):
                m.weight.copy_(torch.randn(m.weight.shape, generator=g) * 0.05)
    x = torch.randn(1, 512, generator=g)
    ref = model(x).detach().double().numpy()
    total = D.linear_bytes(model)
    info = D.quantize_dense(model.to(dev), dev, log=lambda *a: None)
    assert info["layers"] == 2 and info["bytes_before"] == total  # the 8-output head stays nn.Linear
    assert isinstance(model[0], D.QLinear) and isinstance(model[2], D.QLinear) and isinstance(model[3], nn.Linear)
    got = model(x.to(dev)).detach().double().cpu().numpy()
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-2  # int8 weights against float ones
