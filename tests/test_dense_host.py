"""CPU tests of the dense-part int8 module's host logic: which layers it takes (moelab's rule:
nn.Linear with >= 64 outputs and even in_features), their byte count, and that a QLinear refuses
an input that is not on the GPU (no computation elsewhere)."""

import pytest
import torch
import torch.nn as nn

from moelab_hip import denseq as D


def test_quantizable_follows_the_reference_rule():
    model = nn.Sequential(nn.Linear(64, 128), nn.Linear(128, 63), nn.Linear(33, 64), nn.Linear(128, 64))
    names = [n for n, _ in D.quantizable(model)]
    assert names == ["0", "3"]  # 63 outputs: too small; 33 inputs: odd
    assert D.linear_bytes(model) == (64 * 128 + 128 * 64) * 4


def test_qlinear_refuses_a_host_input():
    q = torch.zeros(64, 64, dtype=torch.int8)
    s = torch.ones(64, 1, dtype=torch.float16)
    ql = D.QLinear(q, s, 64, None, torch.float16)
    assert ql.kernel and ql.in_features == 64 and ql.out_features == 64
    with pytest.raises(RuntimeError, match="GPU"):
        ql(torch.zeros(1, 64, dtype=torch.float16))
