"""
Oracle: a CPU restatement of moelab's MoE-layer algorithm, used ONLY as a checker.

This package is test infrastructure. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only to compute expected results or to
time the reference's CPU expert path. The product (`moe-offload-lab_amd/moelab_hip`)
never imports it and never falls back to it.

Everything is numpy (float64/float32/float16 and integer arithmetic), restated from the
reference's files, each function citing the file:line it follows:

- quant.py      int4/int8 group-size quantisation, packing, dequantize, FP8 block dequant
- store.py      record layout / encode / views / materialize
- policy.py     HOBBIT unimportance, levels, vote, level_to_precision
- router        transformers' OlmoeTopKRouter / Qwen3MoeTopKRouter / Qwen3NextTopKRouter
- runtime.py    dispatch (_decide_general), expert_ffn, combine, the CPU expert branch

`oracle/cpu_path.py` restates the CPU expert branch (runtime.py:646-702) in torch for bench.py's
reported CPU baseline; tests/test_oracle.py checks it against moe_ref.

Pinning (what fixes each function independently of this restatement) is listed in
`oracle/moe_ref.py`'s module docstring.
"""

from .moe_ref import *  # noqa: F401,F403
