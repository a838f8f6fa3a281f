"""
CPU restatement (numpy) of moelab's MoE-layer hot path — the checker for the HIP kernels.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg. Never imported by the product.

Each function cites the reference file:line it restates (moelab is read as text, never
imported). Numerics follow the reference exactly where the reference fixes them (fp16 scale
rounding, round-half-to-even, fp16 dequantisation products) and use float64 where the
reference's own reduction order is implementation-defined (F.linear, index_add_).

How each part is pinned (tests/test_oracle.py):
- int4/int8 packing + unpack: the reference's known answer (tests/test_units.py:33-38,
  w=[7,-7] -> byte 0x1F), brute force over all 256 byte values, quantize/dequantize
  round-trip tolerances of tests/test_units.py:19-30 on the same torch-seeded inputs.
- absmax scales: closed form on hand-made groups (zero group -> fp16(1e-7), exact powers of two).
- mse scales: known answer of tests/test_requant.py:35-42 (scale -1.0), and the invariant of
  tests/test_requant.py:21-33 (never worse than absmax, group by group).
- GPTQ: the reference's property test (tests/test_requant.py:45-60: at least 15 % less output
  error than mse on correlated inputs), a diagonal Hessian (no error to carry: exactly the mse
  quantisation), dead columns (zero weights), and Hinv against its definition (U^T U = H^-1).
- record layout: the record sizes computed independently for the three model shapes, 4096-B
  record alignment (tests/test_units.py:49-60), round trips at the reference tolerances.
- FP8 e4m3fn decode: all 256 codes against torch.float8_e4m3fn (a library routine).
- HOBBIT: the known answer of tests/test_units.py:168-187 (docs/06 example) and
  tests/test_optim.py:116-136 (per-layer t1, level_to_precision).
- router: transformers' OlmoeTopKRouter / Qwen3NextTopKRouter run on the same inputs
  (library routine), ties excluded; closed-form cases with planted ties (lowest index wins).
- dispatch: a brute-force loop formulation on small inputs.
- expert FFN + combine: transformers' OlmoeExperts.forward and Qwen3NextSparseMoeBlock
  (shared expert + sigmoid gate) on the dequantised weights (library routine).
"""

from __future__ import annotations

import math

import numpy as np

# ----------------------------------------------------------------------------------------
# Small float helpers (bfloat16 is not a numpy dtype)
# ----------------------------------------------------------------------------------------


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even (torch's .to(bfloat16))."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to `dtype` ('float16' | 'bfloat16' | 'float32'), returned as float32."""
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_bf16(np.asarray(x, dtype=np.float32))
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


def fp8_e4m3fn_to_f32(code: np.ndarray) -> np.ndarray:
    """OCP float8 e4m3fn decode (sign, 4-bit exponent with bias 7, 3-bit mantissa, no inf,
    S.1111.111 = NaN). Textbook formula; pinned against torch.float8_e4m3fn for all codes."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int32)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    sub = m.astype(np.float64) / 8.0 * 2.0 ** -6
    nor = (1.0 + m.astype(np.float64) / 8.0) * np.exp2(e.astype(np.float64) - 7.0)
    v = s * np.where(e == 0, sub, nor)
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return v.astype(np.float32)


def f32_to_fp8_e4m3fn(x: np.ndarray) -> np.ndarray:
    """Nearest e4m3fn code (ties to even); |x| above the largest finite value (448) saturates.
    Only used to build FP8 fixtures (checkpoint-like inputs), never to check kernels."""
    table = fp8_e4m3fn_to_f32(np.arange(256, dtype=np.uint8))
    pos = np.arange(0, 127, dtype=np.uint8)  # +0 .. +448 (code 127 is NaN)
    pv = table[pos].astype(np.float64)
    a = np.abs(np.asarray(x, dtype=np.float64)).clip(0, 448.0)
    i = np.searchsorted(pv, a)  # pv[i-1] < a <= pv[i]
    i = i.clip(1, len(pv) - 1)
    lo, hi = pv[i - 1], pv[i]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((pos[i] & 1) == 0))
    code = np.where(pick_hi, pos[i], pos[i - 1]).astype(np.uint8)
    code = np.where(a == 0, 0, code).astype(np.uint8)
    neg = np.signbit(np.asarray(x, dtype=np.float64)) & (code != 0)
    return (code | np.where(neg, 0x80, 0)).astype(np.uint8)


# ----------------------------------------------------------------------------------------
# quant.py
# ----------------------------------------------------------------------------------------

QMAX = {8: 127, 4: 7}  # quant.py:43
QMIN = {8: -127, 4: -8}  # quant.py:44
_GRID = [1.0 - 0.02 * i for i in range(16)]  # quant.py:46


def pick_group_size(in_features: int, preferred: int = 64) -> int:
    """quant.py:49-54: largest even group size <= preferred dividing in_features."""
    for gs in range(min(preferred, in_features), 1, -1):
        if in_features % gs == 0 and gs % 2 == 0:
            return gs
    raise ValueError(f"no even group size divides {in_features}")


def bits_per_weight(bits: int, group_size: int) -> float:
    """quant.py:222-224."""
    return bits + 16 / group_size


def _safe(s: np.ndarray) -> np.ndarray:
    """quant.py:57-61: scale rounded to fp16 (the stored value), never zero (fp16(1e-7))."""
    s16 = np.asarray(s, dtype=np.float32).astype(np.float16)
    return np.where(s16 == 0, np.float16(1e-7), s16)


def choose_scales(wf: np.ndarray, bits: int, method: str = "absmax") -> np.ndarray:
    """quant.py:64-93. wf (..., gs) float32 -> fp16 scales (..., 1)."""
    qmin, qmax = QMIN[bits], QMAX[bits]
    wf = np.asarray(wf, dtype=np.float32)
    absmax = np.abs(wf).max(axis=-1, keepdims=True)
    if method == "absmax":
        return _safe(np.maximum(absmax / np.float32(qmax), np.float32(1e-7)))
    if method != "mse":
        raise ValueError(method)
    bases = [absmax / np.float32(qmax)]
    if qmin == -qmax - 1:  # int4: the largest-magnitude weight lands on -8 (quant.py:78-80)
        mx = np.take_along_axis(wf, np.abs(wf).argmax(axis=-1)[..., None], axis=-1)
        bases.append(mx / np.float32(qmin))
    best_s = best_e = None
    for b in bases:
        for f in _GRID:
            s = _safe(b * np.float32(f))
            sf = s.astype(np.float32)
            q = np.clip(np.rint(wf / sf), qmin, qmax)
            err = ((q * sf - wf) ** 2).sum(axis=-1, keepdims=True, dtype=np.float32)
            if best_s is None:
                best_s, best_e = s, err
            else:
                better = err < best_e  # strict: the first best candidate is kept
                best_s = np.where(better, s, best_s)
                best_e = np.where(better, err, best_e)
    return best_s


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """quant.py:96-101: int8 as is; int4 stored q+8, low nibble = even column."""
    if bits == 8:
        return np.ascontiguousarray(q.astype(np.int8))
    u = (q + 8).astype(np.uint8)
    return np.ascontiguousarray(u[:, 0::2] | (u[:, 1::2] << 4))


def quantize(w: np.ndarray, bits: int, group_size: int, method: str = "absmax"):
    """quant.py:104-127 -> (packed q, fp16 scales (out, in/gs))."""
    w = np.asarray(w, dtype=np.float32)
    out_f, in_f = w.shape
    if in_f % group_size:
        raise ValueError("in_features not divisible by group_size")
    wf = w.reshape(out_f, in_f // group_size, group_size)
    s = choose_scales(wf, bits, method)
    q = np.clip(np.rint(wf / s.astype(np.float32)), QMIN[bits], QMAX[bits]).astype(np.int16)
    return pack(q.reshape(out_f, in_f), bits), np.ascontiguousarray(s.reshape(out_f, in_f // group_size))


def gptq_hinv(hessian: np.ndarray, damp: float = 0.01):
    """quant.py:151-166: dead columns (zero diagonal) get H[d, d] = 1, then damp * mean(diag) on
    the diagonal (again on each failed factorisation, up to 6 tries); Hinv = the upper Cholesky
    factor of H^-1, float32 throughout. Returns (Hinv, dead) or (None, dead) when every try
    failed (the reference then falls back to plain `quantize`). The factorisations are LAPACK's
    (numpy), so Hinv agrees with torch's to rounding, not bit for bit."""
    H = np.array(hessian, dtype=np.float32, copy=True)
    dead = np.diag(H) == 0
    H[dead, dead] = 1.0
    add = np.float32(damp) * np.float32(np.mean(np.diag(H), dtype=np.float32))
    H[np.diag_indices_from(H)] += add
    for _ in range(6):
        try:
            L = np.linalg.cholesky(H.astype(np.float32))
            Li = np.linalg.inv(L).astype(np.float32)
            Hi_full = (Li.T @ Li).astype(np.float32)  # (L L^T)^-1, what cholesky_inverse(L) returns
            U = np.linalg.cholesky(Hi_full).T.astype(np.float32)  # upper=True: Hi_full = U^T U
            if not np.all(np.isfinite(U)):
                raise np.linalg.LinAlgError("non-finite factor")
            return np.ascontiguousarray(U), dead
        except np.linalg.LinAlgError:
            add = np.float32(damp) * np.float32(np.mean(np.diag(H), dtype=np.float32))
            H[np.diag_indices_from(H)] += add
    return None, dead


def gptq_sweep(W1: np.ndarray, Hi: np.ndarray, bits: int, group_size: int, method: str = "mse"):
    """quant.py:172-186, one block of columns: left to right, a group's scale is chosen (on the
    weights as corrected so far) at its first column; q = rint(col / s) clamped; err = (col -
    q s) / Hi[i, i]; the columns from i on lose err * Hi[i, i:] (each product and difference
    rounded to float32). W1 (out, nb) float32 is updated in place. Returns (q int16 (out, nb),
    scales fp16 (out, nb / gs), E1 float32 (out, nb))."""
    qmin, qmax = QMIN[bits], QMAX[bits]
    out_f, nb = W1.shape
    Q = np.zeros((out_f, nb), np.int16)
    S = np.zeros((out_f, nb // group_size), np.float16)
    E1 = np.zeros((out_f, nb), np.float32)
    sf = None
    for i in range(nb):
        if i % group_size == 0:
            sc = choose_scales(W1[:, None, i:i + group_size], bits, method).reshape(-1)
            S[:, i // group_size] = sc
            sf = sc.astype(np.float32)
        col = W1[:, i].copy()
        q = np.clip(np.rint(col / sf), qmin, qmax).astype(np.float32)
        Q[:, i] = q.astype(np.int16)
        err = ((col - q * sf) / Hi[i, i]).astype(np.float32)
        W1[:, i:] -= (err[:, None] * Hi[i, i:][None, :]).astype(np.float32)
        E1[:, i] = err
    return Q, S, E1


def gptq_quantize(w: np.ndarray, hessian: np.ndarray, bits: int, group_size: int, method: str = "mse",
                  damp: float = 0.01, block: int = 128):
    """quant.py:130-188 (GPTQ, Frantar et al. 2023, in the store's format) -> (packed q, fp16
    scales (out, in/gs)). The lazy update of the columns right of a block is one float32 matrix
    product (BLAS order)."""
    W = np.array(w, dtype=np.float32, copy=True)
    out_f, in_f = W.shape
    if in_f % group_size or block % group_size:
        raise ValueError("in_features and block must be multiples of group_size")
    Hinv, dead = gptq_hinv(hessian, damp)
    if Hinv is None:
        return quantize(w, bits, group_size, method)
    W[:, dead] = 0.0
    Q = np.zeros((out_f, in_f), np.int16)
    S = np.zeros((out_f, in_f // group_size), np.float16)
    for i1 in range(0, in_f, block):
        i2 = min(i1 + block, in_f)
        W1 = W[:, i1:i2].copy()
        q, sc, E1 = gptq_sweep(W1, Hinv[i1:i2, i1:i2], bits, group_size, method)
        Q[:, i1:i2] = q
        S[:, i1 // group_size:i2 // group_size] = sc
        W[:, i2:] -= (E1 @ Hinv[i1:i2, i2:]).astype(np.float32)
    return pack(Q, bits), S


def unpack_int4(q: np.ndarray) -> np.ndarray:
    """Stored nibbles -> signed int values in [-8, 7] (quant.py:197-199), (O, 2*P) int8."""
    q = np.asarray(q, dtype=np.uint8)
    out = np.empty((q.shape[0], q.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = (q & 0x0F).astype(np.int8) - 8
    out[:, 1::2] = (q >> 4).astype(np.int8) - 8
    return out


def dequantize(q: np.ndarray, s: np.ndarray, bits: int, dtype: str = "float32") -> np.ndarray:
    """quant.py:191-205. The product q*s is rounded to `dtype` (exact in float32)."""
    if bits == 8:
        vals = np.asarray(q).view(np.int8).astype(np.float32)
    elif bits == 4:
        vals = unpack_int4(q).astype(np.float32)
    else:
        raise ValueError(bits)
    out_f, in_f = vals.shape
    gs = in_f // s.shape[1]
    sc = round_to(np.asarray(s, dtype=np.float16).astype(np.float32), dtype)
    prod = vals.reshape(out_f, in_f // gs, gs) * sc[:, :, None]
    return round_to(prod, dtype).reshape(out_f, in_f)


def dequantize_fp8_block(w_code: np.ndarray, scale_inv: np.ndarray, block=(128, 128)) -> np.ndarray:
    """quant.py:208-219: W = w_fp8 * scale_inv[r // bo, c // bi] (the scale MULTIPLIES)."""
    bo, bi = block
    out_f, in_f = w_code.shape
    exp = (math.ceil(out_f / bo), math.ceil(in_f / bi))
    if tuple(scale_inv.shape) != exp:
        raise ValueError(f"fp8 scales {scale_inv.shape}, expected {exp}")
    s = np.repeat(np.repeat(np.asarray(scale_inv, np.float32), bo, 0)[:out_f], bi, 1)[:, :in_f]
    return fp8_e4m3fn_to_f32(w_code) * s


def quantize_fp8_block(w: np.ndarray, block=(128, 128)):
    """Checkpoint-style FP8 block quantisation used to build fixtures: scale = amax/448 per
    128x128 block (the reference's fixture, tests/conftest.py:52-75)."""
    bo, bi = block
    w = np.asarray(w, dtype=np.float32)
    O, I = w.shape
    so, si = math.ceil(O / bo), math.ceil(I / bi)
    scale = np.zeros((so, si), np.float32)
    code = np.zeros((O, I), np.uint8)
    for a in range(so):
        for b in range(si):
            blk = w[a * bo:(a + 1) * bo, b * bi:(b + 1) * bi]
            amax = np.float32(np.abs(blk).max())
            sc = np.float32(amax / np.float32(448.0)) if amax > 0 else np.float32(1.0)
            scale[a, b] = sc
            code[a * bo:(a + 1) * bo, b * bi:(b + 1) * bi] = f32_to_fp8_e4m3fn(blk / sc)
    return code, scale


# ----------------------------------------------------------------------------------------
# store.py: record layout
# ----------------------------------------------------------------------------------------

ALIGN = 4096  # store.py:36
FIELD_ALIGN = 64  # store.py:37
PRECISIONS = {  # store.py:39-45 (+ "fp8": block-scaled e4m3fn, a record kind the reference lacks)
    "fp32": {"kind": "float", "dtype": "float32"},
    "fp16": {"kind": "float", "dtype": "float16"},
    "bf16": {"kind": "float", "dtype": "bfloat16"},
    "int8": {"kind": "int", "bits": 8},
    "int4": {"kind": "int", "bits": 4},
    "fp8": {"kind": "fp8"},
}
ELEM_SIZE = {"float32": 4, "float16": 2, "bfloat16": 2, "int8": 1, "uint8": 1}
FP8_BLOCK = 128


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def record_layout(prec: str, hidden: int, inter: int, group_size: int = 64, scale: str | None = None) -> dict:
    """store.py:76-115 (same dict shape: precision, fields [name, shape, dtype, offset],
    record_bytes, group_sizes, scale). fp8: [gate_up.q (2I,H) e4m3 bytes, gate_up.s (ceil(2I/128),
    ceil(H/128)) f32, down.q (H,I), down.s (ceil(H/128), ceil(I/128)) f32], same alignment rules."""
    spec = PRECISIONS[prec]
    if spec["kind"] == "int" and scale is None:
        scale = "mse" if spec["bits"] == 4 else "absmax"
    mats = {"gate_up": (2 * inter, hidden), "down": (hidden, inter)}
    raw = []
    groups = {}
    if spec["kind"] == "float":
        for name, shape in mats.items():
            raw.append((name, shape, spec["dtype"]))
    elif spec["kind"] == "fp8":
        for name, (o, i) in mats.items():
            raw.append((f"{name}.q", (o, i), "uint8"))
            raw.append((f"{name}.s", (math.ceil(o / FP8_BLOCK), math.ceil(i / FP8_BLOCK)), "float32"))
    else:
        bits = spec["bits"]
        for name, (o, i) in mats.items():
            gs = pick_group_size(i, group_size)
            groups[name] = gs
            raw.append((f"{name}.q", (o, i) if bits == 8 else (o, i // 2), "int8" if bits == 8 else "uint8"))
            raw.append((f"{name}.s", (o, i // gs), "float16"))
    fields, off = [], 0
    for name, shape, dtype in raw:
        nb = ELEM_SIZE[dtype] * int(np.prod(shape))
        fields.append([name, list(shape), dtype, off])
        off = _align(off + nb, FIELD_ALIGN)
    lay = {"precision": prec, "fields": fields, "record_bytes": _align(off, ALIGN), "group_sizes": groups}
    if spec["kind"] == "int":
        lay["scale"] = scale
    return lay


def field(layout: dict, name: str):
    for n, shape, dtype, off in layout["fields"]:
        if n == name:
            return tuple(shape), dtype, off
    raise KeyError(name)


_NP = {"float32": np.float32, "float16": np.float16, "int8": np.int8, "uint8": np.uint8, "bfloat16": np.uint16}


def encode_record(layout: dict, gate_up: np.ndarray, down: np.ndarray, method: str | None = None) -> np.ndarray:
    """store.py:122-150: bytes of one record from float32 weights (bf16 stored as raw bits)."""
    prec = layout["precision"]
    spec = PRECISIONS[prec]
    buf = np.zeros(layout["record_bytes"], dtype=np.uint8)
    t = {}
    if spec["kind"] == "float":
        dt = spec["dtype"]
        for name, w in (("gate_up", gate_up), ("down", down)):
            w = np.asarray(w, np.float32)
            t[name] = bf16_bits(w) if dt == "bfloat16" else w.astype(_NP[dt])
    elif spec["kind"] == "fp8":
        for name, w in (("gate_up", gate_up), ("down", down)):
            t[f"{name}.q"], t[f"{name}.s"] = quantize_fp8_block(w)
    else:
        m = method or layout.get("scale") or "absmax"
        m = "absmax" if m == "gptq" else m
        for name, w in (("gate_up", gate_up), ("down", down)):
            t[f"{name}.q"], t[f"{name}.s"] = quantize(w, spec["bits"], layout["group_sizes"][name], m)
    for name, shape, dtype, off in layout["fields"]:
        a = np.ascontiguousarray(t[name])
        if tuple(a.shape) != tuple(shape):
            raise ValueError(f"{name}: {a.shape} != {shape}")
        raw = a.view(np.uint8).reshape(-1)
        buf[off:off + raw.size] = raw
    return buf


def views(layout: dict, blob: np.ndarray) -> dict:
    """store.py:153-161: typed zero-copy views into a record."""
    out = {}
    for name, shape, dtype, off in layout["fields"]:
        nb = ELEM_SIZE[dtype] * int(np.prod(shape))
        out[name] = blob[off:off + nb].view(_NP[dtype]).reshape(shape)
    return out


def materialize(layout: dict, blob: np.ndarray, dtype: str = "float32"):
    """store.py:164-174: record -> (gate_up, down) as float32 arrays holding `dtype` values."""
    v = views(layout, blob)
    spec = PRECISIONS[layout["precision"]]
    if spec["kind"] == "float":
        def f(a, name):
            src = bf16_to_f32(a) if spec["dtype"] == "bfloat16" else a.astype(np.float32)
            return round_to(src, dtype)
        return f(v["gate_up"], "gate_up"), f(v["down"], "down")
    if spec["kind"] == "fp8":
        return (round_to(dequantize_fp8_block(v["gate_up.q"], v["gate_up.s"]), dtype),
                round_to(dequantize_fp8_block(v["down.q"], v["down.s"]), dtype))
    bits = spec["bits"]
    return (dequantize(v["gate_up.q"], v["gate_up.s"], bits, dtype),
            dequantize(v["down.q"], v["down.s"], bits, dtype))


# ----------------------------------------------------------------------------------------
# policy.py: HOBBIT precision levels
# ----------------------------------------------------------------------------------------


def unimportance(weights: np.ndarray) -> np.ndarray:
    """policy.py:77-87: s = sum of the normalised weights of the better-ranked experts."""
    w = np.asarray(weights, dtype=np.float32)
    w = w / np.maximum(w.sum(axis=-1, keepdims=True, dtype=np.float32), np.float32(1e-12))
    order = np.argsort(-w, axis=-1, kind="stable")
    sw = np.take_along_axis(w, order, axis=-1)
    s_sorted = np.cumsum(sw, axis=-1, dtype=np.float32) - sw
    s = np.empty_like(s_sorted)
    np.put_along_axis(s, order, s_sorted, axis=-1)
    return s


class Policy:
    """policy.py:20-72 (the fields the level rule reads)."""

    def __init__(self, mode="hobbit", t1=0.6, t2=None, protect_layers=(), hi_vote=0.5, t_mid=None, t1_layers=None):
        self.mode, self.t1, self.t2, self.t_mid = mode, t1, t2, t_mid
        self.protect_layers = frozenset(protect_layers)
        self.hi_vote = hi_vote
        self.t1_layers = dict(t1_layers) if t1_layers else None

    def t1_for(self, layer):  # policy.py:71-72
        return self.t1_layers.get(layer, self.t1) if self.t1_layers else self.t1

    def _fixed(self, layer):  # policy.py:103-108
        if self.mode == "hi" or layer in self.protect_layers:
            return 0
        if self.mode == "lo":
            return 2
        return None

    def levels(self, layer, weights):
        """policy.py:110-123 -> (levels (T,k) int8, skip (T,k) bool)."""
        w = np.asarray(weights, np.float32)
        T, k = w.shape
        none = np.zeros((T, k), bool)
        fixed = self._fixed(layer)
        if fixed is not None:
            return np.full((T, k), fixed, np.int8), none
        if self.mode == "weight":  # the benchmark configurations' rule (not in moelab): w >= t1 -> level 0
            return np.where(w >= np.float32(self.t1), 0, 2).astype(np.int8), none
        s = unimportance(w)
        lvl = np.full((T, k), 2, np.int8)
        if self.t_mid is not None:
            lvl[s <= np.float32(self.t_mid + 1e-6)] = 1
        lvl[s <= np.float32(self.t1_for(layer) + 1e-6)] = 0
        skip = (s > np.float32(self.t2 + 1e-6)) & (lvl != 0) if self.t2 is not None else none
        return lvl, skip

    def levels_one(self, layer, weights):
        """policy.py:89-98 + 125-137: the same rule for ONE token in float64 Python arithmetic
        (moelab's default decode path, runtime.py:494-517): total = sum of the weights, s = the
        exclusive running sum of weight / total in stable descending order, thresholds t + 1e-6 in
        float64. Returns (levels list, skip list, s list)."""
        ws = [float(v) for v in np.asarray(weights, np.float32).reshape(-1)]
        k = len(ws)
        fixed = self._fixed(layer)
        if fixed is not None:
            return [fixed] * k, [False] * k, [0.0] * k
        if self.mode == "weight":
            return [0 if np.float32(v) >= np.float32(self.t1) else 2 for v in ws], [False] * k, [0.0] * k
        total = sum(ws) or 1e-12
        s = [0.0] * k
        acc = 0.0
        for j in sorted(range(k), key=lambda j: -ws[j]):
            s[j] = acc
            acc += ws[j] / total
        t1 = self.t1_for(layer) + 1e-6
        tm = None if self.t_mid is None else self.t_mid + 1e-6
        lvl = [0 if v <= t1 else (1 if tm is not None and v <= tm else 2) for v in s]
        if self.t2 is None:
            return lvl, [False] * k, s
        return lvl, [v > self.t2 + 1e-6 and lv != 0 for v, lv in zip(s, lvl)], s

    def expert_level(self, token_levels) -> int:
        """policy.py:148-154: most precise level requested by >= hi_vote of the expert's tokens."""
        tl = np.asarray(token_levels)
        n = tl.size
        for level in (0, 1):
            if (tl <= level).sum() >= (self.hi_vote - 1e-9) * n:
                return level
        return 2


def level_to_precision(level: int, precisions: list) -> str:
    """policy.py:188-192."""
    if len(precisions) >= 3:
        return precisions[min(level, len(precisions) - 1)]
    return precisions[0] if level == 0 else precisions[-1]


# ----------------------------------------------------------------------------------------
# Router (transformers OlmoeTopKRouter.forward, modeling_olmoe.py:337-346; same code in
# Qwen3MoeTopKRouter and Qwen3NextTopKRouter)
# ----------------------------------------------------------------------------------------


def router(x: np.ndarray, W: np.ndarray, k: int, renorm: bool, dtype: str = "float16"):
    """logits = F.linear(x, W) in the model dtype (float64 sum, one rounding), probs = fp32
    softmax, top-k with the lowest index first on equal logits, optional renorm, cast to dtype.
    Returns (logits (T,E) float32 holding dtype values, idx (T,k) int64, w (T,k) float32
    holding dtype values, w32 (T,k) float32 before the cast)."""
    x64 = np.asarray(x, np.float64)
    W64 = np.asarray(W, np.float64)
    logits = round_to((x64 @ W64.T).astype(np.float64), dtype)
    l32 = logits.astype(np.float32)
    m = l32.max(axis=-1, keepdims=True)
    e = np.exp((l32 - m).astype(np.float64))
    probs = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    T, E = l32.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -l32), axis=-1)
    idx = order[:, :k].astype(np.int64)
    v = np.take_along_axis(probs, idx, axis=-1)
    if renorm:
        v = (v / v.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return logits, idx, round_to(v, dtype), v


def topk_margin(logits: np.ndarray, k: int) -> np.ndarray:
    """Per token: gap between the k-th and (k+1)-th largest logit (0 = a tie at the boundary)."""
    srt = -np.sort(-np.asarray(logits, np.float64), axis=-1)
    if srt.shape[-1] <= k:
        return np.full(srt.shape[0], np.inf)
    return srt[:, k - 1] - srt[:, k]


# ----------------------------------------------------------------------------------------
# runtime.py: dispatch, expert FFN, combine, CPU expert branch
# ----------------------------------------------------------------------------------------


def dispatch(idx: np.ndarray, E: int, skip: np.ndarray | None = None):
    """runtime.py:471-482 (_decide_general): drop skipped pairs, stable sort of the flat
    expert ids. Returns (sorted_e, sorted_pos = token*k + slot, counts (E,), offsets (E+1,))."""
    idx = np.asarray(idx, np.int64)
    T, k = idx.shape
    keep = np.ones(T * k, bool) if skip is None else ~np.asarray(skip, bool).reshape(-1)
    flat_e = idx.reshape(-1)[keep]
    flat_pos = np.arange(T * k)[keep]
    order = np.argsort(flat_e, kind="stable")
    se, sp = flat_e[order], flat_pos[order]
    counts = np.bincount(se, minlength=E)[:E].astype(np.int64)
    offsets = np.zeros(E + 1, np.int64)
    offsets[1:] = np.cumsum(counts)
    return se, sp, counts, offsets


def decide_general(policy: "Policy", layer: int, idx: np.ndarray, w32: np.ndarray, precisions: list):
    """runtime.py:459-492 (`_decide_general`, T > 1): per-token levels and skip
    (policy.levels, policy.py:110-123), then for every expert with kept pairs, in ascending id,
    the vote policy.expert_level over its pairs' levels (policy.py:148-154) and
    level_to_precision (policy.py:188-192). Returns (skip (T, k) bool, {expert: (level,
    precision)})."""
    idx = np.asarray(idx, np.int64)
    lvl, skip = policy.levels(layer, np.asarray(w32, np.float32))
    keep = ~np.asarray(skip, bool)
    out = {}
    for e in np.unique(idx[keep]):
        lev = policy.expert_level(lvl[(idx == e) & keep])
        out[int(e)] = (lev, level_to_precision(lev, precisions))
    return np.asarray(skip, bool), out


def silu(v):
    return v / (1.0 + np.exp(-v))


def expert_ffn(x: np.ndarray, gate_up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """runtime.py:165-168 with act = SiLU, in float64: down(silu(gate x) * up x)."""
    x = np.asarray(x, np.float64)
    gu = x @ np.asarray(gate_up, np.float64).T
    I = gu.shape[-1] // 2
    return (silu(gu[..., :I]) * gu[..., I:]) @ np.asarray(down, np.float64).T


def moe_layer(x, idx, w, weights_of, skip=None, shared=None):
    """out[t] = sum_j w[t,j] * expert(idx[t,j])(x[t])  (runtime.py:342-353; OlmoeExperts.forward,
    modeling_olmoe.py:301-325), plus optionally the Qwen3-Next shared expert
    sigmoid(x g) * FFN_s(x) (modeling_qwen3_next.py:786-797). `weights_of(e)` returns the
    (gate_up, down) float arrays of expert e; `shared` is (gate_up_s, down_s, g (H,)) or None.
    float64 result."""
    x = np.asarray(x, np.float64)
    idx = np.asarray(idx)
    w = np.asarray(w, np.float64)
    T, k = idx.shape
    out = np.zeros_like(x)
    cache = {}
    for t in range(T):
        for j in range(k):
            if skip is not None and skip[t, j]:
                continue
            e = int(idx[t, j])
            if e not in cache:
                cache[e] = weights_of(e)
            out[t] += w[t, j] * expert_ffn(x[t], *cache[e])
    if shared is not None:
        gu, dn, g = shared
        gate = 1.0 / (1.0 + np.exp(-(x @ np.asarray(g, np.float64))))
        out += gate[:, None] * expert_ffn(x, gu, dn)
    return out


def moe_layer_grouped(x, idx, w, weights_of, skip=None):
    """moe_layer for many tokens evaluated expert by expert (runtime.py:418-436: per expert
    y = expert_ffn(x[tok]) on the expert's tokens, then out.index_add_(tok, y * w),
    runtime.py:352-353): the same float64 result up to summation order."""
    x = np.asarray(x, np.float64)
    idx = np.asarray(idx)
    w = np.asarray(w, np.float64)
    out = np.zeros_like(x)
    keep = np.ones(idx.shape, bool) if skip is None else ~np.asarray(skip, bool)
    for e in np.unique(idx[keep]):
        tok, slot = np.nonzero((idx == e) & keep)
        y = expert_ffn(x[tok], *weights_of(int(e)))
        np.add.at(out, tok, w[tok, slot][:, None] * y)
    return out


def cpu_expert_path(x: np.ndarray, entries, layouts) -> np.ndarray:
    """The reference's CPU expert branch for one token (runtime.py:646-702, decode case):
    x in float32; per expert materialize(float32) -> expert_ffn -> out += w * y. `entries` is
    [(prec, blob, w)]. float32 arithmetic like the reference (torch fp32 on CPU)."""
    x = np.asarray(x, np.float32).reshape(1, -1)
    out = np.zeros_like(x)
    for prec, blob, wt in entries:
        gu, dn = materialize(layouts[prec], blob, "float32")
        g = x @ gu.T
        I = g.shape[-1] // 2
        h = (g[:, :I] / (np.float32(1) + np.exp(-g[:, :I]))) * g[:, I:]
        out += np.float32(wt) * (h @ dn.T)
    return out
