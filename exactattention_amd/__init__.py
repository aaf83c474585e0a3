"""exactattention_amd: certified split-KV ExactAttention on AMD Instinct MI355X (gfx950).

The public names mirror the reference package (src/exactattn/__init__.py:3-14): `attention`,
`attention_row`, `default_alpha`, `float_to_bf16_bits`, `bf16_bits_to_float32`,
`ExactAttentionDomainError`, with the same signatures and bf16-bit-pattern dtypes. Here the rows
are computed on the GPU by hand-written HIP kernels (libexactattn_hip.so); every returned bit
equals the ExactAttention definition. `attention_hip` mirrors the reference's attention_triton /
attention_cpu backends (returns (out, flags)), and `launch_hip` the device-level launcher.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import problem
from .formats import (
    ExactAttentionDomainError,
    ExactAttentionUncertifiedError,
    bf16_bits_to_float32,
    default_alpha,
    alpha_fp32_bits,
    default_alpha_bits,
    float_to_bf16_bits,
)

__all__ = [
    "ExactAttentionDomainError",
    "ExactAttentionUncertifiedError",
    "attention",
    "attention_row",
    "attention_hip",
    "attention_geom",
    "bf16_bits_to_float32",
    "default_alpha",
    "float_to_bf16_bits",
    "launch_hip",
    "trace_row",
    "RowTrace",
]


def _alpha_bits(alpha, alpha_bits) -> int:
    """`alpha` is a value (numpy's float32 conversion, as the reference decodes it); a raw fp32
    pattern comes only through the keyword `alpha_bits`."""
    return alpha_fp32_bits(alpha, alpha_bits)


def _finish(res: np.ndarray, out: str) -> np.ndarray:
    return res.view(np.float32) if out == "fp32" else res


def attention_hip(q_bits, k_bits, v_bits, alpha=None, kv_len=None, row_ptr=None, key_idx=None, out: str = "bf16",
                  splits: int = 0, merge_order=None, fallback: bool = True, device: str = "cuda", *,
                  alpha_bits=None):
    """numpy-level GPU backend (mirrors src/exactattn/triton_kernels.py:1522-1560 and
    src/exactattn/cpu.py:70-109). q (R, d), k (n, d), v (n, dv) bf16 bits. Row r attends keys
    [0, kv_len[r]) (causal, decode, prefill), or key_idx[row_ptr[r]:row_ptr[r+1]] (any mask), or
    all keys. Returns (out, flags): out uint16 bf16 bits, or float32 for out="fp32". `alpha` is
    the fp32 scale as a value; `alpha_bits=` passes its bit pattern instead."""
    from .hip import attention_problem
    ab = _alpha_bits(alpha, alpha_bits)
    q = np.asarray(q_bits, dtype=np.uint16)
    k = np.asarray(k_bits, dtype=np.uint16)
    v = np.asarray(v_bits, dtype=np.uint16)
    R, n = q.shape[0], k.shape[0]
    if R == 0:
        # no query rows: an empty (0, dv) result, as the reference's attention() returns
        # (src/exactattn/reference.py:150-161); the library is still required
        from .hip import load
        load()
        empty = np.zeros((0, v.shape[1] if v.ndim == 2 else 0), np.uint32 if out == "fp32" else np.uint16)
        return _finish(empty, out), np.zeros(0, np.uint8)
    if row_ptr is None:
        # prefix rows: one segment of R tokens over one contiguous cache (shares K/V tiles)
        kv_len = np.full(R, n) if kv_len is None else np.asarray(kv_len, dtype=np.int64).reshape(R)
        if np.any(kv_len < 0) or np.any(kv_len > n):
            raise ValueError("kv_len must lie in [0, n]")
        prob = problem.contiguous(q.reshape(1, R, 1, -1), k.reshape(1, 1, n, -1), v.reshape(1, 1, n, -1),
                                  kv_len.reshape(1, R))
        res, flags, _ = attention_problem(prob, None, out, splits, merge_order, True, fallback, device, alpha_bits=ab)
        return _finish(res.reshape(R, -1), out), flags
    # CSR rows: rows whose key lists are prefixes of one list share a sequence (and its K/V reads),
    # as the C drop-in ea_attention_hip groups them; rows with no key are +0, certified
    from .hip import csr_layout
    row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int64)
    key_idx = np.ascontiguousarray(key_idx if key_idx is not None else np.zeros(0), dtype=np.int64)
    if row_ptr.shape != (R + 1,):
        raise ValueError("row_ptr must have rows + 1 entries")
    lay = csr_layout(row_ptr, key_idx, n, arrays=True)
    dv = v.shape[1]
    res = np.zeros((R, dv), np.uint32 if out == "fp32" else np.uint16)
    flags = np.zeros(R, np.uint8)
    if lay["num_seqs"] > 0:
        prob = problem.csr(q, k, v, lay)
        r, fl, _ = attention_problem(prob, None, out, splits, merge_order, True, fallback, device, alpha_bits=ab)
        tok = lay["tok_row"]
        m = tok >= 0
        res[tok[m]] = r.reshape(-1, dv)[m]
        flags[tok[m]] = fl[m]
    return _finish(res, out), flags


def attention_geom(prob: dict, alpha=None, out: str = "bf16", splits: int = 0, merge_order=None,
                   fallback: bool = True, device: str = "cuda", *, alpha_bits=None):
    """Serving-geometry problem (exactattention_amd.problem) on the GPU -> (out (B,T,Hq,dv), flags, stats)."""
    from .hip import attention_problem
    ab = _alpha_bits(alpha, alpha_bits)
    res, flags, st = attention_problem(prob, None, out, splits, merge_order, True, fallback, device, alpha_bits=ab)
    return _finish(res, out), flags, st


def attention(q_bits, k_bits, v_bits, alpha=None, mask=None, out: str = "bf16", *, alpha_bits=None) -> np.ndarray:
    """Batched attention (src/exactattn/reference.py:150-161): q (r, d), k (n, d), v (n, dv),
    mask (r, n) bool or None. Returns (r, dv) uint16 bf16 bits, or float32 for out="fp32".
    `alpha` is the fp32 scale as a value; `alpha_bits=` passes its bit pattern instead."""
    q = np.asarray(q_bits, dtype=np.uint16)
    if out not in ("bf16", "fp32"):
        raise ValueError("out must be 'bf16' or 'fp32'")
    ab = _alpha_bits(alpha, alpha_bits)
    if mask is None:
        res, _ = attention_hip(q, k_bits, v_bits, out=out, alpha_bits=ab)
        return res
    mask = np.asarray(mask, dtype=bool)
    counts = mask.sum(axis=1)
    row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    key_idx = np.concatenate([np.flatnonzero(m) for m in mask]).astype(np.int64) if mask.size else np.zeros(0, np.int64)
    res, _ = attention_hip(q, k_bits, v_bits, row_ptr=row_ptr, key_idx=key_idx, out=out, alpha_bits=ab)
    return res


def attention_row(q_bits, k_bits, v_bits, alpha=None, out: str = "bf16", *, alpha_bits=None) -> np.ndarray:
    """One query row over all given keys (src/exactattn/reference.py:146-147)."""
    q = np.asarray(q_bits, dtype=np.uint16).reshape(1, -1)
    k = np.asarray(k_bits, dtype=np.uint16).reshape(-1, q.shape[1])
    v = np.asarray(v_bits, dtype=np.uint16)
    v = v.reshape(k.shape[0], -1) if v.size else np.zeros((k.shape[0], v.shape[-1] if v.ndim else 0), np.uint16)
    return attention(q, k, v, alpha, out=out, alpha_bits=alpha_bits)[0]


@dataclass
class RowTrace:
    """Every intermediate of one row (the reference's RowTrace, src/exactattn/reference.py:63-71):
    exact scores s and weights w as (M, E) = M * 2**E, fp32 logits t as Python floats, the exact
    denominator Z and per-channel numerators N as (M, E), and the output bits."""
    s: list
    t: list
    w: list
    Z: tuple
    N: list
    out: np.ndarray


def _decode(bits: np.ndarray):
    b = np.asarray(bits, dtype=np.uint16).astype(np.int64)
    f = (b >> 7) & 0xFF
    if np.any(f == 0xFF):
        raise ExactAttentionDomainError("bf16 NaN or infinity in input")
    m = np.where(f != 0, (b & 0x7F) | 0x80, b & 0x7F) * np.where(b & 0x8000, -1, 1)
    return m, np.where(f != 0, f - 134, -133)


# The reference's limit on the spread of weight exponents in one row (src/exactattn/reference.py:30)
MAX_EXPONENT_SPREAD = 1 << 20


def trace_row(q_bits, k_bits, v_bits, alpha=None, out: str = "bf16", *, alpha_bits=None) -> RowTrace:
    """One row with every intermediate (src/exactattn/reference.py:82-143). The logits, weights
    and output bits come from the library's host exact tier (ea_exact_row); the exact scores and
    sums are assembled from them here with Python integers. Like the reference, a row whose
    weight exponents spread over more than 2^20 raises ExactAttentionDomainError
    (src/exactattn/reference.py:109-110), even where the output bits alone are decidable."""
    from .hip import exact_row
    if out not in ("bf16", "fp32"):
        raise ValueError("out must be 'bf16' or 'fp32'")
    q = np.asarray(q_bits, dtype=np.uint16).reshape(-1)
    d = q.shape[0]
    k = np.asarray(k_bits, dtype=np.uint16).reshape(-1, d)
    n = k.shape[0]
    v = np.asarray(v_bits, dtype=np.uint16)
    dv = v.shape[-1] if v.ndim == 2 else 0
    v = v.reshape(n, dv)
    res, tb, wm, we = exact_row(q, k, v, _alpha_bits(alpha, alpha_bits), out, trace=True)
    qm, qe = _decode(q)
    km, ke = _decode(k)
    vm, ve = _decode(v)
    s = []
    for j in range(n):
        pm, pe = (qm * km[j]).tolist(), (qe + ke[j]).tolist()
        terms = [(m_, e_) for m_, e_ in zip(pm, pe) if m_]
        if not terms:
            s.append((0, 0))
            continue
        e0 = min(e_ for _, e_ in terms)
        s.append((sum(m_ << (e_ - e0) for m_, e_ in terms), e0))
    t = [float(x) for x in np.asarray(tb, dtype=np.uint32).view(np.float32)]
    # The library saturates weight exponents at +-2^62 (logits of magnitude 2^100 and more); such a
    # logit is an integer, so its weight is exactly 2^t = 2^23 * 2^(t - 23).
    w = [(int(a), int(b)) if abs(int(b)) < (1 << 62) else (1 << 23, int(tj) - 23) for a, b, tj in zip(wm, we, t)]
    if n and max(e_ for _, e_ in w) - min(e_ for _, e_ in w) > MAX_EXPONENT_SPREAD:
        raise ExactAttentionDomainError("weight exponent spread exceeds reference limit")
    if n == 0:
        return RowTrace(s, t, w, (0, 0), [(0, 0)] * dv, res if out == "bf16" else res.view(np.float32))
    e0 = min(e_ for _, e_ in w)
    Z = (sum(m_ << (e_ - e0) for m_, e_ in w), e0)
    N = []
    for c in range(dv):
        terms = [(w[j][0] * int(vm[j, c]), w[j][1] + int(ve[j, c])) for j in range(n) if vm[j, c]]
        if not terms:
            N.append((0, 0))
            continue
        b0 = min(e_ for _, e_ in terms)
        N.append((sum(m_ << (e_ - b0) for m_, e_ in terms), b0))
    return RowTrace(s, t, w, Z, N, res if out == "bf16" else res.view(np.float32))


def launch_hip(*args, **kwargs):
    """Device-level launch on torch tensors (see exactattention_amd.hip.launch_hip)."""
    from .hip import launch_hip as _l
    return _l(*args, **kwargs)
