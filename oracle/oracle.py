"""CPU oracle, part 3: ctypes bindings and the combined checker.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).

* `liboracle.so` (oracle/ea_oracle.c): the reference's certified CPU algorithm restated in C.
* `_ref/libexactattn_cpu.so`: the reference's own csrc/exact_attention_cpu.cpp, compiled from
  the reference checkout by oracle/Makefile (absent when the checkout was not available).
* `attention_csr` / `attention_geom`: run the C oracle and recompute every flagged row with the
  Python exact oracle (oracle/exact.py), mirroring src/exactattn/cpu.py:70-109. Every returned
  row is exactly the spec's value; domain errors raise exact.DomainError.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import exact

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libexactattn_cpu.so")

_lib = None
_ref = None
P = ctypes.c_void_p


class Geom(ctypes.Structure):
    """Serving geometry; same field order and meaning as the GPU library's ea_geometry."""
    _fields_ = [(n, ctypes.c_int32) for n in ("num_seqs", "num_tokens", "num_q_heads", "num_kv_heads",
                                              "head_dim", "head_dim_v")] + \
               [(n, ctypes.c_int64) for n in ("q_seq_stride", "q_tok_stride", "q_head_stride",
                                              "o_seq_stride", "o_tok_stride", "o_head_stride",
                                              "k_page_stride", "k_slot_stride", "k_head_stride",
                                              "v_page_stride", "v_slot_stride", "v_head_stride")] + \
               [(n, ctypes.c_int32) for n in ("page_size", "block_table_stride", "max_seq_len", "pad0")]


class GBufs(ctypes.Structure):
    _fields_ = [(n, P) for n in ("q", "k", "v", "seq_len", "kv_len", "block_table", "block_table_offset",
                                 "tree_mask", "tree_base", "out", "flags")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        lib.ea_attention_cpu.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_float, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P, P, P]
        lib.ea_attention_cpu.restype = ctypes.c_int
        lib.oracle_attention_geom.argtypes = [ctypes.POINTER(Geom), ctypes.POINTER(GBufs), ctypes.c_uint32,
                                              ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_uint64, ctypes.c_int, P]
        lib.oracle_attention_geom.restype = ctypes.c_int
        lib.oracle_round_ratio_bits.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_int)]
        lib.oracle_round_ratio_bits.restype = ctypes.c_uint32
        lib.oracle_weight.argtypes = [ctypes.c_uint32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)]
        lib.oracle_weight.restype = ctypes.c_int
        lib.oracle_logit.argtypes = [P, P, ctypes.c_int, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]
        lib.oracle_logit.restype = ctypes.c_int
        lib.oracle_ln2.argtypes = [P]
        _lib = lib
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def _load_ref():
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_LIB)
        lib.ea_attention_cpu.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_float, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P, P, P]
        lib.ea_attention_cpu.restype = ctypes.c_int
        _ref = lib
    return _ref


def _alpha_f32(alpha_bits: int) -> np.float32:
    return np.array([alpha_bits], dtype=np.uint32).view(np.float32)[0]


def csr_from_kv_len(kv_len) -> tuple[np.ndarray, np.ndarray]:
    kv_len = np.asarray(kv_len, dtype=np.int64)
    row_ptr = np.concatenate([[0], np.cumsum(kv_len)]).astype(np.int64)
    key_idx = np.concatenate([np.arange(n, dtype=np.int64) for n in kv_len]) if len(kv_len) else np.zeros(0, np.int64)
    return row_ptr, key_idx


def raw_csr(q, k, v, alpha_bits, row_ptr=None, key_idx=None, out="bf16", acc_bits=64, tile=64, splits=1,
            order_seed=0, threads=None, reference=False):
    """One call of ea_attention_cpu (the oracle's, or the reference's with reference=True).
    Returns (out bits, flags, stats) without any fallback."""
    lib = _load_ref() if reference else _load()
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    rows, d = q.shape
    n, dv = v.shape
    if row_ptr is None:
        row_ptr = np.arange(rows + 1, dtype=np.int64) * n
        key_idx = np.tile(np.arange(n, dtype=np.int64), rows)
    row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int64)
    key_idx = np.ascontiguousarray(key_idx, dtype=np.int64)
    fp32 = out == "fp32"
    res = np.zeros((rows, dv), dtype=np.uint32 if fp32 else np.uint16)
    flags = np.zeros(rows, dtype=np.uint8)
    st = np.zeros(3, dtype=np.int64)
    threads = threads or os.cpu_count() or 1
    rc = lib.ea_attention_cpu(q.ctypes.data, rows, d, k.ctypes.data, v.ctypes.data, n, dv,
                              ctypes.c_float(float(_alpha_f32(alpha_bits))), row_ptr.ctypes.data,
                              key_idx.ctypes.data, int(fp32), acc_bits, tile, splits, order_seed, threads,
                              res.ctypes.data, flags.ctypes.data, st.ctypes.data)
    if rc != 0:
        raise ValueError(f"ea_attention_cpu: invalid arguments (code {rc})")
    return res, flags, st


def attention_csr(q, k, v, alpha_bits, row_ptr=None, key_idx=None, out="bf16", acc_bits=64, tile=64, splits=1,
                  order_seed=0, threads=None):
    """Spec bits for every row of a CSR mask: C oracle, then the Python exact oracle for flagged rows
    (src/exactattn/cpu.py:70-109). Raises exact.DomainError if any row hits a domain error."""
    res, flags, st = raw_csr(q, k, v, alpha_bits, row_ptr, key_idx, out, acc_bits, tile, splits, order_seed, threads)
    if np.any(flags == 2):
        raise exact.DomainError("non-finite input or logit overflow")
    rows, n = q.shape[0], np.asarray(v).shape[0]
    if row_ptr is None:
        row_ptr = np.arange(rows + 1, dtype=np.int64) * n
        key_idx = np.tile(np.arange(n, dtype=np.int64), rows)
    for r in np.flatnonzero(flags):
        sel = np.asarray(key_idx)[row_ptr[r]:row_ptr[r + 1]]
        res[r] = exact.attention_row(q[r], np.asarray(k)[sel], np.asarray(v)[sel], alpha_bits, out)
    return res, flags


def _ptr(a):
    return None if a is None else a.ctypes.data


def raw_geom(prob: dict, alpha_bits: int, out="bf16", acc_bits=64, tile=64, splits=1, order_seed=0, threads=None):
    """The C oracle over a serving-geometry problem (see exactattention_amd.problem for the dict
    layout). Returns (out array shaped like the problem's output, flags per row, stats)."""
    lib = _load()
    g = Geom(**{f: int(prob["geom"][f]) for f, _ in Geom._fields_ if f != "pad0"})
    fp32 = out == "fp32"
    res = np.zeros(prob["out_shape"], dtype=np.uint32 if fp32 else np.uint16)
    rows = g.num_seqs * g.num_tokens * g.num_q_heads
    flags = np.zeros(rows, dtype=np.uint8)
    arrs = {k: (None if prob.get(k) is None else np.ascontiguousarray(prob[k])) for k in
            ("q", "k", "v", "seq_len", "kv_len", "block_table", "block_table_offset", "tree_mask", "tree_base")}
    b = GBufs(**{k: _ptr(a) for k, a in arrs.items()}, out=res.ctypes.data, flags=flags.ctypes.data)
    st = np.zeros(3, dtype=np.int64)
    threads = threads or os.cpu_count() or 1
    rc = lib.oracle_attention_geom(ctypes.byref(g), ctypes.byref(b), alpha_bits, int(fp32), acc_bits, tile, splits,
                                   order_seed, threads, st.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle_attention_geom: invalid arguments (code {rc})")
    return res, flags, st


def row_keys(prob: dict, row: int):
    """(q row, K rows, V rows) of one flattened row of a geometry problem, gathered in key order."""
    gm = prob["geom"]
    T, Hq, Hkv = gm["num_tokens"], gm["num_q_heads"], gm["num_kv_heads"]
    grp = Hq // Hkv
    b, t, hq = row // (T * Hq), (row // Hq) % T, row % Hq
    hk = hq // grp
    tok = b * T + t
    # visible keys: the prefix below min(kv_len, seq_len), then the tree keys at or past it and
    # below seq_len, each key once
    slen = int(prob["seq_len"][b])
    L = max(0, min(int(prob["kv_len"][tok]), slen))
    keys = list(range(L))
    if prob.get("tree_mask") is not None:
        m = int(prob["tree_mask"][tok])
        tb = int(prob["tree_base"][b])
        keys += [tb + i for i in range(64) if (m >> i) & 1 and L <= tb + i < slen]
    kflat, vflat, qflat = prob["k"].reshape(-1), prob["v"].reshape(-1), prob["q"].reshape(-1)
    d, dv = gm["head_dim"], gm["head_dim_v"]

    def addr(n, pfx):
        if prob.get("block_table") is not None:
            off = prob["block_table_offset"][b] if prob.get("block_table_offset") is not None \
                else b * gm["block_table_stride"]
            page = int(prob["block_table"].reshape(-1)[off + n // gm["page_size"]])
            slot = n % gm["page_size"]
        else:
            page, slot = b, n
        return page * gm[pfx + "_page_stride"] + slot * gm[pfx + "_slot_stride"] + hk * gm[pfx + "_head_stride"]

    K = np.array([kflat[addr(n, "k"):addr(n, "k") + d] for n in keys], dtype=np.uint16).reshape(-1, d)
    V = np.array([vflat[addr(n, "v"):addr(n, "v") + dv] for n in keys], dtype=np.uint16).reshape(-1, dv)
    qa = b * gm["q_seq_stride"] + t * gm["q_tok_stride"] + hq * gm["q_head_stride"]
    return qflat[qa:qa + d], K, V


def out_index(prob: dict, row: int):
    gm = prob["geom"]
    T, Hq = gm["num_tokens"], gm["num_q_heads"]
    return row // (T * Hq), (row // Hq) % T, row % Hq


def attention_geom(prob: dict, alpha_bits: int, out="bf16", acc_bits=64, tile=64, splits=1, order_seed=0,
                   threads=None):
    """Spec bits for every row of a serving-geometry problem: C oracle plus Python exact fallback.
    Returns (out shaped (B, T, Hq, dv), flags of the C oracle)."""
    res, flags, st = raw_geom(prob, alpha_bits, out, acc_bits, tile, splits, order_seed, threads)
    if np.any(flags == 2):
        raise exact.DomainError("non-finite input or logit overflow")
    flat = res.reshape(-1, res.shape[-1])
    for r in np.flatnonzero(flags):
        qrow, K, V = row_keys(prob, int(r))
        flat[r] = exact.attention_row(qrow, K, V, alpha_bits, out)
    return res, flags


def round_ratio_bits(a: int, b: int, E: int, neg: bool, fp32: bool):
    lib = _load()
    ov = ctypes.c_int(0)
    bits = lib.oracle_round_ratio_bits(a >> 64, a & ((1 << 64) - 1), b >> 64, b & ((1 << 64) - 1), E, int(neg),
                                       int(fp32), ctypes.byref(ov))
    return int(bits), bool(ov.value)


def weight(t_bits: int):
    lib = _load()
    M, E = ctypes.c_int32(0), ctypes.c_int64(0)
    ok = lib.oracle_weight(t_bits, ctypes.byref(M), ctypes.byref(E))
    return (int(M.value), int(E.value)) if ok else None


def logit_bits(q, k, alpha_bits: int):
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    t = ctypes.c_uint32(0)
    ok = lib.oracle_logit(q.ctypes.data, k.ctypes.data, q.shape[0], alpha_bits, ctypes.byref(t))
    return int(t.value) if ok else None


def ln2_126() -> tuple[int, int]:
    lib = _load()
    a = np.zeros(4, dtype=np.uint64)
    lib.oracle_ln2(a.ctypes.data)
    return (int(a[0]) << 64) | int(a[1]), (int(a[2]) << 64) | int(a[3])
