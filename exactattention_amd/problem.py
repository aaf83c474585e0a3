"""Serving-geometry problems: one description of queries, a (paged) KV cache and per-row key sets.

A problem is a plain dict of numpy arrays and integers, the host-side image of the C ABI's
ea_geometry + ea_buffers (include/exactattn_hip.h):

    geom            dict of the ea_geometry fields
    q               (B, T, Hq, d) uint16 bf16 bits (any strides are expressed through geom)
    k, v            KV cache storage (contiguous (B, Hkv, S, d) or a page pool)
    seq_len         (B,) int32 keys stored per sequence
    kv_len          (B*T,) int32 visible prefix per query token
    block_table     optional int32 page table, block_table_offset optional int64 per sequence
    tree_mask       optional (B*T,) uint64, tree_base (B,) int32
    out_shape       (B, T, Hq, dv)

Rows are (sequence, token, query head) in that order. The same dict drives the device library
and, in tests, the CPU oracle, so both see exactly the same inputs.
"""

from __future__ import annotations

import numpy as np


def _geom(B, T, Hq, Hkv, d, dv, q_strides, o_strides, k_strides, v_strides, page_size, bt_stride, max_seq_len):
    g = dict(num_seqs=B, num_tokens=T, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=d, head_dim_v=dv,
             q_seq_stride=q_strides[0], q_tok_stride=q_strides[1], q_head_stride=q_strides[2],
             o_seq_stride=o_strides[0], o_tok_stride=o_strides[1], o_head_stride=o_strides[2],
             k_page_stride=k_strides[0], k_slot_stride=k_strides[1], k_head_stride=k_strides[2],
             v_page_stride=v_strides[0], v_slot_stride=v_strides[1], v_head_stride=v_strides[2],
             page_size=page_size, block_table_stride=bt_stride, max_seq_len=max_seq_len)
    return {k: int(x) for k, x in g.items()}


def contiguous(q, k, v, kv_len, seq_len=None, tree_mask=None, tree_base=None):
    """q (B, T, Hq, d); k (B, Hkv, S, d); v (B, Hkv, S, dv); kv_len (B, T)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, T, Hq, d = q.shape
    _, Hkv, S, dv = v.shape
    kv_len = np.ascontiguousarray(np.asarray(kv_len, dtype=np.int32).reshape(B * T))
    seq_len = np.full(B, S, np.int32) if seq_len is None else np.ascontiguousarray(seq_len, dtype=np.int32)
    g = _geom(B, T, Hq, Hkv, d, dv, (T * Hq * d, Hq * d, d), (T * Hq * dv, Hq * dv, dv),
              (Hkv * S * d, d, S * d), (Hkv * S * dv, dv, S * dv), 1, 0, S)
    return dict(geom=g, q=q, k=k, v=v, seq_len=seq_len, kv_len=kv_len, block_table=None, block_table_offset=None,
                tree_mask=None if tree_mask is None else np.ascontiguousarray(tree_mask, dtype=np.uint64).reshape(-1),
                tree_base=None if tree_base is None else np.ascontiguousarray(tree_base, dtype=np.int32),
                out_shape=(B, T, Hq, dv))


def paged(q, k_pages, v_pages, block_table, kv_len, seq_len, layout="NHD", tree_mask=None, tree_base=None):
    """Paged cache. NHD pages: (num_pages, page_size, Hkv, d); HND: (num_pages, Hkv, page_size, d).
    block_table (B, max_pages) int32."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k_pages = np.ascontiguousarray(k_pages, dtype=np.uint16)
    v_pages = np.ascontiguousarray(v_pages, dtype=np.uint16)
    B, T, Hq, d = q.shape
    dv = v_pages.shape[-1]
    if layout == "NHD":
        _, P, Hkv, _ = k_pages.shape
        ks = (P * Hkv * d, Hkv * d, d)
        vs = (P * Hkv * dv, Hkv * dv, dv)
    elif layout == "HND":
        _, Hkv, P, _ = k_pages.shape
        ks = (Hkv * P * d, d, P * d)
        vs = (Hkv * P * dv, dv, P * dv)
    else:
        raise ValueError(layout)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    seq_len = np.ascontiguousarray(seq_len, dtype=np.int32)
    g = _geom(B, T, Hq, Hkv, d, dv, (T * Hq * d, Hq * d, d), (T * Hq * dv, Hq * dv, dv), ks, vs, P, bt.shape[1],
              int(seq_len.max(initial=0)))
    return dict(geom=g, q=q, k=k_pages, v=v_pages, seq_len=seq_len,
                kv_len=np.ascontiguousarray(np.asarray(kv_len, dtype=np.int32).reshape(B * T)),
                block_table=bt, block_table_offset=None,
                tree_mask=None if tree_mask is None else np.ascontiguousarray(tree_mask, dtype=np.uint64).reshape(-1),
                tree_base=None if tree_base is None else np.ascontiguousarray(tree_base, dtype=np.int32),
                out_shape=(B, T, Hq, dv))


def csr(q, k, v, layout: dict) -> dict:
    """The reference CPU ABI's form (csrc/exact_attention_cpu.cpp:585-588: q (R, d), k (n, d),
    v (n, dv), row r attends key_idx[row_ptr[r]:row_ptr[r+1]]) as the serving geometry the
    library's ea_csr_layout gives it (`layout` from hip.csr_layout(..., arrays=True)): each
    key-list family is a sequence whose tokens are its rows and whose pages are runs of
    `page_size` keys of k and v. Token i of the flattened (B, T) grid is CSR row
    layout["tok_row"][i] (-1: padding, kv_len 0)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    d, dv = q.shape[1], v.shape[1]
    B, T, P = layout["num_seqs"], layout["num_tokens"], layout["page_size"]
    tok = layout["tok_row"]
    qg = np.zeros((B * T, d), np.uint16)
    qg[tok >= 0] = q[tok[tok >= 0]]
    n = k.shape[0]
    npages = max(1, -(-n // P))
    kp = np.zeros((npages * P, d), np.uint16)
    vp = np.zeros((npages * P, dv), np.uint16)
    kp[:n], vp[:n] = k, v
    g = _geom(B, T, 1, 1, d, dv, (T * d, d, 0), (T * dv, dv, 0), (P * d, d, 0), (P * dv, dv, 0), P, 0,
              layout["max_seq_len"])
    return dict(geom=g, q=qg.reshape(B, T, 1, d), k=kp.reshape(npages, P, 1, d), v=vp.reshape(npages, P, 1, dv),
                seq_len=np.ascontiguousarray(layout["seq_len"], dtype=np.int32),
                kv_len=np.ascontiguousarray(layout["kv_len"], dtype=np.int32),
                block_table=np.ascontiguousarray(layout["block_table"], dtype=np.int32),
                block_table_offset=np.ascontiguousarray(layout["bt_off"], dtype=np.int64),
                tree_mask=None, tree_base=None, out_shape=(B, T, 1, dv))


def to_paged(prob: dict, page_size: int, rng: np.random.Generator, layout: str = "NHD", extra_pages: int = 3) -> dict:
    """The same problem (same keys per sequence) stored in a shuffled page pool."""
    g = prob["geom"]
    if prob["block_table"] is not None:
        raise ValueError("to_paged takes a contiguous problem")
    B, Hkv, d, dv = g["num_seqs"], g["num_kv_heads"], g["head_dim"], g["head_dim_v"]
    S = prob["k"].shape[2]
    k, v = prob["k"], prob["v"]
    npp = -(-S // page_size)
    n_pages = B * npp + extra_pages
    perm = rng.permutation(n_pages)
    bt = perm[:B * npp].reshape(B, npp).astype(np.int32)
    shape_k = (n_pages, page_size, Hkv, d) if layout == "NHD" else (n_pages, Hkv, page_size, d)
    shape_v = (n_pages, page_size, Hkv, dv) if layout == "NHD" else (n_pages, Hkv, page_size, dv)
    # unused slots and pages hold finite junk (bf16 1.5), which no row may read
    kp = np.full(shape_k, 0x3FC0, dtype=np.uint16)
    vp = np.full(shape_v, 0x3FC0, dtype=np.uint16)
    pad = npp * page_size - S
    kk = np.pad(k, ((0, 0), (0, 0), (0, pad), (0, 0)), constant_values=0x3FC0)
    vv = np.pad(v, ((0, 0), (0, 0), (0, pad), (0, 0)), constant_values=0x3FC0)
    kk = kk.reshape(B, Hkv, npp, page_size, d)
    vv = vv.reshape(B, Hkv, npp, page_size, dv)
    if layout == "NHD":
        kp[bt.reshape(-1)] = kk.transpose(0, 2, 3, 1, 4).reshape(B * npp, page_size, Hkv, d)
        vp[bt.reshape(-1)] = vv.transpose(0, 2, 3, 1, 4).reshape(B * npp, page_size, Hkv, dv)
    else:
        kp[bt.reshape(-1)] = kk.transpose(0, 2, 1, 3, 4).reshape(B * npp, Hkv, page_size, d)
        vp[bt.reshape(-1)] = vv.transpose(0, 2, 1, 3, 4).reshape(B * npp, Hkv, page_size, dv)
    kv_len = prob["kv_len"].reshape(B, -1)
    return paged(prob["q"], kp, vp, bt, kv_len, prob["seq_len"], layout, prob["tree_mask"], prob["tree_base"])


def flat_rows(prob: dict, out: np.ndarray) -> np.ndarray:
    """(rows, dv) view of an output array in row order (sequence, token, query head)."""
    return np.asarray(out).reshape(-1, prob["geom"]["head_dim_v"])
