"""Seeded generators of the five benchmark configurations (BASELINE configs C1-C5).

Frozen choices (they fix the inputs every later measurement and golden hash uses):
  * numpy default_rng(seed) with seeds 1001..1005; values float_to_bf16_bits(standard_normal);
    alpha = default_alpha(128); draw order q, k, v unless stated;
  * C1: the 64 queries are the last 64 positions of a 1024-key sequence: row r attends [0, 961 + r);
  * C2: paged NHD cache [pages, 16, 8, 128], pages in a seeded permutation, block table (32, 256);
  * C3: one causal sequence, row t attends [0, t];
  * C4: per sequence a 16-node draft tree; node 0 hangs off the prefix, node i > 0 takes a parent
    uniform in 0..i-1, redrawn until its depth is at most 5; node keys sit after the prefix;
  * C5: kv lengths integers(8192, 131072, endpoint=True); per KV head 4 distinct channels of k are
    scaled by 30 before rounding; k and v are drawn per sequence (k then v) to bound host memory.
"""

from __future__ import annotations

import numpy as np

from . import problem
from .formats import default_alpha_bits, float_to_bf16_bits

D = 128
HQ, HKV = 16, 8


def _bf16(rng, shape, scale=1.0):
    return float_to_bf16_bits(rng.standard_normal(shape, dtype=np.float64) * scale)


def alpha_bits() -> int:
    return default_alpha_bits(D)


def c1() -> dict:
    rng = np.random.default_rng(1001)
    q = _bf16(rng, (64, D))
    k = _bf16(rng, (1024, D))
    v = _bf16(rng, (1024, D))
    kv_len = 961 + np.arange(64)
    p = problem.contiguous(q.reshape(1, 64, 1, D), k.reshape(1, 1, 1024, D), v.reshape(1, 1, 1024, D),
                           kv_len.reshape(1, 64))
    p["name"] = "C1"
    return p


def c2(page_size: int = 16, layout: str = "NHD") -> dict:
    rng = np.random.default_rng(1002)
    B, S = 32, 4096
    q = _bf16(rng, (B, 1, HQ, D))
    k = _bf16(rng, (B, HKV, S, D))
    v = _bf16(rng, (B, HKV, S, D))
    base = problem.contiguous(q, k, v, np.full((B, 1), S))
    p = problem.to_paged(base, page_size, rng, layout=layout, extra_pages=0)
    p["name"] = "C2"
    return p


def c3(T: int = 4096) -> dict:
    rng = np.random.default_rng(1003)
    q = _bf16(rng, (1, T, HQ, D))
    k = _bf16(rng, (1, HKV, T, D))
    v = _bf16(rng, (1, HKV, T, D))
    p = problem.contiguous(q, k, v, (np.arange(T) + 1).reshape(1, T))
    p["name"] = "C3"
    return p


def draft_tree(rng, n_nodes: int = 16, max_depth: int = 5) -> list[int]:
    """parent[i] for i < n_nodes; -1 = the prefix tail."""
    parent = [-1]
    depth = [1]
    for i in range(1, n_nodes):
        while True:
            p = int(rng.integers(0, i))
            if depth[p] + 1 <= max_depth:
                break
        parent.append(p)
        depth.append(depth[p] + 1)
    return parent


def path_of(parent: list[int], i: int) -> list[int]:
    out = []
    while i != -1:
        out.append(i)
        i = parent[i]
    return out[::-1]


def c4(B: int = 8, prefix: int = 8192, nodes: int = 16) -> dict:
    rng = np.random.default_rng(1004)
    parents = [draft_tree(rng, nodes) for _ in range(B)]
    S = prefix + nodes
    q = _bf16(rng, (B, nodes, HQ, D))
    k = _bf16(rng, (B, HKV, S, D))
    v = _bf16(rng, (B, HKV, S, D))
    mask = np.zeros((B, nodes), dtype=np.uint64)
    for b in range(B):
        for i in range(nodes):
            m = 0
            for a in path_of(parents[b], i):
                m |= 1 << a
            mask[b, i] = m
    p = problem.contiguous(q, k, v, np.full((B, nodes), prefix), tree_mask=mask, tree_base=np.full(B, prefix))
    p["name"] = "C4"
    p["parents"] = parents
    return p


def c5(page_size: int = 16, B: int = 16, lo: int = 8192, hi: int = 131072, lens=None) -> dict:
    rng = np.random.default_rng(1005)
    if lens is None:
        lens = rng.integers(lo, hi, size=B, endpoint=True).astype(np.int32)
    outl = np.stack([rng.choice(D, size=4, replace=False) for _ in range(HKV)])
    q = _bf16(rng, (B, 1, HQ, D))
    npp = (int(lens.max()) + page_size - 1) // page_size
    pages_per = [(int(n) + page_size - 1) // page_size for n in lens]
    n_pages = sum(pages_per)
    perm = rng.permutation(n_pages)
    bt = np.zeros((B, npp), dtype=np.int32)
    kp = np.zeros((n_pages, page_size, HKV, D), dtype=np.uint16)
    vp = np.zeros((n_pages, page_size, HKV, D), dtype=np.uint16)
    scale = np.ones((HKV, D))
    for h in range(HKV):
        scale[h, outl[h]] = 30.0
    pos = 0
    for b in range(B):
        n = int(lens[b])
        kb = float_to_bf16_bits(rng.standard_normal((n, HKV, D)) * scale[None])
        vb = _bf16(rng, (n, HKV, D))
        for j in range(pages_per[b]):
            pg = int(perm[pos + j])
            bt[b, j] = pg
            s0, s1 = j * page_size, min(n, (j + 1) * page_size)
            kp[pg, :s1 - s0] = kb[s0:s1]
            vp[pg, :s1 - s0] = vb[s0:s1]
        pos += pages_per[b]
    p = problem.paged(q, kp, vp, bt, lens.reshape(B, 1), lens, "NHD")
    p["name"] = "C5"
    p["outlier_channels"] = outl
    return p


def c5_repage(p: dict, page_size: int) -> dict:
    """The C5 problem with the same keys stored in pages of another size (same page order)."""
    g = p["geom"]
    B, Hkv, d = g["num_seqs"], g["num_kv_heads"], g["head_dim"]
    P0 = g["page_size"]
    lens = p["seq_len"]
    npp = (int(lens.max()) + page_size - 1) // page_size
    pages_per = [(int(n) + page_size - 1) // page_size for n in lens]
    kp = np.zeros((sum(pages_per), page_size, Hkv, d), dtype=np.uint16)
    vp = np.zeros_like(kp)
    bt = np.zeros((B, npp), dtype=np.int32)
    pos = 0
    for b in range(B):
        n = int(lens[b])
        idx = np.arange(n)
        src_pages = p["block_table"][b][idx // P0]
        kb = p["k"][src_pages, idx % P0]
        vb = p["v"][src_pages, idx % P0]
        for j in range(pages_per[b]):
            bt[b, j] = pos + j
            s0, s1 = j * page_size, min(n, (j + 1) * page_size)
            kp[pos + j, :s1 - s0] = kb[s0:s1]
            vp[pos + j, :s1 - s0] = vb[s0:s1]
        pos += pages_per[b]
    out = problem.paged(p["q"], kp, vp, bt, lens.reshape(B, 1), lens, "NHD")
    out["name"] = p["name"]
    return out


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}
