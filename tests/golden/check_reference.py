"""Cross-checks the committed golden hashes (baseline_sha256.json, made by make_golden.py with the
oracle) against the reference's own certified C++ kernel, compiled from the reference checkout
into oracle/_ref (csrc/exact_attention_cpu.cpp, ea_attention_cpu :585-628). Every configuration
is converted to the kernel's CSR form (row_ptr/key_idx over per-(sequence, KV head) key rows);
rows the reference kernel flags (flag 1) are recomputed with the exact definition
(oracle/exact.py), as the reference's host tier does (src/exactattn/cpu.py:105-108).

    python tests/golden/check_reference.py [C1 C2 ...]

Records "reference_cpp_equal" and "reference_flagged_rows" per configuration. Needs oracle/_ref
(built by `make -C oracle` where /root/reference exists); test infrastructure only.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)

from exactattention_amd import configs  # noqa: E402
from oracle import exact, oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(__file__), "baseline_sha256.json")


def kv_rows(p: dict, which: str, b: int, hk: int, n: np.ndarray) -> np.ndarray:
    """K or V rows of keys n of sequence b, KV head hk, through the geometry's address formula."""
    g = p["geom"]
    pre = "k" if which == "k" else "v"
    d = g["head_dim"] if which == "k" else g["head_dim_v"]
    if p.get("block_table") is not None:
        ps = g["page_size"]
        off = (p["block_table_offset"][b] if p.get("block_table_offset") is not None
               else b * g["block_table_stride"])
        page = p["block_table"].reshape(-1)[off + n // ps].astype(np.int64)
        slot = (n % ps).astype(np.int64)
    else:
        page = np.full(n.shape, b, np.int64)
        slot = n.astype(np.int64)
    base = page * g[f"{pre}_page_stride"] + slot * g[f"{pre}_slot_stride"] + hk * g[f"{pre}_head_stride"]
    flat = p[which].reshape(-1)
    return flat[base[:, None] + np.arange(d)[None, :]]


def to_csr(p: dict):
    g = p["geom"]
    B, T, Hq, Hkv = g["num_seqs"], g["num_tokens"], g["num_q_heads"], g["num_kv_heads"]
    grp = Hq // Hkv
    seq = p["seq_len"].astype(np.int64)
    seg_base = np.zeros(B * Hkv + 1, np.int64)
    seg_base[1:] = np.cumsum(np.repeat(seq, Hkv))
    K = np.empty((int(seg_base[-1]), g["head_dim"]), np.uint16)
    V = np.empty((int(seg_base[-1]), g["head_dim_v"]), np.uint16)
    for b in range(B):
        n = np.arange(seq[b])
        for hk in range(Hkv):
            s = b * Hkv + hk
            K[seg_base[s]:seg_base[s + 1]] = kv_rows(p, "k", b, hk, n)
            V[seg_base[s]:seg_base[s + 1]] = kv_rows(p, "v", b, hk, n)
    q = p["q"].reshape(B * T * Hq, -1)
    lens, idx = [], []
    for b in range(B):
        for t in range(T):
            tok = b * T + t
            keys = np.arange(int(p["kv_len"][tok]), dtype=np.int64)
            if p.get("tree_mask") is not None:
                m = int(p["tree_mask"][tok])
                tk = np.array([int(p["tree_base"][b]) + i for i in range(64) if (m >> i) & 1], np.int64)
                keys = np.concatenate([keys, tk])
            for hq in range(Hq):
                idx.append(seg_base[b * Hkv + hq // grp] + keys)
                lens.append(keys.size)
    row_ptr = np.zeros(len(lens) + 1, np.int64)
    row_ptr[1:] = np.cumsum(lens)
    key_idx = np.concatenate(idx) if idx else np.zeros(0, np.int64)
    return q, K, V, row_ptr, key_idx


def main(names):
    if not oracle.ref_available():
        sys.exit("oracle/_ref is not built (make -C oracle, with the reference checkout present)")
    data = json.load(open(OUT))
    ab = configs.alpha_bits()
    for name in names:
        t0 = time.time()
        p = configs.CONFIGS[name]()
        q, K, V, rp, ki = to_csr(p)
        del p
        t1 = time.time()
        res, flags, _ = oracle.raw_csr(q, K, V, ab, rp, ki, "bf16", 64, 64, 8, 0, os.cpu_count(), reference=True)
        t2 = time.time()
        for r in np.flatnonzero(flags):
            keys = ki[rp[r]:rp[r + 1]]
            res[r] = exact.attention_row(q[r], K[keys], V[keys], ab)
        h = hashlib.sha256(np.ascontiguousarray(res).tobytes()).hexdigest()
        ok = h == data[name]["sha256"]
        data[name]["reference_cpp_equal"] = bool(ok)
        data[name]["reference_flagged_rows"] = int((flags != 0).sum())
        print(name, "reference C++ kernel:", "EQUAL" if ok else "DIFFERENT", h[:16], f"csr {t1 - t0:.1f}s",
              f"kernel {t2 - t1:.1f}s", f"flagged {int((flags != 0).sum())}", flush=True)
        with open(OUT, "w") as f:
            json.dump(data, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:] or ["C1", "C2", "C3", "C4", "C5"])
