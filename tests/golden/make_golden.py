"""Writes tests/golden/baseline_sha256.json: SHA-256 of the output bits of the five benchmark
configurations (exactattention_amd.configs), computed by the CPU oracle (C restatement of the
reference's certified kernel, Python exact definition for the rows it flags), plus the number
of rows the oracle's certified path left to the exact definition.

    python tests/golden/make_golden.py [C1 C2 ...]

C1 is additionally recomputed row by row with the pure-Python definition.
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


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main(names):
    data = json.load(open(OUT)) if os.path.exists(OUT) else {}
    ab = configs.alpha_bits()
    for name in names:
        t0 = time.time()
        p = configs.CONFIGS[name]()
        t1 = time.time()
        out, flags = oracle.attention_geom(p, ab, "bf16", splits=1, tile=64)
        t2 = time.time()
        entry = {"sha256": sha(out), "rows": int(flags.size), "oracle_flagged_rows": int((flags != 0).sum()),
                 "shape": list(out.shape), "gen_s": round(t1 - t0, 1), "oracle_s": round(t2 - t1, 1)}
        if name == "C1":
            for r in range(flags.size):
                qr, K, V = oracle.row_keys(p, r)
                assert np.array_equal(out.reshape(-1, out.shape[-1])[r], exact.attention_row(qr, K, V, ab))
            entry["python_exact_rows_checked"] = int(flags.size)
        if name == "C5":
            p64 = configs.c5_repage(p, 64)
            out64, _ = oracle.attention_geom(p64, ab, "bf16", splits=3, tile=64)
            assert np.array_equal(out64, out), "page size 64 disagrees"
            entry["page64_same_bits"] = True
        data[name] = entry
        print(name, entry, flush=True)
        with open(OUT, "w") as f:
            json.dump(data, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:] or ["C1", "C2", "C3", "C4", "C5"])
