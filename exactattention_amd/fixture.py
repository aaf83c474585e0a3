"""Fixture check on real activations (the reference's scripts/fixture.py `check` mode, :36-59 and
:110-124): every causal row of each fixture head goes through the GPU library, the bf16 output
is hashed with SHA-256 over its contiguous uint16 bytes, and the hash is compared with the
published one.

    python -m exactattention_amd.fixture check --backend hip:rocm [--only 0_0,27_11]

The fixture (Qwen3-0.6B q/k/v heads on WikiText-2, 2048 rows each) and its expected hashes are
the reference's data files, kept under tests/golden/.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
FIXTURE = os.path.join(ROOT, "tests", "golden", "qwen3_0.6b_heads.npz")
EXPECTED = os.path.join(ROOT, "tests", "golden", "expected_sha256.json")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_backend(backend: str, q, k, v, alpha):
    """Causal rows: row r attends keys [0, r + 1). Returns (out uint16 (L, dv), flags)."""
    kind, _, dev = backend.partition(":")
    if kind != "hip":
        raise ValueError(f"backend {backend!r}: this package provides hip:rocm only")
    from . import attention_hip
    L = q.shape[0]
    return attention_hip(q, k, v, alpha, kv_len=np.arange(1, L + 1), splits=8, device="cuda")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["check"])
    ap.add_argument("--backend", default="hip:rocm")
    ap.add_argument("--only", default="")
    ap.add_argument("--fixture", default=FIXTURE)
    ap.add_argument("--expected", default=EXPECTED)
    args = ap.parse_args(argv)
    z = np.load(args.fixture)
    expected = json.load(open(args.expected))
    only = set(args.only.split(",")) if args.only else None
    print(f"host {platform.node()} | {platform.processor() or platform.machine()} | backend {args.backend}")
    ok = True
    for key, info in expected["heads"].items():
        if only is not None and key not in only:
            continue
        q, k, v = z[f"q_{key}"], z[f"k_{key}"], z[f"v_{key}"]
        alpha = np.float32(z[f"alpha_{key}"])
        t0 = time.perf_counter()
        out, flags = run_backend(args.backend, q, k, v, alpha)
        dt = time.perf_counter() - t0
        h = sha(out)
        match = h == info["sha256"]
        ok &= match
        print(f"head {key}: {'MATCH' if match else 'MISMATCH'} sha256 {h[:16]}...  ({dt:.1f}s, "
              f"{int((flags != 0).sum())} fallback rows)", flush=True)
    print("ALL MATCH" if ok else "MISMATCH")
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
