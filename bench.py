#!/usr/bin/env python
"""Benchmark of the certified split-KV attention path on one MI355X.

Workload: BASELINE config C2 (batched paged decode: B=32, 16 query / 8 KV heads, d=128, 4096 keys
per sequence, NHD pages of 16, one query token per sequence), inputs resident in HBM. One step =
one ea_hip_attention call (q prep, tier-1 split kernel, combine with certified rounding, tier 2).

Prints one JSON line: whole-step decode throughput in GB/s over the algorithmic bytes (bf16 K+V,
q, out, block table), the decode kernel's roofline fraction (HIP events on its launch stream
around back-to-back launches, the basis of a rocprofv3 trace average; the events around its
single launches inside the timed steps beside it), bit-exactness against the committed golden hash, the tier-1 fallback-row rate, and the
reference's own C++ certified CPU kernel (oracle/_ref, built from the reference source) timed on
this host's cores as the CPU baseline.

The "prefill" object holds config C3 (causal prefill, 4096 tokens, 16 query / 8 KV heads) on the
int8-MFMA prefill kernel: step time, algorithmic int8 ops (visible pairs x 6912) over the
ea_pf_main launch time as a fraction of the dense int8 MFMA peak, bit-exactness and fallback rows.
`--only C3` runs just that workload (for profiler runs).
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode KV GB/s & prefill int8-MFMA TOPS (% roofline), bit-exact, fallback-row %"
HBM_PEAK_GBS = 8000.0
GOLDEN = os.path.join(ROOT, "tests", "golden", "baseline_sha256.json")
TRAFFIC = os.path.join(ROOT, "profiles", "ea_decode_C2_traffic.md")


def algorithmic_bytes(prob: dict) -> int:
    """bf16 K+V of every visible key, q, out and the block table (per step)."""
    g = prob["geom"]
    B, Hkv, d, dv, Hq, T = (g[x] for x in ("num_seqs", "num_kv_heads", "head_dim", "head_dim_v", "num_q_heads",
                                          "num_tokens"))
    keys = int(prob["seq_len"].astype(np.int64).sum())
    kv = keys * Hkv * (d + dv) * 2
    q = B * T * Hq * d * 2
    out = B * T * Hq * dv * 2
    bt = 0 if prob.get("block_table") is None else int(prob["block_table"].size) * 4
    return kv + q + out + bt


class HipEvents:
    """Raw hipEvent_t handles (libamdhip64) so the library can record them on its launch stream."""

    def __init__(self, n: int):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = (ctypes.c_void_p * n)()
        for i in range(n):
            e = ctypes.c_void_p()
            rc = self.h.hipEventCreate(ctypes.byref(e))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate: {rc}")
            self.ev[i] = e
        self.n = n

    def slot(self, i: int):
        return ctypes.cast(ctypes.byref(self.ev, i * ctypes.sizeof(ctypes.c_void_p)), ctypes.c_void_p)

    def ms(self, a: int, b: int) -> float:
        rc = self.h.hipEventSynchronize(self.ev[b])
        t = ctypes.c_float(0)
        rc = rc or self.h.hipEventElapsedTime(ctypes.byref(t), self.ev[a], self.ev[b])
        if rc != 0:
            raise RuntimeError(f"HIP event timing: {rc}")
        return float(t.value)

    def close(self):
        for i in range(self.n):
            self.h.hipEventDestroy(self.ev[i])


def c2_csr(prob: dict):
    """C2 in the reference CPU ABI's CSR form: q (B*Hq, d); K, V rows of (sequence, KV head) s at
    s*S .. s*S + len - 1; rows (sequence, query head), each over its sequence's keys."""
    g = prob["geom"]
    B, Hkv, Hq, d, dv = g["num_seqs"], g["num_kv_heads"], g["num_q_heads"], g["head_dim"], g["head_dim_v"]
    P = g["page_size"]
    S = int(prob["seq_len"].max())
    n = np.arange(S)
    pages = prob["block_table"][:, n // P]                   # (B, S)
    K = prob["k"][pages, (n % P)[None, :]]                  # (B, S, Hkv, d)
    V = prob["v"][pages, (n % P)[None, :]]
    Kf = np.ascontiguousarray(K.transpose(0, 2, 1, 3).reshape(-1, d))
    Vf = np.ascontiguousarray(V.transpose(0, 2, 1, 3).reshape(-1, dv))
    q = prob["q"].reshape(B * Hq, d)
    grp = Hq // Hkv
    seg = (np.arange(B)[:, None] * Hkv + np.arange(Hq)[None, :] // grp).reshape(-1)
    L = prob["seq_len"].repeat(Hq).astype(np.int64)
    row_ptr = np.concatenate([[0], np.cumsum(L)]).astype(np.int64)
    key_idx = np.concatenate([s * S + np.arange(l) for s, l in zip(seg, L)]).astype(np.int64)
    return q, Kf, Vf, row_ptr, key_idx


def cpu_baseline(prob: dict, alpha_bits: int, threads: int, csr=None):
    """The reference's certified CPU kernel (oracle/_ref, compiled from its csrc) on the full
    C2 workload in its CSR form; the oracle's C restatement when that build is absent."""
    from oracle import oracle
    q, Kf, Vf, row_ptr, key_idx = csr if csr is not None else c2_csr(prob)
    L = np.diff(row_ptr)
    ref = oracle.ref_available()
    kind = "reference" if ref else "port"
    run = lambda: oracle.raw_csr(q, Kf, Vf, alpha_bits, row_ptr, key_idx, "bf16", 64, 64, 8, 0, threads,
                                 reference=ref)
    run()  # warm-up
    times = []
    res = None
    for _ in range(3):
        t0 = time.perf_counter()
        res, flags, _ = run()
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    pairs = int(L.sum())
    model = next((ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name")),
                 "unknown") if os.path.exists("/proc/cpuinfo") else "unknown"
    return {"value": round(algorithmic_bytes(prob) / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "cpu_model": model, "host_cpus": os.cpu_count(),
            "sample": f"full C2 step ({pairs} query-key pairs, splits=8, 64-key tiles, int64), median of 3 "
                      f"after 1 warm-up; {pairs / t / 1e6:.2f} M pairs/s; {int((flags != 0).sum())} rows flagged",
            "wall_s": round(t, 3)}, res


def drop_in_line(prob: dict, alpha_bits: int, csr, reps: int = 3) -> dict:
    """The C drop-in ea_attention_hip (the reference's ea_attention_cpu ABI: host arrays in, host
    arrays out) on C2 in its CSR form, the same arrays and arguments the CPU baseline takes
    (splits=8, 64-key tiles, int64): wall time per call with the host-to-device copy of q, K, V
    and the CSR metadata and the copy back, median of `reps` after a warm-up call (which sizes the
    library's device arena). Throughput over the same algorithmic bytes as the CPU baseline's."""
    import torch
    from exactattention_amd import hip
    q, Kf, Vf, row_ptr, key_idx = csr
    alpha = np.array([alpha_bits], np.uint32).view(np.float32)[0]
    lay = hip.csr_layout(row_ptr, key_idx, Kf.shape[0])
    hip.ea_attention_hip(q, Kf, Vf, alpha, row_ptr, key_idx, splits=8)  # warm-up
    times = []
    res = flags = None
    for _ in range(reps):
        t0 = time.perf_counter()
        res, flags, st = hip.ea_attention_hip(q, Kf, Vf, alpha, row_ptr, key_idx, splits=8)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    # the host-to-device copy of the K and V arrays alone (pageable numpy memory), for scale
    t0 = time.perf_counter()
    kd = torch.from_numpy(Kf.view(np.int16)).to("cuda:0")
    vd = torch.from_numpy(Vf.view(np.int16)).to("cuda:0")
    torch.cuda.synchronize()
    h2d = time.perf_counter() - t0
    del kd, vd
    torch.cuda.empty_cache()
    golden = json.load(open(GOLDEN)).get("C2", {}).get("sha256") if os.path.exists(GOLDEN) else None
    pairs = int(np.diff(row_ptr).sum())
    return {"workload": "C2 in CSR form through ea_attention_hip (host arrays, the CPU baseline's arguments)",
            "value": round(algorithmic_bytes(prob) / t / 1e9, 3), "unit": "GB/s", "ms_per_call": round(t * 1e3, 3),
            "pairs_per_s": round(pairs / t, 1), "h2d_kv_ms": round(h2d * 1e3, 3),
            "layout": lay, "bit_exact": (hashlib.sha256(res.tobytes()).hexdigest() == golden) if golden else None,
            "flags_nonzero": int((flags != 0).sum()),
            "basis": "wall clock per call, median of 3 after a warm-up; includes the host-to-device copies"}


# The reference's published ExactAttention step times on one RTX PRO 6000 Blackwell (ms): run 1122
# (docs/DESIGN.md:1055-1065) and the best per shape of run 1124 (:1228-1229), from
# scripts/bench_vs_flashinfer.py: 16 query / 8 KV heads, d = 128, bf16, K/V contiguous per
# (sequence, KV head), decode T = 1 over n keys, verify T = 8 draft tokens causal at the end of n
# keys, CUDA graphs.
PUBLISHED_SHAPES = [  # (T, B, n, run 1122 ms, best of run 1124 ms or None)
    (1, 1, 4096, 0.073, None), (1, 1, 16384, 0.193, 0.177), (1, 1, 65536, 0.534, None),
    (1, 8, 16384, 0.950, 0.909), (1, 32, 16384, 4.301, 3.668),
    (8, 1, 4096, 0.303, None), (8, 1, 16384, 0.686, 0.617), (8, 8, 4096, 0.859, 0.820), (8, 8, 16384, 2.591, None)]


def published_shapes_line(steps: int, warmup: int) -> dict:
    """The reference's published shapes (PUBLISHED_SHAPES) on this library: bf16 N(0,1) q, K, V
    drawn on the device (torch, seed 2024), K/V contiguous per (sequence, KV head) as the
    reference lays them out, the step captured in a HIP graph and replayed. GB/s counts the bf16 K
    and V bytes only, as the reference's harness does. Bits: the auto split count's output equals
    a one-split run's (the certified bits cannot depend on the schedule), 0 rows flagged."""
    import torch
    from exactattention_amd import configs, problem
    from exactattention_amd.hip import STATS, DeviceProblem, launch_hip
    ab = configs.alpha_bits()
    Hq, Hkv, d = 16, 8, 128
    out = []
    for T, B, n, ref_ms, ref_best in PUBLISHED_SHAPES:
        gen = torch.Generator(device="cuda:0").manual_seed(2024)
        q = torch.randn((B, T, Hq, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        k = torch.randn((B, Hkv, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn((B, Hkv, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        kv_len = np.tile(n - T + 1 + np.arange(T), B).astype(np.int32)
        g = problem._geom(B, T, Hq, Hkv, d, d, (T * Hq * d, Hq * d, d), (T * Hq * d, Hq * d, d),
                          (Hkv * n * d, d, n * d), (Hkv * n * d, d, n * d), 1, 0, n)
        prob = dict(geom=g, q=q, k=k, v=v, seq_len=np.full(B, n, np.int32), kv_len=kv_len, block_table=None,
                    block_table_offset=None, tree_mask=None, tree_base=None, out_shape=(B, T, Hq, d))
        one = DeviceProblem(prob, "bf16", 1, "cuda:0")
        launch_hip(one, ab)
        torch.cuda.synchronize()
        want = one.out.cpu().numpy().view(np.uint16)
        del one
        dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
        ms, got = graph_steps(dp, ab, steps, warmup)
        st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
        kv_bytes = 2 * B * Hkv * n * d * 2
        gbs = kv_bytes / (ms * 1e-3) / 1e9
        kernel = "prefill" if st["prefill_kernel_rows"] else ("decode" if st["decode_kernel_rows"] else "general")
        out.append({"shape": f"{'decode' if T == 1 else 'verify T=8'} B={B} n={n}", "ms": round(ms, 5),
                    "kv_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": kernel,
                    "nsplit": dp.nsplit, "ref_ms_run1122": ref_ms, "ref_ms_best_run1124": ref_best,
                    "speedup_vs_ref_best": round((ref_best or ref_ms) / ms, 2),
                    "bits_equal_one_split": bool(np.array_equal(got, want)),
                    "rows_flagged": int(st["tier1_flagged"])})
        del dp, prob, q, k, v
        torch.cuda.empty_cache()
    return {"basis": "HIP-graph replays (events around them); bf16 K+V bytes only; reference figures from one "
                     "RTX PRO 6000 Blackwell (about 1.79 TB/s), a different GPU: context, not a like-for-like "
                     "comparison", "shapes": out}


MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, vendor figure (256 CUs, 2.4 GHz)
PF_TRAFFIC = os.path.join(ROOT, "profiles", "ea_pf_main_C3_traffic.md")
C4_TRAFFIC = os.path.join(ROOT, "profiles", "ea_pf_main_C4_traffic.md")
C5_TRAFFIC = os.path.join(ROOT, "profiles", "ea_decode_C5_traffic.md")


def prefill_ops(prob: dict) -> int:
    """Algorithmic int8 MFMA work of a step: visible query-key pairs x (3x4 score slice products
    + 5x3 P.V slice products) x 128 x 2 ops (bound and recompute products excluded)."""
    g = prob["geom"]
    kv = prob["kv_len"].astype(np.int64)
    pairs = int(kv.sum()) * g["num_q_heads"]
    return pairs * (12 * g["head_dim"] * 2 + 15 * g["head_dim_v"] * 2), pairs


def read_traffic(path: str):
    if os.path.exists(path):
        for ln in open(path):
            if ln.startswith("traffic_bytes_per_launch:"):
                return int(ln.split(":")[1])
    return None


def run_config(name: str, steps: int, warmup: int, splits: int = 0, breakdown_steps: int = 10, digits: bool = False,
               prob=None):
    """Generate config `name`, run warm-up steps, check the bits against the golden hash, then time
    `steps` steps. Inside the timed region HIP events (recorded on the launch stream) bracket only
    the main kernel of each step: that kernel's mean duration feeds the prefill lines' rooflines
    and is reported beside the decode kernel's back-to-back figure. A separate,
    untimed pass of `breakdown_steps` steps records events between every kernel for the
    per-kernel breakdown (each event record is one more packet in the stream, so the timed steps
    carry only the two the roofline needs). digits=True keeps the K/V digit tiles in a KVDigits
    cache sliced once before the steps (the KV write path's format), which the int8 path reads."""
    import torch
    from exactattention_amd import configs
    from exactattention_amd.hip import STATS, DeviceProblem, KVDigits, launch_hip
    t0 = time.time()
    if prob is None:
        prob = configs.CONFIGS[name]()
    ab = configs.alpha_bits()
    gen_s = time.time() - t0
    dp = DeviceProblem(prob, "bf16", splits, "cuda:0")
    cache = None
    slice_ms = None
    if digits:
        S = int(prob["seq_len"].max())
        cache = KVDigits(dp, (S + 63) // 64)
        z = torch.zeros(dp.geom["num_seqs"], dtype=torch.int32, device="cuda:0")
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        cache.update(dp, z, dp.t["seq_len"], S)
        torch.cuda.synchronize()
        slice_ms = (time.perf_counter() - t1) * 1e3
    for _ in range(warmup):
        launch_hip(dp, ab, kv_digits=cache)
    torch.cuda.synchronize()
    out = dp.out.cpu().numpy().view(np.uint16)
    golden = json.load(open(GOLDEN)).get(name, {}).get("sha256") if os.path.exists(GOLDEN) else None
    bit_exact = (hashlib.sha256(out.tobytes()).hexdigest() == golden) if golden else None
    ev = HipEvents(2 * steps)
    slots = [(ctypes.c_void_p * 5)(None, ev.ev[2 * i], ev.ev[2 * i + 1], None, None) for i in range(steps)]
    dp.stats.zero_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        launch_hip(dp, ab, events=slots[i], kv_digits=cache)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    main_ms = float(np.mean([ev.ms(2 * i, 2 * i + 1) for i in range(steps)]))
    ev.close()
    st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    evb = HipEvents(5 * breakdown_steps)
    for i in range(breakdown_steps):
        launch_hip(dp, ab, events=ctypes.cast(evb.slot(5 * i), ctypes.POINTER(ctypes.c_void_p)), kv_digits=cache)
    torch.cuda.synchronize()
    phases = np.array([[evb.ms(5 * i + j, 5 * i + j + 1) for j in range(4)] for i in range(breakdown_steps)])
    evb.close()
    return {"prob": prob, "ab": ab, "dp": dp, "out": out, "gen_s": gen_s, "bit_exact": bit_exact,
            "ms_step": (t1 - t0) * 1e3 / steps, "main_ms": main_ms, "phases": phases.mean(0), "stats": st,
            "cache": cache, "slice_ms": slice_ms}


class _Dim3(ctypes.Structure):
    _fields_ = [("x", ctypes.c_uint32), ("y", ctypes.c_uint32), ("z", ctypes.c_uint32)]


class _KernelNodeParams(ctypes.Structure):
    # hipKernelNodeParams (hip_runtime_api.h)
    _fields_ = [("blockDim", _Dim3), ("extra", ctypes.c_void_p), ("func", ctypes.c_void_p), ("gridDim", _Dim3),
                ("kernelParams", ctypes.c_void_p), ("sharedMemBytes", ctypes.c_uint32)]


def back_to_back_ms(dp, ab: int, block_x: int, reps: int) -> float | None:
    try:
        return _back_to_back_ms(dp, ab, block_x, reps)
    except (AssertionError, RuntimeError) as e:  # a measurement only: the line falls back to in-step events
        print(f"bench.py: back-to-back timing unavailable ({e!r}); the roofline uses the in-step events",
              file=sys.stderr, flush=True)
        return None


def _back_to_back_ms(dp, ab: int, block_x: int, reps: int) -> float | None:
    """Mean duration of one kernel of the step launched `reps` times back to back on one stream,
    from HIP events around the launches: the same basis as a rocprofv3 trace average plus the
    dispatch gap between consecutive kernels (the events around single launches in the timed steps
    also hold the gap after the event). The kernel is the captured step's only kernel node with
    `block_x` threads per block and dynamic LDS (the decode kernel); its launch parameters are the
    captured ones, so the repeats redo that kernel's work exactly: it reads q, K and V and rewrites
    the same split partials, and touches no work list or counter that another kernel resets (the
    stats counters it adds to are read before this runs). None when the step has no single such
    node."""
    import torch
    from exactattention_amd.graph import HipGraph, hip_rt
    from exactattention_amd.hip import launch_hip
    h = hip_rt()
    h.hipGraphKernelNodeGetParams.argtypes = [ctypes.c_void_p, ctypes.POINTER(_KernelNodeParams)]
    h.hipLaunchKernel.argtypes = [ctypes.c_void_p, _Dim3, _Dim3, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    s = torch.cuda.Stream()
    g = HipGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.capture(s, lambda: launch_hip(dp, ab))
    def ok(rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what}: {rc}")

    try:
        n = ctypes.c_size_t(0)
        ok(h.hipGraphGetNodes(g.graph, None, ctypes.byref(n)), "hipGraphGetNodes")
        nodes = (ctypes.c_void_p * n.value)()
        ok(h.hipGraphGetNodes(g.graph, nodes, ctypes.byref(n)), "hipGraphGetNodes")
        picked = []
        for i in range(n.value):
            t = ctypes.c_int(-1)
            ok(h.hipGraphNodeGetType(nodes[i], ctypes.byref(t)), "hipGraphNodeGetType")
            if t.value != 0:
                continue
            kp = _KernelNodeParams()
            ok(h.hipGraphKernelNodeGetParams(nodes[i], ctypes.byref(kp)), "hipGraphKernelNodeGetParams")
            if kp.blockDim.x == block_x and kp.sharedMemBytes > 0:
                picked.append(kp)
        if len(picked) != 1:
            return None
        kp = picked[0]
        ev = HipEvents(2)
        ev.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        st = ctypes.c_void_p(s.cuda_stream)
        for i in range(reps + 2):  # two untimed launches first
            if i == 2:
                ok(ev.h.hipEventRecord(ev.ev[0], st), "hipEventRecord")
            ok(h.hipLaunchKernel(kp.func, kp.gridDim, kp.blockDim, kp.kernelParams, kp.sharedMemBytes, st),
               "hipLaunchKernel")
        ok(ev.h.hipEventRecord(ev.ev[1], st), "hipEventRecord")
        ms = ev.ms(0, 1) / reps
        s.synchronize()
        ev.close()
        return ms
    finally:
        s.synchronize()
        g.close()


def decode_roofline(nbytes: int, in_step_ms: float, b2b_ms: float | None, reps: int, traffic) -> dict:
    """The decode kernel's HBM roofline object. `achieved` divides the algorithmic bytes by the
    kernel's mean duration back to back (back_to_back_ms: the basis of the rocprofv3 trace average
    it is compared with); the events around its single launches inside the timed steps, which also
    count the dispatch after each event, are reported beside it."""
    ms = b2b_ms if b2b_ms is not None else in_step_ms
    achieved = nbytes / (ms * 1e-3) / 1e9
    in_step = nbytes / (in_step_ms * 1e-3) / 1e9
    basis = (f"algorithmic bytes over the decode kernel's mean duration in {reps} launches back to back on its "
             "stream with the captured step's parameters (HIP events around them; the rocprofv3 trace average's "
             "basis plus the gap between consecutive dispatches)" if b2b_ms is not None else
             "algorithmic bytes over the decode kernel's mean HIP-event duration inside the timed steps")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "ea_decode",
            "kernel_ms": round(ms, 5), "basis": basis,
            "in_step_events_ms": round(in_step_ms, 5), "frac_in_step_events": round(in_step / HBM_PEAK_GBS, 4),
            "in_step_events_basis": "HIP events recorded by the library right before and after the decode kernel "
                                    "in each timed step (they also hold the dispatch after the first event)"}


def graph_steps(dp, ab: int, steps: int, warmup: int, kv_digits=None):
    """The step captured once in a HIP graph (exactattention_amd.graph) and replayed `steps` times
    back to back; returns (ms per step from HIP events around the replays, output after them)."""
    import torch
    from exactattention_amd.graph import HipGraph
    from exactattention_amd.hip import launch_hip
    s = torch.cuda.Stream()
    g = HipGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.capture(s, lambda: launch_hip(dp, ab, kv_digits=kv_digits))
    for _ in range(warmup):
        g.replay(s)
    s.synchronize()
    ev = HipEvents(2)
    ev.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    ev.h.hipEventRecord(ev.ev[0], ctypes.c_void_p(s.cuda_stream))
    for _ in range(steps):
        g.replay(s)
    ev.h.hipEventRecord(ev.ev[1], ctypes.c_void_p(s.cuda_stream))
    ms = ev.ms(0, 1) / steps
    s.synchronize()
    ev.close()
    g.close()
    return ms, dp.out.cpu().numpy().view(np.uint16)


def baseline_split_line(prob: dict, ab: int, nsplit: int, steps: int, warmup: int, golden) -> dict:
    """C2 at the split count BASELINE names (8) instead of the auto count: the graph-replayed step
    and the decode kernel back to back, timed as the main line times them; the bits must equal the
    golden hash (the certified output cannot depend on the split count)."""
    import torch
    from exactattention_amd.hip import DeviceProblem
    dp = DeviceProblem(prob, "bf16", nsplit, "cuda:0")
    ms_step, gout = graph_steps(dp, ab, steps, warmup)
    b2b = back_to_back_ms(dp, ab, 128, steps)
    nbytes = algorithmic_bytes(prob)
    out = {"nsplit": dp.nsplit, "ms_per_step": round(ms_step, 5), "value": round(nbytes / (ms_step * 1e-3) / 1e9, 2),
           "unit": "GB/s", "kernel_ms": round(b2b, 5) if b2b else None,
           "kernel_frac": round(nbytes / (b2b * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if b2b else None,
           "bit_exact": (hashlib.sha256(gout.tobytes()).hexdigest() == golden) if golden else None}
    del dp
    torch.cuda.empty_cache()
    return out


def tree_line(steps: int, warmup: int, timers: bool = False) -> dict:
    """C4 speculative tree verification (8 sequences: an 8192-key prefix and a 16-node draft tree
    each, 16 query / 8 KV heads): 32 rows per (sequence, KV head) take the int8 prefill kernel
    with key splits, reading the K/V digit tiles from the cache the KV write path keeps (sliced
    once, before the steps, and timed separately). Roofline: HBM, over the algorithmic bf16 K+V +
    q + out bytes; the digit tiles the kernel actually streams are 69,632 B per 64 keys and KV
    head (2.125x the bf16 bytes), reported beside it."""
    import torch
    from exactattention_amd import hip
    r = run_config("C4", steps, warmup, digits=True)
    prob, st, dp = r["prob"], r["stats"], r["dp"]
    nbytes = algorithmic_bytes(prob)
    g = prob["geom"]
    tiles = g["num_seqs"] * g["num_kv_heads"] * ((int(prob["seq_len"].max()) + 63) // 64)
    main_ms = r["main_ms"]
    achieved = nbytes / (main_ms * 1e-3) / 1e9
    sl, mk, cb, t2 = (float(x) for x in r["phases"])
    line = {"workload": "C4 tree verification (B=8, prefix 8192, 16-node trees, 16 q / 8 KV heads, d=128)",
            "ms_per_step": round(r["ms_step"], 5), "gbs_step": round(nbytes / (r["ms_step"] * 1e-3) / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(C4_TRAFFIC),
                         "kernel": "ea_pf_main", "kernel_ms": round(main_ms, 5),
                         "basis": "algorithmic bf16 bytes over the kernel's mean HIP-event duration on its stream"},
            "digit_tile_gbs": round(tiles * hip.EA_PF_TILE_BYTES / (main_ms * 1e-3) / 1e9, 1),
            "kernels_ms": {"q_slice": round(sl, 5), "ea_pf_main": round(mk, 5), "ea_pf_combine": round(cb, 5),
                           "tier2": round(t2, 5)},
            "key_splits": dp.nsplit, "algorithmic_bytes_per_step": nbytes,
            "kv_digits_slice_ms_all_keys": round(r["slice_ms"], 3),
            "bit_exact": r["bit_exact"], "fallback_rows_pct": round(100.0 * st["tier1_flagged"] / max(1, st["rows"]), 4),
            "input_gen_s": round(r["gen_s"], 1)}
    if timers:
        line["phase_clocks"] = prefill_timers(r)
    del r
    torch.cuda.empty_cache()
    return line


GQA_SHAPES = [(32, 8, 8, 4096), (32, 8, 32, 16384), (64, 8, 4, 8192), (64, 8, 32, 4096)]  # (Hq, Hkv, B, n)


def gqa_line(steps: int, warmup: int) -> dict:
    """Decode at GQA 4 and 8 (32 or 64 query heads on 8 KV heads, one token per sequence: the
    decode kernel in 2-row blocks, a segment's 2 or 4 row blocks on one XCD), bf16 N(0,1) data
    drawn on the device (torch, seed 2024), contiguous K/V, the step as a HIP-graph replay. GB/s
    over the bf16 K+V bytes; the bits must equal a one-split run's."""
    import torch
    from exactattention_amd import configs, problem
    from exactattention_amd.hip import STATS, DeviceProblem, launch_hip
    ab = configs.alpha_bits()
    d = 128
    out = []
    for Hq, Hkv, B, n in GQA_SHAPES:
        gen = torch.Generator(device="cuda:0").manual_seed(2024)
        q = torch.randn((B, 1, Hq, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        k = torch.randn((B, Hkv, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn((B, Hkv, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        g = problem._geom(B, 1, Hq, Hkv, d, d, (Hq * d, Hq * d, d), (Hq * d, Hq * d, d),
                          (Hkv * n * d, d, n * d), (Hkv * n * d, d, n * d), 1, 0, n)
        prob = dict(geom=g, q=q, k=k, v=v, seq_len=np.full(B, n, np.int32), kv_len=np.full(B, n, np.int32),
                    block_table=None, block_table_offset=None, tree_mask=None, tree_base=None,
                    out_shape=(B, 1, Hq, d))
        one = DeviceProblem(prob, "bf16", 1, "cuda:0")
        launch_hip(one, ab)
        torch.cuda.synchronize()
        want = one.out.cpu().numpy().view(np.uint16)
        del one
        dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
        ms, got = graph_steps(dp, ab, steps, warmup)
        st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
        kv_bytes = 2 * B * Hkv * n * d * 2
        out.append({"shape": f"GQA {Hq // Hkv} ({Hq}/{Hkv} heads) B={B} n={n}", "ms": round(ms, 5),
                    "kv_gbs": round(kv_bytes / (ms * 1e-3) / 1e9, 1), "nsplit": dp.nsplit,
                    "equal_share_plan": bool(st["decode_equal_share_steps"]),
                    "bits_equal_one_split": bool(np.array_equal(got, want)), "rows_flagged": int(st["tier1_flagged"])})
        del dp, prob, q, k, v
        torch.cuda.empty_cache()
    return {"basis": "HIP-graph replays (events around them); bf16 K+V bytes only", "shapes": out}


def exact_tier_line(reps: int = 3) -> dict:
    """What a row that tier 1 leaves costs on the device tier 2: ea_options.force_tier2 lists every
    row, on one row of 32,768 keys (tier 2 splits its keys over its 32 blocks) and on 32 such rows
    (one block each), bf16 N(0,1) data drawn on the device (torch, seed 7), contiguous K/V. The
    time is the events around tier 2 in the step (min of `reps`); the bits must equal tier 1's."""
    import torch
    from exactattention_amd import configs, problem
    from exactattention_amd.hip import STATS, DeviceProblem, launch_hip
    ab = configs.alpha_bits()
    d, n = 128, 32768
    out = []
    for rows in (1, 32):
        gen = torch.Generator(device="cuda:0").manual_seed(7)
        q = torch.randn((1, 1, rows, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        k = torch.randn((1, rows, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn((1, rows, n, d), generator=gen, device="cuda:0").to(torch.bfloat16)
        g = problem._geom(1, 1, rows, rows, d, d, (rows * d, rows * d, d), (rows * d, rows * d, d),
                          (rows * n * d, d, n * d), (rows * n * d, d, n * d), 1, 0, n)
        prob = dict(geom=g, q=q, k=k, v=v, seq_len=np.full(1, n, np.int32), kv_len=np.full(1, n, np.int32),
                    block_table=None, block_table_offset=None, tree_mask=None, tree_base=None,
                    out_shape=(1, 1, rows, d))
        dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
        launch_hip(dp, ab)
        torch.cuda.synchronize()
        want = dp.out.cpu().numpy().copy()
        ev = HipEvents(5)
        times = []
        for _ in range(reps):
            dp.stats.zero_()
            launch_hip(dp, ab, events=ctypes.cast(ev.slot(0), ctypes.POINTER(ctypes.c_void_p)), force_tier2=True)
            torch.cuda.synchronize()
            times.append(ev.ms(3, 4))
        ev.close()
        st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
        out.append({"rows": rows, "keys_per_row": n, "tier2_ms": round(min(times), 4),
                    "blocks_per_row": 32 // rows, "tier2_certified": st["tier2_certified"],
                    "bits_equal_tier1": bool(np.array_equal(dp.out.cpu().numpy(), want))})
        del dp, prob, q, k, v
        torch.cuda.empty_cache()
    return {"basis": "force_tier2, HIP events around the work-list and tier-2 launches, min of 3", "cases": out}


def long_context_line(steps: int, warmup: int) -> dict:
    """C5 ragged long-context decode (16 sequences of 8K-131K keys, outlier channels in k, page 16)
    on the fp64 decode kernel: HBM roofline over the algorithmic bytes, bits against the golden
    hash, fallback rows."""
    import torch
    r = run_config("C5", steps, warmup)
    prob, st, dp = r["prob"], r["stats"], r["dp"]
    nbytes = algorithmic_bytes(prob)
    b2b_ms = back_to_back_ms(dp, r["ab"], 128, steps)
    line = {"workload": "C5 ragged decode (B=16, kv 8K-131K, 16 q / 8 KV heads, d=128, page 16)",
            "ms_per_step": round(r["ms_step"], 5), "gbs_step": round(nbytes / (r["ms_step"] * 1e-3) / 1e9, 1),
            "roofline": decode_roofline(nbytes, r["main_ms"], b2b_ms, steps, read_traffic(C5_TRAFFIC)),
            "kernels_ms": {k: round(float(r["phases"][j]), 5) for j, k in enumerate(("prep", "split", "combine",
                                                                                     "tier2"))},
            "nsplit": dp.nsplit, "algorithmic_bytes_per_step": nbytes,
            "bit_exact": r["bit_exact"], "fallback_rows_pct": round(100.0 * st["tier1_flagged"] / max(1, st["rows"]), 4),
            "input_gen_s": round(r["gen_s"], 1)}
    del r
    torch.cuda.empty_cache()
    return line


PF_PHASES = {14: "dma_wait", 0: "barrier1", 1: "score_mfma", 2: "rebase_digits", 3: "barrier2_dma_fold",
             4: "pv_mfma_cert", 5: "cold_path", 6: "exchange", 7: "loop_rest", 15: "prologue", 9: "drain",
             10: "row_totals", 11: "epochs_recip", 12: "round_normal", 13: "round_general"}


def prefill_timers(r: dict, reps: int = 3) -> dict:
    """Phase clocks of the prefill kernel's TIMERS build (s_memtime cycles summed over waves): per
    wave and tile for the loop phases, per wave for the prologue and epilogue."""
    import torch
    from exactattention_amd.hip import launch_hip
    tm = torch.zeros(16, dtype=torch.int64, device="cuda:0")
    for _ in range(reps):
        launch_hip(r["dp"], r["ab"], timers=tm, kv_digits=r["cache"])
    torch.cuda.synchronize()
    tv = tm.cpu().numpy().astype(float)
    tiles = max(1.0, tv[8])  # tiles counted once per wave
    g = r["dp"].geom
    r_seg = g["num_tokens"] * (g["num_q_heads"] // g["num_kv_heads"])
    waves = reps * 8 * g["num_seqs"] * g["num_kv_heads"] * ((r_seg + 31) // 32) * r["dp"].nsplit
    loop = [14, 0, 1, 2, 3, 4, 5, 6, 7]
    tot = sum(tv[i] for i in loop)
    return {"cycles_per_wave_tile": {PF_PHASES[i]: round(tv[i] / tiles, 1) for i in loop},
            "loop_share": {PF_PHASES[i]: round(tv[i] / tot, 4) for i in loop},
            "cycles_per_wave": {PF_PHASES[i]: round(tv[i] / waves, 1) for i in (15, 9, 10, 11, 12, 13)},
            "wave_tiles": int(tv[8])}


def prefill_line(steps: int, warmup: int, timers: bool = False) -> dict:
    """C3 (causal prefill, 4096 tokens) on the int8-MFMA prefill kernel."""
    import torch
    r = run_config("C3", steps, warmup)
    ops, pairs = prefill_ops(r["prob"])
    st = r["stats"]
    slice_ms, _, _, t2_ms = (float(x) for x in r["phases"])
    main_ms = r["main_ms"]
    tops = ops / (main_ms * 1e-3) / 1e12
    line = {
        "workload": "C3 causal prefill (T=4096, 16 q / 8 KV heads, d=128)", "ms_per_step": round(r["ms_step"], 5),
        "tops_step": round(ops / (r["ms_step"] * 1e-3) / 1e12, 2),
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s (int8)",
                     "frac": round(tops / MFMA_I8_PEAK_TOPS, 4), "traffic": read_traffic(PF_TRAFFIC),
                     "kernel": "ea_pf_main", "kernel_ms": round(main_ms, 5)},
        "kernels_ms": {"slice": round(slice_ms, 5), "ea_pf_main": round(main_ms, 5), "tier2": round(t2_ms, 5)},
        "algorithmic_ops_per_step": ops, "pairs_per_step": pairs,
        "bit_exact": r["bit_exact"], "prefill_kernel_rows_per_step": st["prefill_kernel_rows"] // steps,
        "fallback_rows_pct": round(100.0 * st["tier1_flagged"] / max(1, st["rows"]), 4),
        "per_step": {"epoch_folds": st["prefill_epoch_folds"] / steps, "cold_waves": st["prefill_cold_waves"] / steps,
                     "cold_pairs": st["slow_path_scores"] / steps},
        "input_gen_s": round(r["gen_s"], 1),
    }
    line["kv_digits"] = kv_digits_line(r)
    if timers:
        line["phase_clocks"] = prefill_timers(r)
    del r
    torch.cuda.empty_cache()
    return line


def kv_digits_line(r: dict, reps: int = 20) -> dict:
    """The KV write path on C3: the digit-tile cache (ea_hip_kv_digits_update) after an append of
    64 keys per sequence (one tile per KV head) and after all 4096, and one C3 step that reads its
    K/V tiles from the cache instead of slicing them; the step's bits against the golden hash."""
    import torch
    from exactattention_amd.hip import KVDigits, launch_hip
    dp, ab = r["dp"], r["ab"]
    S = int(r["prob"]["seq_len"].max())
    cache = KVDigits(dp, (S + 63) // 64)
    z = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    e = torch.full((1,), S, dtype=torch.int32, device="cuda:0")
    b64 = torch.full((1,), S - 64, dtype=torch.int32, device="cuda:0")
    cache.update(dp, z, e, S)
    torch.cuda.synchronize()
    ev = HipEvents(6)

    def timed(fn, i):
        ev.h.hipEventRecord(ev.ev[2 * i], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        for _ in range(reps):
            fn()
        ev.h.hipEventRecord(ev.ev[2 * i + 1], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return ev.ms(2 * i, 2 * i + 1) / reps

    ev.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    full_ms = timed(lambda: cache.update(dp, z, e, S), 0)
    tile_ms = timed(lambda: cache.update(dp, b64, e, 64), 1)
    step_ms = timed(lambda: launch_hip(dp, ab, kv_digits=cache), 2)
    ev.close()
    out = dp.out.cpu().numpy().view(np.uint16)
    golden = json.load(open(GOLDEN)).get("C3", {}).get("sha256") if os.path.exists(GOLDEN) else None
    return {"update_ms_all_4096_keys": round(full_ms, 5), "update_ms_append_64_keys": round(tile_ms, 5),
            "step_ms_reading_cache": round(step_ms, 5), "step_ms_slicing": round(r["ms_step"], 5),
            "bit_exact_reading_cache": (hashlib.sha256(out.tobytes()).hexdigest() == golden) if golden else None}


def serving_line(prob: dict, ab: int, steps: int, warmup: int = 3) -> dict:
    """C2 through the serving layer (exactattention_amd.serving): the 32 sequences' first 4095 keys
    loaded into a PagedKVCache (with its digit-tile cache), then decode steps of one token per
    sequence through ExactAttentionBackend.forward: the K/V append (device scatter and digit
    re-slice) plus one certified attention launch, host bookkeeping included. The first step is
    C2 itself (its bits against the golden hash); later steps grow every sequence by one key."""
    import torch
    from exactattention_amd.serving import ExactAttentionBackend, PagedKVCache
    B, S, P = prob["seq_len"].shape[0], int(prob["seq_len"].max()), prob["geom"]["page_size"]
    bt = prob["block_table"].astype(np.int64)
    n = np.arange(S)
    K = np.stack([prob["k"][bt[b, n // P], n % P] for b in range(B)])   # (B, S, Hkv, d)
    V = np.stack([prob["v"][bt[b, n // P], n % P] for b in range(B)])
    q = prob["q"].reshape(B, -1, K.shape[3])
    Hq, Hkv, d = q.shape[1], K.shape[2], K.shape[3]
    extra = 2 * (warmup + steps) + 1
    cache = PagedKVCache(num_pages=B * ((S + extra + P - 1) // P), page_size=P, num_kv_heads=Hkv, head_dim=d,
                         max_seqs=B, max_seq_len=S + extra, device="cuda:0")
    be = ExactAttentionBackend(cache, Hq, alpha_bits=ab)
    seqs = [cache.add_sequence() for _ in range(B)]
    cache.append_batch(seqs, [S - 1] * B, K[:, :S - 1].reshape(-1, Hkv, d), V[:, :S - 1].reshape(-1, Hkv, d))
    dev = torch.device("cuda:0")
    qd = torch.from_numpy(q.view(np.int16)).to(dev)
    kd = torch.from_numpy(np.ascontiguousarray(K[:, S - 1]).view(np.int16)).to(dev)
    vd = torch.from_numpy(np.ascontiguousarray(V[:, S - 1]).view(np.int16)).to(dev)
    del K, V
    ones = [1] * B
    out, fl = be.forward(qd, kd, vd, seqs, ones)
    be.check_flags(fl)
    first = out.cpu().numpy().view(np.uint16)
    golden = json.load(open(GOLDEN)).get("C2", {}).get("sha256") if os.path.exists(GOLDEN) else None
    for _ in range(warmup):
        be.forward(qd, kd, vd, seqs, ones)
    torch.cuda.synchronize()
    ev = HipEvents(2)
    ev.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    t0 = time.perf_counter()
    ev.h.hipEventRecord(ev.ev[0], stream)
    for _ in range(steps):
        out, fl = be.forward(qd, kd, vd, seqs, ones)
    t_host = time.perf_counter()
    ev.h.hipEventRecord(ev.ev[1], stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    be.check_flags(fl)
    gpu_ms = ev.ms(0, 1) / steps
    wall_ms = (t1 - t0) * 1e3 / steps
    line = {"workload": "C2 decode through serving.ExactAttentionBackend.forward (32 sequences, one token each, "
                        "K/V append + digit re-slice + attention)",
            "ms_per_step": round(wall_ms, 5), "gpu_ms_per_step": round(gpu_ms, 5),
            "host_enqueue_ms_per_step": round((t_host - t0) * 1e3 / steps, 5),
            "tokens_per_s": round(B / (wall_ms * 1e-3), 1),
            "kv_len": [S + warmup + 1, S + warmup + steps],
            "bit_exact_first_step": (hashlib.sha256(first.tobytes()).hexdigest() == golden) if golden else None}
    # the same decode loop as one captured HIP graph per step (serving.DecodeGraph): block-table
    # update, K/V scatter, digit re-slice and attention replayed, one metadata copy per step
    from exactattention_amd.serving import DecodeGraph
    L0 = cache.length[seqs[0]]
    dg = DecodeGraph(be, seqs, max_len=S + extra)
    dg.q.copy_(qd.view(B, 1, Hq, d))
    dg.k.copy_(kd)
    dg.v.copy_(vd)
    for _ in range(warmup):
        dg.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev.h.hipEventRecord(ev.ev[0], stream)
    for _ in range(steps):
        dg.step()
    t_host = time.perf_counter()
    ev.h.hipEventRecord(ev.ev[1], stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    dg.check_flags()
    g_wall = (t1 - t0) * 1e3 / steps
    line["graph"] = {"ms_per_step": round(g_wall, 5), "gpu_ms_per_step": round(ev.ms(0, 1) / steps, 5),
                     "host_enqueue_ms_per_step": round((t_host - t0) * 1e3 / steps, 5),
                     "tokens_per_s": round(B / (g_wall * 1e-3), 1),
                     "kv_len": [L0 + warmup + 1, L0 + warmup + steps],
                     "flags_clean": not bool(dg.flags.any().item())}
    dg.close()
    ev.close()
    del cache, be
    torch.cuda.empty_cache()
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the C3 prefill measurement")
    ap.add_argument("--only", choices=("C2", "C3", "C4", "C5", "serving", "shapes", "drop_in", "exact_tier", "gqa"),
                    default=None,
                    help="run one workload only, no CPU baseline (for profiler runs)")
    ap.add_argument("--timers", action="store_true",
                    help="after the timed steps, run steps of the phase-clock build and report them (C2, C3, C4)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 5 device-to-device copies of BYTES (scales rocprofv3 FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        src = torch.ones(args.copy_calibration // 2, dtype=torch.int16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": args.copy_calibration}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by sequence x KV head, with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch
    from exactattention_amd.hip import launch_hip

    if args.only == "C3":
        print(json.dumps({"prefill": prefill_line(args.steps, args.warmup, args.timers)}), flush=True)
        return
    if args.only == "C4":
        print(json.dumps({"tree_verify": tree_line(args.steps, args.warmup, args.timers)}), flush=True)
        return
    if args.only == "C5":
        print(json.dumps({"long_context": long_context_line(args.steps, args.warmup)}), flush=True)
        return
    if args.only == "gqa":
        print(json.dumps({"gqa": gqa_line(args.steps, args.warmup)}), flush=True)
        return
    if args.only == "exact_tier":
        print(json.dumps({"exact_tier": exact_tier_line()}), flush=True)
        return
    if args.only == "shapes":
        print(json.dumps({"published_shapes": published_shapes_line(args.steps, args.warmup)}), flush=True)
        return
    if args.only == "drop_in":
        from exactattention_amd import configs
        p2 = configs.c2()
        print(json.dumps({"drop_in": drop_in_line(p2, configs.alpha_bits(), c2_csr(p2))}), flush=True)
        return
    if args.only == "serving":
        from exactattention_amd import configs
        print(json.dumps({"serving": serving_line(configs.c2(), configs.alpha_bits(), args.steps, args.warmup)}),
              flush=True)
        return
    r = run_config("C2", args.steps, args.warmup, args.splits)
    prob, ab, dp, out, st = r["prob"], r["ab"], r["dp"], r["out"], r["stats"]
    nbytes = algorithmic_bytes(prob)
    # the timed steps: the step captured in a HIP graph and replayed (as the reference times its
    # step, in captured CUDA graphs); the eager steps' time is reported beside it
    ms_step, gout = graph_steps(dp, ab, args.steps, args.warmup)
    # the decode kernel (the step's only 128-thread kernel) alone, back to back: the trace's basis
    b2b_ms = back_to_back_ms(dp, ab, 128, args.steps)
    golden = json.load(open(GOLDEN)).get("C2", {}).get("sha256") if os.path.exists(GOLDEN) else None
    graph_exact = (hashlib.sha256(gout.tobytes()).hexdigest() == golden) if golden else None
    split_ms = r["main_ms"]
    flagged_pct = 100.0 * st["tier1_flagged"] / max(1, st["rows"])
    traffic = read_traffic(TRAFFIC)  # HBM bytes per decode launch, from the committed rocprofv3 PMC summary
    roof = decode_roofline(nbytes, split_ms, b2b_ms, args.steps, traffic)
    roof["traffic_source"] = "profiles/ea_decode_C2_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)"
    line = {
        "metric": METRIC, "value": round(nbytes / (ms_step * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": "C2 batched paged decode", "batch": 32, "q_heads": 16, "kv_heads": 8,
                   "head_dim": 128, "kv_len": 4096, "page_size": 16, "layout": "NHD", "nsplit": dp.nsplit,
                   "nsplit_note": "auto split count; BASELINE names 8: the bits are identical at 1, 4 and 8 "
                                  "splits (tests/test_gpu_parity.py test_config_golden_hash)",
                   "algorithmic_bytes_per_step": nbytes},
        "roofline": roof,
        "kernels_ms": {k: round(float(r["phases"][j]), 5) for j, k in enumerate(("prep", "split", "combine",
                                                                                  "tier2"))},
        "ms_per_step_eager": round(r["ms_step"], 5), "step_timing": "HIP graph replays, events around the replays",
        "bit_exact": bool(r["bit_exact"] and graph_exact), "fallback_rows_pct": round(flagged_pct, 4),
        "tier2_certified_rows": st["tier2_certified"], "uncertified_rows": st["uncertified"],
        "tier1_causes": {k: st[k] for k in ("uncertified_scores", "undecided_weights", "uncertified_final", "slow_path_scores")},
        "input_gen_s": round(r["gen_s"], 1),
    }
    if args.timers:
        from exactattention_amd.hip import TIMER_PHASES
        tm = torch.zeros(16, dtype=torch.int64, device="cuda:0")
        for _ in range(5):
            launch_hip(dp, ab, timers=tm)
        torch.cuda.synchronize()
        tv = tm.cpu().numpy()[:8].astype(float)
        tot = tv[:7].sum()
        line["phase_clocks"] = {"cycles_per_wave_tile": {k: round(tv[i] / max(1.0, 4 * tv[7]), 1)
                                                         for i, k in enumerate(TIMER_PHASES[:7])},
                                "share": {k: round(tv[i] / tot, 4) for i, k in enumerate(TIMER_PHASES[:7])}}
    del r, dp
    torch.cuda.empty_cache()
    if args.splits == 0:
        line["baseline_nsplit"] = baseline_split_line(prob, ab, 8, args.steps, args.warmup, golden)
    if args.only is None and not args.no_prefill:
        line["prefill"] = prefill_line(max(5, min(args.steps, 20)), 2)
        line["tree_verify"] = tree_line(max(5, min(args.steps, 20)), 2)
        line["long_context"] = long_context_line(max(5, min(args.steps, 10)), 2)
    if args.only is None:
        line["serving"] = serving_line(prob, ab, max(5, min(args.steps, 20)))
        line["published_shapes"] = published_shapes_line(max(5, min(args.steps, 20)), 2)
        line["exact_tier"] = exact_tier_line()
        line["gqa"] = gqa_line(max(5, min(args.steps, 20)), 2)
    if args.only is None and not args.no_cpu:
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        csr = c2_csr(prob)
        line["drop_in"] = drop_in_line(prob, ab, csr)
        cb, cres = cpu_baseline(prob, ab, threads, csr)
        line["cpu_baseline"] = cb
        line["cpu_bits_equal"] = bool(np.array_equal(cres.reshape(out.shape), out)) if cres is not None else None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
