"""ctypes binding of libexactattn_hip.so and the device-level launcher.

`launch_hip` mirrors launch() of src/exactattn/triton_kernels.py:1324-1519: device tensors in,
work enqueued on torch's current stream, no host transfer and no synchronisation, flags left on
the device. `attention_problem` is the numpy-level round trip used by the public API.

There is no CPU fallback: if the library is missing the calls raise, and a row that no device
tier certifies is reported, never replaced by a host computation.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .formats import ExactAttentionDomainError, ExactAttentionUncertifiedError, alpha_fp32_bits

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libexactattn_hip.so")
P = ctypes.c_void_p
_lib = None

GEOM_FIELDS = (["num_seqs", "num_tokens", "num_q_heads", "num_kv_heads", "head_dim", "head_dim_v"],
               ["q_seq_stride", "q_tok_stride", "q_head_stride", "o_seq_stride", "o_tok_stride", "o_head_stride",
                "k_page_stride", "k_slot_stride", "k_head_stride", "v_page_stride", "v_slot_stride", "v_head_stride"],
               ["page_size", "block_table_stride", "max_seq_len", "pad0"])


class Geometry(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_int32) for n in GEOM_FIELDS[0]] + [(n, ctypes.c_int64) for n in GEOM_FIELDS[1]]
                + [(n, ctypes.c_int32) for n in GEOM_FIELDS[2]])


class Buffers(ctypes.Structure):
    _fields_ = [(n, P) for n in ("q", "k", "v", "seq_len", "kv_len", "block_table", "block_table_offset",
                                 "tree_mask", "tree_base", "out", "flags")]


class Options(ctypes.Structure):
    _fields_ = [("alpha_bits", ctypes.c_uint32), ("out_fp32", ctypes.c_int32), ("splits", ctypes.c_int32),
                ("tier2", ctypes.c_int32), ("merge_order", P), ("stats", P), ("events", P), ("timers", P),
                ("kv_digits", P), ("kv_digits_tiles", ctypes.c_int32), ("pad1", ctypes.c_int32),
                ("kv_digits_slot", P), ("force_tier2", ctypes.c_int32), ("kernel", ctypes.c_int32),
                ("prefill_waves", ctypes.c_int32), ("pad2", ctypes.c_int32)]


# ea_options.kernel (include/exactattn_hip.h EA_KERNEL_*)
KERNELS = {"auto": 0, "prefill": 1, "decode": 2, "general": 3}


EA_PF_TILE_BYTES = 69632  # one 64-key digit tile (ea_params.h)

STATS = ["rows", "tier1_flagged", "tier2_certified", "uncertified", "domain_errors", "uncertified_scores",
         "undecided_weights", "uncertified_final", "slow_path_scores",
         "decode_kernel_rows", "prefill_kernel_rows", "prefill_epoch_folds", "prefill_cold_waves",
         "host_exact_rows", "host_exact_refused", "decode_equal_share_steps"]


def available() -> bool:
    return os.path.exists(LIB_PATH)


def load():
    """Load the in-tree library; raises if it was not built (no silent fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m exactattention_amd.build` (or "
                               "__graft_entry__.build()) first; there is no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        lib.ea_hip_workspace_size.argtypes = [ctypes.POINTER(Geometry), ctypes.POINTER(Options),
                                              ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_int32)]
        lib.ea_hip_workspace_size.restype = ctypes.c_int
        lib.ea_hip_reads_kv_digits.argtypes = [ctypes.POINTER(Geometry), ctypes.POINTER(Options),
                                               ctypes.POINTER(ctypes.c_int32)]
        lib.ea_hip_reads_kv_digits.restype = ctypes.c_int
        lib.ea_hip_attention.argtypes = [ctypes.POINTER(Geometry), ctypes.POINTER(Buffers), ctypes.POINTER(Options),
                                         P, ctypes.c_size_t, P]
        lib.ea_hip_attention.restype = ctypes.c_int
        # the reference's ea_attention_cpu argtypes (src/exactattn/cpu.py:35-38)
        lib.ea_attention_hip.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_float, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P, P, P]
        lib.ea_attention_hip.restype = ctypes.c_int
        lib.ea_csr_layout.argtypes = [ctypes.c_int64, P, P, ctypes.c_int64, P, P, P, P, P, P]
        lib.ea_csr_layout.restype = ctypes.c_int
        lib.ea_round_ratio.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_int)]
        lib.ea_round_ratio.restype = ctypes.c_float
        lib.ea_hip_exact_rows.argtypes = [ctypes.POINTER(Geometry), ctypes.POINTER(Buffers), ctypes.POINTER(Options),
                                          P]
        lib.ea_hip_exact_rows.restype = ctypes.c_int
        lib.ea_exact_row.argtypes = [P, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32,
                                     ctypes.c_int, P, P, P, P]
        lib.ea_exact_row.restype = ctypes.c_int
        lib.ea_hip_kat_weight.argtypes = [ctypes.c_int64] + [P] * 7 + [P]
        lib.ea_hip_kat_weight.restype = ctypes.c_int
        lib.ea_hip_kat_round.argtypes = [ctypes.c_int64, P, P, ctypes.c_int32, P, P, P]
        lib.ea_hip_kat_round.restype = ctypes.c_int
        lib.ea_hip_kat_round_ratio.argtypes = [ctypes.c_int64] + [P] * 6 + [ctypes.c_int32, P, P, P]
        lib.ea_hip_kat_round_ratio.restype = ctypes.c_int
        lib.ea_hip_kat_certify_quotient.argtypes = [ctypes.c_int64, P, ctypes.c_int32, P, P, P]
        lib.ea_hip_kat_certify_quotient.restype = ctypes.c_int
        lib.ea_hip_kv_append.argtypes = [P, P, ctypes.c_int64, ctypes.c_int64, P, P, P, ctypes.c_int64, P,
                                         ctypes.c_int64, P, P, ctypes.c_int64, P]
        lib.ea_hip_kv_append.restype = ctypes.c_int
        lib.ea_hip_kv_digits_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        lib.ea_hip_kv_digits_bytes.restype = ctypes.c_size_t
        lib.ea_hip_kv_digits_update.argtypes = [ctypes.POINTER(Geometry), ctypes.POINTER(Buffers), P, P,
                                                ctypes.c_int32, P, ctypes.c_int32, P]
        lib.ea_hip_kv_digits_update.restype = ctypes.c_int
        lib.ea_hip_kat_rn32_prod.argtypes = [ctypes.c_int64] + [P] * 6 + [P]
        lib.ea_hip_kat_rn32_prod.restype = ctypes.c_int
        lib.ea_hip_kat_wave_max.argtypes = [ctypes.c_int64, P, P, P]
        lib.ea_hip_kat_wave_max.restype = ctypes.c_int
        lib.ea_hip_version.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"{what}: error code {rc}")


def geometry(g: dict) -> Geometry:
    return Geometry(**{f: int(g.get(f, 0)) for f, _ in Geometry._fields_})


def _stream_ptr(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def workspace_size(g: dict, splits: int = 0, out_fp32: bool = False, kernel: int = 0) -> tuple[int, int]:
    lib = load()
    o = Options(splits=splits, out_fp32=int(out_fp32), tier2=1, kernel=kernel)
    nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
    _check(lib.ea_hip_workspace_size(ctypes.byref(geometry(g)), ctypes.byref(o), ctypes.byref(nb), ctypes.byref(ns)),
           "ea_hip_workspace_size")
    return int(nb.value), int(ns.value)


class DeviceProblem:
    """A problem's arrays resident on the GPU, plus output, flags, workspace and stats buffers.
    Built once; `launch_hip` then runs steps on it with no allocation."""

    def __init__(self, prob: dict, out: str = "bf16", splits: int = 0, device: str = "cuda", kernel: str = "auto",
                 prefill_waves: int = 0):
        import torch
        self.torch = torch
        self.prob = prob
        self.geom = dict(prob["geom"])
        self.out_fp32 = out == "fp32"
        self.splits = splits
        self.kernel = KERNELS[kernel]
        self.prefill_waves = int(prefill_waves)
        dev = torch.device(device)

        def t(a, dt=None):
            if a is None:
                return None
            if hasattr(a, "data_ptr"):  # a torch tensor: bf16 as its bit pattern, kept where it is on dev
                if a.dtype == torch.bfloat16:
                    a = a.view(torch.int16)
                return a.to(dev).contiguous()
            a = np.ascontiguousarray(a)
            if a.dtype == np.uint16:
                a = a.view(np.int16)
            elif a.dtype == np.uint64:
                a = a.view(np.int64)
            return torch.from_numpy(a).to(dev)

        self.t = {k: t(prob.get(k)) for k in ("q", "k", "v", "seq_len", "kv_len", "block_table",
                                               "block_table_offset", "tree_mask", "tree_base")}
        rows = int(np.prod(prob["out_shape"][:3]))
        self.rows = rows
        self.out = torch.empty(prob["out_shape"], dtype=torch.int32 if self.out_fp32 else torch.int16, device=dev)
        self.flags = torch.empty(rows, dtype=torch.uint8, device=dev)
        nb, self.nsplit = workspace_size(self.geom, splits, self.out_fp32, self.kernel)
        self.workspace = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
        self.ws_bytes = nb
        self.stats = torch.zeros(16, dtype=torch.int64, device=dev)
        self._geom_c = geometry(self.geom)

    def buffers(self) -> Buffers:
        ptr = {k: (None if v is None else v.data_ptr()) for k, v in self.t.items()}
        return Buffers(**ptr, out=self.out.data_ptr(), flags=self.flags.data_ptr())


TIMER_PHASES = ["prologue", "tile_barrier", "scores", "score_barrier", "weights", "pv", "epilogue", "tiles"]


def options(dp: "DeviceProblem", alpha_bits: int, merge_order=None, tier2: bool = True, events=None, timers=None,
            kv_digits=None, force_tier2: bool = False) -> Options:
    """The ea_options of a step on dp (its kernel choice and prefill block shape come from dp)."""
    mo = merge_order if (merge_order is not None and hasattr(merge_order, "data_ptr")) else None
    return Options(alpha_bits=alpha_bits, out_fp32=int(dp.out_fp32), splits=dp.splits, tier2=int(tier2),
                   merge_order=None if mo is None else mo.data_ptr(), stats=dp.stats.data_ptr(),
                   events=None if events is None else ctypes.cast(events, P),
                   timers=None if timers is None else timers.data_ptr(),
                   kv_digits=None if kv_digits is None else kv_digits.buf.data_ptr(),
                   kv_digits_tiles=0 if kv_digits is None else kv_digits.tiles,
                   force_tier2=int(force_tier2), kernel=dp.kernel, prefill_waves=dp.prefill_waves)


def launch_hip(dp: DeviceProblem, alpha_bits: int, merge_order=None, tier2: bool = True, events=None,
               timers=None, kv_digits=None, force_tier2: bool = False) -> None:
    """Enqueue one step on torch's current stream (no sync, no host copies, no allocation).
    `events`: optional ctypes array of 5 hipEvent_t handles recorded between the kernels.
    `kv_digits`: optional KVDigits cache; the int8 prefill path then reads its K/V tiles there.
    `force_tier2`: every row through the device tier 2 (tests of the exact tier)."""
    lib = load()
    o = options(dp, alpha_bits, merge_order, tier2, events, timers, kv_digits, force_tier2)
    b = dp.buffers()
    _check(lib.ea_hip_attention(ctypes.byref(dp._geom_c), ctypes.byref(b), ctypes.byref(o), dp.workspace.data_ptr(),
                                dp.ws_bytes, _stream_ptr(dp.torch)), "ea_hip_attention")


def exact_rows(dp: DeviceProblem, alpha_bits: int) -> None:
    """The host exact tier on dp's last step: waits for torch's current stream, recomputes every
    row left at flag 1 exactly on the host and writes its bits and flag (ea_hip_exact_rows)."""
    lib = load()
    o = options(dp, alpha_bits)
    b = dp.buffers()
    _check(lib.ea_hip_exact_rows(ctypes.byref(dp._geom_c), ctypes.byref(b), ctypes.byref(o), _stream_ptr(dp.torch)),
           "ea_hip_exact_rows")


class KVDigits:
    """A device digit-tile cache of a problem's K/V (the KV slice format kept across steps):
    `tiles` 64-key tiles per (sequence, KV head), EA_PF_TILE_BYTES each, laid out as
    include/exactattn_hip.h describes for ea_hip_kv_digits_update."""

    def __init__(self, dp: DeviceProblem, tiles: int):
        import torch
        lib = load()
        g = dp.geom
        n = lib.ea_hip_kv_digits_bytes(int(g["num_seqs"]), int(g["num_kv_heads"]), int(tiles))
        if n == 0:
            raise ValueError("empty digit cache")
        self.tiles = int(tiles)
        self.buf = torch.zeros(n, dtype=torch.uint8, device=dp.out.device)

    def update(self, dp: DeviceProblem, key_begin, key_end, max_new_keys: int) -> None:
        """Re-slice the tiles that hold keys key_begin[b] .. key_end[b] - 1 of each sequence
        (device int32 tensors), after they were written to dp's bf16 cache."""
        lib = load()
        b = dp.buffers()
        _check(lib.ea_hip_kv_digits_update(ctypes.byref(dp._geom_c), ctypes.byref(b), key_begin.data_ptr(),
                                           key_end.data_ptr(), int(max_new_keys), self.buf.data_ptr(), self.tiles,
                                           _stream_ptr(dp.torch)), "ea_hip_kv_digits_update")


def merge_order_tensor(order, nsplit: int, device="cuda"):
    """Keep the caller's order for splits that exist, append the rest (as the reference launcher
    does, src/exactattn/triton_kernels.py:1471-1479)."""
    import torch
    given = [int(i) for i in order if 0 <= int(i) < nsplit]
    seen = set()
    given = [i for i in given if not (i in seen or seen.add(i))]
    full = given + [i for i in range(nsplit) if i not in given]
    return torch.tensor(full, dtype=torch.int32, device=device)


def attention_problem(prob: dict, alpha=None, out: str = "bf16", splits: int = 0, merge_order=None,
                      tier2: bool = True, fallback: bool = True, device: str = "cuda", kernel: str = "auto",
                      force_tier2: bool = False, prefill_waves: int = 0, *, alpha_bits=None):
    """Run a problem on the GPU. Returns (out bits shaped (B, T, Hq, dv): uint16 for bf16, uint32
    for fp32; flags (rows,) uint8; stats dict). fallback=False returns the device tiers' flags as
    they are. With fallback=True rows the device tiers leave at flag 1 are recomputed by the host
    exact tier (ea_hip_exact_rows, counted in stats["host_exact_rows"]), and flag 2 raises
    ExactAttentionDomainError, as the reference's backends do (src/exactattn/cpu.py:103-108).
    `alpha` is the fp32 scale as a value; `alpha_bits=` passes its bit pattern instead."""
    import torch
    alpha_bits = alpha_fp32_bits(alpha, alpha_bits)
    dp = DeviceProblem(prob, out, splits, device, kernel, prefill_waves)
    mo = merge_order_tensor(merge_order, dp.nsplit, device) if merge_order is not None else None
    launch_hip(dp, int(alpha_bits), mo, tier2, force_tier2=force_tier2)
    torch.cuda.synchronize()
    flags = dp.flags.cpu().numpy()
    if fallback and np.any(flags == 1):
        exact_rows(dp, int(alpha_bits))
        torch.cuda.synchronize()
        flags = dp.flags.cpu().numpy()
    res = dp.out.cpu().numpy()
    res = res.view(np.uint32) if dp.out_fp32 else res.view(np.uint16)
    st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    st["nsplit"] = dp.nsplit
    if fallback:
        if np.any(flags == 2):
            raise ExactAttentionDomainError(f"non-finite input, fp32 logit overflow or an exponent spread past "
                                            f"2^20 in rows {np.flatnonzero(flags == 2)[:8].tolist()}")
        if np.any(flags == 1):
            raise ExactAttentionUncertifiedError(f"rows {np.flatnonzero(flags == 1)[:8].tolist()} not certified")
    return res, flags, st


def ea_attention_hip(q, k, v, alpha, row_ptr, key_idx, out="bf16", splits=8, acc_bits=64, tile=64):
    """The drop-in C entry point (host pointers; the reference's ea_attention_cpu argument list and
    argtypes, src/exactattn/cpu.py:35-38,86-94). Returns (out bits, flags, stats[3])."""
    lib = load()
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("q, k and v must be 2-D arrays (rows x d, keys x d, keys x dv)")
    rows, d = q.shape
    n, dv = v.shape
    if k.shape != (n, d):
        raise ValueError(f"k has shape {k.shape}; q and v need ({n}, {d})")
    rp = np.ascontiguousarray(row_ptr, dtype=np.int64)
    ki = np.ascontiguousarray(key_idx, dtype=np.int64)
    # the C entry point takes bare pointers: it reads row_ptr[0 .. rows] and the key_idx entries
    # those delimit, so the lengths are checked here
    if rp.shape != (rows + 1,):
        raise ValueError(f"row_ptr must have rows + 1 = {rows + 1} entries, got shape {rp.shape}")
    if ki.ndim != 1 or (rows > 0 and (rp[0] < 0 or rp[-1] > ki.shape[0])):
        raise ValueError("key_idx must be 1-D and hold every entry row_ptr delimits")
    fp32 = out == "fp32"
    res = np.zeros((rows, dv), dtype=np.uint32 if fp32 else np.uint16)
    flags = np.zeros(rows, dtype=np.uint8)
    st = np.zeros(3, dtype=np.int64)
    rc = lib.ea_attention_hip(q.ctypes.data, rows, d, k.ctypes.data, v.ctypes.data, n, dv,
                              ctypes.c_float(float(np.float32(alpha))), rp.ctypes.data, ki.ctypes.data, int(fp32),
                              acc_bits, tile, splits, 0, 1, res.ctypes.data, flags.ctypes.data, st.ctypes.data)
    _check(rc, "ea_attention_hip")
    return res, flags, st


def csr_layout(row_ptr, key_idx, nkeys: int, arrays: bool = False) -> dict:
    """The serving geometry ea_attention_hip gives a CSR problem (ea_csr_layout): sequences
    (key-list families), tokens per sequence, page size, longest list; with arrays=True also the
    token -> row map (-1 padding), visible lengths, sequence lengths, block-table offsets and the
    block table. Host only."""
    lib = load()
    rp = np.ascontiguousarray(row_ptr, dtype=np.int64)
    ki = np.ascontiguousarray(key_idx, dtype=np.int64)
    dims = np.zeros(6, np.int64)
    kp = ki.ctypes.data if ki.size else None
    _check(lib.ea_csr_layout(rp.shape[0] - 1, rp.ctypes.data, kp, int(nkeys), dims.ctypes.data,
                             None, None, None, None, None), "ea_csr_layout")
    B, T, Pg, maxlen, nbt, BT = (int(x) for x in dims)
    lay = dict(num_seqs=B, num_tokens=T, page_size=Pg, max_seq_len=maxlen)
    if arrays:
        lay.update(tok_row=np.zeros(BT, np.int64), kv_len=np.zeros(BT, np.int32), seq_len=np.zeros(B, np.int32),
                   bt_off=np.zeros(B, np.int64), block_table=np.zeros(max(nbt, 1), np.int32))
        _check(lib.ea_csr_layout(rp.shape[0] - 1, rp.ctypes.data, kp, int(nkeys), dims.ctypes.data,
                                 lay["tok_row"].ctypes.data, lay["kv_len"].ctypes.data, lay["seq_len"].ctypes.data,
                                 lay["bt_off"].ctypes.data, lay["block_table"].ctypes.data), "ea_csr_layout")
    return lay


def exact_row(q, k, v, alpha_bits: int, out: str = "bf16", trace: bool = False):
    """The host exact tier on one row of host arrays (ea_exact_row): q (d,), k (n, d), v (n, dv)
    bf16 bits. Returns the output bits, plus (t bits, w_m, w_e) per key when trace=True. Raises
    ExactAttentionDomainError for NaN/inf, an fp32 logit overflow or a spread past 2^20 bits."""
    lib = load()
    q = np.ascontiguousarray(q, dtype=np.uint16).reshape(-1)
    d = q.shape[0]
    k = np.ascontiguousarray(k, dtype=np.uint16).reshape(-1, d)
    n = k.shape[0]
    v = np.ascontiguousarray(v, dtype=np.uint16)
    dv = v.shape[-1]
    v = v.reshape(n, dv)
    fp32 = out == "fp32"
    res = np.zeros(dv, dtype=np.uint32 if fp32 else np.uint16)
    tb = np.zeros(max(n, 1), np.uint32)
    wm = np.zeros(max(n, 1), np.int32)
    we = np.zeros(max(n, 1), np.int64)
    rc = lib.ea_exact_row(q.ctypes.data, d, k.ctypes.data, v.ctypes.data, n, dv, int(alpha_bits), int(fp32),
                          res.ctypes.data, tb.ctypes.data if trace else None, wm.ctypes.data if trace else None,
                          we.ctypes.data if trace else None)
    if rc == 2 or rc == 3:
        raise ExactAttentionDomainError("non-finite input, fp32 logit overflow or an exponent spread past 2^20")
    _check(rc, "ea_exact_row")
    return (res, tb[:n], wm[:n], we[:n]) if trace else res
