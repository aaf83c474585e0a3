"""Host-side checks that need no GPU: the C ABI library loads and exports every symbol the header
declares, argument validation returns the documented codes before any device work, the problem
builders lay out what the geometry says, and the benchmark configurations are deterministic."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from exactattention_amd import configs, problem
from exactattention_amd.formats import default_alpha_bits
from gen import bf16

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exactattn_hip.h")


def _lib():
    from exactattention_amd import hip
    if not hip.available():
        pytest.skip("libexactattn_hip.so not built (run __graft_entry__.build())")
    return hip.load()


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(ea_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib()
    names = _declared_functions()
    assert len(names) >= 8, names
    for n in names:
        assert hasattr(lib, n), n
    assert b"gfx950" in lib.ea_hip_version()


def _c2_geom(**over):
    p = problem.paged(np.zeros((32, 1, 16, 128), np.uint16), np.zeros((8192, 16, 8, 128), np.uint16),
                      np.zeros((8192, 16, 8, 128), np.uint16), np.zeros((32, 256), np.int32),
                      np.full((32, 1), 4096), np.full(32, 4096))
    g = dict(p["geom"])
    g.update(over)
    return g


def _ws(g, splits=0, **opt):
    from exactattention_amd import hip
    lib = _lib()
    o = hip.Options(splits=splits, tier2=1, **opt)
    nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
    rc = lib.ea_hip_workspace_size(ctypes.byref(hip.geometry(g)), ctypes.byref(o), ctypes.byref(nb),
                                   ctypes.byref(ns))
    return rc, nb.value, ns.value


def test_workspace_size_and_split_plan():
    rc, nb, ns = _ws(_c2_geom(), splits=8)
    assert rc == 0 and ns == 8
    rows = 32 * 16
    assert nb >= rows * 128 * 8 + 8 * rows * 128 * 8  # q in fp64 + the N partials
    rc, _, ns_auto = _ws(_c2_geom())
    assert rc == 0 and 1 <= ns_auto <= 64


@pytest.mark.parametrize("bad,code", [
    (dict(num_q_heads=12, num_kv_heads=8), -1),   # heads not a multiple
    (dict(head_dim=256), -1),                    # above 128
    (dict(head_dim=100), -1),                    # not a multiple of 8
    (dict(head_dim_v=127), -1),                  # odd
    (dict(page_size=12), -1),                    # not a power of two
    (dict(page_size=0), -1),
    (dict(num_tokens=0), -1),
    (dict(num_seqs=-1), -1),
    (dict(num_q_heads=0), -1),
    (dict(num_kv_heads=0), -1),
    (dict(head_dim=0), -1),
    (dict(head_dim_v=0), -1),
    (dict(head_dim_v=130), -1),                  # above 128
    (dict(max_seq_len=-1), -1),
])
def test_workspace_size_rejects_bad_geometry(bad, code):
    assert _ws(_c2_geom(**bad))[0] == code


def test_negative_splits_is_an_option_error():
    assert _ws(_c2_geom(), splits=-1)[0] == -2


@pytest.mark.parametrize("opt", [dict(kernel=-1), dict(kernel=4), dict(prefill_waves=5), dict(prefill_waves=-8)])
def test_bad_options_are_option_errors(opt):
    assert _ws(_c2_geom(), **opt)[0] == -2
    assert _ws(_c2_geom(), **{k: 0 for k in opt})[0] == 0  # the same call with the field at its default


def test_attention_validates_before_any_device_work():
    from exactattention_amd import hip
    lib = _lib()
    g = hip.geometry(_c2_geom())
    fake = 4096  # never dereferenced: each call below returns before touching memory or the device
    full = hip.Buffers(q=fake, k=fake, v=fake, seq_len=fake, kv_len=fake, out=fake, flags=fake)
    nan = hip.Options(alpha_bits=0x7FC00000, tier2=1)
    ok = hip.Options(alpha_bits=default_alpha_bits(128), tier2=1)
    _, nb, _ = _ws(_c2_geom())
    # missing required buffer
    rc = lib.ea_hip_attention(ctypes.byref(g), ctypes.byref(hip.Buffers(q=fake)), ctypes.byref(ok), fake, nb, None)
    assert rc == -1
    # workspace too small
    rc = lib.ea_hip_attention(ctypes.byref(g), ctypes.byref(full), ctypes.byref(ok), fake, nb - 1, None)
    assert rc == -2
    # non-finite alpha
    rc = lib.ea_hip_attention(ctypes.byref(g), ctypes.byref(full), ctypes.byref(nan), fake, nb, None)
    assert rc == -3


def test_empty_batch_needs_no_buffers():
    """num_seqs 0: nothing to read or write, so no buffer or workspace; the geometry, options and
    alpha are still checked. The call returns before any device work (no GPU here)."""
    from exactattention_amd import hip
    lib = _lib()
    g0 = dict(_c2_geom(), num_seqs=0)
    ok = hip.Options(alpha_bits=default_alpha_bits(128), tier2=1)
    for f in (lib.ea_hip_attention, lambda g, b, o, *rest: lib.ea_hip_exact_rows(g, b, o, None)):
        assert f(ctypes.byref(hip.geometry(g0)), None, ctypes.byref(ok), None, 0, None) == 0
        nan = hip.Options(alpha_bits=0x7F800000, tier2=1)
        assert f(ctypes.byref(hip.geometry(g0)), None, ctypes.byref(nan), None, 0, None) == -3
        bad = dict(g0, head_dim=0)
        assert f(ctypes.byref(hip.geometry(bad)), None, ctypes.byref(ok), None, 0, None) == -1
        assert f(ctypes.byref(hip.geometry(g0)), None, ctypes.byref(hip.Options(alpha_bits=ok.alpha_bits, kernel=9)),
                 None, 0, None) == -2
    # with rows, the same null buffers are an error
    assert lib.ea_hip_attention(ctypes.byref(hip.geometry(_c2_geom())), None, ctypes.byref(ok), None, 0, None) == -1


def _reads_digits(g, kv_digits, **opt):
    from exactattention_amd import hip
    o = hip.Options(tier2=1, kv_digits=kv_digits, kv_digits_tiles=(g["max_seq_len"] + 63) // 64, **opt)
    r = ctypes.c_int32(-7)
    rc = _lib().ea_hip_reads_kv_digits(ctypes.byref(hip.geometry(g)), ctypes.byref(o), ctypes.byref(r))
    return rc, r.value


def test_reads_kv_digits_follows_the_kernel_choice():
    """ea_hip_reads_kv_digits (host logic only): 1 exactly when the call takes the int8 prefill path
    with a digit cache set; C2's decode geometry (2 rows per KV head) reads the bf16 cache."""
    fake = 4096
    prefill = _c2_geom(num_tokens=64, q_tok_stride=16 * 128, q_seq_stride=64 * 16 * 128,
                       o_tok_stride=16 * 128, o_seq_stride=64 * 16 * 128)
    assert _reads_digits(prefill, fake) == (0, 1)
    assert _reads_digits(prefill, None) == (0, 0)                     # no cache given
    assert _reads_digits(prefill, fake, kernel=2) == (0, 0)           # EA_KERNEL_DECODE
    assert _reads_digits(_c2_geom(), fake) == (0, 0)                  # decode geometry
    assert _reads_digits(_c2_geom(), fake, kernel=1) == (0, 1)        # EA_KERNEL_PREFILL forces it
    assert _reads_digits(prefill, fake, splits=-1)[0] == -2           # the plan's own checks
    assert _reads_digits(_c2_geom(head_dim=100), fake)[0] == -1


def test_kv_append_validates_before_any_device_work():
    """ea_hip_kv_append returns -1 on bad arguments and 0 for an empty append, launching nothing."""
    lib = _lib()
    fake = 4096
    call = lambda **a: lib.ea_hip_kv_append(a.get("kp", fake), a.get("vp", fake), a.get("rows", 10),
                                            a.get("row", 1024), a.get("kn", fake), a.get("vn", fake),
                                            a.get("dst", fake), a.get("n", 1), a.get("bt", fake),
                                            a.get("bte", 8), a.get("pos", fake), a.get("val", fake),
                                            a.get("nbt", 0), None)
    assert call(n=0, nbt=0) == 0
    assert call(n=-1) == -1
    assert call(row=0) == -1
    assert call(kp=None) == -1
    assert call(dst=None) == -1
    assert call(n=0, nbt=2, bt=None) == -1
    assert call(n=0, nbt=-1) == -1


def test_to_paged_preserves_every_key():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 0x3F80, (2, 1, 4, 16), dtype=np.uint16)
    k = rng.integers(0, 0x3F80, (2, 2, 37, 16), dtype=np.uint16)
    v = rng.integers(0, 0x3F80, (2, 2, 37, 16), dtype=np.uint16)
    base = problem.contiguous(q, k, v, np.full((2, 1), 37))
    for ps in (1, 4, 16):
        for layout in ("NHD", "HND"):
            p = problem.to_paged(base, ps, np.random.default_rng(ps), layout)
            g = p["geom"]
            kp = p["k"].reshape(-1)
            for b in range(2):
                for hk in range(2):
                    for n in range(37):
                        page = p["block_table"][b, n // ps]
                        off = page * g["k_page_stride"] + (n % ps) * g["k_slot_stride"] + hk * g["k_head_stride"]
                        assert np.array_equal(kp[off:off + 16], k[b, hk, n]), (ps, layout, b, hk, n)


def test_configs_are_deterministic_and_sized():
    a, b = configs.c1(), configs.c1()
    for key in ("q", "k", "v", "kv_len"):
        assert np.array_equal(a[key], b[key])
    assert int(a["kv_len"].sum()) == 63520
    assert configs.alpha_bits() == 0x3E0293EE


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_attention_of_no_query_rows_is_empty():
    """attention() with zero query rows returns an empty (0, dv) array of the output type, with or
    without a mask, as the reference's attention() does (src/exactattn/reference.py:150-161);
    nothing runs on the device, but the library must still be there."""
    import exactattention_amd as ea
    _lib()
    rng = np.random.default_rng(8)
    k, v = bf16(rng, (5, 16)), bf16(rng, (5, 8))
    q = np.zeros((0, 16), np.uint16)
    a = ea.default_alpha(16)
    r = ea.attention(q, k, v, a)
    assert r.shape == (0, 8) and r.dtype == np.uint16
    r = ea.attention(q, k, v, a, out="fp32")
    assert r.shape == (0, 8) and r.dtype == np.float32
    r = ea.attention(q, k, v, a, mask=np.zeros((0, 5), bool))
    assert r.shape == (0, 8) and r.dtype == np.uint16


def test_alpha_is_read_as_a_value():
    """An alpha given as an int, bool, numpy int or float is the fp32 value numpy converts it to,
    as the reference's decode_fp32 reads it (src/exactattn/formats.py:120-130); a raw pattern
    comes only through alpha_bits=, and NaN/inf raise the domain error."""
    import exactattention_amd as ea
    from exactattention_amd.formats import alpha_fp32_bits
    for a in (1, True, np.int32(1), np.int64(1), 1.0, np.float32(1.0), np.float64(1.0), np.array(1.0)):
        assert alpha_fp32_bits(a) == 0x3F800000, a
    assert alpha_fp32_bits(np.int32(2)) == 0x40000000
    assert alpha_fp32_bits(0.1) == int(np.float32(0.1).view(np.uint32))
    assert alpha_fp32_bits(alpha_bits=0x3E0293EE) == 0x3E0293EE
    assert alpha_fp32_bits(alpha_bits=np.uint32(1)) == 1
    with pytest.raises(ValueError):
        alpha_fp32_bits(1.0, alpha_bits=0x3F800000)
    with pytest.raises(TypeError):
        alpha_fp32_bits()
    with pytest.raises(TypeError):
        alpha_fp32_bits(alpha_bits=1.0)
    with pytest.raises(ValueError):
        alpha_fp32_bits(alpha_bits=1 << 32)
    for bad in (float("nan"), float("inf"), -np.inf):
        with pytest.raises(ea.ExactAttentionDomainError):
            alpha_fp32_bits(bad)
    with pytest.raises(ea.ExactAttentionDomainError):
        alpha_fp32_bits(alpha_bits=0x7F800000)


def test_public_entry_points_pass_alpha_as_a_value(monkeypatch):
    """attention / attention_row / attention_hip / attention_geom hand the device launch the fp32
    pattern of the value (1 -> 0x3F800000, never 2^-149), and alpha_bits= passes a pattern through."""
    import exactattention_amd as ea
    from exactattention_amd import hip
    seen = []

    def fake(prob, alpha=None, out="bf16", *args, alpha_bits=None, **kw):
        seen.append(hip.alpha_fp32_bits(alpha, alpha_bits))
        rows = prob["q"].shape[0] * prob["q"].shape[1] * prob["q"].shape[2]
        dv = prob["v"].shape[-1]
        res = np.zeros((rows, dv), np.uint16)
        return res, np.zeros(rows, np.uint8), {}

    monkeypatch.setattr(hip, "attention_problem", fake)
    rng = np.random.default_rng(9)
    q, k, v = bf16(rng, (3, 16)), bf16(rng, (5, 16)), bf16(rng, (5, 8))
    ea.attention(q, k, v, 1)
    ea.attention(q, k, v, True, mask=np.ones((3, 5), bool))
    ea.attention_row(q[0], k, v, np.int32(1))
    ea.attention_hip(q, k, v, 1.0)
    ea.attention_geom(problem.contiguous(q.reshape(1, 3, 1, 16), k.reshape(1, 1, 5, 16), v.reshape(1, 1, 5, 8),
                                         np.full((1, 3), 5)), np.float32(1))
    assert seen == [0x3F800000] * 5
    ea.attention(q, k, v, alpha_bits=1)
    assert seen[-1] == 1


def test_trace_row_reads_alpha_as_a_value():
    """trace_row (the host exact tier, no GPU needed) gives the same bits for alpha 1, True,
    np.int32(1) and np.float32(1.0), equal to the oracle's alpha = 1.0 row and different from
    the raw-pattern alpha 2^-149."""
    import exactattention_amd as ea
    from oracle import exact
    _lib()
    rng = np.random.default_rng(10)
    q, k, v = bf16(rng, (16,)), bf16(rng, (7, 16)), bf16(rng, (7, 8))
    want = exact.attention_row(q, k, v, 0x3F800000)
    for a in (1, True, np.int32(1), np.float32(1.0)):
        assert np.array_equal(ea.trace_row(q, k, v, a).out, want), a
    assert np.array_equal(ea.trace_row(q, k, v, alpha_bits=0x3F800000).out, want)
    tiny = exact.attention_row(q, k, v, 1)
    assert np.array_equal(ea.trace_row(q, k, v, alpha_bits=1).out, tiny)
    assert not np.array_equal(tiny, want)


def _layout_keys(lay, i):
    """Keys token i of the CSR layout sees: its sequence's pages, first kv_len keys."""
    T, P = lay["num_tokens"], lay["page_size"]
    b = i // T
    L = int(lay["kv_len"][i])
    pos = np.arange(L)
    return lay["block_table"][lay["bt_off"][b] + pos // P].astype(np.int64) * P + pos % P


def _check_layout(row_ptr, key_idx, nkeys):
    from exactattention_amd import hip
    lay = hip.csr_layout(row_ptr, key_idx, nkeys, arrays=True)
    R = len(row_ptr) - 1
    tok = lay["tok_row"]
    B, T = lay["num_seqs"], lay["num_tokens"]
    assert tok.shape == (B * T,)
    lens = np.diff(row_ptr)
    # every non-empty row appears exactly once, and its token sees exactly its key list
    real = tok[tok >= 0]
    assert sorted(real.tolist()) == [r for r in range(R) if lens[r] > 0]
    for i in np.flatnonzero(tok >= 0):
        r = tok[i]
        assert np.array_equal(_layout_keys(lay, i), key_idx[row_ptr[r]:row_ptr[r + 1]]), (i, r)
        assert lay["kv_len"][i] <= lay["seq_len"][i // T] <= lay["max_seq_len"]
    assert not lay["kv_len"][tok < 0].any()
    # the pages hold whole aligned runs of the caller's keys
    assert lay["page_size"] in (1, 2, 4, 8, 16, 32, 64)
    return lay


def test_csr_layout_groups_rows_into_key_list_families():
    """ea_csr_layout (the drop-in's grouping): decode rows of a GQA batch pair up per KV head,
    a causal prefix becomes one sequence with pages of 64, arbitrary lists keep page size 1; every
    row's token sees exactly its own key list through the block table."""
    _lib()
    # C2-like decode in CSR form: B=3 sequences x 2 KV heads x 2 query heads, 320 keys each
    B, Hkv, grp, S = 3, 2, 2, 320
    seg = (np.arange(B)[:, None] * Hkv + np.arange(Hkv * grp)[None, :] // grp).reshape(-1)
    lens = np.array([320, 320, 320, 320, 100, 100, 100, 100, 5, 5, 5, 5])
    row_ptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    key_idx = np.concatenate([s * S + np.arange(l) for s, l in zip(seg, lens)]).astype(np.int64)
    lay = _check_layout(row_ptr, key_idx, B * Hkv * S)
    assert (lay["num_seqs"], lay["num_tokens"], lay["page_size"]) == (6, 2, 64)
    # causal prefill of 200 tokens over two heads sharing one key range (GQA 2)
    T = 200
    rows = [np.arange(t + 1) for t in range(T) for _ in range(2)]
    row_ptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    lay = _check_layout(row_ptr, np.concatenate(rows).astype(np.int64), T)
    assert (lay["num_seqs"], lay["num_tokens"], lay["page_size"], lay["max_seq_len"]) == (1, 2 * T, 64, T)
    # random lists (repeats, any order) and empty rows: one family per row, page size 1
    rng = np.random.default_rng(11)
    lens = rng.integers(0, 40, size=30)
    row_ptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    key_idx = rng.integers(0, 500, size=int(lens.sum())).astype(np.int64)
    lay = _check_layout(row_ptr, key_idx, 500)
    assert lay["page_size"] == 1
    # prefix families of mixed sizes: padding stays within a quarter of the rows (plus 64)
    rows = []
    for f in range(12):
        base = 1000 * f + np.arange(int(rng.integers(50, 300)))
        for _ in range(int(rng.integers(1, 40))):
            rows.append(base[:int(rng.integers(1, len(base) + 1))])
    row_ptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    lay = _check_layout(row_ptr, np.concatenate(rows).astype(np.int64), 12000)
    assert lay["num_seqs"] * lay["num_tokens"] <= len(rows) * 5 // 4 + 64
    assert lay["page_size"] == 8  # families start at multiples of 1000 = 8 x 125


def test_csr_layout_rejects_bad_lists():
    from exactattention_amd import hip
    _lib()
    with pytest.raises(ValueError):
        hip.csr_layout(np.array([0, 3]), np.array([0, 1, 7]), 5)       # key past nkeys
    with pytest.raises(ValueError):
        hip.csr_layout(np.array([0, 2, 1]), np.array([0, 1]), 5)       # decreasing row_ptr
    lay = hip.csr_layout(np.array([0, 0, 0]), np.zeros(0, np.int64), 5, arrays=True)
    assert lay["num_seqs"] == 0


def test_drop_in_wrapper_checks_array_shapes():
    """The C drop-in reads row_ptr[0 .. rows] and key_idx through bare pointers: the Python wrapper
    refuses arrays whose lengths or shapes would make it read past them (before any device call)."""
    from exactattention_amd import hip
    _lib()
    q = np.zeros((2, 8), np.uint16)
    k = np.zeros((5, 8), np.uint16)
    v = np.zeros((5, 4), np.uint16)
    ki = np.array([0, 1, 2], np.int64)
    with pytest.raises(ValueError):
        hip.ea_attention_hip(q, k, v, 1.0, np.array([0, 3]), ki)        # row_ptr of 1 row for 2
    with pytest.raises(ValueError):
        hip.ea_attention_hip(q, k, v, 1.0, np.array([0, 1, 4]), ki)     # past the end of key_idx
    with pytest.raises(ValueError):
        hip.ea_attention_hip(q, k[:4], v, 1.0, np.array([0, 1, 3]), ki)  # k and v key counts differ
    with pytest.raises(ValueError):
        hip.ea_attention_hip(q.reshape(-1), k, v, 1.0, np.array([0, 1, 3]), ki)  # q not 2-D


def test_kernel_choice_for_verification_segments():
    """The int8 kernel takes segments of 24-31 rows (12-15 draft tokens at GQA 2) with 8K+ keys on
    16+ segments, or 32K+ keys on any; 16-23 rows stay on the decode kernel at any length, and so do
    24-row segments with fewer keys (host logic of the kernel choice, seen through the digit-cache
    query)."""
    fake = 4096

    def geom(tokens, seqs, keys):
        return _c2_geom(num_tokens=tokens, num_seqs=seqs, max_seq_len=keys, q_tok_stride=16 * 128,
                        q_seq_stride=tokens * 16 * 128, o_tok_stride=16 * 128, o_seq_stride=tokens * 16 * 128)

    assert _reads_digits(geom(12, 32, 8192), fake) == (0, 1)     # 24 rows, 256 segments, 8K keys
    assert _reads_digits(geom(12, 2, 8192), fake) == (0, 1)      # 16 segments
    assert _reads_digits(geom(12, 32, 4096), fake) == (0, 0)     # 24 rows, 4K keys: decode
    assert _reads_digits(geom(12, 1, 16384), fake) == (0, 0)     # 8 segments, 16K keys: decode
    assert _reads_digits(geom(12, 1, 32768), fake) == (0, 1)     # 8 segments, 32K keys
    assert _reads_digits(geom(8, 32, 65536), fake) == (0, 0)     # 16 rows: decode at any length
    assert _reads_digits(geom(16, 1, 1024), fake) == (0, 1)      # 32 rows: always the int8 kernel
