"""GPU: the exact tiers behind tier 1, and the product's public entry points.

* Tier 2 (the device's 128-bit exact recompute) run on every row (ea_options.force_tier2) on all
  input kinds, bf16 and fp32, after each tier-1 kernel: its bits against the oracle's.
* The reference's adversarial cases on each tier-1 kernel (decode, int8 prefill, general split):
  the fully-lost V channel (V ch1 = 2^-40 ch0 on every key, bf16 0x2B80; reference
  tests/test_triton.py:257-285) and keys that lose bits when sliced (K[[40, 64, 70, 200], 5] =
  2^-40; reference tests/test_triton.py:219-254), on real Qwen3 rows.
* Tier 3 (the host exact tier inside the library) on a row no device tier can certify: two
  weights carry v = +-2^100 and a third key 2^-130 lighter, so the numerator is the light key's
  term alone, 130 bits below the others.
* The public entry points on the GPU: attention (with a mask), attention_row, attention_hip on a
  CSR mask, the reference-compatible C entry point ea_attention_hip bound with the reference's
  argtypes, and the fixture harness's `check --backend hip:rocm`.
"""

import ctypes
import os

import numpy as np
import pytest

from exactattention_amd import problem
from exactattention_amd.formats import default_alpha_bits, float_to_bf16_bits
from gen import KINDS, bf16

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _run(prob, ab, out="bf16", splits=0, **kw):
    from exactattention_amd.hip import attention_problem
    return attention_problem(prob, None, out, splits, None, True, False, alpha_bits=ab, **kw)


def _oracle(prob, ab, out="bf16"):
    from oracle import oracle
    return oracle.attention_geom(prob, ab, out)


def _rand(rng, kind, vkind, B, T, Hq, Hkv, S, d, dv):
    q = bf16(rng, (B, T, Hq, d), kind)
    k = bf16(rng, (B, Hkv, S, d), kind)
    v = bf16(rng, (B, Hkv, S, dv), vkind)
    seq = rng.integers(max(1, S // 2), S + 1, size=B)
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    return problem.contiguous(q, k, v, kv, seq_len=seq)


# kernel name, geometry: the decode kernel (d = 128, few rows), the int8 prefill kernel (forced on
# a small problem), the general split kernel (d = 64)
KERNEL_SHAPES = {"decode": dict(B=2, T=2, Hq=4, Hkv=2, S=150, d=128, dv=128),
                 "prefill": dict(B=1, T=40, Hq=4, Hkv=2, S=120, d=128, dv=128),
                 "general": dict(B=2, T=3, Hq=4, Hkv=2, S=150, d=64, dv=64)}


@pytest.mark.parametrize("kernel", list(KERNEL_SHAPES))
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_forced_tier2_matches_oracle(gpu, kernel, kind, out):
    rng = np.random.default_rng(abs(hash(("t2", kernel, kind, out))) % (1 << 32))
    shp = KERNEL_SHAPES[kernel]
    prob = _rand(rng, kind, "wide" if kind == "normal" else "normal", **shp)
    ab = default_alpha_bits(shp["d"])
    want, _ = _oracle(prob, ab, out)
    got, flags, st = _run(prob, ab, out, kernel=kernel, force_tier2=True)
    rows = _rows(prob)
    assert st["tier2_certified"] == rows and not flags.any(), st
    assert np.array_equal(got, want)


def _rows(prob):
    return prob["q"].shape[0] * prob["q"].shape[1] * prob["q"].shape[2]


@pytest.mark.parametrize("nrows,kind", [(1, "normal"), (3, "wide"), (7, "outlier"), (2, "subnormal")])
def test_forced_tier2_splits_few_long_rows(gpu, nrows, kind):
    """Fewer listed rows than tier 2's 32 blocks: each row's keys are split over 32 // rows blocks
    (1 row: 32 chunks, 3: 10, 7: 4, 2: 16) whose partials the row's last block merges. Ragged key
    counts (some rows shorter than their chunk count would need) and every input kind; bits equal
    the oracle's, every row certified by tier 2."""
    rng = np.random.default_rng(900 + nrows)
    d = dv = 128
    S = 2500
    q = bf16(rng, (nrows, 1, 1, d), kind)
    k = bf16(rng, (nrows, 1, S, d), kind)
    v = bf16(rng, (nrows, 1, S, dv), "wide" if kind == "normal" else "normal")
    seq = np.array([S, 17, 1, 900, 2049, 31, 2500][:nrows], dtype=np.int32)
    prob = problem.contiguous(q, k, v, seq.reshape(nrows, 1), seq_len=seq)
    ab = default_alpha_bits(d)
    want, _ = _oracle(prob, ab)
    for kernel in ("decode", "general"):
        got, flags, st = _run(prob, ab, kernel=kernel, force_tier2=True)
        assert st["tier2_certified"] == nrows and not flags.any(), st
        assert np.array_equal(got, want)


def _qwen_rows(d=128):
    z = np.load(os.path.join(GOLD, "qwen3_0.6b_heads.npz"))
    q, k, v = z["q_27_11"], z["k_27_11"], z["v_27_11"]
    ab = int(np.asarray(z["alpha_27_11"], dtype=np.float32).view(np.uint32))
    return q, k, v, ab


def _prefix_problem(Q, K, V, kv_len):
    R = Q.shape[0]
    n = K.shape[0]
    return problem.contiguous(Q.reshape(1, R, 1, -1), K.reshape(1, 1, n, -1), V.reshape(1, 1, n, -1),
                              np.asarray(kv_len).reshape(1, R))


@pytest.mark.parametrize("kernel", ["decode", "prefill", "general"])
def test_lossy_keys_on_every_kernel(gpu, kernel):
    """Four keys carry one element 2^-40, far below their largest (they lose bits when sliced into
    digits); rows 300-315 of a real Qwen3 head see them. Certified bits equal the oracle's."""
    q, k, v, ab = _qwen_rows()
    rows = np.arange(300, 316)
    Q, kv_len = q[rows].copy(), rows + 1
    K, V = k[:316].copy(), v[:316].copy()
    K[[40, 64, 70, 200], 5] = float_to_bf16_bits(np.full(4, 2.0 ** -40))
    prob = _prefix_problem(Q, K, V, kv_len)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab, splits=2, kernel=kernel)
    assert not flags.any(), st
    assert np.array_equal(got, want), st


@pytest.mark.parametrize("kernel", ["decode", "prefill", "general"])
def test_fully_lost_v_channel_on_every_kernel(gpu, kernel):
    """V channel 1 is 2^-40 of channel 0 on every key: the channel lives only below every digit
    window, so a tier that dropped it would certify 0; the rows must come out with channel 1 =
    2^-40 exactly (bf16 0x2B80), whichever tier certifies them."""
    rng = np.random.default_rng(5)
    d, dv, R, n = 128, 128, 16, 40
    Q = float_to_bf16_bits(rng.standard_normal((R, d)))
    K = float_to_bf16_bits(rng.standard_normal((n, d)))
    vv = rng.standard_normal((n, dv))
    vv[:, 0], vv[:, 1] = 1.0, 2.0 ** -40
    V = float_to_bf16_bits(vv)
    kv_len = rng.integers(1, n + 1, size=R)
    prob = _prefix_problem(Q, K, V, kv_len)
    ab = default_alpha_bits(d)
    want, _ = _oracle(prob, ab)
    assert np.all(want.reshape(R, dv)[:, 1] == 0x2B80)
    got, flags, st = _run(prob, ab, splits=2, kernel=kernel)
    assert not flags.any(), st
    assert np.array_equal(got, want), st


def _cancellation_problem(B=1):
    """Row: q = e_0; keys 0 and 1 score 0 (weight 1) and carry v_0 = +2^100 and -2^100, key 2
    scores -130 at alpha = 1 (weight 2^-130) with v_0 = +2^100. N_0 = 2^-30 exactly, 130 bits
    below its largest terms: outside tier 2's 124-bit window. Channel 1 is 1 on every key."""
    d, dv = 128, 128
    q = np.zeros((B, 1, 1, d), np.uint16)
    q[..., 0] = 0x3F80
    k = np.zeros((B, 1, 3, d), np.uint16)
    k[:, 0, 2, 0] = float_to_bf16_bits(np.array([-130.0]))[0]
    v = np.zeros((B, 1, 3, dv), np.uint16)
    big = float_to_bf16_bits(np.array([2.0 ** 100]))[0]
    v[:, 0, :, 0] = [big, big | 0x8000, big]
    v[:, 0, :, 1] = 0x3F80
    return problem.contiguous(q, k, v, np.full((B, 1), 3)), 0x3F800000


def _overlap_problem(rng, B, T, Hq, Hkv, S, d, dv):
    """Visible sets built from overlapping pieces: kv_len past seq_len on some tokens, and tree masks
    whose keys start inside the prefix and run past seq_len (the storage holds S keys, seq_len is
    shorter, so the keys past it are never read)."""
    q, k, v = bf16(rng, (B, T, Hq, d)), bf16(rng, (B, Hkv, S, d)), bf16(rng, (B, Hkv, S, dv))
    seq = np.array([S - 9 - 17 * b for b in range(B)], dtype=np.int32)
    kv = rng.integers(0, S + 1, size=(B, T))
    tb = (seq - 40).astype(np.int32)
    tm = rng.integers(0, 2 ** 63, size=(B, T), dtype=np.int64).astype(np.uint64) | np.uint64(1 << 63)
    return problem.contiguous(q, k, v, kv, seq_len=seq, tree_mask=tm, tree_base=tb)


@pytest.mark.parametrize("kernel", list(KERNEL_SHAPES))
def test_visible_set_is_a_union_below_seq_len(gpu, kernel):
    """Every tier attends one set per row: the prefix below min(kv_len, seq_len) and the tree keys
    at or past it and below seq_len, each key once. Tier 1 on each kernel, tier 2 forced on every
    row, and the host exact tier on every row (flags set to 1 before ea_hip_exact_rows) all equal
    the oracle's bits."""
    import torch
    from exactattention_amd.hip import DeviceProblem, exact_rows, launch_hip
    shp = dict(KERNEL_SHAPES[kernel])
    shp["S"] = 200
    prob = _overlap_problem(np.random.default_rng(41), **shp)
    ab = default_alpha_bits(shp["d"])
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab, kernel=kernel)
    assert not flags.any(), st
    assert np.array_equal(got, want)
    got2, flags2, st2 = _run(prob, ab, kernel=kernel, force_tier2=True)
    assert not flags2.any() and st2["tier2_certified"] == st2["rows"], st2
    assert np.array_equal(got2, want)
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0", kernel)
    launch_hip(dp, ab)
    dp.flags.fill_(1)
    dp.out.zero_()
    exact_rows(dp, ab)
    torch.cuda.synchronize()
    assert not dp.flags.any().item()
    assert np.array_equal(dp.out.cpu().numpy().view(np.uint16).reshape(want.shape), want)


def test_host_exact_tier_finishes_rows_the_device_cannot(gpu):
    from exactattention_amd.hip import attention_problem
    prob, ab = _cancellation_problem()
    want, _ = _oracle(prob, ab)
    assert want[0, 0, 0, 0] == 0x3000 and want[0, 0, 0, 1] == 0x3F80  # 2^-31 and 1
    for kernel in ("decode", "general"):
        raw, flags, st = _run(prob, ab, kernel=kernel)
        assert flags[0] == 1 and st["uncertified"] == 1, st  # tier 1 and tier 2 cannot decide it
        got, flags, st = attention_problem(prob, kernel=kernel, alpha_bits=ab)  # fallback: the host exact tier
        assert not flags.any() and st["host_exact_rows"] == 1, st
        assert np.array_equal(got, want)


def test_public_entry_points_on_the_cancellation_row(gpu):
    """attention(), attention_hip(fallback=True) and the C drop-in ea_attention_hip return the
    oracle's bits for the row no device tier certifies."""
    import exactattention_amd as ea
    from exactattention_amd.hip import ea_attention_hip
    prob, ab = _cancellation_problem()
    want, _ = _oracle(prob, ab)
    q, k, v = prob["q"].reshape(1, -1), prob["k"].reshape(3, -1), prob["v"].reshape(3, -1)
    alpha = np.float32(1.0)
    assert np.array_equal(ea.attention(q, k, v, alpha), want.reshape(1, -1))
    got, flags = ea.attention_hip(q, k, v, alpha, kv_len=[3])
    assert not flags.any() and np.array_equal(got, want.reshape(1, -1))
    res, fl, st = ea_attention_hip(q, k, v, alpha, np.array([0, 3]), np.arange(3), splits=2)
    assert not fl.any() and np.array_equal(res, want.reshape(1, -1))


def test_attention_with_mask_and_attention_row(gpu):
    """exactattn.attention(q, k, v, alpha, mask) (src/exactattn/reference.py:150-161) on the GPU:
    a random mask (rows with no key give +0), bf16 and fp32 outputs; attention_row on one row."""
    import exactattention_amd as ea
    from oracle import exact
    rng = np.random.default_rng(40)
    r, n, d, dv = 12, 90, 64, 32
    q, k, v = bf16(rng, (r, d), "outlier"), bf16(rng, (n, d), "outlier"), bf16(rng, (n, dv))
    mask = rng.random((r, n)) < 0.4
    mask[3] = False
    ab = default_alpha_bits(d)
    alpha = np.array([ab], np.uint32).view(np.float32)[0]
    for out in ("bf16", "fp32"):
        got = ea.attention(q, k, v, alpha, mask=mask, out=out)
        want = exact.attention(q, k, v, ab, mask=mask, out=out)
        assert np.array_equal(got.view(np.uint32) if out == "fp32" else got, want), out
    assert not ea.attention(q, k, v, alpha, mask=mask)[3].any()
    assert np.array_equal(ea.attention_row(q[0], k, v, alpha), exact.attention_row(q[0], k, v, ab))


def test_attention_hip_csr_rows(gpu):
    """attention_hip with (row_ptr, key_idx): each row its own key list (a page-size-1 cache whose
    block table is the list), out of order and with repeats, on the general and decode kernels."""
    import exactattention_amd as ea
    from oracle import oracle
    rng = np.random.default_rng(41)
    for d in (64, 128):
        r, n = 10, 200
        q, k, v = bf16(rng, (r, d)), bf16(rng, (n, d), "wide"), bf16(rng, (n, d))
        lens = rng.integers(0, 150, size=r)
        row_ptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        key_idx = rng.integers(0, n, size=int(lens.sum())).astype(np.int64)
        ab = default_alpha_bits(d)
        alpha = np.array([ab], np.uint32).view(np.float32)[0]
        got, flags = ea.attention_hip(q, k, v, alpha, row_ptr=row_ptr, key_idx=key_idx, splits=3)
        want, _ = oracle.attention_csr(q, k, v, ab, row_ptr, key_idx)
        assert not flags.any()
        assert np.array_equal(got, want), d


def test_drop_in_with_the_reference_binding(gpu):
    """ea_attention_hip bound exactly as the reference binds ea_attention_cpu (argtypes of
    src/exactattn/cpu.py:35-38, float alpha), on causal rows of a real Qwen3 head: bits equal the
    oracle's, flags 0, stats[0..2] the tier-1 fallback counts (non-negative, summed)."""
    from exactattention_amd import hip
    from oracle import oracle
    lib = ctypes.CDLL(hip.LIB_PATH)
    P = ctypes.c_void_p
    lib.ea_attention_hip.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_float, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P, P, P]
    lib.ea_attention_hip.restype = ctypes.c_int
    q, k, v, ab = _qwen_rows()
    rows = np.arange(1000, 1040)
    Q = np.ascontiguousarray(q[rows])
    row_ptr = np.concatenate([[0], np.cumsum(rows + 1)]).astype(np.int64)
    key_idx = np.concatenate([np.arange(r + 1) for r in rows]).astype(np.int64)
    alpha = float(np.array([ab], np.uint32).view(np.float32)[0])
    for fp32 in (0, 1):
        res = np.zeros((rows.size, 128), np.uint32 if fp32 else np.uint16)
        flags = np.zeros(rows.size, np.uint8)
        st = np.zeros(3, np.int64)
        K, V = np.ascontiguousarray(k), np.ascontiguousarray(v)
        rc = lib.ea_attention_hip(Q.ctypes.data, rows.size, 128, K.ctypes.data, V.ctypes.data, K.shape[0], 128,
                                  ctypes.c_float(alpha), row_ptr.ctypes.data, key_idx.ctypes.data, fp32, 64, 64, 8,
                                  0, 8, res.ctypes.data, flags.ctypes.data, st.ctypes.data)
        assert rc == 0
        want, _ = oracle.attention_csr(Q, K, V, ab, row_ptr, key_idx, "fp32" if fp32 else "bf16")
        assert not flags.any() and np.all(st >= 0)
        assert np.array_equal(res, want), fp32


def _ref_bound_dropin():
    from exactattention_amd import hip
    lib = ctypes.CDLL(hip.LIB_PATH)
    P = ctypes.c_void_p
    lib.ea_attention_hip.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_float, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_uint64, ctypes.c_int, P, P, P]
    lib.ea_attention_hip.restype = ctypes.c_int

    def call(Q, K, V, ab, row_ptr, key_idx, splits=8):
        R, d = Q.shape
        dv = V.shape[1]
        res = np.full((R, dv), 0x5A5A, np.uint16)
        flags = np.full(R, 9, np.uint8)
        st = np.zeros(3, np.int64)
        alpha = float(np.array([ab], np.uint32).view(np.float32)[0])
        rc = lib.ea_attention_hip(Q.ctypes.data, R, d, K.ctypes.data, V.ctypes.data, K.shape[0], dv,
                                  ctypes.c_float(alpha), row_ptr.ctypes.data, key_idx.ctypes.data, 0, 64, 64, splits,
                                  0, 8, res.ctypes.data, flags.ctypes.data, st.ctypes.data)
        assert rc == 0
        return res, flags
    return call


def _gqa_decode_csr(rng, B, Hkv, grp, S, lens):
    """A GQA decode batch in the reference's CSR form (cpu_baseline's layout): K/V rows of
    (sequence, KV head) s at s * S .. s * S + len - 1; rows (b, query head)."""
    d = 128
    q = bf16(rng, (B * Hkv * grp, d))
    K = bf16(rng, (B * Hkv * S, d), "outlier")
    V = bf16(rng, (B * Hkv * S, d))
    seg = (np.arange(B)[:, None] * Hkv + np.arange(Hkv * grp)[None, :] // grp).reshape(-1)
    L = np.repeat(lens, Hkv * grp)
    row_ptr = np.concatenate([[0], np.cumsum(L)]).astype(np.int64)
    key_idx = np.concatenate([s * S + np.arange(l) for s, l in zip(seg, L)]).astype(np.int64)
    return q, K, V, row_ptr, key_idx


def test_csr_families_take_the_tuned_kernels(gpu):
    """CSR rows grouped into key-list families run on the decode kernel (a GQA decode batch) and
    on the int8 prefill kernel (a causal prefix over GQA 2), through attention_problem on the
    layout ea_attention_hip uses: bits equal the oracle's row by row, and the stats name the
    kernel. The C drop-in gives the same bits on both, called twice (larger, then smaller: its
    device arena is reused)."""
    from exactattention_amd import hip
    from oracle import oracle
    rng = np.random.default_rng(42)
    ab = default_alpha_bits(128)
    dropin = _ref_bound_dropin()
    q, K, V, row_ptr, key_idx = _gqa_decode_csr(rng, 5, 4, 2, 700, rng.integers(1, 701, size=5))
    T = 150
    qc = bf16(rng, (2 * T, 128))
    Kc, Vc = bf16(rng, (T, 128), "wide"), bf16(rng, (T, 128))
    rows = [np.arange(t + 1) for t in range(T) for _ in range(2)]
    rp_c = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    ki_c = np.concatenate(rows).astype(np.int64)
    for (Q, Kx, Vx, rp, ki), kernel_stat in (((q, K, V, row_ptr, key_idx), "decode_kernel_rows"),
                                              ((qc, Kc, Vc, rp_c, ki_c), "prefill_kernel_rows")):
        want, _ = oracle.attention_csr(Q, Kx, Vx, ab, rp, ki)
        lay = hip.csr_layout(rp, ki, Kx.shape[0], arrays=True)
        got, flags, st = _run(problem.csr(Q, Kx, Vx, lay), ab)
        assert st[kernel_stat] > 0, st
        tok = lay["tok_row"]
        g = np.zeros_like(want)
        g[tok[tok >= 0]] = got.reshape(-1, 128)[tok >= 0]
        assert not flags.any() and np.array_equal(g, want), kernel_stat
        res, fl = dropin(Q, Kx, Vx, ab, rp, ki)
        assert not fl.any() and np.array_equal(res, want), kernel_stat


def test_fixture_harness_check(gpu, capsys):
    """`python -m exactattention_amd.fixture check --backend hip:rocm`: the reference's published
    SHA-256 of both Qwen3 heads, every causal row, through attention_hip; exit code 0."""
    from exactattention_amd import fixture
    assert fixture.main(["check", "--backend", "hip:rocm"]) == 0
    assert "MATCH" in capsys.readouterr().out
