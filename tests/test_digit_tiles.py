"""The K/V digit-tile cache format (ea_hip_kv_digits_update) against an independent numpy model.

CPU: the model is pinned by hand-derived rows (lsb, digits, inexact elements, bounds, NaN rows,
subnormals, signed zero) and by its layout covering the K and V regions with no byte written
twice. GPU: every byte of the library's cache equals the model's, for contiguous and paged K/V
caches, over rows built to reach each branch of the slicing.
"""

import numpy as np
import pytest

import digit_tiles as dt
from gen import bf16

ONE, NEG_ONE_HALF, TWO_M30, NEG_TWO_M30, TWO_M22 = 0x3F80, 0xBFC0, 0x3080, 0xB080, 0x3480


def _row(*vals):
    r = np.zeros(128, np.uint16)
    r[:len(vals)] = vals
    return r


def test_model_rows_by_hand():
    r = dt.slice_row(_row(ONE))  # 1 = 128 2^-7: lead 0, lsb -29, X = 2^29 = 32 * 256^3
    assert r["lsb"] == -29 and list(r["dig"][:, 0]) == [0, 0, 0, 32]
    assert r["amax"] == r["xmax"] == 2 ** 29 and not r["need0"] and not r["inex"].any() and not r["bad"]
    r = dt.slice_row(_row(NEG_ONE_HALF))  # -1.5 = -192 2^-7: X = -3 2^28 = -48 * 256^3
    assert list(r["dig"][:, 0]) == [0, 0, 0, -48] and r["amax"] == 48 * 2 ** 24
    r = dt.slice_row(_row(ONE, TWO_M30, NEG_TWO_M30))  # 2^-30 = half a unit of 2^-29: rounds away from 0
    assert list(r["dig"][:, 1]) == [1, 0, 0, 0] and list(r["dig"][:, 2]) == [-1, 0, 0, 0]
    assert list(r["inex"][:3]) == [False, True, True] and r["need0"]
    r = dt.slice_row(_row(ONE, TWO_M22))  # 2^-22 = 128 units of 2^-29: exact, digits -128 + 1 * 256
    assert list(r["dig"][:, 1]) == [-128, 1, 0, 0] and not r["inex"].any() and r["need0"]
    r = dt.slice_row(_row(0x0001))  # the smallest subnormal 2^-133: lead -133
    assert r["lsb"] == -162 and list(r["dig"][:, 0]) == [0, 0, 0, 32]
    r = dt.slice_row(_row(0x8000, 0x0000))  # signed zeros only: no lead, lsb 0, all digits 0
    assert r["lsb"] == 0 and not r["dig"].any() and r["amax"] == 0
    r = dt.slice_row(_row(0x7FC0, ONE))  # a NaN: the row is flagged and sliced as zeros
    assert r["bad"] and r["lsb"] == -29 and not r["dig"].any() and not r["inex"].any()
    r = dt.slice_row(_row(0x7F80))  # +inf alone
    assert r["bad"] and r["lsb"] == 0 and not r["dig"].any()


def test_model_layout_writes_each_byte_once():
    rng = np.random.default_rng(3)
    k = bf16(rng, (64, 128), "normal")
    v = bf16(rng, (64, 128), "normal")
    t = dt.tile_bytes(k, v, 64)
    # K digit 3 of key 5, dim 37: chunk 2 ^ 5 = 7, byte 5 of it
    r = dt.slice_row(k[5])
    assert t[8192 * 3 + 128 * 5 + 16 * 7 + 5] == r["dig"][3:4, 37].view(np.uint8)[0]
    # mark every position the model writes: each K and V byte exactly once
    hits = np.zeros(dt.META_OFF, np.int64)
    c = np.arange(128)
    p = np.arange(4)[:, None]
    for key in range(64):
        np.add.at(hits, (8192 * p + 128 * key + 16 * ((c >> 4) ^ (key & 7)) + (c & 15)).ravel(), 1)
        kt, g, i = key >> 4, (key >> 2) & 3, key & 3
        np.add.at(hits, (32768 + 8192 * p + 64 * c + 16 * (g ^ ((c >> 1) & 3)) + 4 * kt + i).ravel(), 1)
    assert np.all(hits == 1)
    meta = np.frombuffer(t[dt.META_OFF:dt.META_OFF + dt.META.itemsize].tobytes(), dt.META)[0]
    assert meta["lsbk"][5] == r["lsb"] and meta["kX"][5] == r["xmax"]


def _tile_problem(rng):
    """B = 2, Hkv = 2, 150 keys (the last tile partial, the second sequence ends at 97), with rows
    that reach every branch: wide and subnormal rows, rounded elements, a NaN in a K row, an inf in
    a V row, all-zero and signed-zero rows, a row whose only nonzero element is tiny."""
    from exactattention_amd import problem
    B, Hkv, S, d, T, Hq = 2, 2, 150, 128, 1, 4
    k = bf16(rng, (B, Hkv, S, d), "normal")
    v = bf16(rng, (B, Hkv, S, d), "normal")
    k[0, 0, 10:30] = bf16(rng, (20, d), "wide")
    v[0, 1, 40:70] = bf16(rng, (30, d), "wide")
    k[1, 1, 0:20] = bf16(rng, (20, d), "subnormal")
    v[1, 0, 64:90] = bf16(rng, (26, d), "outlier")
    k[0, 0, 3, 17] = 0x7FC0
    v[1, 1, 5, 99] = 0x7F80
    k[0, 1, 7] = 0
    v[0, 1, 8] = 0x8000
    k[1, 0, 9] = 0
    k[1, 0, 9, 5] = 0x0003
    k[0, 0, 130, :8] = [ONE, TWO_M30, NEG_TWO_M30, TWO_M22, 0, 0x8000, 0x0001, NEG_ONE_HALF]
    q = bf16(rng, (B, T, Hq, d), "normal")
    seq = np.array([150, 97])
    return problem.contiguous(q, k, v, seq.reshape(B, 1), seq_len=seq), k, v, seq


@pytest.mark.gpu
@pytest.mark.parametrize("paged", [False, True])
def test_kv_digit_cache_bytes_match_the_model(gpu, paged):
    import torch
    from exactattention_amd import problem
    from exactattention_amd.hip import DeviceProblem, KVDigits
    prob, k, v, seq = _tile_problem(np.random.default_rng(71))
    if paged:
        prob = problem.to_paged(prob, 16, np.random.default_rng(72), "NHD")
    tiles = 3
    want = dt.cache_bytes(k, v, seq, tiles)
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
    cache = KVDigits(dp, tiles)
    assert cache.buf.numel() == want.size
    cache.update(dp, torch.zeros(2, dtype=torch.int32, device="cuda"), dp.t["seq_len"].clone(), int(seq.max()))
    torch.cuda.synchronize()
    got = cache.buf.cpu().numpy()
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ, first at tile {bad[0] // dt.TILE_BYTES}, offset {bad[0] % dt.TILE_BYTES}"
