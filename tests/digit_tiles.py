"""Numpy model of the K/V digit-tile format (the caller-visible KV slice cache written by
ea_hip_kv_digits_update; layout in exactattention_amd/csrc/ea_params.h, sizes in
include/exactattn_hip.h). Test infrastructure: it restates the format from its description, row by
row in plain integer arithmetic, so the GPU test can compare every byte the library writes.

Per key row (the key's 128 K elements, and separately its 128 V elements):
  * each bf16 x decodes to an integer significand m and exponent e with x = m 2^e (normal:
    m = +-(128 + frac), e = field - 134; subnormal: m = +-frac, e = -133); field 0xFF is NaN/inf.
  * lead = the highest set bit position (m 2^e scale) over the finite nonzero elements; the row's
    lsb = lead - 29 (0 for a row with none), so every element is an integer X below 2^30 in units
    of 2^lsb: X = m 2^(e - lsb) rounded half away from zero; an element that loses bits is inexact.
    A row with a NaN/inf element is all zeros (and flagged).
  * X as four balanced radix-256 digits d_0..d_3 in [-128, 127]: the bytes of X + 0x80808080,
    each xor 0x80, stored as int8.
Tile of 64 keys (keys at or past seq_len slice as an all-zero row):
  [0, 32768)      K digit t of (key k, dim c): byte 8192 t + 128 k + 16 ((c >> 4) ^ (k & 7)) + (c & 15)
  [32768, 65536)  V digit t of (key 16 kt + 4 g + i, channel ch):
                  byte 32768 + 8192 t + 64 ch + 16 (g ^ ((ch >> 1) & 3)) + 4 kt + i
  [65536, 69632)  metadata (META below), the rest of the 4 KB untouched
"""

from __future__ import annotations

import numpy as np

TILE = 64
TILE_BYTES = 69632
META_OFF = 65536
EV_UNIT = 0.5 * (2.0 ** 38 + 1.0)

META = np.dtype([("lsbk", "<i4", 64), ("vlsb", "<i4", 64), ("kA", "<f8", 64), ("kX", "<f8", 64),
                 ("kfl", "<i4", 64), ("EV", "<f8", 128), ("tfl", "<i4"), ("pad", "<i4"), ("EVt", "<f8")])


def _decode(x: int):
    f = (x >> 7) & 0xFF
    m = (x & 0x7F) | (0x80 if f else 0)
    if x & 0x8000:
        m = -m
    return m, (f if f else 1) - 134, f == 0xFF


def slice_row(bits) -> dict:
    """The row's lsb, int8 digits (4, n), NaN/inf flag, inexact mask, need of digit 0, the bound
    sum_t |d_t| 256^t maximised over the row, and max |X|."""
    dec = [_decode(int(x)) for x in bits]
    bad = any(b for _, _, b in dec)
    lead = max((e + abs(m).bit_length() - 1 for m, e, b in dec if m and not b), default=None)
    lsb = 0 if lead is None else lead - 29
    X, inex = [], []
    for m, e, b in dec:
        if bad or m == 0:
            X.append(0)
            inex.append(False)
            continue
        sh, a = e - lsb, abs(m)
        if sh >= 0:
            r, lost = a << sh, False
        else:
            r = (a + (1 << (-sh - 1))) >> -sh
            lost = (r << -sh) != a
        X.append(-r if m < 0 else r)
        inex.append(lost)
    dig = np.zeros((4, len(bits)), np.int8)
    amax = 0
    for i, x in enumerate(X):
        u = (x + 0x80808080) & 0xFFFFFFFF
        ds = [((u >> (8 * t)) & 0xFF) - 0x80 for t in range(4)]
        assert sum(d << (8 * t) for t, d in enumerate(ds)) == x
        dig[:, i] = ds
        amax = max(amax, sum(abs(d) << (8 * t) for t, d in enumerate(ds)))
    return {"lsb": lsb, "dig": dig, "bad": bad, "inex": np.array(inex), "need0": bool(np.any(dig[0] != 0)),
            "amax": amax, "xmax": max(abs(x) for x in X)}


def tile_bytes(k_rows, v_rows, n_valid: int) -> np.ndarray:
    """One tile from the K and V rows (uint16 bit patterns, (64, 128) each) of its keys; keys at or
    past n_valid are zero rows."""
    t = np.zeros(TILE_BYTES, np.uint8)
    meta = np.zeros((), META)
    lost = np.zeros(128, np.int64)
    tfl = 0
    for key in range(TILE):
        zero = np.zeros(128, np.uint16)
        K = slice_row(k_rows[key] if key < n_valid else zero)
        V = slice_row(v_rows[key] if key < n_valid else zero)
        c = np.arange(128)
        p = np.arange(4)[:, None]
        t[8192 * p + 128 * key + 16 * ((c >> 4) ^ (key & 7)) + (c & 15)] = K["dig"].view(np.uint8)
        kt, g, i = key >> 4, (key >> 2) & 3, key & 3
        t[32768 + 8192 * p + 64 * c + 16 * (g ^ ((c >> 1) & 3)) + 4 * kt + i] = V["dig"].view(np.uint8)
        bad = K["bad"] or V["bad"]
        meta["lsbk"][key] = K["lsb"]
        meta["vlsb"][key] = V["lsb"]
        meta["kA"][key] = np.ldexp(float(K["amax"]), K["lsb"])
        meta["kX"][key] = float(K["xmax"])
        nk = int(K["inex"].sum())
        meta["kfl"][key] = (min(nk, 255) << 8) | (1 if bad else 0)
        tfl |= (1 << kt) if K["need0"] else 0
        tfl |= 32 if nk else 0
        tfl |= 16 if bad else 0
        lost += V["inex"].astype(np.int64)
    meta["EV"] = EV_UNIT * lost.astype(np.float64)
    meta["tfl"] = tfl
    meta["EVt"] = EV_UNIT * float(lost.sum())
    t[META_OFF:META_OFF + META.itemsize] = np.frombuffer(meta.tobytes(), np.uint8)
    return t


def cache_bytes(k, v, seq_len, tiles: int) -> np.ndarray:
    """The whole cache for contiguous k, v (B, Hkv, S, d) bit patterns: tile t of (b, hk) at
    ((b Hkv + hk) tiles + t) TILE_BYTES."""
    B, Hkv, S, _ = k.shape
    out = np.zeros((B, Hkv, tiles, TILE_BYTES), np.uint8)
    for b in range(B):
        for hk in range(Hkv):
            for ti in range(tiles):
                rows = slice(ti * TILE, min(S, (ti + 1) * TILE))
                kr = np.zeros((TILE, 128), np.uint16)
                vr = np.zeros((TILE, 128), np.uint16)
                kr[:rows.stop - rows.start] = k[b, hk, rows]
                vr[:rows.stop - rows.start] = v[b, hk, rows]
                out[b, hk, ti] = tile_bytes(kr, vr, max(0, min(TILE, int(seq_len[b]) - ti * TILE)))
    return out.reshape(-1)
