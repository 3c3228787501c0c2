"""Philox4x32-10 counter RNG in numpy — TEST INFRASTRUCTURE ONLY.

Restates the published algorithm (Salmon, Moraes, Dror, Shaw, "Parallel random
numbers: as easy as 1, 2, 3", SC'11): 10 rounds of
  (c0, c1, c2, c3) -> (hi(M1*c2) ^ c1 ^ k0, lo(M1*c2), hi(M0*c0) ^ c3 ^ k1, lo(M0*c0))
with M0 = 0xD2511F53, M1 = 0xCD9E8D57 and the key bumped by (0x9E3779B9,
0xBB67AE85) after each round. Pinned by the known-answer vectors distributed
with the Random123 library (tests/test_oracle_philox.py).

The walk stream: uniform for global walk id w, step l is word (l % 4) of
Philox(counter = (w_lo, w_hi, off_lo + l//4, off_hi), key = (seed_lo, seed_hi)),
mapped to (x >> 8) * 2^-24.

The attention-dropout stream: head h of the entry at slot s of query row r is
word (h % 4) of Philox(counter = (s, r, off_lo + h//4, off_hi), key = (seed_lo,
seed_hi)), mapped the same way and kept iff below 1 - rate.
"""
from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = 0x9E3779B9
W1 = 0xBB67AE85
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: tuple) -> np.ndarray:
    """ctr: uint32 [..., 4]; key: (k0, k1). Returns uint32 [..., 4]."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
        k0 = (k0 + W0) & 0xFFFFFFFF
        k1 = (k1 + W1) & 0xFFFFFFFF
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def walk_uniforms(q_lo: int, n_q: int, walks_per_node: int, walk_length: int, seed: int,
                  offset: int = 0) -> np.ndarray:
    """float32 [n_q*P, L]: the uniforms the production walk draws."""
    P, L = walks_per_node, walk_length
    w = (np.arange(q_lo, q_lo + n_q, dtype=np.uint64)[:, None] * np.uint64(P)
         + np.arange(P, dtype=np.uint64)[None, :]).reshape(-1)
    out = np.empty((w.size, L), dtype=np.float32)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    key = (seed & 0xFFFFFFFF, seed >> 32)
    for blk in range((L + 3) // 4):
        b = (int(offset) + blk) & 0xFFFFFFFFFFFFFFFF
        ctr = np.stack([w & MASK, w >> np.uint64(32), np.full_like(w, b & 0xFFFFFFFF),
                        np.full_like(w, b >> 32)], axis=-1)
        r = philox4x32_10(ctr, key)
        for j in range(4):
            l = blk * 4 + j
            if l < L:
                out[:, l] = (r[:, j] >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return out


def dropout_keep(rows, slots, num_heads: int, rate: float, seed: int, offset: int = 0) -> np.ndarray:
    """bool [E, H]: the GraphGPS attention-dropout keep mask the attention kernels draw, for entries given by
    their query row and their slot in that row (rows[i], slots[i], int arrays of length E). Head h of the
    entry at slot s of row r: word h % 4 of Philox(counter = (s, r, (offset + h // 4)_lo, _hi), key =
    (seed_lo, seed_hi)) mapped to (x >> 8) * 2^-24; kept iff that is below 1 - rate (float32)."""
    r = np.asarray(rows, dtype=np.uint64).reshape(-1)
    s_ = np.asarray(slots, dtype=np.uint64).reshape(-1)
    assert r.shape == s_.shape
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    key = (seed & 0xFFFFFFFF, seed >> 32)
    keep_below = np.float32(1.0) - np.float32(rate)
    out = np.zeros((r.size, num_heads), dtype=bool)
    for blk in range((num_heads + 3) // 4):
        b = (int(offset) + blk) & 0xFFFFFFFFFFFFFFFF
        ctr = np.stack([s_ & MASK, r & MASK, np.full_like(r, b & 0xFFFFFFFF), np.full_like(r, b >> 32)], axis=-1)
        x = philox4x32_10(ctr, key)
        for j in range(4):
            h = blk * 4 + j
            if h < num_heads:
                u = (x[:, j] >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
                out[:, h] = u < keep_below
    return out


def dropout_keep_csr(qptr, num_heads: int, rate: float, seed: int, offset: int = 0) -> np.ndarray:
    """dropout_keep for every entry of a query-major CSR (row pointers qptr [n_q + 1]), in CSR order: entry
    e of row r sits at slot e - qptr[r]."""
    qptr = np.asarray(qptr, dtype=np.int64)
    lens = np.diff(qptr)
    rows = np.repeat(np.arange(lens.size, dtype=np.int64), lens)
    slots = np.arange(int(qptr[-1]) - int(qptr[0]), dtype=np.int64) - np.repeat(qptr[:-1] - qptr[0], lens)
    return dropout_keep(rows, slots, num_heads, rate, seed, offset)
