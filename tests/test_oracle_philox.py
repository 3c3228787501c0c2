"""Pins oracle/philox.py: the Philox4x32-10 block function against the known-answer
vectors published with the Random123 library (Salmon et al., SC'11; file
kat_vectors, rows "philox4x32 10"), and the walk-stream layout the walk kernels
draw from (word l % 4 of counter (w_lo, w_hi, off_lo + l // 4, off_hi), key
(seed_lo, seed_hi), mapped to (x >> 8) * 2^-24) by values worked from those
vectors by hand.
"""
import numpy as np
import pytest

from oracle import philox

# (counter words c0..c3, key words k0, k1) -> output words, as published.
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", KAT)
def test_random123_known_answers(ctr, key, expect):
    got = philox.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
    assert [int(x) for x in got] == list(expect)


def test_known_answers_batched_in_one_call():
    """The vectorised form gives every row its own answer (no cross-row mixing)."""
    ctrs = np.array([c for c, _, _ in KAT], dtype=np.uint32)
    for i, (_, key, expect) in enumerate(KAT):
        got = philox.philox4x32_10(ctrs, key)[i]
        assert [int(x) for x in got] == list(expect)


def _u24(word: int) -> np.float32:
    return np.float32((word >> 8) / 16777216.0)


def test_walk_stream_first_block_is_the_zero_vector():
    """Walk 0, seed 0, offset 0: steps 0..3 are the four words of Philox(0; 0), step 4 opens block 1."""
    u = philox.walk_uniforms(0, 1, 1, 5, seed=0, offset=0)
    expect = [_u24(w) for w in KAT[0][2]]
    assert u.shape == (1, 5)
    assert list(u[0, :4]) == expect
    # hand-worked: 0x6627E8D5 >> 8 = 0x6627E8 = 6694888 -> 6694888 / 2^24
    assert u[0, 0] == np.float32(6694888 / 16777216.0)
    # step 4 is word 0 of counter (0, 0, 1, 0): differs from step 0
    assert u[0, 4] != u[0, 0]


def test_walk_stream_layout_with_high_words():
    """Walk id, offset and seed above 2^32: each lands in its counter / key word.

    Query q_lo = 2^31 with P = 2 gives walk id 2^32 (w_lo = 0, w_hi = 1); offset
    2^32 + 5 gives block words (5 + l // 4, 1); seed 2^32 * 7 + 3 gives key (3, 7).
    Each uniform is checked against a direct block call on the counter built by hand.
    """
    q_lo, P, L = 1 << 31, 2, 6
    seed = (7 << 32) | 3
    off = (1 << 32) | 5
    u = philox.walk_uniforms(q_lo, 1, P, L, seed=seed, offset=off)
    for p in range(P):
        w = q_lo * P + p
        for l in range(L):
            blk = off + l // 4
            ctr = np.array([[w & 0xFFFFFFFF, w >> 32, blk & 0xFFFFFFFF, blk >> 32]], dtype=np.uint32)
            word = int(philox.philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))[0, l % 4])
            assert u[p, l] == _u24(word), (p, l)
    assert q_lo * P == 1 << 32   # the walk id's high word is exercised


def test_walk_stream_reaches_the_all_ones_vector():
    """Counter and key all ones (the second vector) through the uniform mapping."""
    ctr = np.array([[0xFFFFFFFF] * 4], dtype=np.uint32)
    r = philox.philox4x32_10(ctr, (0xFFFFFFFF, 0xFFFFFFFF))[0]
    assert [int(x) for x in r] == list(KAT[1][2])
    # the same words through the uniform mapping: top 24 bits over 2^24
    assert _u24(int(r[0])) == np.float32(0x408F27 / 16777216.0)


def test_uniform_range_endpoints():
    """(x >> 8) * 2^-24 spans [0, 1 - 2^-24]: exact in float32 at both ends."""
    assert _u24(0) == np.float32(0.0)
    assert _u24(0xFFFFFFFF) == np.float32(1.0 - 2.0 ** -24)
    assert _u24(0xFFFFFFFF) < np.float32(1.0)


def test_dropout_keep_layout_and_hand_values():
    """The attention-dropout mask: head h of the entry at slot s of query row r is word h % 4 of
    Philox(counter (s, r, offset + h // 4)), kept iff (x >> 8) * 2^-24 < 1 - rate. Slot 0 of row 0 with
    seed 0, offset 0 draws the published zero vector (heads 0..3): u = 0x6627E8, 0xE169C5, 0xBC57AC, 0x9B00DB
    over 2^24 = 0.3990, 0.8805, 0.7357, 0.6055."""
    m = philox.dropout_keep([0], [0], 4, 0.5, seed=0, offset=0)[0]
    assert list(m) == [True, False, False, False]          # only 0.399 < 0.5
    m = philox.dropout_keep([0], [0], 4, 0.3, seed=0, offset=0)[0]
    assert list(m) == [True, False, False, True]           # below 0.7: 0.399, 0.6055
    # heads 4..7 take the next counter block; every element against a direct block call, with the slot in
    # the counter's first word and the row in its second (a swap of the two fails here)
    seed, off, H = (5 << 32) | 9, 11, 8
    rows = np.array([0, 3, 3, 17, 2 ** 31 - 1])
    slots = np.array([0, 1, 5, 3, 7])
    m = philox.dropout_keep(rows, slots, H, 0.25, seed=seed, offset=off)
    for i in range(rows.size):
        for h in range(H):
            blk = off + h // 4
            ctr = np.array([[slots[i], rows[i], blk, 0]], dtype=np.uint32)
            word = int(philox.philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))[0, h % 4])
            assert m[i, h] == (np.float32((word >> 8) / 16777216.0) < np.float32(0.75)), (i, h)
    swapped = philox.dropout_keep(slots[1:4], rows[1:4], H, 0.25, seed=seed, offset=off)
    assert not np.array_equal(swapped, m[1:4])


def test_dropout_keep_csr_rows_and_slots():
    """dropout_keep_csr takes each CSR entry's row and its slot e - qptr[row]: rows of lengths 2, 0, 3, 1
    are the entries (row, slot) = (0,0) (0,1) (2,0) (2,1) (2,2) (3,0); a CSR whose row pointers start past 0
    (a slice of a larger CSR) numbers its slots the same way."""
    qptr = np.array([0, 2, 2, 5, 6])
    want = philox.dropout_keep([0, 0, 2, 2, 2, 3], [0, 1, 0, 1, 2, 0], 8, 0.5, seed=77, offset=4)
    assert np.array_equal(philox.dropout_keep_csr(qptr, 8, 0.5, seed=77, offset=4), want)
    assert np.array_equal(philox.dropout_keep_csr(qptr + 10, 8, 0.5, seed=77, offset=4), want)


def test_dropout_keep_rate_limits_and_statistics():
    rows = np.repeat(np.arange(25_000), 8)
    slots = np.tile(np.arange(8), 25_000)
    assert philox.dropout_keep(rows[:1000], slots[:1000], 8, 0.0, seed=3).all()
    assert not philox.dropout_keep(rows[:1000], slots[:1000], 8, 1.0, seed=3).any()
    m = philox.dropout_keep(rows, slots, 8, 0.5, seed=12345)
    frac = m.mean()
    assert abs(frac - 0.5) < 0.003                         # 1.6M Bernoulli draws: sd 0.0004
    # heads, slots and rows are not correlated: head 0 agrees with head 1 about half the time, and so do
    # neighbouring slots of a row and the same slot of neighbouring rows
    assert abs((m[:, 0] == m[:, 1]).mean() - 0.5) < 0.01
    r = m.reshape(25_000, 8, 8)
    assert abs((r[:, 0, :] == r[:, 1, :]).mean() - 0.5) < 0.01
    assert abs((r[:-1, 0, :] == r[1:, 0, :]).mean() - 0.5) < 0.01
