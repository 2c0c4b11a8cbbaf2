"""The forward's LDS record address from float bits (ekv_lut.hip `lds_record`), checked on
the CPU in IEEE fp32 (numpy rounds float32 sums to nearest even, as v_add_f32 does):
bits(fl(c + (2^20 - lo - 1/16))) & 0x7FFFF8 == (floor(c) - lo) * 8 for every coordinate
the kernels can form (c < 2^15: padded tables of up to 16384 entries, copies included) at
least 1/16 past the window start lo (the kernels' coordinates lie a record or more past it)."""

import numpy as np

MASK = np.uint32(0x7FFFF8)


def bias(lo: np.ndarray) -> np.ndarray:
    """rec_addr_bias: (float)(2^20 - lo) - 0.0625f, exact for 0 <= lo <= 2^19."""
    return ((np.float32(1 << 20) - lo.astype(np.float32)) - np.float32(0.0625)).astype(np.float32)


def address(c: np.ndarray, lo: np.ndarray) -> np.ndarray:
    t = (c.astype(np.float32) + bias(lo)).astype(np.float32)
    return (t.view(np.uint32) & MASK).astype(np.int64)


def expected(c: np.ndarray, lo: np.ndarray) -> np.ndarray:
    return (np.floor(c.astype(np.float64)).astype(np.int64) - lo) * 8


def test_bias_is_exact():
    lo = np.array([0, 1, 2, 17, 4095, 16415, 1 << 18, 1 << 19], np.int64)
    assert np.array_equal(bias(lo).astype(np.float64), 2.0 ** 20 - lo - 0.0625)


def test_random_coordinates_in_window():
    rng = np.random.default_rng(7)
    n = 2_000_000
    lo = rng.integers(0, 16384, n)
    c = (lo + 0.0625 + rng.random(n) * (32768 - 16384)).astype(np.float32)
    c = np.maximum(c, (lo + 0.0625).astype(np.float32))  # fp32 rounding stays in the domain
    assert np.array_equal(address(c, lo), expected(c, lo))


def test_integers_and_their_neighbours():
    """Exact integers (ties on the 1/8 grid) and the floats just below and above them, at
    every magnitude the coordinates reach (fp32 spacing 2^-23 .. 2^-9)."""
    k = np.concatenate([np.arange(0, 64), np.arange(1000, 1100), np.arange(16300, 16500),
                        np.arange(32700, 32767)]).astype(np.float32)
    for lo_val in (0, 1, 5, 300):
        kk = k[k >= lo_val + 1]  # integers past the window start, and their neighbours
        lo = np.full(kk.shape, lo_val, np.int64)
        below = np.nextafter(kk, np.float32(0))
        above = np.nextafter(kk, np.float32(np.inf))
        for c in (kk, below, above, kk + np.float32(0.0625), kk - np.float32(0.0625),
                  kk + np.float32(0.5), kk + np.float32(0.9375)):
            sel = c >= lo_val
            assert np.array_equal(address(c[sel], lo[sel]), expected(c[sel], lo[sel])), lo_val


def test_window_start():
    """The domain starts at c = lo + 1/16 (record 0); below it the sum stays under 2^20, where
    the mask no longer reads the record, so the kernels keep their coordinates a record or
    more past lo."""
    lo = np.arange(0, 20000, 7, dtype=np.int64)
    start = (lo + 0.0625).astype(np.float32)
    for c in (start, np.nextafter(start, np.float32(np.inf)), (lo + 0.999).astype(np.float32)):
        assert np.array_equal(address(c, lo), np.zeros_like(lo))
    assert not np.any(address(lo.astype(np.float32), lo) == 0)  # c == lo: 2^20 - 1/16, outside


def test_integer_address_would_differ_only_by_the_window():
    """The kernels' other address, (unsigned)c * 8 from table record lo, is the same record."""
    rng = np.random.default_rng(3)
    c = (rng.random(100000) * 16000 + 20).astype(np.float32)
    lo = rng.integers(0, 20, c.shape[0])
    trunc = c.astype(np.uint32).astype(np.int64)
    assert np.array_equal(address(c, lo), (trunc - lo) * 8)
