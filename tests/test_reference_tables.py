"""The reference's bf16 tables, byte for byte (CPU only, no GPU).

`LUT_DTYPE = "bfloat16"` must give the bytes `_cpu_lut_cached` gives
(`src/isa/approximations/delta_lut.py:25-35`): an fp32 intermediate built with torch's fp32
CPU ops, then cast to bf16 round-to-nearest-even. The oracle's statement-by-statement
restatement (`oracle.reference_lut_tables`) is pinned here by what is independent of it:

* the reference's own test of that function (`tests/test_flash_formula.py:56-84`: grid
  (-1, 3, 257), rtol 8e-3, atol 3e-3);
* the float64 closed form, tightly where fp32 evaluation is benign (a dropped term, a wrong
  sign or factor fails these), and the fp32 signature of the reference's construction where
  it is not: `1 - exp(-sp)` cancels to exactly 0 once sp < 2^-25, so the derivative table is
  exactly zero at the subthreshold end (a table evaluated in higher precision fails this);
* round-to-nearest-even restated on the integer bit patterns (a truncating or
  round-half-up cast fails this).

The product's host builder (`isa.approximations.delta_lut.reference_bf16_tables`) is then
checked against the pinned restatement at every table size the configurations use.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle
from tests.helpers import flash_cfg
from tests.test_oracle import REF_TEST_CFG, _closed_form_table


def _rne_bits(f32: np.ndarray) -> np.ndarray:
    """bf16 bit patterns of fp32 values by round-to-nearest-even (finite inputs)."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def _bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_reference_tables_meet_the_reference_test():
    """tests/test_flash_formula.py:56-84, run on the restated bf16 current table."""
    _, _, bi, _ = oracle.reference_lut_tables(dict(REF_TEST_CFG), size=257, delta_min=-1.0, delta_max=3.0)
    delta = torch.linspace(-1.0, 3.0, 257, dtype=torch.float32)
    k = 1.0 / (2.0 * REF_TEST_CFG["n"] * REF_TEST_CFG["U_T"])
    expected = REF_TEST_CFG["I_S"] * (F.softplus(delta * k).square() - F.softplus((delta - REF_TEST_CFG["V_D"]) * k).square())
    assert torch.allclose(bi.float(), expected, rtol=8.0e-3, atol=3.0e-3)


@pytest.mark.parametrize("size", [257, 4096, 8192, 16384])
def test_reference_fp32_intermediate_against_closed_form(size):
    cfg = flash_cfg(size)
    dmin, dmax, n = oracle.lut_range(cfg)
    ri, rd, _, _ = oracle.reference_lut_tables(cfg)
    ci, cd = _closed_form_table(cfg, dmin, dmax, n)
    delta = dmin + np.arange(n) * (dmax - dmin) / (n - 1)
    ri64, rd64 = ri.astype(np.float64), rd.astype(np.float64)
    # current table: fp32 evaluation error only, wherever sp^2 stays a normal float
    normal = ci > 1e-30
    assert np.all(np.abs(ri64 - ci)[normal] <= 1e-5 * ci[normal])
    assert np.all(np.abs(ri64 - ci)[~normal] <= 1e-35)
    # derivative table: tight above threshold ...
    hi = delta >= -1.0
    assert np.all(np.abs(rd64 - cd)[hi] <= 2e-5 * cd[hi])
    mid = delta >= -2.0
    assert np.all(np.abs(rd64 - cd)[mid] <= 1e-3 * cd[mid])
    # ... and the fp32 cancellation of 1 - exp(-sp) below it: never negative, never more
    # than a few times the true value, exactly zero at the subthreshold end
    assert np.all(rd64 >= 0.0) and np.all(rd64 <= 4.0 * cd)
    assert np.all(rd[delta <= -3.8] == 0.0)
    assert np.all(rd[delta >= -3.6] > 0.0)


@pytest.mark.parametrize("size", [257, 4096, 8192, 16384])
def test_reference_bf16_cast_is_round_to_nearest_even(size):
    ri, rd, bi, bd = oracle.reference_lut_tables(flash_cfg(size))
    assert np.array_equal(_bits(bi), _rne_bits(ri))
    assert np.array_equal(_bits(bd), _rne_bits(rd))


@pytest.mark.parametrize("size", [257, 4096, 8192, 16384])
def test_product_bf16_tables_are_the_reference_bytes(size):
    """The library's LUT_DTYPE=bfloat16 host build equals the pinned restatement bytewise,
    and differs from the rounded fp64 table where the reference's fp32 steps lose accuracy
    (so the comparison can tell the two constructions apart)."""
    from isa.approximations.delta_lut import lut_range, reference_bf16_tables

    cfg = flash_cfg(size, LUT_DTYPE="bfloat16")
    dmin, dmax, n = lut_range(cfg)
    pi, pd = reference_bf16_tables(cfg["n"], cfg["I_S"], cfg["U_T"], cfg["V_D"], dmin, dmax, n)
    _, _, bi, bd = oracle.reference_lut_tables(cfg)
    assert pi.dtype == torch.bfloat16 and pd.dtype == torch.bfloat16 and pi.numel() == n
    assert np.array_equal(_bits(pi), _bits(bi))
    assert np.array_equal(_bits(pd), _bits(bd))
    ti64, td64 = oracle.lut_tables(cfg)
    assert np.count_nonzero(_rne_bits(td64) != _bits(bd)) > n // 4
