"""The random stream: Philox4x32-10 pinned by the Random123 known-answer vectors, the
uniform mapping, and the literal-draw assembly from bit-planes."""
import numpy as np
import pytest

import pyref

# Random123 kat_vectors, philox4x32_10 (ctr, key, expected output).
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expected", KAT)
def test_philox_kat_c_oracle(oracle_mod, ctr, key, expected):
    assert tuple(int(v) for v in oracle_mod.philox4x32_10(ctr, key)) == expected


@pytest.mark.parametrize("ctr,key,expected", KAT)
def test_philox_kat_pyref(ctr, key, expected):
    assert pyref.philox(ctr, key) == expected


def test_philox_c_matches_pyref_random(oracle_mod):
    rng = np.random.default_rng(1)
    for _ in range(200):
        ctr = [int(v) for v in rng.integers(0, 2**32, 4)]
        key = [int(v) for v in rng.integers(0, 2**32, 2)]
        assert tuple(int(v) for v in oracle_mod.philox4x32_10(ctr, key)) == pyref.philox(ctr, key)


def test_uniform_endpoints(oracle_mod):
    # u = ((z >> 8) + 1) * 2^-24 lies in (0, 1]; both ends are reachable and exact.
    assert oracle_mod.uniform_from_word(0) == 2.0**-24
    assert oracle_mod.uniform_from_word(0xFFFFFFFF) == 1.0
    assert oracle_mod.uniform_from_word(0x000000FF) == 2.0**-24  # low byte ignored
    assert oracle_mod.uniform_from_word(0x80000000) == 0.5 + 2.0**-24


def test_u_lit_matches_plane_definition(oracle_mod):
    """orc_u_lit (all 24 planes) equals an independent per-literal assembly."""
    tm = oracle_mod.OracleTM(3, 10, 3.9, (20, 1, 1), 3, seed=123456789)
    st = pyref.Stream(123456789, tm.C, tm.K, tm.P, tm.L, tm.W)
    for t, c, k, l in [(0, 0, 0, 0), (5, 2, 1, 31), (7, 1, 2, 39), (2**33 + 5, 2, 0, 17)]:
        assert tm.u_lit(t, c, k, l) == st.lit(0, t, c, k, l)


def test_literal_draw_rate(oracle_mod):
    """P(u <= 1/s) over many literal draws is 1/s within 5 sigma (a dropped or swapped
    plane would skew it)."""
    tm = oracle_mod.OracleTM(2, 10, 3.9, (20, 1, 1), 2, seed=5)
    us = np.array([tm.u_lit(t, c, k, l) for t in range(40) for c in range(2) for k in range(2) for l in range(40)])
    p = 1 / 3.9
    n = us.size
    assert abs((us <= p).mean() - p) < 5 * np.sqrt(p * (1 - p) / n)
    assert abs(us.mean() - 0.5) < 5 * np.sqrt(1 / 12 / n)
