"""The IQ2_XXS fallback rows turn a codebook entry into signed bytes with a
table of byte masks (ornithology_amd/csrc/oh_mv.hip: iq2_sign_table,
iq2_terms8): for the 7 stored sign bits s7 of a group, the eighth sign is
their parity (the decoder's rule, src/ornith_quant.c:660-680), m byte j is
0xff where sign j is negative, and (g ^ m) + (m & 0x01..) is the entry g with
exactly those bytes negated, byte by byte without carries (every grid byte
is 8, 25 or 43). These CPU tests pin that identity against the plain form
sign_j * byte_j(g) for every sign pattern and every grid entry, and the
exactness the kernels rely on: (db * -g) * x == -((db * g) * x) in f32."""
import re

import numpy as np

import clibs


def _grid():
    text = (clibs.ROOT / "include" / "ornith_iq2xxs_grid.h").read_text()
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", text)]
    assert len(vals) == 256
    return np.array(vals, dtype=np.uint64)


def _masks(s7):
    # the table entry as the kernel builds it
    sg = s7 | ((bin(s7).count("1") & 1) << 7)
    m0 = m1 = 0
    for j in range(4):
        m0 |= ((sg >> j) & 1) * (0xFF << (8 * j))
        m1 |= ((sg >> (j + 4)) & 1) * (0xFF << (8 * j))
    return sg, m0, m1, m0 & 0x01010101, m1 & 0x01010101


def _signed_bytes(word):
    b = np.array([(word >> (8 * j)) & 0xFF for j in range(4)], dtype=np.int64)
    return np.where(b >= 128, b - 256, b)


def test_sign_masks_negate_exactly_the_signed_bytes():
    grid = _grid()
    for s7 in range(128):
        sg, m0, m1, m01lo, m01hi = _masks(s7)
        assert bin(sg).count("1") % 2 == 0          # the eighth sign makes the parity even
        sign = np.array([-1 if (sg >> j) & 1 else 1 for j in range(8)], dtype=np.int64)
        for g in grid:
            g = int(g)
            lo, hi = g & 0xFFFFFFFF, g >> 32
            gs_lo = ((lo ^ m0) + m01lo) & 0xFFFFFFFF
            gs_hi = ((hi ^ m1) + m01hi) & 0xFFFFFFFF
            got = np.concatenate([_signed_bytes(gs_lo), _signed_bytes(gs_hi)])
            mag = np.array([(g >> (8 * j)) & 0xFF for j in range(8)], dtype=np.int64)
            assert np.array_equal(got, sign * mag), (s7, hex(g))


def test_negated_grid_byte_gives_the_negated_term_in_f32():
    rng = np.random.default_rng(3)
    db = rng.standard_normal(4096).astype(np.float32) * np.float32(0.01)
    x = rng.standard_normal(4096).astype(np.float32)
    for g in (8, 25, 43):
        pos = (db * np.float32(g)) * x
        neg = (db * np.float32(-g)) * x
        assert np.array_equal(neg, -pos)
