"""CPU: the oracle's codecs, Q8_K quantiser and integer dots.

Pinned against (a) the reference's own outputs committed in tests/golden/
(codecs.npz, written by tests/golden/make_golden.py from oracle/_ref), (b) the
known answers and error bounds of the reference tests (tests/test_quant.c,
tests/test_qdot.c), (c) closed forms: IEEE binary16 via numpy, exact integer
brute force of the qdot inner sums, construction of rounding ties.
"""
import hashlib
import re
import struct

import numpy as np
import pytest

import clibs
from clibs import F32, IQ2_XXS, Q4_K, Q6_K, Q8_0, bp, f32p

GOLD = np.load(clibs.ROOT / "tests" / "golden" / "codecs.npz")


def test_iq2xxs_grid_hash():
    text = (clibs.ROOT / "include" / "ornith_iq2xxs_grid.h").read_text()
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", text)]
    assert len(vals) == 256
    raw = b"".join(struct.pack("<Q", v) for v in vals)
    assert hashlib.sha256(raw).hexdigest() == "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54"
    mags = {(v >> (8 * j)) & 0xFF for v in vals for j in range(8)}
    assert mags == {8, 25, 43}
    assert vals[0] == 0x0808080808080808 and vals[255] == 0x2B2B2B1908081908


def test_block_geometry(orc):
    # tests/test_quant.c:108-180
    assert orc.orc_row_bytes(Q8_0, 64) == 68 and orc.orc_row_bytes(Q8_0, 7) == 0
    assert orc.orc_row_bytes(Q4_K, 256) == 144 and orc.orc_row_bytes(Q6_K, 256) == 210
    assert orc.orc_row_bytes(IQ2_XXS, 512) == 132


def test_f16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.orc_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_round_to_nearest_even(orc):
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # bias toward the f16 range, include subnormal/overflow edges and exact ties
    ties = (np.arange(1, 2048, dtype=np.uint32) << 13 | 0x1000) + (112 << 23)
    x = np.concatenate([bits.view(np.float32), (rng.standard_normal(100000) * 300).astype(np.float32),
                        ties.view(np.float32), np.float32([6.1e-5, 5.96e-8, 2.98e-8, 65504, 65520, 1e9, -0.0])])
    x = x[~np.isnan(x)]
    got = np.array([orc.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    # known values (tests/test_quant.c:114-116)
    for v in (1.0, -0.5, 0.0):
        assert orc.orc_f16_to_f32(orc.orc_f32_to_f16(v)) == v


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, IQ2_XXS])
@pytest.mark.parametrize("n", [2048, 512])
def test_codecs_match_reference_bytes(orc, t, n):
    name = clibs.TYPE_NAMES[t]
    w = clibs.gauss(0, f"w.{name}.{n}", 16 * n, 0.02)
    enc = clibs.quantize(orc, t, w)
    assert np.array_equal(enc, GOLD[f"{name}_{n}_enc"]), "encoder bytes differ from the reference"
    dec = clibs.dequantize(orc, t, enc, 16 * n)
    assert np.array_equal(dec.view(np.uint32), GOLD[f"{name}_{n}_dec"].view(np.uint32))


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, IQ2_XXS])
@pytest.mark.parametrize("n", [2048, 512])
def test_dots_match_reference_bits(orc, t, n):
    name = clibs.TYPE_NAMES[t]
    x = GOLD[f"act{n}"]
    xq = clibs.q8k(orc, x)
    assert np.array_equal(xq.view(np.uint8), GOLD[f"act{n}_q8k"])
    enc = GOLD[f"{name}_{n}_enc"]
    rb = clibs.row_bytes(t, n)
    out = np.zeros(16, np.float32)
    orc.orc_matvec(t, bp(enc), n, 16, f32p(np.ascontiguousarray(x)), f32p(out), 0, 1)
    assert np.array_equal(out.view(np.uint32), GOLD[f"{name}_{n}_dot"].view(np.uint32))
    if orc.orc_qdot_can(t, n):
        for r in range(16):
            row = np.ascontiguousarray(enc[r * rb:(r + 1) * rb])
            assert orc.orc_qdot(t, n, bp(row), bp(xq)) == out[r]


def test_roundtrip_bounds(orc):
    # tests/test_quant.c:130-255
    src = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.3)) * 5).astype(np.float32)
    amax = np.abs(src).max()
    d = clibs.dequantize(orc, Q8_0, clibs.quantize(orc, Q8_0, src), 64)
    assert np.abs(d - src).max() <= amax / 127 + 1e-4
    i = np.arange(256, dtype=np.float32)
    k = (np.sin(i * np.float32(0.11)) * 0.6 + np.cos(i * np.float32(0.37)) * 0.2).astype(np.float32)
    kamax = np.abs(k).max()
    d6 = clibs.dequantize(orc, Q6_K, clibs.quantize(orc, Q6_K, k), 256)
    assert np.abs(d6 - k).max() < kamax / 30
    d4 = clibs.dequantize(orc, Q4_K, clibs.quantize(orc, Q4_K, k), 256)
    assert np.abs(d4 - k).max() < kamax / 8
    di = clibs.dequantize(orc, IQ2_XXS, clibs.quantize(orc, IQ2_XXS, k), 256)
    assert np.isfinite(di).all()
    assert ((di - k) ** 2).sum() < 0.5 * (k ** 2).sum()
    big = np.abs(k) > 0.5 * kamax
    assert np.all((k[big] > 0) == (di[big] >= 0))


def test_iq2xxs_sign_parity(orc):
    # every decoded 8-group has an even number of negative entries: bit 7 of a
    # sign byte is the parity of its low 7 bits
    w = clibs.gauss(3, "parity", 256 * 8, 1.0)
    d = clibs.dequantize(orc, IQ2_XXS, clibs.quantize(orc, IQ2_XXS, w), w.size).reshape(-1, 8)
    assert np.all((d < 0).sum(axis=1) % 2 == 0)


def q8k_numpy_props(x, blk):
    """Closed-form properties of a Q8_K block."""
    q = blk["qs"].astype(np.int32)
    assert q.min() >= -128 and q.max() <= 127
    assert np.array_equal(q.reshape(16, 16).sum(1), blk["bsums"].astype(np.int32))
    d = np.float32(blk["d"])
    if np.abs(x).max() == 0:
        assert d == 0 and not q.any()
        return
    j = int(np.argmax(np.abs(x)))          # first index of the largest magnitude
    iscale = np.float32(-127.0) / x[j]
    assert d == np.float32(1.0) / iscale
    assert np.array_equal(q, np.clip(np.rint(iscale * x), -128, 127).astype(np.int32))


def test_q8k_properties_and_ties(orc):
    rng = np.random.default_rng(11)
    cases = [rng.standard_normal(256).astype(np.float32), np.zeros(256, np.float32)]
    t = np.zeros(256, np.float32)
    t[3], t[10] = 2.0, -2.0                  # equal magnitudes: the first sets the sign
    cases.append(t)
    t2 = np.array([(k % 9) - 4.5 for k in range(256)], np.float32)
    t2[0] = -127.0                           # iscale = 1: x.5 values are exact rint ties
    cases.append(t2)
    for x in cases:
        blk = clibs.q8k(orc, x)[0]
        q8k_numpy_props(x, blk)
    b = clibs.q8k(orc, cases[2])[0]
    assert b["d"] < 0 and b["qs"][3] == -127 and b["qs"][10] == 127
    b2 = clibs.q8k(orc, cases[3])[0]
    # x = -3.5 .. 3.5 at iscale 1: round half to even (lrintf)
    assert list(b2["qs"][1:9]) == [-4, -2, -2, 0, 0, 2, 2, 4]


def _unpack_q4k(blk):
    d = np.frombuffer(blk[0:2].tobytes(), np.float16)[0].astype(np.float32)
    dmin = np.frombuffer(blk[2:4].tobytes(), np.float16)[0].astype(np.float32)
    s = blk[4:16].astype(np.int32)
    sc, mn = np.zeros(8, np.int64), np.zeros(8, np.int64)
    for j in range(8):
        if j < 4:
            sc[j], mn[j] = s[j] & 63, s[j + 4] & 63
        else:
            sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
            mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    qs = blk[16:144].astype(np.int64)
    lv = np.zeros(256, np.int64)
    for j in range(8):
        b = qs[32 * (j // 2): 32 * (j // 2) + 32]
        lv[32 * j:32 * j + 32] = (b >> (4 * (j & 1))) & 15
    return d, dmin, sc, mn, lv


def test_qdot_q4k_integer_brute_force(orc):
    rng = np.random.default_rng(2)
    n = 1024
    w = (rng.standard_normal(n) * 0.05).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    enc = clibs.quantize(orc, Q4_K, w)
    xq = clibs.q8k(orc, x)
    acc = np.float32(0)
    for i in range(n // 256):
        d, dmin, sc, mn, lv = _unpack_q4k(enc[144 * i:144 * i + 144])
        q8 = xq[i]["qs"].astype(np.int64)
        isum = int(sum(sc[j] * (lv[32 * j:32 * j + 32] * q8[32 * j:32 * j + 32]).sum() for j in range(8)))
        mins = int(sum(mn[j] * (int(xq[i]["bsums"][2 * j]) + int(xq[i]["bsums"][2 * j + 1])) for j in range(8)))
        yd = np.float32(xq[i]["d"])
        term = np.float32(np.float32(yd * d) * np.float32(isum)) + np.float32(np.float32(-yd * dmin) * np.float32(mins))
        acc = np.float32(acc + np.float32(term))
    assert orc.orc_qdot(Q4_K, n, bp(enc), bp(xq)) == acc


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0])
def test_qdot_tracks_f32_dot(orc, t):
    # tests/test_qdot.c:33-85: relative error vs dequant . f32 activation < 3e-2
    n = 512
    i = np.arange(n, dtype=np.float32)
    w = (np.sin(i * np.float32(0.11)) * 0.6 + np.cos(i * np.float32(0.37)) * 0.2).astype(np.float32)
    x = (np.cos(i * np.float32(0.07)) * 1.3 - np.sin(i * np.float32(0.19)) * 0.5).astype(np.float32)
    enc = clibs.quantize(orc, t, w)
    wd = clibs.dequantize(orc, t, enc, n).astype(np.float64)
    got = orc.orc_qdot(t, n, bp(enc), bp(clibs.q8k(orc, x)))
    ref = float(wd @ x.astype(np.float64))
    assert abs(got - ref) / (abs(ref) + 1e-6) < 3e-2


def test_qdot_gates(orc):
    # tests/test_qdot.c:64-66
    assert not orc.orc_qdot_can(Q4_K, 200)
    assert not orc.orc_qdot_can(13, 256)       # Q5_K
    assert not orc.orc_qdot_can(F32, 256)
    assert orc.orc_qdot_can(Q8_0, 256) and orc.orc_qdot_can(Q6_K, 512)
