"""GPU: ornith_qdot kernels through the C ABI against the oracle and the
reference's golden vectors. Bar: bit-exact (Q8_K bytes, decoded floats, dot
results, router indices and weights)."""
import numpy as np
import pytest

import clibs
from clibs import F32, IQ2_XXS, Q4_K, Q6_K, Q8_0, bp, f32p, i32p

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "codecs.npz")


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def q8k_cases():
    rng = np.random.default_rng(1)
    out = [GOLD["act2048"], GOLD["act512"], np.zeros(512, np.float32)]
    for sc in (1e-3, 1.0, 1e3):
        out.append((rng.standard_normal(4096) * sc).astype(np.float32))
    t = np.zeros(256, np.float32); t[7], t[200] = -3.0, 3.0
    out.append(t)
    t2 = np.array([(k % 9) - 4.5 for k in range(256)], np.float32); t2[0] = -127.0
    out.append(t2)
    out.append(np.concatenate([np.zeros(256, np.float32), rng.standard_normal(256).astype(np.float32)]))
    out.append((rng.standard_normal(16384)).astype(np.float32))   # two 8192-element passes
    return out


def test_q8k_bitexact(hip_ctx, orc):
    for i, x in enumerate(q8k_cases()):
        got = hip_ctx.quantize_q8k(x)
        ref = clibs.q8k(orc, x)
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), i
    assert np.array_equal(hip_ctx.quantize_q8k(GOLD["act2048"]).view(np.uint8), GOLD["act2048_q8k"])


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, IQ2_XXS])
@pytest.mark.parametrize("n", [2048, 512])
def test_matvec_and_decode_golden(hip_ctx, t, n):
    name = clibs.TYPE_NAMES[t]
    W = hip_ctx.upload(f"w.{name}.{n}", t, GOLD[f"{name}_{n}_enc"], (n, 16))
    y = W.matvec(GOLD[f"act{n}"])
    assert np.array_equal(u32(y), u32(GOLD[f"{name}_{n}_dot"]))
    d = W.dequant()
    assert np.array_equal(u32(d), u32(GOLD[f"{name}_{n}_dec"]))
    W.free()


SHAPES = [(2048, 4096), (512, 2048), (4096, 300), (256, 64), (8192, 96), (1024, 257), (3072, 40)]


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("shape", SHAPES)
def test_matvec_vs_oracle(hip_ctx, orc, t, shape):
    n, out = shape
    name = clibs.TYPE_NAMES[t]
    w = clibs.gauss(5, f"mv.{name}.{n}.{out}", n * out, 0.02)
    enc = clibs.quantize(orc, t, w)
    x = clibs.gauss(6, f"x.{n}", n, 1.0)
    ref = np.zeros(out, np.float32)
    orc.orc_matvec(t, bp(enc), n, out, f32p(x), f32p(ref), 0, 8)
    W = hip_ctx.upload("w", t, enc, (n, out))
    y = W.matvec(x)
    assert np.array_equal(u32(y), u32(ref)), f"{name} {shape}: {np.nonzero(u32(y) != u32(ref))[0][:8]}"
    # several columns in one call (matmul_batch_q Tn semantics)
    x3 = np.concatenate([x, -x, x * np.float32(0.5)])
    y3 = W.matvec(x3)
    for c, xc in enumerate((x, -x, x * np.float32(0.5))):
        r = np.zeros(out, np.float32)
        orc.orc_matvec(t, bp(enc), n, out, f32p(np.ascontiguousarray(xc)), f32p(r), 0, 8)
        assert np.array_equal(u32(y3[c * out:(c + 1) * out]), u32(r))
    if n <= 2048:
        # more columns than one LDS tile of the batched kernel
        cols = [x * np.float32(1.0 + 0.25 * k) for k in range(70)]
        y70 = W.matvec(np.concatenate(cols))
        for c in (0, 1, 31, 32, 63, 64, 69):
            r = np.zeros(out, np.float32)
            orc.orc_matvec(t, bp(enc), n, out, f32p(np.ascontiguousarray(cols[c])), f32p(r), 0, 8)
            assert np.array_equal(u32(y70[c * out:(c + 1) * out]), u32(r)), (c, name, shape)
    W.free()


@pytest.mark.parametrize("t", [Q4_K, Q6_K], ids=["Q4_K", "Q6_K"])
@pytest.mark.parametrize("shape,ncol", [((2048, 1024), 70), ((512, 384), 1), ((4096, 256), 130), ((1024, 200), 65),
                                         ((512, 256), 70), ((256, 128), 65)])
def test_batched_q4k_distinct_columns(hip_ctx, orc, monkeypatch, shape, ncol, t):
    """Batched Q4_K / Q6_K products (matmul_batch_q Tn semantics) on
    independent columns: the matrix-core path (rows a multiple of 128) and the
    vector-ALU path (ORNITH_HIP_MMQ=0, and 200 rows) both equal the oracle's
    per-column qdot bit for bit; partial 64-column tiles included. K = 512 and
    256 take the one-stage Q6_K kernel, the longer rows the two-stage one."""
    n, out = shape
    w = clibs.gauss(11, f"bq.{n}.{out}", n * out, 0.02)
    if t == Q6_K:
        w = w * np.float32(40.0)          # wide code and scale ranges (large |sc * (q6 - 32)|)
    enc = clibs.quantize(orc, t, w)
    W = hip_ctx.upload("w", t, enc, (n, out))
    cols = [clibs.gauss(12 + c, f"bx.{n}.{c}", n, 1.0) for c in range(ncol)]
    ref = []
    for c in range(ncol):
        r = np.zeros(out, np.float32)
        orc.orc_matvec(t, bp(enc), n, out, f32p(np.ascontiguousarray(cols[c])), f32p(r), 0, 8)
        ref.append(r)
    for mmq in ("1", "0"):
        monkeypatch.setenv("ORNITH_HIP_MMQ", mmq)
        y = W.matvec(np.concatenate(cols))
        for c in range(ncol):
            got = y[c * out:(c + 1) * out]
            assert np.array_equal(u32(got), u32(ref[c])), (mmq, c, np.nonzero(u32(got) != u32(ref[c]))[0][:8])
    W.free()


@pytest.mark.parametrize("t,shape", [(IQ2_XXS, (2048, 48)), (IQ2_XXS, (512, 33)), (F32, (512, 100)), (F32, (1000, 7))])
def test_fallback_matvec_vs_oracle(hip_ctx, orc, t, shape):
    n, out = shape
    w = clibs.gauss(8, f"fb.{t}.{n}", n * out, 0.02)
    enc = clibs.quantize(orc, t, w) if t != F32 else w.view(np.uint8)
    x = clibs.gauss(9, f"xf.{n}", n, 1.0)
    ref = np.zeros(out, np.float32)
    orc.orc_matvec(t, bp(enc), n, out, f32p(x), f32p(ref), 0, 8)
    W = hip_ctx.upload("w", t, enc, (n, out))
    assert np.array_equal(u32(W.matvec(x)), u32(ref))
    if t != F32:
        assert np.array_equal(u32(W.dequant()), u32(clibs.dequantize(orc, t, enc, n * out)))
    W.free()


def test_expert_stack_rows(hip_ctx, orc):
    """A 3-D [in, out, ne] stack decodes and multiplies as ne*out rows."""
    n, out, ne = 512, 64, 6
    w = clibs.gauss(10, "stack", n * out * ne, 0.02)
    enc = clibs.quantize(orc, Q4_K, w)
    W = hip_ctx.upload("stack", Q4_K, enc, (n, out, ne))
    x = clibs.gauss(11, "xs", n, 1.0)
    ref = np.zeros(out * ne, np.float32)
    orc.orc_matvec(Q4_K, bp(enc), n, out * ne, f32p(x), f32p(ref), 0, 8)
    assert np.array_equal(u32(W.matvec(x)), u32(ref))
    assert np.array_equal(u32(W.dequant(out * 3, out)), u32(clibs.dequantize(orc, Q4_K, enc, n * out * ne)[n * out * 3: n * out * 4]))
    W.free()


def test_router_bitexact(hip_ctx, orc):
    rng = np.random.default_rng(4)
    for trial in range(60):
        ne = int(rng.choice([16, 64, 256, 512]))
        k = int(rng.choice([1, 4, 8, 10]))
        lg = (rng.standard_normal(ne) * 2).astype(np.float32)
        if trial % 3 == 0:
            lg = np.round(lg, 1).astype(np.float32)     # exact ties
        i1, w1 = hip_ctx.moe_route(lg, k)
        i2, w2 = np.zeros(k, np.int32), np.zeros(k, np.float32)
        orc.orc_moe_route(f32p(lg), ne, k, i32p(i2), f32p(w2))
        assert np.array_equal(i1, i2) and np.array_equal(u32(w1), u32(w2)), trial
    i, w = hip_ctx.moe_route(np.float32([0.1, 2.0, -1.0, 1.5, 0.5, 1.9]), 3)
    assert list(i) == [1, 5, 3]


def test_upload_rejects_bad_sizes(hip_ctx):
    import ornithology_amd as oa
    with pytest.raises(oa.HipError):
        hip_ctx.upload("bad", Q4_K, np.zeros(100, np.uint8), (256, 1))
    with pytest.raises(oa.HipError):
        hip_ctx.upload("bad2", Q8_0, np.zeros(34, np.uint8), (32, 1))   # 32-wide Q8_0 rows unsupported


CODECS = np.load(clibs.ROOT / "tests" / "golden" / "codecs.npz")


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, IQ2_XXS])
@pytest.mark.parametrize("n", [2048, 512])
def test_device_encoders_equal_reference(hip_ctx, t, n):
    """oq_quantize on the device against the reference's own encodings of the
    same N(0, 0.02) rows (golden codecs.npz), byte for byte."""
    tn = clibs.TYPE_NAMES[t]
    w = clibs.gauss(0, f"w.{tn}.{n}", 16 * n, 0.02)
    got = hip_ctx.quantize(t, w)
    want = CODECS[f"{tn}_{n}_enc"]
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:8]


def test_iq2xxs_encoder_edge_blocks(hip_ctx, orc):
    """IQ2_XXS edge cases against the oracle encoder (pinned to the reference
    by the golden rows): an all-zero block, a block with one zero group, an odd
    number of negatives with tied smallest magnitudes, and large values."""
    rng = np.random.default_rng(3)
    blocks = [np.zeros(256, np.float32)]
    b = rng.normal(0, 0.02, 256).astype(np.float32)
    b[32:64] = 0.0
    blocks.append(b)
    c = np.full(256, 0.01, np.float32)
    c[::3] *= -1.0
    blocks.append(c)
    blocks.append(rng.normal(0, 30.0, 256).astype(np.float32))
    x = np.concatenate(blocks)
    assert np.array_equal(hip_ctx.quantize(IQ2_XXS, x), clibs.quantize(orc, IQ2_XXS, x))
