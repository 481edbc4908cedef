"""GPU: the GQA attention output itself, before attn_output's Q8_K (which
absorbs any error smaller than one int8 step), against the oracle's
ornith_gqa_step (src/ornith_attn.c:87-149) over the same Q8 KV cache.

The engine's own cache, queries (after q_norm + RoPE) and gate are read back
after a decode step or a prompt chunk; the oracle attends over exactly those
positions (orc_gqa_attend), then o *= sigmoid(gate) as full_attn does
(src/ornith_rforward.c:419-455). This isolates the attention kernels from
everything upstream.

* Contexts inside the exact walk (<= 1024 positions): bit-identical.
* Past it: the flash decode on the matrix cores (ORNITH_HIP_FLASH_MFMA=1) and
  on the vector ALUs (=0), and the matrix-core prompt attention
  (oh_k_attn_mfma_rows), re-associate the softmax and V sums. Bar: relative
  L2 of the whole output vector <= 1e-5 for the decode forms and <= 1e-3 for
  the fp16-operand prompt kernel (the values are printed), also with K and V
  scales outside fp16's range.
Head geometries: C3's (16 q / 2 kv heads, head_dim 256) and C4's (32 / 2).
"""
import ctypes as C

import numpy as np
import pytest

import clibs
from clibs import OrcKV, f32p

pytestmark = pytest.mark.gpu

Q4 = dict(t_default=clibs.Q4_K, t_attn_v=clibs.Q4_K, t_ffn_down=clibs.Q4_K, t_output=clibs.Q4_K,
          t_embd=clibs.Q4_K)
# the last of the 4 layers is the full-attention layer (the one read back)
C3H = dict(clibs.C1, hidden=1024, n_layers=4, full_interval=4, vocab=512, nh=16, nkv=2, hd=256, nk=16, nv=32,
           dhead=128, ne=8, top_k=2, moe_inter=512, shared_inter=512, seed=13, **Q4)
C4H = dict(C3H, nh=32, nv=64, seed=14)


def oracle_attn(orc, kq, ks, vq, vs, T, nkv, hd, q, g, nh):
    """orc_gqa_attend over the first T cached positions, then * sigmoid(gate)"""
    kqT = np.ascontiguousarray(kq[:T * nkv * hd])
    vqT = np.ascontiguousarray(vq[:T * nkv * hd])
    ksT = np.ascontiguousarray(ks[:T * nkv])
    vsT = np.ascontiguousarray(vs[:T * nkv])
    kv = OrcKV()
    kv.Kq = kqT.ctypes.data_as(C.POINTER(C.c_int8))
    kv.Vq = vqT.ctypes.data_as(C.POINTER(C.c_int8))
    kv.Ks = ksT.ctypes.data_as(clibs.fp)
    kv.Vs = vsT.ctypes.data_as(clibs.fp)
    kv.quantized, kv.capacity, kv.len, kv.n_kv_heads, kv.head_dim = 1, T, T, nkv, hd
    out = np.zeros(nh * hd, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    orc.orc_gqa_attend(C.byref(kv), f32p(q), nh, f32p(out), C.c_float(0.0))
    sg = np.array([orc.orc_sigmoid(float(x)) for x in g], np.float32)
    return (out * sg).astype(np.float32)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


def check(orc, s, cfg, row):
    q, g, o, pos = s.attn(row)
    layer = cfg["n_layers"] - 1
    kq, ks, vq, vs = s.kv(layer)
    ref = oracle_attn(orc, kq, ks, vq, vs, pos + 1, cfg["nkv"], cfg["hd"], q, g, cfg["nh"])
    return o, ref, pos


@pytest.mark.parametrize("cfg", [C3H, C4H], ids=["c3-heads", "c4-heads"])
@pytest.mark.parametrize("form", ["1", "0"], ids=["flash-mfma", "flash-valu"])
def test_decode_attention_output_vs_oracle(hip_ctx, orc, monkeypatch, cfg, form):
    monkeypatch.setenv("ORNITH_HIP_FLASH_MFMA", form)
    m = hip_ctx.synth(**cfg)
    prompt = clibs.ids(31, "attn.prompt", 4100, cfg["vocab"])
    # exact walk: a short context, one decode step
    s = m.session(64)
    s.eval(prompt[:40])
    s.step(int(prompt[40]))
    o, ref, pos = check(orc, s, cfg, -1)
    assert pos == 40
    assert np.array_equal(o.view(np.uint32), ref.view(np.uint32)), rel_l2(o, ref)
    s.free()
    # past the exact walk: 4096 cached positions, then two decode steps
    s = m.session(4200)
    s.eval(prompt[:4096])
    worst = 0.0
    for k in range(2):
        s.step(int(prompt[4096 + k]))
        o, ref, pos = check(orc, s, cfg, -1)
        assert pos == 4096 + k
        r = rel_l2(o, ref)
        worst = max(worst, r)
        print(f"flash_mfma={form} pos {pos}: attention output rel L2 {r:.3e}, "
              f"max |d| {float(np.max(np.abs(o - ref))):.3e}")
        assert np.isfinite(o).all()
    assert worst <= 1e-5
    s.free()
    m.free()


@pytest.mark.parametrize("cfg", [C3H, C4H], ids=["c3-heads", "c4-heads"])
def test_prompt_attention_output_vs_oracle(hip_ctx, orc, monkeypatch, cfg):
    """one 1500-token prompt chunk: rows at positions < 1024 take the exact
    walk (bit-identical), the rest the matrix-core prompt attention"""
    m = hip_ctx.synth(**cfg)
    prompt = clibs.ids(32, "attn.prompt2", 1500, cfg["vocab"])
    s = m.session(1600)
    s.eval(prompt)
    o, ref, pos = check(orc, s, cfg, 700)
    assert pos == 700
    assert np.array_equal(o.view(np.uint32), ref.view(np.uint32)), rel_l2(o, ref)
    worst = 0.0
    for row in (1024, 1200, 1499):
        o, ref, pos = check(orc, s, cfg, row)
        r = rel_l2(o, ref)
        worst = max(worst, r)
        print(f"prompt row at pos {pos}: attention output rel L2 {r:.3e}")
        assert np.isfinite(o).all()
    assert worst <= 1e-3
    s.free()
    m.free()


def scale_kv_scales(path, cfg, layer, kexp, vexp):
    """multiply the cached K and V scales of a full-attention layer in an
    ORNSESS v1 file by 2^kexp and 2^vexp (exact)"""
    b = bytearray(open(path, "rb").read())
    off = 8 + 4 + 13 * 4 + 4 + 4 + 8 + 4                   # magic .. have_logits
    cc = 2 * cfg["nk"] * cfg["dhead"] + cfg["nv"] * cfg["dhead"]
    for l in range(cfg["n_layers"]):
        if (l + 1) % cfg["full_interval"]:
            off += cfg["nv"] * cfg["dhead"] * cfg["dhead"] * 4 + 8 + (cfg["conv_k"] - 1) * cc * 4
            continue
        quant, n, nkv, hd = np.frombuffer(bytes(b[off:off + 16]), np.int32)
        assert quant == 1 and nkv == cfg["nkv"] and hd == cfg["hd"]
        off += 16 + 2 * n * nkv * hd
        if l == layer:
            for e in (kexp, vexp):
                sc = np.frombuffer(bytes(b[off:off + 4 * n * nkv]), np.float32)
                b[off:off + 4 * n * nkv] = np.ldexp(sc, e).astype(np.float32).tobytes()
                off += 4 * n * nkv
        else:
            off += 8 * n * nkv
    open(path, "wb").write(bytes(b))


@pytest.mark.parametrize("cfg", [C3H, C4H], ids=["c3-heads", "c4-heads"])
@pytest.mark.parametrize("exp", [30, -30], ids=["scales-x2^30", "scales-x2^-30"])
def test_prompt_attention_fp16_range(hip_ctx, orc, monkeypatch, tmp_path, cfg, exp):
    """K and V scales far outside fp16's range (the cached scales of 200
    positions multiplied by 2^30 or 2^-30 through a session snapshot, codes
    times scale far past fp16's largest and below its smallest normal): the
    matrix-core prompt attention carries each scale's exponent in fp32, so a
    following 64-token chunk's rows (all past the exact walk, limited to 64
    positions here) stay within the same bar against the oracle over that
    cache."""
    monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", "64")
    m = hip_ctx.synth(**cfg)
    prompt = clibs.ids(33, "attn.prompt3", 264, cfg["vocab"])
    s = m.session(300)
    s.eval(prompt[:200])
    path = str(tmp_path / "kv.ornsess")
    s.save(path)
    s.free()
    layer = cfg["n_layers"] - 1
    scale_kv_scales(path, cfg, layer, exp, exp)
    s = m.load_session(path, 100)
    ks = s.kv(layer)[1]
    assert np.isfinite(ks).all()
    s.eval(prompt[200:])
    worst = 0.0
    for row in (0, 31, 63):
        o, ref, pos = check(orc, s, cfg, row)
        r = rel_l2(o, ref)
        worst = max(worst, r)
        print(f"scales x2^{exp}, prompt row at pos {pos}: attention output rel L2 {r:.3e} "
              f"(|o| max {float(np.max(np.abs(ref))):.3e})")
        assert np.isfinite(o).all()
    assert worst <= 1e-3
    s.free()
    m.free()
