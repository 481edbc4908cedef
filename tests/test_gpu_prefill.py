"""GPU: the layer-major prefill (every layer over a chunk of prompt tokens with
batched projections, src/ornith_rforward.c:647-682) in both of the
reference's prompt modes: ORNITH_PREFILL_SERIAL=1 (token recurrence) against
the reference and against the token-by-token path (ORNITH_HIP_PREFILL=0), and
the default chunked delta scan (src/ornith_attn.c:215-349) against the
reference's golden fixture and the oracle. MoE models with IQ2_XXS routed
experts take the same batched path with the experts per (token, expert) slot
(the reference's prompt runs ffn_moe per token).

Bar: bit-exact prompt logits and 64 greedy tokens on C1 against the
reference's serial golden fixture; bit-identical logits, tokens and session
state (delta state, conv window, Q8 KV cache) between the two paths, and
against the oracle's chunked mode, on Q4_K/Q6_K models with MoE and dense FFNs,
on prompts that span several chunks, with odd and even chunk starts and
partial delta chunks, on the exact and flash attention paths."""
import ctypes as C

import numpy as np
import pytest

import clibs
from clibs import i32p

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")

MIX = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=512, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, seed=5)
DENSE = dict(MIX, ne=0, top_k=0, moe_inter=0, shared_inter=1024, seed=7)


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_prefill_c1_matches_reference(hip_ctx, monkeypatch):
    monkeypatch.setenv("ORNITH_HIP_PREFILL", "1")
    m = hip_ctx.synth(**clibs.C1)
    s = m.session(104)
    s.eval(GOLD["prompt"])
    assert np.array_equal(u32(s.logits()), u32(GOLD["serial_prompt_logits"]))
    assert np.array_equal(s.generate(64), GOLD["serial_tokens"])
    s.free()
    m.free()


def test_prefill_dense_matches_oracle(hip_ctx, orc, tmp_path, monkeypatch):
    """A dense-FFN model (ffn_gate/ffn_up/ffn_down, src/ornith_rforward.c:325-333)
    against the oracle's token path: prompt logits bit-exact."""
    monkeypatch.setenv("ORNITH_HIP_PREFILL", "1")
    path = tmp_path / "dense.gguf"
    clibs.write_c1_gguf(path, DENSE)
    om = C.c_void_p()
    assert orc.orc_model_load(str(path).encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    os_ = orc.orc_session_new(om, 40, 1)
    p = np.random.default_rng(4).integers(0, DENSE["vocab"], 20).astype(np.int32)
    assert orc.orc_session_eval(os_, i32p(p), 20, 1) == 0
    want = np.ctypeslib.as_array(orc.orc_session_logits(os_), (DENSE["vocab"],)).copy()
    m = hip_ctx.synth(**DENSE)
    s = m.session(40)
    s.eval(p)
    assert np.array_equal(u32(s.logits()), u32(want))
    s.free()
    m.free()
    orc.orc_session_free(os_)
    orc.orc_model_free(om)


def evals(m, chunks, cap, prefill, monkeypatch, exact_max):
    monkeypatch.setenv("ORNITH_HIP_PREFILL", "1" if prefill else "0")
    monkeypatch.setenv("ORNITH_HIP_PREFILL_CHUNK", "96")
    # the prompt's flash chunks are the decode step's VALU flash chunks
    # (bit-identical); the matrix-core prompt and decode attention are checked
    # to tolerance (below and in test_gpu_flash_decode.py)
    monkeypatch.setenv("ORNITH_HIP_ATTN_MFMA", "0")
    monkeypatch.setenv("ORNITH_HIP_FLASH_MFMA", "0")
    if exact_max is not None:
        monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", str(exact_max))
    s = m.session(cap)
    logits = []
    for c in chunks:
        s.eval(c)
        logits.append(s.logits().copy())
    return s, logits


def oracle_state(orc, os_, arch, layer, pos):
    """The oracle session's state in the layouts of Session.delta_state/conv_state/kv."""
    if (layer + 1) % arch["full_interval"]:
        cc = 2 * arch["nk"] * arch["dk"] + arch["nv"] * arch["dv"]
        S = np.ctypeslib.as_array(orc.orc_session_delta(os_, layer), (arch["nv"] * arch["dv"] * arch["dk"],))
        W = np.ctypeslib.as_array(orc.orc_session_conv(os_, layer), ((arch["conv_k"] - 1) * cc,))
        return S.copy(), W.copy()
    kv = orc.orc_session_kv(os_, layer).contents
    n = pos * arch["nkv"] * arch["hd"]
    return (np.ctypeslib.as_array(kv.Kq, (n,)).copy(), np.ctypeslib.as_array(kv.Ks, (pos * arch["nkv"],)).copy(),
            np.ctypeslib.as_array(kv.Vq, (n,)).copy(), np.ctypeslib.as_array(kv.Vs, (pos * arch["nkv"],)).copy())


@pytest.mark.parametrize("cfg", ["moe", "dense"])
def test_chunked_mode_matches_oracle(hip_ctx, orc, tmp_path, monkeypatch, cfg):
    """The reference's default prompt mode over several evaluations: a
    300-token prompt (engine chunks of 96 tokens: four, the last partial,
    with a partial last delta chunk), then 7, 1 (a one-token chunk) and 33
    tokens; logits after each and the whole session state bit-identical to
    the oracle's chunked mode."""
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")
    monkeypatch.setenv("ORNITH_HIP_PREFILL_CHUNK", "96")
    c = MIX if cfg == "moe" else DENSE
    path = tmp_path / "m.gguf"
    clibs.write_c1_gguf(path, c)
    om = C.c_void_p()
    assert orc.orc_model_load(str(path).encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    os_ = orc.orc_session_new(om, 400, 1)
    m = hip_ctx.synth(**c)
    a = m.arch
    s = m.session(400)
    rng = np.random.default_rng(6)
    for n in (300, 7, 1, 33):
        p = rng.integers(0, a["vocab"], n).astype(np.int32)
        assert orc.orc_session_eval(os_, i32p(p), n, 0) == 0
        s.eval(p)
        want = np.ctypeslib.as_array(orc.orc_session_logits(os_), (a["vocab"],))
        assert np.array_equal(u32(s.logits()), u32(want)), n
    for l in range(a["n_layers"]):
        want = oracle_state(orc, os_, a, l, s.pos)
        got = (s.delta_state(l), s.conv_state(l)) if (l + 1) % a["full_interval"] else s.kv(l)
        for x, y in zip(got, want):
            assert np.array_equal(np.ascontiguousarray(x).view(np.uint8), np.ascontiguousarray(y).view(np.uint8)), l
    s.free()
    m.free()
    orc.orc_session_free(os_)
    orc.orc_model_free(om)


def same_state(m, a, b):
    arch = m.arch
    assert a.pos == b.pos
    for l in range(arch["n_layers"]):
        if (l + 1) % arch["full_interval"]:
            assert np.array_equal(u32(a.delta_state(l)), u32(b.delta_state(l))), l
            assert np.array_equal(u32(a.conv_state(l)), u32(b.conv_state(l))), l
        else:
            for x, y in zip(a.kv(l), b.kv(l)):
                assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), l


HD256 = dict(MIX, hd=256, seed=9)     # head_dim 256: the four-token exact prompt walk
# IQ2_XXS routed experts (C4's type): the prompt runs the token step's expert
# kernels over its (token, expert) slots, in the f32 fallback's element order
# or (ORNITH_HIP_IQ2_TREE=1) as tree-summed gate/up pairs
IQ2X = dict(MIX, t_exps=clibs.IQ2_XXS, seed=13)


@pytest.mark.parametrize("cfg", ["moe", "dense", "hd256", "iq2", "iq2-tree"])
@pytest.mark.parametrize("exact_max", [None, 0], ids=["exact", "flash"])
def test_prefill_equals_token_path(hip_ctx, monkeypatch, cfg, exact_max):
    if cfg == "iq2-tree":
        monkeypatch.setenv("ORNITH_HIP_IQ2_TREE", "1")
    m = hip_ctx.synth(**{"moe": MIX, "dense": DENSE, "hd256": HD256, "iq2": IQ2X, "iq2-tree": IQ2X}[cfg])
    a = m.arch
    rng = np.random.default_rng(3)
    # 300 tokens span four engine chunks of 96; then evals starting at odd and
    # even positions
    chunks = [rng.integers(0, a["vocab"], n).astype(np.int32) for n in (300, 7, 2, 33)]
    sp, lp = evals(m, chunks, 400, True, monkeypatch, exact_max)
    st, lt = evals(m, chunks, 400, False, monkeypatch, exact_max)
    for x, y in zip(lp, lt):
        assert np.array_equal(u32(x), u32(y))
    same_state(m, sp, st)
    assert np.array_equal(sp.generate(24), st.generate(24))
    assert np.array_equal(u32(sp.logits()), u32(st.logits()))
    sp.free()
    st.free()
    m.free()


@pytest.mark.parametrize("cfg,n,exact_max,chunk", [("moe", 300, 64, 96), ("c1", 1200, None, 2048)],
                         ids=["moe-hd128-chunks", "c1-hd64-past-1024"])
def test_mfma_prompt_attention_within_tolerance(hip_ctx, orc, tmp_path, monkeypatch, cfg, n, exact_max, chunk):
    """Prompt attention past the exact walk on the matrix cores (fp16 operands
    with the Q8 scales folded in, fp32 accumulation and online softmax):
    against the reference order (the oracle's chunked mode) the prompt logits
    stay within 1e-2 relative L2 and pick the same next token, for prompts that
    cross the exact-walk limit, inside one engine chunk and over several. The
    flash chunks (ORNITH_HIP_ATTN_MFMA=0) on the same prompt meet the same bar."""
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")
    monkeypatch.setenv("ORNITH_HIP_PREFILL_CHUNK", str(chunk))
    if exact_max is not None:
        monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", str(exact_max))
    c = MIX if cfg == "moe" else clibs.C1
    path = tmp_path / "m.gguf"
    clibs.write_c1_gguf(path, c)
    om = C.c_void_p()
    assert orc.orc_model_load(str(path).encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    os_ = orc.orc_session_new(om, n + 8, 1)
    p = np.random.default_rng(8).integers(0, c["vocab"], n).astype(np.int32)
    assert orc.orc_session_eval(os_, i32p(p), n, 0) == 0
    want = np.ctypeslib.as_array(orc.orc_session_logits(os_), (c["vocab"],)).copy()
    orc.orc_session_free(os_)
    orc.orc_model_free(om)
    m = hip_ctx.synth(**c)
    for mfma in ("1", "0"):
        monkeypatch.setenv("ORNITH_HIP_ATTN_MFMA", mfma)
        s = m.session(n + 8)
        s.eval(p)
        got = s.logits()
        rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
        print(f"{cfg} n={n} mfma={mfma}: rel L2 {rel:.3e}")
        assert np.isfinite(got).all() and rel < 1e-2, (mfma, rel)
        assert int(np.argmax(got)) == int(np.argmax(want)), mfma
        s.free()
    m.free()
