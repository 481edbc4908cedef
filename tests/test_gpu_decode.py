"""GPU: the decode step as one persistent launch (oh_k_decode, opt-in with
ORNITH_HIP_DECODE=1) against the per-launch HIP-graph step (ORNITH_HIP_DECODE=0),
which the other GPU tests pin to the oracle and the reference's golden
vectors. Bar: bit-identical logits after every step and identical greedy
tokens, over prompts through the layer-major prefill followed by decode
steps, on C1 (all Q8_0), a Q4_K_M mix (Q6_K attn_v / ffn_down: the split
input projection and the Q6_K down projection), C3's head geometry, and
contexts past the exact attention walk (flash chunks, both forms). C1's
greedy tokens also equal the reference build's golden fixture."""
import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu

GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")
Q4M = dict(t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K, t_ffn_down=clibs.Q6_K, t_output=clibs.Q4_K,
           t_embd=clibs.Q4_K)
MIX = dict(clibs.C1, hidden=1024, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=512, seed=5, **Q4M)
C3H = dict(clibs.C1, hidden=1024, n_layers=4, full_interval=4, vocab=512, nh=16, nkv=2, hd=256, nk=16, nv=32,
           dhead=128, ne=8, top_k=2, moe_inter=512, shared_inter=512, seed=13, **Q4M)


def run(model, prompt, steps, fused=False):
    if fused:
        # the decode launch exists for this model (profile_decode raises
        # otherwise); it runs a real step, so on a session of its own
        p = model.session(prompt.size + 8)
        p.eval(prompt)
        assert len(p.profile_decode()) > 0
        p.free()
    s = model.session(prompt.size + steps + 8)
    s.eval(prompt)
    out = [s.logits().copy()]
    toks = []
    for _ in range(steps):
        t = int(np.argmax(out[-1]))
        toks.append(t)
        s.step(t)
        out.append(s.logits().copy())
    gen = s.generate(4)
    s.free()
    return np.stack(out), np.array(toks), gen


@pytest.mark.parametrize("cfg,n,steps", [(clibs.C1, 12, 24), (MIX, 40, 16), (C3H, 24, 8)],
                         ids=["c1-q80", "q4km-mix-hd128", "c3-heads"])
def test_decode_launch_equals_per_launch_step(hip_ctx, monkeypatch, cfg, n, steps):
    prompt = clibs.ids(9, "dec.prompt", n, cfg["vocab"])
    m = hip_ctx.synth(**cfg)
    monkeypatch.setenv("ORNITH_HIP_DECODE", "0")
    ref, rt, rg = run(m, prompt, steps)
    monkeypatch.setenv("ORNITH_HIP_DECODE", "1")
    got, gt, gg = run(m, prompt, steps, fused=True)
    m.free()
    bad = [i for i in range(len(ref)) if not np.array_equal(got[i].view(np.uint32), ref[i].view(np.uint32))]
    assert not bad, f"steps with differing logits: {bad[:8]}"
    assert np.array_equal(gt, rt) and np.array_equal(gg, rg)


def test_decode_launch_c1_golden_tokens(hip_ctx, tmp_path, monkeypatch):
    """64 greedy tokens after C1's 32-token prompt (serial prompt mode), as the
    reference build's golden fixture"""
    monkeypatch.setenv("ORNITH_HIP_DECODE", "1")
    path = tmp_path / "c1.gguf"
    clibs.write_c1_gguf(path)
    m = hip_ctx.load(str(path))
    s = m.session(128)
    s.eval(GOLD["prompt"].astype(np.int32))
    toks = s.generate(64)
    s.free()
    m.free()
    assert np.array_equal(toks, GOLD["serial_tokens"])


@pytest.mark.parametrize("form", ["1", "0"], ids=["flash-mfma", "flash-valu"])
def test_decode_launch_flash_contexts(hip_ctx, monkeypatch, form):
    """attention past the exact walk from the first position (flash chunks and
    their merge as operations of the launch)"""
    monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", "0")
    monkeypatch.setenv("ORNITH_HIP_FLASH_MFMA", form)
    prompt = clibs.ids(10, "dec.flash", 300, C3H["vocab"])
    m = hip_ctx.synth(**C3H)
    monkeypatch.setenv("ORNITH_HIP_DECODE", "0")
    ref, rt, _ = run(m, prompt, 6)
    monkeypatch.setenv("ORNITH_HIP_DECODE", "1")
    got, gt, _ = run(m, prompt, 6, fused=True)
    m.free()
    for i in range(len(ref)):
        assert np.array_equal(got[i].view(np.uint32), ref[i].view(np.uint32)), i
    assert np.array_equal(gt, rt)
