"""GPU: the persistent step kernel (ORNITH_HIP_STEP=1: one cooperative launch
per decode step, its operations as phases between grid barriers) against the
reference and against the launch-per-operation path.

Bar: bit-exact prompt logits and 64 greedy tokens on C1 against the
reference's golden fixture; bit-identical logits, tokens and session state
between the two execution paths on a Q4_K/Q6_K MoE mix (routing, paired
gate/up, fused down), on the flash-attention path and past a second eval (the
barrier counters carry over between launches)."""
import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")

MIX = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=512, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, seed=5)


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run(m, prompt, n_gen, cap, step, monkeypatch, exact_max=None):
    monkeypatch.setenv("ORNITH_HIP_STEP", "1" if step else "0")
    if exact_max is not None:
        monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", str(exact_max))
    s = m.session(cap)
    s.eval(prompt)
    first = s.logits().copy()
    toks = s.generate(n_gen)
    last = s.logits().copy()
    return s, first, toks, last


def test_step_c1_matches_reference(hip_ctx, monkeypatch):
    m = hip_ctx.synth(**clibs.C1)
    s, first, toks, _ = run(m, GOLD["prompt"], 64, 104, True, monkeypatch)
    assert np.array_equal(u32(first), u32(GOLD["serial_prompt_logits"]))
    assert np.array_equal(toks, GOLD["serial_tokens"])
    s.free()
    m.free()


@pytest.mark.parametrize("exact_max", [None, 0], ids=["exact", "flash"])
def test_step_equals_launch_path_on_moe_mix(hip_ctx, monkeypatch, exact_max):
    m = hip_ctx.synth(**MIX)
    a = m.arch
    prompt = np.random.default_rng(1).integers(0, a["vocab"], 24).astype(np.int32)
    sg, fg, tg, lg = run(m, prompt, 40, 96, False, monkeypatch, exact_max)
    ss, fs, ts, ls = run(m, prompt, 40, 96, True, monkeypatch, exact_max)
    assert np.array_equal(u32(fg), u32(fs))
    assert np.array_equal(tg, ts)
    assert np.array_equal(u32(lg), u32(ls))
    # session state after 64 positions
    for l in range(a["n_layers"]):
        if (l + 1) % a["full_interval"]:
            assert np.array_equal(u32(sg.delta_state(l)), u32(ss.delta_state(l))), l
    # a second eval on the same sessions: the step kernel's barrier counters
    # and epochs carry over between launches
    more = np.random.default_rng(2).integers(0, a["vocab"], 5).astype(np.int32)
    sg.eval(more)
    ss.eval(more)
    assert np.array_equal(u32(sg.logits()), u32(ss.logits()))
    sg.free()
    ss.free()
    m.free()


def test_step_phase_profile(hip_ctx, monkeypatch):
    monkeypatch.setenv("ORNITH_HIP_STEP", "1")
    m = hip_ctx.synth(**MIX)
    s = m.session(32)
    s.eval(np.arange(8, dtype=np.int32))
    ph = s.profile_phases()
    kinds = [k for k, _, _ in ph]
    assert kinds[0] == "embed" and kinds.count("moe_down") == m.arch["n_layers"]
    assert all(us > 0 for _, _, us in ph) and s.pos == 8
    us, by, n = s.time_kind("step_body", 3)
    assert us > 0 and by > 0 and n == 1
    s.free()
    m.free()
