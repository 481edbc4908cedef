"""GPU: on-device random-init synthesis equals the oracle generator's GGUF
byte for byte (value streams and the Q8_0 / Q4_K / Q6_K encoders), and the
synthesised C1 model decodes the same greedy tokens as the reference."""
import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")

MIX = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=256, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, seed=3)
DENSE = dict(MIX, ne=0, top_k=0, moe_inter=0, shared_inter=1024, seed=7)
# C4's type mix at a small shape: IQ2_XXS routed experts, Q4_K / Q6_K elsewhere
IQX = dict(clibs.C1, hidden=256, n_layers=2, full_interval=2, vocab=512, nh=2, nkv=1, hd=128, nk=1, nv=2,
           dhead=128, ne=2, top_k=1, moe_inter=256, shared_inter=256, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, t_exps=clibs.IQ2_XXS, seed=9)

# C4's head geometry at a small hidden size: 64 value heads of 128 (the gated
# norm prologue of ssm_out over 8192 inputs), 32 query heads of 256
# (attn_output over 8192 inputs), 12288 conv channels, IQ2_XXS experts over
# several super-blocks per row
C4X = dict(clibs.C1, hidden=1024, n_layers=4, full_interval=4, vocab=512, nh=32, nkv=2, hd=256, nk=16, nv=64,
           dhead=128, ne=4, top_k=2, moe_inter=512, shared_inter=512, t_default=clibs.Q4_K, t_attn_v=clibs.Q4_K,
           t_ffn_down=clibs.Q4_K, t_output=clibs.Q4_K, t_embd=clibs.Q4_K, t_exps=clibs.IQ2_XXS, seed=11)


@pytest.mark.parametrize("cfg", [clibs.C1, MIX, DENSE, IQX], ids=["C1-Q8_0", "Q4_K_M-mix", "dense", "IQ2_XXS-experts"])
def test_synth_equals_generator_bytes(hip_ctx, tmp_path, cfg):
    p = tmp_path / "gen.gguf"
    clibs.write_c1_gguf(p, cfg)
    ref = clibs.gguf_tensors(p)
    m = hip_ctx.synth(**cfg)
    assert m.nbytes == sum(v[2].nbytes for v in ref.values())
    for name, (t, dims, raw) in ref.items():
        info = m.tensor_info(name)
        assert info is not None and info["type"] == t, name
        got = m.tensor(name).download(info["nbytes"])
        assert np.array_equal(got, raw), name
    m.free()


def test_synth_c1_greedy_matches_reference(hip_ctx):
    m = hip_ctx.synth(**clibs.C1)
    s = m.session(104)
    s.eval(GOLD["prompt"])
    assert np.array_equal(s.logits().view(np.uint32), GOLD["serial_prompt_logits"].view(np.uint32))
    assert np.array_equal(s.generate(64), GOLD["serial_tokens"])
    s.free()
    m.free()


def test_profile_step_reports_every_launch(hip_ctx):
    m = hip_ctx.synth(**clibs.C1)
    s = m.session(16)
    s.eval(GOLD["prompt"][:4])
    rec = s.profile_step()
    kinds = [k for k, _, _ in rec]
    # per layer: input projections, output projection, router (+ routing),
    # experts gate/up, fused down + combine; then lm_head
    assert sum(k.startswith("matvec") for k in kinds) == 4 * 4 + 1 and kinds.count("moe_down") == 4
    assert kinds.count("delta_step") == 3 and kinds.count("argmax") == 1
    assert "rmsnorm_q8k" not in kinds and "moe_route" not in kinds and "moe_combine" not in kinds
    assert all(ms > 0 for _, _, ms in rec) and s.pos == 5
    s.free()
    m.free()


@pytest.mark.parametrize("cfg", [IQX, C4X], ids=["IQ2_XXS-experts", "C4-heads"])
def test_iq2xxs_experts_decode_matches_oracle(hip_ctx, orc, tmp_path, cfg):
    """C4's path at a small shape: the IQ2_XXS routed experts through the
    reference's f32 fallback (dequantised row . f32 activation,
    src/ornith_rforward.c:119-133): prompt logits and 6 greedy steps
    bit-identical to the oracle. The device synthesis (byte-identical to the
    generator, test_synth_equals_generator_bytes) is written out for the
    oracle, which would take minutes to encode the IQ2_XXS experts itself."""
    import ctypes as C
    from clibs import i32p
    p = tmp_path / "iqx.gguf"
    m = hip_ctx.synth(**cfg)
    clibs.write_model_gguf(m, cfg, p)
    om = C.c_void_p()
    assert orc.orc_model_load(str(p).encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    os_ = orc.orc_session_new(om, 40, 1)
    prompt = np.random.default_rng(2).integers(0, cfg["vocab"], 12).astype(np.int32)
    assert orc.orc_session_eval(os_, i32p(prompt), 12, 1) == 0
    s = m.session(40)
    s.eval(prompt)
    V = cfg["vocab"]
    for k in range(7):
        want = np.ctypeslib.as_array(orc.orc_session_logits(os_), (V,)).copy()
        assert np.array_equal(s.logits().view(np.uint32), want.view(np.uint32)), k
        tok = int(np.argmax(want))
        assert orc.orc_session_step(os_, tok) == 0
        s.step(tok)
    s.free()
    m.free()
    orc.orc_session_free(os_)
    orc.orc_model_free(om)
