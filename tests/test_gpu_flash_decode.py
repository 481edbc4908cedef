"""GPU: decode attention past the exact walk on the matrix cores (flash chunks
with every query head of a KV head per block, fp16 operands split into high
and low parts, fp32 softmax). It re-associates the reference's softmax and V
sums, so the bar is the tolerance of north_star: final logits within 1e-2
relative L2 of the reference order (the oracle, src/ornith_attn.c:87-149) and
the same greedy token. The VALU flash chunks (ORNITH_HIP_FLASH_MFMA=0) meet the
same bar, and the two forms agree with each other far more closely."""
import ctypes as C

import numpy as np
import pytest

import clibs
from clibs import i32p

pytestmark = pytest.mark.gpu

Q4 = dict(t_default=clibs.Q4_K, t_attn_v=clibs.Q4_K, t_ffn_down=clibs.Q4_K, t_output=clibs.Q4_K,
          t_embd=clibs.Q4_K)
# C3's attention geometry (16 q / 2 kv heads, head_dim 256) and C4's (32 / 2)
C3H = dict(clibs.C1, hidden=1024, n_layers=4, full_interval=4, vocab=512, nh=16, nkv=2, hd=256, nk=16, nv=32,
           dhead=128, ne=8, top_k=2, moe_inter=512, shared_inter=512, seed=13, **Q4)
C4H = dict(C3H, nh=32, nv=64, seed=14)
MIXH = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
            ne=8, top_k=2, moe_inter=512, shared_inter=512, seed=5, **Q4)


@pytest.mark.parametrize("cfg,n", [(clibs.C1, 4200), (C3H, 700), (C4H, 300), (MIXH, 500)],
                         ids=["c1-hd64-two-tiles-per-block", "c3-heads", "c4-heads", "hd128-g4"])
def test_flash_decode_within_tolerance(hip_ctx, orc, tmp_path, monkeypatch, cfg, n):
    path = tmp_path / "m.gguf"
    clibs.write_c1_gguf(path, cfg)
    om = C.c_void_p()
    assert orc.orc_model_load(str(path).encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    os_ = orc.orc_session_new(om, n + 8, 1)
    p = np.random.default_rng(21).integers(0, cfg["vocab"], n).astype(np.int32)
    # serial mode: the token recurrence, as the engine's token path below
    assert orc.orc_session_eval(os_, i32p(p), n, 1) == 0
    want = np.ctypeslib.as_array(orc.orc_session_logits(os_), (cfg["vocab"],)).copy()
    orc.orc_session_free(os_)
    orc.orc_model_free(om)

    # every prompt token through the decode step, attention split from the
    # first position on
    monkeypatch.setenv("ORNITH_HIP_PREFILL", "0")
    monkeypatch.setenv("ORNITH_HIP_EXACT_ATTN_MAX", "0")
    m = hip_ctx.synth(**cfg)
    got = {}
    for form in ("1", "0"):
        monkeypatch.setenv("ORNITH_HIP_FLASH_MFMA", form)
        s = m.session(n + 8)
        s.eval(p)
        lg = s.logits().copy()
        s.free()
        rel = float(np.linalg.norm(lg - want) / np.linalg.norm(want))
        print(f"n={n} flash_mfma={form}: rel L2 {rel:.3e} vs reference order")
        assert np.isfinite(lg).all() and rel < 1e-2, (form, rel)
        assert int(np.argmax(lg)) == int(np.argmax(want)), form
        got[form] = lg
    d = float(np.linalg.norm(got["1"] - got["0"]) / np.linalg.norm(got["0"]))
    print(f"matrix-core vs VALU flash: rel L2 {d:.3e}")
    assert d < 1e-5
    m.free()
