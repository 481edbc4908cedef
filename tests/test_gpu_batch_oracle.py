"""GPU: decode of several sessions at once (ornith_hip_batch_step) against the
oracle's token step of each session (orc_session_step = rforward_token,
reference src/ornith_rforward.c:686-706), on the GGUF the device model writes.

Four sessions of different capacities and contexts step together, so the
attention grid and LDS taken as the maximum over the sessions cover sessions
that need fewer blocks:
* three inside the exact attention walk (5, 40 and 300 prompt tokens):
  logits bit-identical to the oracle after every step, same greedy tokens;
* one past it (a 4100-token prompt, capacity 4160: the prompt rows past 1024
  on the matrix-core prompt attention, the steps on the flash decode with
  128 blocks per KV head, as the bench's 4096 context has): teacher-forced on
  the batch's tokens, logits within 1e-2 relative L2 of the oracle (values
  printed), and the same greedy token wherever the oracle's best two logits
  are further apart than 1e-2 of the best one's magnitude.
Both batch plans: the slotted fused launches and the column-streaming batched
kernels. That mix of capacities and paths is refused by the engine (see the
skip reason); the runnable form below keeps one capacity and the exact walk:
three sessions of capacity 330 at 5, 40 and 300 prompt tokens step together,
their logits bit-identical to the oracle's after every step."""
import ctypes as C
import os

import numpy as np
import pytest

import clibs
from clibs import i32p

pytestmark = [pytest.mark.gpu,
              pytest.mark.skip(reason="batch decode is switched off: a batch run faulted the GPU for the fourth time (slotted launches, C1, "
                 "three sessions of capacity 330 inside the exact walk, a case that had passed before); cause not "
                 "found; the engine refuses ornith_hip_batch_step")]

MIX = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=512, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, seed=5)
CFGS = {"c1": clibs.C1, "moe": MIX}
PROMPTS = [5, 40, 300, 4100]
CAPS = [16, 64, 330, 4160]
EXACT = 3                     # sessions [0, EXACT) stay inside the exact walk
STEPS = 6
THREADS = min(os.cpu_count() or 8, 16)


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg", ["c1", "moe"])
@pytest.mark.parametrize("fused", ["1", "0"], ids=["slotted-launches", "batched-kernels"])
@pytest.mark.skip(reason="faulted the GPU on its first run (MoE model, four sessions of capacities 16..4160, "
                         "contexts inside and past the exact walk); cause not found; the engine now refuses "
                         "batches that mix KV capacities or attention paths")
def test_batch_step_matches_oracle_per_session(hip_ctx, orc, tmp_path, monkeypatch, cfg, fused):
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")
    monkeypatch.setenv("ORNITH_HIP_BATCH_FUSED", fused)
    c = CFGS[cfg]
    m = hip_ctx.synth(**c)
    V = m.arch["vocab"]
    prompts = [clibs.ids(40 + b, "batch.oracle", PROMPTS[b], V) for b in range(len(PROMPTS))]
    path = os.path.join(str(tmp_path), f"batch_{cfg}.gguf")
    clibs.write_model_gguf(m, c, path)
    om = C.c_void_p()
    assert orc.orc_model_load(path.encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, THREADS)
    sess, osess = [], []
    for b, p in enumerate(prompts):
        s = m.session(CAPS[b])
        s.eval(p)
        sess.append(s)
        o = orc.orc_session_new(om, CAPS[b], 1)
        assert orc.orc_session_eval(o, i32p(p), p.size, 0) == 0
        osess.append(o)

    def oracle_logits(b):
        return np.ctypeslib.as_array(orc.orc_session_logits(osess[b]), (V,)).copy()

    worst = 0.0
    for b in range(len(sess)):
        got, ref = sess[b].logits(), oracle_logits(b)
        if b < EXACT:
            assert np.array_equal(u32(got), u32(ref)), ("prompt", b)
        else:
            r = rel_l2(got, ref)
            worst = max(worst, r)
            print(f"[{cfg} fused={fused}] session {b} prompt logits rel L2 {r:.3e}")
    toks = np.array([int(np.argmax(s.logits())) for s in sess], np.int32)
    flips = 0
    for step in range(STEPS):
        nxt = m.batch_step(sess, toks)
        for b in range(len(sess)):
            assert orc.orc_session_step(osess[b], int(toks[b])) == 0
            got, ref = sess[b].logits(), oracle_logits(b)
            assert sess[b].pos == PROMPTS[b] + step + 1
            assert int(nxt[b]) == int(np.argmax(got))
            if b < EXACT:
                assert np.array_equal(u32(got), u32(ref)), (step, b)
                continue
            r = rel_l2(got, ref)
            worst = max(worst, r)
            print(f"[{cfg} fused={fused}] session {b} step {step}: logits rel L2 {r:.3e}")
            top2 = np.sort(ref)[-2:]
            if int(np.argmax(got)) != int(np.argmax(ref)):
                flips += 1
                assert top2[1] - top2[0] <= 1e-2 * abs(top2[1]), (step, b, top2)
        toks = nxt
    assert worst <= 1e-2
    print(f"[{cfg} fused={fused}] worst rel L2 past the exact walk {worst:.3e}; near-tie argmax flips {flips}")
    for s in sess:
        s.free()
    for o in osess:
        orc.orc_session_free(o)
    orc.orc_model_free(om)
    m.free()


@pytest.mark.timeout(300)
@pytest.mark.parametrize("cfg", ["c1", "moe"])
@pytest.mark.parametrize("fused", ["1", "0"], ids=["slotted-launches", "batched-kernels"])
def test_batch_step_exact_walk_contexts_match_oracle(hip_ctx, orc, tmp_path, monkeypatch, cfg, fused):
    """Sessions of one capacity at different contexts inside the exact walk:
    the batch's attention grid and LDS (the maximum over the sessions) cover
    sessions that need fewer positions; every logit bit-identical to the
    oracle's token step of the same session, every greedy token the same."""
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")
    monkeypatch.setenv("ORNITH_HIP_BATCH_FUSED", fused)
    c = CFGS[cfg]
    cap, lens = 330, PROMPTS[:EXACT]
    m = hip_ctx.synth(**c)
    V = m.arch["vocab"]
    prompts = [clibs.ids(40 + b, "batch.oracle", lens[b], V) for b in range(len(lens))]
    path = os.path.join(str(tmp_path), f"batch_exact_{cfg}.gguf")
    clibs.write_model_gguf(m, c, path)
    om = C.c_void_p()
    assert orc.orc_model_load(path.encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, THREADS)
    sess, osess = [], []
    for p in prompts:
        s = m.session(cap)
        s.eval(p)
        sess.append(s)
        o = orc.orc_session_new(om, cap, 1)
        assert orc.orc_session_eval(o, i32p(p), p.size, 0) == 0
        osess.append(o)

    def oracle_logits(b):
        return np.ctypeslib.as_array(orc.orc_session_logits(osess[b]), (V,)).copy()

    for b in range(len(sess)):
        assert np.array_equal(u32(sess[b].logits()), u32(oracle_logits(b))), ("prompt", b)
    toks = np.array([int(np.argmax(s.logits())) for s in sess], np.int32)
    for step in range(STEPS):
        nxt = m.batch_step(sess, toks)
        for b in range(len(sess)):
            assert orc.orc_session_step(osess[b], int(toks[b])) == 0
            got, ref = sess[b].logits(), oracle_logits(b)
            assert sess[b].pos == lens[b] + step + 1
            assert np.array_equal(u32(got), u32(ref)), (cfg, fused, step, b)
            assert int(nxt[b]) == int(np.argmax(ref))
        toks = nxt
    for s in sess:
        s.free()
    for o in osess:
        orc.orc_session_free(o)
    orc.orc_model_free(om)
    m.free()
