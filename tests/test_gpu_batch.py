"""GPU: decode of several sessions at once (ornith_hip_batch_step) against
each session's own token step (ornith_hip_session_step = rforward_token) and
against the oracle's token step of each session (orc_session_step,
reference src/ornith_rforward.c:686-706) on the GGUF the device model writes.

Bar: every session's logits after every batch step bit-identical to the same
session stepped alone, and the greedy tokens identical, on C1 (Q8_0) and on
Q4_K/Q6_K MoE and dense models; sessions at different positions, on the exact
and flash attention paths; a session that joins or leaves between steps.
Against the oracle: bit-identical logits on the exact walk; on the flash path
(which re-associates the attention sums) within 1e-2 relative L2, with the
same greedy token wherever the oracle's best two logits are further apart
than 1e-2 of the best one's magnitude."""
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
DENSE = dict(MIX, ne=0, top_k=0, moe_inter=0, shared_inter=1024, seed=7)
CFGS = {"c1": clibs.C1, "moe": MIX, "dense": DENSE}


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def prompts(vocab, n, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, 3 + 7 * b).astype(np.int32) for b in range(n)]


@pytest.mark.parametrize("cfg", ["c1", "moe", "dense"])
@pytest.mark.parametrize("n", [1, 3, 8])
@pytest.mark.parametrize("exact_max", [None, 0], ids=["exact", "flash"])
@pytest.mark.parametrize("fused", ["1", "0"], ids=["slotted-launches", "batched-kernels"])
def test_batch_step_equals_single_steps(hip_ctx, orc, tmp_path, monkeypatch, cfg, n, exact_max, fused):
    """Both batch plans: the token step's fused launches with one slot per
    session, and the column-streaming batched kernels."""
    if exact_max is not None:
        pytest.skip("batch steps past the exact attention walk are switched off: one of them (batched kernels, "
                    "flash path, 3 sessions, MoE model) faulted the GPU, as two batch runs on the flash path did "
                    "before; cause not found")
    monkeypatch.setenv("ORNITH_HIP_BATCH_FUSED", fused)
    m = hip_ctx.synth(**CFGS[cfg])
    V = m.arch["vocab"]
    ps = prompts(V, n, 11)
    single = [m.session(128) for _ in range(n)]
    batch = [m.session(128) for _ in range(n)]
    for b in range(n):
        single[b].eval(ps[b])
        batch[b].eval(ps[b])
    toks = np.array([int(np.argmax(s.logits())) for s in single], np.int32)
    fed, hist = [], []
    for step in range(6):
        nxt = m.batch_step(batch, toks)
        want = []
        for b in range(n):
            single[b].step(int(toks[b]))
            lg = single[b].logits()
            got = batch[b].logits()
            assert np.array_equal(u32(got), u32(lg)), (cfg, n, step, b)
            want.append(int(np.argmax(lg)))
            assert batch[b].pos == single[b].pos
        assert np.array_equal(nxt, np.array(want, np.int32)), (nxt, want)
        fed.append(toks.copy())
        hist.append([batch[b].logits().copy() for b in range(n)])
        toks = nxt
    for s in single + batch:
        s.free()
    path = os.path.join(str(tmp_path), f"batch_{cfg}.gguf")
    clibs.write_model_gguf(m, CFGS[cfg], path)
    m.free()
    oracle_replay(orc, path, ps, fed, hist, exact=exact_max is None, tag=f"{cfg} n={n} fused={fused}")


def oracle_replay(orc, path, ps, fed, hist, exact, tag):
    """each session's prompt and tokens through the oracle's token step, its
    logits against the batch's after every step"""
    om = C.c_void_p()
    assert orc.orc_model_load(path.encode(), C.byref(om)) == 0
    orc.orc_model_set_threads(om, 8)
    V = orc.orc_model_arch(om).contents.vocab
    worst = 0.0
    serial = 1 if os.environ.get("ORNITH_PREFILL_SERIAL") == "1" else 0     # the engine's prompt mode
    for b, p in enumerate(ps):
        o = orc.orc_session_new(om, 128, 1)
        assert orc.orc_session_eval(o, i32p(p), p.size, serial) == 0
        for step, toks in enumerate(fed):
            assert orc.orc_session_step(o, int(toks[b])) == 0
            ref = np.ctypeslib.as_array(orc.orc_session_logits(o), (V,)).copy()
            got = hist[step][b]
            if exact:
                assert np.array_equal(u32(got), u32(ref)), ("oracle", tag, step, b)
                continue
            r = float(np.linalg.norm(got.astype(np.float64) - ref) / np.linalg.norm(ref.astype(np.float64)))
            worst = max(worst, r)
            assert r <= 1e-2, ("oracle", tag, step, b, r)
            if int(np.argmax(got)) != int(np.argmax(ref)):
                top2 = np.sort(ref)[-2:]
                assert top2[1] - top2[0] <= 1e-2 * abs(top2[1]), ("oracle", tag, step, b, top2)
        orc.orc_session_free(o)
    orc.orc_model_free(om)
    if not exact:
        print(f"[{tag}] flash path against the oracle: worst logits rel L2 {worst:.3e}")


def test_batch_membership_changes(hip_ctx):
    """Sessions join and leave the batch between steps; a session stepped in a
    batch continues with its own token step and generate."""
    m = hip_ctx.synth(**MIX)
    V = m.arch["vocab"]
    ps = prompts(V, 4, 12)
    a = [m.session(96) for _ in range(4)]
    r = [m.session(96) for _ in range(4)]
    for b in range(4):
        a[b].eval(ps[b])
        r[b].eval(ps[b])
    groups = [[0, 1, 2, 3], [1, 3], [2, 0, 3], [3]]
    for g in groups:
        toks = np.array([int(np.argmax(r[b].logits())) for b in g], np.int32)
        m.batch_step([a[b] for b in g], toks)
        for b, t in zip(g, toks):
            r[b].step(int(t))
            assert np.array_equal(u32(a[b].logits()), u32(r[b].logits())), (g, b)
    for b in range(4):
        assert np.array_equal(a[b].generate(5), r[b].generate(5))
    with pytest.raises(Exception):
        m.batch_step([a[0], a[0]], np.array([1, 2], np.int32))
    # sessions of different KV capacities are refused before any launch
    c = m.session(160)
    c.eval(ps[0])
    import ornithology_amd as oa
    with pytest.raises(oa.HipError):
        m.batch_step([a[0], c], np.array([1, 2], np.int32))
    assert c.pos == ps[0].size
    c.free()
    for s in a + r:
        s.free()
    m.free()
