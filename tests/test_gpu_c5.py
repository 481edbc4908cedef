"""GPU: C5 at its own size (the C3 weights, 32768-token prompts), checked by
properties that a long context fixes without an oracle run (the oracle's
prefill of 32768 tokens on this model takes hours on the host):

* chunk size: the prompt through 2048-token chunks against 1024-token chunks
  (ORNITH_HIP_PREFILL_CHUNK). The delta-net scan's 32-token chunks and the
  matrix-core attention's 32-row query blocks fall on the same positions
  either way, and every projection is per token. Bar: final prompt logits
  within 1e-2 relative L2 (printed) and the same next token, then 8 greedy
  steps with identical tokens.
* batch 8 at 32K: eight sessions with their own 32768-token prompts stepped
  together by the batch step (rforward_token per session, reference
  src/ornith_rforward.c:686-706) against each session stepped alone: logits
  bit-identical after every one of 4 steps, identical greedy tokens.
"""
import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu

C3 = dict(hidden=2048, n_layers=40, vocab=248320, full_interval=4, nh=16, nkv=2, hd=256,
          nk=16, nv=32, dhead=128, conv_k=4, ne=256, top_k=8, moe_inter=512, shared_inter=512,
          t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K, t_ffn_down=clibs.Q6_K, t_output=clibs.Q4_K,
          t_embd=clibs.Q4_K, seed=0, sigma=0.02)
T = 32768


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


@pytest.fixture(scope="module")
def c3(hip_ctx):
    m = hip_ctx.synth(**C3)
    yield m
    m.free()


@pytest.mark.timeout(600)
def test_c5_prefill_chunk_2048_against_1024(c3, monkeypatch):
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")          # the reference's default prompt mode
    prompt = np.random.default_rng(0).integers(0, C3["vocab"], T, dtype=np.int64).astype(np.int32)
    out = {}
    for chunk in (2048, 1024):
        monkeypatch.setenv("ORNITH_HIP_PREFILL_CHUNK", str(chunk))
        s = c3.session(T + 16)
        s.eval(prompt)
        lp = s.logits().copy()
        toks = s.generate(8)
        s.free()
        out[chunk] = (lp, toks)
        print(f"[c5] chunk {chunk}: next token {int(np.argmax(lp))}, greedy {toks.tolist()}", flush=True)
    r = rel_l2(out[2048][0], out[1024][0])
    print(f"[c5] prompt logits, chunk 2048 against 1024: rel L2 {r:.3e}")
    assert r <= 1e-2
    assert int(np.argmax(out[2048][0])) == int(np.argmax(out[1024][0]))
    assert np.array_equal(out[2048][1], out[1024][1])


@pytest.mark.timeout(900)
@pytest.mark.skip(reason="batch steps past the exact attention walk are switched off (an unexplained GPU fault "
                         "in batch steps on the flash path); the engine refuses them")
def test_c5_batch8_at_32k_equals_single_sessions(c3, monkeypatch):
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "0")
    n, steps = 8, 4
    rng = np.random.default_rng(1)
    prompts = [rng.integers(0, C3["vocab"], T, dtype=np.int64).astype(np.int32) for _ in range(n)]
    single = [c3.session(T + 16) for _ in range(n)]
    batch = [c3.session(T + 16) for _ in range(n)]
    for b in range(n):
        single[b].eval(prompts[b])
        batch[b].eval(prompts[b])
    print(f"[c5] {2 * n} sessions prefilled with {T} tokens", flush=True)
    toks = np.array([int(np.argmax(s.logits())) for s in single], np.int32)
    for step in range(steps):
        nxt = c3.batch_step(batch, toks)
        for b in range(n):
            single[b].step(int(toks[b]))
            assert np.array_equal(u32(batch[b].logits()), u32(single[b].logits())), (step, b)
        want = np.array([int(np.argmax(s.logits())) for s in single], np.int32)
        assert np.array_equal(nxt, want)
        toks = nxt
    print(f"[c5] batch of {n} at {T} positions: {steps} steps bit-identical to the single sessions")
    for s in single + batch:
        s.free()
