"""GPU: session snapshots (rmodel_session_save / rmodel_session_load,
src/ornith_rforward.c:986-1171) from device state.

Bar: the file written after the C1 prompt and 8 greedy tokens is
byte-identical (SHA-256) to the reference's own snapshot of the same session,
in both prompt modes (golden c1_session.json); a loaded session continues
exactly as the uninterrupted one (logits, greedy tokens, state) on C1 and on
a Q4_K/Q6_K MoE model; the reference's load errors."""
import hashlib
import json

import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")
SNAP = json.loads((clibs.ROOT / "tests" / "golden" / "c1_session.json").read_text())

MIX = dict(clibs.C1, hidden=768, n_layers=4, vocab=1000, nh=4, nkv=1, hd=128, nk=2, nv=4, dhead=128,
           ne=8, top_k=2, moe_inter=512, shared_inter=512, t_default=clibs.Q4_K, t_attn_v=clibs.Q6_K,
           t_ffn_down=clibs.Q6_K, t_output=clibs.Q6_K, t_embd=clibs.Q4_K, seed=5)


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("mode", ["chunked", "serial"])
def test_snapshot_bytes_equal_reference(hip_ctx, tmp_path, monkeypatch, mode):
    monkeypatch.setenv("ORNITH_PREFILL_SERIAL", "1" if mode == "serial" else "0")
    want = SNAP["modes"][mode]
    m = hip_ctx.synth(**clibs.C1)
    s = m.session(104)
    s.eval(GOLD["prompt"])
    toks = s.generate(SNAP["generated"])
    assert toks.tolist() == want["tokens"]
    f = tmp_path / "s.ornsess"
    s.save(f)
    data = f.read_bytes()
    assert len(data) == want["bytes"]
    assert hashlib.sha256(data).hexdigest() == want["sha256"]
    s.free()
    m.free()


@pytest.mark.parametrize("cfg", ["c1", "moe"])
def test_snapshot_round_trip_continues(hip_ctx, tmp_path, cfg):
    m = hip_ctx.synth(**(clibs.C1 if cfg == "c1" else MIX))
    a = m.arch
    rng = np.random.default_rng(8)
    s = m.session(96)
    s.eval(rng.integers(0, a["vocab"], 37).astype(np.int32))
    s.generate(3)
    f = tmp_path / "s.ornsess"
    s.save(f)
    r = m.load_session(f, extra_cap=40)
    assert r.pos == s.pos == 40
    assert np.array_equal(u32(r.logits()), u32(s.logits()))
    for l in range(a["n_layers"]):
        if (l + 1) % a["full_interval"]:
            assert np.array_equal(u32(r.delta_state(l)), u32(s.delta_state(l)))
            assert np.array_equal(u32(r.conv_state(l)), u32(s.conv_state(l)))
        else:
            for x, y in zip(r.kv(l), s.kv(l)):
                assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
    # both continue identically: greedy tokens, then a prompt, then steps
    assert np.array_equal(r.generate(6), s.generate(6))
    more = rng.integers(0, a["vocab"], 9).astype(np.int32)
    r.eval(more)
    s.eval(more)
    assert np.array_equal(u32(r.logits()), u32(s.logits()))
    for t in (5, 17, 3):
        r.step(t)
        s.step(t)
        assert np.array_equal(u32(r.logits()), u32(s.logits()))
    # the reloaded session saves the same file again
    f2 = tmp_path / "s2.ornsess"
    s.save(f)
    r.save(f2)
    assert f.read_bytes() == f2.read_bytes()
    r.free()
    s.free()
    m.free()


def test_snapshot_load_errors(hip_ctx, tmp_path):
    import ornithology_amd as oa
    m = hip_ctx.synth(**clibs.C1)
    s = m.session(40)
    s.eval(GOLD["prompt"][:10])
    f = tmp_path / "s.ornsess"
    s.save(f)
    data = f.read_bytes()
    cases = {"magic": b"X" + data[1:], "version": data[:8] + b"\x02" + data[9:], "truncated": data[:-100]}
    flipped = bytearray(data)
    flipped[-4 * m.arch["vocab"] - 4] ^= 1          # a history token: the prefix hash no longer matches
    cases["hash"] = bytes(flipped)
    for name, blob in cases.items():
        g = tmp_path / f"{name}.ornsess"
        g.write_bytes(blob)
        with pytest.raises(oa.HipError) as e:
            m.load_session(g)
        assert e.value.status == 2, name                 # ORNITH_ERR_FORMAT
    other = hip_ctx.synth(**MIX)
    with pytest.raises(oa.HipError) as e:
        other.load_session(f)
    assert "fingerprint" in str(e.value)
    with pytest.raises(oa.HipError) as e:
        m.load_session(tmp_path / "missing.ornsess")
    assert e.value.status == 1                           # ORNITH_ERR_IO
    other.free()
    s.free()
    m.free()
