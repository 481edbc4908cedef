"""CPU: the oracle forward, sessions and GGUF handling on the C1 config.

The C1 GGUF written by the oracle's generator must be byte-identical to the
one tests/golden/make_golden.py wrote with the reference's own encoder and
writer (sha256 in c1.npz), and the oracle's prompt logits, per-step logits and
64 greedy tokens must equal the reference's bit for bit, for the default
chunked prefill and for ORNITH_PREFILL_SERIAL=1.
"""
import ctypes as C
import hashlib
import struct

import numpy as np
import pytest

import clibs
from clibs import f32p, i32p

GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")


@pytest.fixture(scope="module")
def c1_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("c1") / "c1.gguf"
    clibs.write_c1_gguf(p)
    return p


def test_c1_gguf_matches_reference_writer(c1_path):
    h = hashlib.sha256(c1_path.read_bytes()).hexdigest()
    assert h == str(GOLD["gguf_sha256"])


def load(orc, path):
    m = C.c_void_p()
    st = orc.orc_model_load(str(path).encode(), C.byref(m))
    return st, m


@pytest.mark.parametrize("mode,serial", [("serial", 1), ("chunked", 0)])
def test_c1_greedy_matches_reference(orc, c1_path, mode, serial):
    st, m = load(orc, c1_path)
    assert st == 0
    orc.orc_model_set_threads(m, 8)
    a = orc.orc_model_arch(m).contents
    assert (a.hidden, a.n_layers, a.vocab, a.nh, a.nkv, a.hd, a.nk, a.nv, a.dk, a.ne, a.top_k) == \
        (512, 4, 4096, 8, 2, 64, 4, 8, 64, 16, 4)
    s = orc.orc_session_new(m, 104, 1)
    prompt = np.ascontiguousarray(GOLD["prompt"])
    assert orc.orc_session_eval(s, i32p(prompt), prompt.size, serial) == 0
    pl = np.ctypeslib.as_array(orc.orc_session_logits(s), (4096,)).copy()
    assert np.array_equal(pl.view(np.uint32), GOLD[f"{mode}_prompt_logits"].view(np.uint32))
    toks = np.zeros(64, np.int32)
    n = C.c_int(0)
    trace = np.zeros((64, 4096), np.float32)
    assert orc.orc_session_generate(s, 64, i32p(toks), C.byref(n), f32p(trace)) == 0
    assert n.value == 64 and np.array_equal(toks, GOLD[f"{mode}_tokens"])
    for i, k in enumerate(GOLD[f"{mode}_trace_steps"]):
        assert np.array_equal(trace[k].view(np.uint32), GOLD[f"{mode}_trace_logits"][i].view(np.uint32)), k
    orc.orc_session_free(s)
    orc.orc_model_free(m)


def test_prefill_equals_decode_within_tolerance(orc, c1_path):
    """Chunked prefill and token steps agree to fp tolerance on one layer's
    delta state for a short prompt (test_forward.c:60-73 pattern)."""
    st, m = load(orc, c1_path)
    orc.orc_model_set_threads(m, 8)
    states = []
    for serial in (0, 1):
        s = orc.orc_session_new(m, 16, 1)
        p = np.ascontiguousarray(GOLD["prompt"][:4])
        orc.orc_session_eval(s, i32p(p), 4, serial)
        states.append(np.ctypeslib.as_array(orc.orc_session_delta(s, 0), (8 * 64 * 64,)).copy())
        orc.orc_session_free(s)
    orc.orc_model_free(m)
    assert np.abs(states[0] - states[1]).max() < 1e-4


def test_capacity_and_loader_errors(orc, c1_path, tmp_path):
    st, m = load(orc, c1_path)
    s = orc.orc_session_new(m, 4, 1)
    p = np.ascontiguousarray(GOLD["prompt"][:8])
    assert orc.orc_session_eval(s, i32p(p), 8, 1) == 3          # capacity -> UNSUPPORTED
    assert b"capacity" in orc.orc_last_error()
    orc.orc_session_free(s)
    orc.orc_model_free(m)
    assert load(orc, tmp_path / "missing.gguf")[0] == 1          # IO
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + bytes(32))
    assert load(orc, bad)[0] == 2                                 # FORMAT (magic)
    raw = c1_path.read_bytes()
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(raw[: len(raw) // 2])
    assert load(orc, trunc)[0] == 2                               # data past EOF


def test_generator_deterministic_streams(orc):
    a = clibs.gauss(0, "x", 1000, 0.02)
    b = clibs.gauss(0, "x", 1000, 0.02)
    c = clibs.gauss(1, "x", 1000, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    g = clibs.gauss(7, "moments", 200000, 1.0).astype(np.float64)
    assert abs(g.mean()) < 0.01 and abs(g.std() - 1) < 0.01 and np.abs(g).max() <= 6.0
    # counter-based: element i does not depend on where the fill started
    L = clibs.oracle()
    part = np.zeros(10, np.float32)
    L.orc_fill_gauss(L.orc_stream_key(0, b"x"), 0.02, f32p(part), 10, 500)
    assert np.array_equal(part, a[500:510])


def test_session_adopt_continues_bit_identically(orc, c1_path):
    """orc_session_adopt (a test aid: a state copied in through the state
    accessors, then declared at its position with its last logits) pinned
    against the session it was copied from: after a 40-token chunked prompt,
    the copy and the original give bit-identical logits over 12 greedy
    steps. A copy missing one layer's state, or declared one position off,
    parts from the original at once (checked below), so the aid cannot hide a
    dropped layer or an off-by-one position."""
    st, m = load(orc, c1_path)
    assert st == 0
    orc.orc_model_set_threads(m, 8)
    arch = clibs.orc_arch_dict(orc, m)
    V = arch["vocab"]
    prompt = clibs.ids(9, "adopt", 40, V)
    a = orc.orc_session_new(m, 64, 1)
    assert orc.orc_session_eval(a, i32p(prompt), prompt.size, 0) == 0
    nv, dv, dk = arch["nv"], arch["dv"], arch["dk"]
    cc = 2 * arch["nk"] * dk + nv * dv
    K = arch["conv_k"]

    def delta_of(l):
        return np.ctypeslib.as_array(orc.orc_session_delta(a, l), (nv * dv * dk,)).copy()

    def conv_of(l):
        return np.ctypeslib.as_array(orc.orc_session_conv(a, l), ((K - 1) * cc,)).copy()

    def kv_of(l):
        kv = orc.orc_session_kv(a, l).contents
        n = kv.len * kv.n_kv_heads
        return (np.ctypeslib.as_array(kv.Kq, (n * kv.head_dim,)).copy(), np.ctypeslib.as_array(kv.Ks, (n,)).copy(),
                np.ctypeslib.as_array(kv.Vq, (n * kv.head_dim,)).copy(), np.ctypeslib.as_array(kv.Vs, (n,)).copy())

    def logits(s):
        return np.ctypeslib.as_array(orc.orc_session_logits(s), (V,)).copy()

    def copy(skip_layer=None, pos=40):
        b = orc.orc_session_new(m, 64, 1)
        zero = lambda l, f, n: np.zeros(n, np.float32) if l == skip_layer else f(l)
        clibs.adopt_state(orc, b, arch, pos, logits(a),
                          lambda l: zero(l, delta_of, nv * dv * dk), lambda l: zero(l, conv_of, (K - 1) * cc), kv_of)
        return b

    b = copy()
    assert orc.orc_session_pos(b) == 40
    bad_layer, bad_pos = copy(skip_layer=0), copy(pos=39)
    tok = int(np.argmax(logits(a)))
    for step in range(12):
        for s in (a, b, bad_layer, bad_pos):
            assert orc.orc_session_step(s, tok) == 0
        ref = logits(a)
        assert np.array_equal(logits(b).view(np.uint32), ref.view(np.uint32)), step
        if step == 0:
            assert not np.array_equal(logits(bad_layer), ref)
            assert not np.array_equal(logits(bad_pos), ref)
        tok = int(np.argmax(ref))
    for s in (a, b, bad_layer, bad_pos):
        orc.orc_session_free(s)
    orc.orc_model_free(m)
