"""CPU: the oracle's attention core, router and f32 helpers.

Restates the reference's own tests (tests/test_attn.c, tests/test_moe.c,
tests/test_tensor.c) against the oracle, adds closed-form checks (brute-force
top-k by full sort, naive O(T^2) GQA in float64), and, where oracle/_ref is
built, bit-for-bit equality with the reference's own functions on random
inputs.
"""
import ctypes as C
import math

import numpy as np
import pytest

import clibs
from clibs import OrcKV, f32p, i32p

ref_only = pytest.mark.skipif(not clibs.have_ref(), reason="oracle/_ref not built (reference tree absent)")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rnd(seed, n, lo=-1.0, hi=1.0):
    return clibs.uniform(seed, f"attn{seed}", n, lo, hi)


# ---- gated delta rule (tests/test_attn.c:28-83) --------------------------------
def test_delta_prefill_equals_steps(orc):
    dk, dv, T = 6, 5, 17
    Q, K, V = rnd(1, T * dk), rnd(2, T * dk), rnd(3, T * dv)
    al = clibs.uniform(4, "al", T, 0.85, 0.999)
    be = clibs.uniform(5, "be", T, 0.1, 0.9)
    S = np.zeros(dk * dv, np.float32)
    Od = np.zeros(T * dv, np.float32)
    for t in range(T):
        o = np.zeros(dv, np.float32)
        orc.orc_delta_step(f32p(S), dk, dv, f32p(Q[t * dk:]), f32p(K[t * dk:]), f32p(V[t * dv:]),
                           float(al[t]), float(be[t]), f32p(o))
        Od[t * dv:(t + 1) * dv] = o
    for chunk in (1, 2, 3, 4, 5, 8, 16, T):
        Sp = np.zeros(dk * dv, np.float32)
        Op = np.zeros(T * dv, np.float32)
        orc.orc_delta_prefill(f32p(Sp), dk, dv, f32p(Q), f32p(K), f32p(V), f32p(al), f32p(be), T, chunk, f32p(Op))
        assert np.abs(Op - Od).max() < 2e-4 and np.abs(Sp - S).max() < 2e-4, chunk
    # carried non-zero state across a split
    Sp = np.zeros(dk * dv, np.float32)
    Op = np.zeros(T * dv, np.float32)
    s = 7
    orc.orc_delta_prefill(f32p(Sp), dk, dv, f32p(Q), f32p(K), f32p(V), f32p(al), f32p(be), s, 3, f32p(Op))
    Q2, K2, V2 = [np.ascontiguousarray(a[s * w:]) for a, w in ((Q, dk), (K, dk), (V, dv))]
    O2 = np.zeros((T - s) * dv, np.float32)
    orc.orc_delta_prefill(f32p(Sp), dk, dv, f32p(Q2), f32p(K2), f32p(V2), f32p(np.ascontiguousarray(al[s:])),
                          f32p(np.ascontiguousarray(be[s:])), T - s, 4, f32p(O2))
    Op[s * dv:] = O2
    assert np.abs(Op - Od).max() < 2e-4


def test_delta_step_closed_form(orc):
    # S_t = alpha S (I - beta k k^T) + beta v k^T ; o = S_t q   (src/ornith_attn.h:15-30)
    dk, dv = 8, 6
    S0 = rnd(6, dk * dv).astype(np.float64).reshape(dv, dk)
    q, k, v = rnd(7, dk), rnd(8, dk), rnd(9, dv)
    a, b = 0.9, 0.4
    S = S0.astype(np.float32).ravel().copy()
    o = np.zeros(dv, np.float32)
    orc.orc_delta_step(f32p(S), dk, dv, f32p(q), f32p(k), f32p(v), a, b, f32p(o))
    kd = k.astype(np.float64)
    St = a * S0 @ (np.eye(dk) - b * np.outer(kd, kd)) + b * np.outer(v.astype(np.float64), kd)
    assert np.abs(S.reshape(dv, dk) - St).max() < 1e-5
    assert np.abs(o - St @ q.astype(np.float64)).max() < 1e-5


# ---- GQA (tests/test_attn.c:87-158) ----------------------------------------------
def naive_gqa(Q, K, V, T, nh, nkv, hd):
    Q, K, V = (a.astype(np.float64) for a in (Q, K, V))
    O = np.zeros((T, nh, hd))
    g = nh // nkv
    for i in range(T):
        for h in range(nh):
            kvh = h // g
            s = np.array([Q[i * nh * hd + h * hd:][:hd] @ K[j * nkv * hd + kvh * hd:][:hd] for j in range(i + 1)])
            s = s / math.sqrt(hd)
            p = np.exp(s - s.max()); p /= p.sum()
            O[i, h] = sum(p[j] * V[j * nkv * hd + kvh * hd:][:hd] for j in range(i + 1))
    return O.ravel()


@pytest.mark.parametrize("quant,tol,shape", [(0, 1e-5, (4, 2, 8, 11)), (1, 5e-2, (4, 2, 16, 13))])
def test_gqa_step_vs_naive(orc, quant, tol, shape):
    nh, nkv, hd, T = shape
    Q, K, V = rnd(10, T * nh * hd), rnd(11, T * nkv * hd), rnd(12, T * nkv * hd)
    kv = OrcKV()
    assert orc.orc_kv_init(C.byref(kv), T, nkv, hd, quant) == 0
    O = np.zeros(T * nh * hd, np.float32)
    for t in range(T):
        o = np.zeros(nh * hd, np.float32)
        orc.orc_gqa_step(C.byref(kv), f32p(Q[t * nh * hd:]), f32p(K[t * nkv * hd:]), f32p(V[t * nkv * hd:]),
                         nh, f32p(o), 0.0)
        O[t * nh * hd:(t + 1) * nh * hd] = o
    orc.orc_kv_free(C.byref(kv))
    assert np.abs(O - naive_gqa(Q, K, V, T, nh, nkv, hd)).max() < tol
    if quant:   # Q8 KV is well under half of fp32 per token
        assert 2 * (nkv * hd + nkv * 4) * 2 <= 2 * nkv * hd * 4


def test_gqa_single_position_returns_v(orc):
    nh, nkv, hd = 4, 2, 8
    q, k, v = rnd(13, nh * hd), rnd(14, nkv * hd), rnd(15, nkv * hd)
    kv = OrcKV()
    orc.orc_kv_init(C.byref(kv), 1, nkv, hd, 0)
    o = np.zeros(nh * hd, np.float32)
    orc.orc_gqa_step(C.byref(kv), f32p(q), f32p(k), f32p(v), nh, f32p(o), 0.0)
    orc.orc_kv_free(C.byref(kv))
    assert np.abs(o[:hd] - v[:hd]).max() < 1e-5


def test_kv_quant_vec(orc):
    x = rnd(16, 64)
    q = np.zeros(64, np.int8)
    s = orc.orc_kv_quant_vec(f32p(x), 64, C.c_void_p(q.ctypes.data))
    amax = np.float32(np.abs(x).max())
    assert s == np.float32(amax / np.float32(127))
    inv = np.float32(np.float32(127) / amax)
    assert np.array_equal(q, np.clip(np.rint(x * inv), -127, 127).astype(np.int8))
    z = np.zeros(64, np.float32)
    assert orc.orc_kv_quant_vec(f32p(z), 64, C.c_void_p(q.ctypes.data)) == 0.0 and not q.any()


# ---- conv (tests/test_attn.c:162-192) ----------------------------------------------
def test_conv_step_causal(orc):
    K, Cc, T = 4, 3, 9
    X, w, b = rnd(17, T * Cc), rnd(18, Cc * K), rnd(19, Cc, -0.2, 0.2)
    buf = np.zeros((K - 1) * Cc, np.float32)
    O = np.zeros(T * Cc, np.float32)
    for t in range(T):
        o = np.zeros(Cc, np.float32)
        orc.orc_conv_step(f32p(buf), K, Cc, f32p(X[t * Cc:]), f32p(w), f32p(b), f32p(o))
        O[t * Cc:(t + 1) * Cc] = o
    assert np.abs(O[:Cc] - (b + w[K - 1::K] * X[:Cc])).max() < 1e-5
    # closed form: out_t[c] = b + sum_j w[c,j] x_{t-(K-1)+j}[c]
    Xr = X.reshape(T, Cc).astype(np.float64)
    for t in range(T):
        e = b.astype(np.float64).copy()
        for j in range(K):
            src = t - (K - 1) + j
            if src >= 0:
                e += w.reshape(Cc, K)[:, j] * Xr[src]
        assert np.abs(O[t * Cc:(t + 1) * Cc] - e).max() < 1e-5


# ---- router (tests/test_moe.c:18-32) ------------------------------------------------
def route(orc, logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    idx, w = np.zeros(k, np.int32), np.zeros(k, np.float32)
    orc.orc_moe_route(f32p(logits), logits.size, k, i32p(idx), f32p(w))
    return idx, w


def test_route_known_answer(orc):
    idx, w = route(orc, [0.1, 2.0, -1.0, 1.5, 0.5, 1.9], 3)
    assert list(idx) == [1, 5, 3]
    assert abs(w.sum() - 1) < 1e-6 and w[0] > w[1] > w[2]
    e = np.exp(np.float32([0.0, -0.1, -0.5]))
    assert abs(w[0] - e[0] / e.sum()) < 1e-5


def test_route_brute_force_ties(orc):
    rng = np.random.default_rng(3)
    for trial in range(200):
        ne, k = int(rng.integers(4, 64)), int(rng.integers(1, 4))
        lg = np.round(rng.standard_normal(ne), 1).astype(np.float32)   # many exact ties
        idx, _ = route(orc, lg, k)
        order = sorted(range(ne), key=lambda e: (-lg[e], e))           # ties -> lower index
        assert list(idx) == order[:k]


# ---- f32 helpers (tests/test_tensor.c) ------------------------------------------------
def test_tensor_known_answers(orc):
    x = np.float32([1, 2, 3, 4]); out = np.zeros(4, np.float32)
    orc.orc_rmsnorm(f32p(x), None, f32p(out), 4, 0.0)
    r = math.sqrt(7.5)
    assert abs(out[0] - 1 / r) < 1e-5 and abs(out[3] - 4 / r) < 1e-5
    s = np.float32([1, 2, 3]); orc.orc_softmax(f32p(s), 3)
    e = np.exp([-2.0, -1.0, 0.0]); assert abs(s.sum() - 1) < 1e-6 and abs(s[0] - e[0] / e.sum()) < 1e-5
    assert abs(orc.orc_sigmoid(0.0) - 0.5) < 1e-6 and abs(orc.orc_silu(1.0) - 0.7310586) < 1e-5
    assert abs(orc.orc_softplus(0.0) - 0.6931472) < 1e-5 and abs(orc.orc_softplus(100.0) - 100) < 1e-3
    assert 0 <= orc.orc_softplus(-100.0) < 1e-3
    y = np.zeros(4, np.float32); orc.orc_l2norm_eps(f32p(np.float32([3, 4, 0, 0])), f32p(y), 4, 0.0)
    assert abs(y[0] - 0.6) < 1e-5 and abs(y[1] - 0.8) < 1e-5
    v = np.float32([0.3, -0.7, 1.1, 0.5]); n0 = np.linalg.norm(v)
    orc.orc_rope_partial(f32p(v), 4, 4, 5, 10000.0); assert abs(np.linalg.norm(v) - n0) < 1e-4
    w = np.float32([1, 2, 3, 4]); orc.orc_rope_partial(f32p(w), 4, 4, 0, 10000.0)
    assert np.array_equal(w, np.float32([1, 2, 3, 4]))


# ---- bit-for-bit against the reference's own functions ---------------------------------
@ref_only
def test_helpers_bitexact_vs_reference(orc):
    R = clibs.ref()
    rng = np.random.default_rng(7)
    for n in (64, 128, 2048):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = rng.uniform(0.9, 1.1, n).astype(np.float32)
        a, b = np.zeros(n, np.float32), np.zeros(n, np.float32)
        orc.orc_rmsnorm(f32p(x), f32p(w), f32p(a), n, 1e-6); R.ot_rmsnorm(f32p(x), f32p(w), f32p(b), n, 1e-6)
        assert np.array_equal(bits(a), bits(b))
        orc.orc_l2norm_eps(f32p(x), f32p(a), n, 1e-6); R.ot_l2norm_eps(f32p(x), f32p(b), n, 1e-6)
        assert np.array_equal(bits(a), bits(b))
        a, b = x.copy(), x.copy(); orc.orc_softmax(f32p(a), n); R.ot_softmax(f32p(b), n)
        assert np.array_equal(bits(a), bits(b))
        for pos in (0, 1, 37, 4095):
            a, b = x[:256].copy() if n >= 256 else x.copy(), x[:256].copy() if n >= 256 else x.copy()
            hd = a.size
            orc.orc_rope_partial(f32p(a), hd, 64, pos, 1e7); R.ot_rope_partial(f32p(b), hd, 64, pos, 1e7)
            assert np.array_equal(bits(a), bits(b))
    for v in rng.standard_normal(2000).astype(np.float32) * 10:
        assert orc.orc_softplus(float(v)) == R.ot_softplus(float(v))
        assert orc.orc_sigmoid(float(v)) == R.ot_sigmoid(float(v))


@ref_only
def test_attn_core_bitexact_vs_reference(orc):
    R = clibs.ref()
    dk = dv = 16
    T = 21
    Q, K, V = rnd(20, T * dk), rnd(21, T * dk), rnd(22, T * dv)
    al = clibs.uniform(23, "al", T, 0.5, 0.99)
    be = clibs.uniform(24, "be", T, 0.1, 0.9)
    for chunk in (1, 5, 32):
        S1 = rnd(25, dk * dv); S2 = S1.copy()
        O1, O2 = np.zeros(T * dv, np.float32), np.zeros(T * dv, np.float32)
        orc.orc_delta_prefill(f32p(S1), dk, dv, f32p(Q), f32p(K), f32p(V), f32p(al), f32p(be), T, chunk, f32p(O1))
        st = clibs.RefDelta(f32p(S2), dk, dv)
        R.ornith_delta_prefill(C.byref(st), f32p(Q), f32p(K), f32p(V), f32p(al), f32p(be), T, chunk, f32p(O2))
        assert np.array_equal(bits(O1), bits(O2)) and np.array_equal(bits(S1), bits(S2))
    S1 = rnd(26, dk * dv); S2 = S1.copy()
    o1, o2 = np.zeros(dv, np.float32), np.zeros(dv, np.float32)
    orc.orc_delta_step(f32p(S1), dk, dv, f32p(Q), f32p(K), f32p(V), 0.8, 0.3, f32p(o1))
    st = clibs.RefDelta(f32p(S2), dk, dv)
    R.ornith_delta_step(C.byref(st), f32p(Q), f32p(K), f32p(V), 0.8, 0.3, f32p(o2))
    assert np.array_equal(bits(o1), bits(o2)) and np.array_equal(bits(S1), bits(S2))
    # GQA over the Q8 cache, 40 positions
    nh, nkv, hd, T = 8, 2, 64, 40
    Q, K, V = rnd(27, T * nh * hd), rnd(28, T * nkv * hd), rnd(29, T * nkv * hd)
    a, b = OrcKV(), clibs.RefKV()
    orc.orc_kv_init(C.byref(a), T, nkv, hd, 1); R.ornith_kv_init_ex(C.byref(b), T, nkv, hd, 1)
    for t in range(T):
        o1, o2 = np.zeros(nh * hd, np.float32), np.zeros(nh * hd, np.float32)
        args = (f32p(Q[t * nh * hd:]), f32p(K[t * nkv * hd:]), f32p(V[t * nkv * hd:]), nh)
        orc.orc_gqa_step(C.byref(a), *args, f32p(o1), 0.0)
        R.ornith_gqa_step(C.byref(b), *args, f32p(o2), 0.0)
        assert np.array_equal(bits(o1), bits(o2)), t
    orc.orc_kv_free(C.byref(a)); R.ornith_kv_free(C.byref(b))
    # conv
    Kc, Cc = 4, 48
    w = rnd(30, Cc * Kc)
    b1 = np.zeros((Kc - 1) * Cc, np.float32)
    st = clibs.RefConv(f32p(np.zeros((Kc - 1) * Cc + 1, np.float32)), Kc, Cc)
    for t in range(6):
        x = rnd(31 + t, Cc)
        o1, o2 = np.zeros(Cc, np.float32), np.zeros(Cc, np.float32)
        orc.orc_conv_step(f32p(b1), Kc, Cc, f32p(x), f32p(w), None, f32p(o1))
        R.ornith_conv_step(C.byref(st), f32p(x), f32p(w), None, f32p(o2))
        assert np.array_equal(bits(o1), bits(o2))


@ref_only
def test_route_bitexact_vs_reference(orc):
    R = clibs.ref()
    rng = np.random.default_rng(9)
    for _ in range(100):
        ne, k = 256, 8
        lg = (rng.standard_normal(ne) * 2).astype(np.float32)
        i1, w1 = route(orc, lg, k)
        i2, w2 = np.zeros(k, np.int32), np.zeros(k, np.float32)
        R.ornith_moe_route(f32p(lg), ne, k, i32p(i2), f32p(w2))
        assert np.array_equal(i1, i2) and np.array_equal(bits(w1), bits(w2))
