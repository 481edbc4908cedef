"""Regenerate the golden fixtures in tests/golden/ from the reference's own code.

Runs only where oracle/_ref/libornith_ref.so exists (the reference C sources
compiled in place by oracle/Makefile). Everything it writes is data: input
seeds/ids and the reference's outputs.

  c1.npz      C1 (tiny all-Q8_0 qwen35moe) GGUF sha256, prompt, 64 greedy
              tokens and logits at several steps, for the default chunked
              prefill and for ORNITH_PREFILL_SERIAL=1, both with ORNITH_KV_Q8=1.
  c1_session.json  SHA-256 and size of the reference's ORNSESS snapshot of a
              C1 session after the prompt and 8 greedy tokens, per prompt mode.
  codecs.npz  reference encodings of N(0,0.02) rows for Q8_0/Q4_K/Q6_K/IQ2_XXS
              at in=2048 and in=512, their decoded floats, the Q8_K bytes of
              N(0,1) seed-1 activations and the reference qdot / fallback dot.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import clibs  # noqa: E402
from clibs import (F32, IQ2_XXS, Q4_K, Q6_K, Q8_0, bp, f32p, i32p)  # noqa: E402

C1 = clibs.C1
PROMPT_LEN, N_GEN = 32, 64
TRACE_STEPS = (0, 1, 2, 4, 8, 16, 32, 63)


def c1_tensors(cfg: dict):
    """(name, kind, dims, type, lo, hi) in the exact order or_gen.c writes them."""
    H, V = cfg["hidden"], cfg["vocab"]
    qd = cfg["nk"] * cfg["dhead"]
    vd = cfg["nv"] * cfg["dhead"]
    cc = 2 * qd + vd
    T = []
    T.append(("token_embd.weight", "g", (H, V), cfg["t_embd"]))
    T.append(("output_norm.weight", "u", (H,), (0.9, 1.1)))
    T.append(("output.weight", "g", (H, V), cfg["t_output"]))
    for l in range(cfg["n_layers"]):
        full = l % cfg["full_interval"] == cfg["full_interval"] - 1
        b = f"blk.{l}."
        T.append((b + "attn_norm.weight", "u", (H,), (0.9, 1.1)))
        T.append((b + "post_attention_norm.weight", "u", (H,), (0.9, 1.1)))
        if full:
            T.append((b + "attn_q.weight", "g", (H, 2 * cfg["nh"] * cfg["hd"]), cfg["t_default"]))
            T.append((b + "attn_k.weight", "g", (H, cfg["nkv"] * cfg["hd"]), cfg["t_default"]))
            T.append((b + "attn_v.weight", "g", (H, cfg["nkv"] * cfg["hd"]), cfg["t_attn_v"]))
            T.append((b + "attn_q_norm.weight", "u", (cfg["hd"],), (0.9, 1.1)))
            T.append((b + "attn_k_norm.weight", "u", (cfg["hd"],), (0.9, 1.1)))
            T.append((b + "attn_output.weight", "g", (cfg["nh"] * cfg["hd"], H), cfg["t_default"]))
        else:
            T.append((b + "attn_qkv.weight", "g", (H, cc), cfg["t_default"]))
            T.append((b + "ssm_conv1d.weight", "u", (cfg["conv_k"], cc), (-0.2, 0.2)))
            T.append((b + "ssm_a", "u", (cfg["nv"],), (-0.8, -0.2)))
            T.append((b + "ssm_dt.bias", "u", (cfg["nv"],), (-0.05, 0.05)))
            T.append((b + "ssm_norm.weight", "u", (cfg["dhead"],), (0.9, 1.1)))
            T.append((b + "ssm_alpha.weight", "g", (H, cfg["nv"]), cfg["t_default"]))
            T.append((b + "ssm_beta.weight", "g", (H, cfg["nv"]), cfg["t_default"]))
            T.append((b + "attn_gate.weight", "g", (H, vd), cfg["t_default"]))
            T.append((b + "ssm_out.weight", "g", (vd, H), cfg["t_default"]))
        I, ne = cfg["moe_inter"], cfg["ne"]
        T.append((b + "ffn_gate_inp.weight", "g", (H, ne), cfg["t_default"]))
        T.append((b + "ffn_gate_exps.weight", "g", (H, I, ne), cfg["t_default"]))
        T.append((b + "ffn_up_exps.weight", "g", (H, I, ne), cfg["t_default"]))
        T.append((b + "ffn_down_exps.weight", "g", (I, H, ne), cfg["t_ffn_down"]))
        if cfg["shared_inter"] > 0:
            sI = cfg["shared_inter"]
            T.append((b + "ffn_gate_shexp.weight", "g", (H, sI), cfg["t_default"]))
            T.append((b + "ffn_up_shexp.weight", "g", (H, sI), cfg["t_default"]))
            T.append((b + "ffn_down_shexp.weight", "g", (sI, H), cfg["t_ffn_down"]))
            T.append((b + "ffn_gate_inp_shexp.weight", "g", (H,), cfg["t_default"]))
    return T


def write_with_reference(path: str, cfg: dict) -> None:
    """Same tensors and metadata as or_gen.c, but encoded and serialised by
    the reference's oq_quantize and ogguf writer."""
    R = clibs.ref()
    w = R.ogguf_writer_new()
    R.ogguf_w_string(w, b"general.architecture", b"qwen35moe")
    R.ogguf_w_string(w, b"general.name", b"ornith-hip-random-init")
    R.ogguf_w_u32(w, b"qwen35moe.block_count", cfg["n_layers"])
    R.ogguf_w_u32(w, b"qwen35moe.expert_used_count", cfg["top_k"])
    R.ogguf_w_u32(w, b"qwen35moe.rope.dimension_count", 64)
    R.ogguf_w_f32(w, b"qwen35moe.rope.freq_base", 1e7)
    R.ogguf_w_f32(w, b"qwen35moe.attention.layer_norm_rms_epsilon", 1e-6)
    toks = (C.c_char_p * cfg["vocab"])(*[f"t{i}".encode() for i in range(cfg["vocab"])])
    R.ogguf_w_arr_str(w, b"tokenizer.ggml.tokens", toks, cfg["vocab"])
    keep = []
    for name, kind, dims, extra in c1_tensors(cfg):
        n = int(np.prod(dims))
        if kind == "g":
            f = clibs.gauss(cfg["seed"], name, n, cfg["sigma"])
            data = clibs.quantize(R, extra, f, ref_api=True)
            t = extra
        else:
            data = clibs.uniform(cfg["seed"], name, n, *extra)
            t = F32
        keep.append(data)
        d = (C.c_uint64 * len(dims))(*dims)
        assert R.ogguf_w_tensor(w, name.encode(), len(dims), d, t, bp(data), data.nbytes) == 0
    assert R.ogguf_writer_write(w, str(path).encode()) == 0, R.ornith_last_error()
    R.ogguf_writer_free(w)


def sha256(path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def run_reference(path: str, prompt: np.ndarray, serial: bool):
    """Prompt eval + 64 greedy tokens through the reference session API with
    the Q8 KV cache; returns (tokens, {step: logits}, prompt_logits)."""
    R = clibs.ref()
    os.environ["ORNITH_KV_Q8"] = "1"
    if serial:
        os.environ["ORNITH_PREFILL_SERIAL"] = "1"
    else:
        os.environ.pop("ORNITH_PREFILL_SERIAL", None)
    m = C.c_void_p()
    assert R.rmodel_load(str(path).encode(), C.byref(m)) == 0, R.ornith_last_error()
    s = R.rmodel_session_new(m, PROMPT_LEN + N_GEN + 8)
    assert R.rmodel_session_eval(s, i32p(prompt), len(prompt)) == 0
    V = C1["vocab"]
    prompt_logits = np.ctypeslib.as_array(R.rmodel_session_logits(s), (V,)).copy()
    toks, trace = [], {}

    def on_token(tok, piece, ud):
        k = len(toks)
        if k in TRACE_STEPS and k > 0:
            # logits that produced token k = output of the forward of token k-1
            trace[k - 1] = np.ctypeslib.as_array(R.rmodel_session_logits(s), (V,)).copy()
        toks.append(tok)

    cb = clibs.TOKEN_CB(on_token)
    fin = C.c_int(0)
    assert R.rmodel_session_generate(s, N_GEN, None, 0, None, cb, None, C.byref(fin)) == 0
    trace[N_GEN - 1] = np.ctypeslib.as_array(R.rmodel_session_logits(s), (V,)).copy()
    R.rmodel_session_free(s)
    R.rmodel_free(m)
    os.environ.pop("ORNITH_PREFILL_SERIAL", None)
    return np.array(toks, np.int32), trace, prompt_logits


def make_c1(out: Path) -> None:
    with tempfile.TemporaryDirectory() as td:
        p_ref = Path(td) / "c1_ref.gguf"
        p_orc = Path(td) / "c1_oracle.gguf"
        write_with_reference(p_ref, C1)
        clibs.write_c1_gguf(p_orc, C1)
        h_ref, h_orc = sha256(p_ref), sha256(p_orc)
        assert h_ref == h_orc, f"oracle GGUF {h_orc} != reference GGUF {h_ref}"
        prompt = clibs.ids(C1["seed"], "prompt", PROMPT_LEN, C1["vocab"])
        res = {}
        for mode, serial in (("chunked", False), ("serial", True)):
            toks, trace, pl = run_reference(p_ref, prompt, serial)
            res[f"{mode}_tokens"] = toks
            res[f"{mode}_prompt_logits"] = pl
            steps = sorted(trace)
            res[f"{mode}_trace_steps"] = np.array(steps, np.int32)
            res[f"{mode}_trace_logits"] = np.stack([trace[k] for k in steps])
        np.savez_compressed(out / "c1.npz", gguf_sha256=np.array(h_ref), prompt=prompt,
                            file_size=np.array(p_ref.stat().st_size), **res)
        print("c1:", h_ref, "tokens", res["chunked_tokens"][:16], "...")


SESSION_GEN = 8


def make_session(out: Path) -> None:
    """rmodel_session_save after the C1 prompt and SESSION_GEN greedy tokens,
    Q8 KV, for the chunked and the serial prompt mode: the file's hash."""
    import json
    R = clibs.ref()
    res = {}
    with tempfile.TemporaryDirectory() as td:
        p_ref = Path(td) / "c1_ref.gguf"
        write_with_reference(p_ref, C1)
        prompt = clibs.ids(C1["seed"], "prompt", PROMPT_LEN, C1["vocab"])
        for mode, serial in (("chunked", False), ("serial", True)):
            os.environ["ORNITH_KV_Q8"] = "1"
            if serial:
                os.environ["ORNITH_PREFILL_SERIAL"] = "1"
            else:
                os.environ.pop("ORNITH_PREFILL_SERIAL", None)
            m = C.c_void_p()
            assert R.rmodel_load(str(p_ref).encode(), C.byref(m)) == 0, R.ornith_last_error()
            s = R.rmodel_session_new(m, PROMPT_LEN + SESSION_GEN + 8)
            assert R.rmodel_session_eval(s, i32p(prompt), len(prompt)) == 0
            toks = []
            cb = clibs.TOKEN_CB(lambda tok, piece, ud: toks.append(tok))
            fin = C.c_int(0)
            assert R.rmodel_session_generate(s, SESSION_GEN, None, 0, None, cb, None, C.byref(fin)) == 0
            f = Path(td) / f"{mode}.ornsess"
            assert R.rmodel_session_save(s, str(f).encode()) == 0
            data = f.read_bytes()
            res[mode] = {"pos": PROMPT_LEN + SESSION_GEN, "tokens": [int(t) for t in toks],
                         "bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}
            R.rmodel_session_free(s)
            R.rmodel_free(m)
            os.environ.pop("ORNITH_PREFILL_SERIAL", None)
    (out / "c1_session.json").write_text(json.dumps({"prompt_len": PROMPT_LEN, "generated": SESSION_GEN,
                                                      "modes": res}, indent=1) + "\n")
    print("c1 session:", {k: v["sha256"][:16] for k, v in res.items()})


def make_codecs(out: Path) -> None:
    R = clibs.ref()
    rows = 16
    res = {}
    for n in (2048, 512):
        x = clibs.gauss(1, f"act{n}", n, 1.0)
        xq = clibs.q8k(R, x, ref_api=True)
        res[f"act{n}"] = x
        res[f"act{n}_q8k"] = xq.view(np.uint8)
        for t in (Q8_0, Q4_K, Q6_K, IQ2_XXS):
            tn = clibs.TYPE_NAMES[t]
            w = clibs.gauss(0, f"w.{tn}.{n}", rows * n, 0.02)
            enc = clibs.quantize(R, t, w, ref_api=True)
            dec = clibs.dequantize(R, t, enc, rows * n, ref_api=True)
            rb = clibs.row_bytes(t, n)
            dots = np.zeros(rows, np.float32)
            for r in range(rows):
                row = np.ascontiguousarray(enc[r * rb:(r + 1) * rb])
                if R.qdot_can(t, n):
                    s = C.c_float(0)
                    R.qdot_vec_dot(t, n, C.byref(s), bp(row), bp(xq))
                    dots[r] = s.value
                else:  # reference f32 fallback: dequantised row . f32 activation
                    wr = np.ascontiguousarray(dec[r * n:(r + 1) * n])
                    dots[r] = R.ot_dot(f32p(wr), f32p(x), n)
            res[f"{tn}_{n}_enc"] = enc
            res[f"{tn}_{n}_dec"] = dec
            res[f"{tn}_{n}_dot"] = dots
    np.savez_compressed(out / "codecs.npz", **res)
    print("codecs: done")


if __name__ == "__main__":
    if not clibs.have_ref():
        sys.exit("oracle/_ref/libornith_ref.so not built: run `make -C oracle` where the reference tree exists")
    make_codecs(HERE)
    make_c1(HERE)
    make_session(HERE)
