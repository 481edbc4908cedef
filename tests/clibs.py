"""ctypes bindings for the CPU checker libraries (test infrastructure).

``oracle()`` loads oracle/liboracle.so (this repository's C restatement of the
reference decode path); ``ref()`` loads oracle/_ref/libornith_ref.so, the
reference's own C sources compiled in place by oracle/Makefile (present only
where /root/reference was available at build time). Neither is ever used by
the HIP engine itself.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libornith_ref.so"

F32, F16, Q8_0, Q4_K, Q6_K, IQ2_XXS, BF16 = 0, 1, 8, 12, 14, 16, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K",
              IQ2_XXS: "IQ2_XXS", BF16: "BF16"}
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144),
         Q6_K: (256, 210), IQ2_XXS: (256, 66)}

fp = C.POINTER(C.c_float)
ip = C.POINTER(C.c_int32)
vp = C.c_void_p


def row_bytes(t: int, n: int) -> int:
    be, bb = BLOCK[t]
    assert n % be == 0
    return n // be * bb


def f32p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(fp)


def i32p(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(ip)


def bp(a: np.ndarray):
    assert a.flags.c_contiguous
    return C.c_void_p(a.ctypes.data)


Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8K_DTYPE.itemsize == 292


class GenCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden", "n_layers", "vocab", "full_interval", "nh", "nkv", "hd",
        "nk", "nv", "dhead", "conv_k", "ne", "top_k", "moe_inter", "shared_inter")] + [
        ("t_default", C.c_uint32), ("t_attn_v", C.c_uint32), ("t_ffn_down", C.c_uint32),
        ("t_output", C.c_uint32), ("t_embd", C.c_uint32), ("seed", C.c_uint64),
        ("sigma", C.c_float), ("t_exps", C.c_uint32)]


class Arch(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden", "n_layers", "vocab", "full_interval", "nh", "nkv", "hd", "rope_dim",
        "nk", "nv", "dk", "dv", "conv_k", "ne", "top_k", "moe_inter", "shared_inter")] + [
        ("rope_theta", C.c_float), ("eps", C.c_float), ("eos", C.c_int)]


class OrcTensor(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("type", C.c_uint32), ("n_elements", C.c_uint64), ("data", C.c_void_p),
                ("nbytes", C.c_uint64)]


class OrcKV(C.Structure):
    _fields_ = [("K", fp), ("V", fp), ("Kq", C.POINTER(C.c_int8)), ("Vq", C.POINTER(C.c_int8)),
                ("Ks", fp), ("Vs", fp), ("quantized", C.c_int), ("capacity", C.c_int),
                ("len", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int)]


# Benchmark configurations. C1 is the tiny all-Q8_0 model; C3 the 35B shape.
C1 = dict(hidden=512, n_layers=4, vocab=4096, full_interval=4, nh=8, nkv=2, hd=64,
          nk=4, nv=8, dhead=64, conv_k=4, ne=16, top_k=4, moe_inter=256, shared_inter=256,
          t_default=Q8_0, t_attn_v=Q8_0, t_ffn_down=Q8_0, t_output=Q8_0, t_embd=Q8_0,
          seed=0, sigma=0.02)


def gen_cfg(**kw) -> GenCfg:
    return GenCfg(**kw)


_oracle = None
_ref = None


def oracle():
    """The restatement library; raises if it has not been built."""
    global _oracle
    if _oracle is not None:
        return _oracle
    if not ORACLE_SO.exists():
        raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle` (or __graft_entry__.build())")
    L = C.CDLL(str(ORACLE_SO))
    sig = {
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_row_bytes": (C.c_size_t, [C.c_uint32, C.c_size_t]),
        "orc_quantize": (C.c_int, [C.c_uint32, fp, vp, C.c_size_t]),
        "orc_dequantize": (C.c_int, [C.c_uint32, vp, fp, C.c_size_t]),
        "orc_quantize_q8k": (None, [fp, vp, C.c_int64]),
        "orc_qdot_can": (C.c_int, [C.c_uint32, C.c_int]),
        "orc_qdot": (C.c_float, [C.c_uint32, C.c_int, vp, vp]),
        "orc_matvec": (None, [C.c_uint32, vp, C.c_int, C.c_int, fp, fp, C.c_int, C.c_int]),
        "orc_rmsnorm": (None, [fp, fp, fp, C.c_int, C.c_float]),
        "orc_softmax": (None, [fp, C.c_int]),
        "orc_sigmoid": (C.c_float, [C.c_float]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_softplus": (C.c_float, [C.c_float]),
        "orc_dot": (C.c_float, [fp, fp, C.c_int]),
        "orc_l2norm_eps": (None, [fp, fp, C.c_int, C.c_float]),
        "orc_rope_partial": (None, [fp, C.c_int, C.c_int, C.c_int, C.c_float]),
        "orc_kv_init": (C.c_int, [C.POINTER(OrcKV), C.c_int, C.c_int, C.c_int, C.c_int]),
        "orc_kv_free": (None, [C.POINTER(OrcKV)]),
        "orc_kv_quant_vec": (C.c_float, [fp, C.c_int, vp]),
        "orc_gqa_step": (None, [C.POINTER(OrcKV), fp, fp, fp, C.c_int, fp, C.c_float]),
        "orc_gqa_attend": (None, [C.POINTER(OrcKV), fp, C.c_int, fp, C.c_float]),
        "orc_delta_step": (None, [fp, C.c_int, C.c_int, fp, fp, fp, C.c_float, C.c_float, fp]),
        "orc_delta_prefill": (None, [fp, C.c_int, C.c_int, fp, fp, fp, fp, fp, C.c_int, C.c_int, fp]),
        "orc_conv_step": (None, [fp, C.c_int, C.c_int, fp, fp, fp, fp]),
        "orc_moe_route": (None, [fp, C.c_int, C.c_int, ip, fp]),
        "orc_stream_key": (C.c_uint64, [C.c_uint64, C.c_char_p]),
        "orc_fill_gauss": (None, [C.c_uint64, C.c_float, fp, C.c_size_t, C.c_size_t]),
        "orc_fill_uniform": (None, [C.c_uint64, C.c_float, C.c_float, fp, C.c_size_t, C.c_size_t]),
        "orc_fill_ids": (None, [C.c_uint64, C.c_int32, ip, C.c_size_t]),
        "orc_gen_write_gguf": (C.c_int, [C.POINTER(GenCfg), C.c_char_p]),
        "orc_model_load": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "orc_model_free": (None, [vp]),
        "orc_model_arch": (C.POINTER(Arch), [vp]),
        "orc_model_set_threads": (None, [vp, C.c_int]),
        "orc_model_set_no_qdot": (None, [vp, C.c_int]),
        "orc_session_new": (vp, [vp, C.c_int, C.c_int]),
        "orc_session_free": (None, [vp]),
        "orc_session_eval": (C.c_int, [vp, ip, C.c_int, C.c_int]),
        "orc_session_generate": (C.c_int, [vp, C.c_int, ip, ip, fp]),
        "orc_session_step": (C.c_int, [vp, C.c_int32]),
        "orc_session_logits": (fp, [vp]),
        "orc_session_pos": (C.c_int, [vp]),
        "orc_session_delta": (fp, [vp, C.c_int]),
        "orc_session_conv": (fp, [vp, C.c_int]),
        "orc_session_kv": (C.POINTER(OrcKV), [vp, C.c_int]),
        "orc_session_seed_context": (C.c_int, [vp, C.c_int, C.c_uint64]),
        "orc_session_adopt": (C.c_int, [vp, C.c_int, fp]),
        "orc_last_error": (C.c_char_p, []),
        "orc_gguf_load": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "orc_gguf_free": (None, [vp]),
        "orc_gguf_n_tensors": (C.c_uint64, [vp]),
        "orc_gguf_tensor": (C.POINTER(OrcTensor), [vp, C.c_uint64]),
        "orc_writer_new": (vp, []),
        "orc_writer_free": (None, [vp]),
        "orc_w_string": (C.c_int, [vp, C.c_char_p, C.c_char_p]),
        "orc_w_u32": (C.c_int, [vp, C.c_char_p, C.c_uint32]),
        "orc_w_f32": (C.c_int, [vp, C.c_char_p, C.c_float]),
        "orc_w_arr_str": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_char_p), C.c_size_t]),
        "orc_w_tensor": (C.c_int, [vp, C.c_char_p, C.c_uint32, C.POINTER(C.c_uint64), C.c_uint32, vp, C.c_uint64]),
        "orc_writer_write": (C.c_int, [vp, C.c_char_p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _oracle = L
    return L


def have_ref() -> bool:
    return REF_SO.exists()


class RefKV(C.Structure):
    _fields_ = [("K", fp), ("V", fp), ("Kq", C.POINTER(C.c_int8)), ("Vq", C.POINTER(C.c_int8)),
                ("Ks", fp), ("Vs", fp), ("quantized", C.c_int), ("capacity", C.c_int),
                ("len", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int)]


class RefDelta(C.Structure):
    _fields_ = [("S", fp), ("dk", C.c_int), ("dv", C.c_int)]


class RefConv(C.Structure):
    _fields_ = [("buf", fp), ("K", C.c_int), ("C", C.c_int)]


TOKEN_CB = C.CFUNCTYPE(None, C.c_int32, C.c_char_p, C.c_void_p)


def ref():
    """The reference's own C code (oracle/_ref), for golden vectors."""
    global _ref
    if _ref is not None:
        return _ref
    if not REF_SO.exists():
        raise RuntimeError(f"{REF_SO} missing (built only where the reference tree exists)")
    L = C.CDLL(str(REF_SO))
    sig = {
        "oq_quantize": (C.c_int, [C.c_uint32, fp, vp, C.c_size_t]),
        "oq_dequantize": (C.c_int, [C.c_uint32, vp, fp, C.c_size_t]),
        "oq_f32_to_f16": (C.c_uint16, [C.c_float]),
        "oq_f16_to_f32": (C.c_float, [C.c_uint16]),
        "qdot_quantize_row_q8_K": (None, [fp, vp, C.c_int64]),
        "qdot_vec_dot": (None, [C.c_uint32, C.c_int, fp, vp, vp]),
        "qdot_can": (C.c_bool, [C.c_uint32, C.c_int]),
        "ornith_moe_route": (None, [fp, C.c_int, C.c_int, ip, fp]),
        "ornith_kv_init_ex": (C.c_int, [C.POINTER(RefKV), C.c_int, C.c_int, C.c_int, C.c_int]),
        "ornith_kv_free": (None, [C.POINTER(RefKV)]),
        "ornith_gqa_step": (None, [C.POINTER(RefKV), fp, fp, fp, C.c_int, fp, C.c_float]),
        "ornith_delta_step": (None, [C.POINTER(RefDelta), fp, fp, fp, C.c_float, C.c_float, fp]),
        "ornith_delta_prefill": (None, [C.POINTER(RefDelta), fp, fp, fp, fp, fp, C.c_int, C.c_int, fp]),
        "ornith_conv_step": (None, [C.POINTER(RefConv), fp, fp, fp, fp]),
        "ot_rmsnorm": (None, [fp, fp, fp, C.c_int, C.c_float]),
        "ot_softmax": (None, [fp, C.c_int]),
        "ot_l2norm_eps": (None, [fp, fp, C.c_int, C.c_float]),
        "ot_rope_partial": (None, [fp, C.c_int, C.c_int, C.c_int, C.c_float]),
        "ot_softplus": (C.c_float, [C.c_float]),
        "ot_sigmoid": (C.c_float, [C.c_float]),
        "ot_dot": (C.c_float, [fp, fp, C.c_int]),
        "ogguf_writer_new": (vp, []),
        "ogguf_writer_free": (None, [vp]),
        "ogguf_w_string": (C.c_int, [vp, C.c_char_p, C.c_char_p]),
        "ogguf_w_u32": (C.c_int, [vp, C.c_char_p, C.c_uint32]),
        "ogguf_w_f32": (C.c_int, [vp, C.c_char_p, C.c_float]),
        "ogguf_w_arr_str": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_char_p), C.c_size_t]),
        "ogguf_w_tensor": (C.c_int, [vp, C.c_char_p, C.c_uint32, C.POINTER(C.c_uint64), C.c_uint32, vp, C.c_uint64]),
        "ogguf_writer_write": (C.c_int, [vp, C.c_char_p]),
        "rmodel_load": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "rmodel_free": (None, [vp]),
        "rmodel_session_new": (vp, [vp, C.c_int]),
        "rmodel_session_free": (None, [vp]),
        "rmodel_session_eval": (C.c_int, [vp, ip, C.c_int]),
        "rmodel_session_logits": (fp, [vp]),
        "rmodel_session_pos": (C.c_int, [vp]),
        "rmodel_session_generate": (C.c_int, [vp, C.c_int, ip, C.c_int, vp, TOKEN_CB, vp, ip]),
        "rmodel_session_save": (C.c_int, [vp, C.c_char_p]),
        "ornith_last_error": (C.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _ref = L
    return L


def gauss(seed: int, name: str, n: int, sigma: float = 1.0) -> np.ndarray:
    L = oracle()
    out = np.empty(n, np.float32)
    L.orc_fill_gauss(L.orc_stream_key(seed, name.encode()), sigma, f32p(out), n, 0)
    return out


def uniform(seed: int, name: str, n: int, lo: float, hi: float) -> np.ndarray:
    L = oracle()
    out = np.empty(n, np.float32)
    L.orc_fill_uniform(L.orc_stream_key(seed, name.encode()), lo, hi, f32p(out), n, 0)
    return out


def ids(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    L = oracle()
    out = np.empty(n, np.int32)
    L.orc_fill_ids(L.orc_stream_key(seed, name.encode()), vocab, i32p(out), n)
    return out


def quantize(L, t: int, x: np.ndarray, ref_api: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(row_bytes(t, x.size), np.uint8)
    fn = L.oq_quantize if ref_api else L.orc_quantize
    assert fn(t, f32p(x), bp(out), x.size) == 0
    return out


def dequantize(L, t: int, b: np.ndarray, n: int, ref_api: bool = False) -> np.ndarray:
    out = np.zeros(n, np.float32)
    fn = L.oq_dequantize if ref_api else L.orc_dequantize
    assert fn(t, bp(np.ascontiguousarray(b)), f32p(out), n) == 0
    return out


def q8k(L, x: np.ndarray, ref_api: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256, Q8K_DTYPE)
    fn = L.qdot_quantize_row_q8_K if ref_api else L.orc_quantize_q8k
    fn(f32p(x), bp(out), x.size)
    return out


def write_c1_gguf(path: str, cfg: dict | None = None) -> None:
    """Write a random-init GGUF with the oracle generator."""
    c = gen_cfg(**(cfg or C1))
    L = oracle()
    st = L.orc_gen_write_gguf(C.byref(c), str(path).encode())
    if st:
        raise RuntimeError(L.orc_last_error().decode())


def gguf_tensors(path) -> dict:
    """name -> (type, dims, bytes) of every tensor of a GGUF, via the oracle loader."""
    L = oracle()
    g = C.c_void_p()
    st = L.orc_gguf_load(str(path).encode(), C.byref(g))
    if st:
        raise RuntimeError(L.orc_last_error().decode())
    out = {}
    for i in range(L.orc_gguf_n_tensors(g)):
        t = L.orc_gguf_tensor(g, i).contents
        raw = C.string_at(t.data, t.nbytes) if t.nbytes else b""
        out[t.name.decode()] = (t.type, tuple(t.dims[:t.n_dims]), np.frombuffer(raw, np.uint8).copy())
    L.orc_gguf_free(g)
    return out


def model_tensor_names(cfg: dict) -> list:
    """The qwen35moe tensor names of a generator configuration (the ones a
    model may hold; absent ones are skipped by the callers)."""
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    fi = cfg.get("full_interval", 4)
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        names += [b + "attn_norm.weight", b + "post_attention_norm.weight"]
        if l % fi == fi - 1:
            names += [b + s for s in ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q_norm.weight",
                                      "attn_k_norm.weight", "attn_output.weight")]
        else:
            names += [b + s for s in ("attn_qkv.weight", "ssm_conv1d.weight", "ssm_a", "ssm_dt.bias",
                                      "ssm_norm.weight", "ssm_alpha.weight", "ssm_beta.weight",
                                      "attn_gate.weight", "ssm_out.weight")]
        names += [b + s for s in ("ffn_gate_inp.weight", "ffn_gate_exps.weight", "ffn_up_exps.weight",
                                  "ffn_down_exps.weight", "ffn_gate_shexp.weight", "ffn_up_shexp.weight",
                                  "ffn_down_shexp.weight", "ffn_gate_inp_shexp.weight", "ffn_gate.weight",
                                  "ffn_up.weight", "ffn_down.weight")]
    return names


def write_model_gguf(model, cfg: dict, path, n_layers: int | None = None) -> None:
    """Write the tensors of a device model (the first n_layers layers) to a
    GGUF with the oracle writer, with the metadata the reference loader reads
    (architecture, expert count, RoPE, eps, vocabulary strings)."""
    L = oracle()
    c = dict(cfg, n_layers=n_layers or cfg["n_layers"])
    ne = cfg["ne"]
    w = L.orc_writer_new()
    L.orc_w_string(w, b"general.architecture", b"qwen35moe")
    L.orc_w_u32(w, b"qwen35moe.block_count", c["n_layers"])
    L.orc_w_u32(w, b"qwen35moe.expert_used_count", cfg["top_k"])
    L.orc_w_u32(w, b"qwen35moe.rope.dimension_count", 64)
    L.orc_w_f32(w, b"qwen35moe.rope.freq_base", 1e7)
    L.orc_w_f32(w, b"qwen35moe.attention.layer_norm_rms_epsilon", 1e-6)
    toks = (C.c_char_p * cfg["vocab"])(*[f"t{i}".encode() for i in range(cfg["vocab"])])
    L.orc_w_arr_str(w, b"tokenizer.ggml.tokens", toks, cfg["vocab"])
    keep = []
    for n in model_tensor_names(c):
        info = model.tensor_info(n)
        if info is None:
            continue
        data = model.tensor(n).download(info["nbytes"])
        keep.append(data)
        dims = [info["cols"], info["rows"]]
        if "_exps." in n:
            dims = [info["cols"], info["rows"] // ne, ne]
        elif info["rows"] == 1 and n.endswith(("_norm.weight", "ssm_a", "ssm_dt.bias", "ffn_gate_inp_shexp.weight")):
            dims = [info["cols"]]
        d = (C.c_uint64 * len(dims))(*dims)
        st = L.orc_w_tensor(w, n.encode(), len(dims), d, info["type"], C.c_void_p(data.ctypes.data), data.nbytes)
        if st:
            raise RuntimeError(L.orc_last_error().decode())
    st = L.orc_writer_write(w, str(path).encode())
    L.orc_writer_free(w)
    if st:
        raise RuntimeError(L.orc_last_error().decode())


def adopt_state(orc, dst, arch, pos, logits, delta_of, conv_of, kv_of):
    """Copy a session's state into the empty oracle session `dst` (delta state
    and conv window of every linear layer, the Q8 KV codes and scales of every
    full-attention layer, in the reference's host layouts) and declare it at
    position `pos` with last logits `logits` (orc_session_adopt), so that the
    oracle's token steps continue from that state. delta_of(l), conv_of(l)
    and kv_of(l) -> (Kq, Ks, Vq, Vs) read the source session."""
    nv, dv, dk = arch["nv"], arch["dv"], arch["dk"]
    cc = 2 * arch["nk"] * dk + nv * dv
    kvn = pos * arch["nkv"] * arch["hd"]
    for l in range(arch["n_layers"]):
        kvp = orc.orc_session_kv(dst, l)
        if kvp:
            kv = kvp.contents
            assert kv.quantized == 1 and kv.capacity > pos
            kq, ks, vq, vs = kv_of(l)
            np.ctypeslib.as_array(kv.Kq, (kvn,))[:] = np.asarray(kq, np.int8).reshape(-1)[:kvn]
            np.ctypeslib.as_array(kv.Vq, (kvn,))[:] = np.asarray(vq, np.int8).reshape(-1)[:kvn]
            ns = pos * arch["nkv"]
            np.ctypeslib.as_array(kv.Ks, (ns,))[:] = np.asarray(ks, np.float32).reshape(-1)[:ns]
            np.ctypeslib.as_array(kv.Vs, (ns,))[:] = np.asarray(vs, np.float32).reshape(-1)[:ns]
        else:
            np.ctypeslib.as_array(orc.orc_session_delta(dst, l), (nv * dv * dk,))[:] = delta_of(l)
            np.ctypeslib.as_array(orc.orc_session_conv(dst, l), ((arch["conv_k"] - 1) * cc,))[:] = conv_of(l)
    lg = np.ascontiguousarray(logits, np.float32)
    assert orc.orc_session_adopt(dst, int(pos), f32p(lg)) == 0


def orc_arch_dict(orc, model) -> dict:
    a = orc.orc_model_arch(model).contents
    return {k: getattr(a, k) for k in ("hidden", "n_layers", "vocab", "nh", "nkv", "hd", "nk", "nv", "dk", "dv",
                                       "conv_k", "ne", "top_k")}
