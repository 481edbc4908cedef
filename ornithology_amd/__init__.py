"""ornithology_amd - Python handle on the MI355X (gfx950) decode engine.

The engine is native: ``libornith_hip.so`` (HIP kernels + C++ host, C ABI in
include/ornith_hip.h). This module only loads it with ctypes and mirrors the
reference session API (``rmodel_load``, ``rmodel_session_new/eval/logits/
generate``, src/ornith_rforward.h:24-130) for tests, the smoke check and
bench.py. There is no CPU fallback: if the library is missing or no GPU is
visible the calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libornith_hip.so"
HEADER = HERE.parent / "include" / "ornith_hip.h"

F32, F16, Q8_0, Q4_K, Q6_K, IQ2_XXS, BF16 = 0, 1, 8, 12, 14, 16, 30
TYPE_IDS = {"F32": F32, "F16": F16, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q6_K": Q6_K,
            "IQ2_XXS": IQ2_XXS, "BF16": BF16}
_BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144),
          Q6_K: (256, 210), IQ2_XXS: (256, 66)}

STATUS = {0: "OK", 1: "ERR_IO", 2: "ERR_FORMAT", 3: "ERR_UNSUPPORTED", 4: "ERR_OOM",
          5: "ERR_NOTFOUND", 6: "ERR_DEVICE"}

Q8K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8K.itemsize == 292

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)


class HipError(RuntimeError):
    def __init__(self, status: int, where: str, msg: str):
        super().__init__(f"{where}: {STATUS.get(status, status)}: {msg}")
        self.status = status


class Arch(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "n_layers", "vocab", "full_interval", "nh", "nkv", "hd", "rope_dim",
        "nk", "nv", "dk", "dv", "conv_k", "ne", "top_k", "moe_inter", "shared_inter")] + [
        ("rope_theta", C.c_float), ("eps", C.c_float), ("eos", C.c_int32)]


class GenCfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "n_layers", "vocab", "full_interval", "nh", "nkv", "hd",
        "nk", "nv", "dhead", "conv_k", "ne", "top_k", "moe_inter", "shared_inter")] + [
        ("t_default", C.c_uint32), ("t_attn_v", C.c_uint32), ("t_ffn_down", C.c_uint32),
        ("t_output", C.c_uint32), ("t_embd", C.c_uint32), ("seed", C.c_uint64),
        ("sigma", C.c_float), ("t_exps", C.c_uint32)]


_SIGS = {
    "ornith_hip_last_error": (C.c_char_p, []),
    "ornith_hip_init": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "ornith_hip_free": (None, [_vp]),
    "ornith_hip_sync": (C.c_int, [_vp]),
    "ornith_hip_upload": (C.c_int, [_vp, C.c_char_p, C.c_uint32, _vp, C.c_uint64, C.c_uint32,
                                    C.POINTER(C.c_uint64), C.POINTER(_vp)]),
    "ornith_hip_tensor_free": (None, [_vp]),
    "ornith_hip_tensor_download": (C.c_int, [_vp, _vp, C.c_uint64]),
    "ornith_hip_quantize_q8K": (C.c_int, [_vp, _fp, C.c_int64, _vp]),
    "ornith_hip_matvec": (C.c_int, [_vp, _vp, _fp, _fp, C.c_int]),
    "ornith_hip_matvec_noalloc": (C.c_int, [_vp, _vp, _fp, _fp, C.c_int]),
    "ornith_hip_dequant": (C.c_int, [_vp, _vp, C.c_int64, C.c_int64, _fp]),
    "ornith_hip_moe_route": (C.c_int, [_vp, _fp, C.c_int, C.c_int, _ip, _fp]),
    "ornith_hip_model_load": (C.c_int, [_vp, C.c_char_p, C.POINTER(_vp)]),
    "ornith_hip_model_synth": (C.c_int, [_vp, C.POINTER(GenCfg), C.POINTER(_vp)]),
    "ornith_hip_model_free": (None, [_vp]),
    "ornith_hip_model_arch": (C.c_int, [_vp, C.POINTER(Arch)]),
    "ornith_hip_model_bytes": (C.c_uint64, [_vp]),
    "ornith_hip_model_tensor_info": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32),
                                               C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                               C.POINTER(C.c_uint64)]),
    "ornith_hip_model_tensor": (_vp, [_vp, C.c_char_p]),
    "ornith_hip_session_new": (C.c_int, [_vp, C.c_int, C.POINTER(_vp)]),
    "ornith_hip_session_free": (None, [_vp]),
    "ornith_hip_session_eval": (C.c_int, [_vp, _ip, C.c_int]),
    "ornith_hip_session_logits": (C.c_int, [_vp, _fp]),
    "ornith_hip_session_pos": (C.c_int, [_vp]),
    "ornith_hip_session_generate": (C.c_int, [_vp, C.c_int, _ip, _ip]),
    "ornith_hip_session_step": (C.c_int, [_vp, C.c_int32]),
    "ornith_hip_batch_step": (C.c_int, [C.POINTER(_vp), C.c_int, _ip, _ip]),
    "ornith_hip_quantize": (C.c_int, [_vp, C.c_uint32, _fp, C.c_uint64, _vp]),
    "ornith_hip_session_save": (C.c_int, [_vp, C.c_char_p]),
    "ornith_hip_session_load": (C.c_int, [_vp, C.c_char_p, C.c_int, C.POINTER(_vp)]),
    "ornith_hip_session_get_delta": (C.c_int, [_vp, C.c_int, _fp]),
    "ornith_hip_session_get_conv": (C.c_int, [_vp, C.c_int, _fp]),
    "ornith_hip_session_get_kv": (C.c_int, [_vp, C.c_int, _vp, _fp, _vp, _fp]),
    "ornith_hip_session_get_attn": (C.c_int, [_vp, C.c_int, _fp, _fp, _fp, _ip]),
    "ornith_hip_session_time_decode": (C.c_int, [_vp, C.c_int, _fp]),
    "ornith_hip_time_matvec": (C.c_int, [_vp, _vp, C.c_int, _fp]),
    "ornith_hip_time_matvec_set": (C.c_int, [_vp, C.POINTER(_vp), C.c_int, C.c_int, _fp]),
    "ornith_hip_session_profile_step": (C.c_int, [_vp, C.c_int, _ip, C.POINTER(C.c_double), _fp, _ip]),
    "ornith_hip_session_time_kind": (C.c_int, [_vp, C.c_int, C.c_int, _fp, C.POINTER(C.c_double), _ip]),
    "ornith_hip_session_profile_phases": (C.c_int, [_vp, C.c_int, _ip, C.POINTER(C.c_double), _fp, _ip]),
    "ornith_hip_session_profile_decode": (C.c_int, [_vp, C.c_int, _ip, _fp, _fp, _ip]),
    "ornith_hip_session_profile_decode_op": (C.c_int, [_vp, C.c_int, _fp, C.c_int, _ip]),
}

_lib = None


def lib():
    """Load libornith_hip.so (built in place by __graft_entry__.build())."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                           " (there is no CPU fallback)")
    L = C.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _lib = L
    return L


def _check(st: int, where: str) -> None:
    if st != 0:
        raise HipError(st, where, (lib().ornith_hip_last_error() or b"").decode())


def _f32(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _i32(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


class Context:
    """One device, one stream (ornith_hip_init)."""

    def __init__(self, device: int = 0):
        L = lib()
        h = _vp()
        _check(L.ornith_hip_init(device, C.byref(h)), "ornith_hip_init")
        self.h = h

    def sync(self) -> None:
        _check(lib().ornith_hip_sync(self.h), "ornith_hip_sync")

    def close(self):
        if self.h:
            lib().ornith_hip_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- ornith_qdot / codecs ------------------------------------------------
    def upload(self, name: str, ggml_type: int, data: np.ndarray, dims) -> "Tensor":
        data = np.ascontiguousarray(data).view(np.uint8)
        d = (C.c_uint64 * len(dims))(*dims)
        h = _vp()
        _check(lib().ornith_hip_upload(self.h, name.encode(), ggml_type, C.c_void_p(data.ctypes.data),
                                       data.nbytes, len(dims), d, C.byref(h)), "ornith_hip_upload")
        return Tensor(self, h, ggml_type, dims)

    def quantize(self, ggml_type: int, x: np.ndarray) -> np.ndarray:
        """oq_quantize on the device (Q8_0, Q4_K, Q6_K, IQ2_XXS): GGUF block bytes."""
        x = np.ascontiguousarray(x, np.float32)
        nbytes = {Q8_0: 34 * 8, Q4_K: 144, Q6_K: 210, IQ2_XXS: 66}[ggml_type] * (x.size // 256)
        out = np.zeros(nbytes, np.uint8)
        _check(lib().ornith_hip_quantize(self.h, ggml_type, _f32(x), x.size, out.ctypes.data_as(_vp)),
               "ornith_hip_quantize")
        return out

    def time_matvec_set(self, tensors, iters: int) -> float:
        """Mean ms per matvec launch, round-robin over distinct tensors of one
        type and shape (cold caches), replayed as one HIP graph."""
        arr = (_vp * len(tensors))(*[t.h for t in tensors])
        ms = C.c_float(0)
        _check(lib().ornith_hip_time_matvec_set(self.h, arr, len(tensors), iters, C.byref(ms)),
               "ornith_hip_time_matvec_set")
        return ms.value

    def quantize_q8k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256, Q8K)
        _check(lib().ornith_hip_quantize_q8K(self.h, _f32(x), x.size, C.c_void_p(out.ctypes.data)),
               "ornith_hip_quantize_q8K")
        return out

    def moe_route(self, logits: np.ndarray, k: int):
        logits = np.ascontiguousarray(logits, np.float32)
        idx = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        _check(lib().ornith_hip_moe_route(self.h, _f32(logits), logits.size, k, _i32(idx), _f32(w)),
               "ornith_hip_moe_route")
        return idx, w

    def load(self, path: str) -> "Model":
        h = _vp()
        _check(lib().ornith_hip_model_load(self.h, str(path).encode(), C.byref(h)), "ornith_hip_model_load")
        return Model(self, h)

    def synth(self, **cfg) -> "Model":
        c = GenCfg(**cfg)
        h = _vp()
        _check(lib().ornith_hip_model_synth(self.h, C.byref(c), C.byref(h)), "ornith_hip_model_synth")
        return Model(self, h)


class Tensor:
    def __init__(self, ctx: Context, h, ggml_type: int, dims):
        self.ctx, self.h, self.type, self.dims = ctx, h, ggml_type, tuple(int(d) for d in dims)
        self.owned = True

    @property
    def rows(self) -> int:
        return int(np.prod(self.dims[1:])) if len(self.dims) > 1 else 1

    @property
    def cols(self) -> int:
        return self.dims[0]

    def matvec(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        tn = x.size // self.cols
        y = np.zeros(tn * self.rows, np.float32)
        _check(lib().ornith_hip_matvec(self.ctx.h, self.h, _f32(x), _f32(y), tn), "ornith_hip_matvec")
        return y

    def matvec_noalloc(self, x: np.ndarray) -> np.ndarray:
        """matvec through the entry point that allocates nothing (the fixed
        per-device scratch array; results equal matvec's)."""
        x = np.ascontiguousarray(x, np.float32)
        tn = x.size // self.cols
        y = np.zeros(tn * self.rows, np.float32)
        _check(lib().ornith_hip_matvec_noalloc(self.ctx.h, self.h, _f32(x), _f32(y), tn),
               "ornith_hip_matvec_noalloc")
        return y

    def dequant(self, row0: int = 0, nrows: int | None = None) -> np.ndarray:
        nrows = self.rows - row0 if nrows is None else nrows
        out = np.zeros(nrows * self.cols, np.float32)
        _check(lib().ornith_hip_dequant(self.ctx.h, self.h, row0, nrows, _f32(out)), "ornith_hip_dequant")
        return out

    def download(self, nbytes: int) -> np.ndarray:
        """The tensor's bytes in GGUF block order."""
        out = np.zeros(nbytes, np.uint8)
        _check(lib().ornith_hip_tensor_download(self.h, C.c_void_p(out.ctypes.data), nbytes),
               "ornith_hip_tensor_download")
        return out

    def time_matvec(self, iters: int) -> float:
        ms = C.c_float(0)
        _check(lib().ornith_hip_time_matvec(self.ctx.h, self.h, iters, C.byref(ms)), "ornith_hip_time_matvec")
        return ms.value

    def free(self):
        if self.h and self.owned:
            lib().ornith_hip_tensor_free(self.h)
        self.h = None


class Model:
    """rmodel_load / rmodel_arch (src/ornith_rforward.c:719-829)."""

    def __init__(self, ctx: Context, h):
        self.ctx, self.h = ctx, h
        a = Arch()
        _check(lib().ornith_hip_model_arch(h, C.byref(a)), "ornith_hip_model_arch")
        self.arch = {f: getattr(a, f) for f, _ in Arch._fields_}

    @property
    def nbytes(self) -> int:
        return int(lib().ornith_hip_model_bytes(self.h))

    def tensor_info(self, name: str):
        t, nb, rows, inn = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        st = lib().ornith_hip_model_tensor_info(self.h, name.encode(), C.byref(t), C.byref(nb),
                                                C.byref(rows), C.byref(inn))
        if st == 5:
            return None
        _check(st, "ornith_hip_model_tensor_info")
        return dict(type=t.value, nbytes=nb.value, rows=rows.value, cols=inn.value)

    def tensor(self, name: str) -> Tensor:
        h = lib().ornith_hip_model_tensor(self.h, name.encode())
        if not h:
            raise KeyError(name)
        info = self.tensor_info(name)
        t = Tensor(self.ctx, _vp(h), info["type"], (info["cols"], info["rows"]))
        t.owned = False
        return t

    def session(self, cap: int) -> "Session":
        h = _vp()
        _check(lib().ornith_hip_session_new(self.h, cap, C.byref(h)), "ornith_hip_session_new")
        return Session(self, h)

    def load_session(self, path, extra_cap: int = 0) -> "Session":
        """rmodel_session_load: a session from an ORNSESS snapshot."""
        h = _vp()
        _check(lib().ornith_hip_session_load(self.h, str(path).encode(), int(extra_cap), C.byref(h)),
               "ornith_hip_session_load")
        return Session(self, h)

    def batch_step(self, sessions, tokens) -> np.ndarray:
        """One token step of each session at once (ornith_hip_batch_step);
        returns each session's greedy next token."""
        n = len(sessions)
        hs = (_vp * n)(*[s.h for s in sessions])
        t = np.ascontiguousarray(tokens, np.int32)
        if t.size != n:
            raise ValueError(f"batch_step: {n} sessions, {t.size} tokens")
        out = np.zeros(n, np.int32)
        _check(lib().ornith_hip_batch_step(hs, n, _i32(t), _i32(out)), "ornith_hip_batch_step")
        return out

    def free(self):
        if self.h:
            lib().ornith_hip_model_free(self.h)
            self.h = None


class Session:
    """rmodel_session_* (src/ornith_rforward.h:92-130), greedy, Q8 KV cache."""

    def __init__(self, model: Model, h):
        self.model, self.h = model, h

    def eval(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, np.int32)
        _check(lib().ornith_hip_session_eval(self.h, _i32(t), t.size), "ornith_hip_session_eval")

    def save(self, path) -> None:
        """rmodel_session_save: the session as an ORNSESS snapshot."""
        _check(lib().ornith_hip_session_save(self.h, str(path).encode()), "ornith_hip_session_save")

    def step(self, token: int) -> None:
        _check(lib().ornith_hip_session_step(self.h, int(token)), "ornith_hip_session_step")

    def logits(self) -> np.ndarray:
        out = np.zeros(self.model.arch["vocab"], np.float32)
        _check(lib().ornith_hip_session_logits(self.h, _f32(out)), "ornith_hip_session_logits")
        return out

    @property
    def pos(self) -> int:
        return int(lib().ornith_hip_session_pos(self.h))

    def generate(self, n_predict: int) -> np.ndarray:
        out = np.zeros(max(n_predict, 1), np.int32)
        n = C.c_int32(0)
        _check(lib().ornith_hip_session_generate(self.h, n_predict, _i32(out), C.byref(n)),
               "ornith_hip_session_generate")
        return out[: n.value].copy()

    def time_decode(self, n_steps: int) -> float:
        ms = C.c_float(0)
        _check(lib().ornith_hip_session_time_decode(self.h, n_steps, C.byref(ms)), "ornith_hip_session_time_decode")
        return ms.value

    KERNEL_KINDS = ("matvec", "rmsnorm_q8k", "swiglu_q8k", "embed", "delta_step", "attn_prep",
                    "attn_scores", "attn_walk", "moe_route", "moe_combine", "argmax", "advance",
                    "moe_down", "attn_flash", "attn_combine", "matvec_q6k", "matvec_q80", "matvec_mixed",
                    "step_body", "step_head", "attn_main", "matvec_q4q6", "delta_mv")

    def time_kind(self, kind: str, reps: int = 5):
        """Back-to-back replay of one step's launches of `kind`: returns
        (us per launch, algorithmic bytes per launch, launches per step).
        Leaves the session state meaningless (measurement only)."""
        us, by, n = C.c_float(), C.c_double(), C.c_int()
        _check(lib().ornith_hip_session_time_kind(self.h, self.KERNEL_KINDS.index(kind), reps, C.byref(us),
                                                  C.byref(by), C.byref(n)), "ornith_hip_session_time_kind")
        return us.value, by.value, n.value

    def profile_step(self, max_launches: int = 4096):
        """One eager decode step with per-launch HIP-event timing: list of
        (kind, algorithmic bytes, ms)."""
        kinds = np.zeros(max_launches, np.int32)
        byts = np.zeros(max_launches, np.float64)
        ms = np.zeros(max_launches, np.float32)
        n = C.c_int32(0)
        _check(lib().ornith_hip_session_profile_step(self.h, max_launches, _i32(kinds),
                                                     byts.ctypes.data_as(C.POINTER(C.c_double)), _f32(ms),
                                                     C.byref(n)), "ornith_hip_session_profile_step")
        k = n.value
        return [(self.KERNEL_KINDS[kinds[i]], float(byts[i]), float(ms[i])) for i in range(k)]

    DECODE_OPS = ("embed", "matvec", "delta", "attn_prep", "attn", "attn_merge", "moe_down", "argmax")

    def profile_decode(self, max_ops: int = 4096):
        """[(kind, first_done_us, last_done_us)] per operation of one run of the
        decode step as a single persistent launch (the position is not advanced)."""
        kinds = np.zeros(max_ops, np.int32)
        a = np.zeros(max_ops, np.float32)
        b = np.zeros(max_ops, np.float32)
        n = C.c_int(0)
        _check(lib().ornith_hip_session_profile_decode(self.h, max_ops, _i32(kinds), _f32(a), _f32(b), C.byref(n)),
               "ornith_hip_session_profile_decode")
        return [(self.DECODE_OPS[kinds[i]], float(a[i]), float(b[i])) for i in range(n.value)]

    def profile_decode_op(self, op: int, max_groups: int = 1024) -> np.ndarray:
        """[groups, 8] sub-phase clocks (us) of operation `op` of the decode launch"""
        us = np.zeros(max_groups * 8, np.float32)
        g = C.c_int(0)
        _check(lib().ornith_hip_session_profile_decode_op(self.h, op, _f32(us), max_groups, C.byref(g)),
               "ornith_hip_session_profile_decode_op")
        return us[:g.value * 8].reshape(g.value, 8)

    def profile_phases(self, max_phases: int = 4096):
        """One step-kernel body launch at the current position (the position
        does not advance): list of (kind or None, algorithmic bytes, us) per
        phase, timed by workgroup 0's clock between grid barriers."""
        kinds = np.zeros(max_phases, np.int32)
        byts = np.zeros(max_phases, np.float64)
        us = np.zeros(max_phases, np.float32)
        n = C.c_int32(0)
        _check(lib().ornith_hip_session_profile_phases(self.h, max_phases, _i32(kinds),
                                                       byts.ctypes.data_as(C.POINTER(C.c_double)), _f32(us),
                                                       C.byref(n)), "ornith_hip_session_profile_phases")
        return [(self.KERNEL_KINDS[kinds[i]] if kinds[i] >= 0 else None, float(byts[i]), float(us[i]))
                for i in range(n.value)]

    def delta_state(self, layer: int) -> np.ndarray:
        a = self.model.arch
        out = np.zeros(a["nv"] * a["dv"] * a["dk"], np.float32)
        _check(lib().ornith_hip_session_get_delta(self.h, layer, _f32(out)), "ornith_hip_session_get_delta")
        return out

    def conv_state(self, layer: int) -> np.ndarray:
        a = self.model.arch
        cc = 2 * a["nk"] * a["dk"] + a["nv"] * a["dv"]
        out = np.zeros((a["conv_k"] - 1) * cc, np.float32)
        _check(lib().ornith_hip_session_get_conv(self.h, layer, _f32(out)), "ornith_hip_session_get_conv")
        return out

    def kv(self, layer: int):
        a = self.model.arch
        n = self.pos
        kq = np.zeros(n * a["nkv"] * a["hd"], np.int8)
        vq = np.zeros_like(kq)
        ks = np.zeros(n * a["nkv"], np.float32)
        vs = np.zeros_like(ks)
        _check(lib().ornith_hip_session_get_kv(self.h, layer, C.c_void_p(kq.ctypes.data), _f32(ks),
                                               C.c_void_p(vq.ctypes.data), _f32(vs)), "ornith_hip_session_get_kv")
        return kq, ks, vq, vs

    def attn(self, row: int = -1):
        """(q, gate, o, pos) of the last full-attention layer: the decode
        step's (row < 0) or row `row` of the most recent prompt chunk."""
        a = self.model.arch
        n = a["nh"] * a["hd"]
        q = np.zeros(n, np.float32)
        g = np.zeros(n, np.float32)
        o = np.zeros(n, np.float32)
        p = C.c_int32(0)
        _check(lib().ornith_hip_session_get_attn(self.h, row, _f32(q), _f32(g), _f32(o), C.byref(p)),
               "ornith_hip_session_get_attn")
        return q, g, o, int(p.value)

    def free(self):
        if self.h:
            lib().ornith_hip_session_free(self.h)
            self.h = None


def row_bytes(t: int, n: int) -> int:
    be, bb = _BLOCK[t]
    if n % be:
        raise ValueError(f"{n} elements is not a whole number of type-{t} blocks")
    return n // be * bb
