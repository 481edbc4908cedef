"""oracle/calibrate.py - speed of the oracle port against the reference's own
build (oracle/_ref/libornith_ref.so) on the tiny C1 config, in this container.

Both run the same work the way `ornith bench` times it
(src/ornith_bench.c:108-146): load the C1 GGUF, a 32-token prompt in the
default chunked prompt mode, then 64 greedy decode steps, R repetitions,
best and mean prefill and decode tok/s. The reference sizes its thread pool
as min(nproc, 64) (src/ornith_rforward.c:811-812); the port is given the
same count. Q8 KV cache for both (ORNITH_KV_Q8=1). The ratio port/reference
is the calibration factor for the port's CPU-baseline figures.

usage: python oracle/calibrate.py [reps]"""
import ctypes as C
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tests"))
import clibs  # noqa: E402
from clibs import i32p  # noqa: E402

N_PROMPT, N_GEN = 32, 64


def port_run(L, path, prompt, threads):
    m = C.c_void_p()
    assert L.orc_model_load(path.encode(), C.byref(m)) == 0
    L.orc_model_set_threads(m, threads)
    s = L.orc_session_new(m, N_PROMPT + N_GEN + 8, 1)
    t0 = time.perf_counter()
    assert L.orc_session_eval(s, i32p(prompt), N_PROMPT, 0) == 0
    t1 = time.perf_counter()
    out = np.zeros(N_GEN, np.int32)
    n = C.c_int(0)
    assert L.orc_session_generate(s, N_GEN, i32p(out), C.byref(n), None) == 0
    t2 = time.perf_counter()
    L.orc_session_free(s)
    L.orc_model_free(m)
    return N_PROMPT / (t1 - t0), N_GEN / (t2 - t1), out


def ref_run(R, path, prompt):
    m = C.c_void_p()
    assert R.rmodel_load(path.encode(), C.byref(m)) == 0
    s = R.rmodel_session_new(m, N_PROMPT + N_GEN + 8)
    t0 = time.perf_counter()
    assert R.rmodel_session_eval(s, i32p(prompt), N_PROMPT) == 0
    t1 = time.perf_counter()
    toks = []
    cb = clibs.TOKEN_CB(lambda tok, piece, ud: toks.append(tok))
    fin = C.c_int(0)
    assert R.rmodel_session_generate(s, N_GEN, None, 0, None, cb, None, C.byref(fin)) == 0
    t2 = time.perf_counter()
    R.rmodel_session_free(s)
    R.rmodel_free(m)
    return N_PROMPT / (t1 - t0), N_GEN / (t2 - t1), np.array(toks, np.int32)


def main() -> int:
    reps = int(sys.argv[1]) if len(sys.argv) > 1 else 5
    os.environ["ORNITH_KV_Q8"] = "1"
    os.environ.pop("ORNITH_PREFILL_SERIAL", None)
    L, R = clibs.oracle(), clibs.ref()
    threads = min(os.cpu_count() or 1, 64)
    prompt = clibs.ids(0, "prompt", N_PROMPT, clibs.C1["vocab"])
    with tempfile.TemporaryDirectory() as td:
        path = str(Path(td) / "c1.gguf")
        clibs.write_c1_gguf(path)
        res = {"port": [], "reference": []}
        for _ in range(reps):
            p = port_run(L, path, prompt, threads)
            r = ref_run(R, path, prompt)
            assert np.array_equal(p[2], r[2]), "port and reference tokens differ"
            res["port"].append(p[:2])
            res["reference"].append(r[:2])
    print(f"C1, {N_PROMPT}-token prompt (chunked) + {N_GEN} greedy steps, {threads} threads, {reps} reps, "
          f"{os.cpu_count()} CPUs")
    for k, v in res.items():
        pf, dec = np.array([x[0] for x in v]), np.array([x[1] for x in v])
        print(f"  {k:9s} prefill tok/s mean {pf.mean():9.1f} best {pf.max():9.1f} | "
              f"decode tok/s mean {dec.mean():8.1f} best {dec.max():8.1f}")
    dp = np.array([x[1] for x in res["port"]]).mean() / np.array([x[1] for x in res["reference"]]).mean()
    pp = np.array([x[0] for x in res["port"]]).mean() / np.array([x[0] for x in res["reference"]]).mean()
    print(f"  port / reference: decode {dp:.3f}, prefill {pp:.3f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
