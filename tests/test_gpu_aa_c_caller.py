"""GPU: the C11 caller of the boundary (tests/c_caller/ornith_generate.c,
built by tests/c_caller/Makefile with gcc -std=c11 -Wall -Wextra -Werror
-pedantic against include/ornith_hip.h and the in-tree libornith_hip.so)
drives load -> arch -> session -> eval -> logits -> generate the way a caller
of the reference's rmodel API does (src/ornith_rforward.h:24-130), on the C1
GGUF. Its greedy tokens equal the reference build's golden tokens in both
prompt modes, and a session one position short of the prompt is refused with
the capacity status.

The program runs as a child process. This file is collected before every
other GPU test, so the child is started before this pytest process has made
any HIP call."""
import os
import subprocess
import sys

import numpy as np
import pytest

import clibs

pytestmark = pytest.mark.gpu
GOLD = np.load(clibs.ROOT / "tests" / "golden" / "c1.npz")
BIN = clibs.ROOT / "tests" / "c_caller" / "ornith_generate"


def gpu_touched() -> bool:
    oa = sys.modules.get("ornithology_amd")
    return oa is not None and getattr(oa, "_lib", None) is not None


@pytest.mark.parametrize("serial,key", [("1", "serial_tokens"), ("0", "chunked_tokens")],
                         ids=["serial", "chunked"])
def test_c_caller_generates_golden_tokens(tmp_path, monkeypatch, serial, key):
    if not BIN.exists():
        pytest.fail(f"{BIN} missing: run `make -C tests/c_caller` (or __graft_entry__.build())")
    if gpu_touched():
        pytest.skip("this process already initialised the GPU; run this file first or on its own")
    path = tmp_path / "c1.gguf"
    clibs.write_c1_gguf(path)
    env = dict(os.environ, ORNITH_PREFILL_SERIAL=serial)
    args = [str(BIN), str(path), "64"] + [str(int(t)) for t in GOLD["prompt"]]
    print(f"[c caller] prompt mode serial={serial}: {BIN.name} with {len(GOLD['prompt'])} prompt tokens",
          flush=True)
    r = subprocess.run(args, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = dict(l.split(" ", 1) for l in r.stdout.strip().splitlines())
    assert lines["arch"].startswith("hidden 512 layers 4 vocab 4096")
    toks = np.array([int(t) for t in lines["tokens"].split()], np.int32)
    assert np.array_equal(toks, GOLD[key])
    assert int(lines["argmax"]) == int(GOLD[key][0])
    assert int(lines["pos"]) == len(GOLD["prompt"]) + 64
