"""CPU: the C-ABI library loads and exports every entry point of
include/ornith_hip.h; without a GPU, initialisation fails with a status and a
message instead of crashing (no compute is attempted here)."""
import ctypes as C
import re

import pytest

import ornithology_amd as oa


def declared_functions():
    text = oa.HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ornith_hip_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("ornith_hip_init", "ornith_hip_quantize_q8K", "ornith_hip_matvec", "ornith_hip_dequant",
                 "ornith_hip_moe_route", "ornith_hip_model_load", "ornith_hip_session_eval",
                 "ornith_hip_session_generate"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = oa.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    # and the Python mirror binds exactly the declared set
    assert set(oa._SIGS) == set(declared_functions())


def test_init_without_gpu_reports_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    L = oa.lib()
    h = C.c_void_p()
    st = L.ornith_hip_init(0, C.byref(h))
    assert st != 0 and not h
    assert L.ornith_hip_last_error()


def test_header_compiles_as_c11_caller(tmp_path):
    """The C caller of the boundary (tests/c_caller/ornith_generate.c)
    compiles as strict C11 against include/ornith_hip.h with every warning an
    error, and links against the in-tree library."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    root = oa.HEADER.parent.parent
    src = root / "tests" / "c_caller" / "ornith_generate.c"
    out = tmp_path / "ornith_generate"
    lib = root / "ornithology_amd"
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", "-O2",
                        f"-I{root / 'include'}", str(src), "-o", str(out), f"-L{lib}", "-lornith_hip",
                        "-Wl,-rpath-link,/opt/rocm/lib"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
