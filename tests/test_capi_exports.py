"""The C ABI library loads and exports exactly what include/*.h declares.

CPU-only: no call here reaches the GPU (argument checks fail before any HIP
runtime call)."""
import ctypes
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(ROOT, "chatterbox.cpp_amd", "lib", "libcbx_sampler.so")


def declared_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(inc, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(cbx_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "chatterbox.cpp_amd")], check=True)
    return ctypes.CDLL(LIB)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("cbx_sampler_create", "cbx_sampler_destroy", "cbx_sample_row",
                 "cbx_sample_row_ex", "cbx_sample_batch", "cbx_last_error", "cbx_max_vocab"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], check=True, capture_output=True,
                         text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared_functions() - exported
    assert not missing, missing
    for name in declared_functions():
        getattr(lib, name)


def test_argument_checks_without_gpu(lib):
    lib.cbx_last_error.restype = ctypes.c_char_p
    lib.cbx_sampler_create.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32]
    assert lib.cbx_sampler_create(None, 0, 6563, 1000) == -1
    assert b"NULL" in lib.cbx_last_error()
    h = ctypes.c_void_p()
    assert lib.cbx_sampler_create(ctypes.byref(h), 0, 0, 1000) == -1
    assert lib.cbx_sampler_create(ctypes.byref(h), 0, 1 << 20, 1000) == -1
    lib.cbx_sample_batch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    assert lib.cbx_sample_batch(None, None, None) == -1
    lib.cbx_max_vocab.restype = ctypes.c_int32
    assert lib.cbx_max_vocab() == 32768


def test_python_binding_refuses_missing_library(tmp_path):
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "cbx_binding_probe", os.path.join(ROOT, "chatterbox.cpp_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    with pytest.raises(FileNotFoundError):
        mod.load_library(str(tmp_path / "absent.so"))


def test_diagnostics_live_in_the_test_library():
    """The device diagnostics (tests/native/cbx_debug.h) are exported by the
    test-only libcbx_debug.so and not by the product library."""
    dbg = os.path.join(HERE, "native", "_build", "libcbx_debug.so")
    if not os.path.exists(dbg):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(HERE, "native", "cbx_debug.h")).read(),
                  flags=re.S)
    names = set(re.findall(r"\b(cbx_debug_\w+)\s*\(", text))
    assert len(names) == 4
    out = subprocess.run(["nm", "-D", "--defined-only", dbg], check=True, capture_output=True,
                         text=True).stdout
    assert names <= {line.split()[-1] for line in out.splitlines() if " T " in line}
    prod = subprocess.run(["nm", "-D", "--defined-only", LIB], check=True, capture_output=True,
                          text=True).stdout
    assert "cbx_debug_" not in prod
