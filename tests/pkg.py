"""Import the package directory chatterbox.cpp_amd (a dotted directory name,
so it is loaded by path) as the module `cbx_amd`."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "chatterbox.cpp_amd")


def load():
    if "cbx_amd" in sys.modules:
        return sys.modules["cbx_amd"]
    spec = importlib.util.spec_from_file_location(
        "cbx_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["cbx_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def workloads():
    load()
    import cbx_amd.workloads as w  # noqa: E402
    return w
