"""The C++ drop-in (include/cbx_sampler.hpp) in the reference's own decode-loop
shape: a C++ program calls cbx::sample_next_token_ex(logits, generated,
params, std::mt19937&) step by step and compares every token with the oracle
driven by libstdc++'s std::discrete_distribution on the same engine seed."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "native", "_build", "shim_engine_loop")


def test_cpp_shim_engine_loop():
    assert os.path.exists(BIN), "build first: make -C tests/native (or __graft_entry__.build())"
    print("[gpu-case] C++ shim engine loop, 300 steps, seed 42", flush=True)
    r = subprocess.run([BIN, "300", "42"], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.startswith("OK 300"), r.stdout
