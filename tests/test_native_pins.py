"""Pins of the two numeric building blocks the GPU path restates:

* the glibc expf algorithm (chatterbox.cpp_amd/csrc/cbx_expf.h), against the
  host libm expf that the reference's std::exp(float) calls (main.cpp:759,
  :789), exhaustively over every binary32 input the sampler can produce;
* Philox4x32-10, oracle and device formulations, against rocRAND's
  independent implementation and the published Random123 check vectors.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
NATIVE = os.path.join(HERE, "native")


def _cpu_has_fma_avx2():
    flags = open("/proc/cpuinfo").read()
    return " fma " in flags and " avx2 " in flags


@pytest.fixture(scope="module")
def expf_bin(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("native") / "expf_exhaustive")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", out,
                    os.path.join(NATIVE, "expf_exhaustive.cpp"), "-lpthread"], check=True)
    return out


@pytest.mark.skipif(not _cpu_has_fma_avx2(),
                    reason="glibc selects its FMA expf only on FMA+AVX2 hosts")
@pytest.mark.parametrize("lo,hi", [
    (0x80000000, 0xC2D00001),   # every x in [-104, -0]: all arguments s - max <= 0
    (0xC2D00001, 0xC4000001),   # (-512, -104): the underflow to 0
    (0x00000000, 0x42B20000),   # [0, 89): positive side, special-case cut-offs
    (0x7F800000, 0x7F800001),   # +inf
    (0xFF800000, 0xFF800001),   # -inf
])
def test_expf_restatement_exhaustive(expf_bin, lo, hi):
    r = subprocess.run([expf_bin, hex(lo), hex(hi), str(os.cpu_count() or 4)],
                       check=True, capture_output=True, text=True)
    bad, count = (int(v) for v in r.stdout.split()[:2])
    assert count == hi - lo
    assert bad == 0, r.stdout


def test_exp2_table_from_mathematics():
    # tab[i] = bits(RN64(2^(i/32))) - (i << 47), evaluated at 200 bits.
    mpmath = pytest.importorskip("mpmath")
    import re
    import struct
    src = open(os.path.join(ROOT, "chatterbox.cpp_amd", "csrc", "cbx_expf.h")).read()
    words = [int(w, 16) for w in re.findall(r"0x([0-9a-f]{16})ull", src)]
    assert len(words) == 32
    mpmath.mp.prec = 200
    for i in range(32):
        d = float(mpmath.power(2, mpmath.mpf(i) / 32))
        b = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert words[i] == (b - (i << 47)) & (2**64 - 1), i


@pytest.fixture(scope="module")
def rocrand_bin(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("native") / "rocrand_philox_kat")
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-o", out,
                        os.path.join(NATIVE, "rocrand_philox_kat.cpp")],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("rocRAND headers not usable: " + r.stderr[-300:])
    return out


# Published Random123 known-answer vectors for philox4x32_10 (counter, key,
# result); they must agree with rocRAND as well as with the oracle.
R123_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


def _rocrand(binpath, ctr, key):
    r = subprocess.run([binpath] + [hex(v) for v in list(ctr) + list(key)], check=True,
                       capture_output=True, text=True)
    return [int(w, 16) for w in r.stdout.split()]


def test_philox_oracle_against_rocrand_and_kat(rocrand_bin):
    for ctr, key, want in R123_KAT:
        assert list(O.philox(ctr, key)) == want
        assert _rocrand(rocrand_bin, ctr, key) == want
    rng = np.random.default_rng(23)
    for _ in range(64):
        ctr = [int(v) for v in rng.integers(0, 2**32, 4)]
        key = [int(v) for v in rng.integers(0, 2**32, 2)]
        assert list(O.philox(ctr, key)) == _rocrand(rocrand_bin, ctr, key)


def test_philox_uniform_construction():
    # u = ((x0 >> 5) * 2^26 + (x1 >> 6)) * 2^-53 from counter {step, stream},
    # key seed: check the mapping of (seed, stream, step) to words and bits.
    seed, stream, step = 0x1122334455667788, 0x99AABBCCDDEEFF00, 0x0123456789ABCDEF
    o = O.philox([step & 0xFFFFFFFF, step >> 32, stream & 0xFFFFFFFF, stream >> 32],
                 [seed & 0xFFFFFFFF, seed >> 32])
    want = ((int(o[0]) >> 5) * 2**26 + (int(o[1]) >> 6)) / 2.0**53
    assert O.philox_uniform(seed, stream, step) == want
    us = [O.philox_uniform(7, s, t) for s in range(50) for t in range(50)]
    assert min(us) >= 0.0 and max(us) < 1.0
    assert abs(np.mean(us) - 0.5) < 0.02


def test_stdsort_replay_matches_libstdcxx(tmp_path):
    """The one-lane restatement of libstdc++'s std::sort (csrc/cbx_stdsort.h)
    orders (id, score) pairs exactly as std::sort does with the reference's
    comparator (main.cpp:752-755): ties, sorted runs and McIlroy adversary
    inputs that reach the heap-sort fallback."""
    out = str(tmp_path / "stdsort_replay")
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", out,
                    os.path.join(NATIVE, "stdsort_replay.cpp")], check=True)
    res = subprocess.run([out], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    cases, bad, heaped = (int(v) for v in res.stdout.split()[-3:])
    assert cases > 5000 and bad == 0
    assert heaped > 0  # the depth-limit fallback was exercised
