"""ctypes view of the test-only diagnostics library (tests/native/cbx_debug.h,
built by `make -C tests/native`): the sampler's device exponential, Philox
uniforms and exact running sums on caller-given inputs."""
import ctypes
import os

import pkg

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "native", "_build", "libcbx_debug.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise FileNotFoundError(f"{LIB} is not built; run `make -C tests/native`")
        pkg.load().load_library()  # torch's HIP runtime first, as for the product library
        L = ctypes.CDLL(LIB)
        vp, i32, i64, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
        L.cbx_debug_expf.argtypes = [i32, vp, vp, i64, vp]
        L.cbx_debug_philox.argtypes = [i32, u64, vp, u64, i32, vp, vp]
        L.cbx_debug_runsum.argtypes = [i32, vp, vp, vp, vp, i32, vp, vp, vp]
        L.cbx_debug_chainsum.argtypes = [i32, vp, vp, vp, i32, vp, vp, vp]
        _lib = L
    return _lib


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ok(rc, name):
    if rc != 0:
        raise RuntimeError(f"{name} returned {rc}")


def expf(x, out, device=0):
    _ok(lib().cbx_debug_expf(device, x.data_ptr(), out.data_ptr(), x.numel(), _stream()), "expf")


def runsum(terms, offsets, thr, desc, sums, hits, device=0):
    _ok(lib().cbx_debug_runsum(device, terms.data_ptr(), offsets.data_ptr(),
                               None if thr is None else thr.data_ptr(),
                               None if desc is None else desc.data_ptr(), offsets.numel() - 1,
                               sums.data_ptr(), hits.data_ptr(), _stream()), "runsum")


def chainsum(terms, offsets, thr, sums, hits, device=0):
    _ok(lib().cbx_debug_chainsum(device, terms.data_ptr(), offsets.data_ptr(),
                                 None if thr is None else thr.data_ptr(), offsets.numel() - 1,
                                 sums.data_ptr(), hits.data_ptr(), _stream()), "chainsum")


def philox(seed, stream_ids, step, n, out, device=0):
    _ok(lib().cbx_debug_philox(device, seed, None if stream_ids is None else stream_ids.data_ptr(),
                               step, n, out.data_ptr(), _stream()), "philox")
