"""The Lean glue (pufferlean_amd/glue/pufferhip_glue.c): it compiles against the library's header and
a stand-in of lean.h with every warning as an error, defines exactly the @[extern] names the reference
binds to GPU code (tests/golden/lean_gpu_externs.txt, written from Puffer/Float/CUDA.lean and
BLAS.lean by make_lean_externs.py), and, without a device, answers through the Lean ABI: IO errors
carry the library's message, the parts the library does not provide answer as documented, and every
owned argument is released."""
import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STUB = os.path.join(ROOT, "tests", "lean_stub")
GLUE = os.path.join(ROOT, "pufferlean_amd", "glue", "pufferhip_glue.c")
NAMES = os.path.join(ROOT, "tests", "golden", "lean_gpu_externs.txt")


@pytest.fixture(scope="module")
def glue_so():
    subprocess.run(["make", "-s", "-C", STUB], check=True)
    return os.path.join(STUB, "libglue_stub.so")


def test_glue_compiles_warning_free(tmp_path):
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter",
                        "-fsyntax-only", f"-I{STUB}", f"-I{os.path.join(ROOT, 'include')}", GLUE],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_glue_defines_every_gpu_extern(glue_so):
    want = set(open(NAMES).read().split())
    assert len(want) == 50
    out = subprocess.run(["nm", "-D", "--defined-only", glue_so], capture_output=True, text=True, check=True)
    defined = {line.split()[-1] for line in out.stdout.splitlines() if line.split()[-2:-1] == ["T"]}
    lean = {n for n in defined if n.startswith("lean_") and not n.startswith("lean_alloc")
            and n in want | {n for n in defined if n.startswith(("lean_cuda_", "lean_ffi_"))}}
    assert want <= defined, sorted(want - defined)
    # nothing else: the CPU entries (OpenBLAS path, C twins) stay in pufferblas.c / pufferffi.c
    assert lean == want, sorted(lean - want)


def _lib(glue_so):
    h = C.CDLL(glue_so)
    vp = C.c_void_p
    h.stub_array.restype = vp
    h.stub_array.argtypes = [C.POINTER(C.c_double), C.c_size_t]
    h.stub_io_ok.argtypes = [vp]
    h.stub_io_value.restype = vp
    h.stub_io_value.argtypes = [vp]
    h.stub_io_error.restype = C.c_char_p
    h.stub_io_error.argtypes = [vp]
    h.stub_unbox.restype = C.c_size_t
    h.stub_unbox.argtypes = [vp]
    h.stub_live.restype = C.c_long
    h.stub_release.argtypes = [vp]
    return h


def _arr(h, vals):
    a = (C.c_double * max(len(vals), 1))(*vals)
    return h.stub_array(a, len(vals))


def test_glue_answers_without_device(glue_so):
    import torch
    if torch.cuda.is_available():
        pytest.skip("checks the no-device answers")
    h = _lib(glue_so)
    vp, sz = C.c_void_p, C.c_size_t
    live0 = h.stub_live()
    # not provided: IO error naming the entry, owned arrays released
    f = h.lean_cuda_plugin_rollout
    f.restype = vp
    f.argtypes = [sz, sz, vp, sz, sz, sz, sz, sz, C.c_uint8, C.c_uint64, vp]
    r = f(0, 0, _arr(h, [1.0, 2.0]), 1, 2, 4, 2, 8, 0, 7, None)
    assert h.stub_io_ok(r) == 0 and b"not provided" in h.stub_io_error(r)
    h.stub_release(r)
    # rollout chain never ready; the LSTM hint and the roll-buffer setting are no-ops
    f = h.lean_cuda_mg_chain_ready
    f.restype = vp
    f.argtypes = [sz, sz, sz, vp]
    r = f(4, 8, 16, None)
    assert h.stub_io_ok(r) == 1 and h.stub_unbox(h.stub_io_value(r)) == 0
    h.stub_release(r)
    for name, args in (("lean_cuda_lstm_reuse_inputs", [C.c_uint8]), ("lean_cuda_set_roll_buffers", [sz, C.c_uint8])):
        f = getattr(h, name)
        f.restype = vp
        f.argtypes = args + [vp]
        r = f(*([1] * len(args)), None)
        assert h.stub_io_ok(r) == 1
        h.stub_release(r)
    # no device: the availability probe says so, and IO entries report the library's error
    f = h.lean_ffi_cuda_available
    f.restype = C.c_uint8
    f.argtypes = [vp]
    assert f(h.stub_array(None, 0)) == 0
    f = h.lean_cuda_policy_load
    f.restype = vp
    f.argtypes = [vp, sz, vp]
    r = f(_arr(h, [0.5] * 8), 4, None)
    assert h.stub_io_ok(r) == 0 and len(h.stub_io_error(r)) > 0
    h.stub_release(r)
    f = h.lean_cuda_mingru_muon_resident
    f.restype = vp
    f.argtypes = [sz, vp, sz, sz, sz, sz] + [C.c_double] * 6 + [vp]
    r = f(0, _arr(h, []), 8, 4, 1, 3, 0.01, 0.0, 0.95, 1e-7, 0.5, 1.0, None)
    assert h.stub_io_ok(r) == 0 and b"no policy handle" in h.stub_io_error(r)
    h.stub_release(r)
    # every owned argument and every result was released
    assert h.stub_live() == live0
