"""Checkpoint byte layout of the trainers (ckptToBytes / bytesToCkpt, Puffer/RL/FFITrain.lean:40-69)
through the C ABI, against an independent restatement with Python's struct module: a little-endian
u64 count, then each double's IEEE bits little-endian. Bit-exact, including signed zero, infinities,
NaN payloads and subnormals; a short file decodes to the whole doubles it holds."""
import ctypes as C
import struct

import numpy as np
import pytest

from pufferlean_amd import _lib as L
from pufferlean_amd import rng


def ref_bytes(w):
    return struct.pack("<Q", len(w)) + b"".join(struct.pack("<Q", struct.unpack("<Q", struct.pack("<d", x))[0])
                                                for x in w)


def encode(w):
    w = np.ascontiguousarray(w, np.float64)
    out = (C.c_uint8 * int(L.lib().ph_ckpt_bytes(len(w))))()
    L.call("ph_ckpt_encode", w.ctypes.data_as(L.dptr), len(w), out)
    return bytes(out)


def decode(b, cap=None):
    buf = (C.c_uint8 * max(len(b), 1)).from_buffer_copy(b if b else b"\0")
    P = C.c_size_t(0)
    L.call("ph_ckpt_decode", buf, len(b), None, 0, C.byref(P))
    w = np.zeros(max(P.value, 1))
    L.call("ph_ckpt_decode", buf, len(b), w.ctypes.data_as(L.dptr), cap if cap is not None else len(w), C.byref(P))
    return w[:P.value]


def special_values():
    nan_payload = struct.unpack("<d", struct.pack("<Q", 0x7FF8DEADBEEF0001))[0]
    return np.array([0.0, -0.0, 1.0, -2.5, np.inf, -np.inf, nan_payload, 5e-324, 2.2250738585072014e-308, 1e308])


def test_encode_matches_struct_restatement():
    w = np.concatenate([special_values(), rng.normal(0xC01, 1000)])
    b = encode(w)
    assert b == ref_bytes(w)
    assert len(b) == 8 * (len(w) + 1)


def test_decode_round_trip_is_bit_exact():
    w = np.concatenate([special_values(), rng.normal(0xC02, 777)])
    back = decode(ref_bytes(w))
    assert back.view(np.uint64).tolist() == w.view(np.uint64).tolist()


@pytest.mark.parametrize("cut", [0, 3, 8, 11, 8 + 8 * 5, 8 + 8 * 5 + 7])
def test_short_file_decodes_the_whole_doubles_present(cut):
    w = rng.normal(0xC03, 10)
    b = ref_bytes(w)[:cut]
    want = max(0, (cut - 8) // 8) if cut >= 8 else 0
    got = decode(b)
    assert len(got) == want
    assert np.array_equal(got, w[:want])


def test_header_larger_or_smaller_than_the_data():
    w = rng.normal(0xC04, 6)
    body = b"".join(struct.pack("<d", x) for x in w)
    assert len(decode(struct.pack("<Q", 100) + body)) == 6   # bounded by the data
    assert np.array_equal(decode(struct.pack("<Q", 4) + body), w[:4])  # the header's count


def test_decode_rejects_a_small_buffer():
    b = ref_bytes(rng.normal(0xC05, 8))
    buf = (C.c_uint8 * len(b)).from_buffer_copy(b)
    w = np.zeros(4)
    P = C.c_size_t(0)
    assert L.lib().ph_ckpt_decode(buf, len(b), w.ctypes.data_as(L.dptr), 4, C.byref(P)) == L.PH_ERR_ARG


@pytest.mark.gpu
def test_policy_handle_save_and_load(gpu):
    P = 5647
    pm = np.concatenate([rng.normal(0xC06, P), rng.normal(0xC07, P)])
    dp = lambda a: np.ascontiguousarray(a, np.float64).ctypes.data_as(L.dptr)
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm), P, C.byref(h))
    out = (C.c_uint8 * int(L.lib().ph_ckpt_bytes(P)))()
    try:
        L.call("ph_cuda_policy_save_ckpt", h.value, P, out)
    finally:
        L.call("ph_cuda_policy_free", h.value)
    assert bytes(out) == ref_bytes(pm[:P])  # the weights only
    h2 = C.c_size_t(0)
    L.call("ph_cuda_policy_load_ckpt", out, len(out), P, C.byref(h2))
    try:
        back = np.zeros(2 * P)
        L.call("ph_cuda_policy_download", h2.value, P, dp(back))
    finally:
        L.call("ph_cuda_policy_free", h2.value)
    assert np.array_equal(back[:P], pm[:P]) and np.all(back[P:] == 0.0)  # momentum restarts at zero
    h3 = C.c_size_t(0)
    assert L.lib().ph_cuda_policy_load_ckpt(out, len(out), P + 1, C.byref(h3)) == L.PH_ERR_ARG
    assert b"this policy needs" in L.lib().ph_last_error()
