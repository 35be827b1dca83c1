"""The allocation-free advantage normalisation against the allocating entry, through the C ABI."""
import ctypes as C

import numpy as np
import pytest
import torch

from pufferlean_amd import _lib
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu

MAX_N = 4096 * 4096


def _fns():
    h = _lib.lib()
    ref = h.ph_adv_normalize
    na = h.ph_adv_normalize_noalloc
    na.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p]
    na.restype = C.c_int
    return ref, na


def _run(fn, dtype, x, with_stats):
    out = torch.empty_like(x)
    stats = torch.zeros(2, dtype=x.dtype, device=x.device) if with_stats else None
    code = _lib.PH_F64 if x.dtype == torch.float64 else _lib.PH_F32
    st = fn(code, x.data_ptr(), x.numel(), out.data_ptr(), stats.data_ptr() if with_stats else None, None)
    _lib.check(st, fn.__name__)
    torch.cuda.synchronize()
    return out, stats


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_matches_allocating_entry(gpu, dtype):
    ref, na = _fns()
    # two calls in a row, the second smaller: the second must not see the first's partials
    for n, seed in ((1_000_003, 71), (262_144, 72), (4097, 73)):
        x = torch.from_numpy(rng.normal(seed, n, 0.3, 1.7)).to(dtype).to(gpu)
        for with_stats in (True, False):
            o_ref, s_ref = _run(ref, dtype, x, with_stats)
            o_na, s_na = _run(na, dtype, x, with_stats)
            assert torch.equal(o_na, o_ref), (n, with_stats)
            if with_stats:
                assert torch.equal(s_na, s_ref), (n, s_na, s_ref)
        xs = x.double().cpu().numpy()
        on = o_na.double().cpu().numpy()
        assert abs(on.mean()) < (1e-5 if dtype == torch.float32 else 1e-12)
        assert abs(on.std() - 1.0) < (1e-4 if dtype == torch.float32 else 1e-7)
        assert xs.size == n


def test_noalloc_rejects_oversize(gpu):
    _, na = _fns()
    x = torch.zeros(8, device=gpu)
    st = na(_lib.PH_F32, x.data_ptr(), MAX_N + 1, x.data_ptr(), None, None)
    assert st == _lib.PH_ERR_ARG
    assert b"exceeds" in _lib.lib().ph_last_error()
    # the largest allowed size runs
    big = torch.from_numpy(rng.normal(74, MAX_N)).float().to(gpu)
    o_ref, _ = _run(_fns()[0], torch.float32, big, False)
    o_na, _ = _run(na, torch.float32, big, False)
    assert torch.equal(o_na, o_ref)
