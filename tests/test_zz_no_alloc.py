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


def test_noalloc_under_graph_capture(gpu):
    """Captured in a HIP graph, first as the process's first call of the entry (its per-device address
    lookup then happens inside the capture; this test is the file's first), then again after eager
    calls: every replay, with eager work and synchronisations between replays, equals the allocating
    entry's eager result bit for bit."""
    ref, na = _fns()
    n = 300_001
    x = torch.from_numpy(rng.normal(75, n, 0.3, 1.7)).float().to(gpu)
    o_ref, s_ref = _run(ref, torch.float32, x, True)
    for attempt in range(2):
        out = torch.empty_like(x)
        stats = torch.zeros(2, device=gpu)
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                _lib.check(na(_lib.PH_F32, x.data_ptr(), n, out.data_ptr(), stats.data_ptr(), s.cuda_stream),
                           "ph_adv_normalize_noalloc")
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for k in range(3):
            out.zero_()
            stats.zero_()
            graph.replay()
            torch.cuda.synchronize()
            _ = (torch.ones(1000, device=gpu) * 2).sum().item()
            assert torch.equal(out, o_ref), (attempt, k)
            assert torch.equal(stats, s_ref), (attempt, k)
        if attempt == 0:
            _run(na, torch.float32, x, True)  # eager calls between the two captures
            _run(na, torch.float32, x[:4097], False)


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
