"""The C-ABI library loads without a GPU and exports every symbol include/*.h declares.

No compute calls here: only loading, symbol lookup and the calls that need no device.
"""
import re
from pathlib import Path

import numpy as np
import pytest

from pufferlean_amd import _lib as L

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_ \*]*?\b(ph_[A-Za-z0-9_]+)\s*\(", re.M)


def declared_symbols():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(DECL.findall(text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "ph_vtrace" in names and "ph_gemm" in names
    assert len(names) >= 10


@pytest.mark.parametrize("name", declared_symbols())
def test_library_exports_symbol(name):
    lib = L.lib()
    assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_signatures_cover_exports():
    for name in L.SIGNATURES:
        assert name in declared_symbols(), f"{name} bound in _lib but not declared"


def test_link_time_contract_symbols():
    """The externs the reference's pufferblas.c resolves at link time (pufferblas.c:38-50)."""
    import ctypes as C
    lib = L.lib()
    assert hasattr(lib, "cuda_lstm_ppo_grad_batch")
    assert C.c_int.in_dll(lib, "g_mgLossOn").value in (0, 1)
    losses = (C.c_double * 7).in_dll(lib, "g_mgLoss")
    assert len(list(losses)) == 7


def test_loss_channel_without_device():
    import ctypes as C
    lib = L.lib()
    L.call("ph_cuda_mg_loss_enable", 1)
    assert C.c_int.in_dll(lib, "g_mgLossOn").value == 1
    L.call("ph_cuda_mg_loss_enable", 0)
    assert C.c_int.in_dll(lib, "g_mgLossOn").value == 0
    out = (C.c_double * 7)()
    L.call("ph_cuda_mg_read_losses", out)


def test_host_entries_reject_bad_arguments_without_device():
    # argument checks run before any device work
    import ctypes as C
    lib = L.lib()
    hs = np.array([1.0, 1.0])  # two heads summing to 2, not A = 3
    assert lib.ph_cuda_mingru_ppo_grad(None, 0, None, 0, None, 0, 1, 1, 8, 8, 1, 3, 2, hs.ctypes.data_as(L.dptr),
                                       2, 0.5, 0.01, 0.2, 0.0, None, 0, None, 0, None, None) == L.PH_ERR_ARG
    assert b"head sizes sum to 2" in lib.ph_last_error()
    assert lib.ph_cuda_mingru_ppo_grad(None, 0, None, 0, None, 0, 1, 1, 8, 8, 1, 3, 2, None, 0,
                                       0.5, 0.01, 0.2, 0.0, None, 0, None, 0, None, None) == L.PH_ERR_ARG
    assert lib.ph_cuda_policy_download(0, 4, None) == L.PH_ERR_ARG


def test_wide_update_rejects_bad_arguments_without_device():
    # the handle is never dereferenced: every check below returns before any device work
    import numpy as np
    NT, D, H = 4, 3, 5
    z = np.zeros(64)
    p = z.ctypes.data_as(L.dptr)
    hs = np.array([2.0, 3.0]).ctypes.data_as(L.dptr)
    bad_perm = np.array([0.0, 1.0, 4.0, 2.0]).ctypes.data_as(L.dptr)  # 4 is outside [0, NT)

    def call(mode, O, W, perm=p, hsp=hs, hsN=2):
        return L.lib().ph_cuda_train_update_wide_resident(1, p, p, p, p, p, None, 0, perm, hsp, hsN, NT, D, H, O, W,
                                                          mode, 1, 1, 0.02, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0.0,
                                                          0.0, 0, p)
    lib = L.lib()
    assert call(3, 6, 2) == L.PH_ERR_ARG and b"mode" in lib.ph_last_error()
    assert call(1, 7, 2) == L.PH_ERR_ARG and b"sum" in lib.ph_last_error()   # sizes sum to 5: O must be 6
    assert call(1, 6, 2, hsN=1) == L.PH_ERR_ARG
    assert call(2, 6, 2) == L.PH_ERR_ARG and b"2d+1" in lib.ph_last_error()  # 2 dims: O must be 5
    assert call(1, 6, 2, perm=bad_perm) == L.PH_ERR_ARG and b"shuffle index" in lib.ph_last_error()


def test_no_device_calls_fail_cleanly():
    lib = L.lib()
    assert lib.ph_version() == 100
    n = lib.ph_device_count()
    assert n >= 0
