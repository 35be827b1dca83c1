"""ctypes binding of libpufferhip.so (the C ABI declared in include/pufferhip.h).

The library is built in-tree by ``python -m pufferlean_amd.build``. Loading fails loudly when it
is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpufferhip.so"

PH_OK, PH_ERR_ARG, PH_ERR_HIP, PH_ERR_NOMEM, PH_ERR_UNSUPPORTED = 0, -1, -2, -3, -4
PH_F32, PH_F64, PH_BF16, PH_I32 = 0, 1, 2, 3
PH_MATH_BF16, PH_MATH_F32, PH_MATH_BF16X3 = 0, 1, 2
PH_EPI_NONE, PH_EPI_BIAS, PH_EPI_BIAS_RELU, PH_EPI_RELU_MASK, PH_EPI_AXPBY = 0, 1, 2, 3, 4

vp, sz, dbl, flt, i32, i64, u8, u64 = (C.c_void_p, C.c_size_t, C.c_double, C.c_float, C.c_int,
                                       C.c_long, C.c_uint8, C.c_uint64)
dptr = C.POINTER(C.c_double)
u32 = C.c_uint32
fptr = C.POINTER(C.c_float)
szptr = C.POINTER(C.c_size_t)


class MinGRUDims(C.Structure):
    _fields_ = [("B", C.c_int), ("T", C.c_int), ("D", C.c_int), ("H", C.c_int), ("L", C.c_int),
                ("A", C.c_int), ("precision", C.c_int)]


class PPOCoefs(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("gamma", "lam", "rho_clip", "c_clip", "clip_eps", "vf_coef",
                                         "ent_coef", "vf_clip")]


class MuonCoefs(C.Structure):
    _fields_ = [("lr", C.c_float), ("wd", C.c_float), ("mu", C.c_float), ("eps", C.c_float),
                ("max_grad_norm", C.c_float), ("gscale", C.c_float), ("nsteps", C.c_int),
                ("math", C.c_int), ("coeffs", C.c_void_p)]

class MLPDims(C.Structure):
    _fields_ = [("N", C.c_int), ("D", C.c_int), ("H", C.c_int), ("L", C.c_int), ("A", C.c_int)]


class ReplayCols(C.Structure):
    _fields_ = [("dtype", C.c_int), ("time_major", C.c_int), ("N", C.c_size_t), ("T", C.c_size_t),
                ("K", C.c_size_t), ("adv", C.c_void_p), ("value", C.c_void_p), ("ratio", C.c_void_p),
                ("act", C.c_void_p), ("logp", C.c_void_p), ("term", C.c_void_p)]


# name -> argtypes (all return int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "ph_last_error": [],
    "ph_version": [],
    "ph_device_count": [],
    "ph_synchronize": [vp],
    "ph_release_scratch": [],
    "ph_scratch_retired": [szptr, szptr],
    "ph_ns_status": [vp],
    "ph_ns_set_spin_limit": [u32],
    "ph_ns_set_queues": [i32],
    "ph_vtrace": [i32, vp, vp, vp, vp, vp, sz, sz, i32, i32, i32, i32, dbl, dbl, dbl, dbl, vp, vp, vp],
    "ph_adv_normalize": [i32, vp, sz, vp, vp, vp],
    "ph_adv_normalize_noalloc": [i32, vp, sz, vp, vp, vp],
    "ph_colsum": [vp, sz, sz, sz, vp, flt, i32, vp],
    "ph_convert": [i32, vp, i32, vp, sz, vp],
    "ph_ppo_grad": [vp, sz, vp, sz, vp, vp, vp, vp, vp, sz, sz, flt, flt, flt, flt, i32, vp, sz,
                    vp, sz, vp, vp, vp, vp],
    "ph_gemm": [i32, i32, i32, i32, i32, i32, vp, i64, i32, vp, i64, i32, vp, i64, i32, i32, vp,
                vp, i64, flt, flt, vp, i64, i32, i32, vp],
    "ph_muon_mat_f64": [i32, i32, vp, vp, vp, vp, vp, dbl, dbl, dbl, dbl, dbl, vp, i32, vp],
    "ph_stepvec_f64": [sz, vp, vp, vp, vp, vp, dbl, dbl, dbl, dbl, vp],
    "ph_newton_schulz": [vp, i32, i32, vp, i32, flt, i32, vp],
    "ph_newton_schulz_batch": [vp, vp, vp, i32, vp, i32, flt, i32, vp],
    "ph_muon_mat": [vp, vp, vp, i32, i32, flt, flt, flt, flt, flt, vp, i32, i32, vp],
    "ph_stepvec": [vp, vp, vp, sz, flt, flt, flt, flt, vp],
    "ph_gclip": [vp, sz, flt, flt, vp],
    "ph_mingru_param_count": [vp],
    "ph_mingru_ppo_grad": [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "ph_mingru_ppo_grad_md": [vp, vp, vp, sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "ph_mingru_muon": [vp, vp, vp, vp, vp, vp],
    "ph_mingru_step": [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "ph_mlp_param_count": [vp],
    "ph_mlp_forward": [vp, i32, vp, vp, vp, vp],
    "ph_mlp_ppo_grad": [vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "ph_mlp_update": [vp, i32, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "ph_seg_l1": [vp, vp, vp],
    "ph_prio_sample": [vp, sz, sz, dbl, dbl, u64, vp, vp, vp],
    "ph_mb_gather": [vp, vp, vp, sz, vp, vp, vp],
    "ph_mb_iterate": [vp, vp, sz, vp, vp, vp],
    "ph_sample_actions": [i32, vp, sz, sz, sz, i32, u64, vp, vp, vp, vp],
    "ph_ppo_grad_md": [vp, sz, vp, vp, vp, vp, vp, sz, vp, sz, flt, flt, flt, flt, vp, sz, vp, vp, vp, vp],
    "ph_ppo_grad_cont": [vp, sz, vp, vp, vp, vp, vp, sz, sz, flt, flt, flt, flt, flt, flt, vp, sz, vp, vp, vp, vp],
    "ph_sample_actions_md": [i32, vp, sz, sz, vp, sz, u64, vp, vp],
    "ph_sample_actions_cont": [i32, vp, sz, sz, sz, u64, dbl, dbl, vp, vp],
    "ph_mingru_rollout_step": [vp, vp, vp, vp, vp, vp],
    # host-buffer layer (reference Lean @[extern] GPU symbols)
    "ph_cuda_vtrace": [dptr, dptr, dptr, dptr, sz, sz, dbl, dbl, dbl, dbl, dptr],
    "ph_cuda_vtrace_mingru": [dptr, dptr, dptr, dptr, dptr, sz, sz, dbl, dbl, dbl, dbl, dptr],
    "ph_cuda_adv_normalize": [dptr, sz, dptr],
    "ph_cuda_mlp_ppo_grad": [dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, dbl, dbl, dbl, u8, dptr],
    "ph_cuda_train_step": [dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, dbl, dbl, dbl, dbl, dbl, dbl,
                           dbl, u8, dptr],
    "ph_cuda_train_update": [dptr, dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, sz, sz, dbl, dbl, dbl,
                             dbl, dbl, dbl, dbl, u8, dptr],
    "ph_cuda_train_update_resident": [sz, dptr, dptr, dptr, dptr, dptr, dptr, sz, dptr, sz, sz, sz, sz, sz,
                                      sz, dbl, dbl, dbl, dbl, dbl, dbl, dbl, dbl, dbl, u8, dptr],
    "ph_ckpt_bytes": [sz],
    "ph_ckpt_encode": [dptr, sz, vp],
    "ph_ckpt_decode": [vp, sz, dptr, sz, szptr],
    "ph_cuda_policy_save_ckpt": [sz, sz, vp],
    "ph_cuda_policy_load_ckpt": [vp, sz, sz, szptr],
    "ph_cuda_train_update_wide_resident": [sz, dptr, dptr, dptr, dptr, dptr, dptr, sz, dptr, dptr, sz, sz, sz,
                                           sz, sz, sz, u32, sz, sz, dbl, dbl, dbl, dbl, dbl, dbl, dbl, dbl, dbl,
                                           u8, dptr],
    "ph_cuda_muon_stepmat": [dptr, dptr, dptr, sz, sz, dbl, dbl, dbl, dbl, dptr],
    "ph_cuda_muon_step_mlp_resident": [sz, dptr, sz, sz, sz, dbl, dbl, dbl, dbl, dbl, dptr],
    "ph_cuda_policy_load": [dptr, sz, szptr],
    "ph_cuda_policy_download": [sz, sz, dptr],
    "ph_cuda_policy_free": [sz],
    "ph_cuda_mg_loss_enable": [u8],
    "ph_cuda_mg_read_losses": [dptr],
    "ph_ffi_dense_forward_gpu": [dptr, dptr, dptr, sz, sz, sz, dptr],
    "ph_ffi_dense_forward_bf16": [dptr, dptr, dptr, sz, sz, sz, dptr],
    "ph_ffi_mlp_forward_batch_bf16": [dptr, dptr, sz, sz, sz, sz, dptr],
    "ph_ffi_bench_bf16_resident": [sz, sz, sz, sz],
    "ph_ffi_cuda_available": [],
    "ph_ffi_mlp_policy_load": [dptr, sz, sz, sz, szptr],
    "ph_ffi_mlp_policy_update": [sz, dptr],
    "ph_ffi_mlp_policy_forward": [sz, dptr, sz, dptr],
    "ph_ffi_mlp_policy_free": [sz],
    "ph_ffi_mlp_policy_outputs": [sz],
    "ph_ffi_bench_mlp2_bf16_resident": [sz, sz, sz, sz, sz],
    "ph_ffi_bench_mlp2_bf16_wres": [sz, sz, sz, sz, sz],
    "ph_cuda_selftest": [sz, dptr],
    "ph_cuda_mingru_ppo_grad": [dptr, sz, dptr, sz, dptr, sz, sz, sz, sz, sz, sz, sz, sz, dptr, sz, dbl, dbl,
                                dbl, dbl, dptr, sz, dptr, sz, dptr, szptr],
    "ph_cuda_mg_resident_grad": [sz, dptr],
    "ph_cuda_mg_prep": [dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz],
    "ph_cuda_mg_cols_ready": [sz, sz, C.POINTER(C.c_uint8)],
    "ph_cuda_mg_obs_traj": [dptr, sz, sz, sz],
    "ph_cuda_mg_vtrace": [sz, sz, dbl, dbl, dbl, dbl, dptr],
    "ph_cuda_mg_vtrace_prio": [sz, sz, dbl, dbl, dbl, dbl, sz, dbl, dbl, u64, C.POINTER(C.c_uint8)],
    "ph_ffi_prio_sample": [dptr, sz, sz, sz, dbl, dbl, u64, dptr, dptr],
    "ph_cuda_sample_actions": [dptr, sz, sz, sz, u64, dptr],
    "ph_cuda_mingru_step": [dptr, dptr, dptr, sz, sz, sz, sz, sz, u8, dptr],
    "ph_cuda_mlp_forward": [dptr, dptr, sz, sz, sz, sz, u8, dptr],
    "ph_cuda_sample_actions_md": [dptr, dptr, sz, sz, sz, u64, dptr],
    "ph_cuda_sample_actions_cont": [dptr, sz, sz, sz, u64, dptr],
    "ph_cuda_mlp_ppo_grad_md": [dptr, dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, dbl, dbl, dbl, u8, dptr],
    "ph_cuda_mlp_ppo_grad_cont": [dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, dbl, dbl, dbl, u8, dptr],
    "ph_ffi_gather_seq_minibatch": [dptr, dptr, dptr, dptr, dptr, dptr, dptr, dptr, sz, sz, sz, sz, dptr],
    "ph_cuda_mingru_muon_resident": [sz, dptr, sz, sz, sz, sz, sz, dbl, dbl, dbl, dbl, dbl, dbl, dptr, szptr],
}
_RESTYPES = {"ph_last_error": C.c_char_p, "ph_mingru_param_count": C.c_long, "ph_mlp_param_count": C.c_long, "ph_ckpt_bytes": C.c_size_t,
             "ph_ffi_bench_bf16_resident": C.c_double, "ph_ffi_bench_mlp2_bf16_resident": C.c_double,
             "ph_ffi_bench_mlp2_bf16_wres": C.c_double, "ph_ffi_mlp_policy_outputs": C.c_size_t, "ph_ffi_cuda_available": C.c_uint8}

_lib = None
_lock = threading.Lock()


class PufferHipError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """The loaded library with argtypes set. Raises if the .so was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise PufferHipError(
                    f"{LIB_PATH} is missing; build it with `python -m pufferlean_amd.build`")
            h = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
            for name, args in SIGNATURES.items():
                fn = getattr(h, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, C.c_int)
            _lib = h
    return _lib


def check(status: int, what: str) -> None:
    if status != PH_OK:
        msg = lib().ph_last_error()
        raise PufferHipError(f"{what} failed with status {status}: {msg.decode() if msg else ''}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
