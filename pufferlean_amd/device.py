"""Stream-ordered device API over the C ABI, taking torch tensors for device memory.

torch only supplies allocation and the current stream; every computation runs in libpufferhip.so.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L

_DT = {torch.float32: L.PH_F32, torch.float64: L.PH_F64, torch.bfloat16: L.PH_BF16,
       torch.int32: L.PH_I32}


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("device API expects tensors on a GPU")


def vtrace(rew, val, term, rho=None, boot=None, *, variant=0, time_major=True, rho_is_log=False,
           clamp=True, gamma=0.99, lam=0.95, rho_clip=1.0, c_clip=1.0, out_adv=None, out_tgt=None,
           want_targets=True):
    """V-trace / GAE reverse scan. Shapes [T, B] (time_major) or [B, T]; returns (adv, tgt)."""
    _dev(rew, val, term, rho, boot)
    if rew.dtype not in (torch.float32, torch.float64):
        raise TypeError("vtrace needs float32 or float64")
    for t in (val, term, rho, boot):
        if t is not None and (t.dtype != rew.dtype or not t.is_contiguous()):
            raise TypeError("vtrace inputs must share dtype and be contiguous")
    if time_major:
        T, B = rew.shape
    else:
        B, T = rew.shape
    adv = out_adv if out_adv is not None else torch.empty_like(rew)
    tgt = out_tgt if out_tgt is not None else (torch.empty_like(rew) if want_targets else None)
    L.call("ph_vtrace", _DT[rew.dtype], _p(rew), _p(val), _p(term), _p(rho), _p(boot), B, T,
           int(variant), int(time_major), int(rho_is_log), int(clamp), gamma, lam, rho_clip,
           c_clip, _p(adv), _p(tgt), _stream())
    return adv, tgt


def adv_normalize(adv, out=None, stats=None):
    _dev(adv)
    out = out if out is not None else torch.empty_like(adv)
    L.call("ph_adv_normalize", _DT[adv.dtype], _p(adv), adv.numel(), _p(out), _p(stats), _stream())
    return out


def colsum(x, out=None, scale=1.0, accumulate=False):
    _dev(x)
    N, J = x.shape
    out = out if out is not None else torch.empty(J, device=x.device, dtype=torch.float32)
    L.call("ph_colsum", _p(x), N, J, x.stride(0), _p(out), scale, int(accumulate), _stream())
    return out


def convert(x, dtype):
    _dev(x)
    y = torch.empty(x.shape, device=x.device, dtype=dtype)
    L.call("ph_convert", _DT[x.dtype], _p(x), _DT[dtype], _p(y), x.numel(), _stream())
    return y


def ppo_grad(logits, values, act, adv, ret, old, ov=None, *, vf_coef=0.5, ent_coef=0.01,
             clip_eps=0.2, vf_clip=0.0, max_shift=True, dlogits=None, dvalues=None, newlp=None,
             newval=None, losses=None):
    """Fused PPO loss gradient. logits [N, >=A] (row stride honoured), values [N] or strided."""
    _dev(logits, values, act, adv, ret, old, ov)
    N, A = logits.shape[0], logits.shape[1]
    if dlogits is None:
        dlogits = torch.empty((N, A), device=logits.device, dtype=torch.float32)
    if dvalues is None:
        dvalues = torch.empty(N, device=logits.device, dtype=torch.float32)
    ldv = values.stride(0)
    lddv = dvalues.stride(0)
    L.call("ph_ppo_grad", _p(logits), logits.stride(0), _p(values), ldv, _p(act), _p(adv),
           _p(ret), _p(old), _p(ov), N, A, vf_coef, ent_coef, clip_eps, vf_clip, int(max_shift),
           _p(dlogits), dlogits.stride(0), _p(dvalues), lddv, _p(newlp), _p(newval), _p(losses),
           _stream())
    return dlogits, dvalues


def gemm(a, b, *, trans_a=False, trans_b=False, out=None, out_dtype=torch.float32, math="bf16",
         epilogue=L.PH_EPI_NONE, bias=None, aux=None, alpha=1.0, beta=0.0, out2=None,
         out2_trans=False, splits=0):
    """C = op(a) @ op(b) on MFMA. a is [M,K] (or [K,M] if trans_a); b is [K,N] (or [N,K])."""
    _dev(a, b, out, bias, aux, out2)
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    Kb = b.shape[1] if trans_b else b.shape[0]
    if K != Kb:
        raise ValueError(f"gemm: inner extents differ ({K} vs {Kb})")
    if out is None:
        out = torch.empty((M, N), device=a.device, dtype=out_dtype)
    m = L.PH_MATH_BF16 if math == "bf16" else L.PH_MATH_F32
    L.call("ph_gemm", int(trans_a), int(trans_b), M, N, K, _DT[a.dtype], _p(a), a.stride(0),
           _DT[b.dtype], _p(b), b.stride(0), _DT[out.dtype], _p(out), out.stride(0), m, epilogue,
           _p(bias), _p(aux), aux.stride(0) if aux is not None else 0, alpha, beta, _p(out2),
           out2.stride(0) if out2 is not None else 0, int(out2_trans), splits, _stream())
    return out
