"""Stream-ordered device API over the C ABI, taking torch tensors for device memory.

torch only supplies allocation and the current stream; every computation runs in libpufferhip.so.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L
from . import _lib as _L

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


REF_COEFFS = [(4.0848, -6.8946, 2.9270), (3.9505, -6.3029, 2.6377), (3.7418, -5.5913, 2.3037),
              (2.8769, -3.1427, 1.2046), (2.8366, -3.0525, 1.2012)]
CONST_COEFFS = [(3.4445, -4.7750, 2.0315)] * 5


def _coeffs(coeffs, dtype):
    import numpy as np
    c = np.ascontiguousarray(np.asarray(coeffs, dtype=dtype).reshape(-1, 3))
    return c, c.ctypes.data_as(C.c_void_p), c.shape[0]


def muon_mat_f64(W, G, M, *, gscale=1.0, lr=0.1, wd=0.0, mu=0.95, eps=1e-7, coeffs=REF_COEFFS,
                 out_w=None, out_m=None):
    """Exact-tier Muon matrix step on f64 device tensors; returns (newW, newM)."""
    _dev(W, G, M)
    rows, cols = W.shape
    nW = out_w if out_w is not None else torch.empty_like(W)
    nM = out_m if out_m is not None else torch.empty_like(M)
    c, cp, ns = _coeffs(coeffs, "float64")
    L.call("ph_muon_mat_f64", rows, cols, _p(W), _p(G), _p(M), _p(nW), _p(nM), gscale, lr, wd, mu,
           eps, cp, ns, _stream())
    return nW, nM


def stepvec_f64(b, g, m, *, gscale=1.0, lr=0.1, wd=0.0, mu=0.95):
    _dev(b, g, m)
    nb, nm = torch.empty_like(b), torch.empty_like(m)
    L.call("ph_stepvec_f64", b.numel(), _p(b), _p(g), _p(m), _p(nb), _p(nm), gscale, lr, wd, mu,
           _stream())
    return nb, nm


def newton_schulz(X, *, coeffs=CONST_COEFFS, eps=1e-7, math="bf16"):
    """In-place fast-tier NS of an fp32 matrix; returns X."""
    _dev(X)
    if X.dtype != torch.float32 or not X.is_contiguous():
        raise TypeError("newton_schulz needs a contiguous fp32 matrix")
    c, cp, ns = _coeffs(coeffs, "float32")
    m = L.PH_MATH_BF16 if math == "bf16" else L.PH_MATH_F32
    L.call("ph_newton_schulz", _p(X), X.shape[0], X.shape[1], cp, ns, eps, m, _stream())
    return X


def ns_status():
    """Synchronises the current stream and raises if a fused Newton-Schulz launch since the last check
    gave up a bounded wait (its matrices are invalid); clears the record."""
    L.call("ph_ns_status", _stream())


def ns_set_spin_limit(polls=0):
    """Bound of the fused Newton-Schulz waits (0: the default)."""
    L.call("ph_ns_set_spin_limit", int(polls))


def ns_set_queues(mode=0):
    """Placement of the fused Newton-Schulz work: 0 by shape (per-XCD queues when every phase of every
    matrix fits one XCD; the default), 1 one device-wide queue, 2 one queue per XCD. All give
    bit-identical matrices."""
    L.call("ph_ns_set_queues", int(mode))


def scratch_retired():
    """(count, bytes) of scratch buffers retired by growth and not yet released."""
    n, b = C.c_size_t(0), C.c_size_t(0)
    L.call("ph_scratch_retired", C.byref(n), C.byref(b))
    return n.value, b.value


def release_scratch():
    L.call("ph_release_scratch")


def newton_schulz_batch(Xs, *, coeffs=CONST_COEFFS, eps=1e-7, math="bf16"):
    """In-place fast-tier NS of several independent fp32 matrices; equal to calling newton_schulz on
    each. bf16: one fused launch per 16 matrices; fp32: concurrently on the library's stream lanes."""
    _dev(*Xs)
    for X in Xs:
        if X.dtype != torch.float32 or not X.is_contiguous():
            raise TypeError("newton_schulz_batch needs contiguous fp32 matrices")
    c, cp, ns = _coeffs(coeffs, "float32")
    m = L.PH_MATH_BF16 if math == "bf16" else L.PH_MATH_F32
    n = len(Xs)
    ptrs = (C.c_void_p * n)(*[X.data_ptr() for X in Xs])
    rows = (C.c_int * n)(*[X.shape[0] for X in Xs])
    cols = (C.c_int * n)(*[X.shape[1] for X in Xs])
    L.call("ph_newton_schulz_batch", ptrs, rows, cols, n, cp, ns, eps, m, _stream())
    return Xs


def muon_mat(W, G, M, *, gscale=1.0, lr=0.015, wd=0.0, mu=0.95, eps=1e-7, coeffs=CONST_COEFFS,
             math="bf16"):
    """In-place fast-tier Muon matrix step on fp32 W and momentum M."""
    _dev(W, G, M)
    c, cp, ns = _coeffs(coeffs, "float32")
    m = L.PH_MATH_BF16 if math == "bf16" else L.PH_MATH_F32
    L.call("ph_muon_mat", _p(W), _p(G), _p(M), W.shape[0], W.shape[1], gscale, lr, wd, mu, eps, cp,
           ns, m, _stream())
    return W, M


def stepvec(b, g, m, *, gscale=1.0, lr=0.015, wd=0.0, mu=0.95):
    _dev(b, g, m)
    L.call("ph_stepvec", _p(b), _p(g), _p(m), b.numel(), gscale, lr, wd, mu, _stream())
    return b, m


def gclip(g, *, scale=1.0, max_norm=0.0):
    _dev(g)
    L.call("ph_gclip", _p(g), g.numel(), scale, max_norm, _stream())
    return g


# ---- MinGRU policy PPO+Muon step ----------------------------------------------------------------

class MinGRUConfig:
    """Dimensions and coefficients of the MinGRU PPO+Muon minibatch step (time-major columns)."""

    def __init__(self, B, T, D, H, L, A, *, gamma=0.99, lam=0.95, rho_clip=1.0, c_clip=1.0,
                 clip_eps=0.2, vf_coef=0.5, ent_coef=0.01, vf_clip=0.0, lr=0.015, wd=0.0, mu=0.95,
                 eps=1e-7, max_grad_norm=0.0, gscale=1.0, coeffs=CONST_COEFFS, math="bf16",
                 precision="bf16"):
        import numpy as np
        self.dims = _L.MinGRUDims(B, T, D, H, L, A, {"bf16": 0, "f32": 1}[precision])
        self.ppo = _L.PPOCoefs(gamma, lam, rho_clip, c_clip, clip_eps, vf_coef, ent_coef, vf_clip)
        self._coeffs = np.ascontiguousarray(np.asarray(coeffs, dtype=np.float32).reshape(-1, 3))
        m = {"bf16": _L.PH_MATH_BF16, "f32": _L.PH_MATH_F32}[math]
        self.muon = _L.MuonCoefs(lr, wd, mu, eps, max_grad_norm, gscale, self._coeffs.shape[0], m,
                                self._coeffs.ctypes.data_as(C.c_void_p))

    @property
    def P(self):
        return int(_L.lib().ph_mingru_param_count(C.byref(self.dims)))


def mingru_ppo_grad(cfg, params, obs, act, adv, ret, oldlp, oldval, done, G=None, newlp=None,
                    newval=None, losses=None):
    _dev(params, obs, act, adv, ret, oldlp, oldval, done)
    TB = cfg.dims.T * cfg.dims.B
    G = G if G is not None else torch.zeros(cfg.P, device=params.device)
    newlp = newlp if newlp is not None else torch.empty(TB, device=params.device)
    newval = newval if newval is not None else torch.empty(TB, device=params.device)
    L.call("ph_mingru_ppo_grad", C.byref(cfg.dims), C.byref(cfg.ppo), _p(params), _p(obs), _p(act),
           _p(adv), _p(ret), _p(oldlp), _p(oldval), _p(done), _p(G), _p(newlp), _p(newval),
           _p(losses), _stream())
    return G, newlp, newval


def mingru_muon(cfg, params, mom, G):
    _dev(params, mom, G)
    L.call("ph_mingru_muon", C.byref(cfg.dims), C.byref(cfg.muon), _p(params), _p(mom), _p(G),
           _stream())
    return params, mom


def mingru_step(cfg, params, mom, obs, act, oldlp, oldval, rew, done, logrho, boot, G=None,
                losses=None):
    _dev(params, mom, obs, act, oldlp, oldval, rew, done, logrho, boot)
    G = G if G is not None else torch.zeros(cfg.P, device=params.device)
    L.call("ph_mingru_step", C.byref(cfg.dims), C.byref(cfg.ppo), C.byref(cfg.muon), _p(params),
           _p(mom), _p(obs), _p(act), _p(oldlp), _p(oldval), _p(rew), _p(done), _p(logrho),
           _p(boot), _p(G), _p(losses), _stream())
    return params, mom, G


# ---- MLP policy (L hidden layers, combined head) -----------------------------------------------------

class MLPConfig:
    """Dimensions and coefficients of the device MLP update: N rows, obs D, L hidden layers of H, A
    actions (+ the value column)."""

    def __init__(self, N, D, H, L, A, *, gamma=0.99, lam=0.95, rho_clip=1.0, c_clip=1.0, clip_eps=0.2,
                 vf_coef=0.5, ent_coef=0.01, vf_clip=0.0, lr=0.015, wd=0.0, mu=0.95, eps=1e-7,
                 max_grad_norm=0.0, gscale=None, coeffs=CONST_COEFFS, math="f32", muon_math="f32"):
        import numpy as np
        self.dims = _L.MLPDims(N, D, H, L, A)
        self.ppo = _L.PPOCoefs(gamma, lam, rho_clip, c_clip, clip_eps, vf_coef, ent_coef, vf_clip)
        self._coeffs = np.ascontiguousarray(np.asarray(coeffs, dtype=np.float32).reshape(-1, 3))
        self.math = {"bf16": _L.PH_MATH_BF16, "f32": _L.PH_MATH_F32}[math]
        mm = {"bf16": _L.PH_MATH_BF16, "f32": _L.PH_MATH_F32}[muon_math]
        self.muon = _L.MuonCoefs(lr, wd, mu, eps, max_grad_norm, 1.0 / N if gscale is None else gscale,
                                 self._coeffs.shape[0], mm, self._coeffs.ctypes.data_as(C.c_void_p))

    @property
    def P(self):
        return int(_L.lib().ph_mlp_param_count(C.byref(self.dims)))


def mlp_forward(cfg, params, obs, out=None):
    _dev(params, obs)
    out = out if out is not None else torch.empty((cfg.dims.N, cfg.dims.A + 1), device=params.device)
    L.call("ph_mlp_forward", C.byref(cfg.dims), cfg.math, _p(params), _p(obs), _p(out), _stream())
    return out


def mlp_ppo_grad(cfg, params, obs, act, adv, ret, old, ov=None, G=None, newlp=None, newval=None, losses=None):
    _dev(params, obs, act, adv, ret, old, ov)
    G = G if G is not None else torch.empty(cfg.P, device=params.device)
    L.call("ph_mlp_ppo_grad", C.byref(cfg.dims), C.byref(cfg.ppo), cfg.math, _p(params), _p(obs), _p(act),
           _p(adv), _p(ret), _p(old), _p(ov), _p(G), _p(newlp), _p(newval), _p(losses), _stream())
    return G


def mlp_update(cfg, T, params, mom, obs, act, behav_logp, rew, done, G=None, losses=None):
    """One PPO+Muon update over N = T*B time-major rows, in place on params/mom; returns G."""
    _dev(params, mom, obs, act, behav_logp, rew, done)
    G = G if G is not None else torch.empty(cfg.P, device=params.device)
    L.call("ph_mlp_update", C.byref(cfg.dims), int(T), C.byref(cfg.ppo), C.byref(cfg.muon), cfg.math,
           _p(params), _p(mom), _p(obs), _p(act), _p(behav_logp), _p(rew), _p(done), _p(G), _p(losses),
           _stream())
    return G


# ---- prioritised replay ----------------------------------------------------------------------------
class ReplayColumns:
    """The rollout columns of N segments x T steps as ph_replay_cols describes them.

    All given tensors share one dtype (float32 or float64) and layout: [T, N] when time_major, else
    [N, T] (the reference's segment-major rows); act holds K values per row ([T, N, K] / [N, T, K]).
    """

    def __init__(self, N, T, *, adv=None, value=None, ratio=None, act=None, logp=None, term=None,
                 time_major=False, K=1):
        ts = [t for t in (adv, value, ratio, act, logp, term) if t is not None]
        if not ts:
            raise ValueError("ReplayColumns needs at least one column")
        dt = ts[0].dtype
        if dt not in (torch.float32, torch.float64):
            raise TypeError("replay columns must be float32 or float64")
        for t in ts:
            _dev(t)
            if t.dtype != dt or not t.is_contiguous():
                raise TypeError("replay columns must share dtype and be contiguous")
        for t in (adv, value, ratio, logp, term):
            if t is not None and t.numel() != N * T:
                raise ValueError("a replay column must hold N*T values")
        if act is not None and act.numel() != N * T * K:
            raise ValueError("act must hold N*T*K values")
        self.N, self.T, self.K, self.dtype = N, T, K, dt
        self.tensors = (adv, value, ratio, act, logp, term)
        self.c = L.ReplayCols(_DT[dt], int(time_major), N, T, K, *(_p(t) for t in self.tensors))

    def ref(self):
        return C.byref(self.c)


def seg_l1(cols, out=None):
    """sum_t |adv| per segment (float64 [N])."""
    out = out if out is not None else torch.empty(cols.N, device="cuda", dtype=torch.float64)
    L.call("ph_seg_l1", cols.ref(), _p(out), _stream())
    return out


def prio_sample(L1, n_draws, *, alpha, beta, rng_state, seg=None, mbprio=None):
    """Prioritised draws: (seg int32 [n_draws], mbprio float64 [n_draws])."""
    _dev(L1)
    if L1.dtype != torch.float64:
        raise TypeError("prio_sample takes float64 L1")
    seg = seg if seg is not None else torch.empty(n_draws, device=L1.device, dtype=torch.int32)
    mbprio = mbprio if mbprio is not None else torch.empty(n_draws, device=L1.device, dtype=torch.float64)
    L.call("ph_prio_sample", _p(L1), L1.numel(), n_draws, alpha, beta, rng_state & 0xFFFFFFFFFFFFFFFF,
           _p(seg), _p(mbprio), _stream())
    return seg, mbprio


def mb_gather(cols, seg, mbprio=None, out=None, stats=None):
    """Packed minibatch columns [(K+5), T, Bmb] = act|adv|ret|old|term|ov (cols' dtype)."""
    _dev(seg, mbprio)
    if seg.dtype != torch.int32 or (mbprio is not None and mbprio.dtype != torch.float64):
        raise TypeError("seg must be int32 and mbprio float64")
    B = seg.numel()
    out = out if out is not None else torch.empty((cols.K + 5) * cols.T * B, device=seg.device,
                                                  dtype=cols.dtype)
    L.call("ph_mb_gather", cols.ref(), _p(seg), _p(mbprio), B, _p(out), _p(stats), _stream())
    return out


def mb_iterate(cols, seg, newlp, newval):
    """In place: value/ratio of the drawn segments from the BPTT's new_logp/new_value ([T, Bmb] f32)."""
    _dev(seg, newlp, newval)
    if newlp.dtype != torch.float32 or newval.dtype != torch.float32 or seg.dtype != torch.int32:
        raise TypeError("newlp/newval must be float32 and seg int32")
    L.call("ph_mb_iterate", cols.ref(), _p(seg), seg.numel(), _p(newlp), _p(newval), _stream())


# ---- rollout forward and sampler -------------------------------------------------------------------
def sample_actions(logits, A, *, rng_state, has_value=True, act=None, logp=None, value=None):
    """Categorical draw per row of logits [N, >= A (+1)] (float32/float64, row stride honoured):
    returns (act int32 [N], logp [N], value [N] or None)."""
    _dev(logits)
    N = logits.shape[0]
    act = act if act is not None else torch.empty(N, device=logits.device, dtype=torch.int32)
    logp = logp if logp is not None else torch.empty(N, device=logits.device, dtype=logits.dtype)
    if has_value and value is None:
        value = torch.empty(N, device=logits.device, dtype=logits.dtype)
    L.call("ph_sample_actions", _DT[logits.dtype], _p(logits), logits.stride(0), N, A, int(has_value),
           rng_state & 0xFFFFFFFFFFFFFFFF, _p(act), _p(logp), _p(value if has_value else None), _stream())
    return act, logp, (value if has_value else None)


def mingru_rollout_step(params, obs, state, out, *, D, H, L_layers, A, precision=0):
    """One rollout timestep over N envs: obs [N, D] fp32, state [N, L, H] fp32 (in place),
    out [N, A+1] fp32 (logits, then the value)."""
    _dev(params, obs, state, out)
    N = obs.shape[0]
    dims = L.MinGRUDims(N, 1, D, H, L_layers, A, precision)
    L.call("ph_mingru_rollout_step", C.byref(dims), _p(params), _p(obs), _p(state), _p(out), _stream())
    return out


# ---- multi-discrete and Gaussian heads -------------------------------------------------------------
def _sizes(head_sizes):
    return (C.c_int * len(head_sizes))(*[int(s) for s in head_sizes])


def ppo_grad_md(out, act, adv, ret, old, ov=None, *, head_sizes, vf_coef=0.5, ent_coef=0.01, clip_eps=0.2,
                vf_clip=0.0, dout=None, newlp=None, newval=None, losses=None):
    """Loss gradient of K categorical heads: out [N, sum(sizes)+1] fp32 (heads' logits, then the value),
    act int32 [N, K]; adv/ret/old (and ov) fp32 [N]. Returns dout [N, sum(sizes)+1]."""
    _dev(out, act, adv, ret, old)
    N = out.shape[0]
    if act.dtype != torch.int32 or out.dtype != torch.float32:
        raise TypeError("out must be float32 and act int32")
    dout = dout if dout is not None else torch.empty_like(out)
    L.call("ph_ppo_grad_md", _p(out), out.stride(0), _p(act), _p(adv), _p(ret), _p(old), _p(ov), N,
           _sizes(head_sizes), len(head_sizes), vf_coef, ent_coef, clip_eps, vf_clip, _p(dout), dout.stride(0),
           _p(newlp), _p(newval), _p(losses), _stream())
    return dout


def ppo_grad_cont(out, act, adv, ret, old, ov=None, *, dim, vf_coef=0.5, ent_coef=0.01, clip_eps=0.2, vf_clip=0.0,
                  ls_lo=-20.0, ls_hi=2.0, dout=None, newlp=None, newval=None, losses=None):
    """Loss gradient of a d-dim diagonal Gaussian: out [N, 2d+1] fp32 (means, raw log-stds, value),
    act fp32 [N, d]. Returns dout [N, 2d+1]."""
    _dev(out, act, adv, ret, old)
    N = out.shape[0]
    dout = dout if dout is not None else torch.empty_like(out)
    L.call("ph_ppo_grad_cont", _p(out), out.stride(0), _p(act), _p(adv), _p(ret), _p(old), _p(ov), N, dim, vf_coef,
           ent_coef, clip_eps, vf_clip, ls_lo, ls_hi, _p(dout), dout.stride(0), _p(newlp), _p(newval), _p(losses),
           _stream())
    return dout


def sample_actions_md(logits, head_sizes, *, rng_state, out=None):
    """Draw every head of every row of logits [N, sum(sizes)+1] (float32/float64). Returns f64
    [(K+2) * N]: actions (head h at h*N + n), joint log-prob, value."""
    _dev(logits)
    N, K = logits.shape[0], len(head_sizes)
    out = out if out is not None else torch.empty((K + 2) * N, device=logits.device, dtype=torch.float64)
    L.call("ph_sample_actions_md", _DT[logits.dtype], _p(logits), logits.stride(0), N, _sizes(head_sizes), K,
           rng_state & 0xFFFFFFFFFFFFFFFF, _p(out), _stream())
    return out


def sample_actions_cont(y, dim, *, rng_state, ls_lo=-20.0, ls_hi=2.0, out=None):
    """Gaussian draw per row of y [N, 2d+1] (float32/float64). Returns f64 [(d+2) * N]: actions (dim i
    at i*N + n), log-prob, value."""
    _dev(y)
    N = y.shape[0]
    out = out if out is not None else torch.empty((dim + 2) * N, device=y.device, dtype=torch.float64)
    L.call("ph_sample_actions_cont", _DT[y.dtype], _p(y), y.stride(0), N, dim, rng_state & 0xFFFFFFFFFFFFFFFF,
           ls_lo, ls_hi, _p(out), _stream())
    return out
