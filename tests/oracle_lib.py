"""ctypes access to the CPU oracle (oracle/liboracle.so) for the tests and the CPU baseline.

The oracle is test infrastructure: it checks the GPU library and is never part of it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent.parent / "oracle"
ORACLE_SO = ORACLE_DIR / "liboracle.so"

d = C.c_double
sz = C.c_size_t
i = C.c_int
vp = C.c_void_p

_SIG = {
    "orc_rng_next": ([C.POINTER(C.c_uint64)], C.c_uint64),
    "orc_uniform01": ([C.c_uint64], d),
    "orc_randf": ([vp, sz, d, d, C.POINTER(C.c_uint64)], None),
    "orc_vtrace_vec": ([vp, vp, vp, vp, sz, sz, d, d, d, d, vp], None),
    "orc_vtrace_mingru": ([vp, vp, vp, vp, vp, sz, sz, d, d, d, d, vp], None),
    "orc_gae_soa": ([vp, vp, vp, sz, sz, d, d, vp], None),
    "orc_gae_boot_norm": ([vp, vp, vp, vp, sz, sz, d, d, vp], None),
    "orc_vtrace_f64": ([vp, vp, vp, vp, vp, sz, sz, i, i, i, i, d, d, d, d, vp, vp], None),
    "orc_vtrace_f32": ([vp, vp, vp, vp, vp, sz, sz, i, i, i, i, C.c_float, C.c_float, C.c_float,
                        C.c_float, vp, vp], None),
    "orc_adv_normalize": ([vp, sz, vp], None),
    "orc_ppo_grad": ([vp, sz, vp, sz, vp, vp, vp, vp, vp, sz, sz, d, d, d, d, i, vp, sz, vp, sz,
                      vp, vp], None),
    "orc_ppo_losses": ([vp, sz, vp, sz, vp, vp, vp, vp, vp, sz, sz, d, d, d, d, vp], None),
    "orc_gemm": ([i, i, sz, sz, sz, d, vp, sz, vp, sz, d, vp, sz, i], None),
    "orc_dense_forward": ([vp, vp, vp, sz, sz, sz, vp], None),
    "orc_mlp_forward": ([vp, vp, sz, sz, sz, sz, vp], None),
    "orc_mlp_ppo_grad": ([vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, d, d, d, vp, i], None),
    "orc_mlp_deep_ppo_grad": ([vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, d, d, d, d, vp, vp, vp, i], None),
    "orc_newton_schulz": ([vp, i, i, vp, i, d, i, vp], None),
    "orc_muon_mat": ([i, i, vp, vp, vp, vp, vp, d, d, d, d, d, vp, i, i], None),
    "orc_stepvec": ([i, vp, vp, vp, vp, vp, d, d, d, d], None),
    "orc_muon_step_mlp": ([vp, vp, sz, sz, sz, d, d, d, d, d, vp], None),
    "orc_gclip": ([vp, sz, d, d], d),
    "orc_mingru_ppo_grad_seq": ([vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, d, d, d, d,
                                 vp], None),
    "orc_mingru_ppo_grad_seq_md": ([vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, vp, sz, d, d, d, d, vp],
                                    None),
    "orc_mingru_heinsen": ([vp, vp, sz, sz, vp], None),
    "orc_seg_l1": ([vp, sz, sz, vp], None),
    "orc_prio_sample": ([vp, sz, sz, d, d, C.c_uint64, vp, vp, vp, vp], None),
    "orc_gather_seq_minibatch": ([vp, vp, vp, vp, vp, vp, vp, sz, sz, vp, vp], None),
    "orc_mb_iterate": ([vp, vp, vp, vp, vp, vp, sz, sz], None),
    "orc_sample_actions": ([vp, sz, sz, sz, C.c_uint64, vp], None),
    "orc_mingru_step": ([vp, vp, vp, sz, sz, sz, sz, sz, vp], None),
    "orc_ppo_grad_md": ([vp, sz, vp, vp, vp, vp, vp, sz, vp, sz, d, d, d, d, vp, sz, vp, vp], None),
    "orc_ppo_grad_cont": ([vp, sz, vp, vp, vp, vp, vp, sz, sz, d, d, d, d, d, d, vp, sz, vp, vp], None),
    "orc_sample_md": ([vp, sz, sz, vp, sz, C.c_uint64, vp], None),
    "orc_sample_cont": ([vp, sz, sz, sz, C.c_uint64, d, d, vp], None),
    "orc_set_threads": ([i], i),
    "orc_vtrace_f32_mt": ([vp, vp, vp, vp, vp, sz, sz, i, i, i, i, C.c_float, C.c_float, C.c_float, C.c_float,
                           vp, vp, i], None),
    "orc_gemm_blocked": ([i, i, sz, sz, sz, vp, sz, vp, sz, vp, sz, i], None),
    "orc_mingru_ppo_grad_batch": ([vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, d, d, d, d, vp, i],
                                  None),
    "orc_wide_losses": ([i, vp, sz, vp, vp, vp, vp, vp, sz, vp, sz, sz, d, d, d, d, d, d, vp], None),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        build()  # make rebuilds only when oracle.c or oracle.h is newer than the library
        h = C.CDLL(str(ORACLE_SO))
        for name, (args, res) in _SIG.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = res
        _lib = h
    return _lib


def P(a: np.ndarray | None):
    """Pointer to a C-contiguous numpy array (or NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- thin numpy wrappers -------------------------------------------------------------------------

def coeffs_array(coeffs) -> np.ndarray:
    return f64(np.asarray(coeffs, dtype=np.float64).reshape(-1, 3))


REF_COEFFS = [(4.0848, -6.8946, 2.9270), (3.9505, -6.3029, 2.6377), (3.7418, -5.5913, 2.3037),
              (2.8769, -3.1427, 1.2046), (2.8366, -3.0525, 1.2012)]
BASELINE_COEFFS = [(3.4445, -4.7750, 2.0315)] * 5


def vtrace(rew, val, term, rho, boot, B, T, *, variant, time_major, rho_is_log=False, clamp=True,
           gamma=0.99, lam=0.95, rho_clip=1.0, c_clip=1.0, dtype=np.float64):
    conv = f64 if dtype == np.float64 else f32
    rew, val, term = conv(rew), conv(val), conv(term)
    rho = None if rho is None else conv(rho)
    boot = None if boot is None else conv(boot)
    adv = np.zeros(B * T, dtype=dtype)
    tgt = np.zeros(B * T, dtype=dtype)
    fn = lib().orc_vtrace_f64 if dtype == np.float64 else lib().orc_vtrace_f32
    fn(P(rew), P(val), P(term), P(rho), P(boot), B, T, variant, int(time_major), int(rho_is_log),
       int(clamp), gamma, lam, rho_clip, c_clip, P(adv), P(tgt))
    return adv, tgt


def gemm(transA, transB, A, B, M, N, K, threads=1):
    A, B = f64(A), f64(B)
    lda = A.shape[1]
    ldb = B.shape[1]
    Cm = np.zeros((M, N))
    lib().orc_gemm(int(transA), int(transB), M, N, K, 1.0, P(A), lda, P(B), ldb, 0.0, P(Cm), N,
                   threads)
    return Cm


def newton_schulz(X0, coeffs, eps=1e-7, form=1):
    X0 = f64(X0)
    rows, cols = X0.shape
    c = coeffs_array(coeffs)
    out = np.zeros_like(X0)
    lib().orc_newton_schulz(P(X0), rows, cols, P(c), c.shape[0], eps, form, P(out))
    return out


def ppo_grad(logits, values, act, adv, ret, old, ov=None, *, vf=0.5, ent=0.01, clip=0.2,
             vfclip=0.0, max_shift=False):
    logits = f64(logits)
    N, A = logits.shape
    values = f64(values)
    dl = np.zeros((N, A))
    dv = np.zeros(N)
    nlp = np.zeros(N)
    nv = np.zeros(N)
    lib().orc_ppo_grad(P(logits), A, P(values), 1, P(f64(act)), P(f64(adv)), P(f64(ret)),
                       P(f64(old)), P(None if ov is None else f64(ov)), N, A, vf, ent, clip,
                       vfclip, int(max_shift), P(dl), A, P(dv), 1, P(nlp), P(nv))
    return dl, dv, nlp, nv


def ppo_losses(logits, values, act, adv, ret, old, ov=None, *, vf=0.5, ent=0.01, clip=0.2,
               vfclip=0.0):
    logits = f64(logits)
    N, A = logits.shape
    L = np.zeros(7)
    lib().orc_ppo_losses(P(logits), A, P(f64(values)), 1, P(f64(act)), P(f64(adv)), P(f64(ret)),
                         P(f64(old)), P(None if ov is None else f64(ov)), N, A, vf, ent, clip,
                         vfclip, P(L))
    return L


def seg_l1(adv, N, T):
    out = np.zeros(N)
    lib().orc_seg_l1(P(f64(adv)), N, T, P(out))
    return out


def prio_sample(L1, mb, alpha, beta, rng_state):
    """(idx, mbPrio, probs, cum) of the CPU twin of the prioritised sampler."""
    L1 = f64(L1)
    N = L1.size
    idx, mp = np.zeros(mb), np.zeros(mb)
    probs, cum = np.zeros(N), np.zeros(N)
    lib().orc_prio_sample(P(L1), N, mb, alpha, beta, rng_state & 0xFFFFFFFFFFFFFFFF, P(idx), P(mp),
                          P(probs), P(cum))
    return idx, mp, probs, cum


def gather_seq_minibatch(act, logp, term, adv, value, seg, mp, T):
    """(out[6*T*Bmb], [mean, std]) of the CPU twin of the minibatch gather."""
    seg, mp = f64(seg), f64(mp)
    Bmb = seg.size
    out = np.zeros(6 * T * Bmb)
    st = np.zeros(2)
    lib().orc_gather_seq_minibatch(P(f64(act)), P(f64(logp)), P(f64(term)), P(f64(adv)), P(f64(value)),
                                   P(seg), P(mp), T, Bmb, P(out), P(st))
    return out, st


def mb_iterate(value, ratio, logp, newlp, newval, seg, T):
    """In-place value/ratio iterate (copies returned)."""
    value, ratio = f64(value).copy(), f64(ratio).copy()
    seg = f64(seg)
    lib().orc_mb_iterate(P(value), P(ratio), P(f64(logp)), P(f32(newlp)), P(f32(newval)), P(seg),
                         seg.size, T)
    return value, ratio


def sample_actions(Y, A, rng_state):
    """(act, logp, value) of the CPU twin of the categorical sampler; Y is N x O (O >= A + 1)."""
    Y = f64(Y)
    N, O = Y.shape
    out = np.zeros(3 * N)
    lib().orc_sample_actions(P(Y), N, A, O, rng_state & 0xFFFFFFFFFFFFFFFF, P(out))
    return out[:N], out[N:2 * N], out[2 * N:]


def mingru_step(params, obs, state, N, D, H, L, A):
    """(out [N, A+1], new_state [N, L, H]) of the f64 single-step MinGRU forward."""
    out = np.zeros(N * (A + 1) + N * L * H)
    lib().orc_mingru_step(P(f64(params)), P(f64(obs)), P(f64(state)), N, D, H, L, A, P(out))
    return out[:N * (A + 1)].reshape(N, A + 1), out[N * (A + 1):].reshape(N, L, H)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def ppo_grad_md(out, act, adv, ret, old, ov, sizes, *, vf=0.5, ent=0.01, clip=0.2, vfclip=0.0):
    out = f64(out)
    N, O = out.shape
    K = len(sizes)
    sz = _i32(sizes)
    d = np.zeros((N, O))
    nlp, nv = np.zeros(N), np.zeros(N)
    lib().orc_ppo_grad_md(P(out), O, P(f64(act)), P(f64(adv)), P(f64(ret)), P(f64(old)),
                          P(None if ov is None else f64(ov)), N, P(sz), K, vf, ent, clip, vfclip, P(d), O, P(nlp),
                          P(nv))
    return d, nlp, nv


def ppo_grad_cont(out, act, adv, ret, old, ov, dim, *, vf=0.5, ent=0.01, clip=0.2, vfclip=0.0, lslo=-20.0,
                  lshi=2.0):
    out = f64(out)
    N, O = out.shape
    d = np.zeros((N, O))
    nlp, nv = np.zeros(N), np.zeros(N)
    lib().orc_ppo_grad_cont(P(out), O, P(f64(act)), P(f64(adv)), P(f64(ret)), P(f64(old)),
                            P(None if ov is None else f64(ov)), N, dim, vf, ent, clip, vfclip, lslo, lshi, P(d), O,
                            P(nlp), P(nv))
    return d, nlp, nv


def wide_losses(mode, out, act, adv, ret, old, ov, *, sizes=None, dim=0, vf=0.5, ent=0.01, clip=0.2, vfclip=0.0,
                lslo=-20.0, lshi=2.0):
    """The 7 dashboard losses of multi-discrete (mode 1, head sizes) or Gaussian (mode 2, dim) rows."""
    out = f64(out)
    N, O = out.shape
    K = len(sizes) if sizes is not None else 0
    L = np.zeros(7)
    lib().orc_wide_losses(mode, P(out), O, P(f64(act)), P(f64(adv)), P(f64(ret)), P(f64(old)),
                          P(None if ov is None else f64(ov)), N, P(_i32(sizes) if sizes is not None else None), K,
                          dim, vf, ent, clip, vfclip, lslo, lshi, P(L))
    return L


def sample_md(Y, sizes, rng_state):
    Y = f64(Y)
    N, O = Y.shape
    K = len(sizes)
    out = np.zeros((K + 2) * N)
    lib().orc_sample_md(P(Y), O, N, P(_i32(sizes)), K, rng_state & 0xFFFFFFFFFFFFFFFF, P(out))
    return out


def sample_cont(Y, dim, rng_state, lslo=-20.0, lshi=2.0):
    Y = f64(Y)
    N, O = Y.shape
    out = np.zeros((dim + 2) * N)
    lib().orc_sample_cont(P(Y), O, N, dim, rng_state & 0xFFFFFFFFFFFFFFFF, lslo, lshi, P(out))
    return out


def mlp_deep_param_count(D, H, L, A):
    return H * D + H + (L - 1) * (H * H + H) + (A + 1) * H + A + 1


def mlp_deep_ppo_grad(p, obs, act, adv, ret, old, ov, N, D, H, L, A, *, vf=0.5, ent=0.01, clip=0.2,
                      vfclip=0.0, threads=8):
    """Summed gradient of the L-hidden-layer combined-head MLP; returns (g, newlp, newval)."""
    g = np.zeros(mlp_deep_param_count(D, H, L, A))
    nlp = np.zeros(N)
    nv = np.zeros(N)
    lib().orc_mlp_deep_ppo_grad(P(f64(p)), P(f64(obs)), P(f64(act)), P(f64(adv)), P(f64(ret)), P(f64(old)),
                                None if ov is None else P(f64(ov)), N, D, H, L, A, vf, ent, clip, vfclip,
                                P(g), P(nlp), P(nv), threads)
    return g, nlp, nv

