"""ctypes front end of the fp64 oracle (gla_oracle.c) and of the reference's own C decode step.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker.  triune_amd never imports this module.

All functions take numpy arrays (any float dtype; converted to contiguous float64) and
return float64 arrays.  Layouts follow the reference: tokens [B, T, H, D], states
[B, H, Dk, Dv].  Reference anchors are listed in gla_oracle.c.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None
_REF = None

_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int32)
_L = ctypes.c_long
_I = ctypes.c_int


def build() -> None:
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(_HERE), "all"], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.is_file():
            build()
        lib = ctypes.CDLL(str(path))
        lib.oracle_gla_fwd.argtypes = [_dp] * 7 + [_L, _L, _L, _I, _I, _L, _I]
        lib.oracle_gla_varlen_fwd.argtypes = [_dp] * 4 + [_ip, _L, _dp, _dp, _dp, _L, _I, _I]
        lib.oracle_gla_closed_form.argtypes = [_dp] * 7 + [_L, _L, _L, _I, _I]
        lib.oracle_gla_decode_step.argtypes = [_dp] * 6 + [_L, _I, _I]
        lib.oracle_recurrent_scan_fwd.argtypes = [_dp] * 5 + [_L, _L, _L, _I, _I]
        lib.oracle_recurrent_scan_bwd.argtypes = [_dp] * 7 + [_L, _L, _L, _I, _I]
        lib.oracle_gla_bwd.argtypes = [_dp] * 12 + [_L, _L, _L, _I, _I, _L, _I]
        lib.oracle_gdn_fwd.argtypes = [_dp] * 5 + [_I, _dp, _dp, _dp, _L, _L, _L, _I, _I]
        lib.oracle_gdn_bwd.argtypes = [_dp] * 5 + [_I] + [_dp] * 9 + [_L, _L, _L, _I, _I]
        lib.oracle_num_threads.restype = _I
        _LIB = lib
    return _LIB


def _d(x):
    """float64 contiguous copy (or None)."""
    if x is None:
        return None
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().cpu().double().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _p(a):
    return None if a is None else a.ctypes.data_as(_dp)


def num_threads() -> int:
    return int(_lib().oracle_num_threads())


def gla_fwd(q, k, v, g, s0=None, chunk=64, clamp_mode=2):
    """GLA forward (token recurrence).  clamp_mode 2 follows fast_chunk_gla's dispatch
    (fast_gla.py:692-778), 1 always clamps g<=0, 0 never clamps.  Returns (o, S_final)."""
    q, k, v, g, s0 = _d(q), _d(k), _d(v), _d(g), _d(s0)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = np.empty((B, T, H, Dv))
    s = np.empty((B, H, Dk, Dv))
    _lib().oracle_gla_fwd(_p(q), _p(k), _p(v), _p(g), _p(s0), _p(o), _p(s), B, T, H, Dk, Dv, chunk, clamp_mode)
    return o, s


def gla_varlen_fwd(q, k, v, g, cu_seqlens, s0=None):
    """Packed ragged GLA.  q,k,g [1 or N_tok, ..., H, Dk] packed rows; cu_seqlens int32 [n+1];
    s0 [n, H, Dk, Dv] or None.  Returns (o [same leading shape], S_final [n, H, Dk, Dv])."""
    q, k, v, g, s0 = _d(q), _d(k), _d(v), _d(g), _d(s0)
    lead = q.shape[:-2]
    H, Dk = q.shape[-2:]
    Dv = v.shape[-1]
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    n = cu.shape[0] - 1
    o = np.empty(lead + (H, Dv))
    s = np.empty((n, H, Dk, Dv))
    _lib().oracle_gla_varlen_fwd(
        _p(q), _p(k), _p(v), _p(g), cu.ctypes.data_as(_ip), n, _p(s0), _p(o), _p(s), H, Dk, Dv
    )
    return o, s


def gla_closed_form(q, k, v, g, s0=None):
    """Non-recurrent closed form of the GLA map (g clamped at 0).  O(T^2): tiny inputs only."""
    q, k, v, g, s0 = _d(q), _d(k), _d(v), _d(g), _d(s0)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = np.empty((B, T, H, Dv))
    s = np.empty((B, H, Dk, Dv))
    _lib().oracle_gla_closed_form(_p(q), _p(k), _p(v), _p(g), _p(s0), _p(o), _p(s), B, T, H, Dk, Dv)
    return o, s


def gla_decode_step(q, k, v, g, state):
    """One decode step (no clamp).  q,k,g [..., Dk]; v [..., Dv]; state [..., Dk, Dv].
    Returns (o, new_state); the input state is not modified."""
    q, k, v, g = _d(q), _d(k), _d(v), _d(g)
    S = _d(state).copy()
    Dk, Dv = S.shape[-2:]
    BH = S.size // (Dk * Dv)
    o = np.empty(v.shape)
    _lib().oracle_gla_decode_step(_p(q), _p(k), _p(v), _p(g), _p(S), _p(o), BH, Dk, Dv)
    return o, S


def recurrent_scan_fwd(kv, decay_k, init):
    """FusedRecurrentScan forward: kv [B,H,N,Dk,Dv], decay_k [B,H,N,Dk,1], init [B,H,Dk,Dv].
    Returns (S_all exclusive [B,H,N,Dk,Dv], final [B,H,Dk,Dv])."""
    kv, init = _d(kv), _d(init)
    dec = _d(decay_k)
    B, H, N, Dk, Dv = kv.shape
    dec = np.ascontiguousarray(np.broadcast_to(dec, (B, H, N, Dk, 1))[..., 0])
    s_all = np.empty_like(kv)
    fin = np.empty((B, H, Dk, Dv))
    _lib().oracle_recurrent_scan_fwd(_p(kv), _p(dec), _p(init), _p(s_all), _p(fin), B, H, N, Dk, Dv)
    return s_all, fin


def recurrent_scan_bwd(d_s_all, d_fin, decay_k, s_all):
    """FusedRecurrentScan backward (fast_gla.py:67-107, :151-203): upstream gradients d_s_all
    [B,H,N,Dk,Dv] and d_fin [B,H,Dk,Dv] (None = zero), decay_k [B,H,N,Dk,1], the forward's
    s_all.  Returns (d_kv [B,H,N,Dk,Dv], d_decay [B,H,N,Dk,1], d_init [B,H,Dk,Dv])."""
    s_all = _d(s_all)
    B, H, N, Dk, Dv = s_all.shape
    dec = np.ascontiguousarray(np.broadcast_to(_d(decay_k), (B, H, N, Dk, 1))[..., 0])
    d_kv = np.empty_like(s_all)
    d_dec = np.empty((B, H, N, Dk))
    d_init = np.empty((B, H, Dk, Dv))
    _lib().oracle_recurrent_scan_bwd(_p(_d(d_s_all)), _p(_d(d_fin)), _p(dec), _p(s_all), _p(d_kv), _p(d_dec),
                                     _p(d_init), B, H, N, Dk, Dv)
    return d_kv, d_dec[..., None], d_init


def gla_bwd(q, k, v, g, s0=None, do=None, ds_fin=None, chunk=64, clamp_mode=2):
    """Gradients of gla_fwd (same clamp semantics) for upstream do [B,T,H,Dv] and ds_fin
    [B,H,Dk,Dv] (None = zero).  Returns (dq, dk, dv, dg, ds0)."""
    q, k, v, g, s0, do, ds_fin = (_d(x) for x in (q, k, v, g, s0, do, ds_fin))
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    dq, dk, dg = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    dv = np.empty_like(v)
    ds0 = np.empty((B, H, Dk, Dv))
    _lib().oracle_gla_bwd(_p(q), _p(k), _p(v), _p(g), _p(s0), _p(do), _p(ds_fin), _p(dq), _p(dk), _p(dv), _p(dg),
                          _p(ds0), B, T, H, Dk, Dv, chunk, clamp_mode)
    return dq, dk, dv, dg, ds0


BETA_NONE, BETA_HEAD, BETA_KEY, BETA_VALUE = 0, 1, 2, 3


def gdn_fwd(q, k, v, g, beta=None, s0=None, beta_kind=None):
    """Reference Gated DeltaNet variant (fast_gla.py:781-836).  beta None, [B,T,H] or
    [B,T,H,D]; for a 4-D beta, beta_kind selects rows (BETA_KEY, the PyTorch path) or
    columns (BETA_VALUE, the Triton path).  Returns (o, S_final)."""
    q, k, v, g, s0 = _d(q), _d(k), _d(v), _d(g), _d(s0)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    if beta is None:
        kind, bt = BETA_NONE, None
    else:
        bt = _d(beta)
        if bt.ndim == 3:
            kind = BETA_HEAD
        else:
            kind = BETA_KEY if beta_kind is None else beta_kind
    o = np.empty((B, T, H, Dv))
    s = np.empty((B, H, Dk, Dv))
    _lib().oracle_gdn_fwd(_p(q), _p(k), _p(v), _p(g), _p(bt), kind, _p(s0), _p(o), _p(s), B, T, H, Dk, Dv)
    return o, s


def gdn_bwd(q, k, v, g, beta=None, s0=None, do=None, ds_fin=None, beta_kind=None):
    """Gradients of gdn_fwd (same beta conventions) for upstream do [B,T,H,Dv] and ds_fin
    [B,H,Dk,Dv] (None = zero): the reference's autograd through fast_recurrent_gated_deltanet
    (fast_gla.py:781-836), which fast_chunk_gated_deltanet runs whenever a gradient is needed
    (:885-904).  Returns (dq, dk, dv, dg, dbeta or None, ds0)."""
    q, k, v, g, s0, do, ds_fin = (_d(x) for x in (q, k, v, g, s0, do, ds_fin))
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    if beta is None:
        kind, bt = BETA_NONE, None
    else:
        bt = _d(beta)
        kind = BETA_HEAD if bt.ndim == 3 else (BETA_KEY if beta_kind is None else beta_kind)
    dq, dk, dg = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    dv = np.empty_like(v)
    db = None if bt is None else np.empty_like(bt)
    ds0 = np.empty((B, H, Dk, Dv))
    _lib().oracle_gdn_bwd(_p(q), _p(k), _p(v), _p(g), _p(bt), kind, _p(s0), _p(do), _p(ds_fin), _p(dq), _p(dk),
                          _p(dv), _p(dg), _p(db), _p(ds0), B, T, H, Dk, Dv)
    return dq, dk, dv, dg, db, ds0


# ---------------------------------------------------------------------------------------
# The reference's own C decode step (csrc/engine/engine.cpp:419-475), compiled from the
# reference sources into oracle/_ref/ by the Makefile.  fp32, polynomial exp
# (engine.cpp:57-69), in place on the state.
# ---------------------------------------------------------------------------------------


# --- VectorisedGLA input pre-processing (reference: triune/model/attention.py:14-179, the fused
# Triton kernels; unfused form :509-528).  Plain float64 numpy restatements. ---------------------
def elu1(x):
    """elu(x) + 1 = x + 1 for x >= 0, exp(x) otherwise (attention.py:39-40, 521)."""
    x = _d(x)
    return np.where(x >= 0.0, x + 1.0, np.exp(np.minimum(x, 0.0)))


def logsigmoid(x):
    """log(1 / (1 + exp(-x))), evaluated without overflow (attention.py:74-75)."""
    x = _d(x)
    return np.minimum(x, 0.0) - np.log1p(np.exp(-np.abs(x)))


def qk_prep(x, cos=None, sin=None):
    """RoPE(normalize(elu(x) + 1)) over the last axis (HD): normalize(a) = a / sqrt(max(sum a^2,
    1e-12)) (attention.py:41-43); RoPE pairs element d with d + HD/2 (attention.py:53-61):
    out[d] = a[d] cos[d] - a[d + HD/2] sin[d], out[d + HD/2] = a[d + HD/2] cos[d + HD/2] +
    a[d] sin[d + HD/2].  cos/sin broadcast against x (None: no rotation)."""
    a = elu1(x)
    a = a / np.sqrt(np.maximum((a * a).sum(axis=-1, keepdims=True), 1e-12))
    if cos is None:
        return a
    half = a.shape[-1] // 2
    rot = np.concatenate([-a[..., half:], a[..., :half]], axis=-1)
    return a * _d(cos) + rot * _d(sin)


def qkv_g_prep(qkv, g, cos=None, sin=None):
    """The in-place pre-processing of qkv [B, T, 3, H, HD] and g [B, T, H, HD], cos/sin [T, HD]
    (attention.py:14-79).  Returns new (qkv, g) arrays; v is copied unchanged."""
    qkv = _d(qkv).copy()
    cs = sn = None
    if cos is not None:
        cs = _d(cos)[None, :, None, :]
        sn = _d(sin)[None, :, None, :]
    qkv[:, :, 0] = qk_prep(qkv[:, :, 0], cs, sn)
    qkv[:, :, 1] = qk_prep(qkv[:, :, 1], cs, sn)
    return qkv, logsigmoid(g)


def fused_decode_step(qkvg, cos, sin, state):
    """The decode step fused with the pre-processing (attention.py:81-179): qkvg [B, 4, H, HD]
    raw, cos/sin [HD] or None, state [B, H, HD, HD] or None (zero).  q, k pre-processed, decay
    sigmoid(g) = exp(logsigmoid(g)), then the GLA step.  Returns (o [B, H, HD], new state)."""
    x = _d(qkvg)
    B, _, H, HD = x.shape
    q = qk_prep(x[:, 0], cos, sin)
    k = qk_prep(x[:, 1], cos, sin)
    s0 = np.zeros((B, H, HD, HD)) if state is None else _d(state)
    return gla_decode_step(q, k, x[:, 2], logsigmoid(x[:, 3]), s0)


def ref_library_path() -> Path:
    return _HERE / "_ref" / "libtriune_core_ref.so"


def ref_available() -> bool:
    return ref_library_path().is_file()


def _ref():
    global _REF
    if _REF is None:
        lib = ctypes.CDLL(str(ref_library_path()))
        vp = ctypes.c_void_p
        lib.triune_gla_recurrent_step_f32.argtypes = [vp] * 6 + [ctypes.c_int, ctypes.c_int]
        lib.triune_gla_recurrent_step_f32.restype = None
        _REF = lib
    return _REF


def ref_c_decode_step_f32(q, k, v, g, state):
    """Call the reference's triune_gla_recurrent_step_f32 on float32 copies.
    q,k,v,g [BH, D]; state [BH, D, D].  Returns (o, new_state) as float32 arrays."""
    f = lambda a: np.ascontiguousarray(np.asarray(a, dtype=np.float32))  # noqa: E731
    q, k, v, g = f(q), f(k), f(v), f(g)
    S = f(state).copy()
    D = q.shape[-1]
    BH = q.size // D
    o = np.empty_like(q)
    _ref().triune_gla_recurrent_step_f32(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data, S.ctypes.data, o.ctypes.data, BH, D
    )
    return o, S
