"""MI355X implementation of the reference's GLA / Gated DeltaNet kernel surface.

Mirrors triune/kernels/fast_gla.py (names, argument meaning, return tuples and [B, T, H, D]
layouts) on top of libtriune_hip.so.  Every function runs the HIP kernels on the tensors'
device; there is no CPU or PyTorch fallback: unsupported inputs raise.

Differences from the reference, by design:
  * final states are returned in float32 (the reference returns q.dtype: fast_gla.py:332,
    :739-743); the recurrent state never round-trips through bf16 between calls;
  * beta of shape [B, T, H] at T == 1 is applied per (token, head); the reference's T == 1
    branch broadcasts it against the wrong axes unless H == head_dim (fast_gla.py:880).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import TriuneHipError, check, dtype_code, lib, onepass_ctrl, ptr, stream_of, strides

__all__ = [
    "fast_chunk_gla",
    "fast_chunk_gla_varlen",
    "gla_decode_step",
    "FusedRecurrentScan",
    "fast_chunk_gated_deltanet",
    "fast_recurrent_gated_deltanet",
    "_triton_chunk_gla_tc_fwd",
    "gla_prefill_noalloc",
    "TriuneHipError",
]

_DIMS = (32, 64, 128)
_PAIRS = ((32, 32), (64, 64), (128, 64), (128, 128))  # (Dk, Dv) the prefill kernels support
_DECODE_PAIRS = ((32, 32), (64, 64), (64, 128), (128, 64), (128, 128))
# Gated DeltaNet prefill: the chunked WY/UT kernels (head dims <= 64, and 128 with 16-bit I/O)
# unless this is False, in which case every call takes the token-serial kernel (kept for fp32 I/O
# at head dim 128 and single tokens).
_chunked_gdn_enabled = True
# Gates with one value per (token, head) take the scalar-decay chunked kernels unless this is False
# (then they run the per-key-dim chunked kernels on the broadcast gate).
_scalar_gdn_enabled = True


def _on_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("triune_amd kernels take HIP device tensors (device='cuda'); got a CPU tensor")


def _round_dk(d: int) -> int:
    for c in _DIMS:
        if d <= c:
            return c
    raise ValueError(f"key head dim {d} > 128 is not supported")


def _pair(dk: int, dv: int, pairs=_PAIRS) -> tuple[int, int]:
    """Smallest supported (Dk, Dv) >= (dk, dv); inputs are zero-padded up to it."""
    best = None
    for a, b in pairs:
        if a >= dk and b >= dv and (best is None or a * b < best[0] * best[1]):
            best = (a, b)
    if best is None:
        raise ValueError(f"head dims ({dk}, {dv}) exceed the supported (128, 128)")
    return best


def _vec_ok(x: torch.Tensor, tok_dim: int | None = None) -> bool:
    """Unit innermost stride and 16-byte aligned rows; tok_dim: the token axis of a token tensor
    ([B, T, H, D]: 1, packed [N, H, D]: 0), whose stride must also be at least the row width (the
    chunk kernels read a sequence's rows only up to its last token, so rows must not overlap)."""
    m = 4 if x.dtype == torch.float32 else 8
    ok = x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(s % m == 0 for s in x.stride()[:-1])
    if ok and tok_dim is not None and x.shape[tok_dim] > 1 and x.stride(tok_dim) < x.shape[-1]:
        ok = False
    return ok


def _vec_layout(x: torch.Tensor, tok_dim: int | None = None) -> torch.Tensor:
    """x if _vec_ok(x, tok_dim), else a contiguous copy (e.g. of a tensor expanded along tokens)."""
    return x if _vec_ok(x, tok_dim) else x.contiguous()


def _pad_last(x: torch.Tensor, d: int) -> torch.Tensor:
    return x if x.shape[-1] == d else F.pad(x, (0, d - x.shape[-1]))


def _state_in(s: torch.Tensor | None, dk: int, dv: int) -> torch.Tensor | None:
    if s is None:
        return None
    s = s.to(torch.float32)
    if s.shape[-2] != dk or s.shape[-1] != dv:
        s = F.pad(s, (0, dv - s.shape[-1], 0, dk - s.shape[-2]))
    return s.contiguous()


def _check_io(q, k, v, g):
    _on_device(q, k, v, g)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must share one dtype")
    if g.dtype not in (q.dtype, torch.float32):
        raise TypeError("g must have q's dtype or float32")


def _tok3(x: torch.Tensor):
    return (x.stride(0), x.stride(1), x.stride(2))


# ---------------------------------------------------------------------------------------
# GLA prefill / decode
# ---------------------------------------------------------------------------------------


def _gate(g, q):
    return g if g.dtype in (q.dtype, torch.float32) else g.float()


# Calls of few chunks (at most 64 per sequence, every chunk-head workgroup resident at once, head
# dim 64, 16-bit I/O) run the single-launch prefill; False forces the three-launch path (tests
# cover both).
ONEPASS = True


def _prefill(q, k, v, g, initial_state, out, flags, save_final=True, out_dtype=None):
    B, T, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    # value columns evolve independently: wide values run as column slices, 128 wide, or 64 wide
    # for fp32 inputs whose pair would be (128, 128) (its fp32 planes exceed the LDS)
    vcap = 64 if (q.dtype == torch.float32 and _pair(Dk0, min(Dv0, 128)) == (128, 128)) else 128
    if Dv0 > vcap:
        outs, states = [], []
        for c in range(0, Dv0, vcap):
            s0 = None if initial_state is None else initial_state[..., c:c + vcap]
            o_c, s_c = _prefill(q, k, v[..., c:c + vcap], g, s0, None, flags, save_final,
                                out.dtype if out is not None else (out_dtype or v.dtype))
            outs.append(o_c)
            states.append(s_c)
        o = torch.cat(outs, dim=-1)
        if out is not None:
            out.copy_(o)
            o = out
        return o, (torch.cat(states, dim=-1) if save_final else None)
    if T == 0 or B == 0:  # nothing to scan: the final state is the initial state
        o = out if out is not None else torch.empty(B, T, H, Dv0, device=q.device, dtype=out_dtype or v.dtype)
        if not save_final:
            return o, None
        if initial_state is None:
            return o, torch.zeros(B, H, Dk0, Dv0, device=q.device, dtype=torch.float32)
        return o, initial_state.to(torch.float32).clone()
    Dk, Dv = _pair(Dk0, Dv0)
    qp, kp, gp = (_vec_layout(_pad_last(x, Dk), 1) for x in (q, k, _gate(g, q)))
    vp = _vec_layout(_pad_last(v, Dv), 1)
    odt = out.dtype if out is not None else (out_dtype or v.dtype)
    if out is not None and out.shape[-1] == Dv and out.stride(-1) == 1 and _vec_layout(out, 1) is out:
        o = out
    else:
        o = torch.empty(B, T, H, Dv, device=q.device, dtype=odt)
    s0 = _state_in(initial_state, Dk, Dv)
    sf = torch.empty(B, H, Dk, Dv, device=q.device, dtype=torch.float32) if save_final else None
    L = lib()
    st = strides(_tok3(qp), _tok3(kp), _tok3(vp), _tok3(gp), _tok3(o))
    if ONEPASS and Dk == Dv == 64 and L.triune_hip_gla_prefill_onepass_supported(
            B, T, H, 64, dtype_code(qp), dtype_code(gp), 0, flags):
        # few chunks: states and outputs in one launch (triune_hip_gla_prefill_onepass)
        ws = torch.empty(int(L.triune_hip_gla_prefill_onepass_workspace_size(B, T, H, 64)), device=q.device,
                         dtype=torch.uint8)
        ctrl = onepass_ctrl(q.device, int(L.triune_hip_gla_prefill_onepass_ctrl_size(B, T, H, 64)))
        rc = L.triune_hip_gla_prefill_onepass(
            ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), st, None, None, 0, 0, 0, ptr(s0),
            ptr(o), dtype_code(o), ptr(sf), B, T, H, 64, flags, ptr(ws), ws.numel(), ptr(ctrl), ctrl.numel(),
            stream_of(q),
        )
        check(rc, "triune_hip_gla_prefill_onepass")
    else:
        wsb = L.triune_hip_gla_prefill_workspace_size(B, T, H, Dk, Dv, flags)
        ws = torch.empty(max(int(wsb), 256), device=q.device, dtype=torch.uint8)
        rc = L.triune_hip_gla_prefill(
            ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), st, ptr(s0), ptr(o), dtype_code(o),
            ptr(sf), B, T, H, Dk, Dv, flags, ptr(ws), ws.numel(), stream_of(q),
        )
        check(rc, "triune_hip_gla_prefill")
    if o is not out:
        res = o[..., :Dv0]
        if out is not None:
            out.copy_(res)
            res = out
        o = res
    if sf is not None and (Dk != Dk0 or Dv != Dv0):
        sf = sf[..., :Dk0, :Dv0].contiguous()
    return o, sf


def gla_decode_step(q, k, v, g, state, out=None, *, inplace=False, slots=None, out_dtype=None):
    """One recurrent decode step for a batch of sequences (reference: fast_gla.py:746-753,
    csrc/engine/engine.cpp:419-475, csrc/kernels/gla.cu:23-75):
        S <- diag(exp(g)) S + k v^T ;  o = S^T q          (g not clamped)
    q, k, g: [B, 1, H, Dk] or [B, H, Dk]; v: [B, 1, H, Dv] or [B, H, Dv]; state fp32
    [B, H, Dk, Dv] (or a pool [N, H, Dk, Dv] addressed by int32 `slots` [B]).
    Returns (o shaped like v, state).  With inplace=True the state tensor is updated in place
    (it must then be a contiguous float32 tensor); otherwise a new state is returned."""
    _check_io(q, k, v, g)
    squeeze = q.dim() == 4
    if squeeze:
        if q.shape[1] != 1:
            raise ValueError("decode step takes one token per sequence (T == 1)")
        q, k, v, g = q[:, 0], k[:, 0], v[:, 0], g[:, 0]
    B, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    Dk, Dv = _pair(Dk0, Dv0, _DECODE_PAIRS)
    padded = (Dk, Dv) != (Dk0, Dv0)
    qp, kp, gp = (_vec_layout(_pad_last(x, Dk)) for x in (q, k, g))
    vp = _vec_layout(_pad_last(v, Dv))
    if slots is None and state.shape[0] != B:
        raise ValueError(f"state has {state.shape[0]} rows for a batch of {B} (pass slots to address a pool)")
    if inplace:
        if padded or state.dtype != torch.float32 or not state.is_contiguous():
            raise ValueError("inplace decode needs a contiguous float32 state with supported head dims")
        s_in = s_out = state
    else:
        s_in = _state_in(state, Dk, Dv)
        # with slots only the addressed rows are written: the others keep their input values
        s_out = torch.empty_like(s_in) if slots is None else s_in.clone()
    odt = out.dtype if out is not None else (out_dtype or v.dtype)
    o = None
    if out is not None and Dv == Dv0:
        ov = out[:, 0] if out.dim() == 4 else out
        if tuple(ov.shape) == (B, H, Dv) and ov.stride(-1) == 1 and _vec_layout(ov) is ov:
            o = ov  # write straight into the caller's buffer
    if o is None:
        o = torch.empty(B, H, Dv, device=q.device, dtype=odt)
    if slots is not None:
        slots = slots.to(device=q.device, dtype=torch.int32).contiguous()
    st = strides(qp.stride()[:2], kp.stride()[:2], vp.stride()[:2], gp.stride()[:2], o.stride()[:2])
    rc = lib().triune_hip_gla_decode_step(
        ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), st, ptr(s_in), ptr(s_out), ptr(slots),
        s_in.shape[0], ptr(o), dtype_code(o), B, H, Dk, Dv, stream_of(q),
    )
    check(rc, "triune_hip_gla_decode_step")
    if not inplace and padded:
        s_out = s_out[..., :Dk0, :Dv0].contiguous()
    if out is not None:
        if o.data_ptr() != out.data_ptr():
            out.copy_(o[..., :Dv0].reshape(out.shape))
        return out, s_out
    o = o[..., :Dv0]
    if squeeze:
        o = o.unsqueeze(1)
    return o, s_out


def _needs_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _prefill_bwd(q, k, v, g, s0, do, ds, flags, grad_dtype=None, outs=None, acc=0):
    """Gradients (dq, dk, dv, dg, ds0) of _prefill for upstream do (of o) and ds (of the fp32
    final state), either of which may be None.  grad_dtype: dtype of dq, dk, dv, dg (default:
    the inputs' own dtypes).  outs: fp32 (dq, dk, dv, dg) views of exactly the kernel width to
    write into (or, for the parts acc names, add into: _lib.FLAG_BWD_ACC_QKG / FLAG_BWD_ACC_V);
    they are returned in place of new tensors."""
    B, T, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    lim = 32 if q.dtype == torch.float32 else 64  # widest head the gradient kernels hold
    if max(Dk0, Dv0) > lim:
        return _prefill_bwd_blocks(q, k, v, g, s0, do, ds, flags, grad_dtype, lim)
    D = 32 if max(Dk0, Dv0) <= 32 else 64
    qp, kp, gp = (_vec_layout(_pad_last(x, D), 1) for x in (q, k, _gate(g, q)))
    vp = _vec_layout(_pad_last(v, D), 1)
    if do is None:
        do = torch.zeros(B, T, H, Dv0, device=q.device, dtype=q.dtype)
    dop = _vec_layout(_pad_last(do.to(q.dtype), D), 1)
    dsf = None
    if ds is not None:
        dsf = _state_in(ds, D, D)
    s0p = _state_in(s0, D, D)
    if outs is not None:
        if Dk0 != D or Dv0 != D or any(t.dtype != torch.float32 or t.shape[-1] != D for t in outs):
            raise ValueError("outs must be fp32 views of the kernel width")
        dq, dk, dv, dg = outs
    else:
        dq = torch.empty(B, T, H, D, device=q.device, dtype=grad_dtype or q.dtype)
        dk, dv = torch.empty_like(dq), torch.empty_like(dq)
        dg = torch.empty(B, T, H, D, device=q.device, dtype=grad_dtype or gp.dtype)
    ds0 = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32) if s0 is not None else None
    L = lib()
    wsb = L.triune_hip_gla_prefill_bwd_workspace_size(B, max(T, 1), H, D, D, flags)
    ws = torch.empty(max(int(wsb), 256), device=q.device, dtype=torch.uint8)
    st = strides(_tok3(qp), _tok3(kp), _tok3(vp), _tok3(gp), _tok3(dop), _tok3(dq), _tok3(dk), _tok3(dv), _tok3(dg))
    rc = L.triune_hip_gla_prefill_bwd(
        ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), ptr(dop), st, ptr(s0p), ptr(dsf),
        ptr(dq), ptr(dk), ptr(dv), dtype_code(dq), ptr(dg), dtype_code(dg), ptr(ds0), B, T, H, D, D, flags | acc,
        ptr(ws), ws.numel(), stream_of(q),
    )
    check(rc, "triune_hip_gla_prefill_bwd")
    if outs is not None:
        return dq, dk, dv, dg, ds0
    dq, dk, dv, dg = dq[..., :Dk0], dk[..., :Dk0], dv[..., :Dv0], dg[..., :Dk0].to(grad_dtype or g.dtype)
    if ds0 is not None:
        ds0 = ds0[..., :Dk0, :Dv0].to(s0.dtype)
    return dq, dk, dv, dg, ds0


def _prefill_bwd_blocks(q, k, v, g, s0, do, ds, flags, grad_dtype, lim):
    """_prefill_bwd for heads wider than the gradient kernels hold, as a sum over blocks of at
    most `lim` key dims and `lim` value columns.  The recurrence is separable in both: state entry
    S[d][c] evolves from k[d], g[d] and v[c] alone and o sums q[d] S[d][c] over d, so block (a, b)
    of (key dims, value columns) is an independent GLA problem with inputs q_a, k_a, g_a, v_b,
    S0[a][b] and upstream do_b, dS[a][b].  dq, dk and dg of key block a sum over the value blocks,
    dv of value block b over the key blocks (in fp32, rounded once), and dS0[a][b] is block
    (a, b)'s own."""
    B, T, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    kbl = [(i, min(i + lim, Dk0)) for i in range(0, Dk0, lim)]
    vbl = [(j, min(j + lim, Dv0)) for j in range(0, Dv0, lim)]
    f32 = torch.float32
    # Blocks of the full kernel width write into (first block) or add into (the others) the fp32
    # gradients in place; a narrower tail block goes through padded temporaries and adds.
    direct = Dk0 % lim == 0 and Dv0 % lim == 0
    alloc = torch.empty if direct else torch.zeros
    dq = alloc(B, T, H, Dk0, device=q.device, dtype=f32)
    dk, dg = alloc(B, T, H, Dk0, device=q.device, dtype=f32), alloc(B, T, H, Dk0, device=q.device, dtype=f32)
    dv = alloc(B, T, H, Dv0, device=q.device, dtype=f32)
    ds0 = torch.empty(B, H, Dk0, Dv0, device=q.device, dtype=f32) if s0 is not None else None
    for ai, (a0, a1) in enumerate(kbl):
        for bi, (b0, b1) in enumerate(vbl):
            args = (q[..., a0:a1], k[..., a0:a1], v[..., b0:b1], g[..., a0:a1],
                    None if s0 is None else s0[..., a0:a1, b0:b1], None if do is None else do[..., b0:b1],
                    None if ds is None else ds[..., a0:a1, b0:b1], flags)
            if direct:
                acc = (_lib.FLAG_BWD_ACC_QKG if bi > 0 else 0) | (_lib.FLAG_BWD_ACC_V if ai > 0 else 0)
                r = _prefill_bwd(*args, outs=(dq[..., a0:a1], dk[..., a0:a1], dv[..., b0:b1], dg[..., a0:a1]),
                                 acc=acc)
            else:
                r = _prefill_bwd(*args, grad_dtype=f32)
                dq[..., a0:a1] += r[0]
                dk[..., a0:a1] += r[1]
                dv[..., b0:b1] += r[2]
                dg[..., a0:a1] += r[3]
            if ds0 is not None:
                ds0[..., a0:a1, b0:b1] = r[4]
    gd = grad_dtype or q.dtype
    return (dq.to(gd), dk.to(gd), dv.to(grad_dtype or v.dtype), dg.to(grad_dtype or g.dtype),
            None if ds0 is None else ds0.to(s0.dtype))


class _ChunkGLA(torch.autograd.Function):
    """fast_chunk_gla with gradients: forward on the prefill kernels (every T, the dispatch
    flags carried in), backward on triune_hip_gla_prefill_bwd."""

    @staticmethod
    def forward(ctx, q, k, v, g, initial_state, flags):
        o, s = _prefill(q, k, v, g, initial_state, None, flags)
        ctx.save_for_backward(q, k, v, g, initial_state)
        ctx.flags = flags
        return o, s

    @staticmethod
    def backward(ctx, do, ds):
        q, k, v, g, s0 = ctx.saved_tensors
        dq, dk, dv, dg, ds0 = _prefill_bwd(q, k, v, g, s0, do, ds, ctx.flags)
        return dq, dk, dv, dg, ds0, None


def fast_chunk_gla(q, k, v, g, initial_state=None, chunk_size=64, out=None):
    """Chunked GLA forward (reference: fast_chunk_gla, triune/kernels/fast_gla.py:692-778).

    q, k, g: [B, T, H, Dk]; v: [B, T, H, Dv]; initial_state: [B, H, Dk, Dv] or None;
    out: optional [B, T, H, Dv] output buffer (may alias g).  Returns (out, final_state) with
    final_state in float32.  g is clamped at 0 for prefill tokens; T == 1 runs the decode step
    (no clamp), and a single-token remainder after whole chunks of `chunk_size` keeps its g
    unclamped, exactly as the reference's dispatch does (fast_gla.py:746-775).  chunk_size only
    affects that dispatch rule: the kernels always use 64-token chunks internally.

    Differentiable: when any input requires a gradient (and grad mode is on) the call goes
    through an autograd.Function whose backward runs the HIP gradient kernels (the reference
    differentiates its PyTorch chunk path, fast_gla.py:720-737); `out` is then not written,
    as in the reference's training path, which ignores it."""
    _check_io(q, k, v, g)
    B, T, H, _ = q.shape
    C = int(chunk_size)
    if _needs_grad(q, k, v, g, initial_state):
        flags = _lib.FLAG_TAIL_UNCLAMPED if (T == 1 or (C > 0 and T > C and T % C == 1)) else 0
        return _ChunkGLA.apply(q, k, v, g, initial_state, flags)
    if T == 1:
        st = initial_state
        if st is None:
            st = torch.zeros(B, H, q.shape[-1], v.shape[-1], device=q.device, dtype=torch.float32)
        return gla_decode_step(q, k, v, g, st, out=out)
    flags = _lib.FLAG_TAIL_UNCLAMPED if (C > 0 and T > C and T % C == 1) else 0
    return _prefill(q, k, v, g, initial_state, out, flags)


def gla_prefill_noalloc(q, k, v, g, initial_state, out, final_state, *, flags=0):
    """fast_chunk_gla's chunked prefill for callers that cannot allocate device memory (graph
    capture, serving loops): runs triune_hip_gla_prefill_noalloc, whose workspace is a static
    per-GPU device array, and allocates nothing itself.  No reference counterpart.

    q, k, g [B, T, H, Dk], v and out [B, T, H, Dv] with (Dk, Dv) a kernel pair (32x32, 64x64,
    128x64, 128x128), unit innermost stride, 16-byte aligned rows, token stride >= the row width
    (nothing is padded or copied: other layouts raise ValueError); initial_state and final_state
    contiguous float32 [B, H, Dk, Dv] or None.  g is clamped at 0 (flags: TRIUNE_FLAG_* as for
    triune_hip_gla_prefill).  Calls on one GPU share its scratch, so calls that overlap (other
    streams or threads) race.  Returns (out, final_state)."""
    _check_io(q, k, v, g)
    _on_device(initial_state, out, final_state)
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    if (Dk, Dv) not in _PAIRS:
        raise ValueError(f"head dims ({Dk}, {Dv}) are not a kernel pair {_PAIRS}")
    if tuple(out.shape) != (B, T, H, Dv):
        raise ValueError("out must be [B, T, H, Dv]")
    if not all(_vec_ok(x, 1) for x in (q, k, v, g, out)):
        raise ValueError("gla_prefill_noalloc copies nothing: q, k, v, g, out need unit innermost stride, "
                         "16-byte aligned rows and token strides of at least a row")
    for st in (initial_state, final_state):
        if st is not None and (st.dtype != torch.float32 or not st.is_contiguous() or
                               tuple(st.shape) != (B, H, Dk, Dv)):
            raise ValueError("states must be contiguous float32 [B, H, Dk, Dv]")
    rc = lib().triune_hip_gla_prefill_noalloc(
        ptr(q), ptr(k), ptr(v), ptr(g), dtype_code(q), dtype_code(g),
        strides(_tok3(q), _tok3(k), _tok3(v), _tok3(g), _tok3(out)), ptr(initial_state), ptr(out),
        dtype_code(out), ptr(final_state), B, T, H, Dk, Dv, flags, stream_of(q),
    )
    check(rc, "triune_hip_gla_prefill_noalloc")
    return out, final_state


def _triton_chunk_gla_tc_fwd(q, k, v, g, initial_state=None, out=None, save_final=True):
    """Drop-in for the reference's fused prefill entry (fast_gla.py:318-380), as called by
    VectorisedGLA (attention.py:443-451, :486-494): returns (out, final_state); when
    save_final is False the second item is a 1-element placeholder, as in the reference."""
    _check_io(q, k, v, g)
    o, sf = _prefill(q, k, v, g, initial_state, out, 0, save_final=save_final)
    if sf is None:
        sf = torch.empty((1,), device=q.device, dtype=torch.float32)
    return o, sf


def fast_chunk_gla_varlen(q, k, v, g, cu_seqlens, initial_state=None, out=None, *, state_pool=None, slots=None):
    """Packed ragged GLA prefill (no reference counterpart; equals one fast_chunk_gla call per
    sequence).  q, k, g: [1, N, H, Dk] or [N, H, Dk]; v likewise with Dv; cu_seqlens: int32
    [n + 1] offsets (device or host); initial_state: [n, H, Dk, Dv] or None.
    Returns (out shaped like v, final_states fp32 [n, H, Dk, Dv]).  g is clamped at 0.

    With state_pool (fp32 contiguous [n_slots, H, Dk, Dv], (Dk, Dv) a kernel pair: 32x32, 64x64,
    128x64 or 128x128) and slots (int32 [n], distinct), sequence i starts from state_pool[slots[i]]
    and its final state is written back there in place; initial_state must then be None and the
    second item returned is state_pool.  A slot of -1 starts from zero and keeps nothing."""
    _check_io(q, k, v, g)
    if state_pool is not None:
        return _varlen_pool(q, k, v, g, cu_seqlens, state_pool, slots, out, initial_state)
    lead1 = q.dim() == 4
    if lead1:
        if q.shape[0] != 1:
            raise ValueError("packed varlen tensors have batch size 1")
        q, k, v, g = q[0], k[0], v[0], g[0]
    N, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    # value columns evolve independently: wide values run as column slices (as _prefill does)
    vcap = 64 if (q.dtype == torch.float32 and _pair(Dk0, min(Dv0, 128)) == (128, 128)) else 128
    if Dv0 > vcap:
        outs, states = [], []
        for c in range(0, Dv0, vcap):
            sl = slice(c, c + vcap)
            o_c, s_c = fast_chunk_gla_varlen(
                q, k, v[..., sl], g, cu_seqlens, None if initial_state is None else initial_state[..., sl],
                None if out is None else (out[0] if out.dim() == 4 else out)[..., sl])
            outs.append(o_c)
            states.append(s_c)
        sf = torch.cat(states, dim=-1)
        if out is not None:
            return out, sf
        o = torch.cat(outs, dim=-1)
        return (o.unsqueeze(0) if lead1 else o), sf
    Dk, Dv = _pair(Dk0, Dv0)
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    n = cu.numel() - 1
    qp, kp, gp = (_vec_layout(_pad_last(x, Dk), 0) for x in (q, k, _gate(g, q)))
    vp = _vec_layout(_pad_last(v, Dv), 0)
    odt = out.dtype if out is not None else v.dtype
    o = None
    if out is not None and Dv == Dv0:
        ov = out[0] if out.dim() == 4 else out
        if tuple(ov.shape) == (N, H, Dv) and ov.stride(-1) == 1 and _vec_layout(ov, 0) is ov:
            o = ov  # write straight into the caller's buffer
    if o is None:
        o = torch.empty(N, H, Dv, device=q.device, dtype=odt)
    s0 = _state_in(initial_state, Dk, Dv)
    sf = torch.empty(n, H, Dk, Dv, device=q.device, dtype=torch.float32)
    L = lib()
    wsb = L.triune_hip_gla_prefill_varlen_workspace_size(n, N, H, Dk, Dv, 0)
    ws = torch.empty(max(int(wsb), 256), device=q.device, dtype=torch.uint8)
    st = strides(qp.stride()[:2], kp.stride()[:2], vp.stride()[:2], gp.stride()[:2], o.stride()[:2])
    rc = L.triune_hip_gla_prefill_varlen(
        ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), st, ptr(cu), n, N, ptr(s0), ptr(o),
        dtype_code(o), ptr(sf), H, Dk, Dv, 0, ptr(ws), ws.numel(), stream_of(q),
    )
    check(rc, "triune_hip_gla_prefill_varlen")
    o = o[..., :Dv0]
    if Dk != Dk0 or Dv != Dv0:
        sf = sf[..., :Dk0, :Dv0].contiguous()
    if out is not None:
        if o.data_ptr() != out.data_ptr():
            out.copy_(o.reshape(out.shape))
        return out, sf
    if lead1:
        o = o.unsqueeze(0)
    return o, sf


def _varlen_pool(q, k, v, g, cu_seqlens, pool, slots, out, initial_state):
    if initial_state is not None:
        raise ValueError("pass either initial_state or state_pool, not both")
    if slots is None:
        raise ValueError("state_pool needs slots")
    _on_device(pool)
    lead1 = q.dim() == 4
    if lead1:
        if q.shape[0] != 1:
            raise ValueError("packed varlen tensors have batch size 1")
        q, k, v, g = q[0], k[0], v[0], g[0]
    N, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    if pool.dtype != torch.float32 or not pool.is_contiguous() or pool.dim() != 4 or tuple(pool.shape[1:]) != (H, Dk0, Dv0):
        raise ValueError(f"state_pool must be a contiguous float32 [n_slots, {H}, {Dk0}, {Dv0}] tensor")
    if _pair(Dk0, Dv0) != (Dk0, Dv0):
        raise ValueError(f"state_pool head dims ({Dk0}, {Dv0}) must be a kernel pair (no padding in place)")
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    n = cu.numel() - 1
    sl = slots.to(device=q.device, dtype=torch.int32).contiguous() if torch.is_tensor(slots) else torch.tensor(
        list(slots), device=q.device, dtype=torch.int32)
    if sl.numel() != n:
        raise ValueError(f"{sl.numel()} slots for {n} sequences")
    qp, kp, gp = (_vec_layout(x, 0) for x in (q, k, _gate(g, q)))
    vp = _vec_layout(v, 0)
    o = None
    if out is not None:
        ov = out[0] if out.dim() == 4 else out
        if tuple(ov.shape) == (N, H, Dv0) and ov.stride(-1) == 1 and _vec_layout(ov, 0) is ov:
            o = ov
    if o is None:
        o = torch.empty(N, H, Dv0, device=q.device, dtype=out.dtype if out is not None else v.dtype)
    L = lib()
    wsb = L.triune_hip_gla_prefill_varlen_workspace_size(n, N, H, Dk0, Dv0, 0)
    ws = torch.empty(max(int(wsb), 256), device=q.device, dtype=torch.uint8)
    st = strides(qp.stride()[:2], kp.stride()[:2], vp.stride()[:2], gp.stride()[:2], o.stride()[:2])
    rc = L.triune_hip_gla_prefill_varlen_pool(
        ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), st, ptr(cu), n, N, ptr(sl), ptr(pool),
        pool.shape[0], ptr(o), dtype_code(o), H, Dk0, Dv0, 0, ptr(ws), ws.numel(), stream_of(q),
    )
    check(rc, "triune_hip_gla_prefill_varlen_pool")
    if out is not None:
        if o.data_ptr() != out.data_ptr():
            out.copy_(o.reshape(out.shape))
        return out, pool
    return (o.unsqueeze(0) if lead1 else o), pool


# ---------------------------------------------------------------------------------------
# FusedRecurrentScan
# ---------------------------------------------------------------------------------------


class FusedRecurrentScan(torch.autograd.Function):
    """Exclusive affine scan over chunk states (reference: FusedRecurrentScan, fast_gla.py:109-203).

    apply(kv [B,H,N,Dk,Dv], decay_k [B,H,N,Dk,1], init_state [B,H,Dk,Dv]) ->
        (S_all [B,H,N,Dk,Dv], final [B,H,Dk,Dv]), both in kv.dtype, where S_all[:, :, n] is the
    state before step n and each step is s <- decay * s + kv.  Differentiable: when a gradient is
    needed the forward keeps its states in fp32 (as the reference saves s_out, fast_gla.py:141)
    and the backward runs triune_hip_recurrent_scan_bwd (reference kernel :67-107), returning
    gradients in kv.dtype (:199-203)."""

    @staticmethod
    def forward(ctx, kv: torch.Tensor, decay_k: torch.Tensor, init_state: torch.Tensor):
        _on_device(kv, decay_k, init_state)
        B, H, N, Dk, Dv = kv.shape
        kvc = kv.contiguous()
        dec = decay_k.expand(B, H, N, Dk, 1)[..., 0].to(torch.float32).contiguous()  # [B,H,N,Dk]: small
        init = init_state.expand(B, H, Dk, Dv).contiguous()
        if Dv % 4 != 0:
            raise ValueError("FusedRecurrentScan needs Dv % 4 == 0")
        grad = any(ctx.needs_input_grad)
        sdt = torch.float32 if grad else kv.dtype
        s_all = torch.empty(kvc.shape, device=kv.device, dtype=sdt)
        fin = torch.empty(B, H, Dk, Dv, device=kv.device, dtype=sdt)
        rc = lib().triune_hip_recurrent_scan_fwd(
            ptr(kvc), dtype_code(kvc), ptr(dec), dtype_code(dec), ptr(init), dtype_code(init), ptr(s_all), ptr(fin),
            dtype_code(s_all), B, H, N, Dk, Dv, stream_of(kv),
        )
        check(rc, "triune_hip_recurrent_scan_fwd")
        if grad:
            if Dv > 256:
                raise ValueError("FusedRecurrentScan backward supports Dv <= 256")
            ctx.save_for_backward(dec, s_all)
            ctx.kv_dtype = kv.dtype
            return s_all.to(kv.dtype), fin.to(kv.dtype)
        return s_all, fin

    @staticmethod
    def backward(ctx, d_s_all, d_fin):
        dec, s32 = ctx.saved_tensors
        B, H, N, Dk, Dv = s32.shape
        dsa = None if d_s_all is None else _vec_layout(d_s_all.contiguous())
        dfi = None if d_fin is None else d_fin.contiguous()
        odt = ctx.kv_dtype
        d_kv = torch.empty(B, H, N, Dk, Dv, device=s32.device, dtype=odt)
        d_dec = torch.empty(B, H, N, Dk, device=s32.device, dtype=odt)
        d_init = torch.empty(B, H, Dk, Dv, device=s32.device, dtype=odt)
        rc = lib().triune_hip_recurrent_scan_bwd(
            ptr(dsa), dtype_code(dsa) if dsa is not None else 0, ptr(dfi), dtype_code(dfi) if dfi is not None else 0,
            ptr(dec), dtype_code(dec), ptr(s32), ptr(d_kv), ptr(d_dec), ptr(d_init), dtype_code(d_kv),
            B, H, N, Dk, Dv, stream_of(s32),
        )
        check(rc, "triune_hip_recurrent_scan_bwd")
        return d_kv, d_dec.unsqueeze(-1), d_init


# ---------------------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------------------


def _scalar_gate(g):
    """The [B, T, H] view of a gate holding one log-decay per (token, head), or None: g of shape
    [B, T, H], [B, T, H, 1], or [B, T, H, D] broadcast over the head dim (stride 0, as
    g.unsqueeze(-1).expand(..., D) makes it)."""
    if g.dim() == 3:
        return g
    if g.dim() == 4 and (g.shape[-1] == 1 or g.stride(-1) == 0):
        return g[..., 0]
    return None


def _gdn(q, k, v, g, beta, initial_state, beta_kind, out_dtype=None):
    _check_io(q, k, v, g)
    if g.dim() == 3 or g.shape[-1] != q.shape[-1]:  # one gate per (token, head): the per-dim kernels take it broadcast
        sg = _scalar_gate(g)
        if sg is None:
            raise ValueError(f"Gated DeltaNet gate of shape {tuple(g.shape)}: expected [B, T, H], [B, T, H, 1], "
                             "[B, T, H, D] broadcast over the head dim, or [B, T, H, Dk]")
        g = sg.unsqueeze(-1).expand(*sg.shape, q.shape[-1])
    _on_device(beta, initial_state)
    if _needs_grad(q, k, v, g, beta, initial_state):
        # the reference differentiates its PyTorch recurrence here (fast_gla.py:885-904)
        return _GatedDeltaNet.apply(q, k, v, g, beta, initial_state, beta_kind, out_dtype)
    return _gdn_fwd(q, k, v, g, beta, initial_state, beta_kind, out_dtype)


def _gdn_bwd(q, k, v, g, beta, initial_state, beta_kind, do, ds):
    """Gradients (dq, dk, dv, dg, dbeta, ds0) of _gdn_fwd for upstream do (of o) and ds (of the
    fp32 final state), either of which may be None, on triune_hip_gdn_bwd.  Head dims are
    zero-padded to the kernels' 64 or 128 (padded rows and columns of the state stay zero)."""
    B, T, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    D = 64 if max(Dk0, Dv0) <= 64 else 128
    if max(Dk0, Dv0) > 128:
        raise ValueError("Gated DeltaNet backward supports head dims up to 128")
    if T == 0 or B == 0:  # no tokens: the initial state's gradient is the final state's
        z = lambda x: torch.zeros_like(x)  # noqa: E731
        ds0 = None
        if initial_state is not None:
            ds0 = (ds if ds is not None else torch.zeros_like(initial_state)).to(initial_state.dtype)
        return z(q), z(k), z(v), z(g), None if beta is None else z(beta), ds0
    qp, kp, vp = (_vec_layout(_pad_last(x, D), 1) for x in (q, k, v))
    gp = _vec_layout(_pad_last(g, D), 1)
    bp, bst = None, (0, 0, 0)
    if beta is not None:
        bp = beta
        if beta_kind in (_lib.BETA_KEY, _lib.BETA_VALUE):
            bp = _vec_layout(_pad_last(beta, D), 1)
        bst = (bp.stride(0), bp.stride(1), bp.stride(2))
    dop = None if do is None else _vec_layout(_pad_last(do, D), 1)
    s0 = _state_in(initial_state, D, D)
    dsf = _state_in(ds, D, D)
    dq, dk, dv = (torch.empty(B, T, H, D, device=q.device, dtype=q.dtype) for _ in range(3))
    dg = torch.empty(B, T, H, D, device=q.device, dtype=gp.dtype)
    db = None
    if beta is not None:
        db = torch.empty(bp.shape if beta_kind == _lib.BETA_HEAD else (B, T, H, D), device=q.device, dtype=bp.dtype)
    ds0 = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32) if initial_state is not None else None
    L = lib()
    wsb = L.triune_hip_gdn_bwd_workspace_size(B, T, H, D, D, beta_kind)
    ws = torch.empty(max(int(wsb), 16), device=q.device, dtype=torch.uint8)
    st = strides(_tok3(qp), _tok3(kp), _tok3(vp), _tok3(gp), bst, _tok3(dop) if dop is not None else (0, 0, 0))
    rc = L.triune_hip_gdn_bwd(
        ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), ptr(bp),
        dtype_code(bp) if bp is not None else 0, beta_kind, st, ptr(s0), ptr(dop),
        dtype_code(dop) if dop is not None else 0, ptr(dsf), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(db), ptr(ds0),
        B, T, H, D, D, ptr(ws), ws.numel(), stream_of(q),
    )
    check(rc, "triune_hip_gdn_bwd")
    dq, dk, dg = dq[..., :Dk0], dk[..., :Dk0], dg[..., :Dk0]
    dv = dv[..., :Dv0]
    if db is not None and beta_kind != _lib.BETA_HEAD:
        db = db[..., :(Dk0 if beta_kind == _lib.BETA_KEY else Dv0)]
    if ds0 is not None:
        ds0 = ds0[..., :Dk0, :Dv0].to(initial_state.dtype)
    return dq, dk, dv, dg.to(g.dtype), None if db is None else db.to(beta.dtype), ds0


class _GatedDeltaNet(torch.autograd.Function):
    """Gated DeltaNet with gradients: forward on the HIP forward kernels, backward on
    triune_hip_gdn_bwd (states recomputed from checkpoints)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, beta_kind, out_dtype):
        o, s = _gdn_fwd(q, k, v, g, beta, initial_state, beta_kind, out_dtype)
        ctx.save_for_backward(q, k, v, g, beta, initial_state)
        ctx.beta_kind = beta_kind
        return o, s

    @staticmethod
    def backward(ctx, do, ds):
        q, k, v, g, beta, s0 = ctx.saved_tensors
        dq, dk, dv, dg, db, ds0 = _gdn_bwd(q, k, v, g, beta, s0, ctx.beta_kind, do, ds)
        return dq, dk, dv, dg, db, ds0, None, None


def _gdn_fwd(q, k, v, g, beta, initial_state, beta_kind, out_dtype=None):
    sg = _scalar_gate(g)
    B, T, H, Dk0 = q.shape
    Dv0 = v.shape[-1]
    if T == 0 or B == 0:  # nothing to scan: the final state is the initial state
        o = torch.empty(B, T, H, Dv0, device=q.device, dtype=out_dtype or v.dtype)
        if initial_state is None:
            return o, torch.zeros(B, H, Dk0, Dv0, device=q.device, dtype=torch.float32)
        return o, initial_state.to(torch.float32).clone()
    D = _round_dk(max(Dk0, Dv0))
    # chunked WY/UT path: (64, 64) heads (smaller ones zero-padded) and (128, 128) heads with 16-bit
    # I/O, every beta kind; a gate with one value per (token, head) and beta none or per token
    # takes the scalar-decay kernels at D <= 64
    chunked = (D <= 64 or (D == 128 and q.dtype != torch.float32)) and T > 1 and _chunked_gdn_enabled
    scalar = (chunked and D <= 64 and sg is not None and beta_kind in (_lib.BETA_NONE, _lib.BETA_HEAD)
              and _scalar_gdn_enabled)
    if chunked and D <= 64:
        D = 64
    qp, kp, vp = (_vec_layout(_pad_last(x, D), 1) for x in (q, k, v))
    gp = sg if scalar else _vec_layout(_pad_last(g, D), 1)
    bp = None
    bst = (0, 0, 0)
    if beta is not None:
        bp = beta
        if beta_kind in (_lib.BETA_KEY, _lib.BETA_VALUE):
            bp = _pad_last(beta, D)
        if (chunked and beta_kind in (_lib.BETA_KEY, _lib.BETA_VALUE)) or T == 1:
            bp = bp.to(torch.float32)  # the per-dim chunked kernels and the decode step read fp32
        bp = bp.contiguous()
        bst = (bp.stride(0), bp.stride(1), bp.stride(2))
    o = torch.empty(B, T, H, D, device=q.device, dtype=out_dtype or v.dtype)
    s0 = _state_in(initial_state, D, D)
    sf = torch.empty(B, H, D, D, device=q.device, dtype=torch.float32)
    st = strides(_tok3(qp), _tok3(kp), _tok3(vp), _tok3(gp), bst, _tok3(o))
    if scalar:
        ws_bytes = lib().triune_hip_gdn_prefill_scalar_decay_workspace_size(B, T, H, D, D)
        ws = torch.empty(max(int(ws_bytes), 16), device=q.device, dtype=torch.uint8)
        rc = lib().triune_hip_gdn_prefill_scalar_decay(
            ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), ptr(bp),
            dtype_code(bp) if bp is not None else 0, beta_kind, st, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, D, D, ptr(ws), ws_bytes, stream_of(q),
        )
        check(rc, "triune_hip_gdn_prefill_scalar_decay")
    elif chunked:
        ws_bytes = lib().triune_hip_gdn_prefill_chunked_workspace_size(B, T, H, D, D)
        ws = torch.empty(max(int(ws_bytes), 16), device=q.device, dtype=torch.uint8)
        rc = lib().triune_hip_gdn_prefill_chunked(
            ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), ptr(bp),
            dtype_code(bp) if bp is not None else 0, beta_kind, st, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, D, D, ptr(ws), ws_bytes, stream_of(q),
        )
        check(rc, "triune_hip_gdn_prefill_chunked")
    else:
        rc = lib().triune_hip_gdn_prefill(
            ptr(qp), ptr(kp), ptr(vp), ptr(gp), dtype_code(qp), dtype_code(gp), ptr(bp),
            dtype_code(bp) if bp is not None else 0, beta_kind, st, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, D, D, stream_of(q),
        )
        check(rc, "triune_hip_gdn_prefill")
    if D != Dv0:
        o = o[..., :Dv0]
    if D != Dk0 or D != Dv0:
        sf = sf[..., :Dk0, :Dv0].contiguous()
    return o, sf


def _beta_kind(beta, orientation):
    if beta is None:
        return _lib.BETA_NONE
    if beta.dim() == 3:
        return _lib.BETA_HEAD
    return _lib.BETA_KEY if orientation == "key" else _lib.BETA_VALUE


def fast_recurrent_gated_deltanet(q, k, v, g, beta=None, initial_state=None, *, out_dtype=None):
    """Gated DeltaNet, reference variant (fast_gla.py:781-836):
        u_t = v_t - S_{t-1}^T k_t ; S_t = diag(exp(min(g_t,0))) S_{t-1} + beta_t (k_t u_t^T) ; o_t = S_t^T q_t
    beta None, [B, T, H] or [B, T, H, D]; a 4-D beta scales rows (key dim), as this reference
    function does.  out_dtype: dtype of the output (default v.dtype; float32 keeps the fp32
    accumulators unrounded).  Differentiable in q, k, v, g, beta and initial_state, as the
    reference's autograd through this loop (backward: triune_hip_gdn_bwd).  Returns (out,
    final_state fp32)."""
    return _gdn(q, k, v, g, beta, initial_state, _beta_kind(beta, "key"), out_dtype)


def fast_chunk_gated_deltanet(q, k, v, g, beta=None, initial_state=None, chunk_size=64, *, out_dtype=None):
    """Gated DeltaNet operator entry (reference: fast_chunk_gated_deltanet, fast_gla.py:839-904).
    A 4-D beta scales columns (value dim) as the reference's GPU kernel does for T > 1
    (fast_gla.py:464-465), and rows at T == 1 (fast_gla.py:880) and whenever a gradient is needed
    (the reference then runs its PyTorch recurrence, fast_gla.py:885-904, which scales rows).
    Differentiable in q, k, v, g, beta and initial_state (backward: triune_hip_gdn_bwd).
    chunk_size is accepted for signature parity.  out_dtype as for
    fast_recurrent_gated_deltanet.  Returns (out, final_state fp32)."""
    T = q.shape[1]
    grad = _needs_grad(q, k, v, g, beta, initial_state)
    orientation = "key" if (T == 1 or grad) else "value"
    return _gdn(q, k, v, g, beta, initial_state, _beta_kind(beta, orientation), out_dtype)
