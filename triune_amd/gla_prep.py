"""GLA input pre-processing on MI355X, and the decode step fused with it.

Mirrors the two Triton kernels of the reference's VectorisedGLA fast path
(triune/model/attention.py:14-79 _fused_qkv_g_prep_inplace_kernel and :81-179
_fused_qkvg_decode_step_kernel) and the way attention.py:405-450 launches them:

  fused_qkv_g_prep_inplace(qkv, g, cos, sin, use_rope)
      qkv [B, T, 3, H, HD] (q, k, v parts), g [B, T, H, HD], cos/sin [T, HD]; in place:
      q, k <- RoPE(normalize(elu(x) + 1)), g <- logsigmoid(g); v untouched.
  fused_qkvg_decode_step(qkvg, cos, sin, initial_state, save_final, use_rope)
      qkvg [B, 4, H, HD] raw projections of one token per sequence; returns (out [B, 1, H, HD],
      final state [B, H, HD, HD] or None), with decay sigmoid(g).

normalize(a) = a / sqrt(max(sum a^2, 1e-12)) over the HD elements of a (token, head) row; RoPE
pairs element d with d + HD/2.  HD in {32, 64, 128}.  Tensors must be on the GPU; there is no CPU
path.
"""

from __future__ import annotations

import torch

from ._lib import check, dtype_code, lib, ptr, stream_of, strides

__all__ = ["fused_qkv_g_prep_inplace", "fused_qkvg_decode_step"]

_HD = (32, 64, 128)


def _cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("triune_amd kernels take HIP device tensors (device='cuda'); got a CPU tensor")


def fused_qkv_g_prep_inplace(qkv: torch.Tensor, g: torch.Tensor, cos=None, sin=None, use_rope: bool = True):
    """In-place pre-processing of qkv [B, T, 3, H, HD] and g [B, T, H, HD] (reference:
    attention.py:14-79, launched at :417-428).  cos/sin: [T, HD] (fp32 or the I/O dtype), used
    when use_rope.  Returns (qkv, g)."""
    _cuda(qkv, g, cos, sin)
    if qkv.dim() != 5 or qkv.shape[2] != 3 or g.dim() != 4:
        raise ValueError("qkv must be [B, T, 3, H, HD] and g [B, T, H, HD]")
    B, T, _, H, HD = qkv.shape
    if tuple(g.shape) != (B, T, H, HD):
        raise ValueError(f"g shape {tuple(g.shape)} does not match qkv {tuple(qkv.shape)}")
    if HD not in _HD:
        raise ValueError(f"head dim {HD} not supported (32, 64 or 128)")
    if g.dtype != qkv.dtype:
        raise TypeError("qkv and g must share a dtype")
    if qkv.stride(-1) != 1 or g.stride(-1) != 1:
        raise ValueError("the head dim must be contiguous")
    cs_st, cs_dt = 0, 0
    if use_rope:
        if cos is None or sin is None:
            raise ValueError("use_rope needs cos and sin")
        if tuple(cos.shape) != (T, HD) or tuple(sin.shape) != (T, HD) or cos.dtype != sin.dtype:
            raise ValueError("cos and sin must be [T, HD] of one dtype")
        if cos.stride(-1) != 1 or sin.stride() != cos.stride():
            raise ValueError("cos and sin must have contiguous rows with equal strides")
        cs_st, cs_dt = cos.stride(0), dtype_code(cos)
    st = strides(qkv.stride()[:4], g.stride()[:3])
    rc = lib().triune_hip_gla_qkvg_prep(
        ptr(qkv), ptr(g), dtype_code(qkv), st, ptr(cos) if use_rope else None, ptr(sin) if use_rope else None, cs_dt,
        cs_st, 1 if use_rope else 0, B, T, H, HD, stream_of(qkv),
    )
    check(rc, "triune_hip_gla_qkvg_prep")
    return qkv, g


def fused_qkvg_decode_step(qkvg: torch.Tensor, cos=None, sin=None, initial_state=None, save_final: bool = True,
                           use_rope: bool = True, state_dtype=None, out=None, inplace: bool = False):
    """One decode step fused with the pre-processing (reference: attention.py:81-179, launched at
    :396-415).  qkvg: [B, 4, H, HD]; cos/sin: [1, HD] or [HD] of the step's position;
    initial_state: [B, H, HD, HD] or None (zero).  The state is kept in state_dtype (default: the
    initial state's dtype, else qkvg.dtype, as the reference does; fp32 is also accepted).
    inplace=True writes the new state into initial_state (contiguous, of state_dtype) instead of a
    new tensor.  Returns (out [B, 1, H, HD] in qkvg.dtype, final state or None)."""
    _cuda(qkvg, cos, sin, initial_state)
    if qkvg.dim() != 4 or qkvg.shape[1] != 4:
        raise ValueError("qkvg must be [B, 4, H, HD]")
    B, _, H, HD = qkvg.shape
    if HD not in _HD:
        raise ValueError(f"head dim {HD} not supported (32, 64 or 128)")
    if qkvg.stride(-1) != 1:
        raise ValueError("the head dim of qkvg must be contiguous")
    if state_dtype is None:
        state_dtype = initial_state.dtype if initial_state is not None else qkvg.dtype
    if state_dtype not in (torch.float32, qkvg.dtype):
        raise TypeError("the state dtype must be float32 or the dtype of qkvg")
    s_in = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (B, H, HD, HD):
            raise ValueError(f"initial_state must be [B, H, HD, HD], got {tuple(initial_state.shape)}")
        s_in = initial_state.to(dtype=state_dtype).contiguous()
    if inplace:
        if s_in is None or s_in.data_ptr() != initial_state.data_ptr() or not save_final:
            raise ValueError("inplace needs a contiguous initial_state of state_dtype and save_final")
        s_out = s_in
    else:
        s_out = torch.empty(B, H, HD, HD, device=qkvg.device, dtype=state_dtype) if save_final else None
    cs_dt = 0
    if use_rope:
        if cos is None or sin is None:
            raise ValueError("use_rope needs cos and sin")
        cos, sin = cos.reshape(-1), sin.reshape(-1)
        if cos.numel() != HD or sin.numel() != HD or cos.dtype != sin.dtype:
            raise ValueError("cos and sin must hold HD values of one dtype")
        cos, sin = cos.contiguous(), sin.contiguous()
        cs_dt = dtype_code(cos)
    if out is None:
        out = torch.empty(B, 1, H, HD, device=qkvg.device, dtype=qkvg.dtype)
    if tuple(out.shape) != (B, 1, H, HD) or out.stride(-1) != 1:
        raise ValueError("out must be [B, 1, H, HD] with a contiguous head dim")
    ov = out[:, 0]
    st = strides(qkvg.stride()[:3])
    ost = strides(ov.stride()[:2])
    rc = lib().triune_hip_gla_fused_decode_step(
        ptr(qkvg), dtype_code(qkvg), st, ptr(cos) if use_rope else None, ptr(sin) if use_rope else None, cs_dt,
        1 if use_rope else 0, ptr(s_in), ptr(s_out), dtype_code(torch.empty(0, dtype=state_dtype)), ptr(ov),
        dtype_code(ov), ost, B, H, HD, stream_of(qkvg),
    )
    check(rc, "triune_hip_gla_fused_decode_step")
    return out, s_out
