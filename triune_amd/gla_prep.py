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
  fused_qkv_g_prep_chunk_gla(qkv, g, cos, sin, initial_state, out, save_final, use_rope)
      fused_qkv_g_prep_inplace followed by _triton_chunk_gla_tc_fwd(qkv[:, :, 0], qkv[:, :, 1],
      qkv[:, :, 2], g, initial_state, out=g), with the pre-processing done by the prefill's
      segment-state kernel as it reads q, k, g (same in-place results, one pass fewer).

normalize(a) = a / sqrt(max(sum a^2, 1e-12)) over the HD elements of a (token, head) row; RoPE
pairs element d with d + HD/2.  HD in {32, 64, 128}.  Tensors must be on the GPU; there is no CPU
path.
"""

from __future__ import annotations

import torch

from ._lib import check, dtype_code, lib, onepass_ctrl, ptr, stream_of, strides

__all__ = ["fused_qkv_g_prep_inplace", "fused_qkvg_decode_step", "fused_qkvg_decode_step_pool",
           "fused_qkv_g_prep_chunk_gla"]

_HD = (32, 64, 128)

# Calls that the single launch does not take run the pre-processing inside the segment-state
# kernel (triune_hip_gla_prefill_prep) only up to this many chunk-head workgroups per compute unit,
# and the pre-processing pass and then the prefill past it.  Both give the same results; the pass
# and the prefill measured faster at every size (B = 4, H = 6 on MI355X: T = 1024 with the single
# launch off 29.1 against 31.0 us, T = 2048 44.4 against 46.7 us, T = 4096 65.8 against 69.9 us,
# T = 16384 176 against 196 us), so 0: never.  Tests and the bench raise it to reach the other form.
FUSED_MAX_CHUNK_HEADS_PER_CU = 0


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


def fused_qkvg_decode_step_pool(qkvg: torch.Tensor, state_pool: torch.Tensor, slots: torch.Tensor, cos=None, sin=None,
                                use_rope: bool = True, out=None):
    """fused_qkvg_decode_step on rows of a state pool, in place (the decode half of serving with a
    device-resident session cache): state_pool [n_slots, H, HD, HD] contiguous, float32 or
    qkvg.dtype; slots: int32 [B] on the device, batch row b updating pool row slots[b].  A slot
    outside [0, n_slots) (a padded batch row) reads no state, stores none and outputs zeros.
    Returns the output [B, 1, H, HD] in qkvg.dtype."""
    _cuda(qkvg, cos, sin, state_pool, slots)
    if qkvg.dim() != 4 or qkvg.shape[1] != 4:
        raise ValueError("qkvg must be [B, 4, H, HD]")
    B, _, H, HD = qkvg.shape
    if HD not in _HD:
        raise ValueError(f"head dim {HD} not supported (32, 64 or 128)")
    if qkvg.stride(-1) != 1:
        raise ValueError("the head dim of qkvg must be contiguous")
    if state_pool.dim() != 4 or tuple(state_pool.shape[1:]) != (H, HD, HD) or not state_pool.is_contiguous():
        raise ValueError(f"state_pool must be a contiguous [n_slots, {H}, {HD}, {HD}] tensor")
    if state_pool.dtype not in (torch.float32, qkvg.dtype):
        raise TypeError("the state dtype must be float32 or the dtype of qkvg")
    if slots.dtype != torch.int32 or slots.dim() != 1 or slots.numel() != B:
        raise ValueError("slots must be an int32 [B] tensor")
    slots = slots.contiguous()
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
    rc = lib().triune_hip_gla_fused_decode_step_slots(
        ptr(qkvg), dtype_code(qkvg), strides(qkvg.stride()[:3]), ptr(cos) if use_rope else None,
        ptr(sin) if use_rope else None, cs_dt, 1 if use_rope else 0, ptr(state_pool), dtype_code(state_pool),
        ptr(slots), state_pool.shape[0], ptr(ov), dtype_code(ov), strides(ov.stride()[:2]), B, H, HD,
        stream_of(qkvg),
    )
    check(rc, "triune_hip_gla_fused_decode_step_slots")
    return out


def fused_qkv_g_prep_chunk_gla(qkv: torch.Tensor, g: torch.Tensor, cos=None, sin=None, initial_state=None, out=None,
                               save_final: bool = True, use_rope: bool = True):
    """VectorisedGLA's prefill (attention.py:425-451): _fused_qkv_g_prep_inplace_kernel, then
    _triton_chunk_gla_tc_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g, initial_state, out=g).
    triune_hip_gla_prefill_prep does the pre-processing inside the prefill's segment-state kernel:
    it reads the raw q, k, v, g once, writes q, k <- RoPE(normalize(elu(x) + 1)) and
    g <- logsigmoid(g) back in place (rounded to the I/O dtype, as the reference's prep kernel
    leaves them) and forms the segment states from those values; the output kernel then reads the
    processed tensors.

    Calls of at most 64 chunks per sequence whose chunk-head workgroups are all resident at once
    (head dim 64; B = 4, H = 6, T = 1024 is 384 of them, VectorisedGLA's prefill tile,
    attention.py:458-499) run everything in one launch, triune_hip_gla_prefill_onepass: each
    workgroup pre-processes its chunk pair, publishes the pair's local state, folds the earlier
    pairs' into the state it enters with and writes its outputs (19.8-20.4 us per call against
    29-31 us for the pre-processing pass and then the prefill).  Other calls run
    fused_qkv_g_prep_inplace and then the prefill, with the same results: the pre-processing inside
    the segment-state kernel (triune_hip_gla_prefill_prep, used while B * H * ceil(T / 64) is at
    most FUSED_MAX_CHUNK_HEADS_PER_CU per compute unit) measured slower at every size, its VALU work
    weighing more inside the chunk kernel's dependent chain than as a bandwidth-bound pass.

    qkv: [B, T, 3, H, HD] raw projections (bf16 or fp16), g: [B, T, H, HD] raw gate (same dtype),
    cos/sin: [T, HD] (used when use_rope; converted to fp32 if needed), initial_state: [B, H, HD,
    HD] or None.  out: [B, T, H, HD] output buffer (default: g's buffer, as the reference writes
    the outputs over g).  HD in {32, 64, 128}.  Returns (out, final state fp32 [B, H, HD, HD], or a
    1-element placeholder when save_final is False, as the reference)."""
    _cuda(qkv, g, cos, sin, initial_state, out)
    if qkv.dim() != 5 or qkv.shape[2] != 3 or g.dim() != 4:
        raise ValueError("qkv must be [B, T, 3, H, HD] and g [B, T, H, HD]")
    B, T, _, H, HD = qkv.shape
    if tuple(g.shape) != (B, T, H, HD):
        raise ValueError(f"g shape {tuple(g.shape)} does not match qkv {tuple(qkv.shape)}")
    if HD not in _HD:
        raise ValueError(f"head dim {HD} not supported (32, 64 or 128)")
    if qkv.dtype not in (torch.bfloat16, torch.float16) or g.dtype != qkv.dtype:
        raise TypeError("qkv and g must share one 16-bit dtype (bfloat16 or float16)")
    from .fast_gla import _tok3, _triton_chunk_gla_tc_fwd, _vec_layout

    from . import fast_gla as _fg

    L = lib()
    onepass = _fg.ONEPASS and HD == 64 and bool(
        L.triune_hip_gla_prefill_onepass_supported(B, T, H, HD, dtype_code(qkv), dtype_code(qkv), 1, 0))
    cus = torch.cuda.get_device_properties(qkv.device).multi_processor_count
    if not onepass and B * H * ((T + 63) // 64) > FUSED_MAX_CHUNK_HEADS_PER_CU * cus:
        fused_qkv_g_prep_inplace(qkv, g, cos, sin, use_rope=use_rope)
        return _triton_chunk_gla_tc_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g, initial_state=initial_state,
                                        out=g if out is None else out, save_final=save_final)
    views = [qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g]
    q, k, v, gp = (_vec_layout(x, 1) for x in views)  # copies only for unaligned layouts
    if out is None:
        out = g
    if tuple(out.shape) != (B, T, H, HD):
        raise ValueError("out must be [B, T, H, HD]")
    o = out if _vec_layout(out, 1) is out else torch.empty(B, T, H, HD, device=qkv.device, dtype=out.dtype)
    cs_st = 0
    if use_rope:
        if cos is None or sin is None:
            raise ValueError("use_rope needs cos and sin")
        if tuple(cos.shape) != (T, HD) or tuple(sin.shape) != (T, HD):
            raise ValueError("cos and sin must be [T, HD]")
        cos, sin = (_vec_layout(x.to(torch.float32), 0) for x in (cos, sin))
        if cos.stride(0) != sin.stride(0):
            sin = sin.contiguous()
            cos = cos.contiguous()
        cs_st = cos.stride(0)
    s0 = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    sf = torch.empty(B, H, HD, HD, device=qkv.device, dtype=torch.float32) if save_final else None
    st = strides(_tok3(q), _tok3(k), _tok3(v), _tok3(gp), _tok3(o))
    if onepass:  # pre-processing, states and outputs in one launch
        ws = torch.empty(int(L.triune_hip_gla_prefill_onepass_workspace_size(B, T, H, HD)), device=qkv.device,
                         dtype=torch.uint8)
        ctrl = onepass_ctrl(qkv.device, int(L.triune_hip_gla_prefill_onepass_ctrl_size(B, T, H, HD)))
        rc = L.triune_hip_gla_prefill_onepass(
            ptr(q), ptr(k), ptr(v), ptr(gp), dtype_code(q), dtype_code(gp), st, ptr(cos) if use_rope else None,
            ptr(sin) if use_rope else None, cs_st, 1, 1 if use_rope else 0, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, HD, 0, ptr(ws), ws.numel(), ptr(ctrl), ctrl.numel(), stream_of(qkv),
        )
        check(rc, "triune_hip_gla_prefill_onepass")
    else:
        wsb = L.triune_hip_gla_prefill_workspace_size(B, T, H, HD, HD, 0)
        ws = torch.empty(max(int(wsb), 256), device=qkv.device, dtype=torch.uint8)
        rc = L.triune_hip_gla_prefill_prep(
            ptr(q), ptr(k), ptr(v), ptr(gp), dtype_code(q), st, ptr(cos) if use_rope else None,
            ptr(sin) if use_rope else None, cs_st, 1 if use_rope else 0, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, HD, ptr(ws), ws.numel(), stream_of(qkv),
        )
        check(rc, "triune_hip_gla_prefill_prep")
    for dst, src in zip(views, (q, k, v, gp)):  # the in-place results reach copied inputs too
        if src is not dst and not (src is gp and o.data_ptr() == gp.data_ptr()):
            dst.copy_(src)
    if o is not out:
        out.copy_(o)
    if sf is None:
        sf = torch.empty((1,), device=qkv.device, dtype=torch.float32)
    return out, sf
