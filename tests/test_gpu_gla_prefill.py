"""GPU parity of the chunked GLA prefill (libtriune_hip.so) against the fp64 oracle.

Protocol for 16-bit I/O (the tolerance cannot hold on a bf16 output tensor: one bf16 rounding of
an O(20) output is ~0.06): the kernel writes fp32 outputs (same code path, fp32 store) and the
outputs and final states must be within max-abs 2e-3 of the oracle; with bf16 outputs every
element must be within one bf16 ULP of the oracle plus that 2e-3.  fp32 I/O: max-abs 1e-5.
The oracle consumes the same (already rounded) inputs as the kernel.
"""

import pytest
import torch

from oracle import oracle as O
from triune_amd import _lib, fast_chunk_gla
from triune_amd.fast_gla import _prefill, _triton_chunk_gla_tc_fwd
from triune_amd.workloads import config0, gla_inputs, ulp_bf16

pytestmark = pytest.mark.gpu

TOL16 = 2e-3  # bf16 / fp16 I/O, fp32 accumulation and outputs
TOL32 = 1e-5  # fp32 I/O


@pytest.fixture(autouse=True, params=["onepass", "three_launch"])
def prefill_path(request, monkeypatch):
    """Every case on both dense paths: calls of few chunks (head dim 64, 16-bit I/O) take the
    single-launch prefill unless it is switched off."""
    import triune_amd.fast_gla as FG

    monkeypatch.setattr(FG, "ONEPASS", request.param == "onepass")
    return request.param


def _run(q, k, v, g, s0, dev, out_dtype=torch.float32, **kw):
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    out = torch.empty(v.shape, device=dev, dtype=out_dtype)
    o, s = fast_chunk_gla(qd, kd, vd, gd, initial_state=None if s0 is None else s0.to(dev), out=out, **kw)
    torch.cuda.synchronize()
    return o.cpu().double(), s.cpu().double()


def _err(a, b):
    return float((a - torch.as_tensor(b)).abs().max())


def _assert_bf16_close(o_bf16, ref):
    """bf16 outputs: within one bf16 ULP of the oracle, plus the fp32-mode tolerance (which
    dominates near zero, where a bf16 ULP is far below the accumulated fp32 error)."""
    ref = torch.as_tensor(ref).double()
    excess = (o_bf16.double() - ref).abs() - (ulp_bf16(ref).double() + TOL16)
    assert float(excess.max()) <= 0.0, float(excess.max())


def test_config0_fp32_full(dev):
    q, k, v, g, s0 = config0()
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL32, _err(o, ro)
    assert _err(s, rs) <= TOL32, _err(s, rs)


@pytest.mark.parametrize("T", [2048, 4096])
def test_config1_shape_bf16(dev, T):
    q, k, v, g, s0 = gla_inputs(2, T, 3, 64, seed=11, dtype=torch.bfloat16, init_std=0.1)
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16, _err(o, ro)
    assert _err(s, rs) <= TOL16, _err(s, rs)
    # production mode: bf16 outputs within 1 ULP of the oracle
    ob, sb = _run(q, k, v, g, s0, dev, out_dtype=torch.bfloat16)
    _assert_bf16_close(ob, ro)
    assert _err(sb, rs) <= TOL16


@pytest.mark.parametrize("T", [1, 2, 17, 63, 64, 65, 127, 128, 129, 200, 320])
@pytest.mark.parametrize("with_init", [False, True])
def test_ragged_lengths(dev, T, with_init):
    q, k, v, g, s0 = gla_inputs(2, T, 2, 64, seed=100 + T, dtype=torch.bfloat16, init_std=0.5 if with_init else 0)
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16, (T, _err(o, ro))
    assert _err(s, rs) <= TOL16, (T, _err(s, rs))


@pytest.mark.parametrize("T,chunk", [(65, 64), (129, 64), (33, 32), (97, 32), (70, 32), (64, 64), (1, 64)])
def test_positive_gates_follow_reference_dispatch(dev, T, chunk):
    """g > 0 exposes the reference's clamp rules: prefill clamps, T == 1 and a 1-token
    remainder after whole chunks do not (fast_gla.py:586, :746-753, :768-775).  Magnitudes as in
    config 0 (q scaled by D^-1/2, S0 of std 0.1), so outputs stay O(1-10) and 1e-5 absolute is
    a meaningful fp32 bar (with unscaled q and S0 outputs reach |o| ~ 120, where 1e-5 is about one
    fp32 ULP)."""
    gen = torch.Generator().manual_seed(T * 7 + chunk)
    q = torch.randn(1, T, 2, 32, generator=gen) * 32**-0.5
    k = torch.randn(1, T, 2, 32, generator=gen)
    v = torch.randn(1, T, 2, 32, generator=gen)
    g = 0.05 * torch.randn(1, T, 2, 32, generator=gen)
    s0 = 0.1 * torch.randn(1, 2, 32, 32, generator=gen)
    o, s = _run(q, k, v, g, s0, dev, chunk_size=chunk)
    ro, rs = O.gla_fwd(q, k, v, g, s0, chunk=chunk, clamp_mode=2)
    print(f"T={T} chunk={chunk}: o {_err(o, ro):.3e} S {_err(s, rs):.3e} (max |o| {abs(ro).max():.1f})")
    assert _err(o, ro) <= TOL32, _err(o, ro)
    assert _err(s, rs) <= TOL32, _err(s, rs)


@pytest.mark.parametrize("Dk,Dv", [(16, 16), (32, 32), (128, 128), (64, 128), (128, 64), (8, 8), (48, 48)])
def test_head_dims(dev, Dk, Dv):
    q, k, v, g, s0 = gla_inputs(1, 300, 2, Dk, seed=Dk + Dv, dtype=torch.bfloat16, init_std=0.1, Dv=Dv)
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16, _err(o, ro)
    assert _err(s, rs) <= TOL16, _err(s, rs)


@pytest.mark.parametrize("seg", [1, 2, 3, 7])
def test_segment_sizes_agree(dev, seg):
    """The result does not depend on how many chunks a work item walks."""
    q, k, v, g, s0 = gla_inputs(2, 1000, 3, 64, seed=5, dtype=torch.bfloat16, init_std=0.1)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = _prefill(qd, kd, vd, gd, s0.to(dev), out, seg << _lib.FLAG_SEG_SHIFT)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o.cpu().double(), ro) <= TOL16
    assert _err(s.cpu().double(), rs) <= TOL16


def test_extreme_decay_tokenwise_chunks(dev):
    """Decay spans beyond the factored range run token by token inside the same kernel;
    mixed with ordinary chunks (reference extreme-decay case: g in [-21, -1], test_kernels.py:399-434)."""
    q, k, v, g, s0 = gla_inputs(2, 256, 2, 64, seed=9, dtype=torch.float32, init_std=0.3)
    g = g.clone()
    g[:, 64:128] = -1.0 - 20.0 * torch.rand(2, 64, 2, 64, generator=torch.Generator().manual_seed(1))
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    print(f"extreme decay: o {_err(o, ro):.3e} S {_err(s, rs):.3e}")
    assert _err(o, ro) <= TOL32, _err(o, ro)
    assert _err(s, rs) <= TOL32, _err(s, rs)


@pytest.mark.parametrize("T", [200, 256])
def test_gate_broadcast_along_tokens(dev, T):
    """g expanded along T (token stride 0, as a per-head constant gate would be passed): the
    rows overlap, so the host copies them; T % 4 == 0 takes the unchecked-row kernels."""
    q, k, v, g, s0 = gla_inputs(2, T, 3, 64, seed=T + 1, dtype=torch.bfloat16, init_std=0.1)
    gb = g[:, :1].expand(2, T, 3, 64)
    assert gb.stride(1) == 0
    qd, kd, vd = (x.to(dev) for x in (q, k, v))
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = fast_chunk_gla(qd, kd, vd, g[:, :1].to(dev).expand(2, T, 3, 64), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(q, k, v, gb, s0)
    assert _err(o.cpu().double(), ro) <= TOL16 and _err(s.cpu().double(), rs) <= TOL16


@pytest.mark.parametrize("T", [200, 1000])
def test_fp32_partial_last_chunk(dev, T):
    """fp32 I/O with T % 4 == 0 but T % 64 != 0: the unchecked-row instances with a partial last
    chunk, at the fp32 bar."""
    q, k, v, g, s0 = gla_inputs(2, T, 2, 64, seed=T, dtype=torch.float32, init_std=0.1)
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL32, _err(o, ro)
    assert _err(s, rs) <= TOL32, _err(s, rs)


def test_fp16_io(dev):
    q, k, v, g, s0 = gla_inputs(1, 500, 2, 64, seed=21, dtype=torch.float16, init_std=0.1)
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16 and _err(s, rs) <= TOL16


def test_fp32_gate_with_bf16_qkv(dev):
    q, k, v, g, s0 = gla_inputs(1, 400, 2, 64, seed=22, dtype=torch.bfloat16, init_std=0.1)
    g = g.float() + 1e-3 * torch.rand(g.shape, generator=torch.Generator().manual_seed(3)) * -1
    o, s = _run(q, k, v, g, s0, dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16 and _err(s, rs) <= TOL16


def test_strided_qkv_views_and_out_aliasing_g(dev):
    """VectorisedGLA passes qkv[:, :, i] views and out=g (attention.py:443-451)."""
    B, T, H, D = 2, 384, 3, 64
    gen = torch.Generator().manual_seed(4)
    qkv = torch.randn(B, T, 3, H, D, generator=gen).bfloat16()
    qkv[:, :, 0] *= D**-0.5
    g = (torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)) / 16).bfloat16()
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    ro, rs = O.gla_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g, s0)
    qkv_d, g_d = qkv.to(dev), g.to(dev)
    o, s = _triton_chunk_gla_tc_fwd(qkv_d[:, :, 0], qkv_d[:, :, 1], qkv_d[:, :, 2], g_d, initial_state=s0.to(dev), out=g_d)
    torch.cuda.synchronize()
    assert o.data_ptr() == g_d.data_ptr()
    _assert_bf16_close(o.cpu(), ro)
    assert _err(s.cpu().double(), rs) <= TOL16
    o2, s2 = _triton_chunk_gla_tc_fwd(qkv_d[:, :, 0], qkv_d[:, :, 1], qkv_d[:, :, 2], g.to(dev), save_final=False)
    assert s2.numel() == 1


@pytest.mark.parametrize("D", [64, 128])
def test_out_aliasing_g_with_tokenwise_chunks(dev, D):
    """out = g while some chunks run token by token (decay span past the factored range) and the
    sequence ends in the reference's 1-token tail (T = 64k + 1): every gate read of a token must
    land before any wave stores that token's output over it."""
    B, T, H = 2, 257, 2
    gen = torch.Generator().manual_seed(17 + D)
    qkv = torch.randn(B, T, 3, H, D, generator=gen).bfloat16()
    qkv[:, :, 0] *= D**-0.5
    g = (torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)) / 16).float()
    g[:, 64:128] = -1.0 - 20.0 * torch.rand(B, 64, H, D, generator=gen)
    g = g.bfloat16()
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    ro, rs = O.gla_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], g, s0)
    qkv_d, g_d = qkv.to(dev), g.to(dev)
    o, s = _triton_chunk_gla_tc_fwd(qkv_d[:, :, 0], qkv_d[:, :, 1], qkv_d[:, :, 2], g_d, initial_state=s0.to(dev), out=g_d)
    torch.cuda.synchronize()
    assert o.data_ptr() == g_d.data_ptr()
    _assert_bf16_close(o.cpu(), ro)
    assert _err(s.cpu().double(), rs) <= TOL16


def test_chunked_prefill_equals_full_prefill(dev):
    """Prefill in slices with a carried fp32 state == one prefill (test_long_context_performance.py:71-107)."""
    q, k, v, g, s0 = gla_inputs(2, 1100, 2, 64, seed=31, dtype=torch.bfloat16, init_std=0.1)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    full, sf = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0.to(dev), out=torch.empty(v.shape, device=dev))
    st = s0.to(dev)
    outs = []
    for a, b in [(0, 512), (512, 1024), (1024, 1100)]:
        o, st = fast_chunk_gla(qd[:, a:b], kd[:, a:b], vd[:, a:b], gd[:, a:b], initial_state=st,
                               out=torch.empty(v[:, a:b].shape, device=dev))
        outs.append(o)
    torch.cuda.synchronize()
    assert float((torch.cat(outs, 1) - full).abs().max()) <= TOL16
    assert float((st - sf).abs().max()) <= TOL16


def test_zero_length_returns_initial_state(dev):
    s0 = torch.randn(2, 2, 64, 64, device=dev)
    z = torch.zeros(2, 0, 2, 64, device=dev, dtype=torch.bfloat16)
    o, s = fast_chunk_gla(z, z, z, z, initial_state=s0)
    torch.cuda.synchronize()
    assert o.shape == (2, 0, 2, 64)
    assert torch.equal(s, s0)


def test_cpu_tensors_rejected():
    q = torch.zeros(1, 4, 1, 64)
    with pytest.raises(ValueError):
        fast_chunk_gla(q, q, q, q)
