"""GPU parity of the chunked GLA backward (triune_hip_gla_prefill_bwd) against the fp64 oracle.

The reference differentiates fast_chunk_gla's PyTorch chunk path (fast_gla.py:569-689, with
FusedRecurrentScan's backward) and checks it against autograd through the token recurrence
(tests/test_kernels.py:266-327, HD = 16, chunk_size = 32, g in [-2.05, -0.05], every gradient and
the initial state's).  The oracle (oracle/gla_oracle.c, pinned in tests/test_oracle.py against
torch autograd and finite differences) computes the same gradients in fp64 from the same inputs.

Tolerances: fp32 inputs, max-abs 1e-5 relative to the gradient's largest magnitude (at least 1);
bf16 / fp16 inputs with fp32 gradients written by the kernel, 2e-3 on the same scale; bf16
gradients within one bf16 ULP of the oracle plus that.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import _lib, fast_chunk_gla, gla
from triune_amd.fast_gla import _prefill_bwd
from triune_amd.workloads import gla_inputs, ulp_bf16

pytestmark = pytest.mark.gpu


def _rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    err = float(np.abs(got.detach().double().cpu().numpy() - ref).max()) if ref.size else 0.0
    return err / max(1.0, float(np.abs(ref).max()) if ref.size else 1.0)


def _upstream(B, T, H, Dk, Dv, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, H, Dv, generator=gen), torch.randn(B, H, Dk, Dv, generator=gen)


@pytest.mark.parametrize("T", [1, 17, 32, 70, 128])
@pytest.mark.parametrize("with_init", [False, True])
def test_reference_gradient_case_fp32(dev, T, with_init):
    """The reference's own gradient check (test_kernels.py:266-327): fp32, B=2, H=4, HD=16,
    chunk_size=32, g = -2*rand - 0.05 (most chunks exceed the factored span: token-wise path)."""
    torch.manual_seed(42 + T)
    B, H, HD = 2, 4, 16
    q, k, v = (torch.randn(B, T, H, HD) for _ in range(3))
    g = -torch.rand(B, T, H, HD) * 2.0 - 0.05
    s0 = torch.randn(B, H, HD, HD) if with_init else None
    do, ds = _upstream(B, T, H, HD, HD, T)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    s0d = s0.to(dev).requires_grad_(True) if with_init else None
    o, s = fast_chunk_gla(*xs, initial_state=s0d, chunk_size=32)
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds, chunk=32)
    for x, r in zip(xs, ref[:4]):
        assert x.grad.dtype == torch.float32
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)
    if with_init:
        assert _rel_err(s0d.grad, ref[4]) <= 1e-5


@pytest.mark.parametrize("T", [64, 200, 1100])
@pytest.mark.parametrize("D", [32, 64])
def test_bf16_fast_path_fp32_gradients(dev, T, D):
    """C1-like inputs (g = logsigmoid(randn)/16: every chunk on the factored MFMA path), bf16 I/O,
    fp32 gradients written by the kernel; several segments at T = 1100."""
    q, k, v, g, s0 = gla_inputs(2, T, 3, D, seed=T + D, dtype=torch.bfloat16, init_std=0.1)
    do, ds = _upstream(2, T, 3, D, D, T)
    do = do.bfloat16()
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    dq, dk, dv, dg, ds0 = _prefill_bwd(qd, kd, vd, gd, s0.to(dev), do.to(dev), ds.to(dev), 0,
                                       grad_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for got, r in zip((dq, dk, dv, dg, ds0), ref):
        assert _rel_err(got, r) <= 2e-3, _rel_err(got, r)


def test_bf16_gradients_within_one_ulp(dev):
    """Autograd path with bf16 inputs: gradients come back in bf16, each within one bf16 ULP of
    the oracle plus the fp32-mode tolerance."""
    B, T, H, D = 2, 300, 2, 64
    q, k, v, g, s0 = gla_inputs(B, T, H, D, seed=5, dtype=torch.bfloat16, init_std=0.1)
    do, ds = _upstream(B, T, H, D, D, 5)
    do = do.bfloat16()
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    o, s = fast_chunk_gla(*xs, initial_state=s0.to(dev))
    ((o.float() * do.float().to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for x, r in zip(xs, ref[:4]):
        assert x.grad.dtype == torch.bfloat16
        rt = torch.from_numpy(r)
        scale = max(1.0, float(rt.abs().max()))
        excess = (x.grad.double().cpu() - rt).abs() - (ulp_bf16(rt).double() + 2e-3 * scale)
        assert float(excess.max()) <= 0.0, float(excess.max())


def test_mixed_tokenwise_and_fast_chunks_with_tail_and_positive_gates(dev):
    """One sequence mixes factored chunks, token-wise chunks (decay span > 64 nats), positive
    gates (clamped: zero gradient) and the reference's unclamped 1-token tail (T % 64 == 1)."""
    B, T, H, D = 2, 321, 2, 32
    q, k, v, g, s0 = gla_inputs(B, T, H, D, seed=13, dtype=torch.float32, init_std=0.3)
    gen = torch.Generator().manual_seed(2)
    g = g.clone()
    g[:, 64:128] = -1.0 - 20.0 * torch.rand(B, 64, H, D, generator=gen)
    g[:, 200:210, :, :4] = 0.3
    g[:, -1] = 0.25
    do, ds = _upstream(B, T, H, D, D, 7)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    s0d = s0.to(dev).requires_grad_(True)
    o, s = fast_chunk_gla(*xs, initial_state=s0d)
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for x, r in zip(xs + [s0d], ref):
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)
    assert float(xs[3].grad[:, 200:210, :, :4].abs().max()) == 0.0  # clamped positive gates
    assert float(xs[3].grad[:, -1].abs().max()) > 0.0  # the unclamped tail passes its gradient


def test_unequal_head_dims_and_missing_upstream(dev):
    """Dk = 16, Dv = 24 (zero-padded to 32); only the output is used (no final-state gradient)
    and no initial state."""
    B, T, H = 1, 150, 3
    gen = torch.Generator().manual_seed(3)
    q, k = torch.randn(2, B, T, H, 16, generator=gen)
    v = torch.randn(B, T, H, 24, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, 16, generator=gen)) / 8
    do = torch.randn(B, T, H, 24, generator=gen)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    o, _ = gla(*xs)
    (o * do.to(dev)).sum().backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, None, do, None)
    for x, r in zip(xs, ref[:4]):
        assert tuple(x.grad.shape) == tuple(x.shape)
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)


def test_fp16_inputs(dev):
    q, k, v, g, s0 = gla_inputs(1, 257, 2, 64, seed=21, dtype=torch.float16, init_std=0.1)
    do, ds = _upstream(1, 257, 2, 64, 64, 21)
    do = do.half()
    dq, dk, dv, dg, ds0 = _prefill_bwd(*(x.to(dev) for x in (q, k, v, g, s0, do, ds)), _lib.FLAG_TAIL_UNCLAMPED,
                                       grad_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for got, r in zip((dq, dk, dv, dg, ds0), ref):
        assert _rel_err(got, r) <= 2e-3, _rel_err(got, r)


def test_backward_matches_finite_difference_of_forward_kernel(dev):
    """Directional derivative of the HIP forward (fp32, central difference) equals the HIP
    backward's gradient contracted with the same direction."""
    B, T, H, D = 1, 96, 2, 32
    q, k, v, g, s0 = gla_inputs(B, T, H, D, seed=17, dtype=torch.float32, init_std=0.2)
    do, ds = _upstream(B, T, H, D, D, 17)
    args = [x.to(dev).double() for x in (q, k, v, g)]
    gen = torch.Generator().manual_seed(8)
    dirs = [torch.randn(x.shape, generator=gen).to(dev).double() for x in args]
    dirs[3] = dirs[3] * 0.01
    eps = 1e-3

    def loss(sign):
        xs = [(x + sign * eps * d).float() for x, d in zip(args, dirs)]
        o, s = fast_chunk_gla(*xs, initial_state=s0.to(dev))
        return float((o.double() * do.to(dev).double()).sum() + (s.double() * ds.to(dev).double()).sum())

    fd = (loss(1) - loss(-1)) / (2 * eps)
    xs = [x.float().requires_grad_(True) for x in args]
    o, s = fast_chunk_gla(*xs, initial_state=s0.to(dev))
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    an = sum(float((x.grad.double() * d).sum()) for x, d in zip(xs, dirs))
    assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (fd, an)


@pytest.mark.parametrize("T", [63, 64, 65, 256])
@pytest.mark.parametrize("with_init", [False, True])
def test_chunk_boundary_lengths_fp32(dev, T, with_init):
    """The lengths of the reference's fallback gradient check (test_attention_fallback.py:42-85:
    T in {1, 63, 64, 65, 128, 256}, outputs, states and every gradient) at chunk_size 64, where
    T = 65 ends in the unclamped one-token tail."""
    gen = torch.Generator().manual_seed(T + 7 * with_init)
    B, H, D = 2, 3, 32
    q, k, v = (torch.randn(B, T, H, D, generator=gen) for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)) / 4
    s0 = torch.randn(B, H, D, D, generator=gen) if with_init else None
    do, ds = _upstream(B, T, H, D, D, T + 1)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    s0d = s0.to(dev).requires_grad_(True) if with_init else None
    o, s = fast_chunk_gla(*xs, initial_state=s0d, chunk_size=64)
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds, chunk=64)
    for x, r in zip(xs + ([s0d] if with_init else []), ref):
        assert _rel_err(x.grad, r) <= 1e-5, (T, _rel_err(x.grad, r))


@pytest.mark.parametrize("use", ["final_only", "out_only"])
def test_bf16_extreme_decay_gradient_flow(dev, use):
    """bf16 inputs with gates in [-21, -1] (the reference's extreme-decay gradient case,
    test_kernels.py:399-434): every gradient finite and equal to the oracle's, with only the
    final state or only the output used."""
    gen = torch.Generator().manual_seed(3 if use == "final_only" else 4)
    B, T, H, D = 2, 200, 2, 64
    q, k, v = (torch.randn(B, T, H, D, generator=gen).bfloat16() for _ in range(3))
    g = (-1.0 - 20.0 * torch.rand(B, T, H, D, generator=gen)).bfloat16()
    do, ds = _upstream(B, T, H, D, D, 9)
    do = do.bfloat16()
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    o, s = fast_chunk_gla(*xs)
    loss = (s * ds.to(dev)).sum() if use == "final_only" else (o.float() * do.float().to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, None, do if use == "out_only" else None, ds if use == "final_only" else None)
    for x, r in zip(xs, ref[:4]):
        assert bool(torch.isfinite(x.grad).all())
        rt = torch.from_numpy(r)
        scale = max(1.0, float(rt.abs().max()))
        excess = (x.grad.double().cpu() - rt).abs() - (ulp_bf16(rt).double() + 2e-3 * scale)
        assert float(excess.max()) <= 0.0, float(excess.max())


# --- heads wider than the gradient kernels hold: block decomposition --------------------------
@pytest.mark.parametrize("T", [130, 700])
def test_bf16_head_dim_128_gradients(dev, T):
    """The default model's head size (GLA_HEAD_DIM = 128, triune/model/config.py:21): gradients
    as sums over 64-wide key / value blocks, fp32 gradients at the 2e-3 bar, and through autograd
    in bf16 within one ULP plus that."""
    B, H, D = 2, 2, 128
    q, k, v, g, s0 = gla_inputs(B, T, H, D, seed=T, dtype=torch.bfloat16, init_std=0.1)
    do, ds = _upstream(B, T, H, D, D, T)
    do = do.bfloat16()
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    got = _prefill_bwd(qd, kd, vd, gd, s0.to(dev), do.to(dev), ds.to(dev), 0, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "ds0"), got, ref):
        e = _rel_err(x, r)
        print(f"D=128 T={T} {name}: {e:.3e}", flush=True)
        assert e <= 2e-3, (name, e)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    o, s = fast_chunk_gla(*xs, initial_state=s0.to(dev))
    ((o.float() * do.float().to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    for x, r in zip(xs, ref[:4]):
        assert x.grad.dtype == torch.bfloat16
        rt = torch.from_numpy(r)
        scale = max(1.0, float(rt.abs().max()))
        excess = (x.grad.double().cpu() - rt).abs() - (ulp_bf16(rt).double() + 2e-3 * scale)
        assert float(excess.max()) <= 0.0, float(excess.max())


@pytest.mark.parametrize("Dk,Dv", [(64, 64), (48, 80), (128, 64)])
def test_fp32_wide_heads_gradients(dev, Dk, Dv):
    """fp32 inputs beyond the 32-wide fp32 kernels (including unequal and non-multiple head
    dims): gradients at the fp32 bar against the oracle."""
    B, T, H = 2, 150, 2
    gen = torch.Generator().manual_seed(Dk + Dv)
    q = torch.randn(B, T, H, Dk, generator=gen) * Dk**-0.5
    k = torch.randn(B, T, H, Dk, generator=gen)
    v = torch.randn(B, T, H, Dv, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, Dk, generator=gen)) / 16
    s0 = 0.1 * torch.randn(B, H, Dk, Dv, generator=gen)
    do, ds = _upstream(B, T, H, Dk, Dv, Dk)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    s0d = s0.to(dev).requires_grad_(True)
    o, s = fast_chunk_gla(*xs, initial_state=s0d)
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gla_bwd(q, k, v, g, s0, do, ds)
    for name, x, r in zip(("dq", "dk", "dv", "dg"), xs, ref[:4]):
        e = _rel_err(x.grad, r)
        print(f"fp32 ({Dk},{Dv}) {name}: {e:.3e}", flush=True)
        assert x.grad.dtype == torch.float32 and e <= 1e-5, (name, e)
    assert _rel_err(s0d.grad, ref[4]) <= 1e-5
