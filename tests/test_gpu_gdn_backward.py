"""GPU parity of the Gated DeltaNet backward (triune_hip_gdn_bwd) against the fp64 oracle.

The reference differentiates fast_recurrent_gated_deltanet (fast_gla.py:781-836) with autograd
whenever a gradient is needed (fast_chunk_gated_deltanet, fast_gla.py:885-904) and checks that the
gradients exist and are finite (tests/test_gated_deltanet_and_advancements.py:22-43: B=2, T=16,
H=4, HD=32, g = -rand).  oracle.gdn_bwd (oracle/gla_oracle.c, pinned in tests/test_oracle.py
against torch autograd of the reference loop and finite differences) computes the same gradients
in fp64 from the same inputs.

Inputs follow config 3 (q, k L2-normalised, beta = sigmoid, g = logsigmoid / 8, some g exactly 0
and some positive, where the clamp passes no gradient).  Tolerances: fp32 inputs, max-abs 1e-5
relative to the gradient's largest magnitude (at least 1); bf16 inputs (gradients in bf16), each
element within one bf16 ULP of the oracle plus 2e-3 on the same scale.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from triune_amd import _lib, fast_chunk_gated_deltanet, fast_recurrent_gated_deltanet
from triune_amd.fast_gla import _gdn_bwd
from triune_amd.workloads import ulp_bf16

pytestmark = pytest.mark.gpu

KINDS = {"none": _lib.BETA_NONE, "head": _lib.BETA_HEAD, "key": _lib.BETA_KEY, "value": _lib.BETA_VALUE}


def _inputs(B, T, H, D, kind, seed, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    v = torch.randn(B, T, H, D, generator=gen)
    g = F.logsigmoid(torch.randn(B, T, H, D, generator=gen) + 2.0) / 8
    g[:, ::5, :, :2] = 0.0  # on the clamp's edge: the gradient passes
    g[:, 1::7, :, 2:4] = 0.05  # clamped: no gradient
    beta = None
    if kind == "head":
        beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    elif kind in ("key", "value"):
        beta = torch.sigmoid(torch.randn(B, T, H, D, generator=gen))
    s0 = 0.2 * torch.randn(B, H, D, D, generator=gen)
    do = torch.randn(B, T, H, D, generator=gen)
    ds = torch.randn(B, H, D, D, generator=gen)
    cast = lambda x: None if x is None else x.to(dtype)
    return cast(q), cast(k), cast(v), cast(g), cast(beta), s0, cast(do), ds


def _rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    err = float(np.abs(got.detach().double().cpu().numpy() - ref).max())
    return err / max(1.0, float(np.abs(ref).max()))


def _ulp_excess(got, ref):
    """Largest |got - ref| beyond one bf16 ULP of ref, relative to max(1, max|ref|)."""
    r = torch.as_tensor(np.asarray(ref, dtype=np.float64))
    d = (got.detach().double().cpu() - r).abs() - ulp_bf16(r.float()).double()
    return float(d.clamp_min(0).max()) / max(1.0, float(r.abs().max())) if r.numel() else 0.0


def _oracle(q, k, v, g, beta, s0, do, ds, kind):
    return O.gdn_bwd(q, k, v, g, beta, s0, do, ds, beta_kind=KINDS[kind] if beta is not None and beta.dim() == 4 else None)


@pytest.mark.parametrize("kind", ["none", "head", "key", "value"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [1, 7, 16, 17, 33, 100])
def test_gdn_bwd_fp32(dev, kind, D, T):
    """Every gradient (q, k, v, g, beta, initial state) through the C-ABI entry, fp32, sub-chunk
    tails.  B * H = 6 leaves room for segments walked in parallel: 8 tokens per sub-chunk at D = 64
    (4 at 128); beta per value column walks one segment of 32-token (16 at 128) sub-chunks."""
    B, H = 2, 3
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, kind, seed=T * 7 + D)
    args = [x.to(dev) if x is not None else None for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), KINDS[kind], do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    ref = _oracle(q, k, v, g, beta, s0, do, ds, kind)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    for name, x, r in zip(names, got, ref):
        if r is None:
            assert x is None
            continue
        assert tuple(x.shape) == r.shape, name
        e = _rel_err(x, r)
        assert e <= 1e-5, (name, e)


@pytest.mark.parametrize("kind", ["none", "head", "key", "value"])
def test_gdn_bwd_bf16_within_one_ulp(dev, kind):
    """bf16 inputs: gradients come back in bf16, each within one bf16 ULP of the oracle plus 2e-3."""
    B, T, H, D = 2, 150, 2, 64
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, kind, seed=11, dtype=torch.bfloat16)
    args = [x.to(dev) if x is not None else None for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), KINDS[kind], do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    ref = _oracle(q, k, v, g, beta, s0, do, ds, kind)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), got[:5], ref[:5]):
        if r is None:
            continue
        assert x.dtype == torch.bfloat16, name
        assert _ulp_excess(x, r) <= 2e-3, (name, _ulp_excess(x, r))
    assert _rel_err(got[5], ref[5]) <= 2e-3


def test_reference_gradient_case(dev):
    """The reference's own check (test_gated_deltanet_and_advancements.py:22-43): B=2, T=16, H=4,
    HD=32, g = -rand, loss = out.sum(); here every gradient is also compared with the oracle (HD = 32
    runs zero-padded to 64).  Its keys are not normalised (|k|^2 ~ 32), so the delta rule grows
    geometrically with T (gradients near 1e37 by T = 64, where fp32 rounding compounds); the
    reference's length keeps them moderate."""
    torch.manual_seed(42)
    B, T, H, HD = 2, 16, 4, 32
    q, k, v = (torch.randn(B, T, H, HD) for _ in range(3))
    g = -torch.rand(B, T, H, HD)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g)]
    out, state = fast_recurrent_gated_deltanet(*xs)
    assert out.shape == (B, T, H, HD) and state.shape == (B, H, HD, HD)
    out.sum().backward()
    torch.cuda.synchronize()
    ref = O.gdn_bwd(q, k, v, g, None, None, torch.ones(B, T, H, HD), None)
    for x, r in zip(xs, ref[:4]):
        assert x.grad is not None and torch.isfinite(x.grad).all()
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)


@pytest.mark.parametrize("kind", ["head", "key"])
def test_operator_autograd_with_init_and_scalar_gate(dev, kind):
    """fast_chunk_gated_deltanet with requires_grad: the reference then runs its recurrence, where a
    4-D beta scales rows (key); a gate of one value per (token, head) ([B, T, H]) gets its gradient
    summed over the head dim; the initial state gets one too."""
    B, T, H, D = 2, 40, 2, 64
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, kind, seed=5)
    g3 = g[..., 0].clone()
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g3, beta)]
    s0d = s0.to(dev).requires_grad_(True)
    o, s = fast_chunk_gated_deltanet(*xs, initial_state=s0d)
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    gfull = g3.unsqueeze(-1).expand(B, T, H, D)
    ref = O.gdn_bwd(q, k, v, gfull, beta, s0, do, ds, beta_kind=KINDS[kind] if kind == "key" else None)
    dq, dk, dv, dg, db, ds0 = ref
    for x, r in ((xs[0], dq), (xs[1], dk), (xs[2], dv), (xs[3], dg.sum(-1)), (xs[4], db), (s0d, ds0)):
        assert tuple(x.grad.shape) == tuple(x.shape)
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)


def test_no_upstream_state_gradient(dev):
    """Only the output is used (the final state's gradient is None) and no initial state."""
    B, T, H, D = 1, 33, 2, 64
    q, k, v, g, beta, _, do, _ = _inputs(B, T, H, D, "value", seed=3)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    o, _ = fast_recurrent_gated_deltanet(*xs[:4], beta=xs[4])  # 4-D beta scales rows here
    (o * do.to(dev)).sum().backward()
    torch.cuda.synchronize()
    ref = O.gdn_bwd(q, k, v, g, beta, None, do, None, beta_kind=_lib.BETA_KEY)
    for x, r in zip(xs, ref[:5]):
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)


def test_fp16_and_fp32_gate(dev):
    """fp16 I/O with an fp32 gate: dq, dk, dv come back in fp16 and dg in fp32 (each gradient in
    its input's dtype), within one bf16 ULP (coarser than fp16's) plus 2e-3 of the oracle."""
    B, T, H, D = 1, 90, 2, 64
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, "key", seed=21, dtype=torch.float16)
    g = g.float()
    args = [x.to(dev) for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), _lib.BETA_KEY, do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    ref = O.gdn_bwd(q, k, v, g, beta, s0, do, ds, beta_kind=_lib.BETA_KEY)
    for name, x, r, dt in zip(("dq", "dk", "dv", "dg", "dbeta"), got[:5], ref[:5],
                              (torch.float16, torch.float16, torch.float16, torch.float32, torch.float16)):
        assert x.dtype == dt, name
        assert _ulp_excess(x, r) <= 2e-3, (name, _ulp_excess(x, r))


def test_unequal_head_dims_zero_padded(dev):
    """Dk = 48, Dv = 80 (run zero-padded to 128): gradients of the unpadded tensors, through the
    operator's autograd, fp32."""
    gen = torch.Generator().manual_seed(4880)
    B, T, H, Dk, Dv = 1, 37, 2, 48, 80
    q, k = (F.normalize(torch.randn(B, T, H, Dk, generator=gen), dim=-1) for _ in range(2))
    v = torch.randn(B, T, H, Dv, generator=gen)
    g = F.logsigmoid(torch.randn(B, T, H, Dk, generator=gen) + 2.0) / 8
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    s0 = 0.2 * torch.randn(B, H, Dk, Dv, generator=gen)
    do, ds = torch.randn(B, T, H, Dv, generator=gen), torch.randn(B, H, Dk, Dv, generator=gen)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    o, s = fast_recurrent_gated_deltanet(*xs[:4], beta=xs[4], initial_state=xs[5])
    ((o * do.to(dev)).sum() + (s * ds.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    ref = O.gdn_bwd(q, k, v, g, beta, s0, do, ds)
    for x, r in zip(xs, (ref[0], ref[1], ref[2], ref[3], ref[4], ref[5])):
        assert tuple(x.grad.shape) == tuple(x.shape)
        assert _rel_err(x.grad, r) <= 1e-5, _rel_err(x.grad, r)


def test_zero_tokens(dev):
    """T = 0: no token gradients, and the initial state's gradient is the final state's."""
    B, H, D = 2, 2, 64
    q = torch.zeros(B, 0, H, D, device=dev, requires_grad=True)
    k, v, g = (torch.zeros(B, 0, H, D, device=dev) for _ in range(3))
    s0 = torch.randn(B, H, D, D, device=dev, requires_grad=True)
    o, s = fast_recurrent_gated_deltanet(q, k, v, g, initial_state=s0)
    ds = torch.randn(B, H, D, D, device=dev)
    (s * ds).sum().backward()
    torch.cuda.synchronize()
    assert q.grad.shape == q.shape
    assert float((s0.grad - ds).abs().max()) == 0.0


def _check_fp32(got, ref):
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), got, ref):
        if r is None:
            assert x is None, name
            continue
        assert _rel_err(x, r) <= 1e-5, (name, _rel_err(x, r))


@pytest.mark.parametrize("kind", ["none", "head", "key"])
@pytest.mark.parametrize("D", [64, 128])
def test_one_segment_short_sub_chunks(dev, kind, D):
    """More than two waves per CU (B * H * D / 8 > 512 on MI355X's 256 CUs) keep each sequence one
    segment, walked in sub-chunks of 1024 / D tokens (the plan of the model's D = 128 shape, B = 4,
    H = 12); fp32 against the oracle with a ragged tail, for each beta kind that can segment."""
    B, T, H = 4, 45, 17 if D == 64 else 9
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert B * H * D // 8 > 2 * cus
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, kind, seed=D + 3)
    args = [x.to(dev) if x is not None else None for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), KINDS[kind], do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    _check_fp32(got, _oracle(q, k, v, g, beta, s0, do, ds, kind))


@pytest.mark.parametrize("D", [64, 128])
def test_value_beta_more_waves_than_cus(dev, D):
    """beta per value column never segments; with more waves than CUs (257-512 on MI355X) it walks
    sub-chunks of 1024 / D tokens instead of 2048 / D; fp32 against the oracle with a tail past
    the last checkpoint."""
    B, T, H = 4, 45, 9 if D == 64 else 5
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert cus < B * H * D // 8 <= 2 * cus
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, "value", seed=D + 1)
    args = [x.to(dev) for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), _lib.BETA_VALUE, do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    _check_fp32(got, _oracle(q, k, v, g, beta, s0, do, ds, "value"))


@pytest.mark.parametrize("kind", ["none", "head", "key"])
@pytest.mark.parametrize("D", [64, 128])
def test_segments_walked_in_parallel(dev, kind, D):
    """Few (b, h) pairs leave resident slots free, so the tokens are cut into segments walked in
    parallel (segment maps, carries both ways, then the per-segment walks): T = 1000 gives segments
    of several sub-chunks and a partial last sub-chunk; fp32 against the oracle at 1e-5."""
    B, T, H = 1, 1000, 2
    q, k, v, g, beta, s0, do, ds = _inputs(B, T, H, D, kind, seed=D + 11)
    args = [x.to(dev) if x is not None else None for x in (q, k, v, g, beta)]
    got = _gdn_bwd(*args, s0.to(dev), KINDS[kind], do.to(dev), ds.to(dev))
    torch.cuda.synchronize()
    ref = _oracle(q, k, v, g, beta, s0, do, ds, kind)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), got, ref):
        if r is None:
            assert x is None
            continue
        assert _rel_err(x, r) <= 1e-5, (name, _rel_err(x, r))
