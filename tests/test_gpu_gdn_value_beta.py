"""GPU parity of Gated DeltaNet with beta per value column at head dim 64 and bf16 I/O (the
reference's Triton orientation, triune/kernels/fast_gla.py:464-465), the case the two-role
whole-sequence walk serves: waves 0-3 form chunk i + 1's factors and tiles while waves 4-7 run
chunk i's solve and state update.  Against the fp64 oracle: fp32 outputs and final states within
2e-3, bf16 outputs within one bf16 ULP + 2e-3 (the bar of the other 16-bit GDN paths)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import fast_chunk_gated_deltanet
from triune_amd.workloads import ulp_bf16

pytestmark = pytest.mark.gpu

TOL16 = 2e-3


def _err(a, b):
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)).max())


def _case(B, T, H, seed, gate_scale=0.2):
    gen = torch.Generator().manual_seed(seed)
    D = 64
    q = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    v = torch.randn(B, T, H, D, generator=gen)
    g = -gate_scale * torch.rand(B, T, H, D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, D, generator=gen))
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    q, k, v, g = (x.bfloat16() for x in (q, k, v, g))
    return q, k, v, g, beta, s0


@pytest.mark.parametrize("T", [2, 63, 64, 65, 200, 301, 1000])
@pytest.mark.parametrize("with_init", [False, True])
def test_value_beta_bf16_d64_matches_oracle(dev, T, with_init):
    """Partial chunks, one chunk, one chunk and a token, ragged (checked-row instances at T not a
    multiple of 4), with and without an initial state."""
    q, k, v, g, beta, s0 = _case(2, T, 3, seed=500 + T)
    s0 = s0 if with_init else None
    args = [x.to(dev) for x in (q, k, v, g)]
    o, s = fast_chunk_gated_deltanet(*args, beta=beta.to(dev), initial_state=None if s0 is None else s0.to(dev),
                                     out_dtype=torch.float32)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=O.BETA_VALUE)
    assert _err(o.cpu(), ro) <= TOL16, _err(o.cpu(), ro)
    assert _err(s.cpu(), rs) <= TOL16, _err(s.cpu(), rs)


def test_value_beta_bf16_outputs_config3_shape(dev):
    """Config 3's shape (B = 4, H = 6, T = 8192: 128 chunks per walk), logsigmoid gates, bf16
    outputs."""
    gen = torch.Generator().manual_seed(5)
    B, T, H, D = 4, 8192, 6, 64
    qk = torch.nn.functional.normalize(torch.randn(B, T, 2, H, D, generator=gen), dim=-1).bfloat16()
    q, k = qk[:, :, 0], qk[:, :, 1]
    v = torch.randn(B, T, H, D, generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)).bfloat16()
    beta = torch.sigmoid(torch.randn(B, T, H, D, generator=gen))
    o, s = fast_chunk_gated_deltanet(*(x.to(dev) for x in (q, k, v, g)), beta=beta.to(dev))
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, None, beta_kind=O.BETA_VALUE)
    ref = torch.from_numpy(np.asarray(ro)).double()
    excess = float(((o.cpu().double() - ref).abs() - (ulp_bf16(ref).double() + TOL16)).max())
    assert excess <= 0, excess
    assert _err(s.cpu(), rs) <= TOL16, _err(s.cpu(), rs)


def test_value_beta_tokenwise_chunks_between_factored_ones(dev):
    """Chunks whose decay span exceeds the factored range walk token by token from the state (in
    the stage-3 role) between factored chunks."""
    q, k, v, g, beta, s0 = _case(2, 700, 2, seed=77)
    g = g.float()
    g[:, 128:192] = -1.0 - 20.0 * torch.rand(2, 64, 2, 64, generator=torch.Generator().manual_seed(3))
    g[:, 450:470, 1] = -3.0 * torch.rand(20, 64, generator=torch.Generator().manual_seed(4))
    g = g.bfloat16()
    o, s = fast_chunk_gated_deltanet(*(x.to(dev) for x in (q, k, v, g)), beta=beta.to(dev),
                                     initial_state=s0.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=O.BETA_VALUE)
    assert _err(o.cpu(), ro) <= TOL16 and _err(s.cpu(), rs) <= TOL16, (_err(o.cpu(), ro), _err(s.cpu(), rs))


def test_value_beta_repeats_bitwise(dev):
    """The walk is deterministic: repeated calls are bitwise equal."""
    q, k, v, g, beta, s0 = (x.to(dev) for x in _case(2, 1000, 3, seed=9))
    o1, s1 = fast_chunk_gated_deltanet(q, k, v, g, beta=beta, initial_state=s0, out_dtype=torch.float32)
    o1, s1 = o1.clone(), s1.clone()
    for _ in range(3):
        o2, s2 = fast_chunk_gated_deltanet(q, k, v, g, beta=beta, initial_state=s0, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(s1, s2)
