"""GPU parity of the single-launch GLA prefill (triune_hip_gla_prefill_onepass) against the fp64
oracle, and of its control-block protocol.

One workgroup per pair of 64-token chunks of each (sequence, head) publishes the pair's state map
and folds the earlier pairs' into the state it enters with (no carry-scan kernel).  The call shapes
are the
prefill tiles the reference's VectorisedGLA runs (B = 4, T <= 1024, H = 6, head dim 64:
triune/model/attention.py:425-451, 458-499) and ragged, token-wise and clamp-dispatch cases.
Tolerances as for the three-launch path: fp32 outputs and states within 2e-3 of the oracle for
16-bit inputs, bf16 outputs within one bf16 ULP plus 2e-3.
"""

import numpy as np
import pytest
import torch

import triune_amd._lib as L
import triune_amd.fast_gla as FG
from oracle import oracle as O
from triune_amd import fast_chunk_gla
from triune_amd.workloads import gla_inputs, ulp_bf16

pytestmark = pytest.mark.gpu

TOL16 = 2e-3


def _err(a, b):
    return float((torch.as_tensor(a).double().cpu() - torch.as_tensor(b).double()).abs().max())


def _ctrl(dev):
    key = (dev.index if dev.index is not None else 0, torch.cuda.current_stream(dev).cuda_stream)
    blk = L._CTRL.get(key)
    assert blk is not None, "no single-launch call ran on this stream"
    return blk[:12].view(torch.int32).cpu().tolist()


def _supported(B, T, H, io=torch.bfloat16, g=None, prep=0, flags=0):
    return bool(L.lib().triune_hip_gla_prefill_onepass_supported(B, T, H, 64, L._DT[io], L._DT[g or io], prep, flags))


def test_reference_tile_is_one_launch_and_longer_calls_are_not(dev):
    """B = 4, T = 1024, H = 6 (24 (sequence, head) pairs x 8 chunk pairs = 192 workgroups, one per
    CU) fits the 256 CUs; the plan refuses more chunk-pair workgroups per XCD than its CUs, and head
    dims other than 64."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert _supported(4, 1024, 6)
    assert _supported(4, 1024, 6, prep=1)
    assert _supported(4, 1024, 6, g=torch.float32)
    assert not _supported(4, 1024, 6, g=torch.float32, prep=1)  # the prep path keeps g in the I/O dtype
    per_xcd = cus // 8  # one workgroup per CU
    nh8 = (4 * 6 + 7) // 8
    t_max = per_xcd // nh8 * 128
    assert _supported(4, t_max, 6) and not _supported(4, t_max + 1, 6)
    assert not bool(L.lib().triune_hip_gla_prefill_onepass_supported(4, 1024, 6, 128, 1, 1, 0, 0))
    assert not _supported(1, 65 * 64, 1)  # more than 64 chunks per sequence


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_reference_tile_matches_oracle(dev, out_dtype):
    """Config-1 distributions at VectorisedGLA's prefill tile, with an initial state."""
    q, k, v, g, s0 = gla_inputs(4, 1024, 6, 64, seed=21, dtype=torch.bfloat16, init_std=0.1)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    out = torch.empty(v.shape, device=dev, dtype=out_dtype)
    before = _ctrl(dev) if (dev.index or 0, torch.cuda.current_stream(dev).cuda_stream) in L._CTRL else None
    o, s = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    if out_dtype == torch.float32:
        assert _err(o, ro) <= TOL16, _err(o, ro)
    else:
        excess = (o.double().cpu() - torch.from_numpy(ro)).abs() - (ulp_bf16(torch.from_numpy(ro)).double() + TOL16)
        assert float(excess.max()) <= 0, float(excess.max())
    assert _err(s, rs) <= TOL16, _err(s, rs)
    hdr = _ctrl(dev)
    assert hdr[1] == 0 and hdr[2] == 0, hdr  # epoch-read count back to zero, no wait ran out
    if before is not None:
        assert hdr[0] == before[0] + 1, (before, hdr)


@pytest.mark.parametrize("T", [2, 3, 63, 64, 65, 100, 128, 200, 257, 640, 1000])
@pytest.mark.parametrize("with_init", [False, True])
def test_ragged_lengths_against_three_launch_and_oracle(dev, T, with_init, monkeypatch):
    """Partial last chunks (checked and unchecked rows), a single chunk, no initial state; the
    three-launch path on the same inputs is held to the same bar."""
    q, k, v, g, s0 = gla_inputs(2, T, 3, 64, seed=300 + T, dtype=torch.bfloat16,
                                init_std=0.3 if with_init else 0)
    assert _supported(2, T, 3)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    s0d = None if s0 is None else s0.to(dev)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    for onepass in (True, False):
        monkeypatch.setattr(FG, "ONEPASS", onepass)
        out = torch.empty(v.shape, device=dev, dtype=torch.float32)
        o, s = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0d, out=out)
        torch.cuda.synchronize()
        assert _err(o, ro) <= TOL16, (onepass, _err(o, ro))
        assert _err(s, rs) <= TOL16, (onepass, _err(s, rs))
    assert _ctrl(dev)[2] == 0


@pytest.mark.parametrize("T", [1100, 2500, 4096])
def test_many_pairs_fold_in_rounds(dev, T, monkeypatch):
    """Up to 64 chunks per sequence (32 pairs): a workgroup folds the earlier pairs' maps eight at a
    time, so T = 1100 (9 pairs) ends on one full round, T = 2500 (20 pairs) on a short third round and
    T = 4096 on four rounds; each chunk group folds half the state rows and the halves meet in LDS.
    Against the oracle, with the three-launch path on the same inputs held to the same bar."""
    q, k, v, g, s0 = gla_inputs(1, T, 2, 64, seed=500 + T, dtype=torch.bfloat16, init_std=0.2)
    assert _supported(1, T, 2)
    qd, kd, vd, gd, s0d = (x.to(dev) for x in (q, k, v, g, s0))
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    for onepass in (True, False):
        monkeypatch.setattr(FG, "ONEPASS", onepass)
        out = torch.empty(v.shape, device=dev, dtype=torch.float32)
        o, s = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0d, out=out)
        torch.cuda.synchronize()
        assert _err(o, ro) <= TOL16, (onepass, _err(o, ro))
        assert _err(s, rs) <= TOL16, (onepass, _err(s, rs))
    assert _ctrl(dev)[2] == 0


@pytest.mark.parametrize("dtype,gdt", [(torch.float16, None), (torch.bfloat16, torch.float32),
                                       (torch.float16, torch.float32)])
def test_fp16_and_fp32_gates(dev, dtype, gdt):
    q, k, v, g, s0 = gla_inputs(3, 777, 2, 64, seed=41, dtype=dtype, init_std=0.2)
    if gdt is not None:
        g = g.float()
    assert _supported(3, 777, 2, io=dtype, g=g.dtype)
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = fast_chunk_gla(*(x.to(dev) for x in (q, k, v, g)), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16 and _err(s, rs) <= TOL16, (_err(o, ro), _err(s, rs))


def test_tokenwise_chunks_mixed_with_factored_ones(dev):
    """Chunks whose decay span exceeds the factored range walk token by token, for the local state
    they publish and for their outputs; later chunks fold those states."""
    q, k, v, g, s0 = gla_inputs(2, 700, 3, 64, seed=52, dtype=torch.bfloat16, init_std=0.3)
    g = g.float()
    gen = torch.Generator().manual_seed(2)
    g[:, 128:192] = -1.0 - 20.0 * torch.rand(2, 64, 3, 64, generator=gen)
    g[:, 400:460, 1] = -3.0 * torch.rand(60, 64, generator=gen)
    g = g.bfloat16()
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = fast_chunk_gla(*(x.to(dev) for x in (q, k, v, g)), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert _err(o, ro) <= TOL16 and _err(s, rs) <= TOL16, (_err(o, ro), _err(s, rs))
    assert _ctrl(dev)[2] == 0


@pytest.mark.parametrize("T", [65, 129, 1025])
def test_unclamped_tail_token(dev, T):
    """fast_chunk_gla's dispatch keeps g > 0 on a 1-token remainder after whole chunks
    (fast_gla.py:768-775): the last chunk walks token by token with that token unclamped."""
    gen = torch.Generator().manual_seed(T)
    q = (torch.randn(2, T, 2, 64, generator=gen) * 0.125).bfloat16()
    k = torch.randn(2, T, 2, 64, generator=gen).bfloat16()
    v = torch.randn(2, T, 2, 64, generator=gen).bfloat16()
    g = (0.05 * torch.randn(2, T, 2, 64, generator=gen)).bfloat16()
    s0 = 0.1 * torch.randn(2, 2, 64, 64, generator=gen)
    assert _supported(2, T, 2, flags=L.FLAG_TAIL_UNCLAMPED) == (T <= 64 * 64)
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = fast_chunk_gla(*(x.to(dev) for x in (q, k, v, g)), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(q, k, v, g, s0, clamp_mode=2)
    assert _err(o, ro) <= TOL16 and _err(s, rs) <= TOL16, (_err(o, ro), _err(s, rs))


def test_out_aliasing_g_and_strided_views(dev):
    """The reference's call (attention.py:443-451): q, k, v as strided views of one qkv buffer and
    the outputs written over g."""
    from triune_amd.fast_gla import _triton_chunk_gla_tc_fwd

    B, T, H = 4, 1024, 6
    q, k, v, g, s0 = gla_inputs(B, T, H, 64, seed=61, dtype=torch.bfloat16, init_std=0.1)
    qkv = torch.stack([q, k, v], dim=2).to(dev)
    gd = g.to(dev)
    o, s = _triton_chunk_gla_tc_fwd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], gd, initial_state=s0.to(dev), out=gd)
    torch.cuda.synchronize()
    assert o.data_ptr() == gd.data_ptr()
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    excess = (o.double().cpu() - torch.from_numpy(ro)).abs() - (ulp_bf16(torch.from_numpy(ro)).double() + TOL16)
    assert float(excess.max()) <= 0, float(excess.max())
    assert _err(s.float(), rs) <= 2 * float(ulp_bf16(torch.from_numpy(rs)).max()) + TOL16


def test_graph_replays_match_eager(dev):
    """Captured in a HIP graph, every replay advances the control block's epoch on the device, so
    flags of earlier replays never satisfy a later one: each replay equals the eager call."""
    q, k, v, g, s0 = (None if x is None else x.to(dev)
                      for x in gla_inputs(4, 1024, 6, 64, seed=71, dtype=torch.bfloat16, init_std=0.1))
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref_o, ref_s = fast_chunk_gla(q, k, v, g, initial_state=s0, out=out)
        ref_o, ref_s = ref_o.clone(), ref_s.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            go, gs = fast_chunk_gla(q, k, v, g, initial_state=s0, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(go, ref_o), i
        assert torch.equal(gs, ref_s), i
        # eager work on the same buffers between replays
        _ = fast_chunk_gla(q, k, v, g, initial_state=s0, out=torch.empty_like(out))
        torch.cuda.synchronize()


def test_alternating_call_sizes_share_the_control_block(dev):
    """Calls of different grid sizes in turn on one stream's control block (the count of epoch
    reads wraps at each call's own workgroup count): every call matches the oracle, advances the
    epoch by one and leaves the count at zero and no error bits."""
    cases = []
    for (B, T, H) in ((4, 1024, 6), (1, 130, 2), (2, 640, 3), (1, 64, 1)):
        q, k, v, g, s0 = gla_inputs(B, T, H, 64, seed=500 + T, dtype=torch.bfloat16, init_std=0.2)
        cases.append(((q, k, v, g, s0), O.gla_fwd(q, k, v, g, s0)))
    for rnd in range(3):
        for (q, k, v, g, s0), (ro, rs) in cases:
            assert _supported(q.shape[0], q.shape[1], q.shape[2])
            key = (dev.index if dev.index is not None else 0, torch.cuda.current_stream(dev).cuda_stream)
            before = _ctrl(dev) if key in L._CTRL else None
            out = torch.empty(v.shape, device=dev, dtype=torch.float32)
            o, s = fast_chunk_gla(q.to(dev), k.to(dev), v.to(dev), g.to(dev), initial_state=s0.to(dev), out=out)
            torch.cuda.synchronize()
            assert _err(o, ro) <= TOL16, (rnd, q.shape, _err(o, ro))
            assert _err(s, rs) <= TOL16, (rnd, q.shape, _err(s, rs))
            hdr = _ctrl(dev)
            assert hdr[1] == 0 and hdr[2] == 0, (rnd, q.shape, hdr)
            if before is not None:
                assert hdr[0] == before[0] + 1, (rnd, q.shape, before, hdr)
