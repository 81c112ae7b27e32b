"""GPU checks of the serving path: varlen prefill over a device state pool, pool decode, and the
graph-captured decode runner (triune_amd/serving.py), against the fp64 oracle and against the
eager calls they replace."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import fast_chunk_gla_varlen, gla_decode_step
from triune_amd.serving import GLADecodeGraphRunner, StateSlotPool
from triune_amd.workloads import gla_inputs

pytestmark = pytest.mark.gpu


def _packed(lens, H, D, seed, dtype):
    q, k, v, g, _ = gla_inputs(1, sum(lens), H, D, seed=seed, dtype=dtype, init_std=0.1)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return q, k, v, g, cu


@pytest.mark.parametrize("D", [64, 128])
def test_varlen_pool_equals_gathered_states(dev, D):
    """Pool form == plain varlen with the slots' states gathered in and the finals scattered
    back; a slot of -1 starts from zero and writes nothing; untouched slots keep their states."""
    lens, H, n_slots = [70, 1, 300, 129, 0, 64], 2, 9
    q, k, v, g, cu = _packed(lens, H, D, 3, torch.bfloat16)
    pool = 0.1 * torch.randn(n_slots, H, D, D, generator=torch.Generator().manual_seed(4))
    slots = torch.tensor([5, 0, -1, 8, 2, 3], dtype=torch.int32)
    init = torch.stack([pool[s] if s >= 0 else torch.zeros(H, D, D) for s in slots.tolist()])
    qd, kd, vd, gd, cud = (x.to(dev) for x in (q, k, v, g, cu))
    o_ref, fin_ref = fast_chunk_gla_varlen(qd, kd, vd, gd, cud, initial_state=init.to(dev))
    pd = pool.to(dev)
    o, ret = fast_chunk_gla_varlen(qd, kd, vd, gd, cud, state_pool=pd, slots=slots.to(dev))
    torch.cuda.synchronize()
    assert ret.data_ptr() == pd.data_ptr()
    assert torch.equal(o.cpu(), o_ref.cpu())
    expect = pool.clone()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            expect[s] = fin_ref[i].cpu()
    assert torch.equal(pd.cpu(), expect)


def test_pool_prefill_then_decode_matches_oracle(dev):
    """Three sessions: packed prefill into their slots, then 5 decode steps on the slots ==
    the oracle over each session's prompt followed by its decode tokens (fp32)."""
    H, D, lens = 2, 64, [100, 37, 64]
    pool = StateSlotPool(num_layers=2, n_slots=8, H=H, Dk=D, Dv=D, device=dev)
    slots = pool.slots_tensor(["s0", "s1", "s2"])
    q, k, v, g, cu = _packed(lens, H, D, 11, torch.float32)
    o_pre = pool.prefill(1, *(x.to(dev) for x in (q, k, v, g, cu)), slots)
    gen = torch.Generator().manual_seed(12)
    steps = [[torch.randn(3, H, D, generator=gen) for _ in range(4)] for _ in range(5)]
    for x in steps:
        x[0] = x[0] * D**-0.5  # config magnitudes: q scaled by D^-1/2
        x[3] = torch.nn.functional.logsigmoid(x[3]) / 8
    outs = [pool.decode_step(1, *(t.to(dev) for t in x), slots) for x in steps]
    torch.cuda.synchronize()
    assert pool.offsets[1][slots.long()].tolist() == [n + 5 for n in lens]
    assert float(pool.states[0].abs().sum()) == 0.0  # other layer untouched
    c = cu.tolist()
    for i in range(3):
        cat = [torch.cat([x[0, c[i]:c[i + 1]], torch.stack([st[j][i] for st in steps])])[None] for j, x in
               enumerate((q, k, v, g))]
        ro, rs = O.gla_fwd(*cat, None, clamp_mode=1)
        e_pre = float(np.abs(o_pre[0, c[i]:c[i + 1]].cpu().numpy() - ro[0, :lens[i]]).max())
        e_dec = max(float(np.abs(outs[t][i].cpu().numpy() - ro[0, lens[i] + t]).max()) for t in range(5))
        e_s = float(np.abs(pool.states[1, slots[i]].cpu().numpy() - rs[0]).max())
        print(f"session {i}: prefill o {e_pre:.3e}, decode o {e_dec:.3e}, state {e_s:.3e}")
        assert e_pre <= 1e-5 and e_dec <= 1e-5 and e_s <= 1e-5


def test_pool_fused_decode_step_counts_and_updates(dev):
    """StateSlotPool.fused_decode_step: the slots' states advance in place through the fused
    pre-processing decode step (equal to the dense step on the gathered states) and each session's
    token offset grows by one."""
    from triune_amd import fused_qkvg_decode_step

    gen = torch.Generator().manual_seed(31)
    H, HD, L = 2, 64, 2
    pool = StateSlotPool(num_layers=L, n_slots=6, H=H, Dk=HD, Dv=HD, device=dev)
    slots = pool.slots_tensor(["a", "b", "c"])
    for layer in range(L):
        pool.states[layer].copy_(0.1 * torch.randn(pool.states[layer].shape, generator=gen).to(dev))
    before = pool.states[1].clone()
    off0 = pool.offsets[1].clone()
    qkvg = torch.randn(3, 4, H, HD, generator=gen).bfloat16().to(dev)
    ang = torch.arange(HD // 2, dtype=torch.float32) * 0.01
    cos = torch.cos(torch.cat([ang, ang])).to(dev)
    sin = torch.sin(torch.cat([ang, ang])).to(dev)
    o = pool.fused_decode_step(1, qkvg, slots, cos, sin)
    do, dfin = fused_qkvg_decode_step(qkvg, cos, sin, initial_state=before[slots.long()], state_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(o, do)
    assert torch.equal(pool.states[1][slots.long()], dfin)
    assert torch.equal((pool.offsets[1] - off0)[slots.long()].cpu(), torch.ones(3, dtype=pool.offsets.dtype))


@pytest.mark.parametrize("steps", [1, 4])
def test_graph_runner_replays_match_eager(dev, steps):
    """Each replay (with fresh inputs written between replays, eager work and syncs in between)
    equals the eager decode steps on a copy of the pool; rows outside the runner's slots stay."""
    H, D, B, n_slots = 3, 64, 5, 12
    gen = torch.Generator().manual_seed(steps)
    pool = (0.1 * torch.randn(n_slots, H, D, D, generator=gen)).to(dev)
    ref = pool.clone()
    slots = torch.tensor([7, 1, 10, 4, 2], dtype=torch.int32, device=dev)
    runner = GLADecodeGraphRunner(pool, slots, steps=steps)
    runner.capture()
    torch.cuda.synchronize()
    assert torch.equal(pool, ref)  # capture (with its warm-up) leaves the states alone
    for rep in range(3):
        xs = [[torch.randn(B, H, D, generator=gen).to(dev) for _ in range(4)] for _ in range(steps)]
        for t, x in enumerate(xs):
            x[3] = torch.nn.functional.logsigmoid(x[3]) / 8
            for buf, src in zip((runner.q, runner.k, runner.v, runner.g), x):
                buf[t].copy_(src.to(buf.dtype))
        o = runner.replay()
        eager = []
        for t in range(steps):
            qb, kb, vb, gb = (buf[t] for buf in (runner.q, runner.k, runner.v, runner.g))
            oe, _ = gla_decode_step(qb, kb, vb, gb, ref, inplace=True, slots=slots)
            eager.append(oe)
        torch.cuda.synchronize()
        for t in range(steps):
            assert torch.equal(o[t], eager[t]), (rep, t)
        assert torch.equal(pool, ref), rep
    if steps == 1:
        x = [torch.randn(B, 1, H, D, generator=gen).to(dev).bfloat16() for _ in range(4)]
        o1 = runner.step(*x).clone()
        oe, _ = gla_decode_step(*x, ref, inplace=True, slots=slots)
        torch.cuda.synchronize()
        assert torch.equal(o1, oe[:, 0]) and torch.equal(pool, ref)
    runner.release()


def test_pool_prefill_and_decode_captured_in_one_graph(dev):
    """StateSlotPool.prefill followed by two decode steps, captured in one HIP graph (no host
    synchronisation inside), replayed three times with fresh inputs written between replays and
    eager work and syncs in between: every replay's outputs, states and offsets equal the same
    calls made eagerly on a second pool."""
    H, D, lens, n_slots = 2, 64, [100, 37, 64], 6
    pools = [StateSlotPool(num_layers=1, n_slots=n_slots, H=H, Dk=D, Dv=D, device=dev) for _ in range(2)]
    init = 0.1 * torch.randn(n_slots, H, D, D, generator=torch.Generator().manual_seed(21))
    for p in pools:
        p.states[0].copy_(init.to(dev))
    slots = torch.tensor([4, 0, 2], dtype=torch.int32, device=dev)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=dev)
    N = int(sum(lens))
    stat = [torch.zeros(1, N, H, D, device=dev, dtype=torch.bfloat16) for _ in range(4)]
    dec = [[torch.zeros(3, H, D, device=dev, dtype=torch.bfloat16) for _ in range(4)] for _ in range(2)]
    outs = [torch.zeros(1, N, H, D, device=dev, dtype=torch.bfloat16)] + [
        torch.zeros(3, H, D, device=dev, dtype=torch.bfloat16) for _ in range(2)]

    def serve(pool, o):
        pool.prefill(0, *stat, cu, slots, out=o[0])
        for t in range(2):
            pool.decode_step(0, *dec[t], slots, out=o[t + 1])

    scratch = StateSlotPool(num_layers=1, n_slots=n_slots, H=H, Dk=D, Dv=D, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        serve(scratch, [torch.empty_like(x) for x in outs])  # warm-up off the live pools
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        serve(pools[0], outs)
    torch.cuda.synchronize()
    assert torch.equal(pools[0].states[0].cpu(), init)  # capture ran nothing
    gen = torch.Generator().manual_seed(22)
    for rep in range(3):
        q, k, v, g, _ = gla_inputs(1, N, H, D, seed=30 + rep, dtype=torch.bfloat16)
        for dst, src in zip(stat, (q, k, v, g)):
            dst.copy_(src.to(dev))
        for t in range(2):
            xs = [torch.randn(3, H, D, generator=gen) for _ in range(4)]
            xs[3] = torch.nn.functional.logsigmoid(xs[3]) / 8
            for dst, src in zip(dec[t], xs):
                dst.copy_(src.to(dev).bfloat16())
        graph.replay()
        eager = [torch.empty_like(x) for x in outs]
        serve(pools[1], eager)
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b), rep
        assert torch.equal(pools[0].states, pools[1].states), rep
        assert torch.equal(pools[0].offsets, pools[1].offsets), rep
    assert pools[0].offsets[0][slots.long()].tolist() == [3 * (n + 2) for n in lens]
    graph.reset()
