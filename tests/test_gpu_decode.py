"""GPU parity of the batched decode step against the fp64 oracle and the reference's own C step."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import fast_chunk_gla, gla_decode_step
from triune_amd.workloads import config2, gla_inputs

pytestmark = pytest.mark.gpu


def _maxerr(a, b):
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)).max())


@pytest.mark.parametrize("D", [32, 64, 128])
def test_decode_steps_match_oracle(dev, D):
    steps, B, H = 6, 64, 3
    q, k, v, g, s0 = config2(steps=steps, B=B, H=H, D=D)
    state = s0.to(dev).clone()
    ref_s = s0.double().numpy()
    for t in range(steps):
        o, state = gla_decode_step(q[t].to(dev), k[t].to(dev), v[t].to(dev), g[t].to(dev), state,
                                   out_dtype=torch.float32)
        ro, ref_s = O.gla_decode_step(q[t][:, 0], k[t][:, 0], v[t][:, 0], g[t][:, 0], ref_s)
        torch.cuda.synchronize()
        scale = max(1.0, float(np.abs(ro).max()))
        assert _maxerr(o[:, 0].cpu(), ro) <= 1e-5 * scale, (t, _maxerr(o[:, 0].cpu(), ro))
        assert _maxerr(state.cpu(), ref_s) <= 1e-5, (t, _maxerr(state.cpu(), ref_s))


def test_decode_inplace_slots_and_bf16_out(dev):
    B, H, D = 16, 2, 64
    q, k, v, g, _ = config2(steps=1, B=B, H=H, D=D)
    gen = torch.Generator().manual_seed(8)
    pool = torch.randn(40, H, D, D, generator=gen)
    slots = torch.randperm(40, generator=gen)[:B].to(torch.int32)
    pool_d = pool.to(dev)
    o, st = gla_decode_step(q[0].to(dev), k[0].to(dev), v[0].to(dev), g[0].to(dev), pool_d, inplace=True,
                            slots=slots.to(dev))
    torch.cuda.synchronize()
    assert st.data_ptr() == pool_d.data_ptr() and o.dtype == torch.bfloat16
    ro, rs = O.gla_decode_step(q[0][:, 0], k[0][:, 0], v[0][:, 0], g[0][:, 0], pool[slots.long()].double().numpy())
    got = pool_d.cpu()
    assert _maxerr(got[slots.long()], rs) <= 1e-5
    untouched = torch.ones(40, dtype=torch.bool)
    untouched[slots.long()] = False
    assert torch.equal(got[untouched], pool[untouched])
    ref = torch.from_numpy(ro).float()
    assert float((o[:, 0].float().cpu() - ref).abs().max()) <= float(ref.abs().max()) * 2**-8


def test_fp32_gate_bf16_io_matches_reference_c_step(dev):
    """The CUDA decode contract of csrc/kernels/gla.cu:23-75 (bf16 q/k/v/out, fp32 gate and state),
    checked against the reference's own CPU C step (engine.cpp:419-475) on the same values."""
    if not O.ref_available():
        pytest.skip("oracle/_ref not built")
    B, H, D = 32, 4, 64
    q, k, v, g, s0 = config2(steps=1, B=B, H=H, D=D)
    g32 = g[0].float()
    o, st = gla_decode_step(q[0].to(dev), k[0].to(dev), v[0].to(dev), g32.to(dev), s0.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    f = lambda x: x[:, 0].float().reshape(B * H, D).numpy()  # noqa: E731
    ro, rs = O.ref_c_decode_step_f32(f(q[0]), f(k[0]), f(v[0]), f(g32), s0.reshape(B * H, D, D).numpy())
    # the reference C step uses a polynomial exp (engine.cpp:57-69): agreement to ~1e-5 relative
    assert _maxerr(st.cpu().reshape(B * H, D, D), rs) <= 2e-5 * max(1.0, float(np.abs(rs).max()))
    assert _maxerr(o[:, 0].cpu().reshape(B * H, D), ro) <= 2e-5 * max(1.0, float(np.abs(ro).max()))


def test_decode_steps_equal_prefill(dev):
    """N decode steps from S0 == prefill of the same N tokens (test_audit_invariants.py:114-141)."""
    q, k, v, g, s0 = gla_inputs(2, 40, 2, 64, seed=77, dtype=torch.bfloat16, init_std=0.1)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    po, ps = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0.to(dev), out=torch.empty(v.shape, device=dev))
    st = s0.to(dev)
    outs = []
    for t in range(40):
        o, st = gla_decode_step(qd[:, t:t + 1], kd[:, t:t + 1], vd[:, t:t + 1], gd[:, t:t + 1], st,
                                out_dtype=torch.float32)
        outs.append(o)
    torch.cuda.synchronize()
    assert float((torch.cat(outs, 1) - po).abs().max()) <= 2e-3
    assert float((st - ps).abs().max()) <= 2e-3


def test_decode_graph_replay_matches_eager(dev):
    """A captured 8-step decode loop replays to the eager result (each replay checked)."""
    B, H, D, steps = 32, 2, 64, 8
    q, k, v, g, s0 = config2(steps=steps, B=B, H=H, D=D)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    eager = s0.to(dev).clone()
    for t in range(steps):
        gla_decode_step(qd[t], kd[t], vd[t], gd[t], eager, inplace=True)
    state = s0.to(dev).clone()
    outs = torch.empty(steps, B, 1, H, D, device=dev, dtype=torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream
        for t in range(steps):
            gla_decode_step(qd[t], kd[t], vd[t], gd[t], state.clone(), out=outs[t])
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for t in range(steps):
            gla_decode_step(qd[t], kd[t], vd[t], gd[t], state, inplace=True, out=outs[t])
    for _ in range(3):
        state.copy_(s0.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(state, eager)


def test_decode_slots_out_of_place_keeps_other_rows(dev):
    """slots with inplace=False: the returned pool holds the updated rows at the slots and the
    input values everywhere else; the input pool is not modified."""
    B, H, D = 8, 2, 64
    q, k, v, g, _ = config2(steps=1, B=B, H=H, D=D)
    gen = torch.Generator().manual_seed(12)
    pool = torch.randn(20, H, D, D, generator=gen)
    slots = torch.randperm(20, generator=gen)[:B].to(torch.int32)
    pool_d = pool.to(dev)
    o, st = gla_decode_step(q[0].to(dev), k[0].to(dev), v[0].to(dev), g[0].to(dev), pool_d, slots=slots.to(dev),
                            out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert st.data_ptr() != pool_d.data_ptr() and torch.equal(pool_d.cpu(), pool)
    ro, rs = O.gla_decode_step(q[0][:, 0], k[0][:, 0], v[0][:, 0], g[0][:, 0], pool[slots.long()].double().numpy())
    got = st.cpu()
    assert _maxerr(got[slots.long()], rs) <= 1e-5
    untouched = torch.ones(20, dtype=torch.bool)
    untouched[slots.long()] = False
    assert torch.equal(got[untouched], pool[untouched])
    assert _maxerr(o[:, 0].cpu(), ro) <= 1e-5 * max(1.0, float(np.abs(ro).max()))


def test_decode_padded_slot_rows_are_skipped(dev):
    """A batch row whose slot is -1 or past the pool (a padded row of a continuous batch) reads and
    writes no state and outputs zeros; the other rows are unaffected."""
    B, H, D = 6, 2, 64
    q, k, v, g, _ = config2(steps=1, B=B, H=H, D=D)
    gen = torch.Generator().manual_seed(13)
    pool = torch.randn(10, H, D, D, generator=gen)
    slots = torch.tensor([4, -1, 7, 10, 0, -5], dtype=torch.int32)
    pool_d = pool.to(dev)
    o, _ = gla_decode_step(q[0].to(dev), k[0].to(dev), v[0].to(dev), g[0].to(dev), pool_d, inplace=True,
                           slots=slots.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    live = torch.tensor([0, 2, 4])
    rows = slots[live].long()
    ro, rs = O.gla_decode_step(q[0][live, 0], k[0][live, 0], v[0][live, 0], g[0][live, 0], pool[rows].double().numpy())
    got = pool_d.cpu()
    assert _maxerr(got[rows], rs) <= 1e-5
    untouched = torch.ones(10, dtype=torch.bool)
    untouched[rows] = False
    assert torch.equal(got[untouched], pool[untouched])
    oc = o[:, 0].cpu()
    assert _maxerr(oc[live], ro) <= 1e-5 * max(1.0, float(np.abs(ro).max()))
    assert float(oc[torch.tensor([1, 3, 5])].abs().max()) == 0.0


@pytest.mark.parametrize("HD", [32, 64, 128])
def test_reference_signature_twins(dev, HD):
    """launch_gla_decode_step (gla.cu:97-114: bf16 Q/K/V/Out, fp32 G, fp32 State in place) and
    triune_gla_recurrent_step_f32 (api.h:94-103: fp32, [batch_heads, head_dim]) on device pointers,
    bound by name the way the reference's ctypes bridge binds its library."""
    from triune_amd._lib import lib

    L = lib()
    B, H = 5, 3
    q, k, v, g, s0 = config2(steps=1, B=B, H=H, D=HD)
    gf = g[0].float()
    Q, K, V = (x[0].to(dev).contiguous() for x in (q, k, v))
    G = gf.to(dev).contiguous()
    S = s0.to(dev).contiguous()
    Out = torch.empty(B, 1, H, HD, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    L.launch_gla_decode_step(Q.data_ptr(), K.data_ptr(), V.data_ptr(), G.data_ptr(), S.data_ptr(), Out.data_ptr(),
                             B, H, HD, stream)
    assert L.triune_hip_last_error() == 0
    torch.cuda.synchronize()
    ro, rs = O.gla_decode_step(q[0][:, 0], k[0][:, 0], v[0][:, 0], gf[:, 0], s0)
    assert _maxerr(S.cpu(), rs) <= 1e-5
    ref = torch.from_numpy(ro).float()
    assert float((Out[:, 0].float().cpu() - ref).abs().max()) <= float(ref.abs().max()) * 2**-8

    bh = B * H
    f32 = lambda x: x[0][:, 0].float().reshape(bh, HD).to(dev).contiguous()  # noqa: E731
    q3, k3, v3, g3 = f32(q), f32(k), f32(v), f32(g)
    S3 = s0.reshape(bh, HD, HD).to(dev).contiguous()
    o3 = torch.empty(bh, HD, device=dev)
    torch.cuda.synchronize()
    L.triune_gla_recurrent_step_f32(q3.data_ptr(), k3.data_ptr(), v3.data_ptr(), g3.data_ptr(), S3.data_ptr(),
                                    o3.data_ptr(), bh, HD)
    assert L.triune_hip_last_error() == 0
    torch.cuda.synchronize()
    ro3, rs3 = O.gla_decode_step(q3.cpu(), k3.cpu(), v3.cpu(), g3.cpu(), s0.reshape(bh, HD, HD))
    assert _maxerr(S3.cpu(), rs3) <= 1e-5
    assert _maxerr(o3.cpu(), ro3) <= 1e-5 * max(1.0, float(np.abs(ro3).max()))
