"""GPU parity of the GLA input pre-processing and the fused decode step against the fp64 oracle
(reference kernels: triune/model/attention.py:14-79 and :81-179)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import fast_chunk_gla, fused_qkv_g_prep_inplace, fused_qkvg_decode_step, fused_qkvg_decode_step_pool
from triune_amd.workloads import ulp_bf16

pytestmark = pytest.mark.gpu


def _tables(T, HD, offset=0, dtype=torch.float32):
    """cos/sin [T, HD] as the reference's RotaryEmbedding builds them (rotary.py:24-29)."""
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float64) / HD))
    t = torch.arange(offset, offset + T, dtype=torch.float64)
    emb = torch.cat([torch.outer(t, inv_freq)] * 2, dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _within_ulp(got, ref, slack=0.0):
    """|got - ref| <= one bf16 ULP of ref (the output's own rounding) + slack."""
    ref_t = torch.from_numpy(np.asarray(ref, dtype=np.float64))
    err = (got.double().cpu() - ref_t).abs()
    return bool((err <= ulp_bf16(ref_t).double() + slack).all()), float(err.max())


@pytest.mark.parametrize("HD", [32, 64, 128])
@pytest.mark.parametrize("rope", [True, False])
def test_prep_bf16_matches_oracle(dev, HD, rope):
    gen = torch.Generator().manual_seed(HD + rope)
    B, T, H = 2, 37, 3  # B*T*H rows not a multiple of the rows per block
    qkv = (2.0 * torch.randn(B, T, 3, H, HD, generator=gen)).bfloat16()
    g = (3.0 * torch.randn(B, T, H, HD, generator=gen)).bfloat16()
    cos, sin = _tables(T, HD, offset=11)
    rq, rg = O.qkv_g_prep(qkv, g, cos if rope else None, sin if rope else None)
    qd, gd = qkv.to(dev), g.to(dev)
    fused_qkv_g_prep_inplace(qd, gd, cos.to(dev), sin.to(dev), use_rope=rope)
    torch.cuda.synchronize()
    ok, err = _within_ulp(qd[:, :, :2], rq[:, :, :2], slack=1e-6)
    assert ok, err
    ok, err = _within_ulp(gd, rg, slack=1e-6)
    assert ok, err
    assert torch.equal(qd[:, :, 2].cpu(), qkv[:, :, 2])  # v untouched


def test_prep_fp32_strided_views(dev):
    """fp32 I/O at 1e-5; qkv and g are views into larger buffers (padded heads and tokens)."""
    gen = torch.Generator().manual_seed(5)
    B, T, H, HD = 2, 19, 4, 64
    big = torch.randn(B, T + 3, 3, H + 1, HD + 8, generator=gen)
    gbig = 4.0 * torch.randn(B, T + 2, H + 2, HD, generator=gen)
    qkv, g = big[:, 1:T + 1, :, :H, :HD], gbig[:, :T, 1:H + 1]
    cos, sin = _tables(T, HD)
    rq, rg = O.qkv_g_prep(qkv, g, cos, sin)
    bd, gdb = big.to(dev), gbig.to(dev)
    qd, gd = bd[:, 1:T + 1, :, :H, :HD], gdb[:, :T, 1:H + 1]
    fused_qkv_g_prep_inplace(qd, gd, cos.to(dev), sin.to(dev))
    torch.cuda.synchronize()
    assert float(np.abs(qd[:, :, :2].double().cpu().numpy() - rq[:, :, :2]).max()) <= 1e-5
    assert float(np.abs(gd.double().cpu().numpy() - rg).max()) <= 1e-5
    # outside the views nothing changed: other tokens, the padding head and the padding dims
    bc, gc = bd.cpu(), gdb.cpu()
    assert torch.equal(bc[:, 0], big[:, 0]) and torch.equal(bc[:, T + 1:], big[:, T + 1:])
    assert torch.equal(bc[..., H:, :], big[..., H:, :]) and torch.equal(bc[..., HD:], big[..., HD:])
    assert torch.equal(bc[:, :, 2], big[:, :, 2])  # v
    assert torch.equal(gc[:, T:], gbig[:, T:]) and torch.equal(gc[:, :, 0], gbig[:, :, 0])


def test_prep_then_prefill_equals_oracle_pipeline(dev):
    """The reference's fused prefill path (attention.py:413-436): prep in place, then the chunked
    scan with out aliasing g."""
    gen = torch.Generator().manual_seed(9)
    B, T, H, HD = 2, 200, 2, 64
    qkv = torch.randn(B, T, 3, H, HD, generator=gen).bfloat16()
    g = torch.randn(B, T, H, HD, generator=gen).bfloat16()
    cos, sin = _tables(T, HD)
    qd, gd = qkv.to(dev), g.to(dev)
    fused_qkv_g_prep_inplace(qd, gd, cos.to(dev), sin.to(dev))
    pq, pk, pv, pg = qd[:, :, 0].cpu(), qd[:, :, 1].cpu(), qd[:, :, 2].cpu(), gd.cpu()  # rounded as the scan sees them
    o, s = fast_chunk_gla(qd[:, :, 0], qd[:, :, 1], qd[:, :, 2], gd, out=gd)
    torch.cuda.synchronize()
    ro, rs = O.gla_fwd(pq, pk, pv, pg)
    ok, err = _within_ulp(o, ro, slack=2e-3)
    assert ok, err
    assert float(np.abs(s.cpu().numpy() - rs).max()) <= 2e-3


@pytest.mark.parametrize("HD", [32, 64, 128])
@pytest.mark.parametrize("state", ["fp32", "io", "none"])
def test_fused_decode_matches_oracle(dev, HD, state):
    gen = torch.Generator().manual_seed(HD)
    B, H = 5, 3
    qkvg = torch.randn(B, 4, H, HD, generator=gen).bfloat16()
    s0 = 0.1 * torch.randn(B, H, HD, HD, generator=gen)
    cos, sin = _tables(1, HD, offset=42)
    init = None if state == "none" else (s0 if state == "fp32" else s0.bfloat16())
    ro, rs = O.fused_decode_step(qkvg, cos[0], sin[0], None if init is None else init.double())
    out, fin = fused_qkvg_decode_step(qkvg.to(dev), cos.to(dev), sin.to(dev),
                                      initial_state=None if init is None else init.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (B, 1, H, HD) and out.dtype == torch.bfloat16
    ok, err = _within_ulp(out[:, 0], ro, slack=1e-4)
    assert ok, err
    if state == "io":
        assert fin.dtype == torch.bfloat16
        ok, err = _within_ulp(fin, rs, slack=1e-6)
        assert ok, err
    else:
        assert fin.dtype == (torch.float32 if state == "fp32" else torch.bfloat16)
        if state == "fp32":
            assert float(np.abs(fin.cpu().numpy() - rs).max()) <= 1e-5
        else:
            ok, err = _within_ulp(fin, rs, slack=1e-6)
            assert ok, err


@pytest.mark.parametrize("HD", [32, 64, 128])
def test_fused_decode_pool_rows(dev, HD):
    """The fused decode step on rows of an fp32 state pool, in place: rows with a slot in the pool
    equal the dense step on the gathered states (bitwise: the same arithmetic) and the fp64 oracle;
    a padded row (slot -1) and a slot past the pool output zeros and touch no state; the other pool
    rows stay as they were."""
    gen = torch.Generator().manual_seed(HD + 7)
    B, H, n_slots = 5, 3, 7
    qkvg = torch.randn(B, 4, H, HD, generator=gen).bfloat16()
    pool0 = 0.1 * torch.randn(n_slots, H, HD, HD, generator=gen)
    cos, sin = _tables(1, HD, offset=9)
    slots = torch.tensor([3, 0, 6, -1, 9], dtype=torch.int32)
    pool = pool0.to(dev)
    out = fused_qkvg_decode_step_pool(qkvg.to(dev), pool, slots.to(dev), cos.to(dev), sin.to(dev))
    valid = [0, 1, 2]
    dense_in = pool0[slots[valid].long()]
    dout, dfin = fused_qkvg_decode_step(qkvg[valid].to(dev), cos.to(dev), sin.to(dev), initial_state=dense_in.to(dev),
                                        state_dtype=torch.float32)
    torch.cuda.synchronize()
    out, pool = out.cpu(), pool.cpu()
    assert torch.equal(out[valid], dout.cpu())
    assert torch.equal(pool[slots[valid].long()], dfin.cpu())
    assert torch.count_nonzero(out[3:]) == 0
    untouched = [i for i in range(n_slots) if i not in (3, 0, 6)]
    assert torch.equal(pool[untouched], pool0[untouched])
    ro, rs = O.fused_decode_step(qkvg[valid], cos[0], sin[0], dense_in.double())
    ok, err = _within_ulp(out[valid, 0], ro, slack=1e-4)
    assert ok, err
    assert float(np.abs(pool[slots[valid].long()].numpy() - rs).max()) <= 1e-5


def test_fused_decode_fp32_no_rope_no_save(dev):
    gen = torch.Generator().manual_seed(1)
    B, H, HD = 3, 2, 64
    qkvg = torch.randn(B, 4, H, HD, generator=gen)
    s0 = 0.1 * torch.randn(B, H, HD, HD, generator=gen)
    ro, _ = O.fused_decode_step(qkvg, None, None, s0)
    out, fin = fused_qkvg_decode_step(qkvg.to(dev), initial_state=s0.to(dev), save_final=False, use_rope=False)
    torch.cuda.synchronize()
    assert fin is None
    assert float(np.abs(out[:, 0].double().cpu().numpy() - ro).max()) <= 1e-5


def test_fused_decode_steps_equal_prep_then_decode(dev):
    """Three fused steps == pre-processing each token, then the plain decode step."""
    from triune_amd import gla_decode_step

    gen = torch.Generator().manual_seed(4)
    B, H, HD = 4, 2, 64
    s = 0.1 * torch.randn(B, H, HD, HD, generator=gen).to(dev)
    s_ref = s.clone()
    for step in range(3):
        x = torch.randn(B, 4, H, HD, generator=gen).to(dev)
        cos, sin = (t.to(dev) for t in _tables(1, HD, offset=step))
        out, s = fused_qkvg_decode_step(x, cos, sin, initial_state=s, state_dtype=torch.float32)
        qkv = torch.stack((x[:, 0], x[:, 1], x[:, 2]), dim=1)[:, None].contiguous()  # [B, 1, 3, H, HD]
        gg = x[:, 3][:, None].contiguous()
        fused_qkv_g_prep_inplace(qkv, gg, cos, sin)
        o2, s_ref = gla_decode_step(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], gg, s_ref)
        torch.cuda.synchronize()
        assert float((out - o2).abs().max()) <= 1e-5
        assert float((s - s_ref).abs().max()) <= 1e-5


# --- the prefill with the pre-processing fused into the segment-state kernel -----------------------
# (triune_hip_gla_prefill_prep): q, k, g are pre-processed in place while the segment states form,
# exactly as the reference's in-place prep kernel leaves them (rounded to the I/O dtype), and the
# scan then runs on those rounded values.  Checked in two parts: the values left in qkv and g
# against oracle.qkv_g_prep (one ULP of the I/O dtype), and the outputs and final states against
# oracle.gla_fwd on the values the device left (2e-3 for fp32 outputs, one bf16 ULP + 2e-3 for

@pytest.fixture(params=["onepass", "in_state", "two_step"])
def prefill_path(request, monkeypatch):
    """The fused pre-processing prefill on its three paths: calls of few chunks at head dim 64 take
    the single launch unless it is switched off; without it the entry runs the pre-processing
    inside the segment-state kernel up to gla_prep.FUSED_MAX_CHUNK_HEADS_PER_CU chunk-heads per
    compute unit (raised here to reach that kernel) and the prep pass then the prefill past it."""
    import triune_amd.fast_gla as FG
    import triune_amd.gla_prep as GP

    monkeypatch.setattr(FG, "ONEPASS", request.param == "onepass")
    monkeypatch.setattr(GP, "FUSED_MAX_CHUNK_HEADS_PER_CU", 1 << 30 if request.param == "in_state" else 0)
    return request.param

# bf16 outputs).
def _fused_case(B, T, H, HD, seed, dtype=torch.bfloat16, gate_shift=0.0):
    gen = torch.Generator().manual_seed(seed)
    qkv = (2.0 * torch.randn(B, T, 3, H, HD, generator=gen)).to(dtype)
    g = (3.0 * torch.randn(B, T, H, HD, generator=gen) + gate_shift).to(dtype)
    s0 = 0.1 * torch.randn(B, H, HD, HD, generator=gen)
    return qkv, g, s0


def _ulp16(ref, dtype):
    ref_t = torch.as_tensor(np.asarray(ref, dtype=np.float64))
    if dtype == torch.bfloat16:
        return ulp_bf16(ref_t).double()
    a = ref_t.abs().clamp_min(2.0**-14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def _check_prepped(qd, gd_pre, qkv, g, cos, sin):
    """The q, k, g left in place are the fp64 pre-processing rounded once (within one ULP)."""
    rq, rg = O.qkv_g_prep(qkv, g, cos, sin)
    for got, ref in ((qd[:, :, :2], rq[:, :, :2]), (gd_pre, rg)):
        err = (got.double().cpu() - torch.from_numpy(np.asarray(ref))).abs()
        assert bool((err <= _ulp16(ref, got.dtype) + 1e-6).all()), float(err.max())
    assert torch.equal(qd[:, :, 2].cpu(), qkv[:, :, 2])  # v untouched


@pytest.mark.parametrize("HD", [32, 64, 128])
@pytest.mark.parametrize("T", [200, 301])
@pytest.mark.parametrize("rope", [True, False])
def test_fused_prep_prefill_matches_oracle(prefill_path, dev, HD, T, rope):
    """T = 200 runs the unchecked-row instances with a partial last chunk, T = 301 the checked ones;
    fp32 outputs in a separate buffer, so g keeps the pre-processed gate for the check."""
    from triune_amd import fused_qkv_g_prep_chunk_gla

    B, H = 2, 3
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=HD + T + rope)
    cos, sin = _tables(T, HD, offset=5)
    qd, gd = qkv.to(dev), g.to(dev)
    out = torch.empty(B, T, H, HD, device=dev, dtype=torch.float32)
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev), out=out,
                                      use_rope=rope)
    torch.cuda.synchronize()
    assert o.data_ptr() == out.data_ptr()
    _check_prepped(qd, gd, qkv, g, cos if rope else None, sin if rope else None)
    ro, rs = O.gla_fwd(qd[:, :, 0].cpu(), qd[:, :, 1].cpu(), qd[:, :, 2].cpu(), gd.cpu(), s0)
    e_o, e_s = float(np.abs(o.double().cpu().numpy() - ro).max()), float(np.abs(s.double().cpu().numpy() - rs).max())
    assert e_o <= 2e-3 and e_s <= 2e-3, (e_o, e_s)


@pytest.mark.parametrize("T", [2500, 4096])
def test_fused_prep_single_launch_many_pairs(dev, T):
    """The single launch with the pre-processing over 20 and 32 chunk pairs per sequence (the fold
    of the earlier pairs' maps in rounds of eight); the values left in place and the outputs and
    final states against the oracle."""
    from triune_amd import fused_qkv_g_prep_chunk_gla
    from triune_amd._lib import lib

    B, H, HD = 1, 2, 64
    assert lib().triune_hip_gla_prefill_onepass_supported(B, T, H, HD, 1, 1, 1, 0)
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=T, gate_shift=3.0)
    cos, sin = _tables(T, HD)
    qd, gd = qkv.to(dev), g.to(dev)
    out = torch.empty(B, T, H, HD, device=dev, dtype=torch.float32)
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    _check_prepped(qd, gd, qkv, g, cos, sin)
    ro, rs = O.gla_fwd(qd[:, :, 0].cpu(), qd[:, :, 1].cpu(), qd[:, :, 2].cpu(), gd.cpu(), s0)
    e_o, e_s = float(np.abs(o.double().cpu().numpy() - ro).max()), float(np.abs(s.double().cpu().numpy() - rs).max())
    assert e_o <= 2e-3 and e_s <= 2e-3, (e_o, e_s)


@pytest.mark.parametrize("HD", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_prep_prefill_out_over_g(prefill_path, dev, HD, dtype):
    """The reference's call shape (attention.py:443-451): outputs written over g in the I/O dtype."""
    from triune_amd import fused_qkv_g_prep_chunk_gla

    B, T, H = 2, 1024, 2
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=HD, dtype=dtype, gate_shift=3.0)
    cos, sin = _tables(T, HD)
    qd, gd = qkv.to(dev), g.to(dev)
    # the pre-processed gate is overwritten by the outputs: take it from a run into a side buffer
    q2, g2 = qkv.to(dev), g.to(dev)
    fused_qkv_g_prep_chunk_gla(q2, g2, cos.to(dev), sin.to(dev), initial_state=s0.to(dev),
                               out=torch.empty(B, T, H, HD, device=dev, dtype=dtype))
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev))
    torch.cuda.synchronize()
    assert o.data_ptr() == gd.data_ptr() and torch.equal(qd, q2)
    _check_prepped(q2, g2, qkv, g, cos, sin)
    ro, rs = O.gla_fwd(q2[:, :, 0].cpu(), q2[:, :, 1].cpu(), q2[:, :, 2].cpu(), g2.cpu(), s0)
    err = (o.double().cpu() - torch.from_numpy(ro)).abs()
    assert bool((err <= _ulp16(ro, dtype) + 2e-3).all()), float(err.max())
    assert float(np.abs(s.cpu().numpy() - rs).max()) <= 2e-3


def test_fused_prep_prefill_tokenwise_chunks_and_no_final(prefill_path, dev):
    """Very negative raw gates (logsigmoid(g) ~ g) push chunks past the factored decay range: the
    output kernel runs them token by token on the pre-processed values; outputs over g."""
    from triune_amd import fused_qkv_g_prep_chunk_gla

    B, T, H, HD = 2, 260, 2, 64
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=77)
    g = g.float()
    g[:, 64:128] = -2.0 - 20.0 * torch.rand(B, 64, H, HD, generator=torch.Generator().manual_seed(3))
    g = g.bfloat16()
    cos, sin = _tables(T, HD)
    q2, g2 = qkv.to(dev), g.to(dev)
    fused_qkv_g_prep_chunk_gla(q2, g2, cos.to(dev), sin.to(dev), initial_state=s0.to(dev),
                               out=torch.empty(B, T, H, HD, device=dev, dtype=torch.bfloat16))
    qd, gd = qkv.to(dev), g.to(dev)
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev))
    torch.cuda.synchronize()
    _check_prepped(q2, g2, qkv, g, cos, sin)
    ro, rs = O.gla_fwd(q2[:, :, 0].cpu(), q2[:, :, 1].cpu(), q2[:, :, 2].cpu(), g2.cpu(), s0)
    ok, err = _within_ulp(o, ro, slack=2e-3)
    assert ok, err
    assert float(np.abs(s.cpu().numpy() - rs).max()) <= 2e-3
    o3, s3 = fused_qkv_g_prep_chunk_gla(qkv.to(dev), g.to(dev), cos.to(dev), sin.to(dev), save_final=False)
    assert s3.numel() == 1


def test_fused_prep_prefill_equals_prep_then_prefill(prefill_path, dev):
    """Against this library's two-step pipeline (the in-place prep kernel, then the prefill): the
    processed tensors agree to one ULP plus 1e-6 (the two kernels round the same fp32 values, formed
    in a different order), and so do the outputs up to what such one-ULP input differences move."""
    from triune_amd import fused_qkv_g_prep_chunk_gla

    B, T, H, HD = 2, 512, 3, 64
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=9, gate_shift=3.0)
    cos, sin = (x.to(dev) for x in _tables(T, HD))
    qa, ga = qkv.to(dev), g.to(dev)
    fused, sf = fused_qkv_g_prep_chunk_gla(qa, ga, cos, sin, initial_state=s0.to(dev),
                                           out=torch.empty(B, T, H, HD, device=dev))
    qb, gb = qkv.to(dev), g.to(dev)
    fused_qkv_g_prep_inplace(qb, gb, cos, sin)
    two, s2 = fast_chunk_gla(qb[:, :, 0], qb[:, :, 1], qb[:, :, 2], gb, initial_state=s0.to(dev),
                             out=torch.empty(B, T, H, HD, device=dev))
    torch.cuda.synchronize()
    ulp = ulp_bf16(qb.double()).to(dev)
    assert bool(((qa.double() - qb.double()).abs() <= ulp + 1e-6).all())
    assert bool(((ga.double() - gb.double()).abs() <= ulp_bf16(gb.double()).to(dev) + 1e-6).all())
    assert float((fused - two).abs().max()) <= 2.0**-7 * float(two.abs().max())
    assert float((sf - s2).abs().max()) <= 2.0**-7 * float(s2.abs().max())


def test_fused_prep_prefill_large_call_takes_two_step_path(dev):
    """B * H * chunks beyond four per compute unit, with the entry's default settings: the call does
    not fit the single launch, so the entry runs the prep kernel and then the prefill (the faster
    arrangement); same checks as the fused paths."""
    from triune_amd import fused_qkv_g_prep_chunk_gla

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    B, H, HD = 4, 8, 64
    T = 64 * (4 * cus // (B * H) + 1)
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=31, gate_shift=3.0)
    cos, sin = _tables(T, HD)
    qd, gd = qkv.to(dev), g.to(dev)
    out = torch.empty(B, T, H, HD, device=dev, dtype=torch.float32)
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    _check_prepped(qd, gd, qkv, g, cos, sin)
    ro, rs = O.gla_fwd(qd[:, :, 0].cpu(), qd[:, :, 1].cpu(), qd[:, :, 2].cpu(), gd.cpu(), s0)
    assert float(np.abs(o.double().cpu().numpy() - ro).max()) <= 2e-3
    assert float(np.abs(s.double().cpu().numpy() - rs).max()) <= 2e-3


@pytest.mark.parametrize("B,H,in_state", [(1, 3, True), (4, 6, False)])
def test_fused_prep_prefill_config1_length(dev, B, H, in_state, monkeypatch):
    """The fused entry at config 1's length (T = 16384) with the pre-processing inside the
    segment-state kernel (forced through gla_prep.FUSED_MAX_CHUNK_HEADS_PER_CU) and on the entry's
    default path (the prep pass and then the prefill), against the oracle on the values the device
    left (2e-3 for fp32 outputs and states, one ULP of the I/O dtype for the pre-processed
    tensors)."""
    import triune_amd.gla_prep as GP
    from triune_amd import fused_qkv_g_prep_chunk_gla

    if in_state:
        monkeypatch.setattr(GP, "FUSED_MAX_CHUNK_HEADS_PER_CU", 1 << 30)

    T, HD = 16384, 64
    qkv, g, s0 = _fused_case(B, T, H, HD, seed=B * 100 + H, gate_shift=3.0)
    cos, sin = _tables(T, HD)
    qd, gd = qkv.to(dev), g.to(dev)
    out = torch.empty(B, T, H, HD, device=dev, dtype=torch.float32)
    o, s = fused_qkv_g_prep_chunk_gla(qd, gd, cos.to(dev), sin.to(dev), initial_state=s0.to(dev), out=out)
    torch.cuda.synchronize()
    _check_prepped(qd, gd, qkv, g, cos, sin)
    ro, rs = O.gla_fwd(qd[:, :, 0].cpu(), qd[:, :, 1].cpu(), qd[:, :, 2].cpu(), gd.cpu(), s0)
    assert float(np.abs(o.double().cpu().numpy() - ro).max()) <= 2e-3
    assert float(np.abs(s.double().cpu().numpy() - rs).max()) <= 2e-3
