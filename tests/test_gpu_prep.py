"""GPU parity of the GLA input pre-processing and the fused decode step against the fp64 oracle
(reference kernels: triune/model/attention.py:14-79 and :81-179)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import fast_chunk_gla, fused_qkv_g_prep_inplace, fused_qkvg_decode_step
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
