"""GPU parity of FusedRecurrentScan, Gated DeltaNet and the packed varlen prefill."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from triune_amd import FusedRecurrentScan, fast_chunk_gla, fast_chunk_gla_varlen
from triune_amd import fast_chunk_gated_deltanet, fast_recurrent_gated_deltanet
from triune_amd.workloads import config3, gla_inputs, ulp_bf16

pytestmark = pytest.mark.gpu


def _err(a, b):
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)).max())


def _bf16_excess(o_bf16, ref):
    """max over elements of |o - ref| - (1 bf16 ULP of ref + 2e-3); <= 0 passes."""
    ref = torch.as_tensor(ref).double()
    return float(((o_bf16.double() - ref).abs() - (ulp_bf16(ref).double() + 2e-3)).max())


# --- FusedRecurrentScan (reference test: tests/test_kernels.py:209-264) ----------------------
@pytest.mark.parametrize("N", [1, 4, 16, 32, 37])
@pytest.mark.parametrize("with_init", [False, True])
def test_recurrent_scan_fp32(dev, N, with_init):
    gen = torch.Generator().manual_seed(42 + N)
    B, H, Dk, Dv = 2, 4, 32, 32
    kv = torch.randn(B, H, N, Dk, Dv, generator=gen)
    decay = torch.rand(B, H, N, Dk, 1, generator=gen)
    init = torch.randn(B, H, Dk, Dv, generator=gen) if with_init else torch.zeros(B, H, Dk, Dv)
    s_all, fin = FusedRecurrentScan.apply(kv.to(dev), decay.to(dev), init.to(dev))
    torch.cuda.synchronize()
    rs, rf = O.recurrent_scan_fwd(kv, decay, init)
    assert s_all.dtype == torch.float32 and fin.dtype == torch.float32
    assert _err(s_all.cpu(), rs) <= 1e-5 and _err(fin.cpu(), rf) <= 1e-5


def test_recurrent_scan_bf16_returns_kv_dtype(dev):
    gen = torch.Generator().manual_seed(3)
    kv = torch.randn(1, 2, 9, 64, 64, generator=gen).bfloat16()
    decay = torch.rand(1, 2, 9, 64, 1, generator=gen)
    init = torch.randn(1, 2, 64, 64, generator=gen)
    s_all, fin = FusedRecurrentScan.apply(kv.to(dev), decay.to(dev), init.to(dev))
    torch.cuda.synchronize()
    rs, rf = O.recurrent_scan_fwd(kv, decay, init)
    assert s_all.dtype == torch.bfloat16 and fin.dtype == torch.bfloat16
    assert _err(fin.float().cpu(), rf) <= np.abs(rf).max() * 2**-7


@pytest.mark.parametrize("N,Dk,Dv", [(1, 32, 32), (16, 32, 32), (37, 64, 64), (9, 5, 12), (7, 3, 256)])
@pytest.mark.parametrize("with_init", [False, True])
def test_recurrent_scan_backward_fp32(dev, N, Dk, Dv, with_init):
    """Gradients through FusedRecurrentScan.apply (reference check: test_kernels.py:244-264) equal
    the oracle's reverse scan; Dv that is not a power of two leaves lanes of a row idle."""
    gen = torch.Generator().manual_seed(N + Dk + Dv)
    B, H = 2, 3
    kv = torch.randn(B, H, N, Dk, Dv, generator=gen)
    decay = torch.rand(B, H, N, Dk, 1, generator=gen)
    init = torch.randn(B, H, Dk, Dv, generator=gen) if with_init else torch.zeros(B, H, Dk, Dv)
    gs = torch.randn(B, H, N, Dk, Dv, generator=gen)
    gf = torch.randn(B, H, Dk, Dv, generator=gen)
    kvd, dd, idd = (x.to(dev).requires_grad_(True) for x in (kv, decay, init))
    s_all, fin = FusedRecurrentScan.apply(kvd, dd, idd)
    ((s_all * gs.to(dev)).sum() + (fin * gf.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    rs, _ = O.recurrent_scan_fwd(kv, decay, init)
    r_kv, r_dec, r_init = O.recurrent_scan_bwd(gs, gf, decay, rs)
    tol = 1e-5 * max(1.0, float(np.abs(r_kv).max()))
    assert _err(kvd.grad.cpu(), r_kv) <= tol
    assert _err(dd.grad.cpu(), r_dec) <= 1e-5 * max(1.0, float(np.abs(r_dec).max()))
    assert _err(idd.grad.cpu(), r_init) <= tol
    assert dd.grad.shape == decay.shape


def test_recurrent_scan_backward_bf16_and_missing_grads(dev):
    """bf16 kv: gradients come back in bf16 (fast_gla.py:199-203); only the final state used, so
    the S_all gradient is absent (None) and every step sees the decayed d_fin alone."""
    gen = torch.Generator().manual_seed(6)
    B, H, N, D = 1, 2, 11, 64
    kv = torch.randn(B, H, N, D, D, generator=gen).bfloat16()
    decay = torch.rand(B, H, N, D, 1, generator=gen)
    init = torch.randn(B, H, D, D, generator=gen)
    gf = torch.randn(B, H, D, D, generator=gen)
    kvd, dd, idd = (x.to(dev).requires_grad_(True) for x in (kv, decay, init))
    _, fin = FusedRecurrentScan.apply(kvd, dd, idd)
    (fin.float() * gf.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert kvd.grad.dtype == torch.bfloat16
    rs, _ = O.recurrent_scan_fwd(kv, decay, init)
    r_kv, r_dec, r_init = O.recurrent_scan_bwd(None, gf, decay, rs)
    rel = 2**-7
    assert _err(kvd.grad.float().cpu(), r_kv) <= rel * np.abs(r_kv).max()
    assert _err(dd.grad.float().cpu(), r_dec) <= rel * np.abs(r_dec).max()
    assert _err(idd.grad.float().cpu(), r_init) <= rel * np.abs(r_init).max()


# --- Gated DeltaNet -----------------------------------------------------------------------------
def _gdn_case(T, D, kind, seed):
    gen = torch.Generator().manual_seed(seed)
    B, H = 2, 2
    q = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    v = torch.randn(B, T, H, D, generator=gen)
    g = -0.2 * torch.rand(B, T, H, D, generator=gen)
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    beta = None
    if kind == "head":
        beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    elif kind in ("key", "value"):
        beta = torch.sigmoid(torch.randn(B, T, H, D, generator=gen))
    return q, k, v, g, beta, s0


@pytest.mark.parametrize("kind", ["none", "head", "key", "value"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_gdn_fp32_matches_oracle(dev, kind, D):
    q, k, v, g, beta, s0 = _gdn_case(150, D, kind, seed=D)
    args = [x.to(dev) for x in (q, k, v, g)]
    bd = None if beta is None else beta.to(dev)
    if kind == "key":
        o, s = fast_recurrent_gated_deltanet(*args, beta=bd, initial_state=s0.to(dev))
        bk = O.BETA_KEY
    else:
        o, s = fast_chunk_gated_deltanet(*args, beta=bd, initial_state=s0.to(dev))
        bk = O.BETA_VALUE
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q, k, v, g, beta, s0, beta_kind=bk)
    assert _err(o.cpu(), ro) <= 1e-5 and _err(s.cpu(), rs) <= 1e-5


@pytest.mark.parametrize("T,B,H,with_init", [(512, 1, 3, False), (2000, 4, 6, True)])
def test_gdn_config3_distributions_bf16(dev, T, B, H, with_init):
    """Config-3 distributions on the chunked WY/UT path (T = 2000: several chunks per segment,
    24 (b, h) rows sharing the resident slots, a ragged tail): fp32 outputs and states within
    2e-3 of the fp64 token-serial oracle, bf16 outputs within one bf16 ULP plus 2e-3 per element."""
    q, k, v, g, beta = config3(T=T, B=B, H=H)
    s0 = 0.1 * torch.randn(B, H, 64, 64, generator=torch.Generator().manual_seed(7)) if with_init else None
    args = [x.to(dev) for x in (q, k, v, g)]
    sd = None if s0 is None else s0.to(dev)
    o32, s32 = fast_chunk_gated_deltanet(*args, beta=beta.to(dev), initial_state=sd, out_dtype=torch.float32)
    ob, sb = fast_chunk_gated_deltanet(*args, beta=beta.to(dev), initial_state=sd)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q, k, v, g, beta, s0)
    assert o32.dtype == torch.float32 and ob.dtype == torch.bfloat16
    assert _err(o32.cpu(), ro) <= 2e-3 and _err(s32.cpu(), rs) <= 2e-3
    assert _bf16_excess(ob.cpu(), ro) <= 0.0
    assert _err(sb.cpu(), rs) <= 2e-3


@pytest.mark.parametrize("kind", ["head", "key", "value"])
@pytest.mark.parametrize("T", [200, 1000, 301])
def test_gdn_chunked_fp32_partial_last_chunk(dev, kind, T):
    """fp32 I/O through the chunked kernels with a partial last chunk (T % 4 == 0: the
    unchecked-row instances; T = 301: the checked ones), beta per head, per key dim and per value
    dim (the column solves), at the fp32 bar."""
    q, k, v, g, beta, s0 = _gdn_case(T, 64, kind, seed=T + len(kind))
    args = [x.to(dev) for x in (q, k, v, g)]
    fn = fast_recurrent_gated_deltanet if kind == "key" else fast_chunk_gated_deltanet
    o, s = fn(*args, beta=beta.to(dev), initial_state=s0.to(dev))
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q, k, v, g, beta, s0, beta_kind=O.BETA_VALUE if kind == "value" else O.BETA_KEY)
    e_o, e_s = _err(o.cpu(), ro), _err(s.cpu(), rs)
    print(f"gdn fp32 {kind} T={T}: o {e_o:.3e} S {e_s:.3e}")
    assert e_o <= 1e-5 and e_s <= 1e-5


@pytest.mark.parametrize("kind", ["head", "value"])
def test_gdn_chunked_extreme_decay_tokenwise_chunks(dev, kind):
    """Chunks whose decay span exceeds the factored range run token by token in the chunked path
    (beta per head, and per value dim)."""
    q, k, v, g, beta, s0 = _gdn_case(256, 64, kind, seed=11)
    g = g.clone()
    g[:, 64:128] = -1.0 - 20.0 * torch.rand(2, 64, 2, 64, generator=torch.Generator().manual_seed(2))
    o, s = fast_chunk_gated_deltanet(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta=beta.to(dev),
                                     initial_state=s0.to(dev))
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q, k, v, g, beta, s0, beta_kind=O.BETA_VALUE)
    print(f"gdn extreme decay {kind}: o {_err(o.cpu(), ro):.3e} S {_err(s.cpu(), rs):.3e}")
    assert _err(o.cpu(), ro) <= 1e-5 and _err(s.cpu(), rs) <= 1e-5


def _excess16(o16, ref):
    """max over elements of |o - ref| - (1 ULP of ref in o16's dtype + 2e-3); <= 0 passes."""
    ref = torch.as_tensor(ref).double()
    if o16.dtype == torch.bfloat16:
        ulp = ulp_bf16(ref).double()
    else:  # fp16: 10 fraction bits, subnormal spacing 2^-24
        ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0**-14))) - 10)
    return float(((o16.double() - ref).abs() - (ulp + 2e-3)).max())


@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kind", ["none", "head", "key", "value"])
@pytest.mark.parametrize("T", [200, 301])
def test_gdn_chunked_d128_16bit(dev, io, kind, T):
    """Head dim 128 with 16-bit I/O on the chunked kernels (eight waves per workgroup, four K
    steps per key-dim product): fp32 outputs and states within 2e-3 of the fp64 oracle on the same
    rounded inputs, 16-bit outputs within one ULP plus 2e-3 per element.  T = 200 runs the
    unchecked-row instances with a partial last chunk, T = 301 the checked ones."""
    q, k, v, g, beta, s0 = _gdn_case(T, 128, kind, seed=T + 3 * len(kind))
    q, k, v, g = (x.to(io) for x in (q, k, v, g))
    args = [x.to(dev) for x in (q, k, v, g)]
    bd = None if beta is None else beta.to(dev)
    fn = fast_recurrent_gated_deltanet if kind == "key" else fast_chunk_gated_deltanet
    o32, s32 = fn(*args, beta=bd, initial_state=s0.to(dev), out_dtype=torch.float32)
    o16, s16 = fn(*args, beta=bd, initial_state=s0.to(dev))
    torch.cuda.synchronize()
    bk = O.BETA_VALUE if kind == "value" else O.BETA_KEY
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=bk)
    e_o, e_s = _err(o32.cpu(), ro), _err(s32.cpu(), rs)
    print(f"gdn D=128 {io} {kind} T={T}: o {e_o:.3e} S {e_s:.3e}")
    assert o16.dtype == io and s16.dtype == torch.float32
    assert e_o <= 2e-3 and e_s <= 2e-3
    assert _excess16(o16.cpu(), ro) <= 0.0
    assert _err(s16.cpu(), rs) <= 2e-3


@pytest.mark.parametrize("kind", ["head", "value"])
@pytest.mark.parametrize("T", [2, 5, 64, 65])
def test_gdn_chunked_d128_short_sequences(dev, kind, T):
    """D = 128, bf16: sequences of one partial chunk, exactly one chunk and one chunk plus a token
    (one segment; checked and unchecked row instances), fp32 outputs and states at 2e-3."""
    q, k, v, g, beta, s0 = _gdn_case(T, 128, kind, seed=T + 40)
    q, k, v, g = (x.bfloat16() for x in (q, k, v, g))
    o, s = fast_chunk_gated_deltanet(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta=beta.to(dev),
                                     initial_state=s0.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=O.BETA_VALUE)
    assert o.shape == (2, T, 2, 128) and s.shape == (2, 2, 128, 128)
    assert _err(o.cpu(), ro) <= 2e-3 and _err(s.cpu(), rs) <= 2e-3


def test_gdn_chunked_d128_model_distributions(dev):
    """The reference model's GDN call at its default head dim (attention.py:509-536: q, k =
    normalize(elu(x) + 1), g = logsigmoid(x), no beta), bf16, 24 (b, h) rows over several
    segments; chunk decay spans of about 52 +- 5 per key dim."""
    gen = torch.Generator().manual_seed(21)
    B, T, H, D = 2, 1500, 12, 128
    qk = torch.nn.functional.normalize(torch.nn.functional.elu(torch.randn(B, T, 2, H, D, generator=gen)) + 1.0,
                                       dim=-1)
    q, k = qk[:, :, 0].bfloat16(), qk[:, :, 1].bfloat16()
    v = torch.randn(B, T, H, D, generator=gen).bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)).bfloat16()
    args = [x.to(dev) for x in (q, k, v, g)]
    o32, s32 = fast_chunk_gated_deltanet(*args, out_dtype=torch.float32)
    ob, sb = fast_chunk_gated_deltanet(*args)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), None, None)
    e_o, e_s = _err(o32.cpu(), ro), _err(s32.cpu(), rs)
    print(f"gdn D=128 model distributions: o {e_o:.3e} S {e_s:.3e}")
    assert e_o <= 2e-3 and e_s <= 2e-3
    assert _excess16(ob.cpu(), ro) <= 0.0


@pytest.mark.parametrize("kind", ["head", "value"])
def test_gdn_chunked_d128_extreme_decay_tokenwise_chunks(dev, kind):
    """D = 128: chunks whose decay span exceeds the factored range run token by token inside the
    chunked kernels (both states of the map kernel, the output kernel), at fp32 outputs; beta per
    head, and per value dim (the column-solve instances' token-by-token update)."""
    q, k, v, g, beta, s0 = _gdn_case(256, 128, kind, seed=12)
    g = g.clone()
    g[:, 64:128] = -1.0 - 20.0 * torch.rand(2, 64, 2, 128, generator=torch.Generator().manual_seed(2))
    q, k, v, g = (x.bfloat16() for x in (q, k, v, g))
    o, s = fast_chunk_gated_deltanet(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta=beta.to(dev),
                                     initial_state=s0.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=O.BETA_VALUE)
    e_o, e_s = _err(o.cpu(), ro), _err(s.cpu(), rs)
    print(f"gdn D=128 extreme decay {kind}: o {e_o:.3e} S {e_s:.3e}")
    assert e_o <= 2e-3 and e_s <= 2e-3


@pytest.mark.parametrize("D,io", [(64, torch.float32), (64, torch.bfloat16), (128, torch.bfloat16)])
def test_gdn_chunked_wide_decay_span(dev, D, io):
    """Chunk decay spans of 112-125 per key dim (just inside the factored form's 128): factors
    reach e^+-62, non-causal products overflow and must be masked out, and the results keep the
    fp32 bar at fp32 I/O and 2e-3 at bf16 I/O."""
    q, k, v, g, beta, s0 = _gdn_case(300, D, "head", seed=D + 1)
    g = -1.75 - 0.2 * torch.rand(g.shape, generator=torch.Generator().manual_seed(5))
    q, k, v, g = (x.to(io) for x in (q, k, v, g))
    o, s = fast_chunk_gated_deltanet(*(x.to(dev) for x in (q, k, v, g)), beta=beta.to(dev),
                                     initial_state=s0.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0)
    e_o, e_s = _err(o.cpu(), ro), _err(s.cpu(), rs)
    print(f"gdn wide span D={D} {io}: o {e_o:.3e} S {e_s:.3e}")
    assert np.isfinite(o.cpu().numpy()).all() and np.isfinite(s.cpu().numpy()).all()
    tol = 1e-5 if io == torch.float32 else 2e-3
    assert e_o <= tol and e_s <= tol


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kind", ["none", "head", "key", "value"])
@pytest.mark.parametrize("io", [torch.float32, torch.bfloat16])
def test_gdn_decode_step_many_rows(dev, D, kind, io):
    """T == 1 of 200 x 6 rows (more rows than decode workgroups, so each walks several) runs the
    decode step; every beta kind (per value dim through the operator's internal entry, as the
    public T == 1 calls apply a 4-D beta to rows), fp32 outputs and states at the fp32 bar, and
    three chained steps against the three-token recurrence."""
    import triune_amd._lib as LB
    from triune_amd import fast_gla as FG
    gen = torch.Generator().manual_seed(D + len(kind))
    B, H, T = 200, 6, 3
    q = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1).to(io)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1).to(io)
    v = torch.randn(B, T, H, D, generator=gen).to(io)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, D, generator=gen)).to(io)
    g[:, :, 0, :3] = 0.5  # positive gates: clamped to 0
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    beta = None
    if kind == "head":
        beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    elif kind in ("key", "value"):
        beta = torch.sigmoid(torch.randn(B, T, H, D, generator=gen))
    bk = {"none": LB.BETA_NONE, "head": LB.BETA_HEAD, "key": LB.BETA_KEY, "value": LB.BETA_VALUE}[kind]
    s = s0.to(dev)
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        bt = None if beta is None else beta[:, sl].to(dev)
        o, s = FG._gdn(q[:, sl].to(dev), k[:, sl].to(dev), v[:, sl].to(dev), g[:, sl].to(dev), bt, s, bk,
                       out_dtype=torch.float32)
        outs.append(o)
    torch.cuda.synchronize()
    o = torch.cat(outs, dim=1).cpu()
    okind = O.BETA_VALUE if kind == "value" else O.BETA_KEY
    ro, rs = O.gdn_fwd(q.float(), k.float(), v.float(), g.float(), beta, s0, beta_kind=okind)
    e_o, e_s = _err(o, ro), _err(s.cpu(), rs)
    print(f"gdn decode D={D} {kind} {io}: o {e_o:.3e} S {e_s:.3e}")
    assert e_o <= 1e-5 and e_s <= 1e-5


def test_gdn_single_token(dev):
    q, k, v, g, beta, s0 = _gdn_case(1, 64, "head", seed=5)
    o, s = fast_chunk_gated_deltanet(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta=beta.to(dev),
                                     initial_state=s0.to(dev))
    torch.cuda.synchronize()
    ro, rs = O.gdn_fwd(q, k, v, g, beta, s0)
    assert _err(o.cpu(), ro) <= 1e-5 and _err(s.cpu(), rs) <= 1e-5


# --- varlen --------------------------------------------------------------------------------------
@pytest.mark.parametrize("D", [64, 128])
def test_varlen_matches_oracle(dev, D):
    lens = [0, 1, 63, 64, 65, 200, 700, 5, 128, 129]
    N = sum(lens)
    q, k, v, g, _ = gla_inputs(1, N, 2, D, seed=D, dtype=torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    s0 = 0.1 * torch.randn(len(lens), 2, D, D, generator=torch.Generator().manual_seed(1))
    out = torch.empty(v.shape, device=dev, dtype=torch.float32)
    o, s = fast_chunk_gla_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), cu.to(dev), initial_state=s0.to(dev),
                                 out=out)
    torch.cuda.synchronize()
    ro, rs = O.gla_varlen_fwd(q, k, v, g, cu.numpy(), s0)
    assert _err(o.cpu(), ro) <= 2e-3 and _err(s.cpu(), rs) <= 2e-3


def test_varlen_equals_dense_batch(dev):
    q, k, v, g, s0 = gla_inputs(3, 333, 2, 64, seed=3, dtype=torch.bfloat16, init_std=0.1)
    qd, kd, vd, gd = (x.to(dev) for x in (q, k, v, g))
    od, sd = fast_chunk_gla(qd, kd, vd, gd, initial_state=s0.to(dev), out=torch.empty(v.shape, device=dev))
    cu = torch.arange(0, 4 * 333, 333, dtype=torch.int32, device=dev)
    pk = lambda x: x.reshape(1, 3 * 333, 2, 64)  # noqa: E731
    ov, sv = fast_chunk_gla_varlen(pk(qd), pk(kd), pk(vd), pk(gd), cu, initial_state=s0.to(dev),
                                   out=torch.empty(1, 999, 2, 64, device=dev))
    torch.cuda.synchronize()
    assert float((ov.reshape(3, 333, 2, 64) - od).abs().max()) <= 1e-4
    assert float((sv - sd).abs().max()) <= 1e-4


def test_gdn_gradients_only_where_requested(dev):
    """A call that needs gradients goes through the autograd function (the reference
    differentiates its PyTorch recurrence there): q's gradient matches the oracle, inputs that do
    not require one get none; under no_grad the outputs carry no graph."""
    gen = torch.Generator().manual_seed(70)
    q, k = (torch.nn.functional.normalize(torch.randn(1, 70, 2, 64, generator=gen), dim=-1) for _ in range(2))
    v = torch.randn(1, 70, 2, 64, generator=gen)
    g = -0.1 * torch.rand(1, 70, 2, 64, generator=gen)
    qd = q.to(dev).requires_grad_(True)
    kd, vd, gd = k.to(dev), v.to(dev), g.to(dev)
    o, s = fast_chunk_gated_deltanet(qd, kd, vd, gd)
    assert o.requires_grad
    o.sum().backward()
    ref = O.gdn_bwd(q, k, v, g, None, None, torch.ones(1, 70, 2, 64), None)
    assert float(np.abs(qd.grad.double().cpu().numpy() - ref[0]).max()) <= 1e-5 * max(1.0, np.abs(ref[0]).max())
    assert kd.grad is None
    with torch.no_grad():
        o, s = fast_chunk_gated_deltanet(qd, kd, vd, gd)
    assert o.shape == (1, 70, 2, 64) and not o.requires_grad


@pytest.mark.parametrize("Dk,Dv", [(128, 128), (48, 80), (100, 200)])
def test_fp32_wide_value_heads_dense_and_varlen(dev, Dk, Dv):
    """fp32 heads whose kernel pair would be (128, 128) (its fp32 planes exceed the LDS), and
    value heads wider than 128: value columns run as slices (they evolve independently), dense
    and packed, at the fp32 bar against the oracle."""
    gen = torch.Generator().manual_seed(Dk + Dv)
    lens = [70, 1, 200]
    N, H = sum(lens), 2
    q = torch.randn(1, N, H, Dk, generator=gen) * Dk**-0.5
    k = torch.randn(1, N, H, Dk, generator=gen)
    v = torch.randn(1, N, H, Dv, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(1, N, H, Dk, generator=gen)) / 16
    s0 = 0.1 * torch.randn(len(lens), H, Dk, Dv, generator=gen)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    o, s = fast_chunk_gla_varlen(q.to(dev), k.to(dev), v.to(dev), g.to(dev), cu.to(dev), initial_state=s0.to(dev))
    torch.cuda.synchronize()
    ro, rs = O.gla_varlen_fwd(q, k, v, g, cu.numpy(), s0)
    assert o.shape == (1, N, H, Dv) and s.shape == (len(lens), H, Dk, Dv)
    assert _err(o.cpu(), ro) <= 1e-5 and _err(s.cpu(), rs) <= 1e-5
    # dense: the first sequence as a batch of one
    od, sd = fast_chunk_gla(q[:, :70].to(dev), k[:, :70].to(dev), v[:, :70].to(dev), g[:, :70].to(dev),
                            initial_state=s0[:1].to(dev))
    torch.cuda.synchronize()
    rd, rsd = O.gla_fwd(q[:, :70], k[:, :70], v[:, :70], g[:, :70], s0[:1])
    assert _err(od.cpu(), rd) <= 1e-5 and _err(sd.cpu(), rsd) <= 1e-5
