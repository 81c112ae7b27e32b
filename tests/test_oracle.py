"""CPU checks that pin the fp64 oracle (oracle/gla_oracle.c) before it is trusted.

Each check is chosen so that a plausible mistake in the oracle (a dropped term, the decay
applied after instead of before the write, a wrong clamp rule, a transposed state, a wrong beta
orientation) fails at least one of them:
  * hand-computed scalar cases of the reference's recurrences,
  * the non-recursive closed form, and its special cases g = 0 (causal linear attention,
    brute force) and k = 0 (pure decay),
  * invariants: carried-state splitting, decode steps == prefill, linearity in v,
  * the reference's own C decode step, compiled from its sources into oracle/_ref,
  * input/output vectors of the reference's fast_recurrent_gated_deltanet (tests/golden/).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.ref_port import fast_chunk_gla_cpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "gdn_reference_cpu.npz"


def _rand(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape)


def _gates(seed, *shape, scale=1.0):
    x = np.random.default_rng(seed).standard_normal(shape)
    return -np.log1p(np.exp(-x)) * scale  # logsigmoid


# ---------------------------------------------------------------------------------------------
# GLA
# ---------------------------------------------------------------------------------------------
def test_gla_scalar_hand_case():
    """D = 1, T = 2: S1 = e^a s + k1 v1, o1 = q1 S1; S2 = e^b S1 + k2 v2, o2 = q2 S2
    (test_attention_fallback.py:12-24: decay, then write, then read)."""
    s, a, b = 0.7, -0.3, -1.1
    q1, q2, k1, k2, v1, v2 = 1.5, -0.5, 2.0, 0.25, -1.0, 3.0
    S1 = np.exp(a) * s + k1 * v1
    S2 = np.exp(b) * S1 + k2 * v2
    f = lambda *x: np.array(x, dtype=np.float64).reshape(1, 2, 1, 1)  # noqa: E731
    o, S = O.gla_fwd(f(q1, q2), f(k1, k2), f(v1, v2), f(a, b), np.full((1, 1, 1, 1), s))
    assert np.allclose(o.ravel(), [q1 * S1, q2 * S2], rtol=0, atol=1e-14)
    assert np.allclose(S.ravel(), [S2], rtol=0, atol=1e-14)


@pytest.mark.parametrize("T,D,Dv", [(1, 4, 4), (9, 4, 6), (40, 8, 8), (70, 5, 3)])
def test_gla_recurrence_equals_closed_form(T, D, Dv):
    q, k = _rand(1, 2, T, 3, D), _rand(2, 2, T, 3, D)
    v, g = _rand(3, 2, T, 3, Dv), _gates(4, 2, T, 3, D)
    s0 = _rand(5, 2, 3, D, Dv)
    o1, s1 = O.gla_fwd(q, k, v, g, s0, clamp_mode=1)
    o2, s2 = O.gla_closed_form(q, k, v, g, s0)
    assert np.abs(o1 - o2).max() < 1e-11 and np.abs(s1 - s2).max() < 1e-11


def test_gla_zero_gate_is_causal_linear_attention():
    """g = 0: o_t = sum_{s<=t} (q_t . k_s) v_s + q_t S0, brute force."""
    T, D = 23, 6
    q, k, v, s0 = _rand(1, 1, T, 2, D), _rand(2, 1, T, 2, D), _rand(3, 1, T, 2, D), _rand(4, 1, 2, D, D)
    o, S = O.gla_fwd(q, k, v, np.zeros_like(q), s0)
    ref = np.zeros_like(o)
    for h in range(2):
        for t in range(T):
            ref[0, t, h] = q[0, t, h] @ s0[0, h]
            for s in range(t + 1):
                ref[0, t, h] += (q[0, t, h] @ k[0, s, h]) * v[0, s, h]
    assert np.abs(o - ref).max() < 1e-11
    kv = np.einsum("thi,thj->hij", k[0], v[0])
    assert np.abs(S[0] - (s0[0] + kv)).max() < 1e-11


def test_gla_zero_keys_is_pure_decay():
    T, D = 17, 5
    q, g, s0 = _rand(1, 1, T, 1, D), _gates(2, 1, T, 1, D), _rand(3, 1, 1, D, D)
    o, S = O.gla_fwd(q, np.zeros_like(q), _rand(4, 1, T, 1, D), g, s0)
    G = np.cumsum(g[0, :, 0], axis=0)
    ref = np.stack([q[0, t, 0] @ (np.exp(G[t])[:, None] * s0[0, 0]) for t in range(T)])
    assert np.abs(o[0, :, 0] - ref).max() < 1e-12
    assert np.abs(S[0, 0] - np.exp(G[-1])[:, None] * s0[0, 0]).max() < 1e-12


def test_gla_clamp_rules_follow_reference_dispatch():
    """clamp_mode 2: T == 1 and the lone remainder token after whole chunks keep g > 0
    (fast_gla.py:746-753, :768-775); every other token is clamped (fast_gla.py:586)."""
    T, C, D = 65, 64, 3
    q, k, v, s0 = _rand(1, 1, T, 1, D), _rand(2, 1, T, 1, D), _rand(3, 1, T, 1, D), _rand(4, 1, 1, D, D)
    g = np.abs(_rand(5, 1, T, 1, D)) * 0.1  # all positive
    o, S = O.gla_fwd(q, k, v, g, s0, chunk=C, clamp_mode=2)
    g_ref = np.zeros_like(g)
    g_ref[:, -1] = g[:, -1]  # only the remainder token keeps its gate
    o2, S2 = O.gla_fwd(q, k, v, g_ref, s0, clamp_mode=0)
    assert np.abs(o - o2).max() < 1e-12 and np.abs(S - S2).max() < 1e-12
    o1, S1 = O.gla_fwd(q[:, :1], k[:, :1], v[:, :1], g[:, :1], s0, clamp_mode=2)
    o1b, S1b = O.gla_decode_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], s0)
    assert np.abs(o1[:, 0] - o1b).max() < 1e-12 and np.abs(S1 - S1b).max() < 1e-12


def test_gla_split_with_carried_state_and_linearity():
    T, D = 90, 4
    q, k, v, v2 = (_rand(i, 2, T, 2, D) for i in range(4))
    g, s0 = _gates(9, 2, T, 2, D), _rand(10, 2, 2, D, D)
    o, S = O.gla_fwd(q, k, v, g, s0, clamp_mode=1)
    oa, Sa = O.gla_fwd(q[:, :37], k[:, :37], v[:, :37], g[:, :37], s0, clamp_mode=1)
    ob, Sb = O.gla_fwd(q[:, 37:], k[:, 37:], v[:, 37:], g[:, 37:], Sa, clamp_mode=1)
    assert np.abs(np.concatenate([oa, ob], 1) - o).max() < 1e-12 and np.abs(Sb - S).max() < 1e-12
    z = np.zeros_like(s0)
    l1, _ = O.gla_fwd(q, k, v, g, z, clamp_mode=1)
    l2, _ = O.gla_fwd(q, k, v2, g, z, clamp_mode=1)
    l3, _ = O.gla_fwd(q, k, v + 2 * v2, g, z, clamp_mode=1)
    assert np.abs(l3 - (l1 + 2 * l2)).max() < 1e-11


def test_gla_varlen_is_per_sequence_recurrence():
    lens = [3, 0, 64, 65, 1]
    N, D = sum(lens), 4
    q, k, v, g = _rand(1, 1, N, 2, D), _rand(2, 1, N, 2, D), _rand(3, 1, N, 2, D), _gates(4, 1, N, 2, D)
    s0 = _rand(5, len(lens), 2, D, D)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    o, S = O.gla_varlen_fwd(q, k, v, g, cu, s0)
    for i, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        oi, Si = O.gla_fwd(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], s0[i:i + 1], clamp_mode=1)
        assert oi.size == 0 or np.abs(o[:, a:b] - oi).max() < 1e-12
        assert np.abs(S[i] - Si[0]).max() < 1e-12


def test_decode_step_matches_reference_c_engine():
    """The reference's own triune_gla_recurrent_step_f32 (csrc/engine/engine.cpp:419-475),
    compiled from its sources; it uses a polynomial exp (engine.cpp:57-69), so agreement is to
    fp32 rounding plus that approximation."""
    if not O.ref_available():
        pytest.skip("oracle/_ref/libtriune_core_ref.so not built (reference tree absent)")
    BH, D = 24, 64
    q, k, v = _rand(1, BH, D), _rand(2, BH, D), _rand(3, BH, D)
    g, S = _gates(4, BH, D, scale=1 / 16), 0.1 * _rand(5, BH, D, D)
    o_ref, S_ref = O.ref_c_decode_step_f32(q, k, v, g, S)
    f32 = lambda a: a.astype(np.float32).astype(np.float64)  # noqa: E731
    o, Sn = O.gla_decode_step(f32(q), f32(k), f32(v), f32(g), f32(S))
    assert np.abs(Sn - S_ref).max() <= 2e-6 * max(1, np.abs(S_ref).max())
    assert np.abs(o - o_ref).max() <= 2e-6 * max(1, np.abs(o_ref).max())


# ---------------------------------------------------------------------------------------------
# FusedRecurrentScan
# ---------------------------------------------------------------------------------------------
def test_scan_scalar_hand_case():
    kv = np.array([1.0, 2.0, 3.0]).reshape(1, 1, 3, 1, 1)
    d = np.array([0.5, 0.25, 2.0]).reshape(1, 1, 3, 1, 1)
    s_all, fin = O.recurrent_scan_fwd(kv, d, np.full((1, 1, 1, 1), 4.0))
    # s: 4 -> 4*0.5+1 = 3 -> 3*0.25+2 = 2.75 -> 2.75*2+3 = 8.5 ; exclusive outputs 4, 3, 2.75
    assert np.allclose(s_all.ravel(), [4.0, 3.0, 2.75]) and np.allclose(fin.ravel(), [8.5])


def test_scan_closed_form():
    """s_all[n] = (prod_{m<n} d_m) init + sum_{m<n} (prod_{m<j<n} d_j) kv_m."""
    B, H, N, Dk, Dv = 2, 3, 7, 4, 5
    kv, init = _rand(1, B, H, N, Dk, Dv), _rand(2, B, H, Dk, Dv)
    d = np.random.default_rng(3).random((B, H, N, Dk, 1))
    s_all, fin = O.recurrent_scan_fwd(kv, d, init)
    for n in range(N + 1):
        ref = np.prod(d[:, :, :n], axis=2) * init
        for m in range(n):
            ref = ref + np.prod(d[:, :, m + 1:n], axis=2) * kv[:, :, m]
        got = s_all[:, :, n] if n < N else fin
        assert np.abs(got - ref).max() < 1e-12


# ---------------------------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("name,kind", [("none", O.BETA_NONE), ("head", O.BETA_HEAD), ("key", O.BETA_KEY)])
def test_gdn_matches_reference_golden_vectors(name, kind):
    z = np.load(GOLDEN)
    beta = z[f"{name}_beta"] if f"{name}_beta" in z.files else None
    o, s = O.gdn_fwd(z[f"{name}_q"], z[f"{name}_k"], z[f"{name}_v"], z[f"{name}_g"], beta, z[f"{name}_s0"],
                     beta_kind=kind)
    assert np.abs(o - z[f"{name}_o"]).max() < 1e-12
    assert np.abs(s - z[f"{name}_s"]).max() < 1e-12


def test_gdn_zero_gate_is_delta_rule_in_transition_form():
    """g = 0: S_t = (I - beta k k^T) S_{t-1} + beta k v^T (the textbook delta rule, computed here
    in that matrix form, not the residual form the oracle uses)."""
    T, D = 12, 5
    q, k, v = _rand(1, 1, T, 1, D), _rand(2, 1, T, 1, D) * 0.4, _rand(3, 1, T, 1, D)
    beta = np.random.default_rng(4).random((1, T, 1))
    S = _rand(5, 1, 1, D, D)
    o, Sf = O.gdn_fwd(q, k, v, np.zeros_like(q), beta, S)
    cur = S[0, 0].copy()
    for t in range(T):
        kt = k[0, t, 0]
        cur = (np.eye(D) - beta[0, t, 0] * np.outer(kt, kt)) @ cur + beta[0, t, 0] * np.outer(kt, v[0, t, 0])
        assert np.abs(o[0, t, 0] - q[0, t, 0] @ cur).max() < 1e-12
    assert np.abs(Sf[0, 0] - cur).max() < 1e-12


def test_gdn_orthonormal_write_then_read():
    """g = 0, beta = 1, zero state: writing v under an orthonormal key and reading with the same
    key returns v exactly (associative recall)."""
    D = 6
    keys = np.linalg.qr(_rand(1, D, D))[0]
    T = D
    k = keys.T.reshape(1, T, 1, D)
    v = _rand(2, 1, T, 1, D)
    o, S = O.gdn_fwd(k, k, v, np.zeros_like(k), np.ones((1, T, 1)), None)
    for t in range(T):
        assert np.abs(o[0, t, 0] - v[0, t, 0]).max() < 1e-12


def test_gdn_zero_beta_is_pure_decay():
    T, D = 9, 4
    q, k, v, g = _rand(1, 1, T, 1, D), _rand(2, 1, T, 1, D), _rand(3, 1, T, 1, D), _gates(4, 1, T, 1, D)
    s0 = _rand(5, 1, 1, D, D)
    o, S = O.gdn_fwd(q, k, v, g, np.zeros((1, T, 1)), s0)
    G = np.cumsum(g[0, :, 0], 0)
    assert np.abs(S[0, 0] - np.exp(G[-1])[:, None] * s0[0, 0]).max() < 1e-12


def test_gdn_beta_orientations_differ_only_for_per_dim_beta():
    T, D = 8, 4
    q, k, v, g = _rand(1, 1, T, 1, D), _rand(2, 1, T, 1, D), _rand(3, 1, T, 1, D), _gates(4, 1, T, 1, D)
    b = np.random.default_rng(6).random((1, T, 1, D))
    ok, _ = O.gdn_fwd(q, k, v, g, b, None, beta_kind=O.BETA_KEY)
    ov, _ = O.gdn_fwd(q, k, v, g, b, None, beta_kind=O.BETA_VALUE)
    assert np.abs(ok - ov).max() > 1e-3
    bh = np.broadcast_to(b[..., :1], b.shape)
    ok, _ = O.gdn_fwd(q, k, v, g, bh, None, beta_kind=O.BETA_KEY)
    ov, _ = O.gdn_fwd(q, k, v, g, bh, None, beta_kind=O.BETA_VALUE)
    oh, _ = O.gdn_fwd(q, k, v, g, b[..., 0], None)
    assert np.abs(ok - ov).max() < 1e-12 and np.abs(ok - oh).max() < 1e-12


# ---------------------------------------------------------------------------------------------
# CPU baseline port (oracle/ref_port.py) against the oracle
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("T", [1, 5, 64, 65, 200, 640])
def test_port_fp64_matches_oracle(T):
    gen = torch.Generator().manual_seed(T)
    q, k, v = (torch.randn(1, T, 2, 8, generator=gen, dtype=torch.float64) for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, 2, 8, generator=gen, dtype=torch.float64))
    s0 = torch.randn(1, 2, 8, 8, generator=gen, dtype=torch.float64)
    o, s = fast_chunk_gla_cpu(q, k, v, g, s0)
    ro, rs = O.gla_fwd(q, k, v, g, s0)
    assert np.abs(o.numpy() - ro).max() < 1e-10 and np.abs(s.numpy() - rs).max() < 1e-10


def test_port_fp32_factored_path_matches_oracle():
    gen = torch.Generator().manual_seed(1)
    T = 1024
    q = torch.randn(1, T, 2, 64, generator=gen) * 0.125
    k, v = torch.randn(1, T, 2, 64, generator=gen), torch.randn(1, T, 2, 64, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, 2, 64, generator=gen)) / 16
    o, s = fast_chunk_gla_cpu(q, k, v, g, None)
    ro, rs = O.gla_fwd(q, k, v, g, None)
    assert np.abs(o.double().numpy() - ro).max() < 1e-4 and np.abs(s.double().numpy() - rs).max() < 1e-4


# ---------------------------------------------------------------------------------------------
# VectorisedGLA input pre-processing (attention.py:14-179)
# ---------------------------------------------------------------------------------------------
def _rope_tables(T, HD, offset=0):
    """cos/sin [T, HD] built like the reference's RotaryEmbedding (rotary.py:24-29), float64."""
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float64) / HD))
    t = torch.arange(offset, offset + T, dtype=torch.float64)
    emb = torch.cat([torch.outer(t, inv_freq)] * 2, dim=-1)
    return emb.cos(), emb.sin()


@pytest.mark.parametrize("HD", [32, 64, 128])
def test_prep_matches_unfused_torch_path(HD):
    """The reference's unfused path (attention.py:509-528): F.normalize(F.elu(x) + 1, eps=1e-6),
    then x * cos + cat(-x2, x1) * sin, evaluated by torch in float64."""
    gen = torch.Generator().manual_seed(HD)
    T = 9
    x = 2.0 * torch.randn(2, T, 3, HD, generator=gen, dtype=torch.float64)
    cos, sin = _rope_tables(T, HD, offset=5)
    a = torch.nn.functional.normalize(torch.nn.functional.elu(x) + 1.0, p=2.0, dim=-1, eps=1e-6)
    a1, a2 = a.chunk(2, dim=-1)
    ref = a * cos[None, :, None] + torch.cat((-a2, a1), dim=-1) * sin[None, :, None]
    got = O.qk_prep(x.numpy(), cos.numpy()[None, :, None], sin.numpy()[None, :, None])
    assert np.abs(got - ref.numpy()).max() <= 1e-12
    assert np.abs(O.qk_prep(x.numpy()) - a.numpy()).max() <= 1e-12


def test_logsigmoid_matches_torch():
    x = torch.tensor([-800.0, -40.0, -3.0, -1e-7, 0.0, 1e-7, 2.5, 40.0, 800.0], dtype=torch.float64)
    assert np.abs(O.logsigmoid(x.numpy()) - torch.nn.functional.logsigmoid(x).numpy()).max() <= 1e-15
    g = torch.randn(1000, generator=torch.Generator().manual_seed(3), dtype=torch.float64) * 6
    assert np.abs(np.exp(O.logsigmoid(g.numpy())) - torch.sigmoid(g).numpy()).max() <= 1e-15


def test_prep_invariants():
    x = _rand(7, 4, 64) * 3
    a = O.qk_prep(x)
    assert np.allclose(np.linalg.norm(a, axis=-1), 1.0, atol=1e-14)  # unit rows without rotation
    one, zero = np.ones(64), np.zeros(64)
    assert np.abs(O.qk_prep(x, one, zero) - a).max() == 0.0  # angle 0 is the identity
    cos, sin = (t.numpy() for t in _rope_tables(4, 64, offset=100))
    r = O.qk_prep(x, cos, sin)
    assert np.allclose(np.linalg.norm(r, axis=-1), 1.0, atol=1e-14)  # a rotation keeps the norm
    # the eps guard: elu(x) + 1 = e^x underflows the 1e-12 floor for very negative rows
    tiny = O.qk_prep(np.full((1, 8), -200.0))
    assert np.allclose(tiny, np.exp(-200.0) * 1e6)


def test_fused_decode_oracle_brute_force():
    """prep q, k; decay sigmoid(g); S <- diag(decay) S + k v^T; o = S^T q, by explicit loops."""
    rng = np.random.default_rng(11)
    B, H, HD = 2, 3, 32
    x = rng.standard_normal((B, 4, H, HD))
    S0 = 0.1 * rng.standard_normal((B, H, HD, HD))
    cos, sin = (t.numpy()[0] for t in _rope_tables(1, HD, offset=17))
    o, S = O.fused_decode_step(x, cos, sin, S0)
    for b in range(B):
        for h in range(H):
            q = O.qk_prep(x[b, 0, h], cos, sin)
            k = O.qk_prep(x[b, 1, h], cos, sin)
            d = 1.0 / (1.0 + np.exp(-x[b, 3, h]))
            Sn = d[:, None] * S0[b, h] + np.outer(k, x[b, 2, h])
            assert np.abs(Sn - S[b, h]).max() <= 1e-13
            assert np.abs(q @ Sn - o[b, h]).max() <= 1e-13
    o0, S0z = O.fused_decode_step(x, None, None, None)  # no rotation, zero state
    assert np.abs(S0z - np.einsum("bhi,bhj->bhij", O.qk_prep(x[:, 1]), x[:, 2])).max() <= 1e-13


# ---------------------------------------------------------------------------------------------
# Backward (gradients of the GLA recurrence and of the exclusive scan)
# ---------------------------------------------------------------------------------------------
def _torch_gla(q, k, v, g, s0, chunk):
    """fp64 token recurrence with fast_chunk_gla's clamp dispatch, differentiated by autograd
    (the reference's own gradient check recurrence, test_kernels.py:270-277)."""
    B, T, H, Dk = q.shape
    S = s0 if s0 is not None else torch.zeros(B, H, Dk, v.shape[-1], dtype=torch.float64)
    outs = []
    for t in range(T):
        clamp = not (T == 1 or (T > chunk and T % chunk == 1 and t == T - 1))
        gt = torch.clamp(g[:, t], max=0.0) if clamp else g[:, t]
        S = S * torch.exp(gt).unsqueeze(-1) + k[:, t].unsqueeze(-1) @ v[:, t].unsqueeze(-2)
        outs.append((q[:, t].unsqueeze(-2) @ S).squeeze(-2))
    return torch.stack(outs, dim=1), S


@pytest.mark.parametrize("T,chunk,with_init", [(1, 64, True), (17, 64, False), (65, 64, True), (70, 32, True),
                                               (33, 32, False)])
def test_gla_bwd_matches_autograd(T, chunk, with_init):
    """Every gradient (q, k, v, g, S0) equals torch autograd through the fp64 recurrence,
    including the clamp mask (positive and exactly-zero gates) and the unclamped tail."""
    B, H, Dk, Dv = 2, 2, 5, 3
    rng = np.random.default_rng(T)
    q, k, v = (torch.tensor(rng.standard_normal((B, T, H, d)), requires_grad=True) for d in (Dk, Dk, Dv))
    gn = -np.abs(rng.standard_normal((B, T, H, Dk)))
    gn[:, ::3, :, 0] = 0.3 * np.abs(gn[:, ::3, :, 0]) + 0.05  # some positive gates (clamped -> zero grad)
    gn[:, 1::4, :, 1] = 0.0  # exact zeros: torch.clamp passes the gradient at the boundary
    gn[:, -1] = 0.2  # the final token's gates positive: unclamped iff it is a 1-token tail
    g = torch.tensor(gn, requires_grad=True)
    s0 = torch.tensor(rng.standard_normal((B, H, Dk, Dv)), requires_grad=True) if with_init else None
    do = torch.tensor(rng.standard_normal((B, T, H, Dv)))
    dsf = torch.tensor(rng.standard_normal((B, H, Dk, Dv)))
    o, s = _torch_gla(q, k, v, g, s0, chunk)
    ((o * do).sum() + (s * dsf).sum()).backward()
    dq, dk, dv, dg, ds0 = O.gla_bwd(q, k, v, g, s0, do, dsf, chunk=chunk)
    for got, ref in ((dq, q.grad), (dk, k.grad), (dv, v.grad), (dg, g.grad)):
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-11, atol=1e-11)
    if with_init:
        np.testing.assert_allclose(ds0, s0.grad.numpy(), rtol=1e-11, atol=1e-11)


def test_gla_bwd_finite_differences():
    """Central differences of the oracle's own forward agree with its backward (no torch)."""
    B, T, H, Dk, Dv = 1, 6, 1, 3, 2
    rng = np.random.default_rng(3)
    q, k = rng.standard_normal((2, B, T, H, Dk))
    v = rng.standard_normal((B, T, H, Dv))
    g = -0.2 - np.abs(rng.standard_normal((B, T, H, Dk)))  # away from the clamp boundary
    s0 = rng.standard_normal((B, H, Dk, Dv))
    W = rng.standard_normal((B, T, H, Dv))
    U = rng.standard_normal((B, H, Dk, Dv))

    def loss(q, k, v, g, s0):
        o, s = O.gla_fwd(q, k, v, g, s0)
        return float((o * W).sum() + (s * U).sum())

    grads = O.gla_bwd(q, k, v, g, s0, W, U)
    args = [q, k, v, g, s0]
    eps = 1e-6
    for a, ga in zip(range(5), grads):
        x = args[a]
        for idx in [tuple(rng.integers(0, n) for n in x.shape) for _ in range(6)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            ap, am = list(args), list(args)
            ap[a], am[a] = xp, xm
            fd = (loss(*ap) - loss(*am)) / (2 * eps)
            assert abs(fd - ga[idx]) <= 1e-7 * max(1.0, abs(fd)), (a, idx, fd, ga[idx])


def test_gla_bwd_zero_gate_brute_force():
    """g = 0: o_t = sum_{s<=t} (q_t . k_s) v_s + S0^T q_t, whose gradients have closed forms:
    dq_t = sum_{s<=t} (do_t . v_s) k_s + S0 do_t, dv_s = sum_{t>=s} (q_t . k_s) do_t,
    dk_s = sum_{t>=s} (do_t . v_s) q_t, dS0 = sum_t q_t do_t^T (no final-state gradient)."""
    B, T, H, D = 1, 9, 1, 4
    rng = np.random.default_rng(8)
    q, k, v, do = rng.standard_normal((4, B, T, H, D))
    s0 = rng.standard_normal((B, H, D, D))
    g = np.zeros((B, T, H, D))
    dq, dk, dv, dg, ds0 = O.gla_bwd(q, k, v, g, s0, do, None)
    Q, K, V, DO = q[0, :, 0], k[0, :, 0], v[0, :, 0], do[0, :, 0]
    M = np.tril(np.ones((T, T)))
    np.testing.assert_allclose(dq[0, :, 0], (M * (DO @ V.T)) @ K + DO @ s0[0, 0].T, atol=1e-12)
    np.testing.assert_allclose(dv[0, :, 0], (M * (Q @ K.T)).T @ DO, atol=1e-12)
    np.testing.assert_allclose(dk[0, :, 0], (M * (DO @ V.T)).T @ Q, atol=1e-12)
    np.testing.assert_allclose(ds0[0, 0], Q.T @ DO, atol=1e-12)


def _torch_gdn(q, k, v, g, beta, s0, kind):
    """fp64 restatement of the reference's fast_recurrent_gated_deltanet loop (fast_gla.py:811-834)
    for autograd; kind 3 scales columns (the Triton kernel's per-value beta, fast_gla.py:464-465)."""
    B, T, H, Dk = q.shape
    S = s0 if s0 is not None else torch.zeros(B, H, Dk, v.shape[-1], dtype=torch.float64)
    d = torch.exp(torch.clamp(g, max=0.0))
    outs = []
    for t in range(T):
        u = v[:, t] - (k[:, t].unsqueeze(-2) @ S).squeeze(-2)
        W = k[:, t].unsqueeze(-1) @ u.unsqueeze(-2)
        if kind == 1:
            W = beta[:, t][..., None, None] * W
        elif kind == 2:
            W = beta[:, t].unsqueeze(-1) * W
        elif kind == 3:
            W = beta[:, t].unsqueeze(-2) * W
        S = S * d[:, t].unsqueeze(-1) + W
        outs.append((q[:, t].unsqueeze(-2) @ S).squeeze(-2))
    return torch.stack(outs, dim=1), S


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("T,with_init", [(1, True), (9, False), (23, True)])
def test_gdn_bwd_matches_autograd(kind, T, with_init):
    """Every gradient (q, k, v, g, beta, S0) of the Gated DeltaNet variant equals torch autograd
    through the fp64 loop, including the clamp mask (positive and exactly-zero gates)."""
    B, H, D = 2, 2, 5
    rng = np.random.default_rng(100 * kind + T)
    q, k, v = (torch.tensor(rng.standard_normal((B, T, H, D)), requires_grad=True) for _ in range(3))
    gn = -np.abs(rng.standard_normal((B, T, H, D)))
    gn[:, ::3, :, 0] = 0.2  # clamped: zero gradient
    gn[:, 1::4, :, 1] = 0.0  # the clamp's boundary: the gradient passes
    g = torch.tensor(gn, requires_grad=True)
    beta = None
    if kind == 1:
        beta = torch.tensor(rng.uniform(0.1, 1.0, (B, T, H)), requires_grad=True)
    elif kind in (2, 3):
        beta = torch.tensor(rng.uniform(0.1, 1.0, (B, T, H, D)), requires_grad=True)
    s0 = torch.tensor(rng.standard_normal((B, H, D, D)), requires_grad=True) if with_init else None
    do = torch.tensor(rng.standard_normal((B, T, H, D)))
    dsf = torch.tensor(rng.standard_normal((B, H, D, D)))
    o, s = _torch_gdn(q, k, v, g, beta, s0, kind)
    ((o * do).sum() + (s * dsf).sum()).backward()
    dq, dk, dv, dg, db, ds0 = O.gdn_bwd(q, k, v, g, beta, s0, do, dsf, beta_kind=kind if kind >= 2 else None)
    for got, ref in ((dq, q.grad), (dk, k.grad), (dv, v.grad), (dg, g.grad)):
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-11, atol=1e-11)
    if beta is not None:
        np.testing.assert_allclose(db, beta.grad.numpy(), rtol=1e-11, atol=1e-11)
    if with_init:
        np.testing.assert_allclose(ds0, s0.grad.numpy(), rtol=1e-11, atol=1e-11)
    # the loop itself is the oracle's forward
    of, sf = O.gdn_fwd(q, k, v, g, beta, s0, beta_kind=kind if kind >= 2 else None)
    np.testing.assert_allclose(of, o.detach().numpy(), atol=1e-12)


@pytest.mark.parametrize("kind", [1, 2])
def test_gdn_bwd_finite_differences(kind):
    """Central differences of the oracle's own Gated DeltaNet forward agree with its backward."""
    B, T, H, D = 1, 5, 1, 3
    rng = np.random.default_rng(7 + kind)
    q, k, v = rng.standard_normal((3, B, T, H, D))
    g = -0.2 - np.abs(rng.standard_normal((B, T, H, D)))
    beta = rng.uniform(0.2, 0.9, (B, T, H) if kind == 1 else (B, T, H, D))
    s0 = rng.standard_normal((B, H, D, D))
    W = rng.standard_normal((B, T, H, D))
    U = rng.standard_normal((B, H, D, D))

    def loss(q, k, v, g, beta, s0):
        o, s = O.gdn_fwd(q, k, v, g, beta, s0)
        return float((o * W).sum() + (s * U).sum())

    dq, dk, dv, dg, db, ds0 = O.gdn_bwd(q, k, v, g, beta, s0, W, U)
    args = [q, k, v, g, beta, s0]
    eps = 1e-6
    for a, ga in enumerate((dq, dk, dv, dg, db, ds0)):
        x = args[a]
        for idx in [tuple(rng.integers(0, n) for n in x.shape) for _ in range(5)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            ap, am = list(args), list(args)
            ap[a], am[a] = xp, xm
            fd = (loss(*ap) - loss(*am)) / (2 * eps)
            assert abs(fd - ga[idx]) <= 1e-7 * max(1.0, abs(fd)), (a, idx, fd, ga[idx])


@pytest.mark.parametrize("with_init", [False, True])
def test_scan_bwd_matches_autograd(with_init):
    """The reference's own check (test_kernels.py:236-264), in fp64: autograd through the
    sequential addcmul loop."""
    B, H, N, Dk, Dv = 2, 3, 7, 4, 5
    rng = np.random.default_rng(11 + with_init)
    kv = torch.tensor(rng.standard_normal((B, H, N, Dk, Dv)), requires_grad=True)
    dec = torch.tensor(rng.random((B, H, N, Dk, 1)), requires_grad=True)
    init = torch.tensor(rng.standard_normal((B, H, Dk, Dv)) if with_init else np.zeros((B, H, Dk, Dv)),
                        requires_grad=True)
    cur, states = init, []
    for i in range(N):
        states.append(cur)
        cur = torch.addcmul(kv[:, :, i], cur, dec[:, :, i])
    s_all = torch.stack(states, dim=2)
    gs = torch.tensor(rng.standard_normal(s_all.shape))
    gf = torch.tensor(rng.standard_normal(cur.shape))
    ((s_all * gs).sum() + (cur * gf).sum()).backward()
    d_kv, d_dec, d_init = O.recurrent_scan_bwd(gs, gf, dec, s_all.detach())
    np.testing.assert_allclose(d_kv, kv.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(d_dec, dec.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(d_init, init.grad.numpy(), rtol=1e-12, atol=1e-12)
    d_kv0, _, d_init0 = O.recurrent_scan_bwd(None, gf, dec, s_all.detach())
    assert np.abs(d_kv0[:, :, -1] - gf.numpy()).max() == 0.0  # the last step sees only d_fin
