"""CPU restatement ("port") of the reference's PyTorch GLA scan, for the CPU baseline.

TEST / BASELINE INFRASTRUCTURE ONLY: timed by bench.py's cpu_baseline leg and checked against
the fp64 oracle by tests/.  triune_amd never imports it.

It follows the reference's op sequence on CPU under torch.no_grad():
  triune/kernels/fast_gla.py:569-689  _run_gla_chunks
    - view [B, T, H, D] as [B, H, N, C, D] chunks; clamp g at 0; cumulative sum over each chunk
    - intra-chunk: if every chunk's decay span is below 55 nats, factor the pairwise decay
      through the per-chunk midpoint m = (G_first + G_last)/2:  (q e^{G-m}) (k e^{m-G})^T,
      causal-masked, cast to the input dtype, times v, evaluated 4 chunks at a time;
      otherwise the pairwise clamped-difference form one chunk at a time
    - inter-chunk: k e^{G_last - G} (clamped at 0) contracted with v per chunk, carried by a
      Hillis-Steele doubling scan (no grad, >= 8 chunks) or a sequential loop, then q e^{G}
      times the state entering each chunk
  triune/kernels/fast_gla.py:692-778  fast_chunk_gla dispatch (T == 1 decode step, T < C single
    chunk, whole chunks plus a remainder that is a decode step when it is one token)
Written independently for this repository; only the algorithm's steps are shared.
"""

from __future__ import annotations

import torch


def _chunks(x: torch.Tensor, C: int) -> torch.Tensor:
    B, T, H, D = x.shape
    return x.reshape(B, T // C, C, H, D).permute(0, 3, 1, 2, 4)  # [B, H, N, C, D]


def _decode_step(q, k, v, g, S):
    """T == 1 expression of the reference (no clamp): S <- e^g S + k v^T ; o = q S."""
    S = S * torch.exp(g[:, 0]).unsqueeze(-1) + k[:, 0].unsqueeze(-1) * v[:, 0].unsqueeze(-2)
    o = (q[:, 0].unsqueeze(-2) @ S).squeeze(-2).unsqueeze(1)
    return o, S


def run_chunks(q, k, v, g, S, C):
    """Chunked GLA over T = N*C tokens from state S [B, H, D, D]; returns (o, S)."""
    B, T, H, D = q.shape
    N = T // C
    dt = q.dtype
    qc, kc, vc = _chunks(q, C), _chunks(k, C), _chunks(v, C)
    G = torch.cumsum(_chunks(g, C).clamp(max=0.0), dim=-2)  # [B, H, N, C, D]
    upper = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=1)

    span_ok = bool(((G[..., :1, :] - G[..., -1:, :]).max() < 55.0).item())
    if span_ok and dt != torch.float64:
        mid = 0.5 * (G[..., :1, :].float() + G[..., -1:, :].float())
        qf = qc.float() * torch.exp(G.float() - mid)
        kf = kc.float() * torch.exp(mid - G.float())
        parts = []
        for a in range(0, N, 4):
            b = min(a + 4, N)
            att = (qf[:, :, a:b] @ kf[:, :, a:b].transpose(-1, -2)).masked_fill(upper, 0.0).to(dt)
            parts.append(att @ vc[:, :, a:b])
        intra = torch.cat(parts, dim=2)
    else:
        parts = []
        for n in range(N):
            Gn = G[:, :, n].float() if dt != torch.float64 else G[:, :, n]
            dlt = (Gn.unsqueeze(-2) - Gn.unsqueeze(-3)).clamp(max=0.0)  # [B, H, C, C, D]
            qq = qc[:, :, n].to(dlt.dtype).unsqueeze(-2)
            kk = kc[:, :, n].to(dlt.dtype).unsqueeze(-3)
            att = (qq * kk * torch.exp(dlt)).sum(-1).masked_fill(upper, 0.0).to(dt)
            parts.append((att @ vc[:, :, n]).unsqueeze(2))
        intra = torch.cat(parts, dim=2)

    Glast = G[..., -1:, :]
    kdec = kc * torch.exp((Glast - G).clamp(max=0.0))
    a = torch.exp(Glast).squeeze(-2).unsqueeze(-1)  # [B, H, N, D, 1]
    qexp = qc * torch.exp(G)
    kv = kdec.transpose(-1, -2) @ vc  # [B, H, N, D, D]
    if N == 1:
        inter = qexp @ S.unsqueeze(2)
        S = kv[:, :, 0] + S * a[:, :, 0]
    elif N >= 8:
        kv[:, :, 0] += S * a[:, :, 0]
        acc = a.clone()
        step = 1
        while step < N:
            kv[:, :, step:] += acc[:, :, step:] * kv[:, :, :-step]
            if 2 * step < N:
                acc[:, :, step:] *= acc[:, :, :-step].clone()
            step *= 2
        entering = torch.cat([S.unsqueeze(2), kv[:, :, :-1]], dim=2)
        S = kv[:, :, -1]
        inter = qexp @ entering
    else:
        entering = []
        for n in range(N):
            entering.append(S)
            S = kv[:, :, n] + S * a[:, :, n]
        inter = qexp @ torch.stack(entering, dim=2)
    o = (intra + inter).permute(0, 2, 3, 1, 4).reshape(B, T, H, D)
    return o, S


@torch.no_grad()
def fast_chunk_gla_cpu(q, k, v, g, initial_state=None, chunk_size=64):
    """fast_chunk_gla's CPU path: returns (o, final_state) in q.dtype."""
    B, T, H, D = q.shape
    S = initial_state.to(q.dtype) if initial_state is not None else torch.zeros(B, H, D, D, dtype=q.dtype)
    if T == 1:
        return _decode_step(q, k, v, g, S)
    C = chunk_size
    if T < C:
        return run_chunks(q, k, v, g, S, T)
    Tc = (T // C) * C
    o, S = run_chunks(q[:, :Tc], k[:, :Tc], v[:, :Tc], g[:, :Tc], S, C)
    if Tc == T:
        return o, S
    if T - Tc == 1:
        o2, S = _decode_step(q[:, Tc:], k[:, Tc:], v[:, Tc:], g[:, Tc:], S)
    else:
        o2, S = run_chunks(q[:, Tc:], k[:, Tc:], v[:, Tc:], g[:, Tc:], S, T - Tc)
    return torch.cat([o, o2], dim=1), S


@torch.no_grad()
def decode_step_cpu(q, k, v, g, S):
    """Batched decode step at [B, 1, H, D] (fast_gla.py:746-753 expression)."""
    return _decode_step(q, k, v, g, S)
