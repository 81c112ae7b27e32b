"""Seeded synthetic inputs for the benchmark configurations of the GLA path.

Config k uses seed k and draws, in order, q, k, v, g, (beta), initial state, on a CPU
torch.Generator, so every consumer (tests, bench, oracle) sees identical values.  16-bit
configs round to bf16 once, here; checkers consume the rounded values.

  0  GLA fp32:        B=1,  H=6,  T=2048,  D=64;  q ~ N(0,1)/sqrt(D), k,v ~ N(0,1),
                      g = logsigmoid(N(0,1))/16, zero initial state
  1  GLA prefill:     B=4,  H=6,  T=16384, D=64;  same draws, bf16 I/O, S0 = 0.1 N(0,1) fp32
  2  GLA decode:      B=256, H=6, D=64; S0 = 0.1 N(0,1) fp32; per step q,k,v ~ N(0,1) bf16,
                      g = logsigmoid(N(0,1))/16 (bf16)
  3  Gated DeltaNet:  B=4,  H=6,  T=8192,  D=64;  q,k L2-normalised per head, v ~ N(0,1),
                      beta = sigmoid(N(0,1)) [B,T,H], alpha = exp(-softplus(N(0,1))/8) [B,T,H],
                      g = log(alpha) broadcast over D, zero initial state, bf16
  4  ragged GLA:      32 sequences, lengths ~ U[128, 8192], packed [1, sum L, 12, 128] bf16,
                      cu_seqlens int32, S0 = 0.1 N(0,1) fp32 per sequence
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def gla_inputs(B, T, H, D, *, seed, dtype=torch.bfloat16, scale_q=True, init_std=0.0, Dv=None):
    """q, k, v, g (and S0 or None) with the GLA config distributions."""
    Dv = Dv or D
    gen = _gen(seed)
    q = torch.randn(B, T, H, D, generator=gen)
    if scale_q:
        q = q * D**-0.5
    k = torch.randn(B, T, H, D, generator=gen)
    v = torch.randn(B, T, H, Dv, generator=gen)
    g = F.logsigmoid(torch.randn(B, T, H, D, generator=gen)) / 16
    s0 = init_std * torch.randn(B, H, D, Dv, generator=gen) if init_std > 0 else None
    q, k, v, g = (x.to(dtype) for x in (q, k, v, g))
    return q, k, v, g, s0


def config0(T=2048, B=1, H=6, D=64):
    return gla_inputs(B, T, H, D, seed=0, dtype=torch.float32)


def config1(T=16384, B=4, H=6, D=64):
    return gla_inputs(B, T, H, D, seed=1, dtype=torch.bfloat16, init_std=0.1)


def config2(steps=512, B=256, H=6, D=64, dtype=torch.bfloat16):
    """(q, k, v, g) each [steps, B, 1, H, D] and S0 [B, H, D, D] fp32."""
    gen = _gen(2)
    s0 = 0.1 * torch.randn(B, H, D, D, generator=gen)
    q = torch.randn(steps, B, 1, H, D, generator=gen)
    k = torch.randn(steps, B, 1, H, D, generator=gen)
    v = torch.randn(steps, B, 1, H, D, generator=gen)
    g = F.logsigmoid(torch.randn(steps, B, 1, H, D, generator=gen)) / 16
    return q.to(dtype), k.to(dtype), v.to(dtype), g.to(dtype), s0


def config3(T=8192, B=4, H=6, D=64, dtype=torch.bfloat16):
    """q, k, v [B,T,H,D], g [B,T,H,D] broadcast over D (a stride-0 view of the per-(token, head)
    log-decay), beta [B,T,H]; zero initial state.  Move g with to_device to keep it a view."""
    gen = _gen(3)
    q = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    v = torch.randn(B, T, H, D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    alpha = torch.exp(-F.softplus(torch.randn(B, T, H, generator=gen)) / 8)
    g = torch.log(alpha).to(dtype).unsqueeze(-1).expand(B, T, H, D)
    return q.to(dtype), k.to(dtype), v.to(dtype), g, beta.to(dtype)


def to_device(x, dev):
    """x on dev.  A tensor broadcast along some dims (stride 0 there, as expand makes it) moves
    once and stays a broadcast view on dev; x.to(dev) would materialise it."""
    if x.dim() and any(st == 0 and n > 1 for n, st in zip(x.shape, x.stride())):
        idx = tuple(slice(0, 1) if (st == 0 and n > 1) else slice(None) for n, st in zip(x.shape, x.stride()))
        return x[idx].to(dev).expand(x.shape)
    return x.to(dev)


def config4_lengths(n_seqs=32, lo=128, hi=8192, seed=4) -> list[int]:
    gen = _gen(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n_seqs,), generator=gen)]


def config4(n_seqs=32, H=12, D=128, lo=128, hi=8192, dtype=torch.bfloat16):
    """Packed q, k, v, g [1, N, H, D], cu_seqlens int32 [n+1], S0 [n, H, D, D] fp32."""
    lens = config4_lengths(n_seqs, lo, hi)
    gen = _gen(40)
    N = sum(lens)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    q = torch.randn(1, N, H, D, generator=gen) * D**-0.5
    k = torch.randn(1, N, H, D, generator=gen)
    v = torch.randn(1, N, H, D, generator=gen)
    g = F.logsigmoid(torch.randn(1, N, H, D, generator=gen)) / 16
    s0 = 0.1 * torch.randn(n_seqs, H, D, D, generator=gen)
    return q.to(dtype), k.to(dtype), v.to(dtype), g.to(dtype), cu, s0


def gla_algorithmic_bytes(n_tok_heads: int, Dk: int, Dv: int, io_bytes: int, g_bytes: int, out_bytes: int) -> int:
    """HBM bytes a prefill must move at minimum: read q, k, g (Dk) and v (Dv), write o (Dv)."""
    return n_tok_heads * (Dk * (2 * io_bytes + g_bytes) + Dv * (io_bytes + out_bytes))


def gla_algorithmic_flops(n_tok_heads: int, Dk: int, Dv: int, chunk: int = 64) -> int:
    """Dense-tile chunked flops per token-head: q k^T (C*Dk), A v (C*Dv), q S (Dk*Dv),
    k^T v (Dk*Dv), 2 flops per multiply-add."""
    return n_tok_heads * 2 * (chunk * Dk + chunk * Dv + 2 * Dk * Dv)


def ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (for 1-ULP comparisons of bf16 outputs)."""
    a = x.abs().float().clamp_min(2.0**-126)
    e = torch.floor(torch.log2(a))
    return torch.exp2(e - 7)


def log2ceil(n: int) -> int:
    return int(math.ceil(math.log2(max(n, 1))))
