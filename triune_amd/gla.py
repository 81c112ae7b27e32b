"""Operator namespace mirroring the reference's triune.ops.gla (triune/ops/gla.py:10-61).

gla(...) and gated_deltanet(...) keep the reference's signatures and return tuples and run on
libtriune_hip.so.  The reference routes CPU fp32 single-token calls to its native C step
(ops/gla.py:47-59); here every call runs the HIP kernels and CPU tensors are rejected.
"""

from __future__ import annotations

import torch

from .fast_gla import fast_chunk_gated_deltanet, fast_chunk_gla


def gated_deltanet(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    chunk_size: int = 64,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gated DeltaNet forward (reference: triune/ops/gla.py:10-23)."""
    return fast_chunk_gated_deltanet(q, k, v, g, beta=beta, initial_state=initial_state, chunk_size=chunk_size)


def gla(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    chunk_size: int = 64,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Chunked GLA forward, [B, T, H, D] inputs, returns (output, final_state)
    (reference: triune/ops/gla.py:26-61)."""
    return fast_chunk_gla(q, k, v, g, initial_state=initial_state, chunk_size=chunk_size)
