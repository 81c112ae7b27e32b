"""Writes tests/golden/gdn_reference_cpu.npz: input/output vectors of the reference's
fast_recurrent_gated_deltanet (triune/kernels/fast_gla.py:781-836) on tiny fp64 CPU inputs.

Run once, in the build container that holds the reference tree (read from REF_ROOT, default
/root/reference).  Only the generated vectors are committed; the reference code is not.
The GDN variant (prediction from the un-decayed state, beta orientation) is the one function of
the oracle that no closed form or reference test pins, hence these vectors.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

REF_ROOT = os.environ.get("REF_ROOT", "/root/reference")
OUT = Path(__file__).resolve().parent / "gdn_reference_cpu.npz"


def main() -> None:
    sys.path.insert(0, REF_ROOT)
    from triune.kernels.fast_gla import fast_recurrent_gated_deltanet  # reference, CPU path

    gen = torch.Generator().manual_seed(2024)
    B, T, H, D = 1, 16, 2, 8
    arrays = {}
    for name, beta_kind in [("none", None), ("head", "head"), ("key", "key")]:
        q = torch.randn(B, T, H, D, generator=gen, dtype=torch.float64)
        k = torch.nn.functional.normalize(torch.randn(B, T, H, D, generator=gen, dtype=torch.float64), dim=-1)
        v = torch.randn(B, T, H, D, generator=gen, dtype=torch.float64)
        g = 0.4 * torch.randn(B, T, H, D, generator=gen, dtype=torch.float64)  # includes g > 0 (clamped)
        s0 = 0.5 * torch.randn(B, H, D, D, generator=gen, dtype=torch.float64)
        beta = None
        if beta_kind == "head":
            beta = torch.rand(B, T, H, generator=gen, dtype=torch.float64)
        elif beta_kind == "key":
            beta = torch.rand(B, T, H, D, generator=gen, dtype=torch.float64)
        with torch.no_grad():
            o, s = fast_recurrent_gated_deltanet(q, k, v, g, beta=beta, initial_state=s0)
        for key, val in dict(q=q, k=k, v=v, g=g, s0=s0, o=o, s=s).items():
            arrays[f"{name}_{key}"] = val.numpy()
        if beta is not None:
            arrays[f"{name}_beta"] = beta.numpy()
    np.savez(OUT, **arrays)
    print(f"wrote {OUT} ({len(arrays)} arrays)")


if __name__ == "__main__":
    main()
