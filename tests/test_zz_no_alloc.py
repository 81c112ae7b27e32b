"""GPU check of the allocation-free prefill entry point (triune_hip_gla_prefill_noalloc) against
the workspace-taking triune_hip_gla_prefill, through the C ABI.

The two entry points run the same kernels on the same segment plan, so outputs and final states
must agree bit for bit.  Calls in a row share the GPU's static scratch: the second call is
smaller than the first, so it runs over the first call's leftovers and must not depend on them.
A call that needs more than the scratch returns TRIUNE_ERR_SCRATCH and launches nothing (checked on
the host, tests/test_abi_host.py).
"""

import pytest
import torch

from triune_amd._lib import check, dtype_code, lib, ptr, stream_of, strides
from triune_amd.fast_gla import _tok3, gla_prefill_noalloc
from triune_amd.workloads import config1, gla_inputs

pytestmark = pytest.mark.gpu

def _dev(xs, dev):
    return [None if x is None else x.to(dev) for x in xs]


def _args(q, k, v, g, s0, o, sf):
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    st = strides(_tok3(q), _tok3(k), _tok3(v), _tok3(g), _tok3(o))
    head = (ptr(q), ptr(k), ptr(v), ptr(g), dtype_code(q), dtype_code(g), st, ptr(s0), ptr(o), dtype_code(o), ptr(sf),
            B, T, H, Dk, Dv, 0)
    return head


def _with_workspace(q, k, v, g, s0, out_dtype):
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = torch.empty(B, T, H, Dv, device=q.device, dtype=out_dtype)
    sf = torch.empty(B, H, Dk, Dv, device=q.device)
    L = lib()
    wsb = int(L.triune_hip_gla_prefill_workspace_size(B, T, H, Dk, Dv, 0))
    ws = torch.empty(wsb, device=q.device, dtype=torch.uint8)
    check(L.triune_hip_gla_prefill(*_args(q, k, v, g, s0, o, sf), ptr(ws), wsb, stream_of(q)), "prefill")
    return o, sf, wsb


def _noalloc(q, k, v, g, s0, out_dtype):
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = torch.full((B, T, H, Dv), float("nan"), device=q.device, dtype=out_dtype)
    sf = torch.full((B, H, Dk, Dv), float("nan"), device=q.device)
    check(lib().triune_hip_gla_prefill_noalloc(*_args(q, k, v, g, s0, o, sf), stream_of(q)), "prefill_noalloc")
    return o, sf


def test_noalloc_matches_workspace_entry_on_consecutive_calls(dev):
    """Config 1 in full, then a smaller ragged call (T % 64 != 0) and a D = 128 call, each against
    the workspace-taking entry point on the same inputs."""
    cases = [
        (config1(), torch.bfloat16),
        (gla_inputs(2, 1000, 3, 64, seed=5, dtype=torch.bfloat16, init_std=0.1), torch.float32),
        (gla_inputs(1, 300, 2, 128, seed=6, dtype=torch.bfloat16, init_std=0.1), torch.bfloat16),
    ]
    cap = int(lib().triune_hip_gla_prefill_noalloc_max_bytes())
    assert cap == 32 << 20
    for i, ((q, k, v, g, s0), odt) in enumerate(cases):
        qd, kd, vd, gd, sd = _dev((q, k, v, g, s0), dev)
        o_ref, s_ref, wsb = _with_workspace(qd, kd, vd, gd, sd, odt)
        assert wsb <= cap
        o, s = _noalloc(qd, kd, vd, gd, sd, odt)
        torch.cuda.synchronize()
        print(f"call {i}: shape {tuple(q.shape)}, workspace {wsb} B, equal o {torch.equal(o, o_ref)}, "
              f"equal S {torch.equal(s, s_ref)}", flush=True)
        assert torch.equal(o, o_ref) and torch.equal(s, s_ref), i


def test_noalloc_python_wrapper_and_limits(dev):
    q, k, v, g, s0 = _dev(gla_inputs(2, 256, 3, 64, seed=8, dtype=torch.bfloat16, init_std=0.1), dev)
    o_ref, s_ref, _ = _with_workspace(q, k, v, g, s0, torch.bfloat16)
    out = torch.empty_like(v)
    fin = torch.empty_like(s_ref)
    o, s = gla_prefill_noalloc(q, k, v, g, s0, out, fin)
    torch.cuda.synchronize()
    assert o.data_ptr() == out.data_ptr() and torch.equal(o, o_ref) and torch.equal(s, s_ref)
    with pytest.raises(ValueError):  # a layout that would need a copy is refused, not copied
        gla_prefill_noalloc(q, k, v, g[:, :1].expand_as(g), s0, out, fin)
    # a call needing more than the scratch (TRIUNE_ERR_SCRATCH, nothing launched) is checked on the
    # host only (tests/test_abi_host.py::test_noalloc_prefill_validation)
