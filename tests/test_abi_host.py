"""CPU tests of the C-ABI boundary and the host-side logic (no GPU compute is launched).

Every call here fails argument validation before any HIP API is touched, so these run in a
container without a GPU."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import triune_amd
import triune_amd._lib as L

HEADER = Path(__file__).resolve().parents[1] / "include" / "triune_hip.h"


# entry points declared under the reference's own names (device twins of its decode step)
REFERENCE_NAMED = ("launch_gla_decode_step", "triune_gla_recurrent_step_f32")


def _declared():
    text = HEADER.read_text()
    names = set(re.findall(r"\b(triune_hip_\w+)\s*\(", text))
    names |= {n for n in REFERENCE_NAMED if re.search(r"\bvoid\s+" + n + r"\s*\(", text)}
    return sorted(names)


def test_library_exports_every_declared_entry_point():
    lib = L.lib()
    declared = _declared()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/triune_hip.h but not exported"
    assert set(declared) == set(L.EXPORTS)


def test_abi_version_matches_header():
    m = re.search(r"#define TRIUNE_HIP_ABI_VERSION (\d+)", HEADER.read_text())
    assert L.lib().triune_hip_abi_version() == int(m.group(1))


def test_error_strings_and_codes_match_header():
    text = HEADER.read_text()
    codes = {k: int(v) for k, v in re.findall(r"(TRIUNE_ERR_\w+) = (-\d+)", text)}
    assert codes == {
        "TRIUNE_ERR_NULL": -1,
        "TRIUNE_ERR_SHAPE": -2,
        "TRIUNE_ERR_DTYPE": -3,
        "TRIUNE_ERR_LAYOUT": -4,
        "TRIUNE_ERR_WORKSPACE": -5,
        "TRIUNE_ERR_LAUNCH": -6,
        "TRIUNE_ERR_SCRATCH": -7,
        "TRIUNE_ERR_MEMORY": -8,
    }
    lib = L.lib()
    for c in [0, *codes.values()]:
        assert lib.triune_hip_error_string(c)
    assert lib.triune_hip_error_string(-99) == b"unknown error"


_FAKE = ctypes.c_void_p(0x1000)  # 16-byte aligned, never dereferenced: validation fails first


def test_reference_twins_refuse_host_memory():
    """The reference's caller of triune_gla_recurrent_step_f32 (triune/ops/_c_bridge.py:259-294,
    guard at :272) hands over host pointers of CPU fp32 tensors; launch_gla_decode_step's caller
    (csrc/kernels/gla.cu:97-114) device pointers.  Given host memory, both twins ask the runtime
    where the pointers live, launch nothing, leave every buffer as it was and report
    TRIUNE_ERR_MEMORY (-8); the reference's own step on the same rows (the fp64 oracle, which is
    pinned to it) is what such a caller computes on the CPU."""
    lib = L.lib()
    gen = torch.Generator().manual_seed(5)
    bh, d = 6, 64
    q, k, v = (torch.randn(bh, d, generator=gen) for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(bh, d, generator=gen)) / 16
    state = 0.1 * torch.randn(bh, d, d, generator=gen)
    out = torch.full((bh, d), 7.0)
    before = [t.clone() for t in (q, k, v, g, state, out)]
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    lib.triune_gla_recurrent_step_f32(ptr(q), ptr(k), ptr(v), ptr(g), ptr(state), ptr(out), bh, d)
    assert lib.triune_hip_last_error() == -8
    for a, b in zip((q, k, v, g, state, out), before):
        assert torch.equal(a, b)
    qb, kb, vb, ob = (t.bfloat16() for t in (q, k, v, out))
    lib.launch_gla_decode_step(ptr(qb), ptr(kb), ptr(vb), ptr(g), ptr(state), ptr(ob), 1, bh, d, None)
    assert lib.triune_hip_last_error() == -8
    assert torch.equal(state, before[4]) and torch.equal(ob, before[5].bfloat16())
    assert b"device memory" in lib.triune_hip_error_string(-8)


def test_output_kernel_event_hook_arms_and_disarms():
    lib = L.lib()
    assert lib.triune_hip_set_output_kernel_events(_FAKE, None) == -1  # exactly one NULL
    assert lib.triune_hip_set_output_kernel_events(None, _FAKE) == -1
    assert lib.triune_hip_set_output_kernel_events(None, None) == 0  # disarmed (nothing recorded)


def _st(n):
    return (ctypes.c_int64 * n)(*([64] * n))


def test_prefill_validation_errors():
    lib = L.lib()
    f = lib.triune_hip_gla_prefill
    ok_args = dict(q=_FAKE, k=_FAKE, v=_FAKE, g=_FAKE, io=1, gdt=1, st=_st(15), s0=None, o=_FAKE, odt=1, sf=None,
                   B=1, T=64, H=1, Dk=64, Dv=64, flags=0, ws=None, wsb=0, stream=None)

    def call(**kw):
        a = {**ok_args, **kw}
        return f(a["q"], a["k"], a["v"], a["g"], a["io"], a["gdt"], a["st"], a["s0"], a["o"], a["odt"], a["sf"],
                 a["B"], a["T"], a["H"], a["Dk"], a["Dv"], a["flags"], a["ws"], a["wsb"], a["stream"])

    assert call(q=None) == -1
    assert call(io=7) == -3
    assert call(Dk=48) == -2
    assert call(Dv=40) == -2
    assert call(H=0) == -2
    assert call(st=(ctypes.c_int64 * 15)(*([63] * 15))) == -4  # rows not 16-byte aligned
    assert call(q=ctypes.c_void_p(0x1002)) == -4
    # token rows closer than a row width (a tensor broadcast along tokens) are refused
    assert call(st=(ctypes.c_int64 * 15)(*([4096, 0, 64] * 5))) == -4
    assert call(st=(ctypes.c_int64 * 15)(*([4096, 32, 64] * 5))) == -4
    assert call(ws=None, wsb=0) == -5  # workspace required once T > 0


def test_decode_and_gdn_and_scan_validation_errors():
    lib = L.lib()
    d = lib.triune_hip_gla_decode_step
    assert d(None, _FAKE, _FAKE, _FAKE, 1, 1, _st(10), _FAKE, _FAKE, None, 1, _FAKE, 1, 1, 1, 64, 64, None) == -1
    assert d(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _st(10), _FAKE, _FAKE, None, 1, _FAKE, 1, 1, 1, 64, 32, None) == -2
    assert d(_FAKE, _FAKE, _FAKE, _FAKE, 5, 1, _st(10), _FAKE, _FAKE, None, 1, _FAKE, 1, 1, 1, 64, 64, None) == -3
    # without slots the state must hold a row per batch entry
    assert d(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _st(10), _FAKE, _FAKE, None, 1, _FAKE, 1, 2, 1, 64, 64, None) == -2
    # the reference-signature twins report through triune_hip_last_error and launch nothing on bad sizes
    lib.launch_gla_decode_step(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 1, 1, 48, None)
    assert lib.triune_hip_last_error() == -2
    lib.triune_gla_recurrent_step_f32(None, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 1, 64)
    assert lib.triune_hip_last_error() == -1
    lib.triune_gla_recurrent_step_f32(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 1, 48)
    assert lib.triune_hip_last_error() == -2
    gdn = lib.triune_hip_gdn_prefill
    assert gdn(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 1, _st(18), None, _FAKE, 1, None, 1, 8, 1, 64, 64, None) == -1
    assert gdn(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 9, _st(18), None, _FAKE, 1, None, 1, 8, 1, 64, 64, None) == -2
    assert gdn(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 0, _st(18), None, _FAKE, 1, None, 1, 8, 1, 48, 48, None) == -2
    # chunked GDN: beta's strides (12..14, zero without beta) are not mistaken for o's (15..17);
    # valid arguments without a workspace fail on the workspace, not on the layout
    gc = lib.triune_hip_gdn_prefill_chunked
    gst = (ctypes.c_int64 * 18)(*([64 * 64, 64, 64] * 4 + [0, 0, 0] + [64 * 64, 64, 64]))
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 0, gst, None, _FAKE, 1, None, 1, 64, 1, 64, 64, None, 0,
              None) == -5
    gst[16] = 32  # o's token stride below the row width
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 0, gst, None, _FAKE, 1, None, 1, 64, 1, 64, 64, None, 0,
              None) == -4
    # head dim 128: 16-bit I/O only (fp32 planes exceed the LDS), square heads only
    g128 = (ctypes.c_int64 * 18)(*([128 * 128, 128, 128] * 4 + [0, 0, 0] + [128 * 128, 128, 128]))
    for io, want in ((1, -5), (2, -5), (0, -3)):
        assert gc(_FAKE, _FAKE, _FAKE, _FAKE, io, io, None, 1, 0, g128, None, _FAKE, io, None, 1, 64, 1, 128, 128,
                  None, 0, None) == want
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, None, 1, 0, g128, None, _FAKE, 1, None, 1, 64, 1, 128, 64, None, 0,
              None) == -2
    # beta per value dim: fp32 only
    vst = (ctypes.c_int64 * 18)(*([64 * 64, 64, 64] * 5 + [64 * 64, 64, 64]))
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _FAKE, 0, 3, vst, None, _FAKE, 1, None, 1, 64, 1, 64, 64, None, 0,
              None) == -5
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _FAKE, 1, 3, vst, None, _FAKE, 1, None, 1, 64, 1, 64, 64, None, 0,
              None) == -3
    vst[13] = 32  # beta rows narrower than Dv
    assert gc(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _FAKE, 0, 3, vst, None, _FAKE, 1, None, 1, 64, 1, 64, 64, None, 0,
              None) == -4
    assert lib.triune_hip_gdn_prefill_chunked_workspace_size(4, 8192, 6, 128, 128) > 0
    assert lib.triune_hip_gdn_prefill_chunked_workspace_size(4, 8192, 6, 128, 64) == 0
    assert lib.triune_hip_gdn_prefill_chunked_workspace_size(4, 8192, 6, 32, 32) == 0
    # scalar-decay GDN: g is [B, T, H] (any non-negative strides, element-aligned), beta none or per token
    sg = lib.triune_hip_gdn_prefill_scalar_decay
    sst = (ctypes.c_int64 * 18)(*([64 * 64, 64, 64] * 3 + [64, 1, 0] + [0, 0, 0] + [64 * 64, 64, 64]))
    args = lambda g, bk, dk, sts: (_FAKE, _FAKE, _FAKE, g, 1, 1, _FAKE if bk else None, 1, bk, sts, None, _FAKE,  # noqa: E731
                                    1, None, 1, 64, 1, dk, dk, None, 0, None)
    assert sg(*args(_FAKE, 0, 64, sst)) == -5  # valid, no workspace
    assert sg(*args(_FAKE, 1, 64, sst)) == -5  # per-token beta
    assert sg(*args(_FAKE, 2, 64, sst)) == -2  # per-key-dim beta needs the per-dim kernels
    assert sg(*args(_FAKE, 0, 128, sst)) == -2
    assert sg(*args(ctypes.c_void_p(0x1001), 0, 64, sst)) == -4  # gate pointer not element-aligned
    sst[10] = -1
    assert sg(*args(_FAKE, 0, 64, sst)) == -4
    sst[10] = 0  # one gate for every token: allowed
    assert sg(*args(_FAKE, 0, 64, sst)) == -5
    assert sg(*args(None, 0, 64, sst)) == -1
    assert lib.triune_hip_gdn_prefill_scalar_decay_workspace_size(4, 8192, 6, 64, 64) > 0
    assert lib.triune_hip_gdn_prefill_scalar_decay_workspace_size(4, 8192, 6, 128, 128) == 0
    sc = lib.triune_hip_recurrent_scan_fwd
    assert sc(None, 0, _FAKE, 0, None, 0, _FAKE, _FAKE, 0, 1, 1, 4, 8, 8, None) == -1
    assert sc(_FAKE, 0, _FAKE, 0, None, 0, _FAKE, _FAKE, 0, 1, 1, 4, 8, 6, None) == -2
    assert sc(_FAKE, 4, _FAKE, 0, None, 0, _FAKE, _FAKE, 0, 1, 1, 4, 8, 8, None) == -3
    sb = lib.triune_hip_recurrent_scan_bwd
    assert sb(None, 0, None, 0, None, 0, _FAKE, _FAKE, _FAKE, _FAKE, 0, 1, 1, 4, 8, 8, None) == -1
    assert sb(None, 0, None, 0, _FAKE, 0, None, _FAKE, _FAKE, _FAKE, 0, 1, 1, 4, 8, 8, None) == -1
    assert sb(None, 0, None, 0, _FAKE, 0, _FAKE, _FAKE, _FAKE, _FAKE, 0, 1, 1, 4, 8, 260, None) == -2
    assert sb(None, 0, None, 0, _FAKE, 0, _FAKE, _FAKE, _FAKE, _FAKE, 0, 1, 1, 4, 8, 6, None) == -2
    assert sb(None, 0, _FAKE, 7, _FAKE, 0, _FAKE, _FAKE, _FAKE, _FAKE, 0, 1, 1, 4, 8, 8, None) == -3


def test_fused_decode_pool_validation():
    """The pool form of the fused decode step: slots and the pool are required, sizes checked
    before any launch (no GPU call is made on these paths)."""
    lib = L.lib()
    f = lib.triune_hip_gla_fused_decode_step_slots
    st = (ctypes.c_int64 * 3)(4 * 3 * 64, 3 * 64, 64)
    ost = (ctypes.c_int64 * 2)(3 * 64, 64)
    args = lambda pool, slots, n, hd, sdt=0: (_FAKE, 1, st, None, None, 0, 0, pool, sdt, slots, n, _FAKE, 1, ost,  # noqa: E731
                                              2, 3, hd, None)
    assert f(*args(None, _FAKE, 4, 64)) == -1
    assert f(*args(_FAKE, None, 4, 64)) == -1
    assert f(*args(_FAKE, _FAKE, -1, 64)) == -2
    assert f(*args(_FAKE, _FAKE, 4, 48)) == -2
    assert f(*args(_FAKE, _FAKE, 4, 64, sdt=2)) == -3  # fp16 state with bf16 I/O
    assert f(*args(ctypes.c_void_p(0x1008), _FAKE, 4, 64)) == -4  # fp32 pool not 16-byte aligned


def test_noalloc_prefill_validation():
    """The allocation-free prefill fails before any launch on bad arguments, and with
    TRIUNE_ERR_SCRATCH when the workspace would exceed its static scratch."""
    lib = L.lib()
    f = lib.triune_hip_gla_prefill_noalloc
    cap = int(lib.triune_hip_gla_prefill_noalloc_max_bytes())
    assert cap == 32 << 20
    st = (ctypes.c_int64 * 15)(*([64 * 128 * 64, 64 * 128, 128] * 5))
    assert f(None, _FAKE, _FAKE, _FAKE, 1, 1, st, None, _FAKE, 1, None, 1, 64, 1, 128, 128, 0, None) == -1
    assert f(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, st, None, _FAKE, 1, None, 1, 64, 1, 48, 48, 0, None) == -2
    assert int(lib.triune_hip_gla_prefill_workspace_size(64, 4096, 64, 128, 128, 0)) > cap
    assert f(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, st, None, _FAKE, 1, None, 64, 4096, 64, 128, 128, 0, None) == -7
    assert b"static scratch" in lib.triune_hip_error_string(-7)


def test_bwd_accumulate_flags_need_fp32_gradients():
    """TRIUNE_FLAG_BWD_ACC_QKG / _V add into the gradient buffers, which only fp32 buffers hold
    exactly: with bf16 gradients the call is rejected before any launch."""
    lib = L.lib()
    f = lib.triune_hip_gla_prefill_bwd
    st = (ctypes.c_int64 * 27)(*([64 * 128 * 64, 64 * 128, 128] * 9))

    def call(d_dt, dg_dt, flags):
        return f(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, _FAKE, st, None, None, _FAKE, _FAKE, _FAKE, d_dt, _FAKE, dg_dt,
                 None, 1, 64, 1, 64, 64, flags, None, 0, None)

    assert call(1, 0, L.FLAG_BWD_ACC_QKG) == -3
    assert call(0, 1, L.FLAG_BWD_ACC_QKG) == -3
    assert call(1, 0, L.FLAG_BWD_ACC_V) == -3
    # fp32 gradients pass the dtype check and stop at the missing workspace
    assert call(0, 0, L.FLAG_BWD_ACC_QKG | L.FLAG_BWD_ACC_V) == -5


def test_gdn_bwd_validation():
    """The Gated DeltaNet backward entry: square heads of 64 or 128, the gradient buffers and (with
    a beta) its gradient required, rows vector-aligned; valid arguments stop at the workspace."""
    lib = L.lib()
    f = lib.triune_hip_gdn_bwd
    st = (ctypes.c_int64 * 18)(*([64 * 64, 64, 64] * 6))

    def call(bk=0, beta=None, db=None, dk=64, dv=64, dq=_FAKE, sts=st, ws=None):
        return f(_FAKE, _FAKE, _FAKE, _FAKE, 1, 1, beta, 0, bk, sts, None, _FAKE, 1, None, dq, _FAKE, _FAKE, _FAKE,
                 db, None, 1, 64, 1, dk, dv, ws, 0, None)

    assert call() == -5  # valid, no workspace
    assert call(dq=None) == -1
    assert call(bk=1, beta=_FAKE) == -1  # beta without its gradient buffer
    assert call(bk=1, beta=_FAKE, db=_FAKE) == -5
    assert call(bk=4, beta=_FAKE, db=_FAKE) == -2
    assert call(dk=32, dv=32) == -2
    assert call(dk=128, dv=64) == -2
    bad = (ctypes.c_int64 * 18)(*([64 * 64, 64, 64] * 6))
    bad[16] = 60  # dout's token stride not a multiple of 8 elements
    assert call(sts=bad) == -4
    assert lib.triune_hip_gdn_bwd_workspace_size(4, 8192, 6, 64, 64, 0) > 0
    assert lib.triune_hip_gdn_bwd_workspace_size(4, 8192, 6, 64, 64, 2) > lib.triune_hip_gdn_bwd_workspace_size(
        4, 8192, 6, 64, 64, 0)
    assert lib.triune_hip_gdn_bwd_workspace_size(4, 8192, 6, 48, 48, 0) == 0


def test_workspace_sizes():
    lib = L.lib()
    w1 = lib.triune_hip_gla_prefill_workspace_size(4, 16384, 6, 64, 64, 0)
    w2 = lib.triune_hip_gla_prefill_workspace_size(4, 2 * 16384, 6, 64, 64, 0)
    assert 0 < w1 < 64 << 20 and w1 <= w2
    assert lib.triune_hip_gla_prefill_workspace_size(1, 64, 1, 48, 64, 0) == 0
    forced = lib.triune_hip_gla_prefill_workspace_size(1, 64 * 100, 1, 64, 64, 10 << L.FLAG_SEG_SHIFT)
    assert forced >= 10 * 64 * 64 * 4  # 10 segments of one 64x64 fp32 state
    assert lib.triune_hip_gla_prefill_varlen_workspace_size(32, 133000, 12, 128, 128, 0) > 0


def test_host_layer_rejects_cpu_tensors_and_bad_dtypes():
    q = torch.zeros(1, 4, 1, 64)
    with pytest.raises(ValueError):
        triune_amd.fast_chunk_gla(q, q, q, q)
    with pytest.raises(ValueError):
        triune_amd.gla(q, q, q, q)
    with pytest.raises(ValueError):
        triune_amd.gated_deltanet(q, q, q, q)
    with pytest.raises(ValueError):
        triune_amd.FusedRecurrentScan.apply(torch.zeros(1, 1, 2, 4, 4), torch.ones(1, 1, 2, 4, 1), torch.zeros(1, 1, 4, 4))
    with pytest.raises(TypeError):
        L.dtype_code(torch.zeros(1, dtype=torch.int32))


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "_LIB", None)
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(L.TriuneHipError):
        L.lib()
