"""CPU checks of the serving helpers (triune_amd/serving.py): the reference's cache formats
(attention.py:333-358), row slicing / scattering (transformer.py:276-317) and the session
bookkeeping of StateSlotPool (the interface of SessionRecurrentStateManager, srsm.py:11-112).
The pool is created on the CPU here: bookkeeping only, no kernel runs."""

import torch

from triune_amd.serving import StateSlotPool, format_cache, parse_cache, scatter_cache, slice_cache


def test_parse_and_format_cache_round_trip():
    s = torch.ones(2, 3, 4, 4)
    assert parse_cache(None) == (None, 0, "none")
    st, off, fmt = parse_cache({"state": s, "offset": 7})
    assert st is s and off == 7 and fmt == "dict"
    st, off, fmt = parse_cache((s, 5))
    assert st is s and off == 5 and fmt == "tuple"
    st, off, fmt = parse_cache(s)
    assert st is s and off == 0 and fmt == "tensor"
    assert format_cache(s, {}, "dict", 7, 3) == {"state": s, "offset": 10}
    assert format_cache(s, (s, 5), "tuple", 5, 2) == (s, 7)
    assert format_cache(s, s, "tensor", 0, 9) is s
    assert format_cache(s, None, "none", 0, 9) is None
    assert format_cache(s, [], "none", 4, 1) == (s, 5)  # a non-None unknown cache gets a tuple


def test_slice_and_scatter_cache_rows():
    torch.manual_seed(0)
    full = [(torch.randn(5, 2, 3, 3), 11), (None, 0), None]
    idx = torch.tensor([4, 1])
    part = slice_cache(full, idx)
    assert torch.equal(part[0][0], full[0][0][[4, 1]]) and part[0][1] == 11
    assert part[1] == (None, 0) and part[2] is None
    upd = [(part[0][0] * 2, 12), (torch.ones(2, 2, 3, 3), 3), None]
    dst = [(full[0][0].clone(), 11), (None, 0), None]
    out = scatter_cache(dst, upd, idx, 5, "cpu")
    assert torch.equal(out[0][0][[4, 1]], part[0][0] * 2) and out[0][1] == 12
    assert torch.equal(out[0][0][[0, 2, 3]], full[0][0][[0, 2, 3]])
    assert out[1][0].shape == (5, 2, 3, 3) and float(out[1][0][[0, 2, 3]].abs().sum()) == 0.0
    assert torch.equal(out[1][0][[4, 1]], torch.ones(2, 2, 3, 3)) and out[1][1] == 3
    assert slice_cache(None, idx) is None and scatter_cache(None, upd, idx, 5, "cpu") is None


def test_pool_sessions_lru_eviction_and_stats():
    pool = StateSlotPool(num_layers=2, n_slots=3, H=2, Dk=4, Dv=4, device="cpu")
    a, b, c = pool.acquire("a"), pool.acquire("b"), pool.acquire("c")
    assert sorted((a, b, c)) == [0, 1, 2] and pool.acquire("a") == a
    pool.states[:, b] = 1.0
    d = pool.acquire("d")  # evicts the least recently used session: "b"
    assert d == b and pool.slot_of("b") is None and pool.slot_of("a") == a
    assert float(pool.states[:, d].abs().sum()) == 0.0  # a new session starts from zero
    st = pool.stats()
    assert st["active_sessions"] == 3 and st["max_sessions"] == 3 and st["free_slots"] == 0
    assert st["total_recurrent_memory_mb"] == round(3 * 2 * 2 * 4 * 4 * 4 / 2**20, 2)
    assert pool.clear_session("a") and not pool.clear_session("a")
    assert pool.stats()["free_slots"] == 1


def test_pool_session_cache_views_and_updates():
    pool = StateSlotPool(num_layers=2, n_slots=4, H=2, Dk=4, Dv=4, device="cpu")
    assert pool.get_session_cache("x", "cpu") is None and pool.get_session_cache("", "cpu") is None
    new = [(torch.full((1, 2, 4, 4), 3.0), 17), {"state": torch.full((2, 4, 4), 5.0), "offset": 9}]
    pool.update_session_cache("x", new, depth=2)
    cache, depth = pool.get_session_cache("x", "cpu")
    slot = pool.slot_of("x")
    assert depth == 2 and cache[0][1] == 17 and cache[1][1] == 9
    assert float(cache[0][0].mean()) == 3.0 and float(cache[1][0].mean()) == 5.0
    cache[0][0].add_(1.0)  # the returned states are views of the pool
    assert float(pool.states[0, slot].mean()) == 4.0
    pool.update_session_cache("x", [(cache[0][0], 18)])  # the pool's own row: no copy needed
    assert float(pool.states[0, slot].mean()) == 4.0 and int(pool.offsets[0, slot]) == 18


def test_pool_ttl_expiry(monkeypatch):
    import triune_amd.serving as S

    now = [1000.0]
    monkeypatch.setattr(S.time, "time", lambda: now[0])
    pool = StateSlotPool(num_layers=1, n_slots=2, H=1, Dk=4, Dv=4, device="cpu", session_ttl_seconds=10.0)
    pool.acquire("old")
    now[0] += 5.0
    pool.acquire("new")
    now[0] += 6.0  # "old" idle 11 s, "new" 6 s
    assert pool.slot_of("old") is None and pool.slot_of("new") is not None
    assert pool.stats()["active_sessions"] == 1
