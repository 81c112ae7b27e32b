"""Serving-side state handling for the GLA path: the reference's (state, offset) cache formats, a
device-resident recurrent-state slot pool, and a graph-captured decode runner.

Reference anchors:
  triune/model/attention.py:333-358   _parse_cache / _format_cache (dict, tuple, tensor caches)
  triune/model/transformer.py:276-317 _slice_cache / _scatter_cache (batch rows for early exits)
  triune/api/srsm.py:11-112           SessionRecurrentStateManager (per-session caches, LRU order,
                                      TTL, kept on the host in pinned memory between requests)
  triune/inference.py:162-300,        graph-captured one-token decode over static buffers
  triune/runtime/cuda_graph.py:19-80

On MI355X a session's recurrent state is small next to 288 GB of HBM (one layer at H=6, D=64 is
96 KB in fp32), so StateSlotPool keeps every live session on the device: one fp32 tensor per
layer of shape [n_slots, H, Dk, Dv], and sessions map to slot indices.  The decode step
(gla_decode_step(..., slots=)) and the packed prefill (fast_chunk_gla_varlen(..., state_pool=,
slots=)) read and write those rows in place, so no state crosses PCIe between requests and no
gather / scatter copies run around the kernels.
"""

from __future__ import annotations

import collections
import threading
import time
from typing import Any, Dict, List, Optional, Tuple

import torch

from .fast_gla import _DECODE_PAIRS, fast_chunk_gla_varlen, gla_decode_step
from .gla_prep import fused_qkvg_decode_step_pool

__all__ = [
    "parse_cache",
    "format_cache",
    "slice_cache",
    "scatter_cache",
    "StateSlotPool",
    "GLADecodeGraphRunner",
]


# ---------------------------------------------------------------------------------------
# Cache formats (attention.py:333-358, transformer.py:276-317)
# ---------------------------------------------------------------------------------------
def parse_cache(cache) -> Tuple[Optional[torch.Tensor], int, str]:
    """(initial_state, offset, format) of a layer cache: {"state", "offset"} dict, (state, offset)
    tuple, a bare state tensor, or None."""
    if isinstance(cache, dict):
        return cache.get("state"), cache.get("offset", 0), "dict"
    if isinstance(cache, tuple):
        state, offset = cache
        return state, offset, "tuple"
    if torch.is_tensor(cache):
        return cache, 0, "tensor"
    return None, 0, "none"


def format_cache(final_state, cache, cache_format: str, offset: int, seq_len: int):
    """The layer cache to hand back after seq_len more tokens, in the caller's format."""
    if cache_format == "dict":
        return {"state": final_state, "offset": offset + seq_len}
    if cache_format == "tuple":
        return (final_state, offset + seq_len)
    if cache_format == "tensor":
        return final_state
    return (final_state, offset + seq_len) if cache is not None else None


def slice_cache(cache: Optional[List[Any]], idx: torch.Tensor) -> Optional[List[Any]]:
    """Rows idx of every (state, offset) entry (the batch rows still running after an early exit)."""
    if cache is None:
        return None
    out = []
    for entry in cache:
        if isinstance(entry, tuple) and entry[0] is not None:
            state, off = entry
            out.append((state.index_select(0, idx), off))
        else:
            out.append(entry)
    return out


def scatter_cache(dst_cache: Optional[List[Any]], src_cache: Optional[List[Any]], idx: torch.Tensor,
                  batch_size: int, device) -> Optional[List[Any]]:
    """Write the rows of src_cache back into rows idx of dst_cache (a zero batch of batch_size
    rows where dst has no state yet); returns dst_cache."""
    if dst_cache is None or src_cache is None:
        return dst_cache
    for layer, entry in enumerate(src_cache):
        if not (isinstance(entry, tuple) and entry[0] is not None):
            continue
        src, off = entry
        cur = dst_cache[layer]
        if isinstance(cur, tuple) and cur[0] is not None:
            dst_cache[layer] = (cur[0].index_copy(0, idx, src.to(cur[0].dtype)), off)
        else:
            full = torch.zeros(batch_size, *src.shape[1:], device=device, dtype=src.dtype)
            dst_cache[layer] = (full.index_copy(0, idx, src), off)
    return dst_cache


# ---------------------------------------------------------------------------------------
# Device-resident session pool (the device form of SessionRecurrentStateManager)
# ---------------------------------------------------------------------------------------
class StateSlotPool:
    """Recurrent states of up to n_slots sessions for num_layers GLA layers, resident on one device.

    states[layer] is an fp32 [n_slots, H, Dk, Dv] tensor; offsets[layer, slot] (an int64 device
    tensor [num_layers, n_slots]) counts the tokens a slot has absorbed (the reference's cache
    offset).  Sessions map to slots in LRU order with a time-to-live, as in the reference's
    SessionRecurrentStateManager (srsm.py:11-112), whose get / update / clear / stats interface
    this class keeps; a new session's slot starts from a zero state.  Thread-safe for the
    bookkeeping; kernel calls follow the caller's stream order.

    prefill() and decode_step() run only device work (the kernels and a device-side update of
    the offsets), with no host synchronisation, so a serving loop can capture them in one graph
    when slots and cu_seqlens are device tensors; a slot outside [0, n_slots) (a padded batch
    row) is skipped by the kernels and by the offset count.
    """

    def __init__(self, num_layers: int, n_slots: int, H: int, Dk: int, Dv: int, device="cuda",
                 session_ttl_seconds: float = 3600.0):
        if num_layers <= 0 or n_slots <= 0:
            raise ValueError("num_layers and n_slots must be positive")
        self.num_layers, self.n_slots, self.H, self.Dk, self.Dv = num_layers, n_slots, H, Dk, Dv
        self.device = torch.device(device)
        self.session_ttl_seconds = session_ttl_seconds
        self.states = torch.zeros(num_layers, n_slots, H, Dk, Dv, device=self.device, dtype=torch.float32)
        self.offsets = torch.zeros(num_layers, n_slots, device=self.device, dtype=torch.int64)
        self._lock = threading.Lock()
        self._free = collections.deque(range(n_slots))
        self._sessions: "collections.OrderedDict[str, Dict[str, Any]]" = collections.OrderedDict()

    # -- bookkeeping -----------------------------------------------------------------------
    def _purge_expired_locked(self) -> None:
        now = time.time()
        for sid in [s for s, e in self._sessions.items() if now - e["last_active"] > self.session_ttl_seconds]:
            self._free.append(self._sessions.pop(sid)["slot"])

    def _reset_slot(self, slot: int) -> None:
        self.states[:, slot].zero_()
        self.offsets[:, slot].zero_()

    def acquire(self, session_id: str) -> int:
        """The slot of session_id, creating the session (zero state, offset 0) if needed; when
        every slot is taken the least recently used session is evicted."""
        if not session_id:
            raise ValueError("empty session id")
        with self._lock:
            self._purge_expired_locked()
            entry = self._sessions.get(session_id)
            if entry is None:
                if not self._free:
                    self._free.append(self._sessions.popitem(last=False)[1]["slot"])
                entry = {"slot": self._free.popleft(), "depth": None}
                self._reset_slot(entry["slot"])
                self._sessions[session_id] = entry
            entry["last_active"] = time.time()
            self._sessions.move_to_end(session_id)
            return entry["slot"]

    def slot_of(self, session_id: str) -> Optional[int]:
        with self._lock:
            self._purge_expired_locked()
            entry = self._sessions.get(session_id)
            return None if entry is None else entry["slot"]

    def slots_tensor(self, session_ids) -> torch.Tensor:
        """int32 device tensor of the sessions' slots (acquired as needed), in order."""
        return torch.tensor([self.acquire(s) for s in session_ids], device=self.device, dtype=torch.int32)

    def clear_session(self, session_id: str) -> bool:
        with self._lock:
            entry = self._sessions.pop(session_id, None)
            if entry is None:
                return False
            self._free.append(entry["slot"])
            return True

    def stats(self) -> Dict[str, Any]:
        with self._lock:
            self._purge_expired_locked()
            per_slot = self.num_layers * self.H * self.Dk * self.Dv * 4
            return {
                "active_sessions": len(self._sessions),
                "max_sessions": self.n_slots,
                "total_recurrent_memory_mb": round(len(self._sessions) * per_slot / (1024 * 1024), 2),
                "free_slots": len(self._free),
            }

    # -- the reference's session-cache interface ----------------------------------------------
    def get_session_cache(self, session_id: str, device=None) -> Optional[Tuple[List[Any], Optional[int]]]:
        """(per-layer (state, offset) cache, depth) of an existing session, or None.  The states
        are [1, H, Dk, Dv] views of the pool: a kernel that updates them in place updates the
        session."""
        if not session_id:
            return None
        with self._lock:
            self._purge_expired_locked()
            entry = self._sessions.get(session_id)
            if entry is None:
                return None
            entry["last_active"] = time.time()
            self._sessions.move_to_end(session_id)
            slot, depth = entry["slot"], entry.get("depth")
        offs = self.offsets[:, slot].tolist()  # one device read per session lookup
        cache = [(self.states[layer, slot:slot + 1], offs[layer]) for layer in range(self.num_layers)]
        return cache, depth

    def update_session_cache(self, session_id: str, cache: List[Any], depth: Optional[int] = None) -> None:
        """Store a per-layer (state [1, H, Dk, Dv] or [H, Dk, Dv], offset) cache into the session's
        slot (copies on the device; entries that already are the pool's own rows cost nothing)."""
        if not session_id or not cache:
            return
        slot = self.acquire(session_id)
        for layer, item in enumerate(cache[: self.num_layers]):
            state, off = parse_cache(item)[:2]
            dst = self.states[layer, slot]
            if state is not None:
                src = state.reshape(self.H, self.Dk, self.Dv)
                if src.data_ptr() != dst.data_ptr():
                    dst.copy_(src.to(device=self.device, dtype=torch.float32))
            self.offsets[layer, slot] = int(off)
        with self._lock:
            if session_id in self._sessions:
                self._sessions[session_id]["depth"] = depth

    # -- kernels over slots --------------------------------------------------------------------
    def _count(self, layer: int, slots: torch.Tensor, n: torch.Tensor) -> None:
        """offsets[layer, slots[i]] += n[i] on the device, skipping slots outside the pool."""
        sl = slots.to(device=self.device, dtype=torch.int64)
        ok = (sl >= 0) & (sl < self.n_slots)
        self.offsets[layer].index_add_(0, torch.where(ok, sl, torch.zeros_like(sl)),
                                       torch.where(ok, n.to(device=self.device, dtype=torch.int64),
                                                   torch.zeros_like(sl)))

    def prefill(self, layer: int, q, k, v, g, cu_seqlens, slots: torch.Tensor, out=None):
        """Packed prefill of len(slots) sequences from their slots' states, final states written
        back to the slots; returns the outputs."""
        o, _ = fast_chunk_gla_varlen(q, k, v, g, cu_seqlens, out=out, state_pool=self.states[layer], slots=slots)
        cu = cu_seqlens.to(device=self.device)
        self._count(layer, slots, cu[1:] - cu[:-1])
        return o

    def decode_step(self, layer: int, q, k, v, g, slots: torch.Tensor, out=None, count_tokens: bool = True):
        """One token for each of len(slots) sessions; states updated in place in their slots."""
        o, _ = gla_decode_step(q, k, v, g, self.states[layer], out=out, inplace=True, slots=slots)
        if count_tokens:
            self._count(layer, slots, torch.ones_like(slots, dtype=torch.int64))
        return o

    def fused_decode_step(self, layer: int, qkvg, slots: torch.Tensor, cos=None, sin=None, use_rope: bool = True,
                          out=None, count_tokens: bool = True):
        """decode_step from raw projections (qkvg [B, 4, H, HD]): VectorisedGLA's fused decode
        (attention.py:81-179; ELU+1, L2 norm, RoPE, logsigmoid, then the update) on the slots'
        states, in place."""
        o = fused_qkvg_decode_step_pool(qkvg, self.states[layer], slots, cos, sin, use_rope=use_rope, out=out)
        if count_tokens:
            self._count(layer, slots, torch.ones_like(slots, dtype=torch.int64))
        return o


# ---------------------------------------------------------------------------------------
# Graph-captured decode
# ---------------------------------------------------------------------------------------
class GLADecodeGraphRunner:
    """`steps` consecutive GLA decode steps of a fixed batch of pool slots, captured once in a
    HIP graph and replayed (the decode half of the reference's graph runner, inference.py:162-300).

    states: an fp32 contiguous [n_slots, H, Dk, Dv] pool (e.g. StateSlotPool.states[layer]);
    slots: int32 [B] device tensor.  Static buffers q, k, g [steps, B, H, Dk], v [steps, B, H, Dv]
    (dtype) and o [steps, B, H, Dv] are the graph's inputs and outputs: write step t's inputs into
    q[t] ... g[t] (as the projections feeding the step would), call replay(), read o.  step()
    does the copy and replay for steps == 1.  Capture warms up on a scratch pool, so the real
    states are only touched by replays."""

    def __init__(self, states: torch.Tensor, slots: torch.Tensor, steps: int = 1, dtype=torch.bfloat16,
                 g_dtype=None):
        if states.dtype != torch.float32 or not states.is_contiguous() or states.dim() != 4 or not states.is_cuda:
            raise ValueError("states must be a contiguous float32 [n_slots, H, Dk, Dv] device tensor")
        _, H, Dk, Dv = states.shape
        if (Dk, Dv) not in _DECODE_PAIRS:
            raise ValueError(f"head dims ({Dk}, {Dv}) must be a decode kernel pair {_DECODE_PAIRS}")
        if steps <= 0:
            raise ValueError("steps must be positive")
        self.states = states
        self.slots = slots.to(device=states.device, dtype=torch.int32).contiguous()
        B = self.slots.numel()
        dev = states.device
        self.steps = steps
        self.q = torch.zeros(steps, B, H, Dk, device=dev, dtype=dtype)
        self.k = torch.zeros_like(self.q)
        self.g = torch.zeros(steps, B, H, Dk, device=dev, dtype=g_dtype or dtype)
        self.v = torch.zeros(steps, B, H, Dv, device=dev, dtype=dtype)
        self.o = torch.zeros(steps, B, H, Dv, device=dev, dtype=dtype)
        self._graph: Optional[torch.cuda.CUDAGraph] = None

    def _run(self, states, slots) -> None:
        for t in range(self.steps):
            gla_decode_step(self.q[t], self.k[t], self.v[t], self.g[t], states, out=self.o[t], inplace=True,
                            slots=slots)

    def capture(self) -> None:
        cur = torch.cuda.current_stream(self.states.device)
        side = torch.cuda.Stream(device=self.states.device)
        side.wait_stream(cur)
        B = self.slots.numel()
        scratch = torch.zeros(B, *self.states.shape[1:], device=self.states.device, dtype=torch.float32)
        rows = torch.arange(B, device=self.states.device, dtype=torch.int32)
        with torch.cuda.stream(side):
            self._run(scratch, rows)
        cur.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._run(self.states, self.slots)
        self._graph = graph

    @property
    def is_captured(self) -> bool:
        return self._graph is not None

    def replay(self) -> torch.Tensor:
        if self._graph is None:
            self.capture()
        self._graph.replay()
        return self.o

    def step(self, q, k, v, g) -> torch.Tensor:
        """One decode step (steps == 1): inputs [B, H, D] or [B, 1, H, D]; returns o [B, H, Dv]
        (the runner's static buffer, overwritten by the next replay)."""
        if self.steps != 1:
            raise ValueError("step() drives a one-step runner; fill q/k/v/g and call replay()")
        for dst, src in ((self.q, q), (self.k, k), (self.v, v), (self.g, g)):
            dst[0].copy_(src.reshape(dst.shape[1:]))
        return self.replay()[0]

    def release(self) -> None:
        if self._graph is not None:
            self._graph.reset()
        self._graph = None
