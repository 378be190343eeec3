"""Optional host residency of expert banks.

With 288 GB of HBM per MI355X every expert of a Drama 3 checkpoint stays on
the device, and that is the default (``residency="hbm"``): a bank that a
loader left in host memory is copied to the device whole, once, on its first
call.  ``residency="host"`` keeps the banks in host memory (page-locked when
``pin_memory``) and moves only the experts a call routes to -- the staging
tier of the reference's ExpertOffloadManager
(src/drama_low_vram/offload.py:359-900, 903-1277), for GPUs shared by several
models or banks larger than the HBM left over:

* a pool of ``max_staged_experts`` device slots shared by every layer;
* with ``cache_experts`` > 0, a per-layer hot cache of that many slots: a
  decode token's experts are kept in it (the ones already there first, then
  the rest in router order), longer prompts only read what it holds;
* a call whose experts are all in one set of slots runs as one backend call
  over those slots (rows chunked so no call exceeds ``max_pair_rows`` pairs);
  otherwise the experts run in groups (the cached ones, then pool-sized
  groups of the others) through ``forward_pairs``, and the fp32 pair
  contributions are added in router slot order, as the resident kernels do.

Expert rows move by async copies from pinned memory on the calling stream,
so they are ordered before the kernels that read them and after the kernels
that read a slot's previous contents.  Slots are chosen free-first, then
least recently used.  Host mode reads the route ids back (one host sync per
call), so its calls cannot be captured in a hipGraph; the resident default
can be.
"""
from __future__ import annotations

import dataclasses
import time

import torch
from torch import Tensor

from .formats import EXPERT_BUFFER_NAMES, QuantizedStore, StagedExperts

RESIDENCY_MODES = ("hbm", "host")


@dataclasses.dataclass
class OffloadStatistics:
    """Cumulative counts and timings of a manager's host traffic: the
    reference's OffloadStatistics (offload.py:59-98) for the fields this tier
    has.  Host banks are pinned whole, once, and their rows copied straight
    into device slots, so there is no gather step, staging area or DMA-source
    wait to count.  ``h2d_seconds`` is HIP-event time of the copies, collected
    only with ``profile_transfers``; the other timings are host wall time;
    ``h2d_copy_calls`` counts tensor copy submissions."""

    forward_calls: int = 0
    grouped_calls: int = 0
    staging_calls: int = 0
    h2d_copy_calls: int = 0
    expert_loads: int = 0
    expert_cache_hits: int = 0
    hot_cache_hits: int = 0
    hot_cache_loads: int = 0
    hot_cache_bytes: int = 0
    hot_cache_capacity_experts: int = 0
    staged_bytes: int = 0
    h2d_bytes: int = 0
    host_staging_seconds: float = 0.0
    h2d_submit_seconds: float = 0.0
    routing_host_seconds: float = 0.0
    h2d_seconds: float = 0.0
    pinned_bytes: int = 0
    device_buffer_bytes: int = 0
    peak_staged_experts: int = 0

    def as_dict(self) -> dict:
        return dataclasses.asdict(self)


class TransferClock:
    """HIP-event timing of host-to-device copies: a start and a stop event
    around each batch on the copying stream, read when the statistics are
    asked for (no host wait on the call path)."""

    def __init__(self, stats: OffloadStatistics, enabled: bool):
        self.stats = stats
        self.enabled = bool(enabled)
        self._pending: list = []

    def start(self, device):
        if not self.enabled or torch.device(device).type != "cuda":
            return None
        event = torch.cuda.Event(enable_timing=True)
        event.record(torch.cuda.current_stream(device))
        return event

    def stop(self, started, device) -> None:
        if started is None:
            return
        event = torch.cuda.Event(enable_timing=True)
        event.record(torch.cuda.current_stream(device))
        self._pending.append((started, event))

    def collect(self) -> None:
        for started, stopped in self._pending:
            stopped.synchronize()
            self.stats.h2d_seconds += started.elapsed_time(stopped) / 1000.0
        self._pending.clear()


def bank_buffers(bank) -> dict:
    """Every per-expert tensor of a bank, each [experts, ...]."""
    names = list(EXPERT_BUFFER_NAMES)
    if isinstance(bank, QuantizedStore):
        names += [n for n in ("w13_zeros", "w2_zeros") if getattr(bank, n) is not None]
    return {n: getattr(bank, n) for n in names}


def bank_like(bank, buffers: dict):
    """A bank of ``bank``'s format and geometry over other per-expert tensors."""
    if isinstance(bank, QuantizedStore):
        return dataclasses.replace(bank, **buffers)
    return StagedExperts(**buffers)


def bank_key(bank) -> tuple:
    """Identity of a bank's tensors (a bank rebuilt over new tensors differs)."""
    return tuple((n, id(t), tuple(t.shape), t.dtype) for n, t in bank_buffers(bank).items())


def bank_device(bank) -> torch.device:
    return bank.w13_weight.device


def device_copy(bank, device):
    """The whole bank copied to ``device``."""
    return bank_like(bank, {n: t.to(device) for n, t in bank_buffers(bank).items()})


class ExpertSlots:
    """``capacity`` expert slots of one bank geometry on one device."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self.buffers: dict = {}
        self.key = None
        self.holds = [-1] * capacity   # expert held by each slot, -1 free
        self.slot_of: dict = {}        # expert -> slot
        self.last_use = [0] * capacity
        self.clock = 0
        self.loads = 0
        self.hits = 0
        self.copy_calls = 0
        self.copied_bytes = 0

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.buffers.values())

    def bind(self, bank, device) -> None:
        """Serve ``bank`` on ``device``.  Another bank drops the slots'
        contents; the buffers are kept when the geometry is the same."""
        key = (torch.device(device), bank_key(bank))
        if key == self.key:
            return
        wanted = {n: ((self.capacity, *t.shape[1:]), t.dtype) for n, t in bank_buffers(bank).items()}
        have = {n: (tuple(t.shape), t.dtype) for n, t in self.buffers.items()}
        if have != wanted or any(t.device != key[0] for t in self.buffers.values()):
            self.buffers = {n: torch.empty(shape, dtype=dtype, device=key[0]) for n, (shape, dtype) in wanted.items()}
        self.key = key
        self.holds = [-1] * self.capacity
        self.slot_of = {}
        self.last_use = [0] * self.capacity

    def _victim(self, keep: set) -> int:
        for slot, expert in enumerate(self.holds):
            if expert < 0:
                return slot
        candidates = [s for s in range(self.capacity) if self.holds[s] not in keep]
        if not candidates:
            raise RuntimeError("Every expert slot holds an expert this call needs")
        return min(candidates, key=lambda s: self.last_use[s])

    def place(self, bank, experts, keep: set) -> dict:
        """Slots holding ``experts`` (at most ``capacity``), copying the
        missing ones from ``bank``; experts in ``keep`` are not evicted."""
        if len(experts) > self.capacity:
            raise ValueError(f"Cannot hold {len(experts)} experts in {self.capacity} slots")
        self.clock += 1
        sources = bank_buffers(bank)
        placed = {}
        for expert in experts:
            slot = self.slot_of.get(expert)
            if slot is None:
                slot = self._victim(keep)
                if self.holds[slot] >= 0:
                    del self.slot_of[self.holds[slot]]
                for name, source in sources.items():
                    self.buffers[name][slot].copy_(source[expert], non_blocking=True)
                    self.copy_calls += 1
                    self.copied_bytes += source[expert].numel() * source.element_size()
                self.holds[slot] = expert
                self.slot_of[expert] = slot
                self.loads += 1
            else:
                self.hits += 1
            self.last_use[slot] = self.clock
            placed[expert] = slot
        return placed

    def lookup(self, experts) -> dict:
        """Slots of the experts already held; nothing is copied."""
        self.clock += 1
        found = {e: self.slot_of[e] for e in experts if e in self.slot_of}
        for slot in found.values():
            self.last_use[slot] = self.clock
        self.hits += len(found)
        return found

    def bank(self, template):
        return bank_like(template, self.buffers)


def check_staging_sizes(max_staged_experts, max_pair_rows, cache_experts, hot_cache_experts):
    if hot_cache_experts is not None:
        if cache_experts not in (0, hot_cache_experts):
            raise ValueError("cache_experts and hot_cache_experts must match when both are set")
        cache_experts = hot_cache_experts
    for name, value in (("max_staged_experts", max_staged_experts), ("max_pair_rows", max_pair_rows),
                        ("cache_experts", cache_experts)):
        if isinstance(value, bool) or not isinstance(value, int):
            raise TypeError(f"{name} must be an integer")
    if max_staged_experts < 1 or max_pair_rows < 1 or cache_experts < 0:
        raise ValueError("Staging capacity and pair row limit must be positive; cache_experts cannot be negative")
    return cache_experts


class HostResidency:
    """Runs calls on banks held in host memory through device slots."""

    def __init__(self, *, max_staged_experts: int = 8, max_pair_rows: int = 64, cache_experts: int = 0,
                 hot_cache_experts: int | None = None, pin_memory: bool = True, profile_transfers: bool = False,
                 statistics: OffloadStatistics | None = None):
        cache_experts = check_staging_sizes(max_staged_experts, max_pair_rows, cache_experts, hot_cache_experts)
        self.max_pair_rows = max_pair_rows
        self.cache_experts = cache_experts
        self.pin_memory = bool(pin_memory)
        self.pool = ExpertSlots(max_staged_experts)
        self.caches: dict = {}
        self._host: dict = {}
        self.calls = 0
        self.grouped_calls = 0
        self.statistics = statistics if statistics is not None else OffloadStatistics()
        self.clock = TransferClock(self.statistics, profile_transfers)

    def stats(self) -> dict:
        return {"calls": self.calls, "grouped_calls": self.grouped_calls, "pool_loads": self.pool.loads,
                "pool_bytes": self.pool.nbytes, "cache_hits": sum(c.hits for c in self.caches.values()),
                "cache_loads": sum(c.loads for c in self.caches.values()),
                "cache_bytes": sum(c.nbytes for c in self.caches.values())}

    def collect(self) -> OffloadStatistics:
        """The cumulative statistics, with the profiled copies' event times
        read and the device buffer sizes refreshed."""
        self.clock.collect()
        st = self.statistics
        st.hot_cache_bytes = sum(c.nbytes for c in self.caches.values())
        st.hot_cache_capacity_experts = self.cache_experts * len(self.caches)
        st.device_buffer_bytes = self.pool.nbytes + st.hot_cache_bytes
        return st

    def _place(self, slots: "ExpertSlots", host, experts, keep: set, *, hot: bool, device) -> dict:
        """slots.place with its copies counted (and timed when profiling)."""
        st = self.statistics
        began = time.perf_counter()
        loads, hits, calls, nbytes = slots.loads, slots.hits, slots.copy_calls, slots.copied_bytes
        started = self.clock.start(device)
        placed = slots.place(host, experts, keep)
        self.clock.stop(started, device)
        loads, hits = slots.loads - loads, slots.hits - hits
        calls, nbytes = slots.copy_calls - calls, slots.copied_bytes - nbytes
        st.h2d_copy_calls += calls
        st.h2d_bytes += nbytes
        if hot:
            st.hot_cache_loads += loads
            st.hot_cache_hits += hits
        else:
            st.staging_calls += 1 if loads else 0
            st.expert_loads += loads
            st.expert_cache_hits += hits
            st.staged_bytes += nbytes
            st.peak_staged_experts = max(st.peak_staged_experts, len(placed))
        elapsed = time.perf_counter() - began
        st.host_staging_seconds += elapsed
        st.h2d_submit_seconds += elapsed if calls else 0.0
        return placed

    def host_bank(self, key, bank):
        """``bank`` in page-locked host memory (copied once per bank) when
        ``pin_memory``, else as it is."""
        if bank_device(bank).type != "cpu":
            raise ValueError("Host residency serves banks held in host memory")
        if not self.pin_memory:
            return bank
        ident = bank_key(bank)
        cached = self._host.get(key)
        if cached is None or cached[0] != ident:
            cached = (ident, bank_like(bank, {n: t.pin_memory() for n, t in bank_buffers(bank).items()}))
            self._host[key] = cached
            self.statistics.pinned_bytes += sum(t.numel() * t.element_size() for t in bank_buffers(bank).values())
        return cached[1]

    @torch.no_grad()
    def forward(self, key, bank, backend, x: Tensor, ids: Tensor, weights: Tensor) -> Tensor:
        """``backend.forward(x, ids, weights, bank)`` for a host-resident
        ``bank``; ``key`` names the layer that owns the bank (its hot cache)."""
        if x.is_cuda and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("Host-resident experts cannot run inside a hipGraph capture: "
                               "each call reads its route ids back")
        if x.shape[0] == 0:
            return torch.zeros_like(x)
        host = self.host_bank(key, bank)
        experts = host.w13_weight.shape[0]
        began = time.perf_counter()
        host_ids = ids.to("cpu", torch.int64)
        self.statistics.routing_host_seconds += time.perf_counter() - began
        self.statistics.forward_calls += 1
        if host_ids.numel() and (int(host_ids.min()) < 0 or int(host_ids.max()) >= experts):
            raise ValueError(f"Expert IDs must be in [0, {experts})")
        self.calls += 1
        tokens, top_k = host_ids.shape
        unique = sorted(set(host_ids.reshape(-1).tolist()))
        cache, cached = None, {}
        if self.cache_experts:
            cache = self.caches.get(key)
            if cache is None:
                cache = self.caches[key] = ExpertSlots(self.cache_experts)
            cache.bind(host, x.device)
            if tokens == 1:
                routed = list(dict.fromkeys(host_ids[0].tolist()))
                chosen = [e for e in routed if e in cache.slot_of] + [e for e in routed if e not in cache.slot_of]
                chosen = chosen[:self.cache_experts]
                cached = self._place(cache, host, chosen, set(chosen), hot=True, device=x.device)
            else:
                cached = cache.lookup(unique)
                self.statistics.hot_cache_hits += len(cached)
        cold = [e for e in unique if e not in cached]
        if top_k <= self.max_pair_rows:
            if not cold:
                return self._whole(backend, x, host_ids, weights, cache.bank(host), cached, experts)
            if not cached and len(cold) <= self.pool.capacity:
                self.pool.bind(host, x.device)
                staged = self._place(self.pool, host, cold, set(cold), hot=False, device=x.device)
                return self._whole(backend, x, host_ids, weights, self.pool.bank(host), staged, experts)
        return self._grouped(backend, x, host_ids, weights, host, cache, cached, cold, experts)

    def _whole(self, backend, x, host_ids, weights, slots_bank, slots: dict, experts: int) -> Tensor:
        lookup = torch.full((experts,), -1, dtype=torch.int64)
        for expert, slot in slots.items():
            lookup[expert] = slot
        local = lookup[host_ids].to(x.device)
        rows = max(1, self.max_pair_rows // host_ids.shape[1])
        out = torch.empty_like(x)
        for start in range(0, x.shape[0], rows):
            stop = min(x.shape[0], start + rows)
            backend.forward(x[start:stop], local[start:stop], weights[start:stop], slots_bank, out=out[start:stop])
        return out

    def _grouped(self, backend, x, host_ids, weights, host, cache, cached: dict, cold: list, experts: int) -> Tensor:
        self.grouped_calls += 1
        self.statistics.grouped_calls += 1
        tokens, top_k = host_ids.shape
        flat = host_ids.reshape(-1)
        pair_out = torch.empty((flat.numel(), x.shape[-1]), dtype=torch.float32, device=x.device)
        flat_weights = weights.reshape(-1)
        groups = []
        if cached:
            groups.append((lambda: (cache.bank(host), cached), sorted(cached)))
        for begin in range(0, len(cold), self.pool.capacity):
            group = cold[begin:begin + self.pool.capacity]

            def stage(group=group):
                self.pool.bind(host, x.device)
                return self.pool.bank(host), self._place(self.pool, host, group, set(group), hot=False,
                                                         device=x.device)
            groups.append((stage, group))
        for prepare, group in groups:
            slots_bank, slots = prepare()
            lookup = torch.full((experts,), -1, dtype=torch.int64)
            for expert, slot in slots.items():
                lookup[expert] = slot
            positions = torch.nonzero(lookup[flat] >= 0).reshape(-1)
            for start in range(0, positions.numel(), self.max_pair_rows):
                part = positions[start:start + self.max_pair_rows]
                where = part.to(x.device)
                values = backend.forward_pairs(x.index_select(0, (part // top_k).to(x.device)),
                                               lookup[flat[part]].to(x.device).unsqueeze(1),
                                               flat_weights.index_select(0, where).unsqueeze(1), slots_bank)
                pair_out.index_copy_(0, where, values)
        # router slot order, fp32, one add at a time
        slots_view = pair_out.view(tokens, top_k, -1)
        total = slots_view[:, 0].clone()
        for slot in range(1, top_k):
            total += slots_view[:, slot]
        return total.to(x.dtype)
