"""Cooperative decode: host cores take the lowest-ranked route slots of a
one-token FP8 layer call while the GPU runs the others.

Reference: ``HybridDecodeRuntime`` (src/drama_low_vram/hybrid_decode.py:33-416)
with the route planner ``partition_routes`` (hybrid_layer.py:17-28; native
drama_partition_routes, native/src/runtime.cpp:291-335) and the native expert
executor ``NativeExpertExecutor`` (native_backend.py:176-380; runtime.cpp:
68-276) with its FP8 boundary guard (``NativeQuantizationBoundary``).

With every expert resident in HBM this is an opt-in mode kept for call-site
parity (a manager configured for it, a thread inside ``decode()``), never a
fallback: the GPU path runs whenever a call is not eligible.  The CPU
executor is this library's own C++ (``dmoe_cpu_*``) and follows the decode
kernels' arithmetic -- the kernels' K order, bf16 gate/up, the device's SiLU
values (``dmoe_silu_table``), FP8 hidden groups, the down fma chain and the
route weight -- with each 128-column block product summed in fp32 in a
fixed lane order, where the FP8 MFMA truncates inside groups of 8 products:
host slots agree with device slots within the path's tolerance.  The GPU slots
are the resident path's own partials, bit for bit.  With the guard on, a
call whose hidden quantization meets an E4M3 rounding midpoint recomputes
its CPU slots on the GPU, as the reference does.
"""
from __future__ import annotations

import ctypes
import threading
from concurrent.futures import ThreadPoolExecutor
from contextlib import contextmanager
from dataclasses import asdict, dataclass

import torch
from torch import Tensor

from . import _lib
from .formats import EXPERT_BUFFER_NAMES, StagedExperts, fp8_bank_struct

CPU_GPU_RECOMPUTE = 1  # DMOE_CPU_GPU_RECOMPUTE
_ISA_NAMES = {1: "scalar", 2: "avx2", 3: "avx512"}
_ISA_CODES = {"auto": 0, "scalar": 1, "avx2": 2, "avx512": 3}


class CpuQuantizationBoundary(RuntimeError):
    """The host executor's hidden quantization met an E4M3 rounding midpoint
    (guard on): recompute those slots on the GPU (the reference's
    NativeQuantizationBoundary, native_backend.py:17)."""


def partition_routes(ids, resident, cpu_jobs: int):
    """(cpu_slots, gpu_slots): cpu_jobs slots for the host -- those whose
    expert is not resident on the GPU first, each kind from the lowest-ranked
    slot up -- and the rest for the GPU, both in slot order
    (hybrid_layer.py:17-28)."""
    ids = [int(i) for i in ids]
    if not 0 <= cpu_jobs <= len(ids):
        raise ValueError("CPU job count must fit the route count")
    cold = [slot for slot in reversed(range(len(ids))) if ids[slot] not in resident]
    hot = [slot for slot in reversed(range(len(ids))) if ids[slot] in resident]
    chosen = set((cold + hot)[:cpu_jobs])
    return ([slot for slot in range(len(ids)) if slot in chosen],
            [slot for slot in range(len(ids)) if slot not in chosen])


def native_partition_routes(ids, resident, experts: int, cpu_jobs: int):
    """partition_routes through the library's planner (dmoe_cpu_partition_routes)."""
    ids_t = torch.as_tensor(list(ids), dtype=torch.int64).contiguous()
    res_t = torch.as_tensor(sorted(int(e) for e in resident), dtype=torch.int64).contiguous()
    count = ids_t.numel()
    cpu = torch.empty(max(cpu_jobs, 1), dtype=torch.int64)
    gpu = torch.empty(max(count - cpu_jobs, 1), dtype=torch.int64)
    _lib.check(_lib.library().dmoe_cpu_partition_routes(
        _lib.ptr(ids_t), count, _lib.ptr(res_t) if res_t.numel() else None, res_t.numel(), experts, cpu_jobs,
        _lib.ptr(cpu), _lib.ptr(gpu)))
    return cpu[:cpu_jobs].tolist(), gpu[:count - cpu_jobs].tolist()


def silu_table(device) -> Tensor:
    """The decode kernels' SiLU for every bf16 gate bit pattern, computed on
    the GPU and returned on the host: fp32 [65536] (the reference's
    build_gpu_silu_table, fp8_decode.py:17-21)."""
    device = torch.device(device)
    table = torch.empty(65536, dtype=torch.float32, device=device)
    _lib.check(_lib.library().dmoe_silu_table(_lib.ptr(table), _lib.stream_handle(device)))
    return table.cpu()


def _quantize_row(x: Tensor, group: int):
    """FP8 row(s) and scales of x on the device, as the decode kernels
    quantize their activations (dmoe_fp8_quantize, groups of 128 or the row)."""
    from .offload import device_state

    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    scales = torch.empty((rows, cols // group), dtype=torch.float32, device=x.device)
    _lib.check(_lib.library().dmoe_fp8_quantize(
        _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), rows, cols, group, _lib.ptr(q), _lib.ptr(scales),
        _lib.ptr(device_state(x.device).status), _lib.stream_handle(x.device)))
    return q, scales


def _host_bank(store) -> StagedExperts:
    if not isinstance(store, StagedExperts):
        raise ValueError("the cooperative decode takes FP8 expert banks")
    if any(getattr(store, name).device.type != "cpu" for name in EXPERT_BUFFER_NAMES):
        raise ValueError("the cooperative decode needs expert banks held in host memory")
    return store


class CpuExpertExecutor:
    """One FP8 activation row -> ordered weighted fp32 partials of up to
    ``capacity`` route slots on the host (the reference's
    NativeExpertExecutor.forward_quantized_pairs, native_backend.py:176-300).
    Calls are synchronous; ctypes releases the GIL during them.  A lock
    serializes calls and close on one executor."""

    def __init__(self, store: StagedExperts, *, capacity: int = 8, threads: int = 4, silu_table: Tensor,
                 implementation: str = "auto", guard_fp8_boundaries: bool = False):
        store = _host_bank(store)
        store.validate()
        if (isinstance(capacity, bool) or not isinstance(capacity, int) or not 1 <= capacity <= 256
                or isinstance(threads, bool) or not isinstance(threads, int) or not 1 <= threads <= 256):
            raise ValueError("Invalid CPU executor capacity or thread count")
        if not isinstance(guard_fp8_boundaries, bool):
            raise ValueError("guard_fp8_boundaries must be a boolean")
        if implementation not in _ISA_CODES:
            raise ValueError(f"Unknown CPU implementation {implementation!r}")
        if (silu_table.device.type != "cpu" or silu_table.dtype != torch.float32
                or tuple(silu_table.shape) != (65536,) or not silu_table.is_contiguous()):
            raise ValueError("The SiLU table must be contiguous host fp32 [65536]")
        self._silu = silu_table.clone()  # the executor borrows it
        self.store, self.capacity = store, capacity
        self._lock = threading.Lock()
        lib = _lib.library()
        self._handle = lib.dmoe_cpu_executor_create(store.hidden, store.intermediate, capacity, threads,
                                                    _ISA_CODES[implementation])
        if not self._handle:
            _lib.check(-1)
        self.threads = lib.dmoe_cpu_executor_threads(self._handle)
        self.implementation = _ISA_NAMES[lib.dmoe_cpu_executor_isa(self._handle)]
        _lib.check(lib.dmoe_cpu_executor_set_silu_table(self._handle, _lib.ptr(self._silu)))
        _lib.check(lib.dmoe_cpu_executor_set_guard(self._handle, int(guard_fp8_boundaries)))

    def _bank(self, store):
        if store is None or store is self.store:
            return self.store
        store = _host_bank(store)
        if (store.hidden, store.intermediate) != (self.store.hidden, self.store.intermediate):
            raise ValueError("Expert bank must match the executor geometry")
        return store

    def forward_quantized_pairs(self, xq: Tensor, scales: Tensor, ids: Tensor, weights: Tensor, *,
                                out: Tensor | None = None, store=None) -> Tensor:
        store = self._bank(store)
        hidden = self.store.hidden
        if (xq.device.type != "cpu" or xq.dtype not in (torch.uint8, torch.float8_e4m3fn) or xq.numel() != hidden
                or not xq.is_contiguous() or scales.device.type != "cpu" or scales.dtype != torch.float32
                or scales.numel() not in (hidden // 128, 1) or not scales.is_contiguous()):
            raise ValueError("Expected contiguous host FP8 activation bytes and fp32 scales")
        if (ids.device.type != "cpu" or ids.dtype != torch.int64 or ids.ndim != 1 or not ids.is_contiguous()
                or not 1 <= ids.numel() <= self.capacity or weights.device.type != "cpu"
                or weights.dtype != torch.float32 or weights.shape != ids.shape or not weights.is_contiguous()):
            raise ValueError("Invalid host route ids / weights")
        shape = (ids.numel(), hidden)
        if out is None:
            out = torch.empty(shape, dtype=torch.float32)
        if out.device.type != "cpu" or out.dtype != torch.float32 or tuple(out.shape) != shape \
                or not out.is_contiguous():
            raise ValueError("Invalid host fp32 output buffer")
        x_group = 128 if scales.numel() == hidden // 128 else hidden
        bank = fp8_bank_struct(store)
        with self._lock:
            if not self._handle:
                raise RuntimeError("CPU expert executor is closed")
            rc = _lib.library().dmoe_cpu_expert_pairs(
                self._handle, ctypes.byref(bank), _lib.ptr(xq.view(torch.uint8)), _lib.ptr(scales), x_group,
                _lib.ptr(ids), _lib.ptr(weights), ids.numel(), _lib.ptr(out))
        if rc == CPU_GPU_RECOMPUTE:
            raise CpuQuantizationBoundary("an FP8 rounding midpoint of the hidden activation: recompute on the GPU")
        _lib.check(rc)
        return out

    def close(self) -> None:
        with self._lock:
            if self._handle:
                _lib.library().dmoe_cpu_executor_destroy(self._handle)
                self._handle = None


@dataclass
class HybridDecodeStatistics:
    calls: int = 0
    cpu_pairs: int = 0
    gpu_pairs: int = 0
    control_d2h_bytes: int = 0
    partial_h2d_bytes: int = 0
    workspace_allocations: int = 0
    fallbacks: int = 0
    boundary_fallback_calls: int = 0
    boundary_recomputed_pairs: int = 0
    completion_host_waits: int = 0
    completion_stream_waits: int = 0


class HybridDecodeRuntime:
    """One workspace shared by every attached layer; the caller serializes
    requests (hybrid_decode.py:33-416).  Stream dependencies fence the shared
    buffers before reuse; the host workers finish before a call returns, and a
    failure drains both streams before the buffers are released.  Only calls
    made inside ``decode()`` on the calling thread are eligible."""

    def __init__(self, manager, *, cpu_jobs: int = 4, threads: int = 4, device="cuda:0", silu_table_values=None,
                 synchronize_return: bool = True, guard_fp8_boundaries: bool = True):
        if isinstance(cpu_jobs, bool) or not isinstance(cpu_jobs, int) or not 1 <= cpu_jobs <= 8:
            raise ValueError("Hybrid CPU jobs must be an integer from 1 to 8")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("Hybrid decode requires a ROCm GPU device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        from .offload import HipExpertBackend

        if not isinstance(manager.backend, HipExpertBackend):
            raise ValueError("Hybrid decode requires the HIP expert backend")
        if manager.backend.gu_dtype not in (None, torch.bfloat16):
            raise ValueError("Hybrid decode rounds gate/up through bf16")
        if manager._closed or not manager.modules:
            raise ValueError("Attach expert modules before configuring hybrid decode")
        stores = [manager._bank_of(module) for module in manager.modules.values()]
        for store in stores:
            _host_bank(store)
        if len({(store.hidden, store.intermediate) for store in stores}) != 1:
            raise ValueError("Hybrid layers must have identical expert geometry")
        self.manager = manager
        self.cpu_jobs = cpu_jobs
        self.stats = HybridDecodeStatistics()
        self._lock = threading.Lock()
        self._scope = threading.local()
        self._closed = False
        self._buffers: dict[str, Tensor] = {}
        self._layer_indices = {id(module): index for index, module in enumerate(manager.modules.values())}
        self._stream = self._returned = self._done = None
        self._pending = False
        self.synchronize_return = bool(synchronize_return)
        table = silu_table(self.device) if silu_table_values is None else silu_table_values
        self.executor = CpuExpertExecutor(stores[0], capacity=8, threads=threads, silu_table=table,
                                          guard_fp8_boundaries=guard_fp8_boundaries)
        self.worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="dmoe-hybrid")

    # ----------------------------------------------------------- scopes
    @contextmanager
    def decode(self, *, layers=None):
        """Mark decode on the calling thread; an optional layer subset."""
        previous = getattr(self._scope, "layers", ())
        self._scope.layers = None if layers is None else frozenset(layers)
        try:
            yield
        finally:
            self._scope.layers = previous

    @contextmanager
    def suspend(self):
        """Run the GPU path for calls made inside (a serialized diagnostic request)."""
        previous = getattr(self._scope, "suspended", False)
        self._scope.suspended = True
        try:
            yield
        finally:
            self._scope.suspended = previous

    def eligible(self, module, x: Tensor, ids: Tensor) -> bool:
        if getattr(self._scope, "suspended", False):
            return False
        layers = getattr(self._scope, "layers", ())
        if layers is not None and self._layer_indices.get(id(module)) not in layers:
            return False
        if self._closed:
            raise RuntimeError("Hybrid decode runtime is closed")
        store = self.manager._bank_of(module)
        ok = (id(module) in self._layer_indices and x.device == self.device and x.dtype == torch.bfloat16
              and x.ndim == 2 and x.shape[0] == 1 and x.is_contiguous() and ids.ndim == 2
              and 1 <= ids.shape[1] <= 8 and isinstance(store, StagedExperts)
              and self.manager.host is None)
        if not ok:
            self.stats.fallbacks += 1
        return ok

    # ---------------------------------------------------------- buffers
    def _allocate(self, store: StagedExperts) -> None:
        if self._buffers:
            return
        hidden = store.hidden
        shapes = {"ids": ((8,), torch.int64), "weights": ((8,), torch.float32), "q": ((1, hidden), torch.uint8),
                  "scales": ((1, hidden // 128), torch.float32), "result": ((8, hidden), torch.float32)}
        buffers = {name: torch.empty(shape, dtype=dtype, pin_memory=True) for name, (shape, dtype) in shapes.items()}
        buffers["device_result"] = torch.empty_like(buffers["result"], device=self.device)
        buffers["ordered"] = torch.empty_like(buffers["result"], device=self.device)
        self._stream = torch.cuda.Stream(device=self.device)
        self._handoff = torch.cuda.Event()
        self._returned = torch.cuda.Event()
        self._done = torch.cuda.Event()
        self._buffers = buffers
        self.stats.workspace_allocations += 1

    def _cpu(self, store, ids: Tensor, weights: Tensor) -> None:
        self.executor.forward_quantized_pairs(self._buffers["q"], self._buffers["scales"], ids, weights, store=store,
                                              out=self._buffers["result"][:ids.numel()])

    # ----------------------------------------------------------- forward
    @torch.inference_mode()
    def forward(self, module, store: StagedExperts, x: Tensor, ids: Tensor, weights: Tensor) -> Tensor:
        from . import fp8_decode

        with self._lock:
            if self._closed:
                raise RuntimeError("Hybrid decode runtime is closed")
            self._allocate(store)
            b = self._buffers
            backend = self.manager.backend
            backend._check(x)
            device_bank = self.manager._on_device(module, store, self.device)
            stream = torch.cuda.current_stream(self.device)
            if self._pending:
                # a later call may come on another stream: order the shared
                # buffers behind the previous merge without a host wait
                stream.wait_event(self._done)
                self.stats.completion_stream_waits += 1
            count = ids.numel()
            future = None
            completed = False
            try:
                group = 128 if backend.x_group == 128 else store.hidden
                q, scales = _quantize_row(x, group)
                b["ids"][:count].copy_(ids.reshape(-1), non_blocking=True)
                b["weights"][:count].copy_(weights.reshape(-1).float(), non_blocking=True)
                b["q"].copy_(q.view(torch.uint8), non_blocking=True)
                host_scales = b["scales"].view(-1)[:scales.numel()]
                host_scales.copy_(scales.reshape(-1), non_blocking=True)
                self._handoff.record(stream)
                self._handoff.synchronize()
                routed = b["ids"][:count].tolist()
                if min(routed) < 0 or max(routed) >= store.count:
                    raise ValueError("Hybrid expert ID outside bank")
                # every expert is resident on the GPU: the lowest-ranked slots go to the host
                cpu_slots, gpu_slots = partition_routes(routed, (), min(self.cpu_jobs, count))
                cpu_index = torch.tensor(cpu_slots, dtype=torch.int64)
                cpu_ids = b["ids"][:count].index_select(0, cpu_index)
                cpu_weights = b["weights"][:count].index_select(0, cpu_index)
                scale_view = host_scales if group != 128 else b["scales"]
                future = self.worker.submit(self.executor.forward_quantized_pairs, b["q"], scale_view, cpu_ids,
                                            cpu_weights, store=store, out=b["result"][:len(cpu_slots)])
                gpu_index = torch.tensor(gpu_slots, dtype=torch.int64, device=self.device)
                cpu_device_index = cpu_index.to(self.device)
                route_ids = ids.reshape(-1)
                route_weights = weights.reshape(-1).float()
                if gpu_slots:
                    gpu_partials = fp8_decode.quantized_pairs(
                        backend.kernel, q, scales, route_ids.index_select(0, gpu_index),
                        route_weights.index_select(0, gpu_index), device_bank)
                recovered = False
                try:
                    future.result()
                except CpuQuantizationBoundary:
                    # the host workers have all joined: recompute their slots on the GPU
                    recovered = True
                    redo = fp8_decode.quantized_pairs(
                        backend.kernel, q, scales, route_ids.index_select(0, cpu_device_index),
                        route_weights.index_select(0, cpu_device_index), device_bank)
                    b["ordered"].index_copy_(0, cpu_device_index, redo)
                future = None
                if not recovered:
                    with torch.cuda.stream(self._stream):
                        b["device_result"][:len(cpu_slots)].copy_(b["result"][:len(cpu_slots)], non_blocking=True)
                        self._returned.record(self._stream)
                    stream.wait_event(self._returned)
                if gpu_slots:
                    b["ordered"].index_copy_(0, gpu_index, gpu_partials)
                if not recovered:
                    b["ordered"].index_copy_(0, cpu_device_index, b["device_result"][:len(cpu_slots)])
                output = torch.empty_like(x)
                _lib.check(_lib.library().dmoe_combine_slots(
                    _lib.ptr(b["ordered"]), b["ordered"].stride(0), _lib.ptr(route_ids),
                    _lib.dtype_code(route_ids.dtype), store.count, 1, count, store.hidden, _lib.ptr(output),
                    _lib.dtype_code(output.dtype), output.stride(0), _lib.stream_handle(self.device)))
                self._done.record(stream)
                self._pending = True
                if self.synchronize_return:
                    self._done.synchronize()
                    self._pending = False
                    self.stats.completion_host_waits += 1
                completed = True
                self.stats.calls += 1
                self.stats.cpu_pairs += len(cpu_slots)
                self.stats.gpu_pairs += len(gpu_slots) + (len(cpu_slots) if recovered else 0)
                self.stats.control_d2h_bytes += count * 12 + store.hidden + scales.numel() * 4
                if recovered:
                    self.stats.boundary_fallback_calls += 1
                    self.stats.boundary_recomputed_pairs += len(cpu_slots)
                else:
                    self.stats.partial_h2d_bytes += len(cpu_slots) * store.hidden * 4
                return output
            finally:
                if not completed:
                    try:
                        if future is not None:
                            future.result()
                    finally:
                        stream.synchronize()
                        if self._stream is not None:
                            self._stream.synchronize()
                        self._pending = False

    # ---------------------------------------------------------- reports
    def report(self) -> dict:
        return {
            **asdict(self.stats), "cpu_jobs": self.cpu_jobs,
            "enabled": not self._closed and not getattr(self._scope, "suspended", False),
            "native_threads": self.executor.threads, "native_implementation": self.executor.implementation,
            "arithmetic": "gfx950 decode contract (exact block products, device SiLU table)",
            "synchronize_return": self.synchronize_return,
            "pinned_workspace_bytes": sum(v.numel() * v.element_size() for v in self._buffers.values()
                                          if v.device.type == "cpu"),
            "device_workspace_bytes": sum(v.numel() * v.element_size() for v in self._buffers.values()
                                          if v.device.type == "cuda"),
        }

    def _drain(self) -> None:
        for s in (self._stream,):
            if s is not None:
                s.synchronize()
        if self._done is not None:
            self._done.synchronize()
        self._buffers.clear()
        self._stream = self._returned = self._done = None
        self._pending = False

    def release_runtime_buffers(self) -> None:
        with self._lock:
            self._drain()

    def close(self) -> None:
        with self._lock:
            if self._closed:
                return
            self.worker.shutdown(wait=True)
            self.executor.close()
            self._drain()
            self._closed = True


__all__ = ["CpuExpertExecutor", "CpuQuantizationBoundary", "HybridDecodeRuntime", "HybridDecodeStatistics",
           "native_partition_routes", "partition_routes", "silu_table"]
