"""HBM-resident routed-expert runtime: the gfx950 ``ExpertBackend`` and a
resident manager that installs it on expert modules.

Reference interface: ``ExpertBackend`` (src/drama_low_vram/offload.py:187-196)
with ``forward`` / ``forward_pairs`` and the Triton backend's
``forward_decode_pairs`` / ``_check`` / ``.kernel`` (offload.py:247-356); the
manager contract of ``ExpertOffloadManager`` / ``install_expert_offload``
(offload.py:903-1063, 1534).  By default all experts are resident, so
``staged`` is the whole bank and local slot ids are global expert ids; the
reference's staging pool and hot cache exist as the optional host-residency
mode of drama_moe.staging (``residency="host"``).

Conventions kept from the reference: kernels run on the caller's current
stream, outputs are freshly allocated, ``ValueError`` for geometry / dtype,
``RuntimeError`` for an unsupported device.  The backend never synchronizes
the host; bad expert ids are reported through a device status word
(``status()`` reads and clears it) and contribute zero.
"""
from __future__ import annotations

import torch
from torch import Tensor, nn

from . import _lib
from .formats import EXPERT_BUFFER_NAMES, FP8_DTYPE, StagedExperts, fp8_bank_struct

DECODE_PAIRS = 256  # route pairs up to which a call runs the decode kernels
MAX_PAIRS = 65536   # route pairs of one call (above DECODE_PAIRS: grouped GEMMs)


class _DeviceState:
    """Per-device workspace and status word of the HIP backends.

    The workspace is zero-filled once when allocated and reused by every call
    on the device (the C ABI keeps what must stay zero at zero).  Growth
    allocates a larger zeroed buffer and RETIRES the old one instead of
    freeing it: a hipGraph captured earlier keeps the old pointer, and its
    replays must still find live memory there.  Growth while a stream is
    being captured is refused (the allocation would belong to the graph's
    private pool): run the call once eagerly, or ``reserve`` first.

    Calls on the device share the buffer, so they are ordered: a call on a
    stream other than the previous call's first waits for that stream (outside
    capture; replays of captured graphs must be ordered by the caller).
    """

    def __init__(self, device: torch.device):
        self.device = device
        self.workspace = torch.zeros(0, dtype=torch.uint8, device=device)
        self.retired: list[Tensor] = []
        self.status = torch.zeros(1, dtype=torch.int32, device=device)
        self._last_stream = None

    def reserve(self, nbytes: int) -> Tensor:
        if self.workspace.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"the expert workspace must grow to {nbytes} bytes inside a graph capture; run this "
                    "call once eagerly (or reserve the workspace) before capturing")
            size = max(nbytes, 2 * self.workspace.numel(), 1 << 20)
            grown = torch.zeros(size, dtype=torch.uint8, device=self.device)
            if self.workspace.numel():
                self.retired.append(self.workspace)
            self.workspace = grown
        return self.workspace

    def workspace_for(self, nbytes: int) -> Tensor:
        ws = self.reserve(nbytes)
        stream = torch.cuda.current_stream(self.device)
        last = self._last_stream
        if last is not None and last != stream and not torch.cuda.is_current_stream_capturing():
            stream.wait_stream(last)
        self._last_stream = stream
        return ws


_STATES: dict[torch.device, _DeviceState] = {}


def device_state(device: torch.device) -> _DeviceState:
    state = _STATES.get(device)
    if state is None:
        state = _STATES[device] = _DeviceState(device)
    return state


def _device_of(x: Tensor) -> torch.device:
    if x.device.type != "cuda":
        raise RuntimeError("The HIP expert backend requires tensors on a ROCm GPU (gfx950); "
                           f"got device {x.device}")
    return torch.device("cuda", x.device.index if x.device.index is not None else torch.cuda.current_device())


class HipExpertBackend:
    """FP8 W8A8 routed experts on gfx950 MFMA (drop-in for TritonExpertBackend).

    ``x_group`` = 128 follows the reference contract (one activation scale per
    128 values); ``"token"`` uses one scale per token row (dynamic per-token
    quantization).  ``gu_dtype`` is the type gate/up are rounded through before
    SiLU (the reference stores them in the compute dtype; ``None`` = x.dtype).
    """

    def __init__(self, *, decode_specialization: bool = True, x_group: int | str = 128,
                 gu_dtype: torch.dtype | None = None) -> None:
        from . import fp8_moe

        if x_group not in (128, "token"):
            raise ValueError("x_group must be 128 or 'token'")
        self.kernel = fp8_moe
        self.decode_specialization = decode_specialization
        self.x_group = x_group
        self.gu_dtype = gu_dtype
        self._checked_devices: set[torch.device] = set()

    # -- reference helpers -------------------------------------------------
    def _check(self, x: Tensor) -> None:
        device = _device_of(x)
        if device not in self._checked_devices:
            if not self.kernel.fp8_gemm_supported([device]):
                raise RuntimeError("The HIP expert backend requires an MI355X-class gfx950 GPU")
            _lib.library()
            self._checked_devices.add(device)

    def status(self, device=None, clear: bool = True) -> int:
        """Read (and clear) the device status bits; synchronizes the stream."""
        state = device_state(torch.device(device) if device is not None else
                             torch.device("cuda", torch.cuda.current_device()))
        value = int(state.status.item())
        if clear:
            state.status.zero_()
        return value

    # -- protocol ----------------------------------------------------------
    def forward(self, x: Tensor, ids: Tensor, weights: Tensor, staged: StagedExperts, *,
                out: Tensor | None = None) -> Tensor:
        self._check(x)
        if x.ndim != 2 or ids.ndim != 2 or ids.shape[0] != x.shape[0] or weights.shape != ids.shape:
            raise ValueError("Expected x [T, H], ids and weights [T, top_k]")
        tokens, top_k = ids.shape
        out = self._out(x, out)
        if tokens == 0:
            return out
        bank = fp8_bank_struct(staged)
        self._validate(x, staged)
        ids, weights = ids.contiguous(), weights.contiguous()
        state = device_state(_device_of(x))
        chunk = max(1, MAX_PAIRS // top_k)
        lib = _lib.library()
        ws = state.workspace_for(lib.dmoe_fp8_workspace_bytes(bank, min(tokens, chunk) * top_k))
        stream = _lib.stream_handle(x.device)
        for start in range(0, tokens, chunk):
            stop = min(tokens, start + chunk)
            _lib.check(lib.dmoe_fp8_moe_forward(
                bank, _lib.ptr(x[start:stop]), _lib.dtype_code(x.dtype), x.stride(0), stop - start,
                _lib.ptr(ids[start:stop]), _lib.dtype_code(ids.dtype), _lib.ptr(weights[start:stop]),
                _lib.dtype_code(weights.dtype), top_k, self._group(x), self._gu(x),
                _lib.ptr(out[start:stop]), _lib.dtype_code(out.dtype), out.stride(0),
                _lib.ptr(ws), ws.numel(), _lib.ptr(state.status), stream))
        return out

    def forward_routed(self, x: Tensor, logits: Tensor, top_k: int, staged: StagedExperts, *,
                       renormalize: bool = True, weights_dtype: torch.dtype | None = None,
                       out: Tensor | None = None):
        """Router + routed experts in one call, no host sync (decode of up to
        64 route pairs: one kernel, else three; prefill: router, permutation,
        quantization, two grouped GEMMs and the combine).  Returns
        (out [T, H], weights [T, top_k], ids [T, top_k])."""
        self._check(x)
        if x.ndim != 2 or logits.ndim != 2 or logits.shape[0] != x.shape[0]:
            raise ValueError("Expected x [T, H] and router logits [T, E]")
        if logits.dtype != torch.float32 or logits.stride(-1) != 1:
            logits = logits.float().contiguous()
        tokens = x.shape[0]
        if tokens * top_k > MAX_PAIRS:
            from .router import route_topk

            weights, ids = route_topk(logits, top_k, renormalize=renormalize,
                                      dtype=weights_dtype or x.dtype)
            return self.forward(x, ids, weights, staged, out=out), weights, ids
        out = self._out(x, out)
        bank = fp8_bank_struct(staged)
        self._validate(x, staged)
        ids = torch.empty((tokens, top_k), dtype=torch.int64, device=x.device)
        weights = torch.empty((tokens, top_k), dtype=weights_dtype or x.dtype, device=x.device)
        state = device_state(_device_of(x))
        lib = _lib.library()
        ws = state.workspace_for(lib.dmoe_fp8_workspace_bytes(bank, tokens * top_k))
        _lib.check(lib.dmoe_fp8_moe_layer(
            bank, _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), tokens, _lib.ptr(logits),
            logits.stride(0), top_k, int(renormalize), _lib.ptr(ids), _lib.ptr(weights),
            _lib.dtype_code(weights.dtype), self._group(x), self._gu(x), _lib.ptr(out),
            _lib.dtype_code(out.dtype), out.stride(0), _lib.ptr(ws), ws.numel(),
            _lib.ptr(state.status), _lib.stream_handle(x.device)))
        return out, weights, ids

    def forward_pairs(self, x: Tensor, ids: Tensor, weights: Tensor, staged: StagedExperts) -> Tensor:
        """Weighted [pairs, hidden] fp32 contributions, before summing."""
        self._check(x)
        if ids.shape != (x.shape[0], 1) or weights.shape != ids.shape:
            raise ValueError("Pair backend expects one expert and weight per input row")
        return self._pairs(x, ids.reshape(-1), weights.reshape(-1), staged, row_div=1)

    def forward_decode_pairs(self, x: Tensor, ids: Tensor, weights: Tensor, staged: StagedExperts) -> Tensor:
        """Small partition of decode rows; fp32 partials (offload.py:346-356)."""
        return self.forward_pairs(x, ids, weights, staged)

    # -- internals ---------------------------------------------------------
    @staticmethod
    def _out(x: Tensor, out: Tensor | None) -> Tensor:
        if out is None:
            return torch.empty_like(x)
        if out.shape != x.shape or out.dtype != x.dtype or out.device != x.device or out.stride(-1) != 1:
            raise ValueError("out must match x in shape, dtype and device, with contiguous rows")
        return out

    def _group(self, x: Tensor) -> int:
        return 128 if self.x_group == 128 else x.shape[-1]

    def _gu(self, x: Tensor) -> int:
        return _lib.dtype_code(self.gu_dtype or x.dtype)

    def _validate(self, x: Tensor, staged: StagedExperts) -> None:
        if x.shape[-1] != staged.hidden:
            raise ValueError(f"Expected hidden rows [N, {staged.hidden}], got {tuple(x.shape)}")
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("Expert compute dtype must be float16, bfloat16 or float32")
        if x.stride(-1) != 1:
            raise ValueError("Hidden rows must be contiguous")
        if staged.device != x.device:
            raise ValueError("Expert bank and activations must share a device")

    def _pairs(self, x: Tensor, ids: Tensor, weights: Tensor, staged: StagedExperts, *,
               row_div: int) -> Tensor:
        pairs = ids.numel()
        out = torch.empty((pairs, staged.hidden), dtype=torch.float32, device=x.device)
        if pairs == 0:
            return out
        bank = fp8_bank_struct(staged)
        self._validate(x, staged)
        ids, weights = ids.contiguous(), weights.contiguous()
        state = device_state(_device_of(x))
        lib = _lib.library()
        ws = state.workspace_for(lib.dmoe_fp8_workspace_bytes(bank, min(pairs, MAX_PAIRS)))
        stream = _lib.stream_handle(x.device)
        shared = x.shape[0] > 1 and x.stride(0) == 0  # an expanded single row
        for start in range(0, pairs, MAX_PAIRS):
            stop = min(pairs, start + MAX_PAIRS)
            if shared:
                rows, div = x[:1], stop - start
            else:
                rows, div = (x if row_div != 1 else x[start:stop]), row_div
            _lib.check(lib.dmoe_fp8_moe_pairs(
                bank, _lib.ptr(rows), _lib.dtype_code(x.dtype), max(rows.stride(0), x.shape[-1]),
                rows.shape[0], div,
                _lib.ptr(ids[start:stop]), _lib.dtype_code(ids.dtype), _lib.ptr(weights[start:stop]),
                _lib.dtype_code(weights.dtype), stop - start, self._group(x), self._gu(x),
                _lib.ptr(out[start:stop]), _lib.ptr(ws), ws.numel(), _lib.ptr(state.status), stream))
        return out


def store_from_module(module: nn.Module):
    """The resident bank of an expert module: the packed store a quantized
    loader bound to it (``_drama_quant_store``, quantized_model.py:106-111),
    else a StagedExperts over its four FP8 buffers (offload.py:107-118)."""
    packed = getattr(module, "_drama_quant_store", None)
    if packed is not None:
        packed.validate()
        return packed
    if not getattr(module, "fp8", False):
        raise ValueError("Expert offload requires FP8 buffers, not dense BF16 weights")
    bank = StagedExperts(**{name: getattr(module, name) for name in EXPERT_BUFFER_NAMES})
    bank.validate()
    return bank


_COMPUTE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def check_route_call(x: Tensor, ids: Tensor, weights: Tensor, hidden: int) -> None:
    """The caller contract of one expert call, checked before any work:
    x [tokens, hidden] in a compute dtype, ids [tokens, top_k >= 1] int32 or
    int64, floating-point weights of the same shape, one device for all."""
    rules = (
        (x.ndim == 2 and x.shape[-1] == hidden,
         lambda: f"Expected hidden rows [N, {hidden}], got {tuple(x.shape)}"),
        (ids.ndim == 2 and ids.shape[0] == x.shape[0] and ids.shape[1] >= 1,
         lambda: "Expert IDs must be [tokens, top_k] with top_k >= 1"),
        (tuple(weights.shape) == tuple(ids.shape), lambda: "Routing weights must have the shape of the expert IDs"),
        (ids.dtype in (torch.int32, torch.int64), lambda: "Expert IDs must be int32 or int64"),
        (weights.is_floating_point(), lambda: "Routing weights must be floating point"),
        (x.dtype in _COMPUTE_DTYPES, lambda: "Expert compute dtype must be float16, bfloat16 or float32"),
        (ids.device == x.device and weights.device == x.device,
         lambda: "Hidden states, expert IDs and routing weights must share a device"),
    )
    for ok, message in rules:
        if not ok:
            raise ValueError(message())


def check_id_range(ids: Tensor, experts: int) -> None:
    """Eager range check of route ids (one host sync)."""
    low, high = (int(v) for v in torch.aminmax(ids))
    if low < 0 or high >= experts:
        raise ValueError(f"Expert IDs must be in [0, {experts})")


def raise_device_status(device: torch.device) -> None:
    """Read (and clear) the device status word of the expert kernels at a
    host sync the caller already has; raise if an earlier call's outputs are
    invalid (a single-launch decode whose hand-off wait gave up) or it met
    expert ids outside the bank."""
    state = device_state(device)
    value = int(state.status.item())
    if not value & (_lib.STATUS_SYNC_TIMEOUT | _lib.STATUS_BAD_EXPERT_ID):
        return
    state.status.zero_()
    if value & _lib.STATUS_SYNC_TIMEOUT:
        raise RuntimeError("an earlier expert call's single-launch decode gave up its hand-off wait (other work "
                           f"held the device's CUs); its outputs are invalid (device status {value:#x})")
    raise ValueError(f"an earlier expert call met expert ids outside the bank (device status {value:#x})")


class _RoutedForward:
    """Forward of an attached expert module: hands ``(x, topk_ids,
    topk_weights)`` to the manager.  ``shadowed`` is the instance-level forward
    it replaced (None when the module used its class's forward), so detaching
    restores exactly what was there."""

    def __init__(self, manager: "ResidentExpertManager", module: nn.Module):
        self.manager = manager
        self.module = module
        self.shadowed = module.__dict__.get("forward")

    def __call__(self, x: Tensor, topk_ids: Tensor, topk_weights: Tensor) -> Tensor:
        return self.manager.forward(self.module, x, topk_ids, topk_weights)


def _attached(module: nn.Module) -> bool:
    # ours (a _RoutedForward instance) or the reference manager's marker
    return isinstance(module.__dict__.get("forward"), _RoutedForward) or hasattr(
        module, "_drama_offload_original_forward")


class ResidentExpertManager:
    """Routes ``experts(x, topk_ids, topk_weights)`` of attached modules to a
    backend -- the caller contract of ExpertOffloadManager.attach / forward
    (offload.py:996-1063).  With ``residency="hbm"`` (default) the whole bank
    is resident in HBM (a host-held bank is copied to the device on its first
    call); with ``residency="host"`` the staging keywords configure the host
    tier of drama_moe.staging (``self.host``).

    Banks are resolved once per module and reused while the module keeps the
    same buffers.  FP8 banks run on ``backend`` (default HipExpertBackend);
    packed banks bound by a quantized loader on a QuantizedExpertBackend of
    their mode.  ``validate_ids=True`` keeps the reference's eager range check
    of the ids (one host sync per call); ``False`` leaves bad ids to the
    device status word so calls can be captured in hipGraphs.  At that host
    sync, ``raise_on_status=True`` (default) also reads the device status
    word and raises if an earlier call's single-launch decode gave up its
    hand-off wait (outputs invalid) or met ids outside the bank; with
    ``validate_ids=False`` there is no sync and the caller reads
    ``backend.status()`` where it has one.
    """

    def __init__(self, *, backend=None, validate_ids: bool = True, residency: str = "hbm",
                 raise_on_status: bool = True, **staging) -> None:
        from .staging import RESIDENCY_MODES, HostResidency, OffloadStatistics, check_staging_sizes

        if residency not in RESIDENCY_MODES:
            raise ValueError(f"residency must be one of {RESIDENCY_MODES}, got {residency!r}")
        unknown = set(staging) - STAGING_KEYWORDS
        if unknown:
            raise TypeError(f"unexpected staging keywords {sorted(unknown)}")
        for flag in ("pin_memory", "profile_transfers", "combined_decode_bank", "packed_staging"):
            if flag in staging and not isinstance(staging[flag], bool):
                raise TypeError(f"{flag} must be a boolean")
        sizes = {k: staging[k] for k in ("max_staged_experts", "max_pair_rows", "cache_experts", "hot_cache_experts")
                 if k in staging}
        check_staging_sizes(sizes.get("max_staged_experts", 8), sizes.get("max_pair_rows", 64),
                       sizes.get("cache_experts", 0), sizes.get("hot_cache_experts"))
        self.backend = backend if backend is not None else HipExpertBackend()
        self.validate_ids = validate_ids
        self.raise_on_status = raise_on_status
        self.residency = residency
        # host mode: the staging tier; hbm mode: the sizes are checked and unused
        self.statistics = OffloadStatistics()
        self.host = HostResidency(pin_memory=staging.get("pin_memory", True),
                                  profile_transfers=staging.get("profile_transfers", False),
                                  statistics=self.statistics, **sizes) if residency == "host" else None
        self.modules: dict[str, nn.Module] = {}
        self.forward_calls = 0
        self._banks: dict[int, tuple] = {}
        self._device_banks: dict[int, tuple] = {}
        self._packed_backends: dict[int, object] = {}
        self.hybrid_decode = None
        self._closed = False

    @property
    def stats(self):
        """Cumulative OffloadStatistics of this manager's host traffic (the
        reference's ``manager.stats``); reading it collects the event times
        of transfers profiled so far."""
        if self.host is not None:
            return self.host.collect()
        return self.statistics

    def _require_open(self) -> None:
        if self._closed:
            raise RuntimeError("This expert manager has been closed")

    def _bank_of(self, module: nn.Module):
        key = tuple(id(getattr(module, name, None)) for name in EXPERT_BUFFER_NAMES) + (
            id(getattr(module, "_drama_quant_store", None)),)
        cached = self._banks.get(id(module))
        if cached is None or cached[0] != key:
            cached = (key, store_from_module(module))
            self._banks[id(module)] = cached
        return cached[1]

    def _backend_for(self, bank):
        if isinstance(bank, StagedExperts):
            return self.backend
        backend = self._packed_backends.get(bank.mode)
        if backend is None:
            from .quantized import QuantizedExpertBackend

            backend = self._packed_backends[bank.mode] = QuantizedExpertBackend(bank.mode)
        return backend

    def attach(self, name: str, module: nn.Module) -> None:
        self._require_open()
        if name in self.modules or _attached(module):
            raise ValueError(f"Expert module {name!r} already has an offload manager")
        self._bank_of(module)
        module.forward = _RoutedForward(self, module)
        self.modules[name] = module

    @torch.no_grad()
    def forward(self, module: nn.Module, x: Tensor, topk_ids: Tensor, topk_weights: Tensor) -> Tensor:
        self._require_open()
        bank = self._bank_of(module)
        check_route_call(x, topk_ids, topk_weights, bank.hidden)
        self.forward_calls += 1
        if x.shape[0] == 0:
            return torch.zeros_like(x)
        backend = self._backend_for(bank)
        if self.host is None:
            self.statistics.forward_calls += 1  # the host tier counts its own calls
        if self.hybrid_decode is not None and self.hybrid_decode.eligible(module, x, topk_ids):
            return self.hybrid_decode.forward(module, bank, x, topk_ids, topk_weights)
        if self.host is not None:
            return self.host.forward(id(module), bank, backend, x, topk_ids, topk_weights)
        if self.validate_ids:
            check_id_range(topk_ids, bank.count)
            if self.raise_on_status:
                raise_device_status(_device_of(x))
        return backend.forward(x, topk_ids, topk_weights, self._on_device(module, bank, x.device))

    def _on_device(self, module: nn.Module, bank, device: torch.device):
        """The bank itself when it lives on ``device``, else its whole copy
        there, made on the module's first call and kept while the module
        holds the same buffers."""
        from .staging import bank_buffers, bank_device, bank_key, device_copy

        if bank_device(bank) == device:
            return bank
        key = (bank_key(bank), device)
        cached = self._device_banks.get(id(module))
        if cached is None or cached[0] != key:
            cached = (key, device_copy(bank, device))
            self._device_banks[id(module)] = cached
            copied = bank_buffers(bank).values()
            self.statistics.h2d_copy_calls += len(copied)
            self.statistics.h2d_bytes += sum(t.numel() * t.element_size() for t in copied)
        return cached[1]

    def configure_hybrid_decode(self, cpu_jobs: int = 0, *, threads: int = 4, device=None,
                                synchronize_return: bool = True, guard_fp8_boundaries: bool = True):
        """Give ``cpu_jobs`` (1-8) route slots of each eligible one-token FP8
        decode call to host cores (drama_moe.hybrid.HybridDecodeRuntime; the
        reference's configure_hybrid_decode, offload.py:1289-1308); 0 turns
        the mode off.  Needs host-held FP8 banks."""
        self._require_open()
        if isinstance(cpu_jobs, bool) or not isinstance(cpu_jobs, int) or not 0 <= cpu_jobs <= 8:
            raise ValueError("Hybrid CPU jobs must be an integer from 0 to 8")
        if isinstance(threads, bool) or not isinstance(threads, int) or not 1 <= threads <= 64:
            raise ValueError("Hybrid native threads must be an integer from 1 to 64")
        replacement = None
        if cpu_jobs:
            from .hybrid import HybridDecodeRuntime

            replacement = HybridDecodeRuntime(
                self, cpu_jobs=cpu_jobs, threads=threads,
                device=device if device is not None else torch.device("cuda", torch.cuda.current_device()),
                synchronize_return=synchronize_return, guard_fp8_boundaries=guard_fp8_boundaries)
        if self.hybrid_decode is not None:
            self.hybrid_decode.close()
        self.hybrid_decode = replacement
        return replacement

    def close(self) -> None:
        if self.hybrid_decode is not None:
            self.hybrid_decode.close()
            self.hybrid_decode = None
        for module in self.modules.values():
            routed = module.__dict__.get("forward")
            if isinstance(routed, _RoutedForward):
                if routed.shadowed is None:
                    del module.forward  # the class's forward shows through again
                else:
                    module.forward = routed.shadowed
        self.modules.clear()
        self._banks.clear()
        self._device_banks.clear()
        self.host = None
        self._closed = True


# Keywords of the reference's install_expert_offload (offload.py:1534-1546)
# that configure its host staging tiers.  With residency="host" the sizes
# and pin_memory configure the staging tier of drama_moe.staging; with every
# expert resident (the default) they are checked and have nothing to
# configure.  profile_transfers times the host tier's copies with HIP events
# (``manager.stats.h2d_seconds``).  combined_decode_bank and packed_staging
# are accepted for call-site compatibility: banks are always staged packed,
# and a decode token whose experts are split between the hot cache and the
# pool runs as grouped pair calls.
STAGING_KEYWORDS = frozenset({"max_staged_experts", "max_pair_rows", "cache_experts", "hot_cache_experts",
                              "pin_memory", "profile_transfers", "combined_decode_bank", "packed_staging"})


def install_expert_offload(backbone: nn.Module, *, backend=None, validate_ids: bool = True, residency: str = "hbm",
                           **staging) -> ResidentExpertManager:
    """Attach a manager to every routed expert module of a backbone (modules
    holding w13_weight and w2_weight, offload.py:1479-1484, 1534).
    ``backend`` is a backend object, or "hip" / "triton" (both mean the gfx950
    FP8 backend).  ``residency`` "hbm" (default) runs every bank from device
    memory, copying a host-held bank to the device once; "host" keeps banks in
    host memory and stages the routed experts per call.  Every bank is
    checked before any forward is replaced."""
    unknown = set(staging) - STAGING_KEYWORDS
    if unknown:
        raise TypeError(f"install_expert_offload() got unexpected keywords {sorted(unknown)}")
    if isinstance(backend, str):
        if backend not in ("hip", "triton"):
            raise ValueError(f"Unknown expert backend {backend!r}: this build provides 'hip'")
        backend = HipExpertBackend()
    targets = [(name, module) for name, module in backbone.named_modules()
               if hasattr(module, "w13_weight") and hasattr(module, "w2_weight")]
    if not targets:
        raise ValueError("Backbone contains no routed expert modules")
    for name, module in targets:
        store_from_module(module)
        if _attached(module):
            raise ValueError("Backbone already has an expert offload manager")
    manager = ResidentExpertManager(backend=backend, validate_ids=validate_ids, residency=residency, **staging)
    for name, module in targets:
        manager.attach(name, module)
    return manager


__all__ = ["HipExpertBackend", "ResidentExpertManager", "install_expert_offload", "check_route_call",
           "store_from_module", "StagedExperts", "FP8_DTYPE", "DECODE_PAIRS"]
