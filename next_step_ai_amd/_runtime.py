"""Device plumbing between torch tensors and the C ABI: raw pointers, the
current HIP stream, per-(device, stream) workspaces and the NF4 code book."""
from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)

_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_codes: dict[int, torch.Tensor] = {}
_supported: dict[int, bool] = {}


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def require_device(t: torch.Tensor, what: str = "input") -> torch.device:
    """The HIP path needs a gfx950 GPU tensor; anything else is an error."""
    if t.device.type != "cuda":
        raise RuntimeError(f"nsmlp: {what} must be a GPU tensor (got {t.device}); there is no CPU path")
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    ok = _supported.get(idx)
    if ok is None:
        ok = bool(_lib.lib().nsmlp_device_supported(idx))
        _supported[idx] = ok
    if not ok:
        raise RuntimeError(f"nsmlp: device {idx} is not a gfx950 GPU")
    return torch.device("cuda", idx)


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Workspace for the current stream of `device`, grown on demand.  Its
    counter region is zeroed once at allocation; kernels keep it zero."""
    key = (device.index, stream_handle(device))
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(int(nbytes), 1 << 20)
            if ws is not None:
                size = max(size, ws.numel() * 2)
            ws = torch.empty(size + 256, dtype=torch.uint8, device=device)
            off = (-ws.data_ptr()) % 256
            ws = ws[off: off + size]
            _lib.call("nsmlp_workspace_init", ptr(ws), ws.numel(), key[1])
            _workspaces[key] = ws
        return ws


_STATUS_TEXT = {
    _lib.NSMLP_STATUS_BLOCK_UNAVAILABLE:
        "a selected block id was out of range, or its block is neither in an HBM slot nor host-copied "
        "(it contributed zero to the output)",
    _lib.NSMLP_STATUS_FIXED_RANGE:
        "a grouped prefill down partial was outside the fixed-point range (|v| >= 2^23, inf or nan); "
        "those outputs are wrong",
}


def status_message(value: int, what: str) -> str:
    parts = [text for bit, text in _STATUS_TEXT.items() if value & bit]
    return f"{what}: " + "; ".join(parts or ["unknown status"]) + f" (status word {value:#x})"


class StatusWord:
    """The kernels' status word, read without stalling the launch stream.

    ``take(ws)`` enqueues ``nsmlp_workspace_take_status``: the workspace's
    status word is ORed into a pinned host word and cleared, and an event
    marks that point of the stream.  ``poll()`` raises ``RuntimeError`` if a
    finished take reported a problem and returns without waiting otherwise;
    ``check()`` waits for the last take first.  The reference raises from
    its gather for such blocks (RT:4530-4578)."""

    def __init__(self, device: torch.device, what: str):
        self.device = device
        self.what = what
        self.host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        out = ctypes.c_void_p()
        _lib.call("nsmlp_host_device_pointer", ctypes.c_void_p(self.host.data_ptr()), ctypes.byref(out))
        self._dptr = int(out.value)
        self._event: torch.cuda.Event | None = None

    def clear(self, ws: torch.Tensor) -> None:
        """Clear the workspace's status word (in stream order) so that the
        next take reports the calls enqueued after this point only, not bits
        an earlier unchecked call on the same workspace left."""
        _lib.call("nsmlp_workspace_take_status", ptr(ws), None, stream_handle(self.device))

    def take(self, ws: torch.Tensor) -> None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"{self.what}: the status check cannot run inside a graph capture")
        _lib.call("nsmlp_workspace_take_status", ptr(ws), self._dptr, stream_handle(self.device))
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._event = ev

    def _read(self) -> None:
        self._event = None
        v = int(self.host[0])
        if v:
            self.host[0] = 0
            raise RuntimeError(status_message(v, self.what))

    def poll(self) -> None:
        if self._event is not None and self._event.query():
            self._read()

    def check(self) -> None:
        if self._event is not None:
            self._event.synchronize()
            self._read()


class BlockCounts:
    """Running counts of the selected blocks a layer's decode calls read from
    HBM slots and from host copies (the reference's runtime status counters,
    RT:1694-1779).  ``take(ws)`` enqueues ``nsmlp_workspace_take_block_counts``
    into a device int64 [2] (no stall; it may be captured in a graph);
    ``hbm``/``host`` read the totals (they wait for the stream)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.counts = torch.zeros(2, dtype=torch.int64, device=device)

    def clear(self, ws: torch.Tensor) -> None:
        """Drop what earlier calls left in the workspace's counters."""
        junk = torch.zeros(2, dtype=torch.int64, device=self.device)
        _lib.call("nsmlp_workspace_take_block_counts", ptr(ws), ptr(junk), stream_handle(self.device))

    def take(self, ws: torch.Tensor) -> None:
        _lib.call("nsmlp_workspace_take_block_counts", ptr(ws), ptr(self.counts), stream_handle(self.device))

    def totals(self) -> tuple[int, int]:
        c = self.counts.to("cpu")
        return int(c[0]), int(c[1])

    def reset(self) -> None:
        self.counts.zero_()


def nf4_code(device: torch.device) -> torch.Tensor:
    t = _codes.get(device.index)
    if t is None:
        t = torch.tensor(NF4_CODE, dtype=torch.float32, device=device)
        _codes[device.index] = t
    return t


def as_f16(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.device != device or t.dtype != torch.float16 or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.float16).contiguous()
    return t


def as_dtype(t: torch.Tensor, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if t.device != device or t.dtype != dtype or not t.is_contiguous():
        t = t.to(device=device, dtype=dtype).contiguous()
    return t


def aligned16(t: torch.Tensor) -> torch.Tensor:
    """`t` itself when it starts on a 16-byte boundary, else a fresh copy
    (allocator blocks are at least 256-byte aligned)."""
    if t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)
