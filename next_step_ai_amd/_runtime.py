"""Device plumbing between torch tensors and the C ABI: raw pointers, the
current HIP stream, per-(device, stream) workspaces and the NF4 code book."""
from __future__ import annotations

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
