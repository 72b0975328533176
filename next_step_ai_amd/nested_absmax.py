"""Double-quantised NF4 absmax (the bitsandbytes nested quant state).

The reference stores NF4 weights with ``compress_statistics`` and resolves
the nested state to fp32 before building its slot tables (RT:4621-4625,
``safetensor_loader.py:403-406``)::

    absmax = dequantize_blockwise(absmax_u8, state2) + offset

Here the u8 codes stay in the slot tables and the kernels resolve each
absmax as ``fp32(fp32(code2[q] * absmax2[f // blocksize]) + offset)`` while
they stream the weights (f = the absmax's index in the full weight), which is
the same value bit for bit and a quarter of the absmax bytes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._runtime import ptr, require_device, stream_handle


def dynamic_map_signed() -> np.ndarray:
    """bitsandbytes' signed dynamic 8-bit map (``create_dynamic_map(signed=True,
    max_exponent_bits=7, total_bits=8)``), built the way its published
    construction builds it, in torch fp32 on the CPU: for exponent i = 0..6,
    the midpoints of ``linspace(0.1, 1, 2^i + 1)`` scaled by 10^(i-6), with
    both signs; then 0 and 1; ascending (256 fp32 values)."""
    parts = []
    for i in range(7):
        bounds = torch.linspace(0.1, 1.0, (1 << i) + 1, dtype=torch.float32)
        mids = (bounds[:-1] + bounds[1:]) / 2.0
        scale = 10.0 ** (i - 6)
        parts += [scale * mids, -scale * mids]
    parts.append(torch.tensor([0.0, 1.0], dtype=torch.float32))
    out = torch.sort(torch.cat(parts)).values.numpy()
    assert out.size == 256 and out.dtype == np.float32
    return out


_maps: dict[int | None, torch.Tensor] = {}


def dynamic_map_device(device: torch.device) -> torch.Tensor:
    t = _maps.get(device.index)
    if t is None:
        t = torch.from_numpy(dynamic_map_signed()).to(device)
        _maps[device.index] = t
    return t


def default_offset(absmax: torch.Tensor) -> float:
    """bitsandbytes' compress_statistics offset: the mean of the absmax,
    summed in fp64 and rounded once to fp32."""
    return float(np.float32(absmax.to(torch.float64).mean().item()))


@dataclass
class NestedAbsmax:
    """u8 absmax codes ``q`` (the fp32 absmax's shape), second-level scales
    ``absmax2`` (one per ``blocksize`` consecutive entries), the 256-entry
    ``code2`` and the ``offset``."""

    q: torch.Tensor
    absmax2: torch.Tensor
    code2: torch.Tensor
    offset: float
    blocksize: int = 256

    @classmethod
    def from_quant_state(cls, quant_state) -> "NestedAbsmax":
        """From a bitsandbytes-style nested quant state: ``absmax`` (u8),
        ``offset``, ``state2.absmax``, ``state2.code``, ``state2.blocksize``."""
        s2 = quant_state.state2
        device = require_device(quant_state.absmax, "absmax")
        return cls(q=quant_state.absmax.to(device=device, dtype=torch.uint8).contiguous(),
                   absmax2=s2.absmax.to(device=device, dtype=torch.float32).contiguous(),
                   code2=s2.code.to(device=device, dtype=torch.float32).contiguous(),
                   offset=float(quant_state.offset), blocksize=int(s2.blocksize))

    @classmethod
    def quantize(cls, absmax: torch.Tensor, *, blocksize: int = 256, code2: torch.Tensor | None = None,
                 offset: float | None = None) -> "NestedAbsmax":
        """Double-quantise an fp32 absmax vector on the device (bitsandbytes
        ``compress_statistics``: offset = mean, blocks of ``blocksize``,
        nearest ``code2`` entry; ``code2`` defaults to the dynamic map)."""
        device = require_device(absmax, "absmax")
        a = absmax.to(dtype=torch.float32).contiguous().reshape(-1)
        c2 = dynamic_map_device(device) if code2 is None else code2.to(device=device, dtype=torch.float32).contiguous()
        off = default_offset(a) if offset is None else float(np.float32(offset))
        n = int(a.numel())
        q = torch.empty(n, dtype=torch.uint8, device=device)
        a2 = torch.empty((n + blocksize - 1) // blocksize, dtype=torch.float32, device=device)
        _lib.call("nsmlp_absmax_dq_quantize", ptr(a), n, int(blocksize), ptr(c2), off, ptr(q), ptr(a2),
                  stream_handle(device))
        return cls(q=q.reshape(absmax.shape), absmax2=a2, code2=c2, offset=off, blocksize=int(blocksize))

    def resolve(self) -> torch.Tensor:
        """fp32 absmax, as the reference resolves it (RT:4621-4625)."""
        device = require_device(self.q, "q")
        q = self.q.contiguous().reshape(-1)
        out = torch.empty(int(q.numel()), dtype=torch.float32, device=device)
        _lib.call("nsmlp_absmax_dq_dequantize", ptr(q), int(q.numel()), int(self.blocksize), ptr(self.code2),
                  ptr(self.absmax2), float(self.offset), ptr(out), stream_handle(device))
        return out.reshape(self.q.shape)
