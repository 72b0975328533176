"""NF4 LM head on the GPU: the reference's ``_lm_head_forward``
(``runtime/lm_head.py:450-474``) over the meta dict that
``_materialize_lm_head_nf4_on_gpu`` builds (``runtime/lm_head.py:267-350``).

The reference evaluates the head with ``triton_sparse_input_linear_4bit``
and every input block active (``active_idx = arange(in / block_size)``,
lm_head.py:341), i.e. a dense NF4 GEMV over the whole ``[V, H]`` weight.
Here the same product runs through ``nsmlp_dense_linear_nf4_f16``: one
streaming pass over the packed weight per two token rows, row-major NF4 (the
layout bitsandbytes' ``quantize_4bit`` of the ``[V, H]`` weight produces and
the loader hands over, lm_head.py:221-241, 292-303).

``lm_head_forward`` keeps the reference's contract: ``hidden`` [B, S, H]
-> logits [B, S, V] in fp16 (the reference returns ``x.dtype``; bf16 inputs
come back in bf16 after an fp16 computation).  A meta whose ``active_idx``
does not list every block once, in order, goes through
``triton_sparse_input_linear_4bit`` exactly as the reference does.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._runtime import aligned16, as_f16, ptr, require_device, stream_handle
from .nested_absmax import NestedAbsmax

__all__ = ["resolve_lm_head_block_size", "lm_head_nf4_meta", "dense_linear_nf4", "lm_head_forward"]


def resolve_lm_head_block_size(in_features: int) -> int:
    """The column block the reference lists in ``active_idx``: the largest of
    256, 128, ..., 1 dividing ``in_features`` (lm_head.py:27-39, without its
    environment override)."""
    for candidate in (256, 128, 64, 32, 16, 8, 4, 2, 1):
        if int(in_features) % candidate == 0:
            return candidate
    return 1


def lm_head_nf4_meta(packed_weight: torch.Tensor, absmax: torch.Tensor | NestedAbsmax, code: torch.Tensor,
                     out_features: int, in_features: int, quant_block_size: int,
                     device: torch.device | None = None) -> dict:
    """The reference's LM-head meta dict (lm_head.py:337-350): packed [V*H/2]
    u8, absmax [V*H/qbs] fp32 (or a :class:`NestedAbsmax`, kept
    double-quantised), code [16], ``active_idx`` = every block of
    ``resolve_lm_head_block_size(in_features)`` columns."""
    dev = device if device is not None else packed_weight.device
    block_size = resolve_lm_head_block_size(in_features)
    num_blocks = max(1, int(in_features) // block_size)
    meta = {
        "packed_weight": packed_weight.to(device=dev, dtype=torch.uint8).contiguous(),
        "code": code.to(device=dev, dtype=torch.float32).contiguous(),
        "out_features": int(out_features),
        "in_features": int(in_features),
        "quant_block_size": int(quant_block_size),
        "block_size": int(block_size),
        "active_idx": torch.arange(num_blocks, device=dev, dtype=torch.int32).view(1, num_blocks).contiguous(),
    }
    if isinstance(absmax, NestedAbsmax):
        meta["absmax_nested"] = absmax
        meta["absmax"] = None
    else:
        meta["absmax"] = absmax.to(device=dev, dtype=torch.float32).contiguous()
    return meta


def dense_linear_nf4(x: torch.Tensor, packed_weight: torch.Tensor, absmax: torch.Tensor | NestedAbsmax,
                     code: torch.Tensor, out_features: int, in_features: int, quant_block_size: int,
                     *, out_f32: torch.Tensor | None = None) -> torch.Tensor:
    """``x [rows, in] @ W.T`` for a row-major NF4 ``W [out, in]`` (no bias),
    fp32 accumulation, fp16 result [rows, out].  ``out_f32`` ([rows, out]
    fp32, optional) receives the sums before the fp16 rounding."""
    device = require_device(x, "x")
    xf = aligned16(as_f16(x, device).reshape(-1, int(in_features)))
    rows = int(xf.shape[0])
    pw = aligned16(packed_weight.to(device=device, dtype=torch.uint8).contiguous())
    if int(pw.numel()) != int(out_features) * int(in_features) // 2:
        raise RuntimeError("packed_weight size does not match [out_features, in_features] NF4 layout")
    m = _lib.Nf4Matrix()
    m.out_features, m.in_features, m.qbs = int(out_features), int(in_features), int(quant_block_size)
    m.packed = ptr(pw)
    cd = code.to(device=device, dtype=torch.float32).contiguous()
    m.code = ptr(cd)
    keep = [pw, cd]
    n_abs = int(out_features) * int(in_features) // int(quant_block_size)
    if isinstance(absmax, NestedAbsmax):
        q = absmax.q.to(device=device, dtype=torch.uint8).contiguous()
        a2 = absmax.absmax2.to(device=device, dtype=torch.float32).contiguous()
        c2 = absmax.code2.to(device=device, dtype=torch.float32).contiguous()
        if int(q.numel()) != n_abs:
            raise RuntimeError(f"nested absmax holds {int(q.numel())} codes, expected {n_abs}")
        m.dq_block, m.qabsmax, m.absmax2, m.code2, m.offset = int(absmax.blocksize), ptr(q), ptr(a2), ptr(c2), \
            float(absmax.offset)
        keep += [q, a2, c2]
    else:
        am = absmax.to(device=device, dtype=torch.float32).contiguous()
        if int(am.numel()) != n_abs:
            raise RuntimeError(f"absmax holds {int(am.numel())} entries, expected {n_abs}")
        m.absmax = ptr(am)
        keep.append(am)
    out = torch.empty((rows, int(out_features)), device=device, dtype=torch.float16)
    of = None
    if out_f32 is not None:
        if out_f32.device != device or out_f32.dtype != torch.float32 or tuple(out_f32.shape) != (rows, int(out_features)) \
                or not out_f32.is_contiguous():
            raise RuntimeError("out_f32 must be a contiguous fp32 [rows, out_features] tensor on the input's device")
        of = out_f32
    _lib.call("nsmlp_dense_linear_nf4_f16", ctypes.byref(m), ptr(xf), rows, ptr(out), ptr(of), stream_handle(device))
    del keep
    return out


def _covers_every_block(meta: dict) -> bool:
    """``active_idx`` lists blocks 0..n-1 once, in order, in every row (the
    reference's LM-head meta).  Checked on the host once per index tensor: the
    verdict is kept in the dict with the tensor it was computed for and that
    tensor's version counter, so a replaced or modified index is checked
    again."""
    idx = meta["active_idx"]
    cached = meta.get("_nsmlp_dense")
    if cached is not None and cached[0] is idx and cached[1] == idx._version \
            and cached[2] == (int(meta["in_features"]), int(meta["block_size"])):
        return cached[3]
    geom = (int(meta["in_features"]), int(meta["block_size"]))
    n = geom[0] // geom[1]
    verdict = False
    if geom[0] % geom[1] == 0 and idx.dim() == 2 and int(idx.shape[-1]) == n:
        ar = torch.arange(n, dtype=torch.int64).view(1, n)
        verdict = bool(torch.equal(idx.to("cpu", torch.int64), ar.expand(int(idx.shape[0]), n)))
    meta["_nsmlp_dense"] = (idx, idx._version, geom, verdict)
    return verdict


def lm_head_forward(hidden: torch.Tensor, meta: dict) -> torch.Tensor:
    """logits [B, S, V] from hidden [B, S, H] (lm_head.py:450-474)."""
    device = require_device(hidden, "hidden")
    out_dtype = hidden.dtype if hidden.dtype in (torch.float16, torch.bfloat16) else torch.float16
    hidden_flat = hidden.reshape(-1, hidden.shape[-1])
    V = int(meta["out_features"])
    in_features = int(meta["in_features"])
    if _covers_every_block(meta) and in_features % 32 == 0 and in_features <= 16384:
        absmax = meta["absmax_nested"] if meta.get("absmax_nested") is not None else meta["absmax"]
        logits = dense_linear_nf4(hidden_flat, meta["packed_weight"], absmax, meta["code"], V,
                                  int(meta["in_features"]), int(meta["quant_block_size"]))
    else:
        from .sparse_mlp import triton_sparse_input_linear_4bit

        if meta.get("absmax") is None:
            raise RuntimeError("a sparse LM-head selection needs the fp32 absmax")
        rows = int(hidden_flat.shape[0])
        idx = meta["active_idx"]
        idx = idx.expand(rows, -1).contiguous() if int(idx.shape[0]) == 1 else idx[:rows]
        logits = triton_sparse_input_linear_4bit(
            hidden_flat.to(device=device), idx, packed_weight=meta["packed_weight"], absmax=meta["absmax"],
            code=meta["code"], out_features=V, in_features=int(meta["in_features"]),
            quant_block_size=int(meta["quant_block_size"]), bias=None, block_size=int(meta["block_size"]))
    logits = logits if out_dtype == torch.float16 else logits.to(out_dtype)
    return logits.view(*hidden.shape[:-1], V)
