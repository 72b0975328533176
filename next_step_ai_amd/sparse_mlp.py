"""Drop-in replacements for the reference's sparse-MLP kernel module.

The reference runtime imports five names from
``llama3_neuroplastic/triton_sparse_mlp.py`` (TSM) at
``llama3_neuroplastic/experiments/streaming_llama_runtime.py:49-82`` (RT) and
one more from ``runtime/lm_head.py:15``.  This module exports the same names
with the same signatures, argument meaning and error behaviour (every
shape/dtype/device violation raises ``RuntimeError``), backed by the gfx950
HIP kernels of ``libnsmlp.so``.  Inputs are coerced to the expected
device/dtype/contiguity the way the reference wrappers do (TSM:85-103,
TSM:1414-1436).

Semantics differ from the reference in one deliberate way: NF4 payloads are
indexed row-major (what the runtime passes, RT:4630-4660, RT:4491-4492), not
with the transposed index of the reference's v1 Triton kernels (TSM:496,
TSM:560, TSM:635), which does not match those callers.

Forward only: decode is inference, and ``quant_weight_ref`` is accepted and
ignored.  Activations are computed in fp16; bf16 inputs are converted and the
result is returned in the input dtype.
"""
from __future__ import annotations

import torch

from . import _lib
from ._runtime import (
    aligned16,
    as_dtype,
    as_f16,
    ptr,
    require_device,
    stream_handle,
    workspace,
)

__all__ = [
    "triton_sparse_mlp_available",
    "triton_sparse_mlp_decode_4bit_single_kernel_sm75",
    "triton_fused_sparse_mlp_decode_4bit",
    "triton_sparse_output_linear_4bit",
    "triton_sparse_input_linear_4bit",
    "hip_sparse_mlp_available",
]


def hip_sparse_mlp_available() -> bool:
    """True when libnsmlp.so loads and a gfx950 GPU is visible (TSM:26-29)."""
    try:
        lib = _lib.lib()
    except (RuntimeError, OSError):
        return False
    if not torch.cuda.is_available():
        return False
    return any(lib.nsmlp_device_supported(i) for i in range(torch.cuda.device_count()))


triton_sparse_mlp_available = hip_sparse_mlp_available


def _u8(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return aligned16(as_dtype(t, torch.uint8, device))


def _f32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return as_dtype(t, torch.float32, device)


def _i32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return as_dtype(t, torch.int32, device)


def _opt_f16(t: torch.Tensor | None, device: torch.device) -> torch.Tensor | None:
    return None if t is None else as_f16(t.reshape(-1), device)


def triton_sparse_mlp_decode_4bit_single_kernel_sm75(
    x_flat: torch.Tensor,
    active_blocks: torch.Tensor,
    gate_packed: torch.Tensor,
    gate_absmax: torch.Tensor,
    gate_code: torch.Tensor,
    up_packed: torch.Tensor,
    up_absmax: torch.Tensor,
    up_code: torch.Tensor,
    down_packed: torch.Tensor,
    down_absmax: torch.Tensor,
    down_code: torch.Tensor,
    out: torch.Tensor,
    out_accum: torch.Tensor,
    hidden_size: int,
    block_size: int,
    quant_block_size: int,
    top_k: int,
) -> torch.Tensor:
    """Fused one-token sparse MLP over gathered blocks (TSM:1378-1509).

    gate/up packed [top_k, 32, H/2] u8 + absmax [top_k, 32, H/qbs] f32;
    down packed [H, top_k, 16] u8 + absmax [H, top_k] f32.  Writes the fp16
    result into ``out`` and the fp32 sum into ``out_accum[:H]``; returns
    ``out.view_as(x_flat)``.  ``active_blocks`` is validated, not used (the
    blocks are already gathered, as in the reference kernel).
    """
    if int(block_size) != 32:
        raise RuntimeError("Single-kernel sparse MLP decode currently requires block_size=32")
    if int(top_k) <= 0:
        raise RuntimeError("Single-kernel sparse MLP decode requires top_k > 0")
    hidden_size = int(hidden_size)
    quant_block_size = int(quant_block_size)
    top_k = int(top_k)
    if hidden_size <= 0 or quant_block_size <= 0:
        raise RuntimeError("hidden_size and quant_block_size must be positive")
    device = require_device(x_flat, "x_flat")
    x_vec = aligned16(x_flat.reshape(-1).to(device=device, dtype=torch.float16).contiguous())
    if int(x_vec.numel()) != hidden_size:
        raise RuntimeError(f"x_flat has {int(x_vec.numel())} elements but hidden_size={hidden_size}")
    if int(active_blocks.numel()) != top_k:
        raise RuntimeError(f"active_blocks has {int(active_blocks.numel())} entries but top_k={top_k}")
    gate_packed, up_packed, down_packed = (_u8(t, device) for t in (gate_packed, up_packed, down_packed))
    gate_absmax, up_absmax, down_absmax = (_f32(t, device) for t in (gate_absmax, up_absmax, down_absmax))
    gate_code, up_code, down_code = (_f32(t, device) for t in (gate_code, up_code, down_code))
    bytes_per_row = hidden_size // 2
    absmax_per_row = hidden_size // quant_block_size
    if bytes_per_row <= 0 or absmax_per_row <= 0:
        raise RuntimeError("Invalid hidden_size/quant_block_size for NF4 decode")
    if int(gate_packed.numel()) != top_k * block_size * bytes_per_row:
        raise RuntimeError("gate_packed size does not match [top_k, block_size, hidden_size/2] layout")
    if int(up_packed.numel()) != top_k * block_size * bytes_per_row:
        raise RuntimeError("up_packed size does not match [top_k, block_size, hidden_size/2] layout")
    if int(gate_absmax.numel()) != top_k * block_size * absmax_per_row:
        raise RuntimeError("gate_absmax size does not match [top_k, block_size, hidden_size/quant_block_size] layout")
    if int(up_absmax.numel()) != top_k * block_size * absmax_per_row:
        raise RuntimeError("up_absmax size does not match [top_k, block_size, hidden_size/quant_block_size] layout")
    if int(down_absmax.numel()) != hidden_size * top_k:
        raise RuntimeError("down_absmax size does not match [hidden_size, top_k] layout")
    if int(down_packed.numel()) != hidden_size * top_k * (block_size // 2):
        raise RuntimeError("down_packed size does not match [hidden_size, top_k, block_size/2] layout")
    if int(out_accum.numel()) < hidden_size:
        raise RuntimeError("out_accum scratch is smaller than hidden_size")
    acc = out_accum if (out_accum.device == device and out_accum.dtype == torch.float32
                        and out_accum.is_contiguous()) else torch.empty(hidden_size, dtype=torch.float32,
                                                                        device=device)
    direct = out.device == device and out.dtype == torch.float16 and out.is_contiguous() and out.numel() >= hidden_size
    out_buf = out if direct else torch.empty(hidden_size, dtype=torch.float16, device=device)
    nbytes = int(_lib.lib().nsmlp_single_kernel_workspace_bytes(hidden_size, top_k))
    ws = workspace(nbytes, device)
    _lib.call(
        "nsmlp_single_kernel_decode_f16",
        ptr(x_vec), ptr(gate_packed), ptr(gate_absmax), ptr(gate_code), ptr(up_packed), ptr(up_absmax), ptr(up_code),
        ptr(down_packed), ptr(down_absmax), ptr(down_code), ptr(out_buf), ptr(acc), hidden_size, int(block_size),
        quant_block_size, top_k, ptr(ws), ws.numel(), stream_handle(device),
    )
    if acc is not out_accum:
        out_accum.reshape(-1)[:hidden_size].copy_(acc)
    if not direct:
        out.reshape(-1)[:hidden_size].copy_(out_buf)
    return out.view_as(x_flat)


def triton_sparse_output_linear_4bit(
    x_flat: torch.Tensor,
    active_idx: torch.Tensor,
    flat_mask: torch.Tensor,
    *,
    packed_weight: torch.Tensor,
    absmax: torch.Tensor,
    code: torch.Tensor,
    input_dim: int,
    quant_block_size: int,
    bias: torch.Tensor | None,
    block_size: int,
    quant_weight_ref: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gate/up over the active slots of each row (TSM:1340-1375):
    ``out[t, s*32+j] = (W[s*32+j] . x[t] + bias) * flat_mask[t, s*32+j]`` for
    the slots s in ``active_idx[t]``, 0 elsewhere.  W is the gathered
    row-major NF4 weight [A*32, input_dim]."""
    del quant_weight_ref
    device = require_device(x_flat, "x_flat")
    out_dtype = x_flat.dtype if x_flat.dtype in (torch.float16, torch.bfloat16) else torch.float16
    if int(block_size) <= 0:
        raise RuntimeError("block_size must be > 0 for triton_sparse_output_linear_4bit")
    if int(input_dim) % int(block_size) != 0:
        raise RuntimeError(f"input_dim ({int(input_dim)}) must be divisible by block_size ({int(block_size)})")
    x = as_f16(x_flat, device)
    rows = int(x.shape[0])
    width = int(flat_mask.shape[1])
    idx = _i32(active_idx, device)
    kk = int(idx.shape[1]) if idx.dim() == 2 else int(idx.numel())
    out = torch.zeros((rows, width), device=device, dtype=torch.float16)
    if rows > 0 and kk > 0 and width > 0:
        if width % int(block_size) != 0:
            raise RuntimeError("flat_mask width must be a multiple of block_size")
        A = width // int(block_size)
        mask = as_f16(flat_mask, device)
        pw = _u8(packed_weight, device)
        if int(pw.numel()) != A * int(block_size) * int(input_dim) // 2:
            raise RuntimeError("packed_weight size does not match [A*block_size, input_dim] NF4 layout")
        nbytes = int(_lib.lib().nsmlp_output_linear_workspace_bytes(rows, kk, int(input_dim)))
        ws = workspace(nbytes, device)
        _lib.call(
            "nsmlp_output_linear_nf4_f16",
            ptr(x), rows, int(input_dim), ptr(idx), kk, A, ptr(mask), ptr(pw), ptr(_f32(absmax, device)),
            ptr(_f32(code, device)), int(quant_block_size), ptr(_opt_f16(bias, device)), int(block_size), ptr(out),
            ptr(ws), ws.numel(), stream_handle(device),
        )
    return out if out_dtype == torch.float16 else out.to(out_dtype)


def triton_sparse_input_linear_4bit(
    x_flat: torch.Tensor,
    active_idx: torch.Tensor,
    *,
    packed_weight: torch.Tensor,
    absmax: torch.Tensor,
    code: torch.Tensor,
    out_features: int,
    in_features: int,
    quant_block_size: int,
    bias: torch.Tensor | None,
    block_size: int,
    quant_weight_ref: torch.Tensor | None = None,
) -> torch.Tensor:
    """Down over the active input slots of each row (TSM:1303-1337):
    ``out[t, o] = sum_{s in active_idx[t]} W[o, s*32:(s+1)*32] . x[t, s*32:(s+1)*32] + bias[o]``
    with W the row-major NF4 weight [out_features, in_features]."""
    del quant_weight_ref
    device = require_device(x_flat, "x_flat")
    out_dtype = x_flat.dtype if x_flat.dtype in (torch.float16, torch.bfloat16) else torch.float16
    if int(block_size) <= 0:
        raise RuntimeError("block_size must be > 0 for triton_sparse_input_linear_4bit")
    if int(in_features) % int(block_size) != 0:
        raise RuntimeError(
            f"in_features ({int(in_features)}) must be divisible by block_size ({int(block_size)})"
        )
    x = as_f16(x_flat, device)
    rows = int(x.shape[0])
    idx = _i32(active_idx, device)
    kk = int(idx.shape[1]) if idx.dim() == 2 else int(idx.numel())
    out = torch.empty((rows, int(out_features)), device=device, dtype=torch.float16)
    if rows == 0 or int(out_features) == 0:
        out.zero_()
    elif kk == 0:
        if bias is not None:
            out.copy_(as_f16(bias, device).reshape(1, -1).expand_as(out))
        else:
            out.zero_()
    else:
        pw = _u8(packed_weight, device)
        if int(pw.numel()) != int(out_features) * int(in_features) // 2:
            raise RuntimeError("packed_weight size does not match [out_features, in_features] NF4 layout")
        _lib.call(
            "nsmlp_input_linear_nf4_f16",
            ptr(x), rows, int(in_features), ptr(idx), kk, ptr(pw), ptr(_f32(absmax, device)),
            ptr(_f32(code, device)), int(quant_block_size), int(out_features), ptr(_opt_f16(bias, device)),
            int(block_size), ptr(out), stream_handle(device),
        )
    return out if out_dtype == torch.float16 else out.to(out_dtype)


def triton_fused_sparse_mlp_decode_4bit(
    x_flat: torch.Tensor,
    active_idx: torch.Tensor,
    flat_mask: torch.Tensor,
    *,
    gate_packed_weight: torch.Tensor,
    gate_absmax: torch.Tensor,
    gate_code: torch.Tensor,
    gate_input_dim: int,
    gate_quant_block_size: int,
    gate_bias: torch.Tensor | None,
    up_packed_weight: torch.Tensor,
    up_absmax: torch.Tensor,
    up_code: torch.Tensor,
    up_input_dim: int,
    up_quant_block_size: int,
    up_bias: torch.Tensor | None,
    down_packed_weight: torch.Tensor,
    down_absmax: torch.Tensor,
    down_code: torch.Tensor,
    down_out_features: int,
    down_in_features: int,
    down_quant_block_size: int,
    down_bias: torch.Tensor | None,
    block_size: int,
) -> torch.Tensor:
    """gate -> up -> silu*up -> down over the active slots (TSM:1519-1585).

    One row (a decode token) with the runtime's layouts (gate/up gathered
    [A*32, H], down gathered [H, A*32] with quant block 32) runs the fused
    two-kernel decode path; anything else runs the composition of the
    output/input linears, as the reference does."""
    device = require_device(x_flat, "x_flat")
    rows = int(x_flat.shape[0])
    H = int(gate_input_dim)
    width = int(flat_mask.shape[1]) if flat_mask.dim() == 2 else int(flat_mask.numel())
    bs = int(block_size)
    fused_ok = (
        rows == 1 and bs == 32 and width % 32 == 0 and width > 0
        and int(up_input_dim) == H and int(gate_quant_block_size) == int(up_quant_block_size)
        and int(down_quant_block_size) == 32 and int(down_in_features) == width
        and int(down_out_features) == H and H % 256 == 0 and int(gate_quant_block_size) % 32 == 0
        and H % int(gate_quant_block_size) == 0
    )
    if fused_ok:
        A = width // 32
        x = aligned16(as_f16(x_flat, device).reshape(-1))
        idx = _i32(active_idx, device).reshape(-1)
        kk = int(idx.numel())
        gp, upk, dp = (_u8(t, device) for t in (gate_packed_weight, up_packed_weight, down_packed_weight))
        if int(gp.numel()) != width * H // 2 or int(upk.numel()) != width * H // 2 or int(dp.numel()) != H * width // 2:
            raise RuntimeError("packed weight sizes do not match the gathered [A*32, H] / [H, A*32] layouts")
        out = torch.empty((1, H), device=device, dtype=torch.float16)
        if kk > 0:
            nbytes = int(_lib.lib().nsmlp_fused_decode_workspace_bytes(H, kk))
            ws = workspace(nbytes, device)
            _lib.call(
                "nsmlp_fused_decode_gathered_f16",
                ptr(x), H, ptr(idx), kk, A, ptr(as_f16(flat_mask, device)),
                ptr(gp), ptr(_f32(gate_absmax, device)), ptr(_f32(gate_code, device)), ptr(_opt_f16(gate_bias, device)),
                ptr(upk), ptr(_f32(up_absmax, device)), ptr(_f32(up_code, device)), ptr(_opt_f16(up_bias, device)),
                ptr(dp), ptr(_f32(down_absmax, device)), ptr(_f32(down_code, device)),
                ptr(_opt_f16(down_bias, device)), int(gate_quant_block_size), ptr(out), ptr(ws), ws.numel(),
                stream_handle(device),
            )
        elif down_bias is not None:
            out.copy_(as_f16(down_bias, device).reshape(1, -1))
        else:
            out.zero_()
        return out if x_flat.dtype != torch.bfloat16 else out.to(torch.bfloat16)
    gate = triton_sparse_output_linear_4bit(
        x_flat, active_idx, flat_mask, packed_weight=gate_packed_weight, absmax=gate_absmax, code=gate_code,
        input_dim=int(gate_input_dim), quant_block_size=int(gate_quant_block_size), bias=gate_bias,
        block_size=bs, quant_weight_ref=None,
    )
    up = triton_sparse_output_linear_4bit(
        x_flat, active_idx, flat_mask, packed_weight=up_packed_weight, absmax=up_absmax, code=up_code,
        input_dim=int(up_input_dim), quant_block_size=int(up_quant_block_size), bias=up_bias,
        block_size=bs, quant_weight_ref=None,
    )
    g16 = as_f16(gate, device)
    u16 = as_f16(up, device)
    activated = torch.empty_like(g16)
    _lib.call("nsmlp_silu_mul_f16", ptr(g16), ptr(u16), ptr(activated), g16.numel(), stream_handle(device))
    return triton_sparse_input_linear_4bit(
        activated if x_flat.dtype != torch.bfloat16 else activated.to(torch.bfloat16), active_idx,
        packed_weight=down_packed_weight, absmax=down_absmax, code=down_code,
        out_features=int(down_out_features), in_features=int(down_in_features),
        quant_block_size=int(down_quant_block_size), bias=down_bias, block_size=bs, quant_weight_ref=None,
    )
