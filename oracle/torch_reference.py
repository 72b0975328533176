"""Torch-CPU restatement of the reference's PyTorch decode path for one layer.

Test and baseline infrastructure only: the CPU baseline the benchmark times
beside the GPU (and a cross-check of the oracle's fallback leg).  Nothing in
the product imports it.

It follows, op for op on the CPU, what the reference runs for one decode
token when its Triton kernels are not used (paths relative to the reference
repository, RT = llama3_neuroplastic/experiments/streaming_llama_runtime.py):

* router, RT:4209-4238 (``_compute_sparse_basis_latent``) and RT:4311-4352
  (``_route_sparse_mlp``): ``F.linear`` latent, the basis_top_k mask when
  basis_top_k < R, ``F.linear`` scores ``clamp_min(0)``, optional
  ``down_block_norm`` scaling, ``topk`` indices;
* active layout, RT:4857-4908 (``_build_sparse_active_layout``): unique
  ordered blocks, ``active_local``, the per-row ``flat_mask``;
* dequant fallback MLP, RT:5433-5492: gate/up rows dequantised to the
  compute dtype as bitsandbytes does (fp32 ``code[nibble] * absmax``, then
  the cast), ``F.linear(x, W) * flat_mask``, ``F.silu(gate) * up``; the down
  columns as ``code.to(dtype)[nibble]`` pairs times ``absmax.to(dtype)``
  (a product in the compute dtype), ``F.linear(act, Wd)``.

The blocks are passed in already gathered (the slot-table layouts the
runtime hands the fallback: gate/up [A, 32, H/2] u8 with [A, 32, H/qbs]
fp32 absmax, down [H, A, 16] u8 with [H, A] fp32 absmax), in the order of
the selection's ascending block ids (the ``ordered_blocks`` order of the
layout on the CPU).  ``dtype`` is the runtime's compute dtype: fp16 (the
reference's default) or fp32 (a labelled variant).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

BLOCK = 32


def route(x: torch.Tensor, enc_w: torch.Tensor, enc_b: torch.Tensor | None, score_w: torch.Tensor,
          score_b: torch.Tensor | None, k: int, *, basis_top_k: int | None = None,
          down_block_norm: torch.Tensor | None = None) -> torch.Tensor:
    """Active block indices [rows, k] (RT:4209-4238, RT:4311-4352)."""
    latent = F.linear(x, enc_w, enc_b)
    R = int(latent.shape[-1])
    btk = R if basis_top_k is None else max(1, min(int(basis_top_k), R))
    if btk < R:
        idx = torch.topk(latent.abs(), k=btk, dim=-1).indices
        mask = torch.zeros_like(latent)
        mask.scatter_(1, idx, 1.0)
        latent = latent * mask
    scores = F.linear(latent, score_w, score_b).clamp_min(0.0)
    if down_block_norm is not None:
        scores = scores * down_block_norm.to(dtype=scores.dtype).unsqueeze(0)
    kk = max(1, min(int(k), int(scores.shape[-1])))
    return scores.topk(kk, dim=-1).indices


def active_layout(active_blocks: torch.Tensor, rows: int, max_valid_blocks: int, dtype: torch.dtype):
    """(ordered_blocks, active_local, flat_mask, active_neurons) as RT:4857-4908
    builds them without a hot cache (the hot-first reorder is the identity)."""
    ab = active_blocks.to(torch.long).view(rows, -1)
    union = ab.reshape(-1)
    if rows > 1:
        union = union.unique(sorted=True)
    ordered = union[(union >= 0) & (union < int(max_valid_blocks))].unique(sorted=False).contiguous()
    A = int(ordered.numel())
    lookup = torch.full((int(max_valid_blocks),), -1, dtype=torch.int32)
    lookup[ordered] = torch.arange(A, dtype=torch.int32)
    local = torch.full(ab.shape, -1, dtype=torch.int32)
    valid = (ab >= 0) & (ab < int(max_valid_blocks))
    local[valid] = lookup[ab[valid]]
    al = local.long()
    vm = al >= 0
    slot_mask = torch.zeros((rows, A), dtype=dtype)
    slot_mask.scatter_(1, al.clamp(min=0), vm.to(dtype))
    flat_mask = slot_mask.repeat_interleave(BLOCK, dim=1).contiguous()
    neurons = (ordered.unsqueeze(-1) * BLOCK + torch.arange(BLOCK, dtype=torch.long)).reshape(-1)
    return ordered, local, flat_mask, neurons


def _dequant_rows(packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor, qbs: int,
                  dtype: torch.dtype) -> torch.Tensor:
    """bitsandbytes NF4 dequantisation of a flat row-major payload: element
    2i is the high nibble of byte i; fp32 code * absmax per qbs elements, then
    the cast to ``dtype``."""
    p = packed.reshape(-1)
    nib = torch.stack(((p >> 4) & 0x0F, p & 0x0F), dim=-1).reshape(-1).to(torch.long)
    w = code.to(torch.float32).index_select(0, nib).view(-1, int(qbs)) * absmax.reshape(-1, 1).to(torch.float32)
    return w.reshape(-1).to(dtype)


def fallback_mlp(x: torch.Tensor, flat_mask: torch.Tensor, gate_packed: torch.Tensor, gate_absmax: torch.Tensor,
                 up_packed: torch.Tensor, up_absmax: torch.Tensor, down_packed: torch.Tensor,
                 down_absmax: torch.Tensor, code: torch.Tensor, qbs: int, dtype: torch.dtype) -> torch.Tensor:
    """The dequant fallback of RT:5433-5492 over gathered blocks; x [rows, H]."""
    H = int(x.shape[-1])
    A = int(down_absmax.shape[1])
    K_S = A * BLOCK
    wg = _dequant_rows(gate_packed, gate_absmax, code, qbs, dtype).view(K_S, H)
    gate = F.linear(x, wg) * flat_mask
    del wg
    wu = _dequant_rows(up_packed, up_absmax, code, qbs, dtype).view(K_S, H)
    up = F.linear(x, wu) * flat_mask
    del wu
    act = F.silu(gate) * up
    code_d = code.to(dtype)
    pd = down_packed.view(H, A, 16)
    pairs = torch.empty((H, A, 16, 2), dtype=dtype)
    hi = ((pd >> 4) & 0x0F).to(torch.long)
    pairs[..., 0] = code_d.index_select(0, hi.reshape(-1)).view_as(hi)
    del hi
    lo = (pd & 0x0F).to(torch.long)
    pairs[..., 1] = code_d.index_select(0, lo.reshape(-1)).view_as(lo)
    del lo
    wd = pairs.reshape(H, A, BLOCK)
    wd.mul_(down_absmax.view(H, A).unsqueeze(-1).to(dtype))
    return F.linear(act, wd.reshape(H, K_S).contiguous())


def decode_layer(x: torch.Tensor, enc_w: torch.Tensor, enc_b: torch.Tensor | None, score_w: torch.Tensor,
                 score_b: torch.Tensor | None, k: int, gathered: tuple, code: torch.Tensor, qbs: int,
                 dtype: torch.dtype = torch.float16):
    """One decode token through one layer: route, layout, fallback MLP.
    ``gathered`` = (gate_packed, gate_absmax, up_packed, up_absmax,
    down_packed, down_absmax) of the selected blocks in ascending id order.
    Returns (out [1, H], ordered block ids)."""
    xd = x.reshape(1, -1).to(dtype)
    active = route(xd, enc_w.to(dtype), None if enc_b is None else enc_b.to(dtype), score_w.to(dtype),
                   None if score_b is None else score_b.to(dtype), k)
    ordered, _, flat_mask, _ = active_layout(active, 1, int(score_w.shape[0]), dtype)
    out = fallback_mlp(xd, flat_mask, *gathered, code, qbs, dtype)
    return out, ordered
