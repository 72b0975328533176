"""Host-side layout logic of the sparse-MLP path.

``MlpBlockBankLayout`` / ``validate_intermediate_mlp_block_bank_params``
keep the contract of ``llama3_neuroplastic/experiments/runtime/block_bank.py``
(:7-101): I % block == 0, NB == I / block, gate/up map H -> I, down I -> H.

``build_sparse_active_layout`` keeps the outputs of RT:4857-4908 for callers
of the reference-signature kernels (``ordered_blocks``, ``active_local``,
``flat_mask``, ``active_neurons``).  The native decode path does not need
it: the router hands the selected blocks to the kernels on the device.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class MlpBlockBankLayout:
    layer_idx: int
    hidden_size: int
    intermediate_size: int
    block_size: int
    num_blocks: int

    def __post_init__(self) -> None:
        if int(self.layer_idx) < 0:
            raise RuntimeError(f"layer_idx must be >= 0, got {int(self.layer_idx)}")
        if int(self.hidden_size) <= 0:
            raise RuntimeError(f"hidden_size must be > 0, got {int(self.hidden_size)}")
        if int(self.intermediate_size) <= 0:
            raise RuntimeError(f"intermediate_size must be > 0, got {int(self.intermediate_size)}")
        if int(self.block_size) <= 0:
            raise RuntimeError(f"block_size must be > 0, got {int(self.block_size)}")
        if int(self.intermediate_size) % int(self.block_size) != 0:
            raise RuntimeError(
                f"intermediate_size={int(self.intermediate_size)} is not divisible by block_size={int(self.block_size)}"
            )
        expected = int(self.intermediate_size) // int(self.block_size)
        if int(self.num_blocks) != expected:
            raise RuntimeError(
                f"num_blocks={int(self.num_blocks)} does not match intermediate_size/block_size={expected}"
            )

    def block_bounds(self, block_idx: int) -> tuple[int, int]:
        i = int(block_idx)
        if i < 0 or i >= int(self.num_blocks):
            raise RuntimeError(f"block index out of range: {i} (num_blocks={int(self.num_blocks)})")
        start = i * int(self.block_size)
        return start, start + int(self.block_size)

    def as_dict(self) -> dict[str, int]:
        return {
            "layer_idx": int(self.layer_idx),
            "hidden_size": int(self.hidden_size),
            "intermediate_size": int(self.intermediate_size),
            "block_size": int(self.block_size),
            "num_blocks": int(self.num_blocks),
        }


def build_intermediate_mlp_block_bank_layout(*, layer_idx: int, hidden_size: int, intermediate_size: int,
                                             block_size: int, num_blocks: int | None = None) -> MlpBlockBankLayout:
    inferred = int(intermediate_size) // max(int(block_size), 1)
    return MlpBlockBankLayout(
        layer_idx=int(layer_idx),
        hidden_size=int(hidden_size),
        intermediate_size=int(intermediate_size),
        block_size=int(block_size),
        num_blocks=int(inferred if num_blocks is None else num_blocks),
    )


def validate_intermediate_mlp_block_bank_params(*, layout: MlpBlockBankLayout, gate_in_features: int,
                                                gate_out_features: int, up_in_features: int, up_out_features: int,
                                                down_in_features: int, down_out_features: int) -> None:
    H, I = int(layout.hidden_size), int(layout.intermediate_size)
    if int(gate_in_features) != H or int(up_in_features) != H:
        raise RuntimeError(
            f"Layer {int(layout.layer_idx)} block-bank mismatch: gate/up in_features must equal hidden_size={H} "
            f"(got gate={int(gate_in_features)}, up={int(up_in_features)})."
        )
    if int(gate_out_features) != I or int(up_out_features) != I:
        raise RuntimeError(
            f"Layer {int(layout.layer_idx)} block-bank mismatch: gate/up out_features must equal "
            f"intermediate_size={I} (got gate={int(gate_out_features)}, up={int(up_out_features)})."
        )
    if int(down_out_features) != H or int(down_in_features) != I:
        raise RuntimeError(
            f"Layer {int(layout.layer_idx)} block-bank mismatch: down_proj expected out={H}, in={I}; "
            f"got out={int(down_out_features)}, in={int(down_in_features)}."
        )


def build_sparse_active_layout(*, active_blocks: torch.Tensor, rows: int, block_size: int, max_valid_blocks: int,
                               dtype: torch.dtype, device: torch.device,
                               hot_blocks: torch.Tensor | None = None):
    """Counterpart of ``_build_sparse_active_layout`` (RT:4857-4908):
    union of the rows' blocks, optional hot-first order (RT:1975-1980), range
    filter, ``unique`` (ascending on the CPU), local slot map and flat mask."""
    ab = active_blocks.detach().to(device="cpu", dtype=torch.long).view(int(rows), -1)
    union = ab.reshape(-1)
    if int(rows) > 1:
        union = union.unique(sorted=True)
    if hot_blocks is not None and int(hot_blocks.numel()) > 0 and int(union.numel()) > 1:
        is_hot = torch.isin(union, hot_blocks.to(dtype=union.dtype))
        union = torch.cat([union[is_hot], union[~is_hot]])
    union = union[(union >= 0) & (union < int(max_valid_blocks))]
    ordered = union.unique(sorted=False).to(dtype=torch.long).contiguous()
    A = int(ordered.numel())
    if A <= 0:
        return (
            ordered,
            torch.empty((int(rows), ab.shape[1]), dtype=torch.int32, device=device),
            torch.empty((int(rows), 0), dtype=dtype, device=device),
            torch.empty((0,), dtype=torch.long),
        )
    lookup = torch.full((int(max_valid_blocks),), -1, dtype=torch.int32)
    lookup[ordered] = torch.arange(A, dtype=torch.int32)
    local = torch.full(ab.shape, -1, dtype=torch.int32)
    valid = (ab >= 0) & (ab < int(max_valid_blocks))
    if bool(valid.any()):
        local[valid] = lookup[ab[valid]]
    slot_mask = torch.zeros((int(rows), A), dtype=dtype)
    for t in range(int(rows)):
        s = local[t][local[t] >= 0].long()
        slot_mask[t, s] = 1
    flat_mask = slot_mask.repeat_interleave(int(block_size), dim=1).contiguous()
    neurons = (ordered.unsqueeze(-1) * int(block_size) + torch.arange(int(block_size))).reshape(-1)
    return ordered, local.to(device), flat_mask.to(device), neurons.contiguous()
