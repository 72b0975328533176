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
    """One layer's intermediate dimension cut into ``num_blocks`` blocks of
    ``block_size`` rows (gate/up) and columns (down).  The field names and
    constructor are those the runtime builds from its routing artifact
    (block_bank.py:7-36, RT:906-912); an inconsistent layout cannot be made."""

    layer_idx: int
    hidden_size: int
    intermediate_size: int
    block_size: int
    num_blocks: int

    def __post_init__(self) -> None:
        if int(self.layer_idx) < 0:
            raise RuntimeError(f"block bank: layer index {int(self.layer_idx)} is negative")
        for field in ("hidden_size", "intermediate_size", "block_size"):
            v = int(getattr(self, field))
            if v < 1:
                raise RuntimeError(f"block bank of layer {int(self.layer_idx)}: {field} = {v}, need at least 1")
        whole, rest = divmod(int(self.intermediate_size), int(self.block_size))
        if rest:
            raise RuntimeError(f"block bank of layer {int(self.layer_idx)}: blocks of {int(self.block_size)} leave "
                               f"{rest} of the {int(self.intermediate_size)} intermediate rows over")
        if int(self.num_blocks) != whole:
            raise RuntimeError(f"block bank of layer {int(self.layer_idx)}: {int(self.intermediate_size)} rows in "
                               f"blocks of {int(self.block_size)} make {whole} blocks, not num_blocks="
                               f"{int(self.num_blocks)}")

    def block_bounds(self, block_idx: int) -> tuple[int, int]:
        """[first, last + 1) intermediate index of a block."""
        b, bs = int(block_idx), int(self.block_size)
        if not 0 <= b < int(self.num_blocks):
            raise RuntimeError(f"block bank of layer {int(self.layer_idx)}: no block {b} "
                               f"(it has {int(self.num_blocks)})")
        return b * bs, (b + 1) * bs

    def as_dict(self) -> dict[str, int]:
        return {f: int(getattr(self, f)) for f in
                ("layer_idx", "hidden_size", "intermediate_size", "block_size", "num_blocks")}


def build_intermediate_mlp_block_bank_layout(*, layer_idx: int, hidden_size: int, intermediate_size: int,
                                             block_size: int, num_blocks: int | None = None) -> MlpBlockBankLayout:
    """The layout of a layer; ``num_blocks`` defaults to the number of whole
    blocks (a given count is checked by the layout itself)."""
    nb = int(intermediate_size) // max(1, int(block_size)) if num_blocks is None else int(num_blocks)
    return MlpBlockBankLayout(layer_idx=int(layer_idx), hidden_size=int(hidden_size),
                              intermediate_size=int(intermediate_size), block_size=int(block_size), num_blocks=nb)


def validate_intermediate_mlp_block_bank_params(*, layout: MlpBlockBankLayout, gate_in_features: int,
                                                gate_out_features: int, up_in_features: int, up_out_features: int,
                                                down_in_features: int, down_out_features: int) -> None:
    """The three projections must map hidden -> intermediate (gate, up) and
    intermediate -> hidden (down) at the layout's sizes (block_bank.py:76-101;
    the runtime checks this before a sparse forward, RT:5171-5172).  Every
    mismatch is named in one RuntimeError."""
    H, I = int(layout.hidden_size), int(layout.intermediate_size)
    expected = {"gate": (H, I), "up": (H, I), "down": (I, H)}
    given = {"gate": (int(gate_in_features), int(gate_out_features)),
             "up": (int(up_in_features), int(up_out_features)),
             "down": (int(down_in_features), int(down_out_features))}
    wrong = [f"{name} maps {given[name][0]} -> {given[name][1]} features, the bank needs "
             f"{expected[name][0]} -> {expected[name][1]}" for name in ("gate", "up", "down")
             if given[name] != expected[name]]
    if wrong:
        raise RuntimeError(f"layer {int(layout.layer_idx)}: projections do not fit the block bank: "
                           + "; ".join(wrong))


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
