"""Seeded synthetic sparse-MLP layers generated on the GPU.

Weights are drawn from N(0, std) with a counter-based generator (the value
of element i depends only on (seed, i)) and quantised to NF4 on the device
(blocksize ``qbs``, fp32 absmax), in the reference layouts: gate/up
``[I, H]`` and down ``[H, I]`` row-major.  With ``double_quant`` the absmax
are then double-quantised as bitsandbytes ``compress_statistics`` does
(second-level blocks of 256, offset = mean, the dynamic 8-bit map); the
layer keeps both that nested state and its fp32 resolution (the absmax the
reference computes with, RT:4621-4625).  The router (encoder, score
weight/bias) is fp16 ~ N(0, std); the token is fp16 ~ N(0, 1).  Seeds follow
``seed = 1000 * config + layer``; each tensor uses a sub-stream of it.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._runtime import ptr, stream_handle
from .nested_absmax import NestedAbsmax
from .slot_table import SparseMlpLayer, SparseMlpRouter, SparseMlpSlotTable

_STREAMS = {"gate": 1, "up": 2, "down": 3, "enc_w": 4, "enc_b": 5, "score_w": 6, "score_b": 7, "x": 8}


def sub_seed(seed: int, name: str) -> int:
    return (int(seed) * 64 + _STREAMS[name]) & 0xFFFFFFFFFFFFFFFF


def synth_nf4(seed: int, n: int, qbs: int, std: float, device: torch.device):
    packed = torch.empty(n // 2, dtype=torch.uint8, device=device)
    absmax = torch.empty(n // qbs, dtype=torch.float32, device=device)
    _lib.call("nsmlp_synth_nf4", seed, n, qbs, float(std), ptr(packed), ptr(absmax), stream_handle(device))
    return packed, absmax


def synth_normal_f16(seed: int, shape, std: float, device: torch.device) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float16, device=device)
    _lib.call("nsmlp_synth_normal_f16", seed, out.numel(), float(std), ptr(out), stream_handle(device))
    return out


def synth_normal_f32(seed: int, shape, std: float, device: torch.device) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float32, device=device)
    _lib.call("nsmlp_synth_normal_f32", seed, out.numel(), float(std), ptr(out), stream_handle(device))
    return out


@dataclass
class SyntheticLayer:
    H: int
    I: int
    R: int
    qbs: int
    seed: int
    gate_packed: torch.Tensor
    gate_absmax: torch.Tensor
    up_packed: torch.Tensor
    up_absmax: torch.Tensor
    down_packed: torch.Tensor | None  # row-major reference layout (None once dropped)
    down_absmax: torch.Tensor | None
    enc_w: torch.Tensor
    enc_b: torch.Tensor
    score_w: torch.Tensor
    score_b: torch.Tensor
    x: torch.Tensor
    # double-quantised absmax ("gate", "up", "down"); the *_absmax fields above
    # then hold its fp32 resolution
    nested: dict | None = None

    @property
    def NB(self) -> int:
        return self.I // 32

    def router(self, basis_top_k: int | None = None) -> SparseMlpRouter:
        return SparseMlpRouter(enc_w=self.enc_w, enc_b=self.enc_b, score_w=self.score_w, score_b=self.score_b,
                               basis_top_k=basis_top_k)

    def routing_dict(self, top_k: int, basis_top_k: int | None = None) -> dict:
        """The runtime's per-layer routing dict shape (RT:956-979)."""
        return {
            "enc_w": self.enc_w, "enc_b": self.enc_b, "route_score_weight": self.score_w,
            "route_score_bias": self.score_b, "down_block_norm": None, "top_k": int(top_k),
            "basis_top_k": int(self.R if basis_top_k is None else basis_top_k), "num_blocks": self.NB,
            "block_size": 32,
        }

    def slot_table(self, resident_blocks: torch.Tensor | None = None, host_copy: bool = False,
                   drop_reference_down: bool = False, absmax: str = "auto",
                   capacity: int | None = None) -> SparseMlpSlotTable:
        """``absmax``: "auto" (the nested state when the layer has one),
        "dq" (nested) or "f32" (fp32 absmax)."""
        if self.down_packed is None:
            raise RuntimeError("the row-major down weight was dropped")
        use_dq = absmax == "dq" or (absmax == "auto" and self.nested is not None)
        if use_dq and self.nested is None:
            raise RuntimeError("the layer has no double-quantised absmax")
        if use_dq:
            ga, ua, da = self.nested["gate"], self.nested["up"], self.nested["down"]
        else:
            if self.gate_absmax is None:
                raise RuntimeError("the fp32 absmax were dropped")
            ga, ua, da = self.gate_absmax, self.up_absmax, self.down_absmax
        t = SparseMlpSlotTable.from_reference(
            gate_packed=self.gate_packed, gate_absmax=ga, up_packed=self.up_packed, up_absmax=ua,
            down_packed=self.down_packed, down_absmax=da, H=self.H, I=self.I, qbs=self.qbs,
            resident_blocks=resident_blocks, host_copy=host_copy, capacity=capacity)
        if drop_reference_down:
            self.down_packed = None
            self.down_absmax = None
        return t

    def layer(self, top_k: int, **kw) -> SparseMlpLayer:
        return SparseMlpLayer(self.router(), self.slot_table(**kw), top_k)


def make_synthetic_layer(*, H: int, I: int, R: int, seed: int, device: torch.device, qbs: int = 64,
                         std: float = 0.02, double_quant: bool = False, keep_f32_absmax: bool = True,
                         dq_block: int = 256, gate_up_std: float | None = None) -> SyntheticLayer:
    """``gate_up_std`` (default ``std``): the gate/up weights' deviation; a
    stack of layers chained as x <- x + mlp(x) with no norm in between stays
    finite when it is small (the MLP's gain grows with |x|^2)."""
    if I % 32 != 0 or (I * H) % qbs != 0:
        raise RuntimeError("I must be a multiple of 32 and I*H a multiple of qbs")
    NB = I // 32
    gu_std = std if gate_up_std is None else float(gate_up_std)
    gp, ga = synth_nf4(sub_seed(seed, "gate"), I * H, qbs, gu_std, device)
    upk, ua = synth_nf4(sub_seed(seed, "up"), I * H, qbs, gu_std, device)
    dp, da = synth_nf4(sub_seed(seed, "down"), H * I, qbs, std, device)
    nested = None
    if double_quant:
        nested = {name: NestedAbsmax.quantize(a, blocksize=dq_block) for name, a in
                  (("gate", ga), ("up", ua), ("down", da))}
        if keep_f32_absmax:
            ga, ua, da = (nested[n].resolve() for n in ("gate", "up", "down"))
        else:
            ga = ua = da = None
    return SyntheticLayer(
        H=H, I=I, R=R, qbs=qbs, seed=seed, nested=nested,
        gate_packed=gp, gate_absmax=ga, up_packed=upk, up_absmax=ua, down_packed=dp, down_absmax=da,
        enc_w=synth_normal_f16(sub_seed(seed, "enc_w"), (R, H), std, device),
        enc_b=synth_normal_f16(sub_seed(seed, "enc_b"), (R,), std, device),
        score_w=synth_normal_f16(sub_seed(seed, "score_w"), (NB, R), std, device),
        score_b=synth_normal_f16(sub_seed(seed, "score_b"), (NB,), std, device),
        x=synth_normal_f16(sub_seed(seed, "x"), (H,), 1.0, device),
    )
