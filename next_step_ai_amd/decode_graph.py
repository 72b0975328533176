"""Graph-captured decode: the per-layer MLP launches of one decode token, or
the whole stack of layers, recorded once into a HIP graph and replayed per
token.

The reference launches each layer's routed MLP from Python every token
(``_mlp_forward_dispatch``, RT:5833-5923, from the decode loop at
RT:7740-7795).  Here a layer's launches (latent, scores, gate/up with the
top-k inside, down; plus the hot-cache promotion when the layer has a cache)
are captured with their device buffers fixed: the input is copied into the
graph's input buffer, the graph is replayed on the current stream, and the
output and selection are read from the graph's buffers.  None of the
captured kernels allocates, frees, synchronises or clears memory with a
memset node; the workspaces' counter regions return to zero at the end of
every kernel that uses them, so each replay starts from the state the
capture saw.
"""
from __future__ import annotations

import torch

from ._runtime import require_device, workspace
from .slot_table import SparseMlpLayer

__all__ = ["LayerGraph", "StackGraph"]


class LayerGraph:
    """One layer's decode MLP as a replayable graph (the per-layer launch of
    the decode loop).  ``run(x)`` returns (out [H] fp16, sel [k] int32); both
    are the graph's own buffers, overwritten by the next ``run``."""

    def __init__(self, layer: SparseMlpLayer, *, warmup: int = 1):
        self.layer = layer
        self.device = layer.device
        H = layer.table.H
        self.x = torch.zeros(H, dtype=torch.float16, device=self.device)
        self.out = torch.empty(H, dtype=torch.float16, device=self.device)
        self.sel = torch.empty(layer.top_k, dtype=torch.int32, device=self.device)
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.ws = workspace(layer.workspace_bytes(), self.device)
            for _ in range(max(1, int(warmup))):  # kernel attributes set, workspaces allocated
                layer.forward(self.x, out=self.out, sel_out=self.sel, ws=self.ws)
        torch.cuda.current_stream(self.device).wait_stream(side)
        with torch.cuda.graph(self.graph, stream=side):
            layer.forward(self.x, out=self.out, sel_out=self.sel, ws=self.ws)

    def run(self, x: torch.Tensor):
        require_device(x, "x")
        self.x.copy_(x.reshape(-1))
        self.graph.replay()
        return self.out, self.sel


class StackGraph:
    """One decode token through a stack of layers, x <- x + mlp_l(x), as one
    graph.  ``run(x)`` returns the final hidden state [H] fp16 (the graph's
    buffer); ``sels[l]`` holds layer l's selection after the replay."""

    def __init__(self, layers: list[SparseMlpLayer], *, warmup: int = 1):
        if not layers:
            raise RuntimeError("StackGraph needs at least one layer")
        self.layers = layers
        self.device = layers[0].device
        H = layers[0].table.H
        if any(m.table.H != H or m.device != self.device for m in layers):
            raise RuntimeError("every layer of a stack must have the same hidden size and device")
        self.x = torch.zeros(H, dtype=torch.float16, device=self.device)
        self.bufs = [torch.empty(H, dtype=torch.float16, device=self.device) for _ in range(2)]
        self.sels = [torch.empty(m.top_k, dtype=torch.int32, device=self.device) for m in layers]
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.ws = workspace(max(m.workspace_bytes() for m in layers), self.device)
            for _ in range(max(1, int(warmup))):
                self._token()
        torch.cuda.current_stream(self.device).wait_stream(side)
        with torch.cuda.graph(self.graph, stream=side):
            self._token()
        self.result = self._last

    def _token(self):
        x = self.x
        for i, m in enumerate(self.layers):
            y = self.bufs[i % 2]
            # y = x + mlp(x): the residual add of the decode loop, fused into the down kernel
            m.forward(x, out=y, sel_out=self.sels[i], ws=self.ws, residual=x)
            x = y
        self._last = x

    def run(self, x: torch.Tensor) -> torch.Tensor:
        require_device(x, "x")
        self.x.copy_(x.reshape(-1))
        self.graph.replay()
        return self.result
