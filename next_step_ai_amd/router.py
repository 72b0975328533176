"""Learned-basis router (RT:4209-4238 latent, RT:4311-4352 route) on the GPU.

``route_sparse_mlp(hidden, routing)`` consumes the runtime's per-layer
routing dict (keys built at RT:956-979: ``enc_w``, ``enc_b``,
``route_score_weight``, ``route_score_bias``, ``down_block_norm``,
``dec_norm_t``, ``top_k``, ``basis_top_k``) and returns the active blocks
``[N, k]`` int64 in ``torch.topk`` order.

Precision contract: every dot product (latent, score) is computed exactly
and rounded once to fp16, then clamped/scaled as in the reference; the k
largest scores are selected with ties broken by the lowest block index.
(``torch.topk`` leaves the order of equal scores unspecified.)
"""
from __future__ import annotations

import torch

from . import _lib
from ._runtime import as_f16, ptr, require_device, stream_handle, workspace


def _prepare(routing: dict, device: torch.device) -> dict:
    """Device fp16 copies of the routing tensors, cached in the dict."""
    cache = routing.get("_nsmlp_dev")
    if isinstance(cache, dict) and cache.get("device") == device:
        return cache
    enc_w = as_f16(routing["enc_w"], device)
    enc_b = routing.get("enc_b")
    sw = routing.get("route_score_weight")
    legacy = not torch.is_tensor(sw)
    if legacy:
        # RT:4332-4334: scores = |latent| @ dec_norm_t, dec_norm_t [R, NB]
        score_w = as_f16(routing["dec_norm_t"].transpose(0, 1), device)
        score_b = None
    else:
        score_w = as_f16(sw, device)
        sb = routing.get("route_score_bias")
        score_b = as_f16(sb.reshape(-1), device) if torch.is_tensor(sb) else None
    dbn = routing.get("down_block_norm")
    NB = int(score_w.shape[0])
    dbn16 = None
    if torch.is_tensor(dbn) and int(dbn.numel()) == NB:
        # RT:4335-4337: down_block_norm (fp32) is cast to the score dtype
        dbn16 = dbn.reshape(-1).to(dtype=torch.float16).to(device)
    cache = {
        "device": device,
        "enc_w": enc_w,
        "enc_b": as_f16(enc_b.reshape(-1), device) if torch.is_tensor(enc_b) else None,
        "score_w": score_w,
        "score_b": score_b,
        "dbn": dbn16,
        "legacy": legacy,
        "R": int(enc_w.shape[0]),
        "NB": NB,
    }
    routing["_nsmlp_dev"] = cache
    return cache


def route_tokens(x: torch.Tensor, routing: dict, k: int, *, sorted_by_score: bool = True,
                 basis_top_k: int | None = None, return_scores: bool = False):
    """Route ``x [N, H]`` (fp16) and return ``sel [N, k]`` int32 (plus the
    fp16 latent ``[N, R]`` and scores ``[N, NB]`` when ``return_scores``)."""
    device = require_device(x, "hidden")
    c = _prepare(routing, device)
    x16 = as_f16(x, device)
    N, H = int(x16.shape[0]), int(x16.shape[1])
    R, NB = c["R"], c["NB"]
    if int(c["enc_w"].shape[1]) != H:
        raise RuntimeError(f"encoder_weight has input dim {int(c['enc_w'].shape[1])}, expected hidden_size={H}")
    kk = max(1, min(int(k), NB))
    btk = int(routing.get("basis_top_k", R) if basis_top_k is None else basis_top_k)
    btk = max(1, min(btk, R))
    flags = (_lib.NSMLP_ROUTE_SORTED if sorted_by_score else 0) | (_lib.NSMLP_ROUTE_LEGACY_ABS if c["legacy"] else 0)
    sel = torch.empty((N, kk), dtype=torch.int32, device=device)
    lat = torch.empty((N, R), dtype=torch.float16, device=device) if return_scores else None
    sc = torch.empty((N, NB), dtype=torch.float16, device=device) if return_scores else None
    nbytes = int(_lib.lib().nsmlp_route_workspace_bytes(N, H, R, NB, kk))
    ws = workspace(nbytes, device)
    _lib.call(
        "nsmlp_route_f16", ptr(x16), N, H, ptr(c["enc_w"]), ptr(c["enc_b"]), R, btk, ptr(c["score_w"]),
        ptr(c["score_b"]), ptr(c["dbn"]), NB, flags, kk, ptr(sel), ptr(lat), ptr(sc), ptr(ws), ws.numel(),
        stream_handle(device),
    )
    if return_scores:
        return sel, lat, sc
    return sel


def route_sparse_mlp(hidden: torch.Tensor, routing: dict | None, *, top_k: int | None = None) -> torch.Tensor | None:
    """Counterpart of ``StreamingLlamaRuntime._route_sparse_mlp`` (RT:4311-4352):
    ``hidden`` [B, T, H] (or [N, H]) -> active blocks ``[B*T, k]`` int64, or
    ``None`` when the layer has no routing state."""
    if routing is None:
        return None
    flat = hidden.reshape(-1, hidden.shape[-1])
    c = _prepare(routing, require_device(flat, "hidden"))
    k = int(routing.get("top_k", c["NB"]) if top_k is None else top_k)
    k = max(1, min(k, c["NB"]))
    return route_tokens(flat, routing, k, sorted_by_score=True).to(torch.int64)
