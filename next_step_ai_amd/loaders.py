"""On-disk formats into device slot tables and routers.

* **bitsandbytes NF4 safetensors** (what the reference's ``SafetensorLoader``
  reads, runtime/safetensor_loader.py:85-102 and :391-472).  A parameter
  ``<name>.weight`` holds the packed nibbles (``[(n + 1) // 2, 1]`` u8, even
  element in the high nibble); its quant state sits beside it:
  ``<name>.weight.absmax``, ``.quant_map`` ([16] f32) and, with double
  quantisation, ``.nested_absmax`` (f32) and ``.nested_quant_map`` ([256]
  f32), plus one ``.quant_state.bitsandbytes__nf4`` u8 tensor holding a JSON
  object (``quant_type``, ``blocksize``, ``dtype``, ``shape`` and, when
  nested, ``nested_blocksize``, ``nested_dtype``, ``nested_offset``).  This is
  bitsandbytes' published serialisation of its quant state, restated here
  because bitsandbytes is not a dependency; the reference resolves the
  nested absmax to fp32 (safetensor_loader.py:403-406), these loaders keep
  the u8 codes for the kernels to resolve.
* **the learned-basis routing artifact** (a ``torch.save`` dict, read at
  RT:779-991), loaded with ``torch.load(weights_only=True)``: nothing in the
  file is executed.  The reference loads it with ``weights_only=False``; a
  file that needs that is refused here.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import torch

from .layout import (MlpBlockBankLayout, build_intermediate_mlp_block_bank_layout,
                     validate_intermediate_mlp_block_bank_params)
from .nested_absmax import NestedAbsmax
from .slot_table import BLOCK, SparseMlpRouter, SparseMlpSlotTable

_QS_PREFIX = "quant_state.bitsandbytes__"


class SafetensorShards:
    """Read access to a safetensors checkpoint: a directory with
    ``model.safetensors.index.json`` (its ``weight_map``) or ``*.safetensors``
    files, or a single file.  Tensors are read on the CPU."""

    def __init__(self, path: str | os.PathLike):
        from safetensors import safe_open  # noqa: F401  (fails early when absent)

        path = os.fspath(path)
        self.weight_map: dict[str, str] = {}
        if os.path.isdir(path):
            self.root = path
            index = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index, encoding="utf-8") as f:
                    self.weight_map = {str(k): str(v) for k, v in json.load(f).get("weight_map", {}).items()}
            else:
                files = sorted(n for n in os.listdir(path) if n.endswith(".safetensors"))
                if not files:
                    raise RuntimeError(f"No safetensors shards found in {path}")
                for fn in files:
                    for name in self._keys(os.path.join(path, fn)):
                        self.weight_map[name] = fn
        else:
            self.root = os.path.dirname(path) or "."
            for name in self._keys(path):
                self.weight_map[name] = os.path.basename(path)
        # quant-state entries grouped by their parameter (RT's rule: the
        # name up to and including ".weight")
        self.aux: dict[str, list[str]] = {}
        for name in self.weight_map:
            if ".weight." in name:
                base = name.split(".weight.", 1)[0] + ".weight"
                self.aux.setdefault(base, []).append(name)

    @staticmethod
    def _keys(file: str) -> list[str]:
        from safetensors import safe_open

        with safe_open(file, framework="pt", device="cpu") as h:
            return [str(k) for k in h.keys()]

    def names(self) -> list[str]:
        return sorted(self.weight_map)

    def get(self, names: list[str]) -> dict[str, torch.Tensor]:
        from safetensors import safe_open

        by_file: dict[str, list[str]] = {}
        for n in names:
            if n not in self.weight_map:
                raise KeyError(f"Tensor '{n}' not found in safetensors index")
            by_file.setdefault(self.weight_map[n], []).append(n)
        out = {}
        for fn, keys in by_file.items():
            with safe_open(os.path.join(self.root, fn), framework="pt", device="cpu") as h:
                for k in keys:
                    out[k] = h.get_tensor(k)
        return out


@dataclass
class Nf4Param:
    """One NF4 weight as stored: packed bytes (flat), absmax (fp32, or the
    nested state), the 16-entry code book, the quant block size and the
    [out, in] shape."""

    packed: torch.Tensor
    absmax: torch.Tensor | NestedAbsmax
    code: torch.Tensor
    blocksize: int
    shape: tuple[int, int]
    dtype: str

    @property
    def nested(self) -> bool:
        return isinstance(self.absmax, NestedAbsmax)


def _unpack_quant_state(blob: torch.Tensor) -> dict:
    try:
        return json.loads(bytes(blob.reshape(-1).to(torch.uint8).tolist()).decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise RuntimeError(f"unreadable bitsandbytes quant state: {e}") from None


def load_nf4_param(shards: SafetensorShards, name: str) -> Nf4Param:
    """The packed weight ``name`` (ending in ``.weight``) and its quant state."""
    aux_names = shards.aux.get(name, [])
    t = shards.get([name, *aux_names])
    weight = t.pop(name)
    if not aux_names:
        raise RuntimeError(f"'{name}' has no bitsandbytes quant state (not a 4-bit weight)")
    qs = {k.split(".weight.", 1)[1]: v for k, v in t.items()}
    blobs = [k for k in qs if k.startswith(_QS_PREFIX)]
    if len(blobs) != 1:
        raise RuntimeError(f"'{name}': expected one '{_QS_PREFIX}*' entry, found {sorted(blobs)}")
    meta = _unpack_quant_state(qs.pop(blobs[0]))
    qtype = str(meta.get("quant_type", blobs[0][len(_QS_PREFIX):]))
    if qtype != "nf4":
        raise RuntimeError(f"'{name}': quant_type '{qtype}' is not supported (NF4 only)")
    for key in ("absmax", "quant_map"):
        if key not in qs:
            raise RuntimeError(f"'{name}': quant state is missing '{key}'")
    shape = meta.get("shape")
    if not isinstance(shape, (list, tuple)) or len(shape) != 2:
        raise RuntimeError(f"'{name}': expected a 2-D shape in the quant state, got {shape}")
    out_f, in_f = int(shape[0]), int(shape[1])
    n = out_f * in_f
    packed = weight.reshape(-1)
    if packed.dtype != torch.uint8 or int(packed.numel()) != (n + 1) // 2:
        raise RuntimeError(f"'{name}': packed weight has {int(packed.numel())} {packed.dtype} values, "
                           f"expected {(n + 1) // 2} uint8 for shape {shape}")
    bs = int(meta["blocksize"])
    n_abs = (n + bs - 1) // bs
    code = qs["quant_map"].to(torch.float32).reshape(-1)
    if int(code.numel()) != 16:
        raise RuntimeError(f"'{name}': quant_map has {int(code.numel())} entries, expected 16")
    absmax = qs["absmax"].reshape(-1)
    if int(absmax.numel()) != n_abs:
        raise RuntimeError(f"'{name}': absmax has {int(absmax.numel())} entries, expected {n_abs}")
    if "nested_absmax" in qs:
        for key in ("nested_quant_map",):
            if key not in qs:
                raise RuntimeError(f"'{name}': nested quant state is missing '{key}'")
        nbs = int(meta["nested_blocksize"])
        a2 = qs["nested_absmax"].to(torch.float32).reshape(-1)
        if int(a2.numel()) != (n_abs + nbs - 1) // nbs:
            raise RuntimeError(f"'{name}': nested_absmax has {int(a2.numel())} entries, expected "
                               f"{(n_abs + nbs - 1) // nbs}")
        if absmax.dtype != torch.uint8:
            raise RuntimeError(f"'{name}': a nested absmax must be uint8 codes, got {absmax.dtype}")
        am = NestedAbsmax(q=absmax, absmax2=a2, code2=qs["nested_quant_map"].to(torch.float32).reshape(-1),
                          offset=float(meta["nested_offset"]), blocksize=nbs)
    else:
        am = absmax.to(torch.float32)
    return Nf4Param(packed=packed, absmax=am, code=code, blocksize=bs, shape=(out_f, in_f),
                    dtype=str(meta.get("dtype", "float16")))


def write_nf4_safetensors(path: str | os.PathLike, params: dict[str, Nf4Param]) -> None:
    """Write NF4 parameters in the same layout (one file).  Each entry of
    ``params`` is keyed by its ``.weight`` name."""
    from safetensors.torch import save_file

    out: dict[str, torch.Tensor] = {}

    def own(t: torch.Tensor) -> torch.Tensor:
        # a tensor the caller passes for several parameters (one code book for
        # gate, up and down) is written once per key, as separate storage
        return t.clone() if any(t.data_ptr() == o.data_ptr() for o in out.values()) else t

    for name, p in params.items():
        meta = {"quant_type": "nf4", "blocksize": int(p.blocksize), "dtype": p.dtype, "shape": list(p.shape)}
        out[name] = own(p.packed.reshape(-1, 1).to("cpu", torch.uint8).contiguous())
        out[f"{name}.quant_map"] = own(p.code.to("cpu", torch.float32).contiguous())
        if p.nested:
            a = p.absmax
            out[f"{name}.absmax"] = own(a.q.reshape(-1).to("cpu", torch.uint8).contiguous())
            out[f"{name}.nested_absmax"] = own(a.absmax2.to("cpu", torch.float32).contiguous())
            out[f"{name}.nested_quant_map"] = own(a.code2.to("cpu", torch.float32).contiguous())
            meta.update({"nested_blocksize": int(a.blocksize), "nested_dtype": "float32",
                         "nested_offset": float(a.offset)})
        else:
            out[f"{name}.absmax"] = own(p.absmax.reshape(-1).to("cpu", torch.float32).contiguous())
        out[f"{name}.{_QS_PREFIX}nf4"] = torch.tensor(list(json.dumps(meta).encode("utf-8")), dtype=torch.uint8)
    save_file(out, os.fspath(path))


def _to_device(p: Nf4Param, device: torch.device):
    packed = p.packed.to(device).contiguous()
    if p.nested:
        a = p.absmax
        am = NestedAbsmax(q=a.q.to(device).contiguous(), absmax2=a.absmax2.to(device).contiguous(),
                          code2=a.code2.to(device).contiguous(), offset=a.offset, blocksize=a.blocksize)
    else:
        am = p.absmax.to(device).contiguous()
    return packed, am


def slot_table_from_safetensors(source: str | os.PathLike | SafetensorShards, layer_idx: int, *,
                                device: torch.device, prefix: str = "model.layers.{layer}.mlp.",
                                resident_blocks: torch.Tensor | None = None, host_copy: bool = False,
                                capacity: int | None = None,
                                block_bank_layout: MlpBlockBankLayout | None = None) -> SparseMlpSlotTable:
    """The slot table of one layer's gate/up/down NF4 weights, read from a
    bitsandbytes safetensors checkpoint straight into block-major device
    slots (double-quantised absmax stay u8 codes).  The checkpoint's shapes
    are validated against ``block_bank_layout`` (the routing dict's
    ``block_bank_layout``; default: the layout of the gate shape) as the
    runtime does before a sparse forward (RT:5171-5172)."""
    shards = source if isinstance(source, SafetensorShards) else SafetensorShards(source)
    pre = prefix.format(layer=int(layer_idx))
    g = load_nf4_param(shards, f"{pre}gate_proj.weight")
    u = load_nf4_param(shards, f"{pre}up_proj.weight")
    d = load_nf4_param(shards, f"{pre}down_proj.weight")
    I, H = g.shape
    layout = block_bank_layout if block_bank_layout is not None else build_intermediate_mlp_block_bank_layout(
        layer_idx=int(layer_idx), hidden_size=H, intermediate_size=I, block_size=BLOCK)
    features = {"gate_in_features": g.shape[1], "gate_out_features": g.shape[0], "up_in_features": u.shape[1],
                "up_out_features": u.shape[0], "down_in_features": d.shape[1], "down_out_features": d.shape[0]}
    validate_intermediate_mlp_block_bank_params(layout=layout, **features)
    H, I = int(layout.hidden_size), int(layout.intermediate_size)
    if len({g.blocksize, u.blocksize, d.blocksize}) != 1:
        raise RuntimeError(f"layer {layer_idx}: quant block sizes differ ({g.blocksize}, {u.blocksize}, "
                           f"{d.blocksize})")
    if not (torch.equal(g.code, u.code) and torch.equal(g.code, d.code)):
        raise RuntimeError(f"layer {layer_idx}: gate/up/down use different quant maps")
    if len({g.nested, u.nested, d.nested}) != 1:
        raise RuntimeError(f"layer {layer_idx}: gate/up/down mix nested and plain absmax")
    (gp, ga), (up, ua), (dp, da) = (_to_device(p, device) for p in (g, u, d))
    t = SparseMlpSlotTable.from_reference(gate_packed=gp, gate_absmax=ga, up_packed=up, up_absmax=ua,
                                          down_packed=dp, down_absmax=da, H=H, I=I, qbs=g.blocksize,
                                          resident_blocks=resident_blocks, host_copy=host_copy, capacity=capacity,
                                          layer_idx=int(layer_idx), block_bank_layout=layout, features=features)
    t.code = g.code.to(device)
    t.as_struct()
    return t


def _stat(state: dict, stats: dict, key: str, default: float) -> float:
    """A per-layer statistic from the layer state or the stats dict (as the
    reference reads rank_effective / explained_variance_ratio)."""
    v = state.get(key)
    if torch.is_tensor(v) and int(v.numel()) == 1:
        return float(v.item())
    if isinstance(v, (int, float)):
        return float(v)
    v = stats.get(key) if isinstance(stats, dict) else None
    if isinstance(v, (int, float)):
        return float(v)
    if torch.is_tensor(v) and int(v.numel()) == 1:
        return float(v.item())
    return float(default)


def load_routing_artifact(path: str | os.PathLike, *, hidden_size: int, intermediate_size: int,
                          sparse_top_k: int | None = None, sparse_basis_top_k: int | None = None,
                          device: torch.device | None = None, dtype: torch.dtype = torch.float16) -> dict[int, dict]:
    """Per-layer routing dicts of an intermediate-block router artifact, as
    RT:779-991 builds them (keys ``enc_w``, ``enc_b``, ``route_score_weight``,
    ``route_score_bias``, ``down_block_norm``, ``dec_norm_t``, ``top_k``,
    ``basis_top_k``, ``num_blocks``, ``block_size`` ...).  Layers of the
    output-reconstruction domain belong to another sparse mode and are
    skipped.  The file is read with ``weights_only=True``."""
    try:
        payload = torch.load(os.fspath(path), map_location="cpu", weights_only=True)
    except Exception as e:  # a file that needs code execution to load is refused
        raise RuntimeError(f"routing artifact {os.fspath(path)} cannot be loaded safely: {e}") from None
    if not isinstance(payload, dict):
        raise RuntimeError("routing artifact must be a dict")
    cfg = payload.get("config", {}) or {}
    block_size = int(cfg.get("block_size", 32))
    target_default = str(cfg.get("artifact_target", "output_reconstruction")).strip().lower()
    domain_default = str(cfg.get("block_domain", "intermediate" if target_default == "intermediate_block_scores"
                                 else "output")).strip().lower()
    default_nb = (int(hidden_size) if domain_default == "output" else int(intermediate_size)) // max(block_size, 1)
    num_blocks = int(cfg.get("num_blocks", default_nb))
    top_k_default = int(sparse_top_k) if sparse_top_k is not None else max(1, int(round(max(1, num_blocks) * 0.02)))
    top_k_by_layer = cfg.get("top_k_by_layer", {}) or {}
    btk_by_layer = cfg.get("basis_top_k_by_layer", {}) or {}
    btk_default = int(sparse_basis_top_k) if sparse_basis_top_k is not None else int(cfg.get("basis_top_k", 64))
    stats = payload.get("stats", {}) or {}
    dev = device if device is not None else torch.device("cpu")
    out: dict[int, dict] = {}
    for lidx_s, state in (payload.get("layer_states", {}) or {}).items():
        lidx = int(lidx_s)
        lstats = stats.get(str(lidx), {}) if isinstance(stats, dict) else {}
        target = str(state.get("artifact_target", cfg.get("artifact_target", target_default))).strip().lower()
        domain = str(state.get("block_domain", cfg.get(
            "block_domain", "intermediate" if target == "intermediate_block_scores" else domain_default))).strip().lower()
        if domain != "intermediate":
            continue
        enc_w = state["encoder_weight"].to(device=dev, dtype=dtype).contiguous()
        enc_b = state["encoder_bias"].to(device=dev, dtype=dtype).contiguous()
        rank = int(enc_w.shape[0])
        if int(enc_w.shape[1]) != int(hidden_size):
            raise RuntimeError(f"Sparse intermediate-router layer {lidx}: encoder_weight has input dim "
                               f"{int(enc_w.shape[1])}, expected hidden_size={int(hidden_size)}.")
        rank_eff = int(max(1, min(int(_stat(state, lstats, "rank_effective", rank)), rank)))
        sw = state.get("score_weight")
        if not torch.is_tensor(sw):
            raise RuntimeError(f"Sparse intermediate-router layer {lidx} is missing score_weight.")
        sw = sw.to(device=dev, dtype=dtype).contiguous()
        if int(sw.ndim) != 2 or int(sw.shape[1]) != rank:
            raise RuntimeError(f"Sparse intermediate-router layer {lidx}: score_weight shape {tuple(sw.shape)} "
                               f"does not match basis_rank={rank}.")
        nb = int(sw.shape[0])
        if nb != int(intermediate_size) // block_size:
            raise RuntimeError(f"Sparse intermediate-router layer {lidx} stores {nb} FFN blocks, expected "
                               f"{int(intermediate_size) // block_size}.")
        sb = state.get("score_bias")
        if torch.is_tensor(sb):
            sb = sb.to(device=dev, dtype=dtype).contiguous().view(-1)
            if int(sb.numel()) != nb:
                raise RuntimeError(f"Sparse intermediate-router layer {lidx}: score_bias has {int(sb.numel())} "
                                   f"values, expected {nb}.")
        else:
            sb = None
        dbn = state.get("down_block_norm")
        if torch.is_tensor(dbn):
            dbn = dbn.to(dtype=torch.float32).contiguous().view(-1)
            if int(dbn.numel()) != nb:
                raise RuntimeError(f"Sparse intermediate-router layer {lidx}: down_block_norm has "
                                   f"{int(dbn.numel())} values, expected {nb}.")
        else:
            dbn = None
        k = int(top_k_by_layer.get(str(lidx), top_k_by_layer.get(lidx, top_k_default)))
        k = int(max(1, min(k, nb)))
        btk = int(sparse_basis_top_k if sparse_basis_top_k is not None
                  else btk_by_layer.get(str(lidx), btk_by_layer.get(lidx, btk_default)))
        btk = int(max(1, min(btk, rank_eff)))
        scale = state.get("scale")
        out[lidx] = {
            "enc_w": enc_w, "enc_b": enc_b, "dec": None, "dec_bias": None,
            "dec_norm_t": sw.transpose(0, 1).abs().contiguous(),
            "route_score_weight": sw, "route_score_bias": sb,
            "down_block_norm": dbn, "down_block_norm_ready": dbn is not None,
            "scale": float(scale.item()) if torch.is_tensor(scale) and int(scale.numel()) == 1 else 1.0,
            "top_k": k, "basis_top_k": btk, "basis_rank": rank, "rank_effective": rank_eff,
            "artifact_target": target, "block_domain": domain, "block_size": block_size, "num_blocks": nb,
            "explained_variance_ratio": _stat(state, lstats, "explained_variance_ratio", 1.0),
            # the layer's block bank, which the sparse forward validates the projections against (RT:906-912)
            "block_bank_layout": build_intermediate_mlp_block_bank_layout(
                layer_idx=lidx, hidden_size=int(hidden_size), intermediate_size=int(intermediate_size),
                block_size=block_size, num_blocks=nb),
        }
    return out


def router_from_routing(routing: dict, device: torch.device) -> SparseMlpRouter:
    """A device router of one layer's routing dict."""
    return SparseMlpRouter(enc_w=routing["enc_w"].to(device), enc_b=routing.get("enc_b"),
                           score_w=routing["route_score_weight"].to(device), score_b=routing.get("route_score_bias"),
                           basis_top_k=routing.get("basis_top_k"), down_block_norm=routing.get("down_block_norm"))
