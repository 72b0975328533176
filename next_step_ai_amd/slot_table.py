"""HBM hot-block slot table and the one-call decode layer.

The reference keeps a per-projection "VRAM hot cache" (RT:2619-2786): a CPU
``lookup_cpu`` (block -> slot or -1), slot storage for the hot blocks, and a
host path that gathers, copies and merges the cold ones every token
(RT:3588-3702, RT:3885-4207, RT:4455-4578).  Here the table lives on the
device and is read by the decode kernels directly:

* ``lookup`` [NB] int32 on the device (block -> slot, -1 = host-resident);
* gate/up slots [n_slots, 32, H/2] u8 + absmax [n_slots, 32, H/qbs] f32
  (the reference's gate/up row blocks are already contiguous: RT:4627-4660);
* down slots block-major [n_slots, H, 16] u8 + absmax [n_slots, H] f32 (the
  reference's [H, n, 16] column gather, RT:4491-4511, transposed so that a
  block's column is one contiguous 256 KB stream at the 405B shape);
* optional pinned host copy of every block in the same layout; misses are
  read by the kernels over the host link, without a host round trip;
* absmax either fp32 or double-quantised (``NestedAbsmax``: u8 codes in the
  same positions, resolved by the kernels; RT:4621-4625).

Misses are promoted into slots on the device (``HotBlockCache``) with the
reference's fixed-capacity slot plan (RT:2576-2617): free slots first, then
the lowest-score slot.  A block is hot iff its lookup entry is >= 0
(RT:3588-3604); the kernels resolve that per block as they read it.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._runtime import BlockCounts, StatusWord, nf4_code, ptr, require_device, stream_handle, workspace
from .layout import (MlpBlockBankLayout, build_intermediate_mlp_block_bank_layout,
                     validate_intermediate_mlp_block_bank_params)
from .nested_absmax import NestedAbsmax

BLOCK = 32


def gather_row_blocks(packed: torch.Tensor | None, absmax: torch.Tensor, blocks: torch.Tensor, in_features: int,
                      qbs: int) -> tuple[torch.Tensor | None, torch.Tensor]:
    """Device gather of gate/up row blocks (RT:4530-4578 semantics):
    returns [n, 32*in/2] u8 and [n, 32*in/qbs] f32 absmax, or, for the u8
    codes of a double-quantised absmax, [n, 16, in/qbs, 2] (rows 2p and 2p+1
    interleaved, the slot layout).  With u8 codes ``packed`` may be None
    (codes only)."""
    device = require_device(absmax, "absmax")
    b = blocks.to(device=device, dtype=torch.int32).contiguous()
    n = int(b.numel())
    q8 = absmax.dtype == torch.uint8
    A = int(in_features) // int(qbs)
    src_blocks = int(absmax.numel()) // (BLOCK * A)
    if packed is None and not q8:
        raise RuntimeError("packed is required with fp32 absmax")
    out_p = None if packed is None else torch.empty((n, BLOCK * int(in_features) // 2), dtype=torch.uint8,
                                                    device=device)
    if q8:
        out_a = torch.empty((n, BLOCK // 2, A, 2), dtype=torch.uint8, device=device)
        _lib.call("nsmlp_gather_row_blocks_q8", ptr(packed), ptr(absmax), src_blocks, ptr(b), n, int(in_features),
                  int(qbs), ptr(out_p), ptr(out_a), stream_handle(device))
    else:
        out_a = torch.empty((n, BLOCK * A), dtype=torch.float32, device=device)
        _lib.call("nsmlp_gather_row_blocks", ptr(packed), ptr(absmax), src_blocks, ptr(b), n, int(in_features),
                  int(qbs), ptr(out_p), ptr(out_a), stream_handle(device))
    return out_p, out_a


def gather_down_columns(packed: torch.Tensor, absmax: torch.Tensor, blocks: torch.Tensor, out_features: int,
                        in_features: int, qbs: int, *, block_major: bool = True):
    """Device gather of down-proj column blocks (RT:4455-4528 semantics):
    block b = bytes [o, 16b:16b+16) and absmax [o, (32b)//qbs] of the
    row-major weight.  block_major -> [n, H, 16] / [n, H]; else the
    reference's [H, n, 16] / [H, n]."""
    device = require_device(packed, "packed")
    b = blocks.to(device=device, dtype=torch.int32).contiguous()
    n = int(b.numel())
    H = int(out_features)
    q8 = absmax.dtype == torch.uint8
    adt = torch.uint8 if q8 else torch.float32
    if block_major:
        out_p = torch.empty((n, H, 16), dtype=torch.uint8, device=device)
        out_a = torch.empty((n, H), dtype=adt, device=device)
        layout = _lib.NSMLP_DOWN_BLOCK_MAJOR
    else:
        out_p = torch.empty((H, n, 16), dtype=torch.uint8, device=device)
        out_a = torch.empty((H, n), dtype=adt, device=device)
        layout = _lib.NSMLP_DOWN_GATHERED
    _lib.call("nsmlp_gather_down_columns_q8" if q8 else "nsmlp_gather_down_columns", ptr(packed), ptr(absmax),
              ptr(b), n, H, int(in_features), int(qbs), layout, ptr(out_p), ptr(out_a), stream_handle(device))
    return out_p, out_a


def _host_dev_ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    out = ctypes.c_void_p()
    _lib.call("nsmlp_host_device_pointer", ctypes.c_void_p(t.data_ptr()), ctypes.byref(out))
    return int(out.value) if out.value is not None else None


def _check_bank(layer_idx, layout, features, H, I, qbs, gp, ga, upk, ua, dp, da) -> None:
    """Block-bank validation of a layer's reference-layout NF4 tensors."""
    if layout is None:
        layout = build_intermediate_mlp_block_bank_layout(layer_idx=layer_idx, hidden_size=H, intermediate_size=I,
                                                          block_size=BLOCK)
    if (int(layout.hidden_size), int(layout.intermediate_size), int(layout.block_size)) != (H, I, BLOCK):
        raise RuntimeError(f"layer {int(layout.layer_idx)}: the block bank is {int(layout.hidden_size)} x "
                           f"{int(layout.intermediate_size)} in blocks of {int(layout.block_size)}, the table "
                           f"{H} x {I} in blocks of {BLOCK}")

    def out_of(packed, in_f):  # out features implied by a packed [out, in] NF4 weight (-1: not whole rows)
        n2 = 2 * int(packed.numel())
        return n2 // in_f if n2 % in_f == 0 else -1

    if features is None:
        features = {"gate_in_features": H, "gate_out_features": out_of(gp, H), "up_in_features": H,
                    "up_out_features": out_of(upk, H), "down_in_features": I, "down_out_features": out_of(dp, I)}
    validate_intermediate_mlp_block_bank_params(layout=layout, **features)
    for name, p, a in (("gate", gp, ga), ("up", upk, ua), ("down", dp, da)):
        if int(p.numel()) * 2 != H * I:
            raise RuntimeError(f"layer {int(layout.layer_idx)}: {name} packed has {int(p.numel())} bytes, "
                               f"expected {H * I // 2}")
        n_abs = int((a.q if isinstance(a, NestedAbsmax) else a).numel())
        if n_abs != H * I // qbs:
            raise RuntimeError(f"layer {int(layout.layer_idx)}: {name} absmax has {n_abs} entries, expected "
                               f"{H * I // qbs} (one per {qbs} weights)")


class SparseMlpSlotTable:
    """Device slot table of one layer's gate/up/down NF4 blocks."""

    def __init__(self, *, H: int, I: int, qbs: int, device: torch.device):
        if int(I) % BLOCK != 0:
            raise RuntimeError(f"intermediate_size={int(I)} is not divisible by block_size={BLOCK}")
        self.H, self.I, self.qbs = int(H), int(I), int(qbs)
        self.NB = self.I // BLOCK
        self.device = device
        self.lookup: torch.Tensor | None = None
        self.block_ids: torch.Tensor | None = None
        self.gate_packed = self.gate_absmax = self.up_packed = self.up_absmax = None
        self.down_packed = self.down_absmax = None
        # double-quantised absmax: *_absmax hold the u8 codes; second-level
        # state per projection
        self.nested: dict[str, NestedAbsmax] | None = None
        self.host: dict[str, torch.Tensor] = {}
        self.down_bias: torch.Tensor | None = None
        self.code = nf4_code(device)
        self._struct: _lib.SlotTable | None = None

    @property
    def n_slots(self) -> int:
        return 0 if self.gate_packed is None else int(self.gate_packed.shape[0])

    @classmethod
    def from_reference(cls, *, gate_packed: torch.Tensor, gate_absmax, up_packed: torch.Tensor, up_absmax,
                       down_packed: torch.Tensor, down_absmax, H: int, I: int, qbs: int = 64,
                       resident_blocks: torch.Tensor | None = None, host_copy: bool = False,
                       capacity: int | None = None, layer_idx: int = 0,
                       block_bank_layout: MlpBlockBankLayout | None = None,
                       features: dict[str, int] | None = None) -> "SparseMlpSlotTable":
        """Build from the reference layouts on the device: gate/up ``[I*H/2]``
        u8 + ``[I*H/qbs]`` absmax, down ``[H*I/2]`` u8 + ``[H*I/qbs]`` absmax.
        The absmax are fp32 tensors, or all three ``NestedAbsmax`` (the
        double-quantised state, kept as u8 codes).  ``resident_blocks``
        (default: all) go to HBM slots in the given order; with ``host_copy``
        every block is also kept in pinned host memory and non-resident
        blocks are served from there.  ``capacity`` (>= the resident count)
        adds empty slots after the resident ones, for promotions.

        The projections are checked against the layer's block bank first, as
        the runtime does before a sparse forward (RT:5171-5172): against
        ``block_bank_layout`` (the routing dict's, RT:906-912) or the layout
        of (H, I, 32-row blocks), with the (in, out) features of each
        projection from ``features`` (keys gate_in_features ... as
        ``validate_intermediate_mlp_block_bank_params`` takes them; e.g. the
        checkpoint's shapes) or else implied by the packed sizes."""
        device = require_device(gate_packed, "gate_packed")
        _check_bank(layer_idx, block_bank_layout, features, int(H), int(I), int(qbs), gate_packed, gate_absmax,
                    up_packed, up_absmax, down_packed, down_absmax)
        t = cls(H=H, I=I, qbs=qbs, device=device)
        nested = [isinstance(x, NestedAbsmax) for x in (gate_absmax, up_absmax, down_absmax)]
        if any(nested):
            if not all(nested):
                raise RuntimeError("gate, up and down absmax must all be fp32 or all NestedAbsmax")
            bs = {int(x.blocksize) for x in (gate_absmax, up_absmax, down_absmax)}
            if len(bs) != 1:
                raise RuntimeError(f"nested absmax block sizes differ: {sorted(bs)}")
            t.nested = {"gate": gate_absmax, "up": up_absmax, "down": down_absmax}
            gate_absmax, up_absmax, down_absmax = gate_absmax.q, up_absmax.q, down_absmax.q
        NB = t.NB
        all_blocks = torch.arange(NB, dtype=torch.int32, device=device)
        if resident_blocks is None:
            t.gate_packed = gate_packed.view(NB, BLOCK * H // 2)
            t.up_packed = up_packed.view(NB, BLOCK * H // 2)
            if t.nested is not None:  # codes in the interleaved slot layout
                t.gate_absmax = gather_row_blocks(None, gate_absmax, all_blocks, H, qbs)[1]
                t.up_absmax = gather_row_blocks(None, up_absmax, all_blocks, H, qbs)[1]
            else:
                t.gate_absmax = gate_absmax.view(NB, BLOCK * H // qbs)
                t.up_absmax = up_absmax.view(NB, BLOCK * H // qbs)
            t.down_packed, t.down_absmax = gather_down_columns(down_packed, down_absmax, all_blocks, H, I, qbs)
            t.lookup = None
            t.block_ids = all_blocks.to("cpu", torch.long)
        else:
            res = resident_blocks.to(device=device, dtype=torch.int32).contiguous()
            t.gate_packed, t.gate_absmax = gather_row_blocks(gate_packed, gate_absmax, res, H, qbs)
            t.up_packed, t.up_absmax = gather_row_blocks(up_packed, up_absmax, res, H, qbs)
            t.down_packed, t.down_absmax = gather_down_columns(down_packed, down_absmax, res, H, I, qbs)
            n_res = int(res.numel())
            if capacity is not None and int(capacity) > n_res:
                def grow(a):
                    g = torch.zeros((int(capacity),) + tuple(a.shape[1:]), dtype=a.dtype, device=device)
                    g[:n_res] = a
                    return g
                t.gate_packed, t.gate_absmax = grow(t.gate_packed), grow(t.gate_absmax)
                t.up_packed, t.up_absmax = grow(t.up_packed), grow(t.up_absmax)
                t.down_packed, t.down_absmax = grow(t.down_packed), grow(t.down_absmax)
            lookup = torch.full((NB,), -1, dtype=torch.int32)
            lookup[res.to("cpu", torch.long)] = torch.arange(int(res.numel()), dtype=torch.int32)
            t.lookup = lookup.to(device)
            t.block_ids = res.to("cpu", torch.long)
        if host_copy:
            dp, da = gather_down_columns(down_packed, down_absmax, all_blocks, H, I, qbs)
            if t.nested is not None:
                ga_h = gather_row_blocks(None, gate_absmax, all_blocks, H, qbs)[1]
                ua_h = gather_row_blocks(None, up_absmax, all_blocks, H, qbs)[1]
            else:
                ga_h, ua_h = gate_absmax.view(NB, -1), up_absmax.view(NB, -1)
            srcs = {
                "gate_packed": gate_packed.view(NB, -1), "gate_absmax": ga_h,
                "up_packed": up_packed.view(NB, -1), "up_absmax": ua_h,
                "down_packed": dp, "down_absmax": da,
            }
            for name, src in srcs.items():
                h = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
                h.copy_(src)
                t.host[name] = h
            del dp, da
        return t

    def lookup_cpu(self) -> torch.Tensor:
        """The reference's ``lookup_cpu`` view (block -> slot or -1)."""
        if self.lookup is None:
            return torch.arange(self.NB, dtype=torch.int32)
        return self.lookup.to("cpu")

    def as_struct(self) -> _lib.SlotTable:
        h = self.host
        st = _lib.SlotTable(
            H=self.H, I=self.I, qbs=self.qbs, n_slots=self.n_slots,
            lookup=ptr(self.lookup),
            gate_packed=ptr(self.gate_packed), gate_absmax=ptr(self.gate_absmax),
            up_packed=ptr(self.up_packed), up_absmax=ptr(self.up_absmax),
            down_packed=ptr(self.down_packed), down_absmax=ptr(self.down_absmax),
            host_gate_packed=_host_dev_ptr(h.get("gate_packed")), host_gate_absmax=_host_dev_ptr(h.get("gate_absmax")),
            host_up_packed=_host_dev_ptr(h.get("up_packed")), host_up_absmax=_host_dev_ptr(h.get("up_absmax")),
            host_down_packed=_host_dev_ptr(h.get("down_packed")),
            host_down_absmax=_host_dev_ptr(h.get("down_absmax")),
            code=ptr(self.code), down_bias=ptr(self.down_bias),
        )
        if self.nested is not None:
            # the u8 codes take the double-quantised fields; the fp32 ones stay NULL
            st.gate_qabsmax, st.up_qabsmax, st.down_qabsmax = st.gate_absmax, st.up_absmax, st.down_absmax
            st.host_gate_qabsmax, st.host_up_qabsmax = st.host_gate_absmax, st.host_up_absmax
            st.host_down_qabsmax = st.host_down_absmax
            st.gate_absmax = st.up_absmax = st.down_absmax = None
            st.host_gate_absmax = st.host_up_absmax = st.host_down_absmax = None
            g, u, d = self.nested["gate"], self.nested["up"], self.nested["down"]
            st.dq_block = int(g.blocksize)
            st.gate_absmax2, st.up_absmax2, st.down_absmax2 = ptr(g.absmax2), ptr(u.absmax2), ptr(d.absmax2)
            st.gate_code2, st.up_code2, st.down_code2 = ptr(g.code2), ptr(u.code2), ptr(d.code2)
            st.gate_offset, st.up_offset, st.down_offset = float(g.offset), float(u.offset), float(d.offset)
        self._struct = st
        return st

    def _status_for(self, ws: torch.Tensor, what: str, check: bool) -> StatusWord | None:
        """With ``check``: a status word for the call about to be enqueued on
        ``ws``, whose earlier bits (from unchecked calls sharing the
        workspace) are cleared first, so the check reports this call alone."""
        if not check:
            return None
        sw = StatusWord(self.device, what)
        sw.clear(ws)
        return sw

    @staticmethod
    def _checked(sw: StatusWord | None, ws: torch.Tensor) -> None:
        """Raise RuntimeError if the call just enqueued on ``ws`` reported a
        block it could not serve (waits for it)."""
        if sw is not None:
            sw.take(ws)
            sw.check()

    def decode(self, x: torch.Tensor, sel: torch.Tensor, out: torch.Tensor | None = None, *,
               check: bool = False) -> torch.Tensor:
        """One decode token over the selected block ids ``sel`` [k].  With
        ``check``, wait for it and raise RuntimeError if a selected block was
        out of range or neither resident nor host-copied (the reference's
        gather raises there, RT:4530-4578)."""
        x16 = x.reshape(-1).to(device=self.device, dtype=torch.float16).contiguous()
        s = sel.reshape(-1).to(device=self.device, dtype=torch.int32).contiguous()
        k = int(s.numel())
        if out is None:
            out = torch.empty(self.H, dtype=torch.float16, device=self.device)
        nbytes = int(_lib.lib().nsmlp_decode_workspace_bytes(self.H, k))
        ws = workspace(nbytes, self.device)
        st = self._struct if self._struct is not None else self.as_struct()
        sw = self._status_for(ws, "sparse MLP decode", check)
        _lib.call("nsmlp_decode_slots_f16", ctypes.byref(st), ptr(x16), ptr(s), k, ptr(out), ptr(ws), ws.numel(),
                  stream_handle(self.device))
        self._checked(sw, ws)
        return out


    def dense_mlp(self, x: torch.Tensor, out: torch.Tensor | None = None,
                  residual: torch.Tensor | None = None, *, check: bool = False) -> torch.Tensor:
        """The dense-guard prefill MLP (RT:5775-5831): every block for every
        token of ``x`` [M, H], as full-width MFMA GEMMs with the reference's
        rounding points (fp16 weights, g, silu(g), u, act); ``out`` [M, H]
        fp16, plus ``residual`` [M, H] when given (fused fp16 add)."""
        x16 = x.reshape(-1, self.H).to(device=self.device, dtype=torch.float16).contiguous()
        M = int(x16.shape[0])
        if out is None:
            out = torch.empty((M, self.H), dtype=torch.float16, device=self.device)
        r16 = None
        if residual is not None:
            r16 = residual.reshape(M, self.H)
            if r16.dtype != torch.float16 or r16.device != self.device or not r16.is_contiguous():
                raise RuntimeError("residual must be a contiguous fp16 [M, H] tensor on the table's device")
        nbytes = int(_lib.lib().nsmlp_dense_mlp_workspace_bytes(self.H, self.I, M))
        ws = workspace(nbytes, self.device)
        st = self._struct if self._struct is not None else self.as_struct()
        sw = self._status_for(ws, "dense-guard MLP", check)
        _lib.call("nsmlp_dense_mlp_slots_f16", ctypes.byref(st), ptr(x16), M, ptr(r16), ptr(out), ptr(ws), ws.numel(),
                  stream_handle(self.device))
        self._checked(sw, ws)
        return out

    def prefill(self, x: torch.Tensor, sel: torch.Tensor, out: torch.Tensor | None = None, *,
                check: bool = False) -> torch.Tensor:
        """M tokens ``x`` [M, H] with their own selected block ids ``sel``
        [M, k] (the multi-token branch, RT:4857-4908 + RT:5453): grouped MFMA
        gate/up/down over the union of the selected blocks; ``out`` [M, H] fp16.
        ``check``: as in ``decode`` (also reports a grouped down partial
        outside the fixed-point range)."""
        x16 = x.reshape(-1, self.H).to(device=self.device, dtype=torch.float16).contiguous()
        s = sel.to(device=self.device, dtype=torch.int32).contiguous()
        M, k = int(x16.shape[0]), int(s.shape[-1])
        if int(s.numel()) != M * k:
            raise RuntimeError(f"sel has {int(s.numel())} entries, expected M*k = {M}*{k}")
        if out is None:
            out = torch.empty((M, self.H), dtype=torch.float16, device=self.device)
        nbytes = int(_lib.lib().nsmlp_prefill_workspace_bytes(self.H, self.NB, M, k))
        ws = workspace(nbytes, self.device)
        st = self._struct if self._struct is not None else self.as_struct()
        sw = self._status_for(ws, "sparse MLP prefill", check)
        _lib.call("nsmlp_prefill_slots_f16", ctypes.byref(st), ptr(x16), M, ptr(s), k, ptr(out), ptr(ws), ws.numel(),
                  stream_handle(self.device))
        self._checked(sw, ws)
        return out


class SparseMlpRouter:
    """Device copy of one layer's router (fp16, as the runtime casts it, RT:850-891)."""

    def __init__(self, *, enc_w: torch.Tensor, enc_b: torch.Tensor | None, score_w: torch.Tensor,
                 score_b: torch.Tensor | None, basis_top_k: int | None = None,
                 down_block_norm: torch.Tensor | None = None, legacy_abs: bool = False):
        device = require_device(enc_w, "enc_w")
        self.device = device
        self.enc_w = enc_w.to(device=device, dtype=torch.float16).contiguous()
        self.enc_b = None if enc_b is None else enc_b.reshape(-1).to(device=device, dtype=torch.float16).contiguous()
        self.score_w = score_w.to(device=device, dtype=torch.float16).contiguous()
        self.score_b = None if score_b is None else score_b.reshape(-1).to(device=device, dtype=torch.float16)
        self.dbn = None if down_block_norm is None else down_block_norm.reshape(-1).to(torch.float16).to(device)
        self.R = int(self.enc_w.shape[0])
        self.NB = int(self.score_w.shape[0])
        self.basis_top_k = self.R if basis_top_k is None else max(1, min(int(basis_top_k), self.R))
        self.legacy_abs = bool(legacy_abs)

    def route(self, x: torch.Tensor, k: int, *, sorted_by_score: bool = False) -> torch.Tensor:
        """Top-k blocks of every row of ``x`` [M, H]: ``sel`` [M, k] int32
        (ascending ids, or torch.topk order with ``sorted_by_score``)."""
        x16 = x.reshape(-1, int(self.enc_w.shape[1])).to(device=self.device, dtype=torch.float16).contiguous()
        M, H = int(x16.shape[0]), int(x16.shape[1])
        kk = max(1, min(int(k), self.NB))
        flags = (_lib.NSMLP_ROUTE_SORTED if sorted_by_score else 0) | (_lib.NSMLP_ROUTE_LEGACY_ABS if self.legacy_abs
                                                                       else 0)
        sel = torch.empty((M, kk), dtype=torch.int32, device=self.device)
        ws = workspace(int(_lib.lib().nsmlp_route_workspace_bytes(M, H, self.R, self.NB, kk)), self.device)
        _lib.call("nsmlp_route_f16", ptr(x16), M, H, ptr(self.enc_w), ptr(self.enc_b), self.R, self.basis_top_k,
                  ptr(self.score_w), ptr(self.score_b), ptr(self.dbn), self.NB,
                  flags, kk, ptr(sel), None, None, ptr(ws), ws.numel(), stream_handle(self.device))
        return sel

    def as_struct(self) -> _lib.Router:
        return _lib.Router(
            R=self.R, basis_top_k=self.basis_top_k, NB=self.NB,
            flags=_lib.NSMLP_ROUTE_LEGACY_ABS if self.legacy_abs else 0,
            enc_w=ptr(self.enc_w), enc_b=ptr(self.enc_b), score_w=ptr(self.score_w), score_b=ptr(self.score_b),
            down_block_norm=ptr(self.dbn),
        )


def recency_weights(rows: int, power: float) -> torch.Tensor:
    """The calibration weight of each row, ((r + 1) / rows) ** power in fp32
    on the CPU (RT:2224-2228)."""
    pos = torch.arange(1, int(rows) + 1, dtype=torch.float32)
    return torch.pow(pos / float(max(int(rows), 1)), float(power))


def record_hot_cache_calibration_blocks(counts: torch.Tensor, active_blocks: torch.Tensor, *,
                                        recency_power: float = 1.0) -> torch.Tensor:
    """Calibration hit counts on the device (RT:2205-2243 without the host
    copy): ``counts`` [NB] fp32 += the row's recency weight for every block id
    of each row of ``active_blocks`` [rows, k] (ids outside [0, NB) skipped),
    added row by row as ``index_add_`` adds them.  Returns ``counts``."""
    device = require_device(counts, "counts")
    if counts.dtype != torch.float32 or not counts.is_contiguous():
        raise RuntimeError("counts must be a contiguous float32 tensor")
    blocks = active_blocks.to(device=device, dtype=torch.int32).contiguous()
    k = int(blocks.shape[-1]) if blocks.ndim > 0 else 1
    rows = int(blocks.numel()) // max(k, 1)
    if rows == 0:
        return counts
    w = recency_weights(rows, recency_power).to(device)
    _lib.call("nsmlp_cache_record_f32", ptr(counts), int(counts.numel()), ptr(blocks), rows, k, ptr(w),
              stream_handle(device))
    return counts


class HotBlockCache:
    """Device-side replacement policy of a slot table: the promotion of
    missed blocks (RT:2809-3018) with the fixed-capacity slot plan of
    RT:2576-2617, run on the table's stream with no host round trip.  The
    table needs its host copies (``host_copy=True``); the promoted blocks are
    copied from them into the slots.  ``grow_only`` uses free slots only (the
    reference's gate/up hot cache, which never evicts)."""

    def __init__(self, table: SparseMlpSlotTable, *, scores: torch.Tensor | None = None,
                 active_count: int | None = None, grow_only: bool = False):
        if not table.host:
            raise RuntimeError("promotion copies blocks from the table's host copies (build it with host_copy=True)")
        device = table.device
        cap = table.n_slots
        if table.lookup is None:  # all blocks resident in order: make the identity lookup explicit
            table.lookup = torch.arange(table.NB, dtype=torch.int32, device=device)
            table.as_struct()
        self.table = table
        self.grow_only = bool(grow_only)
        blocks = table.block_ids.to(torch.int32)
        self.slot_block = torch.full((cap,), -1, dtype=torch.int32)
        self.slot_block[:int(blocks.numel())] = blocks[:cap]
        self.slot_block = self.slot_block.to(device)
        self.slot_score = (torch.zeros(cap, dtype=torch.float32) if scores is None
                           else scores.to(torch.float32).reshape(-1)[:cap].clone()).to(device).contiguous()
        n_active = int(blocks.numel()) if active_count is None else int(active_count)
        self.active = torch.tensor([max(0, min(n_active, cap))], dtype=torch.int32, device=device)
        self._state = _lib.CacheState(capacity=cap, lookup=ptr(table.lookup), slot_block=ptr(self.slot_block),
                                      slot_score=ptr(self.slot_score), active_count=ptr(self.active))

    def promote(self, blocks: torch.Tensor, *, return_slots: bool = False) -> torch.Tensor | None:
        """Promote the non-resident entries of ``blocks`` (a token's selected
        block ids); optionally return the slot given to each entry (-1: none)."""
        device = self.table.device
        b = blocks.reshape(-1).to(device=device, dtype=torch.int32).contiguous()
        n = int(b.numel())
        slots = torch.empty(n, dtype=torch.int32, device=device) if return_slots else None
        ws = workspace(int(_lib.lib().nsmlp_cache_workspace_bytes(n)), device)
        st = self.table._struct if self.table._struct is not None else self.table.as_struct()
        _lib.call("nsmlp_cache_promote", ctypes.byref(st), ctypes.byref(self._state), ptr(b), n,
                  _lib.NSMLP_CACHE_GROW_ONLY if self.grow_only else 0, ptr(slots), ptr(ws), ws.numel(),
                  stream_handle(device))
        return slots

    def state_cpu(self):
        """(slot block ids, slot scores, active count, lookup) on the CPU."""
        return (self.slot_block.to("cpu", torch.long), self.slot_score.to("cpu"), int(self.active.item()),
                self.table.lookup.to("cpu"))


class SparseMlpLayer:
    """Router + slot table: one call per decode token and layer, no host
    round trip (the decode branch of RT:5833-5923)."""

    def __init__(self, router: SparseMlpRouter, table: SparseMlpSlotTable, top_k: int,
                 cache: HotBlockCache | None = None, *, check_blocks: bool = False, count_blocks: bool = False):
        """``check_blocks``: after every ``forward`` the kernels' status word
        is handed to a pinned host word (one small kernel, no stall); the
        next ``forward`` raises RuntimeError if a finished call selected a
        block that is neither resident nor host-copied, and
        ``check_status()`` waits and raises on demand (the reference's gather
        raises for such a block, RT:4530-4578).  Not for graph capture.

        ``count_blocks``: every ``forward`` adds the selected blocks it read
        from HBM slots and from host copies to running device counters (two
        small kernels per call, no stall); ``served_blocks`` and
        ``runtime_status()`` read them (the reference's runtime status,
        RT:1694-1779).

        With a hot-block ``cache`` a ``forward`` routes first, promotes the
        selected blocks that are not resident into slots (copied once from the
        host copies, the fixed-capacity plan of RT:2576-2617), then decodes
        every selected block from HBM: a missed block crosses the host link
        once, as in the reference, which promotes from the copy it already
        moved to the GPU (RT:4094-4131).  A selected block that the plan
        evicts is read from its host copy."""
        if router.NB != table.NB:
            raise RuntimeError(f"router num_blocks {router.NB} != table num_blocks {table.NB}")
        if cache is not None and cache.table is not table:
            raise RuntimeError("the cache belongs to another slot table")
        self.router = router
        self.table = table
        self.cache = cache
        self.top_k = max(1, min(int(top_k), table.NB))
        self._r = router.as_struct()
        self._t = table.as_struct()
        self.device = table.device
        self._lookahead_done: torch.cuda.Event | None = None
        self._status = StatusWord(self.device, "sparse MLP decode layer") if check_blocks else None
        self._counts = BlockCounts(self.device) if count_blocks else None

    @property
    def served_blocks(self) -> tuple[int, int]:
        """(blocks read from HBM slots, blocks read from host copies), summed
        over the ``forward`` calls so far (waits for the stream)."""
        if self._counts is None:
            raise RuntimeError("build the layer with count_blocks=True to count the served blocks")
        return self._counts.totals()

    def runtime_status(self) -> dict[str, int]:
        """The reference's decode counters (RT:1694-1779) for this layer: its
        gate and up projections each count a block (decode_mlp_*), its down
        projection counts it once (decode_down_*)."""
        hbm, host = self.served_blocks
        return {"decode_mlp_hot_blocks_hit": 2 * hbm, "decode_mlp_cold_blocks_streamed": 2 * host,
                "decode_down_hot_blocks_hit": hbm, "decode_down_cold_blocks_streamed": host}

    def check_status(self) -> None:
        """Wait for the last checked ``forward`` and raise RuntimeError if a
        checked call selected a block it could not serve (``check_blocks``)."""
        if self._status is None:
            raise RuntimeError("build the layer with check_blocks=True to check the status word")
        self._status.check()

    def lookahead(self, hidden: torch.Tensor, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Prefetch for this layer before its decode (the decode loop's
        lookahead, RT:7780-7795): route ``hidden`` [H] with this layer's
        router and promote the selected blocks that are not resident into
        slots, on ``stream`` (a copy stream; default: the current stream).
        The next ``forward`` on any stream waits for it.  Returns the
        lookahead selection [k] int32.  Needs the layer's hot-block cache."""
        if self.cache is None:
            raise RuntimeError("lookahead promotes into the hot-block cache: build the layer with cache=")
        cur = torch.cuda.current_stream(self.device)
        s = cur if stream is None else stream
        if s != cur:
            s.wait_stream(cur)  # hidden is produced on the current stream
        with torch.cuda.stream(s):
            sel = self.router.route(hidden.reshape(1, -1), self.top_k).reshape(-1)
            self.cache.promote(sel)
            ev = torch.cuda.Event()
            ev.record(s)
        if s != cur:
            hidden.record_stream(s)
            sel.record_stream(cur)
        self._lookahead_done = ev
        return sel

    def workspace_bytes(self) -> int:
        return int(_lib.lib().nsmlp_layer_workspace_bytes(self.table.H, self.router.R, self.router.NB, self.top_k))

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, sel_out: torch.Tensor | None = None,
                ws: torch.Tensor | None = None, residual: torch.Tensor | None = None):
        """One decode token: (out [H] fp16, sel [k] int32).  With ``residual``
        [H] fp16, out = residual + mlp(x) with the decode loop's fp16 add
        fused into the down kernel (``out`` may be ``residual`` itself)."""
        x16 = x.reshape(-1)
        if x16.dtype != torch.float16 or x16.device != self.device or x16.data_ptr() % 16:
            x16 = x16.to(device=self.device, dtype=torch.float16).contiguous().clone()
        if out is None:
            out = torch.empty(self.table.H, dtype=torch.float16, device=self.device)
        if sel_out is None:
            sel_out = torch.empty(self.top_k, dtype=torch.int32, device=self.device)
        if ws is None:
            ws = workspace(self.workspace_bytes(), self.device)
        r16 = None
        if residual is not None:
            r16 = residual.reshape(-1)
            if r16.dtype != torch.float16 or r16.device != self.device or not r16.is_contiguous() \
                    or int(r16.numel()) != self.table.H:
                raise RuntimeError(f"residual must be a contiguous fp16 [{self.table.H}] tensor on {self.device}")
        if self._status is not None:
            self._status.poll()  # a finished earlier call's report; no wait
            self._status.clear(ws)  # bits other calls left in the shared workspace are not this layer's
        if self._counts is not None:
            self._counts.clear(ws)
        if self._lookahead_done is not None:  # the promotion of a lookahead reads and writes the table
            torch.cuda.current_stream(self.device).wait_event(self._lookahead_done)
            self._lookahead_done = None
        h = stream_handle(self.device)
        if self.cache is not None:
            # route, promote the missed blocks into slots, then decode from HBM
            r = self.router
            flags = _lib.NSMLP_ROUTE_LEGACY_ABS if r.legacy_abs else 0
            _lib.call("nsmlp_route_f16", ptr(x16), 1, self.table.H, ptr(r.enc_w), ptr(r.enc_b), r.R, r.basis_top_k,
                      ptr(r.score_w), ptr(r.score_b), ptr(r.dbn), r.NB, flags, self.top_k, ptr(sel_out), None, None,
                      ptr(ws), ws.numel(), h)
            self.cache.promote(sel_out)
            if r16 is None:
                _lib.call("nsmlp_decode_slots_f16", ctypes.byref(self._t), ptr(x16), ptr(sel_out), self.top_k,
                          ptr(out), ptr(ws), ws.numel(), h)
            else:
                _lib.call("nsmlp_decode_slots_add_f16", ctypes.byref(self._t), ptr(x16), ptr(r16), ptr(sel_out),
                          self.top_k, ptr(out), ptr(ws), ws.numel(), h)
        elif r16 is None:
            _lib.call("nsmlp_decode_layer_f16", ctypes.byref(self._r), ctypes.byref(self._t), ptr(x16), self.top_k,
                      ptr(sel_out), ptr(out), ptr(ws), ws.numel(), h)
        else:
            _lib.call("nsmlp_decode_layer_add_f16", ctypes.byref(self._r), ctypes.byref(self._t), ptr(x16), ptr(r16),
                      self.top_k, ptr(sel_out), ptr(out), ptr(ws), ws.numel(), h)
        if self._status is not None:
            self._status.take(ws)
        if self._counts is not None:
            self._counts.take(ws)
        return out, sel_out

    def prefill(self, x: torch.Tensor, out: torch.Tensor | None = None):
        """M tokens [M, H]: per-token routing (ascending block ids), then the
        grouped MFMA prefill over the union of the selected blocks.
        Returns (out [M, H] fp16, sel [M, k] int32)."""
        x16 = x.reshape(-1, self.table.H).to(device=self.device, dtype=torch.float16).contiguous()
        sel = self.router.route(x16, self.top_k)
        return self.table.prefill(x16, sel, out=out), sel
